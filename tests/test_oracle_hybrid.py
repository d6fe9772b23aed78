"""Pins of the hybrid-model oracle (``oracle/hybrid_ref.py``) on the CPU.

Each function of the oracle is checked against something it does not restate:
the e4m3fn format's closed form, the reference's own fp8 known answer, and the
independent HF transformers modules of the same models (``Qwen3_5Moe*`` and
``GraniteMoeHybrid*``, transformers 5.15) run in f32.  The oracle rounds where
its model's reference rounds (to bf16), so the HF comparisons hold to bf16
tolerance; a dropped term, a swapped gate/up half or a transposed operand
moves the result by O(1) and fails them."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import hybrid_ref as H

hf_q = pytest.importorskip("transformers.models.qwen3_5_moe.modeling_qwen3_5_moe")
hf_g = pytest.importorskip("transformers.models.granitemoehybrid.modeling_granitemoehybrid")


def e4m3fn_closed_form(code: int) -> float:
    """OCP FP8 E4M3 ("fn": no infinities, S.1111.111 is NaN): bias 7, 3-bit
    mantissa, subnormals at exponent field 0."""
    s, e, m = code >> 7, (code >> 3) & 15, code & 7
    if e == 15 and m == 7:
        return math.nan
    mag = (m / 8) * 2.0 ** -6 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7)
    return -mag if s else mag


def test_fp8_decode_every_code_matches_the_closed_form():
    codes = torch.arange(256, dtype=torch.uint8).reshape(1, 256)
    got = H.fp8_dequant(codes, torch.ones(1))[0]
    for c in range(256):
        want = e4m3fn_closed_form(c)
        if math.isnan(want):
            assert math.isnan(got[c].item()), c
        else:
            assert got[c].item() == want, (c, got[c].item(), want)
    assert got[0x7E].item() == 448.0 and got[0x01].item() == 2.0 ** -9


def test_fp8_reference_known_answer_round_trips():
    """tests/ops/test_quant.py:183-199 quantises [224, -112, 7, -1, 3, -12, 96, -48]
    exactly (every value is an e4m3fn value); their codes decode back exactly."""
    vals = torch.tensor([[224.0, -112.0, 7.0, -1.0, 3.0, -12.0, 96.0, -48.0]])
    codes = vals.to(torch.float8_e4m3fn).view(torch.uint8)
    assert torch.equal(H.fp8_dequant(codes, torch.ones(1)), vals)
    assert torch.equal(H.fp8_dequant(codes, torch.tensor([0.5])), vals * 0.5)


def test_gemv_fp8_one_hot_picks_one_scaled_column():
    g = torch.Generator().manual_seed(3)
    codes = torch.randint(0, 256, (24, 64), generator=g, dtype=torch.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x38                       # no NaN codes (0x38 = 1.0)
    scale = torch.rand(24, generator=g) + 0.5
    for k0 in (0, 17, 63):
        x = torch.zeros(1, 64)
        x[0, k0] = 1.0
        y = H.gemv_fp8(codes, scale, x)[0]
        want = torch.tensor([e4m3fn_closed_form(int(c)) for c in codes[:, k0]]) * scale
        assert torch.equal(y, want.float())


def _logits(b, e, seed):
    g = torch.Generator().manual_seed(seed)
    return H.bf(torch.randn(b, e, generator=g) * 2)


def _same_selection(logits, idx, want_idx):
    """The same logits in the same order; the same ids wherever the row has no
    tie among its top k + 1 logits (torch.topk orders ties arbitrarily)."""
    assert torch.equal(logits.gather(1, idx), logits.gather(1, want_idx))
    k = idx.shape[1]
    top = torch.sort(logits, dim=-1, descending=True).values[:, :k + 1]
    untied = (top[:, 1:] != top[:, :-1]).all(dim=1)
    assert torch.equal(idx[untied], want_idx[untied])
    return int(untied.sum())


def test_route_softmax_topk_matches_hf_qwen3_5_router():
    logits = _logits(6, 32, 0)
    cfg = type("C", (), {"num_experts_per_tok": 4, "num_experts": 32, "hidden_size": 32})()
    r = hf_q.Qwen3_5MoeTopKRouter(cfg)
    with torch.no_grad():
        r.weight.copy_(torch.eye(32))
        _, scores, idx = r(logits)
    w, i = H.route_softmax_topk(logits, 4)
    assert _same_selection(logits, i, idx) >= 3
    torch.testing.assert_close(w, scores, atol=0, rtol=0)
    torch.testing.assert_close(w.sum(-1), torch.ones(6))


def test_route_topk_softmax_matches_hf_granite_router():
    logits = _logits(5, 72, 1)
    cfg = type("C", (), {"num_local_experts": 72, "num_experts_per_tok": 10,
                         "hidden_size": 72})()
    r = hf_g.GraniteMoeHybridTopKRouter(cfg).to(torch.bfloat16)
    with torch.no_grad():
        r.weight.copy_(torch.eye(72))
        idx, weights, _ = r(logits.to(torch.bfloat16))
    w, i = H.route_topk_softmax(logits, 10)
    assert _same_selection(logits, i, idx) >= 2
    assert torch.equal(w, weights.float())


def test_routers_rank_like_brute_force():
    """Largest first, equal logits by ascending id (ties included on purpose)."""
    logits = torch.tensor([[0.5, 2.0, 2.0, -1.0, 2.0, 0.5, 3.0, 0.5],
                           [1.0, 1.0, 1.0, 1.0, 1.0, 1.0, 1.0, 1.0]])
    logits = torch.cat([logits, _logits(4, 8, 2)])
    for fn in (H.route_softmax_topk, H.route_topk_softmax):
        _, idx = fn(logits, 5)
        for b in range(logits.shape[0]):
            order = sorted(range(8), key=lambda e: (-logits[b, e].item(), e))[:5]
            assert idx[b].tolist() == order


def test_routers_over_their_own_set_are_the_routers():
    """Weights over the set a router picked are that router's, bit for bit."""
    logits = H.bf(_logits(6, 72, 5))
    for full, over in ((H.route_softmax_topk, H.route_softmax_over),
                       (H.route_topk_softmax, H.route_topk_softmax_over)):
        w, idx = full(logits, 8)
        w2, idx2 = over(logits, idx.flip(-1))          # any order in, router order out
        assert torch.equal(idx2, idx) and torch.equal(w2, w)


def test_follow_near_ties_takes_only_swaps_within_the_slack():
    """k = 3 over logits with the k-th at 1.0 (bf16 ulp 2^-7): an engine set that
    swaps the 4th for the 3rd (1 ulp apart) or the 5th (2 ulps) is followed; one
    that swaps in the 6th (3 ulps) or drops the clear 1st is not."""
    u = 2.0 ** -7
    rlog = torch.tensor([[4.0, 2.0, 1.0, 1.0 - u, 1.0 - 2 * u, 1.0 - 3 * u, -1.0]] * 5)
    own = torch.tensor([[0, 1, 2]] * 5)
    engine = torch.tensor([[1, 0, 2],          # same set, other order
                           [0, 1, 3],          # 4th for 3rd: 1 ulp
                           [4, 0, 1],          # 5th for 3rd: 2 ulps
                           [0, 1, 5],          # 6th for 3rd: 3 ulps
                           [3, 1, 2]])         # 4th for the 1st: far above the 3rd
    use, fol, far, dist = H.follow_near_ties(rlog, own, engine, 3)
    assert fol.tolist() == [False, True, True, False, False]
    assert far.tolist() == [False, False, False, True, True]
    assert dist.tolist() == [0.0, 1.0, 2.0, 3.0, 384.0]
    assert use[0].tolist() == [0, 1, 2] and use[3].tolist() == [0, 1, 2]
    assert sorted(use[1].tolist()) == [0, 1, 3] and sorted(use[2].tolist()) == [0, 1, 4]
    w, idx = H.route_topk_softmax_over(rlog, use)
    assert idx[1].tolist() == [0, 1, 3] and idx[2].tolist() == [0, 1, 4]
    top = torch.softmax(torch.tensor([4.0, 2.0, 1.0 - u]), dim=0)
    assert torch.equal(w[1], H.bf(top))


def _bf_param(module, std, gen):
    with torch.no_grad():
        for p in module.parameters():
            p.copy_(H.bf(torch.randn(p.shape, generator=gen) * std))


def test_moe_c4_matches_hf_sparse_moe_block():
    from transformers.models.qwen3_5_moe.configuration_qwen3_5_moe import Qwen3_5MoeTextConfig
    g = torch.Generator().manual_seed(4)
    hs, inter, e, k = 64, 32, 8, 3
    cfg = Qwen3_5MoeTextConfig(hidden_size=hs, moe_intermediate_size=inter,
                               shared_expert_intermediate_size=48, num_experts=e,
                               num_experts_per_tok=k)
    blk = hf_q.Qwen3_5MoeSparseMoeBlock(cfg)
    _bf_param(blk, 0.2, g)
    x = H.bf(torch.randn(4, hs, generator=g))
    with torch.no_grad():
        want = blk(x[None])[0]
        _, weights, idx = blk.gate(x)
    gu = blk.experts.gate_up_proj.detach()
    se = blk.shared_expert
    got = H.moe_c4(x, weights, idx, gu[:, :inter], gu[:, inter:],
                   blk.experts.down_proj.detach(), se.gate_proj.weight.detach(),
                   se.up_proj.weight.detach(), se.down_proj.weight.detach(),
                   blk.shared_expert_gate.weight.detach())
    err = (got - want).abs().max() / want.abs().max()
    assert err < 1.5e-2, err


def _fp8_linear(shape, gen):
    codes = (torch.randn(shape, generator=gen) * 0.5).to(torch.float8_e4m3fn).view(torch.uint8)
    scale = torch.rand(shape[:-1], generator=gen) * 0.1 + 0.05
    return codes, scale


def test_moe_c5_matches_hf_granite_moe_and_shared_mlp():
    g = torch.Generator().manual_seed(5)
    hs, inter, sh, e, k = 64, 32, 48, 12, 4
    cfg = type("C", (), {"num_local_experts": e, "num_experts_per_tok": k, "hidden_size": hs,
                         "intermediate_size": inter, "shared_intermediate_size": sh,
                         "hidden_act": "silu", "_experts_implementation": None})()
    moe = hf_g.GraniteMoeHybridMoE.__new__(hf_g.GraniteMoeHybridMoE)
    torch.nn.Module.__init__(moe)
    moe.input_size = hs
    moe.router = hf_g.GraniteMoeHybridTopKRouter(cfg)
    moe.experts = hf_g.GraniteMoeHybridExperts(cfg)
    mlp = hf_g.GraniteMoeHybridMLP(cfg)
    gu_c, gu_s = _fp8_linear((e, 2 * inter, hs), g)
    d_c, d_s = _fp8_linear((e, hs, inter), g)
    si_c, si_s = _fp8_linear((2 * sh, hs), g)
    so_c, so_s = _fp8_linear((hs, sh), g)
    deq = lambda c, s: c.view(torch.float8_e4m3fn).float() * s[..., None]
    with torch.no_grad():
        moe.router.weight.copy_(H.bf(torch.randn(e, hs, generator=g) * 0.3))
        moe.experts.gate_up_proj.copy_(deq(gu_c, gu_s))
        moe.experts.down_proj.copy_(deq(d_c, d_s))
        mlp.input_linear.weight.copy_(deq(si_c, si_s))
        mlp.output_linear.weight.copy_(deq(so_c, so_s))
        x = H.bf(torch.randn(3, hs, generator=g))
        want = moe(x[None])[0] + mlp(x)
        idx, weights, _ = moe.router(x)
    got = H.moe_c5(x, H.bf(weights), idx, gu_c[:, :inter], gu_s[:, :inter],
                   gu_c[:, inter:], gu_s[:, inter:], d_c, d_s, si_c, si_s, so_c, so_s)
    err = (got - want).abs().max() / want.abs().max()
    assert err < 2e-2, err


def test_gdn_step_matches_hf_composition():
    """conv update + l2norm + gated delta rule + RMSNormGated as HF's
    Qwen3_5MoeGatedDeltaNet composes them for one token with a cache."""
    g = torch.Generator().manual_seed(6)
    b, hk, hv, dk, dv = 2, 2, 4, 16, 16
    key, val = hk * dk, hv * dv
    conv = 2 * key + val
    proj = H.bf(torch.randn(b, conv + val + 2 * hv, generator=g))
    conv_state = torch.randn(b, conv, 3, generator=g)
    state = torch.randn(b, hv, dk, dv, generator=g) * 0.2
    conv_w = H.bf(torch.randn(conv, 4, generator=g) * 0.5)
    a_log = H.bf(torch.randn(hv, generator=g) * 0.5)
    dt_bias = H.bf(torch.randn(hv, generator=g) * 0.5)
    gamma = H.bf(1 + 0.1 * torch.randn(dv, generator=g))
    got, new_conv, new_state = H.gdn_step(proj, conv_state, state, conv_w, a_log, dt_bias,
                                          gamma, hk=hk, hv=hv, dk=dk, dv=dv)
    cs = conv_state.clone()
    mixed = hf_q.causal_conv1d_update(proj[:, :conv, None], cs, conv_w, None, "silu")[:, :, 0]
    q = mixed[:, :key].reshape(b, 1, hk, dk).repeat_interleave(hv // hk, dim=2)
    k = mixed[:, key:2 * key].reshape(b, 1, hk, dk).repeat_interleave(hv // hk, dim=2)
    v = mixed[:, 2 * key:].reshape(b, 1, hv, dv)
    z = proj[:, conv:conv + val]
    beta = proj[:, conv + val:conv + val + hv].sigmoid()[:, None]
    gg = (-a_log.exp() * F.softplus(proj[:, conv + val + hv:] + dt_bias))[:, None]
    core, st = hf_q.torch_recurrent_gated_delta_rule(q, k, v, gg, beta, state.clone(), True,
                                                     use_qk_l2norm_in_kernel=True)
    norm = hf_q.Qwen3_5MoeRMSNormGated(dv, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(gamma)
        want = norm(core.reshape(-1, dv), z.reshape(-1, dv)).reshape(b, val)
    torch.testing.assert_close(new_conv, cs, atol=0, rtol=0)
    torch.testing.assert_close(new_state, st, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-4)


def test_mamba_step_matches_hf_composition():
    """conv update + selective state update + RMSNormGated as HF's
    GraniteMoeHybridMambaLayer composes them for one token with a cache (f32);
    the oracle rounds to bf16 where the HIR does, so the match is to bf16."""
    g = torch.Generator().manual_seed(7)
    b, nh, pd, ns = 3, 4, 8, 16
    exp_ = nh * pd
    conv = exp_ + 2 * ns
    proj = H.bf(torch.randn(b, exp_ + conv + nh, generator=g))
    conv_state = H.bf(torch.randn(b, conv, 3, generator=g))
    state = torch.randn(b, nh, pd, ns, generator=g) * 0.3
    conv_w = H.bf(torch.randn(conv, 4, generator=g) * 0.5)
    conv_b = H.bf(torch.randn(conv, generator=g) * 0.1)
    a_log = H.bf(torch.randn(nh, generator=g) * 0.5)
    dt_bias = H.bf(torch.randn(nh, generator=g) * 0.5)
    d_skip = H.bf(torch.randn(nh, generator=g))
    gamma = H.bf(1 + 0.1 * torch.randn(exp_, generator=g))
    got, new_conv, new_state = H.mamba_step(proj, conv_state, state, conv_w, conv_b, a_log,
                                            dt_bias, d_skip, gamma, nh=nh, pd=pd, ns=ns, ng=1)
    gate, entry, dt = proj[:, :exp_], proj[:, exp_:exp_ + conv], proj[:, exp_ + conv:]
    cs = conv_state.clone()
    mixed = hf_g.causal_conv1d_update(entry[:, :, None], cs, conv_w, conv_b, "silu")[:, :, 0]
    x = mixed[:, :exp_].reshape(b, nh, pd)
    st = state.clone()
    y = hf_g.mamba2_selective_state_update(
        st, x, dt[:, :, None].expand(-1, -1, pd), (-a_log.exp())[:, None, None].expand(-1, pd, ns),
        mixed[:, exp_:exp_ + ns].reshape(b, 1, ns), mixed[:, exp_ + ns:].reshape(b, 1, ns),
        d_skip[:, None].expand(-1, pd), dt_bias=dt_bias[:, None].expand(-1, pd),
        dt_softplus=True)
    norm = hf_g.GraniteMoeHybridRMSNormGated(exp_, eps=1e-5)
    with torch.no_grad():
        norm.weight.copy_(gamma)
        want = norm(y.reshape(b, exp_), gate)
    torch.testing.assert_close(new_conv, cs, atol=0, rtol=0)
    rel = lambda a, w: ((a - w).abs().max() / w.abs().max()).item()
    assert rel(new_state, st) < 2e-2
    assert rel(got, want) < 3e-2


def _rope_rows(pos, rot, theta=1e6):
    inv = 1.0 / theta ** (torch.arange(0, rot, 2, dtype=torch.float64) / rot)
    f = torch.tensor(pos, dtype=torch.float64)[:, None] * inv[None]
    emb = torch.cat((f, f), dim=-1)
    return H.bf(emb.cos().float()), H.bf(emb.sin().float())


def test_qwen35_attend_matches_hf_attention_pieces():
    """Per-head norm (HF's 1 + w with w = gamma - 1), partial RoPE
    (apply_rotary_pos_emb with a 16-wide cache on 64-wide heads), eager GQA
    attention over the past plus this token, sigmoid output gate."""
    g = torch.Generator().manual_seed(9)
    B, HQ, HKV, D, rot = 3, 8, 2, 64, 16
    past = [5, 0, 17]
    qg = H.bf(torch.randn(B, HQ, 2 * D, generator=g))
    k = H.bf(torch.randn(B, HKV, D, generator=g))
    v = H.bf(torch.randn(B, HKV, D, generator=g))
    k_past = [H.bf(torch.randn(c, HKV, D, generator=g)) for c in past]
    v_past = [H.bf(torch.randn(c, HKV, D, generator=g)) for c in past]
    gq = H.bf(1 + 0.2 * torch.randn(D, generator=g))
    gk = H.bf(1 + 0.2 * torch.randn(D, generator=g))
    cos, sin = _rope_rows(past, rot)
    scale = D ** -0.5
    got, kr = H.qwen35_attend(qg, k, v, k_past, v_past, gq, gk, cos, sin, scale)
    qn = hf_q.Qwen3_5MoeRMSNorm(D, eps=1e-6)
    kn = hf_q.Qwen3_5MoeRMSNorm(D, eps=1e-6)
    module = type("M", (), {"num_key_value_groups": HQ // HKV, "training": False})()
    with torch.no_grad():
        qn.weight.copy_(gq - 1)
        kn.weight.copy_(gk - 1)
        for b in range(B):
            q_b = qn(qg[b, :, :D][None, None]).transpose(1, 2)            # (1, HQ, 1, D)
            k_b = kn(k[b][None, None]).transpose(1, 2)                     # (1, HKV, 1, D)
            q_r, k_r = hf_q.apply_rotary_pos_emb(q_b, k_b, cos[b][None, None], sin[b][None, None])
            keys = torch.cat((k_past[b].permute(1, 0, 2)[None], k_r), dim=2)
            vals = torch.cat((v_past[b].permute(1, 0, 2)[None], v[b][:, None][None]), dim=2)
            o, _ = hf_q.eager_attention_forward(module, q_r, keys, vals, None, scaling=scale)
            want = o.reshape(-1) * torch.sigmoid(qg[b, :, D:].reshape(-1))
            torch.testing.assert_close(got[b], want, atol=2e-5, rtol=1e-4)
            torch.testing.assert_close(kr[b], k_r[0, :, 0], atol=1e-6, rtol=1e-5)


def test_granite_attend_matches_hf_eager_attention():
    g = torch.Generator().manual_seed(10)
    B, HQ, HKV, D = 2, 8, 2, 32
    past = [9, 2]
    q = H.bf(torch.randn(B, HQ, D, generator=g))
    k_new = H.bf(torch.randn(B, HKV, D, generator=g))
    v_new = H.bf(torch.randn(B, HKV, D, generator=g))
    k_past = [H.bf(torch.randn(c, HKV, D, generator=g)) for c in past]
    v_past = [H.bf(torch.randn(c, HKV, D, generator=g)) for c in past]
    scale = 0.25
    got = H.granite_attend(q, k_new, v_new, k_past, v_past, scale)
    module = type("M", (), {"num_key_value_groups": HQ // HKV, "training": False})()
    for b in range(B):
        keys = torch.cat((k_past[b], k_new[b][None])).permute(1, 0, 2)[None]
        vals = torch.cat((v_past[b], v_new[b][None])).permute(1, 0, 2)[None]
        o, _ = hf_g.eager_attention_forward(module, q[b][:, None][None], keys, vals, None,
                                            scaling=scale)
        want = o.reshape(-1)
        err = ((got[b] - want).abs().max() / want.abs().max()).item()
        assert err < 2e-2, err


def test_attend_with_no_past_returns_this_tokens_value():
    """One live position: softmax is exactly 1, so attention returns v_new."""
    g = torch.Generator().manual_seed(11)
    q = H.bf(torch.randn(1, 4, 16, generator=g))
    kv = H.bf(torch.randn(2, 1, 2, 16, generator=g))
    empty = [torch.zeros(0, 2, 16)]
    got = H.granite_attend(q, kv[0], kv[1], empty, empty, 0.3)
    assert torch.equal(got[0], kv[1][0].repeat_interleave(2, dim=0).reshape(-1))
    qg = H.bf(torch.randn(1, 4, 32, generator=g))
    cos, sin = _rope_rows([0], 8)
    got, _ = H.qwen35_attend(qg, kv[0], kv[1], empty, empty, torch.ones(16), torch.ones(16),
                             cos, sin, 0.25)
    want = kv[1][0].repeat_interleave(2, dim=0) * torch.sigmoid(qg[0, :, 16:])
    assert torch.equal(got[0], want.reshape(-1))


def test_rms_norm_tf_rounds_once_like_torch_rms_norm():
    """``tf.rms_norm`` (the evaluator's handler, ir/hir/nn/rms_norm.py:103-110)
    is torch's own fused f32 ``rms_norm`` cast to bf16 once; the Qwen3-order
    norm (rounded before gamma) differs from it on many elements."""
    g = torch.Generator().manual_seed(12)
    x = H.bf(torch.randn(6, 4096, generator=g) * 3)
    gamma = H.bf(1 + 0.3 * torch.randn(4096, generator=g))
    got = H.rms_norm_tf(x, gamma, 1e-5)
    want = F.rms_norm(x, (4096,), gamma, 1e-5).to(torch.bfloat16).float()
    assert torch.equal(got, want)
    r = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-5)
    twice = H.bf(H.bf(x * r) * gamma)
    assert (twice != want).float().mean() > 0.05


def test_partial_rope_matches_hf_apply_rotary_pos_emb():
    """The standalone partial RoPE (the twins' partial_rope / partial_rope_kv) is
    HF's apply_rotary_pos_emb on the first rot dims with the tail passed through."""
    g = torch.Generator().manual_seed(21)
    B, HQ, HKV, D, rot = 3, 8, 2, 64, 16
    past = [4, 0, 31]
    q = torch.randn(B, HQ, D, generator=g)
    k = torch.randn(B, HKV, D, generator=g)
    cos, sin = _rope_rows(past, rot)
    for b in range(B):
        q_r, k_r = hf_q.apply_rotary_pos_emb(q[b][None, :, None], k[b][None, :, None],
                                             cos[b][None, None], sin[b][None, None])
        torch.testing.assert_close(H.partial_rope(q[b:b + 1], cos[b:b + 1], sin[b:b + 1])[0],
                                   q_r[0, :, 0], atol=1e-6, rtol=1e-6)
        torch.testing.assert_close(H.partial_rope(k[b:b + 1], cos[b:b + 1], sin[b:b + 1])[0],
                                   k_r[0, :, 0], atol=1e-6, rtol=1e-6)


def test_moe_c5_dense_equals_the_fp8_form_at_power_of_two_scales():
    """With every row scale a power of two, the dequantised bf16 weights hold the fp8
    products exactly, so the dense restatement and the fp8 one give the same bits; a
    dropped shared MLP or swapped gate/up fails."""
    g = torch.Generator().manual_seed(8)
    hs, inter, sh, e, k, B = 64, 32, 48, 12, 4, 3
    codes = lambda *s: (torch.randn(*s, generator=g) * 0.6).to(torch.float8_e4m3fn).view(torch.uint8)
    p2 = lambda *s: torch.exp2(torch.randint(-8, -4, s, generator=g).float())
    g_c, g_s = codes(e, inter, hs), p2(e, inter)
    u_c, u_s = codes(e, inter, hs), p2(e, inter)
    d_c, d_s = codes(e, hs, inter), p2(e, hs)
    si_c, si_s = codes(2 * sh, hs), p2(2 * sh)
    so_c, so_s = codes(hs, sh), p2(hs)
    deq = lambda c, s: H.bf(c.view(torch.float8_e4m3fn).float() * s[..., None])
    x = H.bf(torch.randn(B, hs, generator=g))
    logits = torch.randn(B, e, generator=g)
    w, idx = H.route_topk_softmax(logits, k)
    want = H.moe_c5(x, w, idx, g_c, g_s, u_c, u_s, d_c, d_s, si_c, si_s, so_c, so_s)
    got = H.moe_c5_dense(x, w, idx, deq(g_c, g_s), deq(u_c, u_s), deq(d_c, d_s),
                         deq(si_c, si_s), deq(so_c, so_s))
    assert torch.equal(got, want)
    swapped = H.moe_c5_dense(x, w, idx, deq(u_c, u_s), deq(g_c, g_s), deq(d_c, d_s),
                             deq(si_c, si_s), deq(so_c, so_s))
    assert not torch.equal(swapped, want)
