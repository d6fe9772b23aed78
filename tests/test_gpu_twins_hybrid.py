"""The hybrid models' runtime twins (authored names, signatures and canonical
weights; tilefoundry_amd/hybrid/twin.py) on the GPU.

* Every authored sub-function -- Qwen3.5's conv_step, l2_normalise, delta_step,
  partial_rope, Granite's in_projection, conv_step, ssm_step, gated_out -- and
  every entry function (linear_attention, full_attention, routing, experts,
  routed_experts, shared_expert; mamba_mixer, qkv, attend, full_attention,
  routing, experts, routed_experts, shared_mlp) against the oracle's restatement
  on the same inputs: f32 functions to f32 rounding, bf16 ones to the bf16 bar
  (the kernels' f32 sums run in another order than the oracle's f64 ones), expert
  ids exactly, ids returned as int64.
* The whole twin decoders (forward / append_cache / prepare_inputs_for_generation
  as authored) against the decode engines on the same draw: Qwen3.5 against
  Qwen35Engine; Granite against GraniteOracle's whole step and GraniteEngine with
  power-of-two fp8 row scales, where the authored bf16 weights hold the fp8
  products exactly.
Shapes: the models' real widths, fewer layers / experts and a 4,096-token
vocabulary, as the engines' own tests."""
import pytest
import torch

from oracle import hybrid_ref as H
from tests._parity import assert_close_bf16
from tilefoundry_amd.hybrid import twin as T
from tilefoundry_amd.hybrid.granite import GraniteConfig, GraniteEngine
from tilefoundry_amd.hybrid.granite import synthetic_weights as granite_weights
from tilefoundry_amd.hybrid.qwen3_5 import Qwen35Config, Qwen35Engine, rope_tables
from tilefoundry_amd.hybrid.qwen3_5 import synthetic_weights as qwen35_weights

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
C4 = Qwen35Config(layers=4, experts=16, vocab=4096)
C5 = GraniteConfig(layers=3, attention_layers=(1,), experts=12, top_k=4, vocab=4096)


def cpu(t):
    return t.detach().float().cpu()


def rel(got, want):
    g, w = cpu(got), cpu(want)
    return ((g - w).abs().max() / w.abs().max().clamp(min=1e-30)).item()


@pytest.fixture(scope="module")
def c4():
    w = qwen35_weights(C4, seed=3, device=DEV)
    can = T.qwen35_canonical(C4, w)
    return w, can, T.Qwen3_5Decoder(C4).load(can)


def _pow2_scales(w):
    """Row scales rounded to the nearest power of two (the codes unchanged)."""
    out = dict(w)
    for k, v in w.items():
        if k.endswith("_scale") or k.split(".")[-1].startswith("s_"):
            out[k] = torch.exp2(torch.round(torch.log2(v)))
    return out


@pytest.fixture(scope="module")
def c5():
    w = _pow2_scales(granite_weights(C5, seed=5, device=DEV))
    can = T.granite_canonical(C5, w)
    return w, can, T.Granite4_0_H_Small(C5, capacity=64).load(can)


# ---------------------------------------------------------------------------
# Qwen3.5 (C4)
# ---------------------------------------------------------------------------
def test_c4_conv_l2_delta_match_oracle(c4):
    _, can, dec = c4
    mixer = dec.layers[0].mixer
    g = torch.Generator().manual_seed(1)
    conv_w = can["layer0.mixer.conv_w"]
    state = H.bf(torch.randn(1, C4.conv_dim, 3, generator=g))
    entry = H.bf(torch.randn(1, C4.conv_dim, 1, generator=g))
    got = mixer.conv_step(state.to(DEV), entry.to(DEV), conv_w)
    want, _ = H.conv_step_c4(state, entry[:, :, 0], cpu(conv_w))
    torch.testing.assert_close(cpu(got), want, atol=1e-6, rtol=1e-5)

    x = torch.randn(1, 1, C4.lin_value_heads, C4.lin_key_dim, generator=g)
    torch.testing.assert_close(cpu(mixer.l2_normalise(x.to(DEV))), H.l2_normalise(x),
                               atol=1e-6, rtol=1e-5)

    hv, dk = C4.lin_value_heads, C4.lin_key_dim
    st = torch.randn(1, hv, dk, dk, generator=g) * 0.1
    q = H.l2_normalise(torch.randn(1, 1, hv, dk, generator=g))
    k = H.l2_normalise(torch.randn(1, 1, hv, dk, generator=g))
    v = torch.randn(1, 1, hv, dk, generator=g)
    gg = -torch.rand(1, 1, hv, generator=g)
    beta = torch.rand(1, 1, hv, generator=g)
    read, upd = mixer.delta_step(st.to(DEV), q.to(DEV), k.to(DEV), v.to(DEV), gg.to(DEV),
                                 beta.to(DEV))
    want_r, want_u = H.delta_step(st, q[:, 0], k[:, 0], v[:, 0], gg[:, 0], beta[:, 0], dk ** -0.5)
    assert read.shape == (1, hv, dk) and upd.shape == (1, hv, dk, dk)
    torch.testing.assert_close(cpu(read), want_r, atol=1e-5, rtol=1e-4)
    torch.testing.assert_close(cpu(upd), want_u, atol=1e-6, rtol=1e-5)


def test_c4_partial_rope_matches_oracle(c4):
    _, _, dec = c4
    attn = dec.layers[3].mixer
    g = torch.Generator().manual_seed(2)
    cos, sin = rope_tables(C4, 64)
    pos = torch.tensor([37], dtype=torch.int32)
    for heads, fn in ((C4.heads, attn.partial_rope), (C4.kv_heads, attn.partial_rope_kv)):
        x = torch.randn(1, 1, heads, C4.head_dim, generator=g)
        got = fn(x.to(DEV), cos.to(DEV), sin.to(DEV), pos.to(DEV))
        want = H.partial_rope(x[0], cos[37:38], sin[37:38])
        torch.testing.assert_close(cpu(got)[0, 0], want[0], atol=1e-6, rtol=1e-5)


def _c4_norm_proj(w, i, hidden):
    xn = H.bf(H._rms_flat(hidden, cpu(w[f"layer{i}.gamma_in"]), C4.eps))
    return xn, H.bf(H.mm_rows(cpu(w[f"layer{i}.w_in"]), xn))


def test_c4_linear_attention_matches_oracle(c4):
    w, can, dec = c4
    m = "layer0.mixer."
    g = torch.Generator().manual_seed(4)
    hidden = torch.randn(1, 1, C4.hidden, generator=g)
    conv = H.bf(torch.randn(1, C4.conv_dim, 3, generator=g))
    state = torch.randn(1, C4.lin_value_heads, C4.lin_key_dim, C4.lin_value_dim,
                        generator=g) * 0.05
    out, entry, upd = dec.layers[0].mixer.linear_attention(
        hidden.to(DEV), can[m + "gamma_in"], can[m + "w_in_qkv"], can[m + "w_in_z"],
        can[m + "w_in_b"], can[m + "w_in_a"], can[m + "conv_w"], can[m + "a_log"],
        can[m + "dt_bias"], conv.to(DEV), state.to(DEV), can[m + "gamma_gdn"], can[m + "w_out"])
    _, proj = _c4_norm_proj(w, 0, hidden[0])
    gated, _, want_state = H.gdn_step(
        proj, conv, state, cpu(w["layer0.conv_w"]), cpu(w["layer0.a_log"]),
        cpu(w["layer0.dt_bias"]), cpu(w["layer0.gamma_gdn"]), hk=C4.lin_key_heads,
        hv=C4.lin_value_heads, dk=C4.lin_key_dim, dv=C4.lin_value_dim, rms_eps=C4.eps)
    want = H.bf(H.mm_rows(cpu(w["layer0.w_out"]), H.bf(gated)))
    assert out.shape == (1, 1, C4.hidden) and entry.shape == (1, C4.conv_dim, 1)
    assert_close_bf16(out[0], want, max_rel=2e-2, name="linear_attention out")
    assert_close_bf16(entry[:, :, 0], proj[:, :C4.conv_dim], max_rel=1e-2, min_exact=0.99,
                      name="entry")
    assert rel(upd, want_state) < 1e-3


def test_c4_full_attention_matches_oracle(c4):
    w, can, dec = c4
    i, m = 3, "layer3.mixer."
    HKV, D = C4.kv_heads, C4.head_dim
    g = torch.Generator().manual_seed(5)
    C = 37
    hidden = torch.randn(1, 1, C4.hidden, generator=g)
    kc = H.bf(torch.randn(1, C, HKV, D, generator=g))
    vc = H.bf(torch.randn(1, C, HKV, D, generator=g))
    _, layer_args, _ = dec.prepare_inputs_for_generation(torch.zeros(C + 1, dtype=torch.int64),
                                                         C, None, device=DEV)
    cos, sin, pos_ids, scale = layer_args[i]
    out, k_rope, v = dec.layers[i].mixer.full_attention(
        hidden.to(DEV), can[m + "gamma_in"], can[m + "w_qg"], can[m + "w_k"], can[m + "w_v"],
        can[m + "gamma_q"], can[m + "gamma_k"], cos, sin, pos_ids, kc.to(DEV), vc.to(DEV),
        scale, can[m + "w_o"])
    _, proj = _c4_norm_proj(w, i, hidden[0])
    HQ = C4.heads
    qg = proj[:, :HQ * 2 * D].reshape(1, HQ, 2 * D)
    k = proj[:, HQ * 2 * D:HQ * 2 * D + HKV * D].reshape(1, HKV, D)
    vv = proj[:, HQ * 2 * D + HKV * D:].reshape(1, HKV, D)
    mixed, kr = H.qwen35_attend(qg, k, vv, [kc[0]], [vc[0]], cpu(w["layer3.gamma_q"]),
                                cpu(w["layer3.gamma_k"]), cpu(cos), cpu(sin), D ** -0.5, C4.eps)
    want = H.bf(H.mm_rows(cpu(w["layer3.w_out"]), H.bf(mixed)))
    assert_close_bf16(out[0], want, max_rel=2e-2, name="full_attention out")
    assert_close_bf16(k_rope[0, 0], H.bf(kr[0]), max_rel=1e-2, min_exact=0.99, name="k_rope")
    assert_close_bf16(v[0, 0], vv[0], max_rel=1e-2, min_exact=0.99, name="v")


def test_c4_routing_and_experts_match_oracle(c4):
    w, can, dec = c4
    e = "layer1.moe."
    moe = dec.layers[1].moe
    g = torch.Generator().manual_seed(6)
    hidden = torch.randn(1, 3, C4.hidden, generator=g)
    tokens = moe.post_norm(hidden.to(DEV), can[e + "gamma_post"])
    xm = H.bf(H._rms_flat(hidden[0], cpu(w["layer1.gamma_post"]), C4.eps))
    torch.testing.assert_close(cpu(tokens), xm, atol=0, rtol=2 ** -7)
    weights, idx = moe.router.routing(tokens, can[e + "router.w_router"])
    assert idx.dtype == torch.int64 and weights.shape == (3, C4.top_k)
    want_w, want_i = H.route_softmax_topk(H.bf(H.mm_rows(cpu(w["layer1.w_router"]), cpu(tokens))),
                                          C4.top_k)
    assert torch.equal(idx.cpu(), want_i)
    torch.testing.assert_close(cpu(weights), want_w, atol=1e-6, rtol=1e-5)
    args = [can[e + n] for n in ("w_gate", "w_up", "w_down")]
    shared = [can[e + n] for n in ("w_shared_gate", "w_shared_up", "w_shared_down",
                                   "w_shared_scale")]
    out = moe.experts(tokens, weights, idx, *args, *shared)
    IS = C4.shared_inter
    want = H.moe_c4(cpu(tokens), cpu(weights), idx.cpu(), cpu(w["layer1.w_gate"]),
                    cpu(w["layer1.w_up"]), cpu(w["layer1.w_down"]),
                    cpu(w["layer1.w_shared_in"])[:IS], cpu(w["layer1.w_shared_in"])[IS:],
                    cpu(w["layer1.w_shared_out"]), cpu(w["layer1.w_shared_scale"])[None])
    assert out.shape == (1, 3, C4.hidden)
    assert_close_bf16(out[0], want, max_rel=2e-2, name="experts")
    routed = moe.routed_experts(tokens, weights, idx, *args)
    dense = moe.shared_expert(tokens, *shared)
    torch.testing.assert_close(cpu(routed) + cpu(dense), cpu(out[0]), atol=1e-5, rtol=1e-5)


def test_c4_decoder_matches_the_engine(c4):
    """The twin's authored step, driven as the reference drives it, gives the
    engine's logits on the same draw (same kernels, same arithmetic)."""
    w, _, dec = c4
    g = torch.Generator().manual_seed(7)
    prompt = torch.randint(0, C4.vocab, (4,), generator=g).tolist()
    new = 3
    eng = Qwen35Engine(C4, w, rows=1, device=DEV, max_steps=32, split_len=16, small=False)
    tokens, _, logits = eng.generate([prompt], new, record_logits=True)
    feed = prompt + tokens[0][:-1]
    ids = torch.tensor(feed, dtype=torch.int64)
    caches = dec.init_caches(device=DEV)
    for step in range(len(feed)):
        tok, layer_args, caches = dec.prepare_inputs_for_generation(ids, step, caches,
                                                                    device=DEV)
        got, fresh = dec.forward(tok, layer_args, caches)
        caches = dec.append_cache(caches, fresh)
        want = logits[step]
        r = rel(got[0], want[0])
        print(f"step {step}: twin vs engine rel {r:.2e}")
        assert r < 2e-3, (step, r)
        if step >= len(prompt) - 1:
            assert int(got[0].argmax()) == tokens[0][step - len(prompt) + 1]


def test_c4_twin_load_rejects_bad_weights(c4):
    _, can, _ = c4
    bad = dict(can)
    bad.pop("layer2.mixer.w_in_z")
    with pytest.raises(KeyError, match="w_in_z"):
        T.Qwen3_5Decoder(C4).load(bad)
    bad = dict(can)
    bad["layer3.mixer.w_o"] = can["layer3.mixer.w_o"][:, :-1]
    with pytest.raises(ValueError, match="w_o"):
        T.Qwen3_5Decoder(C4).load(bad)


# ---------------------------------------------------------------------------
# Granite-4.0-H (C5)
# ---------------------------------------------------------------------------
def test_c5_mamba_pieces_match_oracle(c5):
    _, can, dec = c5
    mamba = dec.layers[0].mixer
    m = "layer0.mixer."
    g = torch.Generator().manual_seed(11)
    nh, pd, ns = C5.mamba_heads, C5.mamba_head_dim, C5.d_state
    hidden = H.bf(torch.randn(1, 1, C5.hidden, generator=g))
    proj = mamba.in_projection(hidden.to(DEV), can[m + "gamma_in"], can[m + "w_in"])
    xn = H.rms_norm_tf(hidden[0], cpu(can[m + "gamma_in"]), C5.eps)
    want_proj = H.bf(H.mm_rows(cpu(can[m + "w_in"]), xn))
    assert_close_bf16(proj, want_proj, max_rel=1e-2, min_exact=0.99, name="in_projection")

    conv = H.bf(torch.randn(1, C5.conv_dim, 3, generator=g))
    entry = H.bf(torch.randn(1, C5.conv_dim, 1, generator=g))
    got = mamba.conv_step(conv.to(DEV), entry.to(DEV), can[m + "conv_w"], can[m + "conv_b"])
    want, _ = H.conv_step_c5(conv, entry[:, :, 0], cpu(can[m + "conv_w"]), cpu(can[m + "conv_b"]))
    assert_close_bf16(got, want, max_rel=1e-2, min_exact=0.99, name="conv_step")

    st = torch.randn(1, nh, pd, ns, generator=g) * 0.1
    x = H.bf(torch.randn(1, nh, pd, generator=g))
    bv = H.bf(torch.randn(1, 1, ns, generator=g))
    cv = H.bf(torch.randn(1, 1, ns, generator=g))
    dt = H.bf(torch.randn(1, nh, generator=g))
    y, upd = mamba.ssm_step(st.to(DEV), x.to(DEV), bv.to(DEV), cv.to(DEV), dt.to(DEV),
                            can[m + "a_log"], can[m + "dt_bias"], can[m + "d_skip"])
    want_y, want_u = H.ssm_step(st, x, bv, cv, dt, cpu(can[m + "a_log"]), cpu(can[m + "dt_bias"]),
                                cpu(can[m + "d_skip"]))
    assert_close_bf16(y, want_y, max_rel=2e-2, min_exact=0.95, name="ssm_step y")
    assert rel(upd, want_u) < 1e-5

    gate = H.bf(torch.randn(1, C5.d_inner, generator=g))
    out = mamba.gated_out(y, gate.to(DEV), can[m + "gamma_ssm"], can[m + "w_out"])
    normed = H.gated_rmsnorm(cpu(y).reshape(1, -1), gate, cpu(can[m + "gamma_ssm"]), C5.eps)
    want_o = H.bf(H.mm_rows(cpu(can[m + "w_out"]), normed))
    assert_close_bf16(out[0], want_o, max_rel=2e-2, name="gated_out")


def test_c5_mamba_mixer_matches_oracle(c5):
    _, can, dec = c5
    m = "layer2.mixer."
    g = torch.Generator().manual_seed(12)
    hidden = H.bf(torch.randn(1, 1, C5.hidden, generator=g))
    conv = H.bf(torch.randn(1, C5.conv_dim, 3, generator=g))
    st = torch.randn(1, C5.mamba_heads, C5.mamba_head_dim, C5.d_state, generator=g) * 0.1
    names = ("gamma_in", "w_in", "conv_w", "conv_b", "a_log", "dt_bias", "d_skip")
    out, entry, upd = dec.layers[2].mixer.mamba_mixer(
        hidden.to(DEV), *[can[m + n] for n in names], conv.to(DEV), st.to(DEV),
        can[m + "gamma_ssm"], can[m + "w_out"])
    xn = H.rms_norm_tf(hidden[0], cpu(can[m + "gamma_in"]), C5.eps)
    proj = H.bf(H.mm_rows(cpu(can[m + "w_in"]), xn))
    normed, _, want_u = H.mamba_step(proj, conv, st, *[cpu(can[m + n]) for n in names[2:]],
                                     cpu(can[m + "gamma_ssm"]), nh=C5.mamba_heads,
                                     pd=C5.mamba_head_dim, ns=C5.d_state, ng=1, eps=C5.eps)
    want = H.bf(H.mm_rows(cpu(can[m + "w_out"]), normed))
    assert_close_bf16(out[0], want, max_rel=2e-2, name="mamba_mixer")
    assert_close_bf16(entry[:, :, 0], proj[:, C5.d_inner:C5.d_inner + C5.conv_dim],
                      max_rel=1e-2, min_exact=0.99, name="entry")
    assert rel(upd, want_u) < 1e-3


def test_c5_attention_matches_oracle(c5):
    _, can, dec = c5
    m = "layer1.mixer."
    attn = dec.layers[1].mixer
    HQ, HKV, D = C5.heads, C5.kv_heads, C5.head_dim
    g = torch.Generator().manual_seed(13)
    cur, cap = 29, 64
    hidden = H.bf(torch.randn(1, 1, C5.hidden, generator=g))
    kc = H.bf(torch.randn(1, cap, HKV, D, generator=g))
    vc = H.bf(torch.randn(1, cap, HKV, D, generator=g))
    q, k, v = attn.qkv(hidden.to(DEV), can[m + "gamma_in"], can[m + "w_q"], can[m + "w_k"],
                       can[m + "w_v"])
    _, layer_args, _ = dec.prepare_inputs_for_generation(torch.zeros(cur + 1, dtype=torch.int64),
                                                         cur, None, device=DEV)
    cur_pos, mask = layer_args[1]
    out, k_next, v_next = attn.full_attention(
        hidden.to(DEV), can[m + "gamma_in"], can[m + "w_q"], can[m + "w_k"], can[m + "w_v"],
        kc.to(DEV), vc.to(DEV), cur_pos, mask, can[m + "w_o"])
    att = H.granite_attend(cpu(q).reshape(1, HQ, D), cpu(k).reshape(1, HKV, D),
                           cpu(v).reshape(1, HKV, D), [kc[0, :cur]], [vc[0, :cur]],
                           C5.attention_multiplier)
    want = H.bf(H.mm_rows(cpu(can[m + "w_o"]), att))
    assert_close_bf16(out[0], want, max_rel=2e-2, name="full_attention")
    assert torch.equal(cpu(k_next[0, cur]), cpu(k[0, 0])) and torch.equal(cpu(k_next[0, :cur]),
                                                                         kc[0, :cur])
    assert torch.equal(cpu(v_next[0, cur]), cpu(v[0, 0]))
    # attend over the updated caches is the same computation
    again = attn.attend(q, k_next, v_next, cur_pos, mask, can[m + "w_o"])
    assert torch.equal(cpu(again), cpu(out))


def test_c5_routing_and_experts_match_oracle(c5):
    _, can, dec = c5
    e = "layer0.moe."
    moe = dec.layers[0].moe
    g = torch.Generator().manual_seed(14)
    hidden = H.bf(torch.randn(1, 2, C5.hidden, generator=g))
    tokens = moe.post_norm(hidden.to(DEV), can[e + "gamma_post"])
    torch.testing.assert_close(cpu(tokens), H.rms_norm_tf(hidden[0], cpu(can[e + "gamma_post"]),
                                                          C5.eps), atol=0, rtol=2 ** -7)
    weights, idx = moe.router.routing(tokens, can[e + "router.w_router"])
    assert idx.dtype == torch.int64 and weights.dtype == torch.bfloat16
    want_w, want_i = H.route_topk_softmax(
        H.bf(H.mm_rows(cpu(can[e + "router.w_router"]), cpu(tokens))), C5.top_k)
    assert torch.equal(idx.cpu(), want_i)
    torch.testing.assert_close(cpu(weights), want_w, atol=0, rtol=2 ** -7)
    ex = [can[e + n] for n in ("w_gate", "w_up", "w_down")]
    sh = [can[e + n] for n in ("w_shared_in", "w_shared_out")]
    out = moe.experts(tokens, weights, idx, *ex, *sh)
    want = H.moe_c5_dense(cpu(tokens), cpu(weights), idx.cpu(), *[cpu(t) for t in ex],
                          *[cpu(t) for t in sh])
    assert_close_bf16(out[0], want, max_rel=2e-2, name="experts")
    routed = moe.routed_experts(tokens, weights, idx, *ex)
    dense = moe.shared_mlp(tokens, *sh)
    assert_close_bf16(H.bf(cpu(routed) + cpu(dense)), cpu(out[0]), max_rel=1e-2, min_exact=0.99,
                      name="routed + shared")


def test_c5_decoder_matches_oracle_and_engine(c5):
    w, _, dec = c5
    g = torch.Generator().manual_seed(15)
    prompt = torch.randint(0, C5.vocab, (3,), generator=g).tolist()
    new = 2
    eng = GraniteEngine(C5, w, rows=1, device=DEV, max_steps=32, split_len=16)
    tokens, _, logits = eng.generate([prompt], new, record_logits=True)
    feed = prompt + tokens[0][:-1]
    ids = torch.tensor(feed, dtype=torch.int64)
    orc = H.GraniteOracle(C5, {k: v.cpu() for k, v in w.items()}, 1)
    caches = dec.init_caches(device=DEV)
    for step in range(len(feed)):
        tok, layer_args, caches = dec.prepare_inputs_for_generation(ids, step, caches,
                                                                    device=DEV)
        got, fresh = dec.forward(tok, layer_args, caches)
        caches = dec.append_cache(caches, fresh)
        want = orc.step([feed[step]])
        r_o, r_e = rel(got[0], want[0]), rel(got[0], logits[step][0])
        print(f"step {step}: twin vs oracle {r_o:.2e}, vs engine {r_e:.2e}")
        assert r_o < 2e-2 and r_e < 2e-2, (step, r_o, r_e)
