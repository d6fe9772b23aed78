"""Pins of the CPU oracle (oracle/qwen3_hir.py) that do not re-type its formulas.

* f32 oracle == Hugging Face ``Qwen3ForCausalLM`` (local modelling code, built from
  a config dict, same weights), every decode position of a greedy run against a
  full-sequence causal forward -- as the reference's own oracle is built
  (tests/models/decode_oracle.py:126-137, qwen3_1_7b/reference.py:44-70);
* bf16 attention within bf16 noise of an f64 brute-force softmax
  (fast/arbitrate.py:22-56);
* the exact-products arithmetic (``exact_products``): equal to the HIR's bit for
  bit where every product is a bf16 value, within bf16 noise of the HIR on
  random inputs and not equal to it there (the switch is live);
* argmax tie rule: first maximal index (tests/ops/test_argmax.py:70-73);
* RoPE: rotation preserves each pair's norm; position 0 is the identity;
* cache growth: append_cache grows every layer by one position per step.
"""
import math

import pytest
import torch

from oracle import qwen3_hir as O
from tilefoundry_amd.qwen3 import TINY, synthetic_weights


def _hf_model(dims, w):
    from transformers import Qwen3Config as HFConfig
    from transformers import Qwen3ForCausalLM

    cfg = HFConfig(
        vocab_size=dims.vocab, hidden_size=dims.hidden, intermediate_size=dims.intermediate,
        num_hidden_layers=dims.layers, num_attention_heads=dims.heads,
        num_key_value_heads=dims.kv_heads, head_dim=dims.head_dim, rms_norm_eps=dims.eps,
        rope_theta=dims.rope_theta, max_position_embeddings=dims.max_positions,
        tie_word_embeddings=True, attention_bias=False, hidden_act="silu",
    )
    cfg._attn_implementation = "eager"
    torch.manual_seed(0)
    model = Qwen3ForCausalLM(cfg).eval().to(torch.float32)
    sd = {"model.embed_tokens.weight": w["w_embed"], "model.norm.weight": w["gamma_final"],
          "lm_head.weight": w["w_head"].t()}
    hf = {"gamma_in": "input_layernorm.weight", "gamma_post": "post_attention_layernorm.weight",
          "gamma_q": "self_attn.q_norm.weight", "gamma_k": "self_attn.k_norm.weight",
          "w_q": "self_attn.q_proj.weight", "w_k": "self_attn.k_proj.weight",
          "w_v": "self_attn.v_proj.weight", "w_o": "self_attn.o_proj.weight",
          "w_gate": "mlp.gate_proj.weight", "w_up": "mlp.up_proj.weight",
          "w_down": "mlp.down_proj.weight"}
    for i in range(dims.layers):
        for ours, theirs in hf.items():
            t = w[f"layer{i}.{ours}"]
            sd[f"model.layers.{i}.{theirs}"] = t[0].t() if t.dim() == 3 else t
    missing, unexpected = model.load_state_dict({k: v.contiguous() for k, v in sd.items()},
                                                strict=False)
    assert not unexpected and all("rotary" in m for m in missing), (missing, unexpected)
    return model


@pytest.mark.parametrize("norms", ["random", "ones"])
def test_f32_oracle_matches_hf_every_position(norms):
    dims = O.C1
    w = synthetic_weights(TINY, seed=0, norms=norms)
    g = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, dims.vocab, (24,), generator=g).tolist()
    run = O.decode(O.Qwen3Oracle(dims, w), prompt, max_new=8)
    seq = torch.tensor(prompt + run.tokens[:-1]).unsqueeze(0)
    model = _hf_model(dims, w)
    with torch.no_grad():
        ref = model(seq).logits[0]                     # [len, V] f32
    for k, got in enumerate(run.logits):
        want = ref[len(prompt) - 1 + k]
        scale = want.abs().max().item()
        err = (got - want).abs().max().item()
        assert err <= 2e-5 * max(scale, 1.0), (k, err, scale)
        assert int(torch.argmax(want)) == run.tokens[k]


def _f64_attention(q, kc, vc, kn, vn, scale):
    """softmax((q.k) * scale) . v over cache + new, in float64 (arbitrate.py:22-56)."""
    g = q.shape[0] // kc.shape[1]
    kk = torch.cat([kc, kn[None]], 0).double().repeat_interleave(g, dim=1)
    vv = torch.cat([vc, vn[None]], 0).double().repeat_interleave(g, dim=1)
    s = (q.double()[None] * kk).sum(-1) * scale
    p = torch.softmax(s, dim=0)
    return (p[..., None] * vv).sum(0)


def test_bf16_attention_core_close_to_f64():
    """The HIR's bf16 attention chain (model.py:183-212) stays within bf16 noise
    of exact softmax attention; a wrong sign, a dropped term or a swapped
    operand in the chain moves it by O(1)."""
    torch.manual_seed(3)
    hq, hkv, d, ctx = 4, 2, 64, 37
    dims = O.Qwen3Dims(hidden=hq * d, heads=hq, kv_heads=hkv, head_dim=d, intermediate=64,
                       vocab=16, layers=1, dtype=torch.bfloat16)
    w = synthetic_weights(TINY.with_(dtype=torch.bfloat16, hidden_size=hq * d,
                                     num_hidden_layers=1, intermediate_size=64, vocab_size=16),
                          seed=5, norms="ones")
    hidden = (torch.randn(1, 1, hq * d) * 0.5).to(torch.bfloat16)
    kc = (torch.randn(1, ctx, hkv, d)).to(torch.bfloat16)
    vc = (torch.randn(1, ctx, hkv, d)).to(torch.bfloat16)
    cos, sin = O.generation_rope(dims, 64)
    pos = torch.tensor([ctx], dtype=torch.int32)
    scale = torch.full((1, 1, 1, 1), d ** -0.5, dtype=torch.bfloat16)
    eye = torch.eye(hq * d, dtype=torch.bfloat16).unsqueeze(0)
    g = lambda n: w[f"layer0.{n}"]  # noqa: E731
    out, k_rope, v = O.self_attention(dims, hidden, g("gamma_in"), g("w_q"), g("w_k"), g("w_v"),
                                      g("gamma_q"), g("gamma_k"), cos, sin, pos, kc, vc, scale,
                                      eye)
    # recompute q_rope the same way and feed f64 attention with identical inputs
    hn = O.input_rms_norm(dims, hidden, g("gamma_in"))
    q = torch.matmul(hn, g("w_q")).reshape(1, 1, hq, d)
    q_rope = O._rope(O._head_rms(q, g("gamma_q"), dims.eps, torch.bfloat16), cos, sin, pos,
                     torch.bfloat16)
    ref = _f64_attention(q_rope[0, 0], kc[0], vc[0], k_rope[0, 0], v[0, 0], d ** -0.5)
    got = out.reshape(hq, d).double()
    rel = ((got - ref).abs().max() / ref.abs().max()).item()
    assert rel < 3e-2, rel
    cos_sim = torch.nn.functional.cosine_similarity(got.flatten(), ref.flatten(), 0).item()
    assert cos_sim > 0.999, cos_sim


def _attention_case(seed, kc, vc, *, zero_new_key=False):
    """One layer's self_attention (o_proj the identity) over the given caches."""
    torch.manual_seed(seed)
    hq, hkv, d = 4, 2, 64
    ctx = kc.shape[1]
    dims = O.Qwen3Dims(hidden=hq * d, heads=hq, kv_heads=hkv, head_dim=d, intermediate=64,
                       vocab=16, layers=1, dtype=torch.bfloat16)
    w = synthetic_weights(TINY.with_(dtype=torch.bfloat16, hidden_size=hq * d,
                                     num_hidden_layers=1, intermediate_size=64, vocab_size=16),
                          seed=5, norms="ones")
    w_k = w["layer0.w_k"] * 0 if zero_new_key else w["layer0.w_k"]
    hidden = (torch.randn(1, 1, hq * d) * 0.5).to(torch.bfloat16)
    cos, sin = O.generation_rope(dims, 128)
    pos = torch.tensor([ctx], dtype=torch.int32)
    scale = torch.full((1, 1, 1, 1), d ** -0.5, dtype=torch.bfloat16)
    eye = torch.eye(hq * d, dtype=torch.bfloat16).unsqueeze(0)
    g = lambda n: w[f"layer0.{n}"]  # noqa: E731
    out, _, _ = O.self_attention(dims, hidden, g("gamma_in"), g("w_q"), w_k, g("w_v"),
                                 g("gamma_q"), g("gamma_k"), cos, sin, pos, kc, vc, scale, eye)
    return out


def _pow2(shape, gen):
    """bf16 entries +-2^e (e in -3..2): a bf16 value times one is a bf16 value."""
    e = torch.randint(-3, 3, shape, generator=gen).float()
    sign = torch.randint(0, 2, shape, generator=gen).float() * 2 - 1
    return (sign * torch.exp2(e)).to(torch.bfloat16)


def test_exact_products_equal_the_hir_where_products_are_bf16():
    """With every cache entry a power of two and the new key zero, each q.k and
    p.v product is itself a bf16 value, so not rounding the products changes
    nothing: under exact sums the two arithmetics agree bit for bit (a dropped
    term, a wrong axis or a wrong operand would not)."""
    gen = torch.Generator().manual_seed(11)
    kc, vc = _pow2((1, 53, 2, 64), gen), _pow2((1, 53, 2, 64), gen)
    with O.exact_sums():
        hir = _attention_case(4, kc, vc, zero_new_key=True)
        with O.exact_products():
            ex = _attention_case(4, kc, vc, zero_new_key=True)
    assert torch.equal(hir, ex)
    assert hir.abs().max() > 0


def test_exact_products_close_to_f64_and_not_the_hir():
    """On random caches the exact-products chain stays within bf16 noise of the
    HIR's (which test_bf16_attention_core_close_to_f64 holds to the f64
    softmax), and differs from it somewhere: the products' rounding is what it
    leaves out."""
    gen = torch.Generator().manual_seed(12)
    kc = torch.randn(1, 61, 2, 64, generator=gen).to(torch.bfloat16)
    vc = torch.randn(1, 61, 2, 64, generator=gen).to(torch.bfloat16)
    hir = _attention_case(6, kc, vc).double()
    with O.exact_products():
        ex = _attention_case(6, kc, vc).double()
    assert not torch.equal(hir, ex)
    rel = ((ex - hir).abs().max() / hir.abs().max()).item()
    assert rel < 2e-2, rel
    cos_sim = torch.nn.functional.cosine_similarity(ex.flatten(), hir.flatten(), 0).item()
    assert cos_sim > 0.9999, cos_sim


def test_argmax_first_index_on_ties():
    assert O.greedy(torch.zeros(1, 10)) == 0
    x = torch.tensor([[0.5, 2.0, 1.0, 2.0, 2.0]])
    assert O.greedy(x) == 1
    x = torch.tensor([[-1.0, -1.0]], dtype=torch.bfloat16)
    assert O.greedy(x) == 0


def test_rope_rotation_invariants():
    dims = O.C1
    cos, sin = O.generation_rope(dims.__class__(**{**dims.__dict__, "dtype": torch.float32}), 64)
    x = torch.randn(1, 1, 2, dims.head_dim)
    half = dims.head_dim // 2
    out0 = O._rope(x, cos, sin, torch.tensor([0]), torch.float32)
    assert torch.equal(out0, x)                              # position 0: identity
    out = O._rope(x, cos, sin, torch.tensor([17]), torch.float32)
    pair_in = x[..., :half] ** 2 + x[..., half:] ** 2
    pair_out = out[..., :half] ** 2 + out[..., half:] ** 2
    assert torch.allclose(pair_in, pair_out, rtol=1e-5, atol=1e-6)
    # rotation angle of pair i at position p is p * theta^(-2i/D)
    i = 3
    ang = 17 * dims.rope_theta ** (-2 * i / dims.head_dim)
    a, b = x[..., i], x[..., i + half]
    assert torch.allclose(out[..., i], a * math.cos(ang) - b * math.sin(ang), atol=1e-5)


def test_cache_grows_one_position_per_step():
    dims = O.C1
    w = synthetic_weights(TINY, seed=1)
    orc = O.Qwen3Oracle(dims, w)
    caches = orc.init_caches()
    ids = torch.tensor([5, 9, 11])
    for step in range(3):
        args = orc.prepare_inputs_for_generation(ids, step, caches)
        _, fresh = orc.forward(*args)
        caches = orc.append_cache(caches, fresh)
        assert all(k.shape == (1, step + 1, dims.kv_heads, dims.head_dim) for k, _ in caches)
