"""Twin functions (HIP kernels) against the CPU oracle, function by function, at
the Qwen3-1.7B layer shape -- the comparison the reference runs with
``tilefoundry check twin.py:LayerTwin.<fn>`` (fast/twin.py:1-17).

Tolerances.  The twin rounds to bf16 at every point the authored HIR does, so
an element differs from the oracle only where an f32 sum taken in a different
order lands on the other side of a bf16 rounding boundary.  Hence: most outputs
bit-identical, every differing element within one bf16 ulp for single-rounding
outputs, and the chained outputs within the north-star bound (max |delta| <= 2e-2
of the output's max magnitude, bf16).
"""
import pytest
import torch

from oracle import qwen3_hir as O
from tests._parity import assert_close_bf16, report, ulp_bf16
from tilefoundry_amd.qwen3 import QWEN3_1_7B, synthetic_weights
from tilefoundry_amd.qwen3.twin import LayerTwin, RootTwin

pytestmark = pytest.mark.gpu

CFG = QWEN3_1_7B.with_(num_hidden_layers=1, vocab_size=4096)
DIMS = O.Qwen3Dims(hidden=CFG.hidden_size, heads=CFG.num_attention_heads,
                   kv_heads=CFG.num_key_value_heads, head_dim=CFG.head_dim,
                   intermediate=CFG.intermediate_size, vocab=CFG.vocab_size, layers=1)


@pytest.fixture(scope="module", params=["ones", "random"])
def setup(request, gpu_device):
    w = synthetic_weights(CFG, seed=11, norms=request.param)
    dev = {k: v.to(gpu_device) for k, v in w.items()}
    return w, dev, LayerTwin(CFG), RootTwin(CFG)


def _layer_args(w, prefix="layer0."):
    return [w[prefix + n] for n in ("gamma_in", "w_q", "w_k", "w_v", "gamma_q", "gamma_k")]


def _hidden(seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(1, 1, CFG.hidden_size, generator=g) * scale).to(torch.bfloat16)


def _cache(seed, ctx):
    g = torch.Generator().manual_seed(seed)
    shape = (1, ctx, CFG.num_key_value_heads, CFG.head_dim)
    return (torch.randn(shape, generator=g).to(torch.bfloat16),
            torch.randn(shape, generator=g).to(torch.bfloat16))


def test_input_rms_norm(setup, gpu_device):
    w, dw, twin, _ = setup
    x = _hidden(1, 3.0)
    want = O.input_rms_norm(DIMS, x, w["layer0.gamma_in"])
    got = twin.input_rms_norm(x.to(gpu_device), dw["layer0.gamma_in"])
    r = report(got, want)
    assert r["within_1ulp"] == 1.0 and r["exact"] > 0.99, r


@pytest.mark.parametrize("ctx", [0, 1, 15, 16, 63, 64, 65, 200, 700])
def test_self_attention(setup, gpu_device, ctx):
    w, dw, twin, _ = setup
    x = _hidden(2 + ctx)
    kc, vc = _cache(100 + ctx, ctx)
    cos, sin = O.generation_rope(DIMS, 4096)
    pos = torch.tensor([ctx], dtype=torch.int32)
    scale = torch.full((1, 1, 1, 1), CFG.head_dim ** -0.5, dtype=torch.bfloat16)
    want = O.self_attention(DIMS, x, *_layer_args(w), cos, sin, pos, kc, vc, scale,
                            w["layer0.w_o"])
    d = lambda t: t.to(gpu_device)  # noqa: E731
    got = twin.self_attention(d(x), *_layer_args(dw), d(cos), d(sin), d(pos), d(kc), d(vc),
                              d(scale), dw["layer0.w_o"])
    for name, g_, w_ in zip(("k_rope", "v"), got[1:], want[1:]):
        r = report(g_, w_)
        assert r["within_1ulp"] >= 0.999 and r["exact"] >= 0.98, (name, r)
    assert_close_bf16(got[0], want[0], name=f"attn out ctx={ctx}", min_exact=0.5)


def test_self_attention_rope_position_differs_from_cache_length(setup, gpu_device):
    """The HIR takes pos_ids and the prior cache separately (model.py:150-152)."""
    w, dw, twin, _ = setup
    x = _hidden(7)
    kc, vc = _cache(8, 40)
    cos, sin = O.generation_rope(DIMS, 4096)
    pos = torch.tensor([123], dtype=torch.int32)
    scale = torch.full((1, 1, 1, 1), CFG.head_dim ** -0.5, dtype=torch.bfloat16)
    want = O.self_attention(DIMS, x, *_layer_args(w), cos, sin, pos, kc, vc, scale,
                            w["layer0.w_o"])
    d = lambda t: t.to(gpu_device)  # noqa: E731
    got = twin.self_attention(d(x), *_layer_args(dw), d(cos), d(sin), d(pos), d(kc), d(vc),
                              d(scale), dw["layer0.w_o"])
    assert report(got[1], want[1])["within_1ulp"] >= 0.999
    assert_close_bf16(got[0], want[0], name="attn out pos!=ctx")


def test_mlp(setup, gpu_device):
    w, dw, twin, _ = setup
    x = _hidden(3)
    names = ("gamma_post", "w_gate", "w_up", "w_down")
    want = O.mlp(DIMS, x, *[w["layer0." + n] for n in names])
    got = twin.mlp(x.to(gpu_device), *[dw["layer0." + n] for n in names])
    assert_close_bf16(got, want, name="mlp", min_exact=0.5)


@pytest.mark.parametrize("ctx", [0, 33, 300])
def test_decoder_layer(setup, gpu_device, ctx):
    w, dw, twin, _ = setup
    x = _hidden(4 + ctx)
    kc, vc = _cache(200 + ctx, ctx)
    cos, sin = O.generation_rope(DIMS, 4096)
    pos = torch.tensor([ctx], dtype=torch.int32)
    scale = torch.full((1, 1, 1, 1), CFG.head_dim ** -0.5, dtype=torch.bfloat16)
    rest = [w["layer0." + n] for n in ("gamma_post", "w_gate", "w_up", "w_down")]
    drest = [dw["layer0." + n] for n in ("gamma_post", "w_gate", "w_up", "w_down")]
    want = O.decoder_layer(DIMS, x, *_layer_args(w), cos, sin, pos, kc, vc, scale,
                           w["layer0.w_o"], *rest)
    d = lambda t: t.to(gpu_device)  # noqa: E731
    got = twin.decoder_layer(d(x), *_layer_args(dw), d(cos), d(sin), d(pos), d(kc), d(vc),
                             d(scale), dw["layer0.w_o"], *drest)
    assert_close_bf16(got[0], want[0], name=f"decoder_layer ctx={ctx}", min_exact=0.5)


def test_root_functions(setup, gpu_device):
    w, dw, _, root = setup
    ids = torch.tensor([1234])
    got = root.embed(dw["w_embed"], ids.to(gpu_device))
    assert torch.equal(got.cpu(), O.embed(DIMS, w["w_embed"], ids))
    x = _hidden(5, 2.0)
    got = root.final_rms_norm(x.to(gpu_device), dw["gamma_final"])
    assert report(got, O.final_rms_norm(DIMS, x, w["gamma_final"]))["within_1ulp"] == 1.0
    xn = O.final_rms_norm(DIMS, x, w["gamma_final"])
    want = O.lm_head(DIMS, xn, w["w_head"])
    got = root.lm_head(xn.to(gpu_device), dw["w_head"])
    r = report(got, want)
    assert r["within_1ulp"] >= 0.999 and r["exact"] >= 0.98, r


def test_embed_rejects_out_of_range_id(setup, gpu_device):
    _, dw, _, root = setup
    with pytest.raises(IndexError):
        root.embed(dw["w_embed"], torch.tensor([CFG.vocab_size], device=gpu_device))
