"""Host-side checks of the boundary, on the CPU: the declared-weight validation
(``Module.load`` semantics, ir/core/module.py:144-159: KeyError for a missing
weight, ValueError for a wrong shape or dtype) and the paged-cache scatter the
engines use to place a context."""
import pytest
import torch

from tilefoundry_amd.qwen3 import TINY, declared_shapes, synthetic_weights, validate
from tilefoundry_amd.qwen3.engine import scatter_cache

CFG = TINY.with_(dtype=torch.bfloat16)


@pytest.fixture(scope="module")
def weights():
    return synthetic_weights(CFG, seed=0)


def test_validate_accepts_the_declared_set(weights):
    validate(CFG, weights)
    assert set(declared_shapes(CFG)) <= set(weights)


def test_validate_missing_weight_is_a_key_error(weights):
    w = dict(weights)
    del w["layer1.w_down"]
    with pytest.raises(KeyError, match="layer1.w_down"):
        validate(CFG, w)


def test_validate_wrong_shape_is_a_value_error(weights):
    w = dict(weights)
    w["layer0.w_q"] = w["layer0.w_q"][..., :-8]
    with pytest.raises(ValueError, match="layer0.w_q"):
        validate(CFG, w)


def test_validate_wrong_dtype_is_a_value_error(weights):
    w = dict(weights)
    w["gamma_final"] = w["gamma_final"].float()
    with pytest.raises(ValueError, match="dtype"):
        validate(CFG, w)


def test_scatter_cache_goes_through_the_page_table():
    """Position p lands in row p % 16 of page table[p // 16]; every other row
    keeps its value; reading back through the table gives the cache."""
    g = torch.Generator().manual_seed(0)
    L, pages, hkv, d, P = 2, 9, 2, 8, 37
    table = torch.randperm(pages, generator=g).to(torch.int32)
    kpool = torch.full((L, pages, hkv, 16, d), -7.0)
    vpool = kpool.clone()
    ks = [torch.randn(P, hkv, d, generator=g) for _ in range(L)]
    vs = [torch.randn(P, hkv, d, generator=g) for _ in range(L)]
    scatter_cache(kpool, vpool, table, ks, vs)
    for i in range(L):
        for p in range(P):
            assert torch.equal(kpool[i, table[p // 16], :, p % 16], ks[i][p])
            assert torch.equal(vpool[i, table[p // 16], :, p % 16], vs[i][p])
    written = P * hkv * d * L
    assert int((kpool != -7.0).sum()) == written and int((vpool != -7.0).sum()) == written


@pytest.mark.parametrize("model", ["qwen3_5", "granite"])
def test_hybrid_validate_rejects_what_the_kernels_cannot_read(model):
    """The hybrid engines hand raw pointers to the kernels, so their weight
    dicts are checked first: every declared name, shape and dtype."""
    from tilefoundry_amd.hybrid import granite as G
    from tilefoundry_amd.hybrid import qwen3_5 as Q

    if model == "qwen3_5":
        mod, cfg = Q, Q.Qwen35Config(hidden=64, layers=4, lin_key_heads=2, lin_value_heads=4,
                                     lin_key_dim=16, lin_value_dim=16, heads=4, kv_heads=2,
                                     head_dim=32, rot_dim=8, experts=8, top_k=2, moe_inter=32,
                                     shared_inter=48, vocab=96)
        victim = "layer3.w_in"                     # a full-attention layer's in-projection
    else:
        mod, cfg = G, G.GraniteConfig(hidden=64, layers=3, attention_layers=(1,), mamba_heads=4,
                                      mamba_head_dim=16, d_state=16, heads=4, kv_heads=2,
                                      head_dim=16, experts=6, top_k=2, moe_inter=32,
                                      shared_inter=48, vocab=96)
        victim = "layer0.s_down"                   # an expert block's row scales
    w = mod.synthetic_weights(cfg, seed=1, device="cpu")
    mod.validate(cfg, w)
    assert set(mod.declared_shapes(cfg)) == set(w)
    missing = dict(w)
    del missing[victim]
    with pytest.raises(KeyError, match=victim):
        mod.validate(cfg, missing)
    short = dict(w)
    short[victim] = w[victim][:-1]
    with pytest.raises(ValueError, match="shape"):
        mod.validate(cfg, short)
    retyped = dict(w)
    retyped[victim] = w[victim].to(torch.float16)
    with pytest.raises(ValueError, match="dtype"):
        mod.validate(cfg, retyped)
