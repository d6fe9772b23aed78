"""Decode steps at the workloads' full context depths, without walking them.

The oracle's ``forward`` takes the KV caches as arguments (ref_src/model.py:
307-317, 139-216), so a step at position P can be checked directly: the caches
of positions 0 .. P-1 are drawn at random, written into the engine's paged pool
through its page table (``place_context``), and one engine step is compared
with the oracle's forward over the same caches.

* C2: the batch-1 engine at positions near the end of the 2,048-token run
  (2,070 and 2,078) and on either side of 2,048 (where the XCD kernel's 32
  ranks per kv head go from one 64-position tile each to two), in both
  persistent kernels and in the per-phase graph, with the Qwen3-1.7B layer
  shape (two layers, a 4,096-token vocabulary so the CPU oracle runs in
  seconds).  The XCD kernel also at depths where a rank's split holds two,
  three and four tiles (up to its 8,192-position limit).
* C3: the batched engine at batch 32 over contexts of 4,000 .. 4,095 positions
  (ragged, the workload's depth), one layer at full width.

Bar: every sequence's logits within 2e-2 of max |logit| (the north-star bf16
bound), cosine >= 0.9999, and the greedy pick equal wherever the oracle's
top-2 margin exceeds twice the measured error.  The XCD kernel is held to the
oracle's exact-products arithmetic (its own) and to the HIR's rounded products
at the north-star bar (cosine >= 0.999 there: the two arithmetics are a bf16
rounding per product apart).
"""
import pytest
import torch

from oracle import qwen3_hir as O
from tests._parity import assert_close_bf16, oracle_arith
from tilefoundry_amd.qwen3 import QWEN3_1_7B, synthetic_weights
from tilefoundry_amd.qwen3.batch_engine import BatchEngine
from tilefoundry_amd.qwen3.engine import Engine

pytestmark = pytest.mark.gpu


def _dims(cfg):
    return O.Qwen3Dims(hidden=cfg.hidden_size, heads=cfg.num_attention_heads,
                       kv_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim,
                       intermediate=cfg.intermediate_size, vocab=cfg.vocab_size,
                       layers=cfg.num_hidden_layers, dtype=cfg.dtype)


def _caches(cfg, P, seed):
    g = torch.Generator().manual_seed(seed)
    shape = (P, cfg.num_key_value_heads, cfg.head_dim)
    ks = [torch.randn(shape, generator=g).to(torch.bfloat16) for _ in range(cfg.num_hidden_layers)]
    vs = [torch.randn(shape, generator=g).to(torch.bfloat16) for _ in range(cfg.num_hidden_layers)]
    return ks, vs


def _oracle_step(cfg, w, token, P, ks, vs):
    dims = _dims(cfg)
    orc = O.Qwen3Oracle(dims, w)
    cos, sin = O.generation_rope(dims, P + 1)
    scale = torch.full((1, 1, 1, 1), cfg.head_dim ** -0.5, dtype=torch.bfloat16)
    caches = tuple((k[None], v[None]) for k, v in zip(ks, vs))
    with torch.no_grad():
        logits, _ = orc.forward(torch.tensor([token]), cos, sin,
                                torch.tensor([P], dtype=torch.int32), scale, caches)
    return logits.float().reshape(-1)


def _check(got, want, name):
    r = assert_close_bf16(got, want, max_rel=2e-2, min_cos=0.9999, name=name)
    err = float((got - want).abs().max())
    top2 = torch.topk(want, 2).values
    if float(top2[0] - top2[1]) > 2 * err:
        assert int(got.argmax()) == int(want.argmax()), name
    return r


C2_SHAPE = QWEN3_1_7B.with_(num_hidden_layers=2, vocab_size=4096)


@pytest.fixture(scope="module")
def c2_weights():
    return synthetic_weights(C2_SHAPE, seed=3, norms="ones")


def _step_at_depth(device, cfg, w, mode, P, max_new=2048, prompt_room=64):
    print(f"[deep] c2 mode={mode} position={P}", flush=True)
    ks, vs = _caches(cfg, P, seed=P)
    token = 1234
    eng = Engine(cfg, w, device=device, max_new=max_new, prompt_room=prompt_room, mode=mode)
    eng.place_context(ks, vs, token)
    eng.run_steps(1)
    torch.cuda.synchronize()
    eng.check_errors()
    got = eng.logits.float().cpu()
    with oracle_arith(mode):
        want = _oracle_step(cfg, w, token, P, ks, vs)
    r = _check(got, want, f"c2 {mode} P={P}")
    print(f"  {r}", flush=True)
    if mode == "xcd":
        # the same step against the HIR's per-product rounding: the north-star
        # bar (the cosine floor of two arithmetics a rounding per product apart)
        hir = _oracle_step(cfg, w, token, P, ks, vs)
        rh = assert_close_bf16(got, hir, max_rel=2e-2, min_cos=0.999, name="vs the HIR")
        print(f"  vs the HIR's rounded products: {rh}", flush=True)
    # the step appended this token's K/V at position P and advanced the position
    assert int(eng.pos.item()) == P + 1


@pytest.mark.parametrize("mode", ["persistent", "xcd", "graph"])
@pytest.mark.parametrize("P", [2047, 2048, 2049, 2070, 2078])
def test_c2_step_at_depth(gpu_device, c2_weights, mode, P):
    _step_at_depth(gpu_device, C2_SHAPE, c2_weights, mode, P)


# tiles per rank's split: 4,095 two (the last such depth); 4,097 and 6,100
# three; 8,100 four (the engine's cache sized to 8,192 positions)
@pytest.mark.parametrize("P", [4095, 4097, 6100, 8100])
def test_c2_xcd_step_past_two_tiles_per_rank(gpu_device, c2_weights, P):
    _step_at_depth(gpu_device, C2_SHAPE, c2_weights, "xcd", P, max_new=8192 - 64)


def test_c3_batch32_step_at_4096_contexts(gpu_device):
    cfg = QWEN3_1_7B.with_(num_hidden_layers=1, vocab_size=4096)
    w = synthetic_weights(cfg, seed=4, norms="ones")
    B = 32
    lens = [4095 - 3 * b for b in range(B)]          # ragged: 4,002 .. 4,095 positions
    print(f"[deep] c3 batch {B} contexts {min(lens)}..{max(lens)}", flush=True)
    g = torch.Generator().manual_seed(77)
    tokens = torch.randint(0, cfg.vocab_size, (B,), generator=g).tolist()
    caches = [_caches(cfg, P, seed=1000 + b) for b, P in enumerate(lens)]
    eng = BatchEngine(cfg, w, batch=B, device=gpu_device, max_new=8, prompt_room=4096)
    eng.place_context([[caches[b][0][0] for b in range(B)]], [[caches[b][1][0] for b in range(B)]],
                      tokens)
    eng.run_steps(1)
    torch.cuda.synchronize()
    eng.check_errors()
    got = eng.logits.float().cpu()
    worst = 0.0
    for b in range(B):
        want = _oracle_step(cfg, w, tokens[b], lens[b], caches[b][0], caches[b][1])
        r = _check(got[b], want, f"c3 seq {b} P={lens[b]}")
        worst = max(worst, r["max_rel"])
    print(f"  worst max_rel over {B} sequences {worst:.4g}", flush=True)
    assert eng.pos.cpu().tolist() == [P + 1 for P in lens]
