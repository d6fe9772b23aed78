"""Batched prompt prefill (tilefoundry_amd/qwen3/prefill.py) on the GPU.

* The cache it fills equals the oracle's walked cache (model.py:339-352: k_rope and v
  of every prompt position, every layer) to the bf16 bar: the rows run through
  MFMA GEMMs whose f32 sums are ordered differently from the oracle's, so a
  rounding may land one bf16 ulp away.
* Greedy decoding after prefill matches the oracle's walk of the prompt: 64
  identical tokens on the config-1 shape (prompts of 40 and 71 tokens: two and
  three 32-row chunks; persistent and graph decoding), and the Qwen3-1.7B layer
  shape at two layers with the engine's usual near-tie rule (persistent and
  XCD decoding).
* The batch engine's prefill (one sequence at a time through its page-table row
  of the shared pool): every sequence's cache equals its own oracle walk, and
  the batched greedy continuation after prefill is each sequence's oracle
  continuation, prompts of different lengths (one of a single token) together.
"""
import types

import pytest
import torch

from oracle import qwen3_hir as O
from tests._parity import assert_close_bf16, oracle_arith
from tests.test_gpu_engine import SMALL, _check_run, _dims, _prompt
from tilefoundry_amd import _lib
from tilefoundry_amd.qwen3 import QWEN3_1_7B, synthetic_weights
from tilefoundry_amd.qwen3.batch_engine import BatchEngine
from tilefoundry_amd.qwen3.engine import Engine

pytestmark = pytest.mark.gpu


def _walk_caches(cfg, w, prompt):
    """The oracle's caches after consuming every token of the prompt but the last."""
    orc = O.Qwen3Oracle(_dims(cfg), w)
    caches = orc.init_caches()
    ids = torch.tensor(prompt, dtype=torch.int64)
    with torch.no_grad():
        for step in range(len(prompt) - 1):
            args = orc.prepare_inputs_for_generation(ids, step, caches)
            _, fresh = orc.forward(*args)
            caches = orc.append_cache(caches, fresh)
    return caches


def _engine_cache(eng, layer, n):
    """Rows 0 .. n-1 of one layer's K and V cache, [n][HKV][D]."""
    p = torch.arange(n, device=eng.device)
    page = eng.page_table.long()[p // _lib.PAGE_SIZE]
    row = p % _lib.PAGE_SIZE
    return eng.kpool[layer][page, :, row].float().cpu(), eng.vpool[layer][page, :, row].float().cpu()


@pytest.mark.parametrize("n", [5, 40])
def test_prefill_cache_matches_the_oracle_walk(gpu_device, n):
    w = synthetic_weights(SMALL, seed=1, norms="random")
    prompt = _prompt(n, SMALL.vocab_size, seed=n)
    want = _walk_caches(SMALL, w, prompt)
    eng = Engine(SMALL, w, device=gpu_device, max_new=8, prompt_room=n)
    eng.prefill(prompt)
    eng.check_errors()
    assert int(eng.pos.item()) == n - 1 and int(eng.ids.item()) == prompt[-1]
    for i, (kc, vc) in enumerate(want):
        k, v = _engine_cache(eng, i, n - 1)
        assert_close_bf16(k, kc[0], max_rel=2e-2, min_exact=0.95, name=f"layer {i} k")
        assert_close_bf16(v, vc[0], max_rel=2e-2, min_exact=0.95, name=f"layer {i} v")


@pytest.mark.parametrize("mode,n", [("persistent", 40), ("graph", 71)])
def test_prefill_then_greedy_64_matches_the_oracle(gpu_device, mode, n):
    w = synthetic_weights(SMALL, seed=0, norms="ones")
    prompt = _prompt(n, SMALL.vocab_size, seed=1)
    orc = O.decode(O.Qwen3Oracle(_dims(SMALL), w), prompt, 64)
    eng = Engine(SMALL, w, device=gpu_device, max_new=64, prompt_room=n, mode=mode)
    run = eng.generate(prompt, 64, record_logits=True, prefill=True)
    eng.check_errors()
    _check_run(run, orc, 64)


@pytest.mark.parametrize("mode", ["persistent", "xcd"])
def test_prefill_at_the_layer_shape(gpu_device, mode):
    """Two layers of the Qwen3-1.7B shape, a 70-token prompt (three chunks): the
    continuation tracks the oracle's walk as decoding does (logits within the
    bar, a divergence only at a near-tie the measured error explains), and the
    engine's own walk of the prompt gives the same logits to the bf16 bar until
    the two runs first pick differently."""
    cfg = QWEN3_1_7B.with_(num_hidden_layers=2)
    w = synthetic_weights(cfg, seed=0, norms="ones")
    prompt = _prompt(70, cfg.vocab_size, seed=2)
    with oracle_arith(mode):
        orc = O.decode(O.Qwen3Oracle(_dims(cfg), w), prompt, 32)
    eng = Engine(cfg, w, device=gpu_device, max_new=32, prompt_room=70, mode=mode)
    run = eng.generate(prompt, 32, record_logits=True, prefill=True)
    eng.check_errors()
    k = _check_run(run, orc, 32, strict=False)
    print(f"{mode}: after prefill, free-running identical for {32 if k is None else k} steps; "
          f"prefill {1e3 * run.prefill_seconds:.1f} ms")
    walked = eng.generate(prompt, 32, record_logits=True)
    kw = next((j for j, (a, b) in enumerate(zip(walked.tokens, run.tokens)) if a != b), None)
    upto = 32 if kw is None else kw + 1
    for j in range(upto):
        assert_close_bf16(run.logits[j], walked.logits[j], max_rel=2e-2, name=f"step {j}")


def _batch_cache(eng, layer, b, n):
    """Rows 0 .. n-1 of sequence b's K and V cache in one layer, [n][HKV][D]."""
    p = torch.arange(n, device=eng.device)
    page = eng.page_table[b].long()[p // _lib.PAGE_SIZE]
    row = p % _lib.PAGE_SIZE
    return eng.kpool[layer][page, :, row].float().cpu(), eng.vpool[layer][page, :, row].float().cpu()


# room 4,096: the prefill's score rows are an allocation of megabytes, whose
# first row is sequence 0's at position 0 -- a split with no prior position,
# which still prefetches its next tile's scores from inside that row
@pytest.mark.parametrize("room", [72, 4096])
def test_batch_prefill_caches_match_the_oracle_walks(gpu_device, room):
    w = synthetic_weights(SMALL, seed=1, norms="random")
    lens = [5, 40, 71]
    prompts = [_prompt(n, SMALL.vocab_size, seed=10 + n) for n in lens]
    eng = BatchEngine(SMALL, w, batch=3, device=gpu_device, max_new=8, prompt_room=room)
    eng.prefill(prompts)
    eng.check_errors()
    assert eng.pos.tolist() == [n - 1 for n in lens]
    assert eng.ids.tolist() == [p[-1] for p in prompts]
    for b, p in enumerate(prompts):
        for i, (kc, vc) in enumerate(_walk_caches(SMALL, w, p)):
            k, v = _batch_cache(eng, i, b, len(p) - 1)
            assert_close_bf16(k, kc[0], max_rel=2e-2, min_exact=0.95, name=f"seq {b} layer {i} k")
            assert_close_bf16(v, vc[0], max_rel=2e-2, min_exact=0.95, name=f"seq {b} layer {i} v")


def test_batch_prefill_then_greedy_matches_the_oracle(gpu_device):
    """Four sequences (prompts of 40, 71, 9 and 1 tokens) prefilled, then 32
    batched greedy steps: each sequence's continuation tracks its oracle walk
    (logits within the bar, a divergence only at a near-tie the measured error
    explains), and so does the engine's own walk of the same prompts."""
    w = synthetic_weights(SMALL, seed=0, norms="ones")
    lens = [40, 71, 9, 1]
    prompts = [_prompt(n, SMALL.vocab_size, seed=20 + n) for n in lens]
    eng = BatchEngine(SMALL, w, batch=4, device=gpu_device, max_new=32, prompt_room=72)
    run = eng.generate(prompts, 32, record_logits=True, prefill=True)
    eng.check_errors()
    assert run.steps == 32
    walked = eng.generate(prompts, 32, record_logits=True)
    for b, p in enumerate(prompts):
        orc = O.decode(O.Qwen3Oracle(_dims(SMALL), w), p, 32)
        for name, r in (("prefill", run), ("walk", walked)):
            k = _check_run(types.SimpleNamespace(tokens=r.tokens[b], logits=r.logits[b]), orc, 32,
                           strict=False)
            print(f"sequence {b} ({len(p)}-token prompt), {name}: identical to the oracle for "
                  f"{32 if k is None else k} of 32 steps", flush=True)
