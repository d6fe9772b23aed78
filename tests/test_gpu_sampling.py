"""tfd_sample_rows on the GPU against the CPU restatement (oracle/sampling.py).

* top-k path (run.py:145-180): rows of random logits at the workloads' vocabulary
  sizes and rows full of ties, k 1..64, temperatures and nuclei; every pick equal
  to the oracle's given the same uniform, except a draw whose uniform lies within
  float32 rounding of a cumulative boundary (counted, at most 1%);
* Gumbel path (granite.cu:716-800): picks equal to the oracle's except where the
  best two perturbed values are within rounding of each other;
* distribution: 4,096 rows of the same logits give the softmax frequencies;
* the counter is read on the device: a captured graph draws anew when it moves;
* refusals.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import sampling as S
from tilefoundry_amd import _lib
from tilefoundry_amd._lib import TFDError, lib, ptr

pytestmark = pytest.mark.gpu


def _sample(logits, *, temperature, top_k, top_p, seed, counter, ldl=None):
    rows, V = logits.shape[0], logits.shape[1]
    ldl = ldl or logits.stride(0)
    sp = _lib.TfdSampling(temperature, top_k, top_p, seed)
    nbytes = lib().tfd_sample_work_bytes(rows, V, top_k)
    work = torch.empty(max(nbytes, 8), dtype=torch.uint8, device=logits.device)
    pick = torch.full((rows,), -1, dtype=torch.int32, device=logits.device)
    lib().tfd_sample_rows(ptr(logits), ldl, rows, V, ctypes.byref(sp), ptr(counter), ptr(pick),
                          ptr(work), nbytes, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return pick.cpu().tolist()


@pytest.mark.parametrize("V,rows", [(1000, 3), (4096, 32), (151936, 4), (248320, 2)])
@pytest.mark.parametrize("top_k,temperature,top_p", [(1, 1.0, 1.0), (20, 1.0, 0.95),
                                                     (64, 0.6, 1.0), (7, 1.7, 0.5)])
def test_topk_picks_equal_the_oracle(gpu_device, V, rows, top_k, temperature, top_p):
    g = torch.Generator().manual_seed(V + top_k)
    logits = (torch.randn(rows, V, generator=g) * 3).to(gpu_device)
    host = logits.cpu().numpy()
    seed = 12345 + top_k
    skipped = checked = 0
    for rep in range(6):
        ctr = torch.randint(0, 1 << 20, (rows,), generator=g, dtype=torch.int32)
        got = _sample(logits, temperature=temperature, top_k=top_k, top_p=top_p, seed=seed,
                      counter=ctr.to(gpu_device))
        for r in range(rows):
            u = S.draw_uniform(seed, r, int(ctr[r]))
            want, dist = S.sample_topk(host[r], temperature, top_k, top_p, u)
            if dist < 1e-5:
                skipped += 1
                continue
            checked += 1
            assert got[r] == want, (V, r, rep, got[r], want, dist)
    assert skipped <= max(1, 0.01 * (checked + skipped)), (skipped, checked)


def test_topk_ties_go_to_the_lower_index(gpu_device):
    """Rows of few distinct values: which of the tied logits enter the top k is
    the lower-index rule; top_k 1 is the argmax (the first maximum)."""
    g = torch.Generator().manual_seed(3)
    rows, V = 8, 50000
    logits = torch.randint(-2, 3, (rows, V), generator=g).float()
    logits[0, :] = 1.0                                   # every logit tied
    logits[1, 7] = float("nan")
    logits[2, :] = float("nan")                          # all NaN: picks 0
    logits[3, :100] = -0.0
    logits[3, 100:] = -1.0                               # -0 ties +0: the first index
    dev = logits.to(gpu_device)
    host = logits.numpy()
    ctr = torch.arange(rows, dtype=torch.int32)
    got1 = _sample(dev, temperature=1.0, top_k=1, top_p=1.0, seed=1, counter=ctr.to(gpu_device))
    for r in range(rows):
        assert got1[r] == S.sample_topk(host[r], 1.0, 1, 1.0, np.float32(0.5))[0], r
    assert got1[0] == 0 and got1[2] == 0 and got1[3] == 0
    got = _sample(dev, temperature=1.0, top_k=64, top_p=1.0, seed=9, counter=ctr.to(gpu_device))
    for r in range(rows):
        want, dist = S.sample_topk(host[r], 1.0, 64, 1.0, S.draw_uniform(9, r, r))
        assert dist < 1e-5 or got[r] == want, (r, got[r], want)
        assert got[r] in S.topk_indices(host[r], 64).tolist()


@pytest.mark.parametrize("V,temperature", [(4096, 1.0), (151936, 0.7), (248320, 1.3)])
def test_gumbel_picks_equal_the_oracle(gpu_device, V, temperature):
    g = torch.Generator().manual_seed(V)
    rows = 6
    logits = (torch.randn(rows, V, generator=g) * 4).to(gpu_device)
    host = logits.cpu().numpy()
    ctr = torch.randint(0, 1 << 20, (rows,), generator=g, dtype=torch.int32)
    got = _sample(logits, temperature=temperature, top_k=0, top_p=1.0, seed=77,
                  counter=ctr.to(gpu_device))
    near = 0
    for r in range(rows):
        want, margin = S.sample_gumbel(host[r], temperature, 77, r, int(ctr[r]))
        if margin < 1e-5:
            near += 1
            continue
        assert got[r] == want, (r, got[r], want, margin)
    assert near <= 1


@pytest.mark.parametrize("top_k", [0, 8])
def test_draws_follow_the_softmax(gpu_device, top_k):
    """4,096 rows of the same 8 logits (each row its own random numbers): the
    picks' frequencies are softmax(v / T) over the row (top_k 0) or over its
    top 8 (the whole row here)."""
    row = torch.tensor([0.0, 1.0, -0.5, 2.0, 0.3, -3.0, 1.5, 0.9])
    rows, T = 4096, 0.8
    logits = row.repeat(rows, 1).to(gpu_device)
    got = _sample(logits, temperature=T, top_k=top_k, top_p=1.0, seed=2024,
                  counter=torch.zeros(rows, dtype=torch.int32, device=gpu_device))
    freq = np.bincount(got, minlength=8) / rows
    want = torch.softmax(row / T, 0).numpy()
    assert np.abs(freq - want).max() < 0.03, (freq, want)


def test_a_captured_sample_draws_anew_when_the_counter_moves(gpu_device):
    rows, V = 4, 4096
    g = torch.Generator().manual_seed(5)
    logits = torch.randn(rows, V, generator=g).to(gpu_device) * 0.1     # flat: many outcomes
    ctr = torch.zeros(rows, dtype=torch.int32, device=gpu_device)
    sp = _lib.TfdSampling(1.0, 0, 1.0, 99)
    nbytes = lib().tfd_sample_work_bytes(rows, V, 0)
    work = torch.empty(nbytes, dtype=torch.uint8, device=gpu_device)
    pick = torch.zeros(rows, dtype=torch.int32, device=gpu_device)
    s = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        lib().tfd_sample_rows(ptr(logits), V, rows, V, ctypes.byref(sp), ptr(ctr), ptr(pick),
                              ptr(work), nbytes, torch.cuda.current_stream().cuda_stream)
    seen = []
    for step in range(4):
        ctr.fill_(step)
        graph.replay()
        torch.cuda.synchronize()
        seen.append(pick.cpu().tolist())
        want = [S.sample_gumbel(logits[r].cpu().numpy(), 1.0, 99, r, step)[0] for r in range(rows)]
        assert seen[-1] == want, (step, seen[-1], want)
    assert len({tuple(x) for x in seen}) > 1
    ctr.fill_(2)
    graph.replay()
    torch.cuda.synchronize()
    assert pick.cpu().tolist() == seen[2]


def test_sample_rows_refuses_bad_arguments(gpu_device):
    logits = torch.zeros(2, 100, device=gpu_device)
    ctr = torch.zeros(2, dtype=torch.int32, device=gpu_device)
    for kw in ({"temperature": 0.0, "top_k": 5, "top_p": 1.0},
               {"temperature": 1.0, "top_k": 65, "top_p": 1.0},
               {"temperature": 1.0, "top_k": 5, "top_p": 0.0},
               {"temperature": 1.0, "top_k": 0, "top_p": 0.9}):
        with pytest.raises(TFDError):
            _sample(logits, seed=0, counter=ctr, **kw)
    sp = _lib.TfdSampling(1.0, 5, 1.0, 0)
    pick = torch.zeros(2, dtype=torch.int32, device=gpu_device)
    work = torch.empty(16, dtype=torch.uint8, device=gpu_device)
    with pytest.raises(TFDError, match="needed"):
        lib().tfd_sample_rows(ptr(logits), 100, 2, 100, ctypes.byref(sp), ptr(ctr), ptr(pick),
                              ptr(work), 16, torch.cuda.current_stream().cuda_stream)
    big = torch.zeros(1, _lib.SAMPLE_MAX_VOCAB + 1, device=gpu_device)
    with pytest.raises(TFDError):
        _sample(big, temperature=1.0, top_k=5, top_p=1.0, seed=0, counter=ctr)


# ---------------------------------------------------------------- engines
def _check_engine_draws(tokens, logits_at, prompts, sp, steps):
    """Every sampled token is the oracle's draw on that step's logits, with the
    sequence's position as the counter; draws within rounding of a boundary
    are counted, not compared."""
    near = 0
    for b, p in enumerate(prompts):
        for j in range(steps):
            ctr = len(p) - 1 + j
            row = logits_at(b, j).numpy()
            if sp.top_k == 0:
                want, gap = S.sample_gumbel(row, sp.temperature, sp.seed, b, ctr)
            else:
                want, gap = S.sample_topk(row, sp.temperature, sp.top_k, sp.top_p,
                                          S.draw_uniform(sp.seed, b, ctr))
            if gap < 1e-5:
                near += 1
                continue
            assert tokens[b][j] == want, (b, j, tokens[b][j], want)
    assert near <= 2, near


def test_batch_engine_samples(gpu_device):
    """BatchEngine (the bf16 config-1 shape, three prompts of different lengths):
    top_k 1 is greedy token for token; a seeded run repeats and another seed
    differs; every token is the oracle's draw on the recorded logits."""
    from tests.test_gpu_engine import SMALL, _prompt
    from tilefoundry_amd.qwen3 import synthetic_weights
    from tilefoundry_amd.qwen3.batch_engine import BatchEngine
    from tilefoundry_amd.sampling import Sampling

    w = synthetic_weights(SMALL, seed=0, norms="ones")
    prompts = [_prompt(n, SMALL.vocab_size, seed=s) for n, s in ((6, 1), (9, 2), (4, 3))]

    def run(sampling, record=False):
        eng = BatchEngine(SMALL, w, batch=3, device=gpu_device, max_new=24, prompt_room=9,
                          sampling=sampling)
        return eng.generate(prompts, 24, record_logits=record)

    greedy = run(None)
    assert run(Sampling(temperature=0.7, top_k=1, seed=5)).tokens == greedy.tokens
    sp = Sampling(temperature=1.0, top_k=20, top_p=0.95, seed=11)
    first = run(sp, record=True)
    assert run(sp).tokens == first.tokens
    assert run(Sampling(temperature=1.0, top_k=20, top_p=0.95, seed=12)).tokens != first.tokens
    assert first.tokens != greedy.tokens
    _check_engine_draws(first.tokens, lambda b, j: first.logits[b][j], prompts, sp, 24)


def test_hybrid_engines_sample(gpu_device):
    """GraniteEngine with Granite's sampler (softmax over the whole vocabulary at a
    temperature) and Qwen35Engine with run.py's (top 8, nucleus 0.9): every token
    the oracle's draw on the recorded logits."""
    from tilefoundry_amd.hybrid import granite as G
    from tilefoundry_amd.hybrid import qwen3_5 as Q
    from tilefoundry_amd.sampling import Sampling

    g = torch.Generator().manual_seed(8)
    prompts = [torch.randint(0, 4096, (3 + b,), generator=g).tolist() for b in range(2)]
    cfg = G.GraniteConfig(layers=3, attention_layers=(1,), experts=12, top_k=4, vocab=4096)
    sp = Sampling(temperature=0.8, top_k=0, seed=21)
    eng = G.GraniteEngine(cfg, G.synthetic_weights(cfg, seed=5, device=gpu_device), rows=2,
                          device=gpu_device, max_steps=64, split_len=16, sampling=sp)
    tokens, _, hist = eng.generate(prompts, 8, record_logits=True)
    _check_engine_draws(tokens, lambda b, j: hist[len(prompts[b]) - 1 + j][b], prompts, sp, 8)

    cfg = Q.Qwen35Config(layers=4, experts=16, vocab=4096)
    sp = Sampling(temperature=1.2, top_k=8, top_p=0.9, seed=4)
    eng = Q.Qwen35Engine(cfg, Q.synthetic_weights(cfg, seed=3, device=gpu_device), rows=2,
                         device=gpu_device, max_steps=64, split_len=16, sampling=sp)
    tokens, _, hist = eng.generate(prompts, 8, record_logits=True)
    _check_engine_draws(tokens, lambda b, j: hist[len(prompts[b]) - 1 + j][b], prompts, sp, 8)
