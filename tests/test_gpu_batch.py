"""Batched decode (BASELINE config 3 path) on the GPU.

* The skinny GEMM against an f64 matmul of the same bf16 operands: every output
  is one f32 sum rounded once, so it lies within one bf16 ulp of the exact value
  plus the f32 accumulation bound, for every epilogue, for row counts 1..32 and
  column counts off the 16-wide tile.
* The batched engine against the oracle's single-sequence greedy loop, sequence
  by sequence, with prompts of different lengths (the device-side token feed
  per sequence), at config 1's shape in bf16 and at the Qwen3-1.7B layer shape.
* Page placement changes no bit.
"""
import pytest
import torch

from oracle import qwen3_hir as O
from tests._parity import report, ulp_bf16
from tests.test_gpu_engine import SMALL, _check_run, _dims, _prompt
from tilefoundry_amd import _lib
from tilefoundry_amd._lib import lib, ptr
from tilefoundry_amd.qwen3 import QWEN3_1_7B, synthetic_weights
from tilefoundry_amd.qwen3.batch_engine import BatchEngine

pytestmark = pytest.mark.gpu


def _gemm(x, w, epi, resid=None):
    M, K = x.shape
    N = w.shape[0]
    if epi == _lib.EPI_SWIGLU:
        out = torch.zeros(M, N // 2, device=x.device, dtype=torch.bfloat16)
    elif epi == _lib.EPI_LOGITS:
        out = torch.zeros(M, N, device=x.device, dtype=torch.float32)
    else:
        out = torch.zeros(M, N, device=x.device, dtype=torch.bfloat16)
    lib().tfd_gemm_skinny_bf16(ptr(x), K, ptr(w), M, K, N, epi,
                               None if resid is None else ptr(resid), N, ptr(out),
                               out.shape[1], torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("M", [1, 5, 16, 17, 32])
@pytest.mark.parametrize("K,N", [(2048, 48), (6144, 40), (64, 16), (2048, 2050)])
def test_skinny_gemm_within_one_ulp_of_exact(gpu_device, M, K, N):
    g = torch.Generator().manual_seed(M * 7919 + K + N)
    x = (torch.randn(M, K, generator=g) * 0.5).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    exact = x.double() @ w.double().t()                          # [M][N]
    want = exact.to(torch.bfloat16).float()
    got = _gemm(x.to(gpu_device), w.to(gpu_device), _lib.EPI_STORE).float()
    # one rounding of an f32 sum: within an ulp of the exact value plus the f32
    # accumulation bound K * 2^-24 * sum |x||w| (which matters only under cancellation)
    acc_bound = K * 2.0 ** -24 * (x.double().abs() @ w.double().abs().t())
    bound = ulp_bf16(want).double() + acc_bound
    bad = (got.double() - exact).abs() > bound
    assert not bad.any(), (int(bad.sum()), got[bad][:4], exact[bad][:4])
    # logits: the same rounding, returned as f32
    lg = _gemm(x.to(gpu_device), w.to(gpu_device), _lib.EPI_LOGITS)
    assert torch.equal(lg, got)
    # residual: bf16(resid + bf16(y))
    r = (torch.randn(M, N, generator=g)).to(torch.bfloat16)
    res = _gemm(x.to(gpu_device), w.to(gpu_device), _lib.EPI_RESID, r.to(gpu_device)).float()
    assert torch.equal(res, (r.float() + got).to(torch.bfloat16).float())
    # swiglu over (gate, up) row pairs, from the kernel's own rounded pair
    if N % 2 == 0:
        sw = _gemm(x.to(gpu_device), w.to(gpu_device), _lib.EPI_SWIGLU).float()
        gate, up = got[:, 0::2], got[:, 1::2]
        act = torch.nn.functional.silu(gate.to(torch.bfloat16)).float()
        want_sw = (act * up).to(torch.bfloat16).float()
        # silu's own f32 evaluation may differ from torch's by an ulp before rounding
        assert ((sw - want_sw).abs() <= ulp_bf16(want_sw)).all()


def _oracle_runs(cfg, w, prompts, max_new):
    return [O.decode(O.Qwen3Oracle(_dims(cfg), w), p, max_new) for p in prompts]


def test_batch_engine_small_bf16_matches_oracle(gpu_device):
    w = synthetic_weights(SMALL, seed=0, norms="ones")
    prompts = [_prompt(n, SMALL.vocab_size, seed=s) for n, s in ((6, 1), (9, 2), (4, 3))]
    eng = BatchEngine(SMALL, w, batch=3, device=gpu_device, max_new=24, prompt_room=9)
    run = eng.generate(prompts, 24, record_logits=True)
    for b, orc in enumerate(_oracle_runs(SMALL, w, prompts, 24)):
        seq = type("Run", (), {"tokens": run.tokens[b], "logits": run.logits[b]})
        _check_run(seq, orc, 24, strict=False)


def test_batch_engine_qwen3_layer_shape(gpu_device):
    cfg = QWEN3_1_7B.with_(num_hidden_layers=2)
    w = synthetic_weights(cfg, seed=0, norms="ones")
    prompts = [_prompt(8, cfg.vocab_size, seed=s) for s in range(4)]
    eng = BatchEngine(cfg, w, batch=4, device=gpu_device, max_new=16, prompt_room=8)
    run = eng.generate(prompts, 16, record_logits=True)
    for b, orc in enumerate(_oracle_runs(cfg, w, prompts, 16)):
        seq = type("Run", (), {"tokens": run.tokens[b], "logits": run.logits[b]})
        k = _check_run(seq, orc, 16, strict=False)
        print(f"sequence {b}: identical for {16 if k is None else k} of 16 steps")


def test_batch_engine_paging_and_graph_change_no_bit(gpu_device):
    w = synthetic_weights(SMALL, seed=5, norms="ones")
    prompts = [_prompt(n, SMALL.vocab_size, seed=9 + n) for n in (3, 7, 5, 5)]
    runs = []
    for page_seed, graph in ((None, True), (3, True), (11, False)):
        eng = BatchEngine(SMALL, w, batch=4, device=gpu_device, max_new=40, prompt_room=7,
                          page_seed=page_seed, graph=graph)
        runs.append(eng.generate(prompts, 40, record_logits=True))
    for r in runs[1:]:
        assert r.tokens == runs[0].tokens
        for a, b in zip(r.logits, runs[0].logits):
            assert torch.equal(a, b)


def test_batch_engine_rejects_bad_input(gpu_device):
    w = synthetic_weights(SMALL, seed=4, norms="ones")
    eng = BatchEngine(SMALL, w, batch=2, device=gpu_device, max_new=4, prompt_room=4,
                      graph=False)
    with pytest.raises(ValueError):
        eng.generate([[1, 2]], 4)                        # wrong batch
    with pytest.raises(ValueError):
        eng.generate([[1], [1, 2, 3, 4, 5]], 4)          # 5 + 4 > 8 steps
    with pytest.raises(ValueError):
        eng.generate([[1], [SMALL.vocab_size]], 2)       # id out of range
    with pytest.raises(ValueError):
        BatchEngine(SMALL, w, batch=33, device=gpu_device)
