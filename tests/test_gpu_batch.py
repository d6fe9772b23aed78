"""Batched decode (workload C3) on the GPU.

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


def _packed(w):
    N, K = w.shape
    out = torch.full((-(-N // 16) * 16, K), float("nan"), device=w.device, dtype=w.dtype)
    lib().tfd_pack_skinny_bf16(ptr(w), K, N, K, ptr(out), torch.cuda.current_stream().cuda_stream)
    return out


def operand_order(x):
    """[M][K] rows (M <= 32) -> the batched path's operand-order layout (flat, 32 x K;
    rows past M hold NaN: they may only reach output rows that are not stored)."""
    M, K = x.shape
    full = torch.full((32, K), float("nan"), dtype=x.dtype, device=x.device)
    full[:M] = x
    return full.view(2, 16, K // 32, 4, 8).permute(2, 0, 3, 1, 4).reshape(-1).contiguous()


def from_operand_order(flat, M, K):
    """Inverse of operand_order (the first M rows)."""
    return flat.view(K // 32, 2, 4, 16, 8).permute(1, 3, 0, 2, 4).reshape(32, K)[:M]


def _gemm(x, w, epi, resid=None, work=None):
    M, K = x.shape
    N = w.shape[0]
    w = _packed(w)
    if epi == _lib.EPI_SWIGLU:
        out = torch.full((32 * (N // 2),), float("nan"), device=x.device, dtype=torch.bfloat16)
    elif epi in (_lib.EPI_LOGITS, _lib.EPI_RESID_F32):
        out = torch.zeros(M, N, device=x.device, dtype=torch.float32)
    else:
        out = torch.zeros(M, N, device=x.device, dtype=torch.bfloat16)
    xo = operand_order(x)                       # held: see the fp8 twin in test_gpu_hybrid
    lib().tfd_gemm_skinny_bf16(ptr(xo), ptr(w), M, K, N, epi,
                               None if resid is None else ptr(resid), N, ptr(out),
                               N, None if work is None else ptr(work),
                               0 if work is None else work.numel(),
                               torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    if epi == _lib.EPI_SWIGLU:
        return from_operand_order(out, M, N // 2).cpu()
    return out.cpu()


@pytest.mark.parametrize("split", [False, True], ids=["one-slice", "split-k"])
@pytest.mark.parametrize("M", [1, 5, 16, 17, 32])
@pytest.mark.parametrize("K,N", [(2048, 64), (6144, 40), (256, 16), (768, 128), (2048, 2050),
                                 (2048, 4200), (2048, 16448)])
def test_skinny_gemm_within_one_ulp_of_exact(gpu_device, M, K, N, split):
    """With a work buffer the library splits K into slices (8 for most shapes
    here, 4 at N = 4200) whose partial tiles the last-arriving wave adds in
    slice order; without one, K up to 2048 runs in one slice and a deeper K is
    refused (it does not fit the LDS stage)."""
    g = torch.Generator().manual_seed(M * 7919 + K + N)
    tiles = (N + 15) // 16
    work = (torch.zeros(_lib.SKINNY_COUNTERS + 16 * tiles * 512, device=gpu_device,
                        dtype=torch.float32) if split else None)
    x = (torch.randn(M, K, generator=g) * 0.5).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    exact = x.double() @ w.double().t()                          # [M][N]
    want = exact.to(torch.bfloat16).float()
    got = _gemm(x.to(gpu_device), w.to(gpu_device), _lib.EPI_STORE, work=work).float()
    # one rounding of an f32 sum: within an ulp of the exact value plus the f32
    # accumulation bound K * 2^-24 * sum |x||w| (which matters only under cancellation)
    acc_bound = K * 2.0 ** -24 * (x.double().abs() @ w.double().abs().t())
    bound = ulp_bf16(want).double() + acc_bound
    bad = (got.double() - exact).abs() > bound
    assert not bad.any(), (int(bad.sum()), got[bad][:4], exact[bad][:4])
    # logits: the same rounding, returned as f32
    lg = _gemm(x.to(gpu_device), w.to(gpu_device), _lib.EPI_LOGITS, work=work)
    assert torch.equal(lg, got)
    # residual: bf16(resid + bf16(y))
    r = (torch.randn(M, N, generator=g)).to(torch.bfloat16)
    res = _gemm(x.to(gpu_device), w.to(gpu_device), _lib.EPI_RESID, r.to(gpu_device),
                work=work).float()
    assert torch.equal(res, (r.float() + got).to(torch.bfloat16).float())
    # f32 residual stream: out = resid + bf16-valued product, in f32
    r32 = torch.randn(M, N, generator=g)
    res32 = _gemm(x.to(gpu_device), w.to(gpu_device), _lib.EPI_RESID_F32, r32.to(gpu_device),
                  work=work)
    assert torch.equal(res32, r32 + got)
    # swiglu over (gate, up) row pairs, from the kernel's own rounded pair
    if N % 64 == 0:
        sw = _gemm(x.to(gpu_device), w.to(gpu_device), _lib.EPI_SWIGLU, work=work).float()
        gate, up = got[:, 0::2], got[:, 1::2]
        act = torch.nn.functional.silu(gate.to(torch.bfloat16)).float()
        want_sw = (act * up).to(torch.bfloat16).float()
        # silu's own f32 evaluation may differ from torch's by an ulp before rounding
        assert ((sw - want_sw).abs() <= ulp_bf16(want_sw)).all()
    if work is not None:
        # every call leaves the tile counters at zero for the next one
        assert not work[:tiles].any()


def test_pack_skinny_layout(gpu_device):
    """The packed layout, element by element: block (tile t, step s) is 1 KiB and
    lane l's 8 values are W[16t + l % 16][32s + 8(l // 16) + j]; padding rows are 0."""
    N, K = 40, 512
    w = torch.arange(N * K, dtype=torch.float32).remainder(251).to(torch.bfloat16)
    w = w.view(N, K).to(gpu_device)
    got = _packed(w).cpu().view(-1, 64, 8)                         # [block][lane][j]
    tiles, steps = -(-N // 16), K // 32
    wp = torch.cat([w.cpu(), torch.zeros(tiles * 16 - N, K, dtype=w.dtype)])
    want = wp.view(tiles, 16, steps, 4, 8).permute(0, 2, 3, 1, 4).reshape(-1, 64, 8)
    assert torch.equal(got, want)


@pytest.mark.parametrize("rows", [1, 7, 32])
def test_rmsnorm_rows_operand_order(gpu_device, rows):
    """The operand-order output of the row norm holds the row-major output's bits."""
    g = torch.Generator().manual_seed(rows)
    H = 2048
    x = torch.randn(rows, H, generator=g).to(torch.bfloat16).to(gpu_device)
    gamma = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16).to(gpu_device)
    flat = torch.zeros(rows, H, dtype=torch.bfloat16, device=gpu_device)
    packed = torch.full((32 * H,), float("nan"), dtype=torch.bfloat16, device=gpu_device)
    s = torch.cuda.current_stream().cuda_stream
    lib().tfd_rmsnorm_rows_bf16(ptr(x), H, ptr(gamma), ptr(flat), H, rows, H, 1e-6, 0, s)
    lib().tfd_rmsnorm_rows_bf16(ptr(x), H, ptr(gamma), ptr(packed), 0, rows, H, 1e-6, 1, s)
    torch.cuda.synchronize()
    assert torch.equal(from_operand_order(packed, rows, H), flat)


@pytest.mark.parametrize("two_stage", [False, True], ids=["one-block", "chunked"])
def test_argmax_rows_first_maximum(gpu_device, two_stage):
    """The first maximal logit of each row, as torch.argmax picks it, with ties
    placed across chunk boundaries, a row of equal values, a NaN-only row (pick
    0) and NaNs beside the maximum."""
    g = torch.Generator().manual_seed(3)
    rows, V = 7, 151936
    x = torch.randn(rows, V, generator=g).to(torch.bfloat16).float()
    x[1, [5, 2374, 2375, 100000]] = 9.0            # ties: the first wins
    x[2] = 0.5                                     # all equal: index 0
    x[3] = float("nan")                            # no pick: 0
    x[4, 77] = float("nan")
    x[4, 150000] = 7.0
    x[5, V - 1] = 50.0                             # the last column
    want = torch.nan_to_num(x, nan=-float("inf")).argmax(dim=1).to(torch.int32)
    want[3] = 0
    xd = x.to(gpu_device)
    pick = torch.zeros(rows, dtype=torch.int32, device=gpu_device)
    work = torch.zeros(rows * _lib.ARGMAX_WORK, dtype=torch.int32, device=gpu_device)
    lib().tfd_argmax_rows(ptr(xd), V, rows, V, ptr(pick), ptr(work) if two_stage else None,
                          torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(pick.cpu(), want), (pick.cpu(), want)


def test_skinny_gemm_shapes_share_one_work_buffer(gpu_device):
    """GEMMs of different tile counts and slice counts in a row on one work
    buffer (the layer's q/k/v, o, gate/up and down) give the bits each gives on
    a fresh buffer: the counters sit at a fixed place and are left at zero."""
    g = torch.Generator().manual_seed(99)
    M = 32
    shapes = [(2048, 4096, _lib.EPI_STORE), (2048, 2048, _lib.EPI_STORE),
              (2048, 12288, _lib.EPI_SWIGLU), (6144, 2048, _lib.EPI_STORE)] * 2
    big = torch.zeros(1 << 21, device=gpu_device, dtype=torch.float32)
    for K, N, epi in shapes:
        x = (torch.randn(M, K, generator=g) * 0.5).to(torch.bfloat16).to(gpu_device)
        w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(gpu_device)
        shared = _gemm(x, w, epi, work=big)
        fresh = _gemm(x, w, epi, work=torch.zeros_like(big))
        assert torch.equal(shared, fresh), (K, N)
    assert not big[:_lib.SKINNY_COUNTERS].any()


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


@pytest.fixture(scope="module")
def long_split_case():
    """Weights, prompts and the oracle's runs of the long-split tests, computed
    once for all their partitions (the oracle decodes on its own)."""
    cfg = QWEN3_1_7B.with_(num_hidden_layers=2)
    w = synthetic_weights(cfg, seed=1, norms="ones")
    prompts = [_prompt(n, cfg.vocab_size, seed=20 + n) for n in (230, 150, 400)]
    return cfg, w, prompts, _oracle_runs(cfg, w, prompts, 8)


@pytest.mark.parametrize("split_tiles,splits", [(1, None), (2, None), (3, None), (4, None),
                                               (8, None), (None, None), (None, 1), (None, 2),
                                               (None, 3), (None, 7)])
def test_batch_engine_long_splits(gpu_device, long_split_case, split_tiles, splits):
    """Splits of several 64-position tiles (the long-context partition) against
    the oracle, with contexts past several splits: fixed split lengths, and
    lengths derived from each sequence's position over 1, 2, 3, 7 (one per
    tile of the cache, so the last splits are empty) or the default number of
    splits."""
    cfg, w, prompts, oracle_runs = long_split_case
    eng = BatchEngine(cfg, w, batch=3, device=gpu_device, max_new=8, prompt_room=400,
                      split_tiles=split_tiles, splits=splits)
    run = eng.generate(prompts, 8, record_logits=True)
    for b, orc in enumerate(oracle_runs):
        seq = type("Run", (), {"tokens": run.tokens[b], "logits": run.logits[b]})
        _check_run(seq, orc, 8, strict=False)


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
