"""tfd_gemm_skinny_bf16_noalloc (the skinny GEMM whose K-split work lives in the
library's own per-device scratch array) against tfd_gemm_skinny_bf16 with a
caller's work buffer of the same size: the same plan, so the same bits.  Calls
run back to back on the shared scratch, the second smaller than the first and
so on, over both kernels, so a later call sees the scratch as the earlier one
left it."""
import pytest
import torch

from tests.test_gpu_batch import _packed, from_operand_order, operand_order
from tilefoundry_amd import _lib
from tilefoundry_amd._lib import lib, ptr

pytestmark = pytest.mark.gpu


def _out(M, N, epi, dev):
    if epi == _lib.EPI_SWIGLU:
        return torch.full((32 * (N // 2),), float("nan"), device=dev, dtype=torch.bfloat16)
    if epi == _lib.EPI_LOGITS:
        return torch.zeros(M, N, device=dev, dtype=torch.float32)
    return torch.zeros(M, N, device=dev, dtype=torch.bfloat16)


def _run(M, K, N, epi, seed, dev):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(M, K, generator=g) * 0.5).to(torch.bfloat16).to(dev)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    r = torch.randn(M, N, generator=g).to(torch.bfloat16).to(dev)
    wp, xo = _packed(w), operand_order(x)
    resid = r if epi == _lib.EPI_RESID else None
    work = torch.zeros(_lib.NOALLOC_SCRATCH_FLOATS, device=dev, dtype=torch.float32)
    want, got = _out(M, N, epi, dev), _out(M, N, epi, dev)
    s = torch.cuda.current_stream().cuda_stream
    L = lib()
    L.tfd_gemm_skinny_bf16(ptr(xo), ptr(wp), M, K, N, epi,
                                None if resid is None else ptr(resid), N, ptr(want), N,
                                ptr(work), work.numel(), s)
    L.tfd_gemm_skinny_bf16_noalloc(ptr(xo), ptr(wp), M, K, N, epi,
                                        None if resid is None else ptr(resid), N, ptr(got), N, s)
    torch.cuda.synchronize()
    if epi == _lib.EPI_SWIGLU:
        want, got = from_operand_order(want, M, N // 2), from_operand_order(got, M, N // 2)
    assert torch.equal(got, want), (M, K, N, epi)
    assert got.float().abs().sum() > 0
    return got


# (M, K, N, epilogue), each call smaller than the one before it: the K-split
# kernel splitting across blocks (o / down shapes, the scratch's counters and
# partials in use), the X-stationary kernel (16,448 columns: no scratch), then
# smaller K-split shapes down to one tile
CALLS = [(32, 6144, 2048, _lib.EPI_RESID), (5, 2048, 1024, _lib.EPI_STORE),
         (32, 2048, 16448, _lib.EPI_LOGITS), (17, 2048, 12288, _lib.EPI_SWIGLU),
         (3, 1024, 2050, _lib.EPI_STORE), (1, 256, 16, _lib.EPI_STORE)]


def test_noalloc_gemm_matches_the_work_buffer_entry(gpu_device):
    for i, (M, K, N, epi) in enumerate(CALLS):
        print(f"[noalloc] call {i}: M={M} K={K} N={N} epi={epi}", flush=True)
        _run(M, K, N, epi, seed=100 + i, dev=gpu_device)


def test_noalloc_gemm_rejects_bad_shapes(gpu_device):
    L = lib()
    dummy = torch.zeros(16, device=gpu_device)
    s = torch.cuda.current_stream().cuda_stream
    with pytest.raises(_lib.TFDError, match="M=33"):
        L.tfd_gemm_skinny_bf16_noalloc(ptr(dummy), ptr(dummy), 33, 256, 16, _lib.EPI_STORE,
                                       None, 0, ptr(dummy), 16, s)
    with pytest.raises(_lib.TFDError, match="K=100"):
        L.tfd_gemm_skinny_bf16_noalloc(ptr(dummy), ptr(dummy), 4, 100, 16, _lib.EPI_STORE,
                                       None, 0, ptr(dummy), 16, s)


def test_noalloc_gemm_replays_in_a_captured_graph(gpu_device):
    """The entry enqueues nothing but the GEMM, so a graph captured around it
    replays it; the K-split counters it leaves at zero make every replay the
    same.  Three replays with eager work and a synchronisation between them,
    each against the work-buffer entry's eager result."""
    M, K, N, epi = 32, 6144, 2048, _lib.EPI_RESID          # splits across blocks
    g = torch.Generator().manual_seed(7)
    x = (torch.randn(M, K, generator=g) * 0.5).to(torch.bfloat16).to(gpu_device)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(gpu_device)
    r = torch.randn(M, N, generator=g).to(torch.bfloat16).to(gpu_device)
    wp, xo = _packed(w), operand_order(x)
    work = torch.zeros(_lib.NOALLOC_SCRATCH_FLOATS, device=gpu_device, dtype=torch.float32)
    want = _out(M, N, epi, gpu_device)
    L = lib()
    L.tfd_gemm_skinny_bf16(ptr(xo), ptr(wp), M, K, N, epi, ptr(r), N, ptr(want), N,
                           ptr(work), work.numel(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    got = _out(M, N, epi, gpu_device)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            L.tfd_gemm_skinny_bf16_noalloc(ptr(xo), ptr(wp), M, K, N, epi, ptr(r), N, ptr(got),
                                           N, side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for k in range(3):
        got.zero_()
        _ = (x.float() @ w.float().t()).sum().item()           # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), k
