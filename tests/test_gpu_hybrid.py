"""The hybrid models' kernels (workloads C4 and C5) against the oracle, on the GPU.

* fp8 skinny GEMM: every output within one bf16 ulp of the exact
  scale[n] * sum_k x e4m3(w) plus the f32 accumulation bound, every epilogue.
* Routers: the oracle's expert ids exactly; weights to f32 rounding (C4) or
  within one bf16 ulp (C5: bf16 weights); ties go to the lower id.
* MoE experts (C4 bf16 / C5 fp8), GDN and Mamba2 steps at the models' real
  widths: against the oracle to the bf16 bar (the kernels' f32 sums run in
  another order than the oracle's f64 ones, so a rounding may land one bf16 ulp
  away and carry on), conv windows bit-exact, recurrent state to f32 rounding,
  over two chained steps.
"""
import ctypes

import pytest
import torch

from oracle import hybrid_ref as H
from tests._parity import assert_close_bf16, report, ulp_bf16
from tests.test_gpu_batch import from_operand_order, operand_order
from tilefoundry_amd import _lib
from tilefoundry_amd._lib import lib, ptr
from tilefoundry_amd.hybrid.qwen3_5 import attention_splits

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _fp8_codes(shape, gen, std=0.6):
    return (torch.randn(shape, generator=gen) * std).to(torch.float8_e4m3fn).view(torch.uint8)


# ---------------------------------------------------------------------------
# fp8 skinny GEMM (per-output-channel scales)
# ---------------------------------------------------------------------------
def _packed_fp8(codes):
    N, K = codes.shape
    out = torch.full((-(-N // 16) * 16 * K,), 0x7F, device=codes.device, dtype=torch.uint8)
    lib().tfd_pack_skinny_fp8(ptr(codes), K, N, K, ptr(out), _stream())
    return out


def _gemm_fp8(x, codes, scale, epi, resid=None):
    M, K = x.shape
    N = codes.shape[0]
    dev = "cuda:0"
    w = _packed_fp8(codes.to(dev))
    if epi == _lib.EPI_SWIGLU:
        out = torch.full((32 * (N // 2),), float("nan"), device=dev, dtype=BF)
    elif epi == _lib.EPI_LOGITS:
        out = torch.zeros(M, N, device=dev, dtype=torch.float32)
    else:
        out = torch.zeros(M, N, device=dev, dtype=BF)
    # device copies held in locals: a temporary freed before the launch could
    # hand its memory to the next copy, which the stream runs first
    xd, sd = operand_order(x.to(dev)), scale.to(dev)
    rd = None if resid is None else resid.to(dev)
    lib().tfd_gemm_skinny_fp8(ptr(xd), ptr(w), ptr(sd), M, K, N, epi,
                              None if rd is None else ptr(rd), N, ptr(out), N, _stream())
    torch.cuda.synchronize()
    if epi == _lib.EPI_SWIGLU:
        return from_operand_order(out, M, N // 2).cpu()
    return out.cpu()


@pytest.mark.parametrize("M", [1, 8, 32])
@pytest.mark.parametrize("K,N", [(4096, 8512), (4096, 4096), (1536, 4096), (768, 4096),
                                 (256, 40)])
def test_fp8_gemm_within_one_ulp_of_exact(gpu_device, M, K, N):
    g = torch.Generator().manual_seed(M * 131 + K + N)
    x = (torch.randn(M, K, generator=g) * 0.5).to(BF)
    codes = _fp8_codes((N, K), g)
    scale = torch.rand(N, generator=g) * 0.02 + 0.005
    exact = H.gemv_fp8(codes, scale, x.float()).double()
    got = _gemm_fp8(x, codes, scale, _lib.EPI_STORE).float()
    raw = codes.view(torch.float8_e4m3fn).double()
    acc_bound = K * 2.0 ** -24 * (x.double().abs() @ raw.abs().t()) * scale.double()
    want = exact.to(BF).float()
    bound = ulp_bf16(want).double() + acc_bound
    bad = (got.double() - exact).abs() > bound
    assert not bad.any(), (int(bad.sum()), got[bad][:4], exact[bad][:4])
    assert torch.equal(_gemm_fp8(x, codes, scale, _lib.EPI_LOGITS), got)
    r = torch.randn(M, N, generator=g).to(BF)
    res = _gemm_fp8(x, codes, scale, _lib.EPI_RESID, r).float()
    assert torch.equal(res, (r.float() + got).to(BF).float())
    if N % 64 == 0:
        sw = _gemm_fp8(x, codes, scale, _lib.EPI_SWIGLU).float()
        act = torch.nn.functional.silu(got[:, 0::2].to(BF)).float()
        want_sw = (act * got[:, 1::2]).to(BF).float()
        assert ((sw - want_sw).abs() <= ulp_bf16(want_sw)).all()


@pytest.mark.parametrize("M", [1, 8, 17])
def test_fp8_gemm_scaled_residual_epilogue(gpu_device, M):
    """tfd_gemm_skinny_fp8_resid_scaled in place on the stream equals the plain
    product followed by torch's bf16 residual add h + y * m (model.py:502-508)."""
    g = torch.Generator().manual_seed(700 + M)
    K, N = 4096, 4096
    x = (torch.randn(M, K, generator=g) * 0.5).to(BF)
    codes = _fp8_codes((N, K), g)
    scale = torch.rand(N, generator=g) * 0.004 + 0.002
    y = _gemm_fp8(x, codes, scale, _lib.EPI_STORE)
    h = (torch.randn(M, N, generator=g)).to(BF)
    dev = "cuda:0"
    w = _packed_fp8(codes.to(dev))
    xd, sd, hd = operand_order(x.to(dev)), scale.to(dev), h.to(dev)
    lib().tfd_gemm_skinny_fp8_resid_scaled(ptr(xd), ptr(w), ptr(sd), M, K, N, ptr(hd), N, 0.22,
                                           ptr(hd), N, _stream())
    torch.cuda.synchronize()
    assert torch.equal(hd.cpu(), h + y * 0.22)


def test_rmsnorm_rows2_writes_both_layouts(gpu_device):
    """One launch of tfd_rmsnorm_rows2_bf16 gives the bits of the row-major and the
    operand-order calls of tfd_rmsnorm_rows_bf16."""
    g = torch.Generator().manual_seed(9)
    rows, n, dev = 8, 4096, "cuda:0"
    x = torch.randn(rows, n, generator=g).to(BF).to(dev)
    gamma = (torch.rand(n, generator=g) + 0.5).to(BF).to(dev)
    o_rows = torch.zeros(rows, n, dtype=BF, device=dev)
    o_pk = torch.zeros(32 * n, dtype=BF, device=dev)
    r2 = torch.zeros_like(o_rows)
    p2 = torch.zeros_like(o_pk)
    L, s = lib(), _stream()
    L.tfd_rmsnorm_rows_bf16(ptr(x), n, ptr(gamma), ptr(o_rows), n, rows, n, 1e-5, 0, s)
    L.tfd_rmsnorm_rows_bf16(ptr(x), n, ptr(gamma), ptr(o_pk), 0, rows, n, 1e-5, 1, s)
    L.tfd_rmsnorm_rows2_bf16(ptr(x), n, ptr(gamma), ptr(r2), n, ptr(p2), rows, n, 1e-5, s)
    torch.cuda.synchronize()
    assert torch.equal(r2, o_rows) and torch.equal(p2, o_pk)
    assert o_rows.abs().sum() > 0


@pytest.mark.parametrize("rows", [1, 8])
def test_tf_rmsnorm_rows_rounds_once(gpu_device, rows):
    """tfd_tf_rmsnorm_rows_bf16 (the HIR's rms_norm op, used by the Granite engine):
    every output within one bf16 ulp of the evaluator's formula (f32, one rounding:
    the oracle's rms_norm_tf) and >= 99% equal to it, in both layouts."""
    g = torch.Generator().manual_seed(13 + rows)
    n, dev = 4096, "cuda:0"
    x = H.bf(torch.randn(rows, n, generator=g) * 3)
    gamma = H.bf(1 + 0.3 * torch.randn(n, generator=g))
    want = H.rms_norm_tf(x, gamma, 1e-5)
    xd, gd = x.to(BF).to(dev), gamma.to(BF).to(dev)
    o_rows = torch.zeros(rows, n, dtype=BF, device=dev)
    o_pk = torch.zeros(32 * n, dtype=BF, device=dev)
    rc = lib().tfd_tf_rmsnorm_rows_bf16(ptr(xd), n, ptr(gd), ptr(o_rows), n, ptr(o_pk), rows, n,
                                        1e-5, _stream())
    assert rc == 0
    torch.cuda.synchronize()
    got = o_rows.float().cpu()
    assert torch.equal(from_operand_order(o_pk, rows, n).float().cpu(), got)
    assert ((got - want).abs() <= ulp_bf16(want)).all()
    assert (got == want).float().mean() >= 0.99


def _proj8_norm(x, gamma, codes, scale, epi, rows_out=True):
    """tfd_proj8_norm over bf16 rows x [M][4096]: (out, normalised rows)."""
    M, K = x.shape
    N = codes.shape[0]
    dev = "cuda:0"
    w = _packed_fp8(codes.to(dev))
    xd, gd, sd = x.to(BF).to(dev), gamma.to(BF).to(dev), scale.to(dev)
    out = torch.zeros(M, N, device=dev, dtype=BF if epi == _lib.EPI_STORE else torch.float32)
    xr = torch.zeros(M, K, device=dev, dtype=BF)
    a = _lib.TfdProj8NormArgs()
    a.x, a.ldx, a.gamma, a.eps = ptr(xd), K, ptr(gd), 1e-5
    a.x_rows, a.ldxr = (ptr(xr), K) if rows_out else (None, 0)
    a.w, a.scale, a.rows, a.K, a.N = ptr(w), ptr(sd), M, K, N
    a.out, a.ldo, a.epilogue = ptr(out), N, epi
    lib().tfd_proj8_norm(ctypes.addressof(a), _stream())
    torch.cuda.synchronize()
    return out.float().cpu(), xr.float().cpu()


@pytest.mark.parametrize("M", [1, 5, 8])
@pytest.mark.parametrize("N,epi", [(72, _lib.EPI_LOGITS), (8512, _lib.EPI_STORE),
                                   (6144, _lib.EPI_STORE)])
def test_proj8_norm_is_the_norm_then_the_fp8_gemm(gpu_device, M, N, epi):
    """tfd_proj8_norm (the HIR RMSNorm as the prologue of an fp8 projection; C5's
    post norm + router) equals tfd_tf_rmsnorm_rows_bf16 followed by
    tfd_gemm_skinny_fp8 bit for bit -- the normalised rows it hands on too -- and
    is within one bf16 ulp plus the f32 bound of the exact product of the
    oracle's normalised rows (rms_norm_tf) with gemv_fp8."""
    g = torch.Generator().manual_seed(7 * M + N)
    K = 4096
    x = H.bf(torch.randn(M, K, generator=g) * 2)
    gamma = H.bf(1 + 0.2 * torch.randn(K, generator=g))
    codes = _fp8_codes((N, K), g)
    scale = torch.rand(N, generator=g) * 0.02 + 0.005
    got, rows = _proj8_norm(x, gamma, codes, scale, epi)
    dev = "cuda:0"
    xd, gd = x.to(BF).to(dev), gamma.to(BF).to(dev)
    o_rows = torch.zeros(M, K, dtype=BF, device=dev)
    o_pk = torch.zeros(32 * K, dtype=BF, device=dev)
    lib().tfd_tf_rmsnorm_rows_bf16(ptr(xd), K, ptr(gd), ptr(o_rows), K, ptr(o_pk), M, K, 1e-5,
                                   _stream())
    torch.cuda.synchronize()
    assert torch.equal(rows, o_rows.float().cpu())
    two = _gemm_fp8(o_rows.float().cpu().to(BF), codes, scale, epi).float()
    assert torch.equal(got, two)
    xn = H.rms_norm_tf(x, gamma, 1e-5)
    exact = H.gemv_fp8(codes, scale, xn).double()
    raw = codes.view(torch.float8_e4m3fn).double()
    acc_bound = K * 2.0 ** -24 * (xn.double().abs() @ raw.abs().t()) * scale.double()
    # the norm may round one input an ulp away from the oracle's (f32 sums in
    # another order): that input's term is bounded by an ulp of it times |w|
    norm_bound = (ulp_bf16(xn).double() @ raw.abs().t()) * scale.double()
    bound = ulp_bf16(exact.float()).double() + acc_bound + norm_bound
    bad = (got.double() - exact).abs() > bound
    assert not bad.any(), (int(bad.sum()), got[bad][:4], exact[bad][:4])


def test_proj8_norm_rejects_bad_shapes(gpu_device):
    g = torch.Generator().manual_seed(3)
    for M, K in ((9, 4096), (4, 2048)):
        x = H.bf(torch.randn(M, K, generator=g))
        with pytest.raises(_lib.TFDError, match="proj8_norm"):
            _proj8_norm(x, torch.ones(K), _fp8_codes((72, K), g), torch.ones(72),
                        _lib.EPI_LOGITS)


@pytest.mark.parametrize("M,V", [(1, 4096), (8, 100352)])
def test_head_logits_divided_by_logits_scaling(gpu_device, M, V):
    """tfd_gemm_skinny_bf16_logits_div (Granite's lm_head / logits_scaling):
    exactly the TFD_EPI_LOGITS logits rounded and divided by 16 (a power of two,
    so exactly logits / 16)."""
    g = torch.Generator().manual_seed(21)
    K, dev = 4096, "cuda:0"
    x = H.bf(torch.randn(M, K, generator=g)).to(BF).to(dev)
    w = (torch.randn(V, K, generator=g) * 0.02).to(BF).to(dev)
    packed = torch.empty(-(-V // 16) * 16 * K, dtype=BF, device=dev)
    L, s = lib(), _stream()
    L.tfd_pack_skinny_bf16(ptr(w), K, V, K, ptr(packed), s)
    xo = operand_order(x)
    work = torch.zeros(1 << 21, dtype=torch.float32, device=dev)
    plain = torch.zeros(M, V, device=dev)
    scaled = torch.zeros(M, V, device=dev)
    assert L.tfd_gemm_skinny_bf16(ptr(xo), ptr(packed), M, K, V, _lib.EPI_LOGITS, None, 0,
                                  ptr(plain), V, ptr(work), work.numel(), s) == 0
    assert L.tfd_gemm_skinny_bf16_logits_div(ptr(xo), ptr(packed), M, K, V, 16.0, ptr(scaled),
                                             V, ptr(work), work.numel(), s) == 0
    torch.cuda.synchronize()
    assert torch.equal(scaled, plain / 16)
    assert plain.abs().max() > 0


def test_fp8_pack_layout(gpu_device):
    """Block (tile t, step s) is 512 bytes; lane l's 8 codes are
    W[16t + l % 16][32s + 8(l // 16) + j]; padding rows are 0."""
    N, K = 40, 512
    codes = (torch.arange(N * K) % 251).to(torch.uint8).view(N, K)
    got = _packed_fp8(codes.to(gpu_device)).cpu().view(-1, 64, 8)
    tiles, steps = -(-N // 16), K // 32
    wp = torch.cat([codes, torch.zeros(tiles * 16 - N, K, dtype=torch.uint8)])
    want = wp.view(tiles, 16, steps, 4, 8).permute(0, 2, 3, 1, 4).reshape(-1, 64, 8)
    assert torch.equal(got, want)


# ---------------------------------------------------------------------------
# Routers
# ---------------------------------------------------------------------------
def _route(logits, k, mode, ldl=None):
    rows, E = logits.shape
    ldl = ldl or E
    buf = torch.full((rows, ldl), float("nan"), device="cuda:0")
    buf[:, :E] = logits.to("cuda:0")
    w = torch.zeros(rows, k, device="cuda:0")
    idx = torch.full((rows, k), -1, dtype=torch.int32, device="cuda:0")
    lib().tfd_route_topk(ptr(buf), ldl, rows, E, k, mode, ptr(w), ptr(idx), _stream())
    torch.cuda.synchronize()
    return w.cpu(), idx.cpu().long()


@pytest.mark.parametrize("rows", [1, 16, 32])
def test_route_softmax_topk_c4(gpu_device, rows):
    g = torch.Generator().manual_seed(rows)
    logits = H.bf(torch.randn(rows, 256, generator=g) * 2)
    w, idx = _route(logits, 8, _lib.ROUTE_SOFTMAX_TOPK, ldl=260)
    want_w, want_i = H.route_softmax_topk(logits, 8)
    assert torch.equal(idx, want_i)
    torch.testing.assert_close(w, want_w, atol=1e-6, rtol=1e-5)


@pytest.mark.parametrize("rows", [1, 8, 32])
def test_route_topk_softmax_c5(gpu_device, rows):
    g = torch.Generator().manual_seed(100 + rows)
    logits = H.bf(torch.randn(rows, 72, generator=g) * 2)
    w, idx = _route(logits, 10, _lib.ROUTE_TOPK_SOFTMAX)
    want_w, want_i = H.route_topk_softmax(logits, 10)
    assert torch.equal(idx, want_i)
    assert ((w - want_w).abs() <= ulp_bf16(want_w)).all(), report(w, want_w)
    assert torch.equal(w, w.to(BF).float())


def test_route_ties_go_to_the_lower_expert(gpu_device):
    logits = torch.zeros(2, 64)
    logits[0, [5, 9, 40]] = 1.0
    logits[1, [63, 2]] = 3.0
    for mode in (_lib.ROUTE_SOFTMAX_TOPK, _lib.ROUTE_TOPK_SOFTMAX):
        _, idx = _route(logits, 4, mode)
        assert idx[0].tolist() == [5, 9, 40, 0]
        assert idx[1].tolist() == [2, 63, 0, 1]


def test_route_rejects_bad_shapes(gpu_device):
    with pytest.raises(_lib.TFDError):
        _route(torch.zeros(1, 300), 8, _lib.ROUTE_SOFTMAX_TOPK)
    with pytest.raises(_lib.TFDError):
        _route(torch.zeros(1, 16), 17, _lib.ROUTE_SOFTMAX_TOPK)


# ---------------------------------------------------------------------------
# MoE experts
# ---------------------------------------------------------------------------
def _pack_rows(w):
    """A [rows][K] weight matrix packed as the skinny GEMMs pack it (bf16 or fp8
    codes), on the GPU."""
    w = w.to("cuda:0").contiguous()
    N, K = w.shape
    out = torch.empty(-(-N // 16) * 16 * K, dtype=w.dtype, device=w.device)
    fn = lib().tfd_pack_skinny_fp8 if w.dtype == torch.uint8 else lib().tfd_pack_skinny_bf16
    fn(ptr(w), K, N, K, ptr(out), _stream())
    return out


def _moe_call(x, weights, idx, *, w_gate, w_up, w_down, w_sin, w_sout, s=None, w_sscale=None,
              fp8=False, policy, expect_err=0, route=None, resid=None, packed=False):
    """resid = (stream, multiplier): the call adds its scaled output into a copy of
    the bf16 stream, which is returned instead of `out`.  packed: the weights
    packed and tfd_moe_experts_packed called (no partials)."""
    dev = "cuda:0"
    rows, hs = x.shape
    k = idx.shape[1]
    experts, inter = w_gate.shape[0], w_gate.shape[1]
    sh = w_sout.shape[1]
    ld = max(inter, sh)
    keep = []

    def d(t):
        t = t.to(dev).contiguous()
        keep.append(t)
        return ptr(t)

    hidden = torch.full((rows, k + 1, ld), float("nan"), device=dev, dtype=BF)
    partial = torch.full((rows, k + 1, hs), float("nan"), device=dev)
    groups = torch.full((_lib.moe_group_words(experts, rows),), -7, dtype=torch.int32,
                        device=dev)
    out = torch.full((rows, hs), float("nan"), device=dev)
    sscale = torch.zeros(rows, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    a = _lib.TfdMoeArgs()
    a.x, a.weights, a.idx = d(x.to(BF)), d(weights.float()), d(idx.to(torch.int32))
    if packed:
        w_gate, w_up = w_gate.reshape(-1, hs), w_up.reshape(-1, hs)
        w_down = w_down.reshape(-1, inter)
        w_gate, w_up, w_down, w_sin, w_sout = (_pack_rows(w) for w in
                                               (w_gate, w_up, w_down, w_sin, w_sout))
    a.w_gate, a.w_up, a.w_down = d(w_gate), d(w_up), d(w_down)
    a.w_shared_in, a.w_shared_out = d(w_sin), d(w_sout)
    if fp8:
        a.s_gate, a.s_up, a.s_down, a.s_shared_in, a.s_shared_out = [d(v) for v in s]
    a.w_shared_scale = None if w_sscale is None else d(w_sscale)
    a.hidden, a.shared_scale, a.out = ptr(hidden), ptr(sscale), ptr(out)
    a.partial, a.groups = (None if packed else ptr(partial)), ptr(groups)
    a.rows, a.k, a.experts, a.hidden_size = rows, k, experts, hs
    a.inter, a.shared_inter, a.hidden_ld = inter, sh, ld
    a.fp8, a.policy, a.err = int(fp8), policy, ptr(err)
    if route is not None:
        a.logits, a.ldl, a.route = d(route[0].float()), route[0].shape[1], route[1]
    stream = None
    if resid is not None:
        stream = resid[0].to(dev, BF).contiguous()
        a.out, a.resid, a.resid_mult = None, ptr(stream), resid[1]
    (lib().tfd_moe_experts_packed if packed else lib().tfd_moe_experts)(ctypes.addressof(a),
                                                                         _stream())
    torch.cuda.synchronize()
    if route is not None:
        idx = keep[2].cpu()                  # the call wrote the ids
    if expect_err:
        assert err.item() == expect_err
    else:
        assert err.item() == 0
        # the groups: every (sequence, slot) once, under the expert it picked
        g = groups.cpu()
        picked = g[1:1 + g[0]].tolist()
        assert picked == sorted(set(idx.reshape(-1).tolist()))
        for e in picked:
            got = sorted(g[1 + 2 * experts + e * rows:][:g[1 + experts + e]].tolist())
            assert got == [i for i, v in enumerate(idx.reshape(-1).tolist()) if v == e]
    return out.cpu() if stream is None else stream.cpu()


def _routing(rows, experts, k, gen):
    idx = torch.stack([torch.randperm(experts, generator=gen)[:k] for _ in range(rows)])
    w = torch.rand(rows, k, generator=gen) + 0.1
    return w / w.sum(-1, keepdim=True), idx


@pytest.mark.parametrize("rows,same", [(1, False), (4, False), (16, False), (16, True),
                                       (32, False)])
def test_moe_experts_c4_bf16(gpu_device, rows, same):
    """Qwen3.5 widths: H 2048, I 512, shared 512, top 8 (16 experts resident, so
    sequences share experts; `same`: every sequence picks the same 8)."""
    g = torch.Generator().manual_seed(rows + 100 * same)
    hs, inter, sh, E, k = 2048, 512, 512, 16, 8
    rnd = lambda *s, std=0.03: H.bf(torch.randn(*s, generator=g) * std)
    x = rnd(rows, hs, std=1.0)
    weights, idx = _routing(rows, E, k, g)
    if same:
        idx = idx[:1].repeat(rows, 1)
    w_gate, w_up, w_down = rnd(E, inter, hs), rnd(E, inter, hs), rnd(E, hs, inter)
    ws_gate, ws_up, ws_down, ws_scale = rnd(sh, hs), rnd(sh, hs), rnd(hs, sh), rnd(1, hs)
    got = _moe_call(x, weights, idx, w_gate=w_gate.to(BF), w_up=w_up.to(BF),
                    w_down=w_down.to(BF), w_sin=torch.cat([ws_gate, ws_up]).to(BF),
                    w_sout=ws_down.to(BF), w_sscale=ws_scale.to(BF), policy=_lib.POLICY_F32)
    want = H.moe_c4(x, weights, idx, w_gate, w_up, w_down, ws_gate, ws_up, ws_down, ws_scale)
    assert_close_bf16(got, want, max_rel=1e-2, min_cos=0.99999, name="moe c4")


@pytest.mark.parametrize("mode", ["softmax_topk", "topk_softmax"])
def test_moe_routes_inside_the_call(gpu_device, mode):
    """Routing folded into the MoE call (its first launch) gives the ids and
    weights tfd_route_topk gives, and the same output bits."""
    g = torch.Generator().manual_seed(21)
    rows, hs, inter, sh, E, k = 5, 512, 128, 128, 32, 6
    rnd = lambda *s: H.bf(torch.randn(*s, generator=g) * 0.05).to(BF)
    x = H.bf(torch.randn(rows, hs, generator=g))
    logits = H.bf(torch.randn(rows, E, generator=g) * 2)
    rmode, mmode, policy = ((_lib.ROUTE_SOFTMAX_TOPK, _lib.MOE_ROUTE_SOFTMAX_TOPK,
                             _lib.POLICY_F32) if mode == "softmax_topk" else
                            (_lib.ROUTE_TOPK_SOFTMAX, _lib.MOE_ROUTE_TOPK_SOFTMAX,
                             _lib.POLICY_BF16))
    w_ref, idx_ref = _route(logits, k, rmode)
    weights = dict(w_gate=rnd(E, inter, hs), w_up=rnd(E, inter, hs), w_down=rnd(E, hs, inter),
                   w_sin=rnd(2 * sh, hs), w_sout=rnd(hs, sh))
    want = _moe_call(x, w_ref, idx_ref, policy=policy, **weights)
    wbuf = torch.zeros(rows, k)
    ibuf = torch.full((rows, k), -1, dtype=torch.int32)
    got = _moe_call(x, wbuf, ibuf, policy=policy, route=(logits, mmode), **weights)
    assert torch.equal(got, want)


def test_moe_experts_flags_a_bad_expert_id(gpu_device):
    g = torch.Generator().manual_seed(3)
    rows, hs, inter, sh, E, k = 2, 256, 64, 64, 8, 2
    rnd = lambda *s: H.bf(torch.randn(*s, generator=g) * 0.1).to(BF)
    weights, idx = _routing(rows, E, k, g)
    idx[1, 0] = E + 3
    _moe_call(H.bf(torch.randn(rows, hs, generator=g)), weights, idx, w_gate=rnd(E, inter, hs),
              w_up=rnd(E, inter, hs), w_down=rnd(E, hs, inter), w_sin=rnd(2 * sh, hs),
              w_sout=rnd(hs, sh), policy=_lib.POLICY_BF16, expect_err=_lib.ERR_TOKEN_RANGE)


@pytest.mark.parametrize("rows", [1, 8])
def test_moe_experts_c5_fp8(gpu_device, rows):
    """Granite widths: H 4096, I 768, shared 1536, top 10 (16 experts resident)."""
    g = torch.Generator().manual_seed(50 + rows)
    hs, inter, sh, E, k = 4096, 768, 1536, 16, 10
    x = H.bf(torch.randn(rows, hs, generator=g))
    weights, idx = _routing(rows, E, k, g)
    weights = H.bf(weights)
    sc = lambda *s: torch.rand(*s, generator=g) * 0.004 + 0.002
    gc, uc, dc = _fp8_codes((E, inter, hs), g), _fp8_codes((E, inter, hs), g), \
        _fp8_codes((E, hs, inter), g)
    gs, us, ds = sc(E, inter), sc(E, inter), sc(E, hs)
    sic, soc = _fp8_codes((2 * sh, hs), g), _fp8_codes((hs, sh), g)
    sis, sos = sc(2 * sh), sc(hs)
    got = _moe_call(x, weights, idx, w_gate=gc, w_up=uc, w_down=dc, w_sin=sic, w_sout=soc,
                    s=(gs, us, ds, sis, sos), fp8=True, policy=_lib.POLICY_BF16)
    want = H.moe_c5(x, weights, idx, gc, gs, uc, us, dc, ds, sic, sis, soc, sos)
    assert torch.equal(got, got.to(BF).float())
    assert_close_bf16(got, want, max_rel=2e-2, min_cos=0.9999, name="moe c5")
    # the same call adding bf16(y * m) into a bf16 stream: the residual add of
    # model.py:502-508 in torch's bf16 arithmetic on the plain output
    h = H.bf(torch.randn(rows, hs, generator=g)).to(BF)
    added = _moe_call(x, weights, idx, w_gate=gc, w_up=uc, w_down=dc, w_sin=sic, w_sout=soc,
                      s=(gs, us, ds, sis, sos), fp8=True, policy=_lib.POLICY_BF16,
                      resid=(h, 0.22))
    assert torch.equal(added, h + got.to(BF) * 0.22)


def _packed_vs_rowmajor(got, ref, name, f32=False):
    """The packed entry's sums run in another order (MFMA accumulators over K):
    with bf16 outputs they equal the row-major entry's up to a one-ulp flip of a
    bf16 rounding, and only rarely; with the f32 policy an output is an f32 sum
    of bf16-rounded slot values, so a flip in any slot moves it by about a bf16
    ulp of that slot -- held within 2^-8 of the largest output."""
    d = (got - ref).abs()
    flips = int((d > 0).sum())
    rel = float(d.max() / ref.abs().max())
    print(f"{name}: {flips} of {d.numel()} outputs differ from the row-major entry, max "
          f"{float(d.max()):.4g} ({rel:.2e} of the largest)", flush=True)
    if f32:
        assert rel <= 2.0 ** -8, (name, rel)
    else:
        assert flips <= max(8, d.numel() // 200), (name, flips)


@pytest.mark.parametrize("rows,same", [(1, False), (5, False), (16, False), (16, True)])
def test_moe_experts_packed_c4_bf16(gpu_device, rows, same):
    """tfd_moe_experts_packed at the Qwen3.5 widths (H 2048, I 512, shared 512, top
    8, shared-expert gate, f32 policy, accumulate off), against the oracle and
    the row-major entry."""
    g = torch.Generator().manual_seed(300 + rows + 100 * same)
    hs, inter, sh, E, k = 2048, 512, 512, 16, 8
    rnd = lambda *s, std=0.03: H.bf(torch.randn(*s, generator=g) * std)
    x = rnd(rows, hs, std=1.0)
    weights, idx = _routing(rows, E, k, g)
    if same:
        idx = idx[:1].repeat(rows, 1)
    w_gate, w_up, w_down = rnd(E, inter, hs), rnd(E, inter, hs), rnd(E, hs, inter)
    ws_gate, ws_up, ws_down, ws_scale = rnd(sh, hs), rnd(sh, hs), rnd(hs, sh), rnd(1, hs)
    kw = dict(w_gate=w_gate.to(BF), w_up=w_up.to(BF), w_down=w_down.to(BF),
              w_sin=torch.cat([ws_gate, ws_up]).to(BF), w_sout=ws_down.to(BF),
              w_sscale=ws_scale.to(BF), policy=_lib.POLICY_F32)
    got = _moe_call(x, weights, idx, packed=True, **kw)
    want = H.moe_c4(x, weights, idx, w_gate, w_up, w_down, ws_gate, ws_up, ws_down, ws_scale)
    assert_close_bf16(got, want, max_rel=1e-2, min_cos=0.99999, name="moe c4 packed")
    _packed_vs_rowmajor(got, _moe_call(x, weights, idx, **kw), "moe c4 packed", f32=True)


@pytest.mark.parametrize("rows", [1, 8, 16])
def test_moe_experts_packed_c5_fp8(gpu_device, rows):
    """tfd_moe_experts_packed at the Granite workload's widths: H 4096, 72 experts
    of I 768, shared 1536, top 10, fp8 with row scales, against the oracle and
    the row-major entry; then routed inside the call (top 10 then softmax) and
    added into a bf16 stream, against the row-major entry doing the same."""
    g = torch.Generator().manual_seed(400 + rows)
    hs, inter, sh, E, k = 4096, 768, 1536, 72, 10
    x = H.bf(torch.randn(rows, hs, generator=g))
    weights, idx = _routing(rows, E, k, g)
    weights = H.bf(weights)
    sc = lambda *s: torch.rand(*s, generator=g) * 0.004 + 0.002
    gc, uc, dc = _fp8_codes((E, inter, hs), g), _fp8_codes((E, inter, hs), g), \
        _fp8_codes((E, hs, inter), g)
    gs, us, ds = sc(E, inter), sc(E, inter), sc(E, hs)
    sic, soc = _fp8_codes((2 * sh, hs), g), _fp8_codes((hs, sh), g)
    sis, sos = sc(2 * sh), sc(hs)
    kw = dict(w_gate=gc, w_up=uc, w_down=dc, w_sin=sic, w_sout=soc, s=(gs, us, ds, sis, sos),
              fp8=True, policy=_lib.POLICY_BF16)
    got = _moe_call(x, weights, idx, packed=True, **kw)
    want = H.moe_c5(x, weights, idx, gc, gs, uc, us, dc, ds, sic, sis, soc, sos)
    assert torch.equal(got, got.to(BF).float())
    assert_close_bf16(got, want, max_rel=2e-2, min_cos=0.9999, name="moe c5 packed")
    _packed_vs_rowmajor(got, _moe_call(x, weights, idx, **kw), "moe c5 packed")
    logits = H.bf(torch.randn(rows, E, generator=g))
    h = H.bf(torch.randn(rows, hs, generator=g)).to(BF)
    zw, zi = torch.zeros(rows, k), torch.zeros(rows, k, dtype=torch.long)
    kw.update(route=(logits, _lib.MOE_ROUTE_TOPK_SOFTMAX), resid=(h, 0.22))
    _packed_vs_rowmajor(_moe_call(x, zw, zi, packed=True, **kw).float(),
                        _moe_call(x, zw, zi, **kw).float(), "moe c5 packed, routed, resid")


def test_moe_experts_packed_rejects_bad_shapes(gpu_device):
    """More than 16 sequences, a hidden size off the 1024 grid, more than 16
    experts per sequence: kBadShape before anything is launched."""
    g = torch.Generator().manual_seed(5)
    inter, sh, E = 256, 256, 32
    rnd = lambda *s: torch.randn(*s, generator=g).to(BF)
    for rows, hs, k in ((17, 1024, 2), (2, 512, 2), (2, 1024, 17)):
        weights, idx = _routing(rows, E, k, g)
        with pytest.raises(_lib.TFDError, match="moe_experts_packed"):
            _moe_call(rnd(rows, hs), weights, idx, w_gate=rnd(E, inter, hs),
                      w_up=rnd(E, inter, hs), w_down=rnd(E, hs, inter), w_sin=rnd(2 * sh, hs),
                      w_sout=rnd(hs, sh), policy=_lib.POLICY_BF16, packed=True)


# ---------------------------------------------------------------------------
# Gated DeltaNet step (C4: 16 key heads, 32 value heads, 128-wide)
# ---------------------------------------------------------------------------
def _gdn_inputs(rows, g, hk=16, hv=32):
    key, val = hk * 128, hv * 128
    conv = 2 * key + val
    proj = H.bf(torch.randn(rows, conv + val + 2 * hv, generator=g))
    return dict(
        proj=proj, conv_state=torch.randn(rows, conv, 3, generator=g),
        state=torch.randn(rows, hv, 128, 128, generator=g) * 0.05,
        conv_w=H.bf(torch.randn(conv, 4, generator=g) * 0.5),
        a_log=H.bf(torch.randn(hv, generator=g) * 0.5),
        dt_bias=H.bf(torch.randn(hv, generator=g) * 0.5),
        gamma=H.bf(1 + 0.1 * torch.randn(128, generator=g)), hk=hk, hv=hv)


def _gdn_gpu(inp, proj, conv_in, state):
    dev = "cuda:0"
    rows = proj.shape[0]
    hk, hv = inp["hk"], inp["hv"]
    val = hv * 128
    proj_d = torch.zeros(rows, proj.shape[1] + 8, device=dev)
    proj_d[:, :proj.shape[1]] = proj.to(dev)
    cin = conv_in.to(dev).contiguous()
    cout = torch.full_like(cin, float("nan"))
    st = state.to(dev).contiguous()
    params = [inp[n].to(dev).to(BF) for n in ("conv_w", "a_log", "dt_bias", "gamma")]
    out = torch.full((32 * val,), float("nan"), device=dev, dtype=BF)
    a = _lib.TfdGdnArgs()
    a.proj, a.proj_ld, a.conv_in, a.conv_out, a.state = ptr(proj_d), proj_d.shape[1], ptr(cin), \
        ptr(cout), ptr(st)
    a.conv_w, a.a_log, a.dt_bias, a.gamma = [ptr(p) for p in params]
    a.out = ptr(out)
    a.rows, a.key_heads, a.value_heads, a.head_k_dim, a.head_v_dim, a.conv_kernel = \
        rows, hk, hv, 128, 128, 4
    a.l2_eps, a.rms_eps = 1e-6, 1e-6
    lib().tfd_gdn_step(ctypes.addressof(a), _stream())
    torch.cuda.synchronize()
    return from_operand_order(out, rows, val).float().cpu(), cout.cpu(), st.cpu()


@pytest.mark.parametrize("rows", [1, 16])
def test_gdn_step_two_tokens(gpu_device, rows):
    g = torch.Generator().manual_seed(7 + rows)
    inp = _gdn_inputs(rows, g)
    conv_state, state = inp["conv_state"], inp["state"]
    gconv, gstate = conv_state, state
    for step in range(2):
        proj = inp["proj"] if step == 0 else H.bf(torch.randn(inp["proj"].shape, generator=g))
        want, conv_state, state = H.gdn_step(
            proj, conv_state, state, inp["conv_w"], inp["a_log"], inp["dt_bias"], inp["gamma"],
            hk=inp["hk"], hv=inp["hv"], dk=128, dv=128)
        got, gconv, gstate = _gdn_gpu(inp, proj, gconv, gstate)
        assert torch.equal(gconv, conv_state), step
        torch.testing.assert_close(gstate, state, atol=1e-5, rtol=1e-4)
        r = assert_close_bf16(got, H.bf(want), max_rel=1e-2, min_cos=0.99999,
                              name=f"gdn step {step}")
        assert r["within_1ulp"] >= 0.999, r


def test_gdn_step_rejects_bad_shapes(gpu_device):
    a = _lib.TfdGdnArgs()
    a.rows = 1
    with pytest.raises(_lib.TFDError):
        lib().tfd_gdn_step(ctypes.addressof(a), _stream())


# ---------------------------------------------------------------------------
# Mamba2 step (C5: 128 heads of 64, state 128, one group)
# ---------------------------------------------------------------------------
def _mamba_inputs(rows, g, nh=128):
    exp_ = nh * 64
    conv = exp_ + 256
    return dict(
        proj=H.bf(torch.randn(rows, exp_ + conv + nh, generator=g)),
        conv_state=H.bf(torch.randn(rows, conv, 3, generator=g)),
        state=torch.randn(rows, nh, 64, 128, generator=g) * 0.3,
        conv_w=H.bf(torch.randn(conv, 4, generator=g) * 0.5),
        conv_b=H.bf(torch.randn(conv, generator=g) * 0.1),
        a_log=H.bf(torch.randn(nh, generator=g) * 0.5),
        dt_bias=H.bf(torch.randn(nh, generator=g) * 0.5),
        d_skip=H.bf(torch.randn(nh, generator=g)),
        gamma=H.bf(1 + 0.1 * torch.randn(exp_, generator=g)), nh=nh)


def _mamba_gpu(inp, proj, conv_in, state):
    dev = "cuda:0"
    rows = proj.shape[0]
    nh = inp["nh"]
    exp_ = nh * 64
    proj_d = torch.zeros(rows, proj.shape[1] + 16, device=dev, dtype=BF)
    proj_d[:, :proj.shape[1]] = proj.to(dev).to(BF)
    cin = conv_in.to(dev).to(BF).contiguous()
    cout = torch.full_like(cin, float("nan"))
    st = state.to(dev).contiguous()
    params = [inp[n].to(dev).to(BF)
              for n in ("conv_w", "conv_b", "a_log", "dt_bias", "d_skip", "gamma")]
    gated = torch.zeros(rows, exp_, device=dev)
    ssq = torch.zeros(rows, nh, device=dev)
    out = torch.full((32 * exp_,), float("nan"), device=dev, dtype=BF)
    a = _lib.TfdMambaArgs()
    a.proj, a.proj_ld, a.conv_in, a.conv_out, a.state = ptr(proj_d), proj_d.shape[1], ptr(cin), \
        ptr(cout), ptr(st)
    a.conv_w, a.conv_b, a.a_log, a.dt_bias, a.d_skip, a.gamma = [ptr(p) for p in params]
    a.gated, a.ssq, a.out = ptr(gated), ptr(ssq), ptr(out)
    a.rows, a.heads, a.head_dim, a.state_dim, a.groups, a.conv_kernel = rows, nh, 64, 128, 1, 4
    a.eps = 1e-5
    lib().tfd_mamba_step(ctypes.addressof(a), _stream())
    torch.cuda.synchronize()
    return from_operand_order(out, rows, exp_).float().cpu(), cout.float().cpu(), st.cpu()


@pytest.mark.parametrize("rows", [1, 8])
def test_mamba_step_two_tokens(gpu_device, rows):
    g = torch.Generator().manual_seed(70 + rows)
    inp = _mamba_inputs(rows, g)
    conv_state, state = inp["conv_state"], inp["state"]
    gconv, gstate = conv_state, state
    for step in range(2):
        proj = inp["proj"] if step == 0 else H.bf(torch.randn(inp["proj"].shape, generator=g))
        want, conv_state, state = H.mamba_step(
            proj, conv_state, state, inp["conv_w"], inp["conv_b"], inp["a_log"], inp["dt_bias"],
            inp["d_skip"], inp["gamma"], nh=inp["nh"], pd=64, ns=128, ng=1)
        got, gconv, gstate = _mamba_gpu(inp, proj, gconv, gstate)
        assert torch.equal(gconv, conv_state), step
        srep = report(gstate, state)
        assert srep["max_rel"] < 1e-3 and srep["cos"] > 0.999999, srep
        r = assert_close_bf16(got, want, max_rel=2e-2, min_cos=0.9999, name=f"mamba {step}")
        assert r["within_1ulp"] >= 0.99, r


# ---------------------------------------------------------------------------
# Full-attention layers (C4: 256-wide heads, RoPE on 64 dims, output gate;
# C5: 128-wide heads, no position embedding, HIR rounding)
# ---------------------------------------------------------------------------
def _paged_pool(pasts, hkv, d, max_pages, gen):
    """Logical caches [C][HKV][D] -> a shuffled page pool (NaN where unused) and
    the page table; every sequence gets max_pages distinct pages."""
    B = len(pasts)
    num_pages = B * max_pages + 3
    table = torch.randperm(num_pages, generator=gen)[:B * max_pages].view(B, max_pages)
    kpool = torch.full((num_pages, hkv, 16, d), float("nan"), dtype=BF)
    vpool = kpool.clone()
    for b, (kp, vp) in enumerate(pasts):
        j = torch.arange(kp.shape[0])
        kpool[table[b, j // 16], :, j % 16] = kp.to(BF)
        vpool[table[b, j // 16], :, j % 16] = vp.to(BF)
    return kpool, vpool, table.to(torch.int32)


def _gqa_call(qkv, pos, table, kpool, vpool, *, heads, kv_heads, head_dim, scale, split_len,
              policy, gamma_q=None, gamma_k=None, cos=None, sin=None, eps=1e-6, nsplit=None):
    """split_len 0: lengths derived from each row's position over nsplit splits
    (default: the engines' choice)."""
    dev = "cuda:0"
    rows = qkv.shape[0]
    max_pages = table.shape[1]
    if split_len == 0:
        nsplit = nsplit or attention_splits(rows, kv_heads, max_pages * 16)
    else:
        nsplit = -(-max_pages * 16 // split_len)
    stride = max_pages * 16
    keep = []

    def d(t):
        t = t.to(dev).contiguous()
        keep.append(t)
        return ptr(t)

    kp, vp = kpool.to(dev), vpool.to(dev)
    out = torch.full((32 * heads * head_dim,), float("nan"), device=dev, dtype=BF)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    counters = torch.zeros(rows * kv_heads, dtype=torch.int32, device=dev)
    a = _lib.TfdGqaArgs()
    a.qkv, a.ldq = d(qkv), qkv.shape[1]
    if policy == _lib.POLICY_F32:
        a.gamma_q, a.gamma_k, a.cos_table, a.sin_table = d(gamma_q.to(BF)), d(gamma_k.to(BF)), \
            d(cos.to(BF)), d(sin.to(BF))
        a.rope_rows, a.rot_dim = cos.shape[0], cos.shape[1]
    a.pos, a.page_table, a.max_pages = d(pos.to(torch.int32)), d(table), max_pages
    a.k_pool, a.v_pool, a.num_pages = ptr(kp), ptr(vp), kpool.shape[0]
    a.rows, a.heads, a.kv_heads, a.head_dim = rows, heads, kv_heads, head_dim
    a.scale, a.eps = scale, eps
    a.scores = d(torch.full((rows * heads * stride,), float("nan")))
    a.score_stride = stride
    a.stats = d(torch.full((rows * heads * nsplit * 2,), float("nan")))
    a.part = d(torch.full((rows * heads * nsplit * head_dim,), float("nan")))
    a.counters = ptr(counters)
    a.nsplit, a.split_len = nsplit, split_len
    a.out, a.policy, a.err = ptr(out), policy, ptr(err)
    lib().tfd_gqa_decode(ctypes.addressof(a), _stream())
    torch.cuda.synchronize()
    assert not counters.any()
    return (from_operand_order(out, rows, heads * head_dim).float().cpu(), kp.cpu(), vp.cpu(),
            int(err.item()))


def _rope_rows(rows, rot, theta):
    inv = 1.0 / theta ** (torch.arange(0, rot, 2, dtype=torch.float64) / rot)
    f = torch.arange(rows, dtype=torch.float64)[:, None] * inv[None]
    emb = torch.cat((f, f), dim=-1)
    return H.bf(emb.cos().float()), H.bf(emb.sin().float())


# the last rows reach the C4 workload's depth (a 32-token prompt + 2,048 new
# tokens: positions up to 2,079) at batch 1 and 16, with fixed split lengths and
# with lengths derived from each row's position (split_len 0: the engines'
# default, over the engines' split count or over 2)
_C4_ROWS16 = [2040 + 3 * i for i in range(13)] + [2078, 2079, 2047]
_C4_MIXED = [0, 15, 16, 17, 127, 128, 129, 300, 511, 512, 640, 700, 701, 750, 3, 64]


@pytest.mark.parametrize("pos,split_len,nsplit", [
    ([0], 128, None), ([511], 128, None), ([700], 512, None), (_C4_MIXED, 128, None),
    ([2040], 64, None), ([2079], 64, None), (_C4_ROWS16, 64, None),
    ([2079], 0, None), (_C4_ROWS16, 0, None), (_C4_MIXED, 0, None), (_C4_MIXED, 0, 2)])
def test_gqa_decode_c4(gpu_device, pos, split_len, nsplit):
    """Qwen3.5 full attention: 16 q / 2 kv heads of 256, RoPE on 64 dims."""
    g = torch.Generator().manual_seed(len(pos) * 1000 + pos[0] + split_len)
    B, HQ, HKV, D, rot = len(pos), 16, 2, 256, 64
    max_pages = max(48, -(-(max(pos) + 1) // 16))
    qg = H.bf(torch.randn(B, HQ, 2 * D, generator=g))
    k = H.bf(torch.randn(B, HKV, D, generator=g))
    v = H.bf(torch.randn(B, HKV, D, generator=g))
    pasts = [(H.bf(torch.randn(p, HKV, D, generator=g)), H.bf(torch.randn(p, HKV, D, generator=g)))
             for p in pos]
    gq = H.bf(1 + 0.2 * torch.randn(D, generator=g))
    gk = H.bf(1 + 0.2 * torch.randn(D, generator=g))
    cos, sin = _rope_rows(max(1024, max(pos) + 1), rot, 1e7)
    scale = D ** -0.5
    ldq = HQ * 2 * D + 2 * HKV * D + 8
    qkv = torch.zeros(B, ldq)
    qkv[:, :HQ * 2 * D] = qg.reshape(B, -1)
    qkv[:, HQ * 2 * D:HQ * 2 * D + HKV * D] = k.reshape(B, -1)
    qkv[:, HQ * 2 * D + HKV * D:HQ * 2 * D + 2 * HKV * D] = v.reshape(B, -1)
    kpool, vpool, table = _paged_pool(pasts, HKV, D, max_pages, g)
    got, kp, vp, err = _gqa_call(qkv, torch.tensor(pos), table, kpool, vpool, heads=HQ,
                                 kv_heads=HKV, head_dim=D, scale=scale, split_len=split_len,
                                 policy=_lib.POLICY_F32, gamma_q=gq, gamma_k=gk, cos=cos,
                                 sin=sin, nsplit=nsplit)
    assert err == 0
    P = torch.tensor(pos)
    want, k_rope = H.qwen35_attend(qg, k, v, [p[0] for p in pasts], [p[1] for p in pasts], gq,
                                   gk, cos[P], sin[P], scale)
    r = assert_close_bf16(got, H.bf(want), max_rel=1e-2, min_cos=0.99999, name="gqa c4")
    assert r["within_1ulp"] >= 0.999, r
    pg = table[torch.arange(B), P // 16].long()
    torch.testing.assert_close(kp[pg, :, P % 16].float(), H.bf(k_rope), atol=0, rtol=1e-2)
    assert torch.equal(vp[pg, :, P % 16].float(), v)


_C5_DEEP = [8191, 8192, 8000, 4095, 8191, 6000, 8190, 7777]
_C5_MIXED = [0, 1, 2, 100, 255, 256, 1000, 2000]


# split_len 0: lengths derived from each row's position over the engines'
# split count, or over 16 at 8,192 positions (512-position splits, the longest)
@pytest.mark.parametrize("pos,split_len,nsplit", [
    (_C5_MIXED, 256, None), ([1999], 16, None), ([37], 512, None), (_C5_DEEP, 256, None),
    (_C5_MIXED, 0, None), (_C5_DEEP, 0, None), ([8191, 1, 511, 4000], 0, 16)])
def test_gqa_decode_c5(gpu_device, pos, split_len, nsplit):
    """Granite attention: 32 q / 8 kv heads of 128, no RoPE, HIR rounding; up to
    the workload's depth (8 rows at 8,192-token contexts)."""
    g = torch.Generator().manual_seed(len(pos) * 100 + pos[0] + split_len)
    B, HQ, HKV, D = len(pos), 32, 8, 128
    max_pages = max(128, -(-(max(pos) + 1) // 16))
    q = H.bf(torch.randn(B, HQ, D, generator=g))
    k = H.bf(torch.randn(B, HKV, D, generator=g))
    v = H.bf(torch.randn(B, HKV, D, generator=g))
    pasts = [(H.bf(torch.randn(p, HKV, D, generator=g)), H.bf(torch.randn(p, HKV, D, generator=g)))
             for p in pos]
    scale = 0.05
    qkv = torch.cat([q.reshape(B, -1), k.reshape(B, -1), v.reshape(B, -1)], dim=1).to(BF)
    kpool, vpool, table = _paged_pool(pasts, HKV, D, max_pages, g)
    got, kp, vp, err = _gqa_call(qkv, torch.tensor(pos), table, kpool, vpool, heads=HQ,
                                 kv_heads=HKV, head_dim=D, scale=scale, split_len=split_len,
                                 policy=_lib.POLICY_BF16, nsplit=nsplit)
    assert err == 0
    want = H.granite_attend(q, k, v, [p[0] for p in pasts], [p[1] for p in pasts], scale)
    r = assert_close_bf16(got, want, max_rel=2e-2, min_cos=0.9999, name="gqa c5")
    assert r["within_1ulp"] >= 0.99, r
    P = torch.tensor(pos)
    pg = table[torch.arange(B), P // 16].long()
    assert torch.equal(kp[pg, :, P % 16].float(), k)
    assert torch.equal(vp[pg, :, P % 16].float(), v)


def test_gqa_decode_flags_a_position_past_the_table(gpu_device):
    """A position beyond the page table raises TFD_ERR_POS_RANGE; no block reads
    the cache for that sequence, the others are served."""
    g = torch.Generator().manual_seed(5)
    B, HQ, HKV, D = 2, 32, 8, 128
    pasts = [(torch.zeros(3, HKV, D), torch.zeros(3, HKV, D))] * 2
    kpool, vpool, table = _paged_pool(pasts, HKV, D, 4, g)
    qkv = H.bf(torch.randn(B, (HQ + 2 * HKV) * D, generator=g)).to(BF)
    _, _, _, err = _gqa_call(qkv, torch.tensor([3, 64]), table, kpool, vpool, heads=HQ,
                             kv_heads=HKV, head_dim=D, scale=0.1, split_len=16,
                             policy=_lib.POLICY_BF16)
    assert err == _lib.ERR_POS_RANGE
