"""The small-batch C4 kernels (rows <= 4; csrc/hybrid_small.hip) on the GPU.

* Row GEMV: every prologue's bf16 rows equal what the batched kernels stage
  (tfd_rmsnorm_f32_rows; tfd_gdn_step's gated norm; the operand-order and
  row-major inputs as given) bit for bit; the outputs within one bf16 ulp of
  bf16(W x) summed in f64 (the f32 sums run in another order) for >= 99.9% of
  them and to the bf16 bar everywhere; the residual epilogue adds exactly the
  value the store epilogue writes.
* The delta rule over value columns: conv windows, recurrent state and the
  gated read-out bit-identical to tfd_gdn_step over two chained tokens, and
  against the oracle's gdn_step to the bf16 bar.
* The two-launch experts: output, routing weights and ids, SwiGLU vectors and
  the shared expert's gate bit-identical to tfd_moe_experts routing inside the
  call, and the output against the oracle's moe_c4.
"""
import ctypes

import pytest
import torch

from oracle import hybrid_ref as H
from tests._parity import assert_close_bf16, report
from tests.test_gpu_batch import from_operand_order, operand_order
from tilefoundry_amd import _lib
from tilefoundry_amd._lib import lib, ptr

pytestmark = pytest.mark.gpu

BF = torch.bfloat16
DEV = "cuda:0"


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _rowgemv(x, ldx, kind, w, out, *, rows, gamma=None, gate=None, ldg=0, resid=False,
             x_rows=None, eps=1e-6):
    N, K = w.shape
    a = _lib.TfdRowGemvArgs()
    a.x, a.ldx, a.x_kind = ptr(x), ldx, kind
    a.gamma = None if gamma is None else ptr(gamma)
    a.gate, a.ldg, a.head_dim, a.eps = gate, ldg, 128, eps
    a.w, a.K, a.N = ptr(w), K, N
    a.out, a.ldo = ptr(out), out.shape[-1]
    a.epilogue = _lib.EPI_RESID_F32 if resid else _lib.EPI_LOGITS
    a.x_rows, a.ldxr = (None, 0) if x_rows is None else (ptr(x_rows), x_rows.shape[-1])
    a.rows = rows
    lib().tfd_rowgemv_bf16(ctypes.addressof(a), _stream())


def _check_gemv(got, w, xb, name, min_cos=0.99999):
    want = H.bf(H.mm_rows(w.float().cpu(), xb.float().cpu()))
    r = assert_close_bf16(got.cpu(), want, max_rel=1e-2, min_cos=min_cos, name=name)
    assert r["within_1ulp"] >= 0.999, (name, r)


# N = 1,001: not a multiple of the rows per wave.  N <= 512 at K = 2,048 takes
# the one-row-per-wave kernel (the C4 router's 256 rows; 509 leaves a ragged
# last block of waves)
@pytest.mark.parametrize("rows,K,N", [(1, 2048, 1001), (3, 2048, 1001), (4, 2048, 1001),
                                      (1, 4096, 1001), (2, 4096, 1001),
                                      (1, 2048, 256), (2, 2048, 256), (4, 2048, 256),
                                      (1, 2048, 509), (3, 2048, 509), (4, 2048, 509)])
def test_rowgemv_norm_prologue(gpu_device, rows, K, N):
    g = torch.Generator().manual_seed(rows * K + N)
    x = (torch.randn(rows, K + 8, generator=g) * 3).to(DEV)
    gamma = (1 + 0.2 * torch.randn(K, generator=g)).to(BF).to(DEV)
    w = (torch.randn(N, K, generator=g) * 0.03).to(BF).to(DEV)
    out = torch.full((rows, N + 3), float("nan"), device=DEV)
    xr = torch.full((rows, K + 16), float("nan"), device=DEV, dtype=BF)
    _rowgemv(x, K + 8, _lib.ROWX_NORM_F32, w, out, rows=rows, gamma=gamma, x_rows=xr)
    want_x = torch.full((rows, K), float("nan"), device=DEV, dtype=BF)
    lib().tfd_rmsnorm_f32_rows(ptr(x), K + 8, ptr(gamma), ptr(want_x), K, None, rows, K, 1e-6,
                               _stream())
    torch.cuda.synchronize()
    assert torch.equal(xr[:, :K], want_x)
    _check_gemv(out[:, :N], w, want_x, f"norm rows={rows} K={K}")
    # the residual epilogue adds the stored value into the stream, in place
    base = torch.randn(rows, N + 3, generator=g).to(DEV)
    acc = base.clone()
    _rowgemv(x, K + 8, _lib.ROWX_NORM_F32, w, acc, rows=rows, gamma=gamma, resid=True)
    torch.cuda.synchronize()
    assert torch.equal(acc[:, :N], base[:, :N] + out[:, :N])
    assert torch.equal(acc[:, N:], base[:, N:])


@pytest.mark.parametrize("rows", [1, 4])
def test_rowgemv_operand_and_row_inputs(gpu_device, rows):
    g = torch.Generator().manual_seed(40 + rows)
    K, N = 4096, 2048
    xb = (torch.randn(rows, K, generator=g)).to(BF).to(DEV)
    w = (torch.randn(N, K, generator=g) * 0.02).to(BF).to(DEV)
    o1 = torch.full((rows, N), float("nan"), device=DEV)
    o2 = torch.full((rows, N), float("nan"), device=DEV)
    xr = torch.full((rows, K), float("nan"), device=DEV, dtype=BF)
    xo = operand_order(xb)
    _rowgemv(xo, 0, _lib.ROWX_OPERAND, w, o1, rows=rows, x_rows=xr)
    _rowgemv(xb, K, _lib.ROWX_ROWS, w, o2, rows=rows)
    torch.cuda.synchronize()
    assert torch.equal(xr, xb)
    assert torch.equal(o1, o2)
    _check_gemv(o1, w, xb, f"operand rows={rows}")


def test_rowgemv_head_shape(gpu_device):
    """The C4 head's shape at batch 1: 248,320 rows, a grid-stride loop of many
    groups per wave."""
    g = torch.Generator().manual_seed(5)
    K, N = 2048, 248320
    x = torch.randn(1, K, generator=g).to(DEV)
    gamma = (1 + 0.1 * torch.randn(K, generator=g)).to(BF).to(DEV)
    w = (torch.randn(N, K, generator=g) * 0.02).to(BF).to(DEV)
    out = torch.full((1, N), float("nan"), device=DEV)
    xr = torch.empty(1, K, device=DEV, dtype=BF)
    _rowgemv(x, K, _lib.ROWX_NORM_F32, w, out, rows=1, gamma=gamma, x_rows=xr)
    torch.cuda.synchronize()
    # (torch's f32 cosine over 248k values carries ~1e-5 of its own error)
    _check_gemv(out, w, xr, "head", min_cos=0.9999)


def test_rowgemv_rejects_bad_shapes(gpu_device):
    w = torch.zeros(16, 1024, device=DEV, dtype=BF)
    out = torch.zeros(1, 16, device=DEV)
    with pytest.raises(_lib.TFDError):                       # K not 2048 / 4096
        _rowgemv(out, 1024, _lib.ROWX_ROWS, w, out, rows=1)
    w = torch.zeros(16, 2048, device=DEV, dtype=BF)
    x = torch.zeros(8, 2048, device=DEV)
    with pytest.raises(_lib.TFDError):                       # rows > 4
        _rowgemv(x, 2048, _lib.ROWX_ROWS, w, torch.zeros(8, 16, device=DEV), rows=5)
    with pytest.raises(_lib.TFDError):                       # the norm needs gamma
        _rowgemv(x, 2048, _lib.ROWX_NORM_F32, w, out, rows=1)


# ---------------------------------------------------------------------------
# Gated DeltaNet over value columns
# ---------------------------------------------------------------------------
def _gdn_inputs(rows, g, hk=16, hv=32):
    key, val = hk * 128, hv * 128
    conv = 2 * key + val
    return dict(
        proj=H.bf(torch.randn(rows, conv + val + 2 * hv, generator=g)),
        conv_state=torch.randn(rows, conv, 3, generator=g),
        state=torch.randn(rows, hv, 128, 128, generator=g) * 0.05,
        conv_w=H.bf(torch.randn(conv, 4, generator=g) * 0.5),
        a_log=H.bf(torch.randn(hv, generator=g) * 0.5),
        dt_bias=H.bf(torch.randn(hv, generator=g) * 0.5),
        gamma=H.bf(1 + 0.1 * torch.randn(128, generator=g)), hk=hk, hv=hv)


def _gdn_args(inp, proj_d, cin, cout, st, params, out):
    rows = proj_d.shape[0]
    a = _lib.TfdGdnArgs()
    a.proj, a.proj_ld, a.conv_in, a.conv_out, a.state = ptr(proj_d), proj_d.shape[1], ptr(cin), \
        ptr(cout), ptr(st)
    a.conv_w, a.a_log, a.dt_bias, a.gamma = [ptr(p) for p in params]
    a.out = None if out is None else ptr(out)
    a.rows, a.key_heads, a.value_heads, a.head_k_dim, a.head_v_dim, a.conv_kernel = \
        rows, inp["hk"], inp["hv"], 128, 128, 4
    a.l2_eps, a.rms_eps = 1e-6, 1e-6
    return a


@pytest.mark.parametrize("rows", [1, 3])
def test_gdn_cols_equal_the_fused_step(gpu_device, rows):
    g = torch.Generator().manual_seed(70 + rows)
    inp = _gdn_inputs(rows, g)
    hv, val = inp["hv"], inp["hv"] * 128
    conv = 2 * inp["hk"] * 128 + val
    params = [inp[n].to(DEV).to(BF) for n in ("conv_w", "a_log", "dt_bias", "gamma")]
    conv_ref, state_ref = inp["conv_state"], inp["state"]
    # two independent copies of the recurrent inputs, one per path
    cin = [inp["conv_state"].to(DEV).contiguous() for _ in range(2)]
    st = [inp["state"].to(DEV).contiguous() for _ in range(2)]
    for step in range(2):
        proj = inp["proj"] if step == 0 else H.bf(torch.randn(inp["proj"].shape, generator=g))
        proj_d = torch.zeros(rows, proj.shape[1] + 8, device=DEV)
        proj_d[:, :proj.shape[1]] = proj.to(DEV)
        cout = [torch.full_like(cin[0], float("nan")) for _ in range(2)]
        fused = torch.full((32 * val,), float("nan"), device=DEV, dtype=BF)
        a0 = _gdn_args(inp, proj_d, cin[0], cout[0], st[0], params, fused)
        lib().tfd_gdn_step(ctypes.addressof(a0), _stream())
        read = torch.full((rows, val), float("nan"), device=DEV)
        a1 = _gdn_args(inp, proj_d, cin[1], cout[1], st[1], params, None)
        lib().tfd_gdn_step_cols(ctypes.addressof(a1), ptr(read), val, _stream())
        # the gated norm as the out-projection's prologue, its bf16 rows kept
        w = torch.zeros(8, val, device=DEV, dtype=BF)
        o = torch.zeros(rows, 8, device=DEV)
        gated = torch.full((rows, val), float("nan"), device=DEV, dtype=BF)
        _rowgemv(read, val, _lib.ROWX_GATED_F32, w, o, rows=rows, gamma=params[3],
                 gate=ptr(proj_d) + 4 * conv, ldg=proj_d.shape[1], x_rows=gated)
        torch.cuda.synchronize()
        assert torch.equal(cout[1], cout[0]), step
        assert torch.equal(st[1], st[0]), step
        assert torch.equal(gated, from_operand_order(fused, rows, val)), step
        want, conv_ref, state_ref = H.gdn_step(
            proj, conv_ref, state_ref, inp["conv_w"], inp["a_log"], inp["dt_bias"],
            inp["gamma"], hk=inp["hk"], hv=hv, dk=128, dv=128)
        assert torch.equal(cout[1].cpu(), conv_ref), step
        torch.testing.assert_close(st[1].cpu(), state_ref, atol=1e-5, rtol=1e-4)
        r = assert_close_bf16(gated.float().cpu(), H.bf(want), max_rel=1e-2, min_cos=0.99999,
                              name=f"gdn cols step {step}")
        assert r["within_1ulp"] >= 0.999, r
        cin = cout


# ---------------------------------------------------------------------------
# Experts in two launches
# ---------------------------------------------------------------------------
def _moe_args(d, *, rows, k, E, hs, inter, route_logits):
    a = _lib.TfdMoeArgs()
    a.x, a.weights, a.idx = ptr(d["x"]), ptr(d["weights"]), ptr(d["idx"])
    a.w_gate, a.w_up, a.w_down = ptr(d["w_gate"]), ptr(d["w_up"]), ptr(d["w_down"])
    a.w_shared_in, a.w_shared_out = ptr(d["w_sin"]), ptr(d["w_sout"])
    a.w_shared_scale = ptr(d["w_sscale"])
    a.hidden, a.shared_scale, a.out = ptr(d["hidden"]), ptr(d["sscale"]), ptr(d["out"])
    a.partial, a.groups = ptr(d["partial"]), ptr(d["groups"])
    a.rows, a.k, a.experts, a.hidden_size = rows, k, E, hs
    a.inter, a.shared_inter, a.hidden_ld = inter, inter, inter
    a.fp8, a.policy, a.err = 0, _lib.POLICY_F32, ptr(d["err"])
    a.accumulate = 1
    a.logits, a.ldl, a.route = ptr(route_logits), E, _lib.MOE_ROUTE_SOFTMAX_TOPK
    return a


@pytest.mark.parametrize("rows,E", [(1, 256), (2, 64), (4, 16)])
def test_moe_small_equals_the_grouped_experts(gpu_device, rows, E):
    g = torch.Generator().manual_seed(90 + rows)
    hs, inter, k = 2048, 512, 8
    rnd = lambda *s, std=0.03: H.bf(torch.randn(*s, generator=g) * std)
    x = rnd(rows, hs, std=1.0)
    logits = H.bf(torch.randn(rows, E, generator=g) * 2)
    w_gate, w_up, w_down = rnd(E, inter, hs), rnd(E, inter, hs), rnd(E, hs, inter)
    ws_gate, ws_up, ws_down, ws_scale = rnd(inter, hs), rnd(inter, hs), rnd(hs, inter), rnd(1, hs)
    base = torch.randn(rows, hs, generator=g)
    shared = dict(x=x.to(BF), w_gate=w_gate.to(BF), w_up=w_up.to(BF), w_down=w_down.to(BF),
                  w_sin=torch.cat([ws_gate, ws_up]).to(BF), w_sout=ws_down.to(BF),
                  w_sscale=ws_scale.to(BF))
    shared = {n: v.to(DEV).contiguous() for n, v in shared.items()}
    lg = logits.to(DEV).contiguous()
    runs = []
    for entry in ("tfd_moe_experts", "tfd_moe_experts_small"):
        d = dict(shared)
        d.update(weights=torch.full((rows, k), float("nan"), device=DEV),
                 idx=torch.full((rows, k), -1, device=DEV, dtype=torch.int32),
                 hidden=torch.zeros(rows, k + 1, inter, device=DEV, dtype=BF),
                 sscale=torch.full((rows,), float("nan"), device=DEV),
                 out=base.to(DEV).clone(),
                 partial=torch.zeros(rows, k + 1, hs, device=DEV),
                 groups=torch.zeros(_lib.moe_group_words(E, rows), device=DEV, dtype=torch.int32),
                 err=torch.zeros(1, device=DEV, dtype=torch.int32))
        a = _moe_args(d, rows=rows, k=k, E=E, hs=hs, inter=inter, route_logits=lg)
        getattr(lib(), entry)(ctypes.addressof(a), _stream())
        torch.cuda.synchronize()
        assert d["err"].item() == 0, entry
        runs.append(d)
    ref, small = runs
    for n in ("idx", "weights", "hidden", "sscale", "out"):
        assert torch.equal(small[n], ref[n]), n
    weights, idx = H.route_softmax_topk(logits, k)
    assert torch.equal(small["idx"].cpu().long(), idx.long())
    want = H.moe_c4(x, weights, idx, w_gate, w_up, w_down, ws_gate, ws_up, ws_down, ws_scale)
    assert_close_bf16((small["out"].cpu() - base), want, max_rel=1e-2, min_cos=0.99999,
                      name=f"moe small rows={rows}")


def test_moe_small_rejects_what_it_does_not_serve(gpu_device):
    a = _lib.TfdMoeArgs()
    with pytest.raises(_lib.TFDError):
        lib().tfd_moe_experts_small(ctypes.addressof(a), _stream())     # null pointers
    t = torch.zeros(64, device=DEV)
    for n in ("x", "weights", "idx", "w_gate", "w_up", "w_down", "w_shared_in", "w_shared_out",
              "hidden", "out"):
        setattr(a, n, ptr(t))
    a.rows, a.k, a.experts, a.hidden_size, a.inter, a.shared_inter, a.hidden_ld = \
        5, 8, 16, 2048, 512, 512, 512
    with pytest.raises(_lib.TFDError):                                   # rows > 4
        lib().tfd_moe_experts_small(ctypes.addressof(a), _stream())
    a.rows, a.fp8 = 1, 1
    with pytest.raises(_lib.TFDError):                                   # fp8 weights
        lib().tfd_moe_experts_small(ctypes.addressof(a), _stream())
