"""Per-kernel HBM roofline of the hybrid models' decode kernels.

    python -m tilefoundry_amd.hybrid.bench [--config c4|c4b16|c5|all] [--reps 20]
    python -m tilefoundry_amd.hybrid.bench --config c4-step --rows 1|16 [--steps 256]
    python -m tilefoundry_amd.hybrid.bench --config c5-step --rows 8 [--steps 256]
    python -m tilefoundry_amd.hybrid.bench --config gemm [--reps 20]

Every kernel runs at its workload's shapes on synthetic data (seeded) with the
launches of one measurement captured in a HIP graph and replayed; HIP events on
the capture stream time the replay, and the average launch duration divides the
kernel's ALGORITHMIC bytes (what one launch must move at least: weights, state
read and written, cache rows) into GB/s against the 8 TB/s HBM peak.  Buffers
rotate over enough copies (weights of other experts, the state of other layers)
that one launch's data is not left in the 256 MB last-level cache by the
previous ones.  One JSON line per kernel.

Shapes (the workloads' published architectures):
  C4 (Qwen3.5-35B-A3B-style, batch 1 or 16): GDN 16 key / 32 value heads of 128,
     conv 4; MoE 256 experts, top 8, hidden 2048, expert 512, shared 512 (bf16);
     full attention 16 q / 2 kv heads of 256, RoPE on 64 dims, context 1024.
  C5 (Granite-4.0-H-small-style, batch 8): Mamba2 64 heads of 64, state 128;
     MoE 72 experts, top 10, hidden 4096, expert 768, shared 1536, fp8 weights;
     attention 32 q / 8 kv heads of 128 over an 8192-token context; the fp8
     in_proj (8512 x 4096) and out_proj (4096 x 4096).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import time

import torch

from .. import _lib
from .._lib import lib, ptr

HBM_PEAK = 8.0e12
BF = torch.bfloat16
DEV = "cuda:0"


def _stream():
    return torch.cuda.current_stream().cuda_stream


def time_graph(calls, reps: int) -> float:
    """Average seconds per launch of `calls` (a list of zero-argument launchers,
    each one kernel entry), replayed `reps` times inside one captured graph."""
    reps = max(1, min(reps, 4096 // len(calls)))
    for c in calls:
        c()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for _ in range(reps):
                for c in calls:
                    c()
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    # the median of five timed replays: one replay of a few short launches can
    # catch an unrelated stall of the device
    times = []
    for _ in range(5):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        e1.synchronize()
        times.append(e0.elapsed_time(e1) * 1e-3)
    return sorted(times)[2] / (reps * len(calls))


def _line(config, kernel, rows, sec, nbytes, **extra):
    out = {"config": config, "kernel": kernel, "rows": rows, "us": round(sec * 1e6, 3),
           "bytes": int(nbytes), "GB/s": round(nbytes / sec / 1e9, 1),
           "frac": round(nbytes / sec / HBM_PEAK, 4), **extra}
    print(json.dumps(out), flush=True)
    return out


def _rn(*shape, gen):
    """N(0, 1) f32 on the device, from the device generator `gen`."""
    return torch.randn(*shape, generator=gen, device=DEV)


def _fp8(shape, gen):
    return (_rn(*shape, gen=gen) * 0.6).to(torch.float8_e4m3fn).view(torch.uint8)


# ---------------------------------------------------------------------------
def bench_gdn(config, rows, reps, gen):
    hk, hv, d = 16, 32, 128
    key, val = hk * d, hv * d
    conv = 2 * key + val
    ldp = conv + val + 2 * hv
    copies = min(256, max(2, -(-(1 << 30) // (rows * hv * d * d * 4))))     # states past the cache
    proj = (_rn(rows, ldp, gen=gen)).to(DEV)
    states = [_rn(rows, hv, d, d, gen=gen).mul_(0.05).to(DEV) for _ in range(copies)]
    cin = _rn(rows, conv, 3, gen=gen).to(DEV)
    couts = [torch.empty_like(cin) for _ in range(copies)]
    conv_w = (_rn(conv, 4, gen=gen) * 0.5).to(BF).to(DEV)
    a_log, dt_bias = [(_rn(hv, gen=gen) * 0.5).to(BF).to(DEV) for _ in range(2)]
    gamma = torch.ones(d, dtype=BF, device=DEV)
    out = torch.empty(32 * val, dtype=BF, device=DEV)
    args = []
    for i in range(copies):
        a = _lib.TfdGdnArgs()
        a.proj, a.proj_ld, a.conv_in, a.conv_out, a.state = ptr(proj), ldp, ptr(cin), \
            ptr(couts[i]), ptr(states[i])
        a.conv_w, a.a_log, a.dt_bias, a.gamma, a.out = ptr(conv_w), ptr(a_log), ptr(dt_bias), \
            ptr(gamma), ptr(out)
        a.rows, a.key_heads, a.value_heads, a.head_k_dim, a.head_v_dim, a.conv_kernel = \
            rows, hk, hv, d, d, 4
        a.l2_eps, a.rms_eps = 1e-6, 1e-6
        args.append(a)
    L = lib()
    calls = [lambda a=a: L.tfd_gdn_step(ctypes.addressof(a), _stream()) for a in args]
    sec = time_graph(calls, reps)
    per_row = hv * d * d * 4 * 2 + conv * 3 * 4 * 2 + ldp * 4 + val * 2
    nbytes = rows * per_row + conv * 4 * 2 + 2 * hv * 2 + d * 2
    return _line(config, "gdn_step", rows, sec, nbytes)


def bench_mamba(config, rows, reps, gen):
    nh, pd, ns = 64, 64, 128
    exp_ = nh * pd
    conv = exp_ + 2 * ns
    ldp = exp_ + conv + nh
    copies = min(256, max(2, -(-(1 << 30) // (rows * nh * pd * ns * 4))))
    proj = _rn(rows, ldp, gen=gen).to(BF).to(DEV)
    states = [_rn(rows, nh, pd, ns, gen=gen).mul_(0.3).to(DEV) for _ in range(copies)]
    cin = _rn(rows, conv, 3, gen=gen).to(BF).to(DEV)
    couts = [torch.empty_like(cin) for _ in range(copies)]
    conv_w = (_rn(conv, 4, gen=gen) * 0.5).to(BF).to(DEV)
    conv_b = (_rn(conv, gen=gen) * 0.1).to(BF).to(DEV)
    small = [(_rn(nh, gen=gen) * 0.5).to(BF).to(DEV) for _ in range(3)]
    gamma = torch.ones(exp_, dtype=BF, device=DEV)
    gated = torch.empty(rows, exp_, device=DEV)
    ssq = torch.empty(rows, nh, device=DEV)
    out = torch.empty(32 * exp_, dtype=BF, device=DEV)
    args = []
    for i in range(copies):
        a = _lib.TfdMambaArgs()
        a.proj, a.proj_ld, a.conv_in, a.conv_out, a.state = ptr(proj), ldp, ptr(cin), \
            ptr(couts[i]), ptr(states[i])
        a.conv_w, a.conv_b = ptr(conv_w), ptr(conv_b)
        a.a_log, a.dt_bias, a.d_skip = [ptr(t) for t in small]
        a.gamma, a.gated, a.ssq, a.out = ptr(gamma), ptr(gated), ptr(ssq), ptr(out)
        a.rows, a.heads, a.head_dim, a.state_dim, a.groups, a.conv_kernel = rows, nh, pd, ns, 1, 4
        a.eps = 1e-5
        args.append(a)
    L = lib()
    calls = [lambda a=a: L.tfd_mamba_step(ctypes.addressof(a), _stream()) for a in args]
    sec = time_graph(calls, reps)
    per_row = (nh * pd * ns * 4 * 2 + conv * 3 * 2 * 2 + ldp * 2 + exp_ * 4 * 2 + nh * 4 * 2 +
               exp_ * 2)
    nbytes = rows * per_row + conv * 4 * 2 + conv * 2 + 3 * nh * 2 + exp_ * 2
    return _line(config, "mamba_step", rows, sec, nbytes)


def _pack_rows(w):
    """[rows][K] weights in the skinny GEMMs' operand blocks (bf16 or fp8 codes)."""
    N, K = w.shape
    out = torch.empty(-(-N // 16) * 16 * K, dtype=w.dtype, device=DEV)
    fn = lib().tfd_pack_skinny_fp8 if w.dtype == torch.uint8 else lib().tfd_pack_skinny_bf16
    fn(ptr(w), K, N, K, ptr(out), _stream())
    return out


def bench_moe(config, rows, reps, gen, *, hs, inter, sh, experts, k, fp8, packed=False):
    """tfd_moe_experts over row-major weights, or with *packed* the matrix-core
    entry tfd_moe_experts_packed over packed weights (no partials)."""
    bpw = 1 if fp8 else 2
    if fp8:
        w_gate, w_up = _fp8((experts, inter, hs), gen), _fp8((experts, inter, hs), gen)
        w_down = _fp8((experts, hs, inter), gen)
        w_sin, w_sout = _fp8((2 * sh, hs), gen), _fp8((hs, sh), gen)
        sc = lambda *s: (torch.rand(*s, generator=gen, device=DEV) * 0.004 + 0.002)
        scales = [sc(experts, inter), sc(experts, inter), sc(experts, hs), sc(2 * sh), sc(hs)]
    else:
        rnd = lambda *s: (_rn(*s, gen=gen) * 0.03).to(BF)
        w_gate, w_up, w_down = rnd(experts, inter, hs), rnd(experts, inter, hs), \
            rnd(experts, hs, inter)
        w_sin, w_sout = rnd(2 * sh, hs), rnd(hs, sh)
        scales = [None] * 5
    dev = [t.to(DEV) if t is not None else None for t in
           (w_gate, w_up, w_down, w_sin, w_sout, *scales)]
    if packed:
        dev[:5] = [_pack_rows(t.reshape(-1, t.shape[-1])) for t in dev[:5]]
    w_sscale = None if fp8 else (_rn(hs, gen=gen) * 0.03).to(BF).to(DEV)
    x = _rn(rows, hs, gen=gen).to(BF).to(DEV)
    ld = max(inter, sh)
    hidden = torch.empty(rows, k + 1, ld, dtype=BF, device=DEV)
    partial = torch.empty(rows, k + 1, hs, device=DEV)
    groups = torch.empty(_lib.moe_group_words(experts, rows), dtype=torch.int32, device=DEV)
    sscale = torch.empty(rows, device=DEV)
    out = torch.empty(rows, hs, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    # a fresh routing per launch (uniform: router logits N(0,1) pick near-uniformly)
    routes = []
    unions = []
    cpu_gen = torch.Generator().manual_seed(1)
    for _ in range(16):
        idx = torch.stack([torch.randperm(experts, generator=cpu_gen)[:k] for _ in range(rows)])
        w = torch.rand(rows, k, generator=cpu_gen) + 0.1
        routes.append(((w / w.sum(-1, keepdim=True)).to(DEV), idx.to(torch.int32).to(DEV)))
        unions.append(len(set(idx.reshape(-1).tolist())))
    args = []
    for wts, idx in routes:
        a = _lib.TfdMoeArgs()
        a.x, a.weights, a.idx = ptr(x), ptr(wts), ptr(idx)
        a.w_gate, a.w_up, a.w_down, a.w_shared_in, a.w_shared_out = [ptr(t) for t in dev[:5]]
        a.s_gate, a.s_up, a.s_down, a.s_shared_in, a.s_shared_out = [ptr(t) for t in dev[5:]]
        a.w_shared_scale = ptr(w_sscale)
        a.hidden, a.shared_scale, a.out = ptr(hidden), ptr(sscale), ptr(out)
        a.partial, a.groups = (None if packed else ptr(partial)), ptr(groups)
        a.rows, a.k, a.experts, a.hidden_size = rows, k, experts, hs
        a.inter, a.shared_inter, a.hidden_ld = inter, sh, ld
        a.fp8, a.policy, a.err = int(fp8), _lib.POLICY_BF16 if fp8 else _lib.POLICY_F32, ptr(err)
        args.append(a)
    L = lib()
    entry = L.tfd_moe_experts_packed if packed else L.tfd_moe_experts
    calls = [lambda a=a: entry(ctypes.addressof(a), _stream()) for a in args]
    sec = time_graph(calls, reps)
    union = sum(unions) / len(unions)
    wbytes = union * 3 * inter * hs * bpw + 3 * sh * hs * bpw
    if fp8:
        wbytes += union * (2 * inter + hs) * 4 + (2 * sh + hs) * 4
    else:
        wbytes += hs * 2
    nbytes = (wbytes + rows * hs * 2 + rows * hs * 4 + rows * (k + 1) * ld * 2 * 2 +
              (0 if packed else rows * (k + 1) * hs * 4 * 2))
    return _line(config, "moe_experts_packed" if packed else "moe_experts", rows, sec, nbytes,
                 experts_touched=round(union, 1))


def bench_route(config, rows, reps, gen, *, experts, k, mode):
    logits = _rn(rows, experts, gen=gen).to(DEV)
    w = torch.empty(rows, k, device=DEV)
    idx = torch.empty(rows, k, dtype=torch.int32, device=DEV)
    L = lib()
    calls = [lambda: L.tfd_route_topk(ptr(logits), experts, rows, experts, k, mode, ptr(w),
                                      ptr(idx), _stream())]
    sec = time_graph(calls, reps)
    return _line(config, "route_topk", rows, sec, rows * experts * 4 + rows * k * 8)


def bench_gqa(config, rows, reps, gen, *, heads, kv_heads, d, ctx, f32, split_len):
    max_pages = -(-(ctx + 1) // 16)
    num_pages = rows * max_pages
    copies = max(1, -(-(1 << 30) // (2 * num_pages * kv_heads * 16 * d * 2)))
    pools = [(_rn(num_pages, kv_heads, 16, d, gen=gen).to(BF).to(DEV),
              _rn(num_pages, kv_heads, 16, d, gen=gen).to(BF).to(DEV))
             for _ in range(copies)]
    cpu_gen = torch.Generator().manual_seed(2)
    table = torch.randperm(num_pages, generator=cpu_gen).view(rows, max_pages).to(torch.int32).to(DEV)
    pos = torch.full((rows,), ctx, dtype=torch.int32, device=DEV)
    qw = 2 * d if f32 else d
    ldq = heads * qw + 2 * kv_heads * d
    qkv = (_rn(rows, ldq, gen=gen).to(DEV) if f32 else
           _rn(rows, ldq, gen=gen).to(BF).to(DEV))
    if split_len is None:           # the engines' choice: lengths follow the position
        from .qwen3_5 import attention_splits
        nsplit, split_len = attention_splits(rows, kv_heads, max_pages * 16), 0
    else:
        nsplit = -(-max_pages * 16 // split_len)
    stride = max_pages * 16
    scores = torch.empty(rows * heads * stride, device=DEV)
    stats = torch.empty(rows * heads * nsplit * 2, device=DEV)
    part = torch.empty(rows * heads * nsplit * d, device=DEV)
    counters = torch.zeros(rows * kv_heads, dtype=torch.int32, device=DEV)
    out = torch.empty(32 * heads * d, dtype=BF, device=DEV)
    err = torch.zeros(1, dtype=torch.int32, device=DEV)
    rot = 64
    cos = torch.ones(ctx + 1, rot, dtype=BF, device=DEV)
    sin = torch.zeros(ctx + 1, rot, dtype=BF, device=DEV)
    gq = torch.ones(d, dtype=BF, device=DEV)
    args = []
    for kp, vp in pools:
        a = _lib.TfdGqaArgs()
        a.qkv, a.ldq = ptr(qkv), ldq
        if f32:
            a.gamma_q, a.gamma_k, a.cos_table, a.sin_table = ptr(gq), ptr(gq), ptr(cos), ptr(sin)
            a.rope_rows, a.rot_dim = ctx + 1, rot
        a.pos, a.page_table, a.max_pages = ptr(pos), ptr(table), max_pages
        a.k_pool, a.v_pool, a.num_pages = ptr(kp), ptr(vp), num_pages
        a.rows, a.heads, a.kv_heads, a.head_dim = rows, heads, kv_heads, d
        a.scale, a.eps = d ** -0.5, 1e-6
        a.scores, a.score_stride, a.stats, a.part = ptr(scores), stride, ptr(stats), ptr(part)
        a.counters, a.nsplit, a.split_len = ptr(counters), nsplit, split_len
        a.out, a.policy, a.err = ptr(out), _lib.POLICY_F32 if f32 else _lib.POLICY_BF16, ptr(err)
        args.append(a)
    L = lib()
    calls = [lambda a=a: L.tfd_gqa_decode(ctypes.addressof(a), _stream()) for a in args]
    sec = time_graph(calls, reps)
    live = ctx + 1
    nbytes = rows * (live * kv_heads * d * 2 * 2 + heads * live * 4 * 2 + ldq * (4 if f32 else 2))
    return _line(config, "gqa_decode (2 launches)", rows, sec, nbytes, context=ctx)


def bench_gemm_fp8(config, rows, reps, gen, *, K, N, name):
    copies = max(2, -(-(1 << 30) // (N * K)))
    ws = []
    for _ in range(copies):
        codes = _fp8((N, K), gen).to(DEV)
        packed = torch.empty(-(-N // 16) * 16 * K, dtype=torch.uint8, device=DEV)
        lib().tfd_pack_skinny_fp8(ptr(codes), K, N, K, ptr(packed), _stream())
        ws.append(packed)
    scale = (torch.rand(N, generator=gen, device=DEV) * 0.01).to(DEV)
    x = _rn(32 * K, gen=gen).to(BF).to(DEV)
    out = torch.empty(rows, N, dtype=BF, device=DEV)
    L = lib()
    calls = [lambda w=w: L.tfd_gemm_skinny_fp8(ptr(x), ptr(w), ptr(scale), rows, K, N,
                                               _lib.EPI_STORE, None, 0, ptr(out), N, _stream())
             for w in ws]
    sec = time_graph(calls, reps)
    nbytes = N * K + N * 4 + rows * K * 2 + rows * N * 2
    flops = 2 * rows * N * K
    return _line(config, f"gemm_skinny_fp8 {name}", rows, sec, nbytes,
                 TFLOPs=round(flops / sec / 1e12, 2), mfma_frac=round(flops / sec / 2.5e15, 4))


def bench_gemm_bf16(config, rows, reps, gen, *, K, N, name, epi):
    """The bf16 skinny MFMA GEMM (tfd_gemm_skinny_bf16) at one projection's shape:
    HBM bytes (weights + activations in and out) and MFMA TFLOP/s (2 M N K flops)
    against the 2.5 PFLOP/s dense bf16 peak."""
    copies = max(2, -(-(1 << 30) // (2 * N * K)))
    ws = []
    for _ in range(copies):
        rows_w = (_rn(N, K, gen=gen) * 0.02).to(BF)
        packed = torch.empty(-(-N // 16) * 16 * K, dtype=BF, device=DEV)
        lib().tfd_pack_skinny_bf16(ptr(rows_w), K, N, K, ptr(packed), _stream())
        ws.append(packed)
        del rows_w
    x = (_rn(32 * K, gen=gen) * 0.5).to(BF)
    if epi == _lib.EPI_SWIGLU:
        out, ldo = torch.empty(32 * (N // 2), dtype=BF, device=DEV), N // 2
    elif epi == _lib.EPI_LOGITS:
        out, ldo = torch.empty(rows, N, dtype=torch.float32, device=DEV), N
    else:
        out, ldo = torch.empty(rows, N, dtype=BF, device=DEV), N
    resid = torch.zeros(rows, N, dtype=BF, device=DEV) if epi == _lib.EPI_RESID else None
    work = torch.zeros(1 << 21, dtype=torch.float32, device=DEV)
    L = lib()
    calls = [lambda w=w: L.tfd_gemm_skinny_bf16(ptr(x), ptr(w), rows, K, N, epi, ptr(resid),
                                                N if resid is not None else 0, ptr(out), ldo,
                                                ptr(work), work.numel(), _stream())
             for w in ws]
    sec = time_graph(calls, reps)
    out_bytes = rows * N * (4 if epi == _lib.EPI_LOGITS else 2) // (2 if epi == _lib.EPI_SWIGLU
                                                                     else 1)
    nbytes = 2 * N * K + rows * K * 2 + out_bytes
    flops = 2 * rows * N * K
    return _line(config, f"gemm_skinny_bf16 {name}", rows, sec, nbytes,
                 TFLOPs=round(flops / sec / 1e12, 2), mfma_frac=round(flops / sec / 2.5e15, 4))


def run_gemm(reps: int) -> list[dict]:
    """Every batched projection on the MFMA path: C3 (batch 32) q/k/v, o, gate/up,
    down and the head; C4 batch 16's GDN and attention in/out projections, router
    and head; C5 batch 8's fp8 in_proj and out_proj."""
    gen = torch.Generator(device=DEV).manual_seed(0)
    res = []
    for name, K, N, epi in (("c3 qkv", 2048, 4096, _lib.EPI_STORE),
                            ("c3 o", 2048, 2048, _lib.EPI_RESID),
                            ("c3 gate/up", 2048, 12288, _lib.EPI_SWIGLU),
                            ("c3 down", 6144, 2048, _lib.EPI_RESID),
                            ("c3 head", 2048, 151936, _lib.EPI_LOGITS)):
        res.append(bench_gemm_bf16("c3", 32, reps, gen, K=K, N=N, name=name, epi=epi))
    for name, K, N in (("c4 gdn in", 2048, 12352), ("c4 gdn out", 4096, 2048),
                       ("c4 attn in", 2048, 9216), ("c4 attn out", 4096, 2048),
                       ("c4 router", 2048, 256), ("c4 head", 2048, 248320)):
        res.append(bench_gemm_bf16("c4b16", 16, reps, gen, K=K, N=N, name=name,
                                   epi=_lib.EPI_LOGITS))
    res.append(bench_gemm_fp8("c5", 8, reps, gen, K=4096, N=8512, name="in_proj"))
    res.append(bench_gemm_fp8("c5", 8, reps, gen, K=4096, N=4096, name="out_proj"))
    return res


def run(config: str, reps: int) -> list[dict]:
    gen = torch.Generator(device=DEV).manual_seed(0)
    res = []
    if config in ("c4", "c4b16"):
        rows = 1 if config == "c4" else 16
        res.append(bench_gdn(config, rows, reps, gen))
        res.append(bench_route(config, rows, reps, gen, experts=256, k=8,
                               mode=_lib.ROUTE_SOFTMAX_TOPK))
        res.append(bench_moe(config, rows, reps, gen, hs=2048, inter=512, sh=512, experts=256,
                             k=8, fp8=False))
        if rows > 1:
            res.append(bench_moe(config, rows, reps, gen, hs=2048, inter=512, sh=512,
                                 experts=256, k=8, fp8=False, packed=True))
        res.append(bench_gqa(config, rows, reps, gen, heads=16, kv_heads=2, d=256, ctx=1024,
                             f32=True, split_len=None))
    elif config == "c5":
        rows = 8
        res.append(bench_mamba(config, rows, reps, gen))
        res.append(bench_route(config, rows, reps, gen, experts=72, k=10,
                               mode=_lib.ROUTE_TOPK_SOFTMAX))
        for packed in (False, True):
            res.append(bench_moe(config, rows, reps, gen, hs=4096, inter=768, sh=1536,
                                 experts=72, k=10, fp8=True, packed=packed))
        res.append(bench_gqa(config, rows, reps, gen, heads=32, kv_heads=8, d=128, ctx=8192,
                             f32=False, split_len=None))
        res.append(bench_gemm_fp8(config, rows, reps, gen, K=4096, N=8512, name="in_proj"))
        res.append(bench_gemm_fp8(config, rows, reps, gen, K=4096, N=4096, name="out_proj"))
    else:
        raise ValueError(config)
    return res


def bench_c4_step(rows: int, steps: int, prompt: int = 32, small: bool | None = None) -> dict:
    """Whole C4 decode steps (Qwen3.5-35B-A3B shape, 40 layers, 248,320-token
    vocabulary, synthetic weights): tok/s over `steps` greedy steps after a
    `prompt`-token random prompt per sequence (walked untimed), and the step's
    algorithmic bytes (dense weights once, the experts the step picked once per
    layer, GDN state read and written, KV read) against 8 TB/s."""
    from .qwen3_5 import Qwen35Config, Qwen35Engine, synthetic_weights

    cfg = Qwen35Config()
    t0 = time.perf_counter()
    w = synthetic_weights(cfg, seed=0, device=DEV)
    eng = Qwen35Engine(cfg, w, rows=rows, device=DEV, max_steps=prompt + steps + 16, small=small)
    print(f"[bench] c4 weights + engine + capture {time.perf_counter() - t0:.1f}s", flush=True)
    g = torch.Generator().manual_seed(0)
    prompts = [torch.randint(0, cfg.vocab, (prompt,), generator=g).tolist() for _ in range(rows)]
    tokens, seconds, _ = eng.generate(prompts, steps)
    touched = len(set(eng.ridx.reshape(-1).tolist()))       # the last layer's picks, last step
    wbytes = eng.weight_bytes_per_step(touched)
    positions = range(prompt - 1, prompt - 1 + steps)
    sbytes = sum(eng.state_bytes_per_step([p] * rows) for p in positions) / steps
    step_s = seconds / steps
    out = {"config": f"c4 step b{rows}", "path": "small" if eng.small else "mfma",
           "tok_s": round(rows * steps / seconds, 1),
           "ms_per_step": round(step_s * 1e3, 4), "steps": steps,
           "bytes_per_step": int(wbytes + sbytes), "experts_touched_sample": touched,
           "GB/s": round((wbytes + sbytes) / step_s / 1e9, 1),
           "frac": round((wbytes + sbytes) / step_s / HBM_PEAK, 4),
           "first_tokens": tokens[0][:8]}
    print(json.dumps(out), flush=True)
    return out


def bench_c5_step(rows: int, steps: int, ctx: int = 8192, context: str = "drawn") -> dict:
    """Whole C5 decode steps (Granite-4.0-H-style, 40 layers, fp8 weights, batch
    `rows`) after a `ctx`-token context per sequence: drawn at random into the
    caches and states (GraniteEngine.synthetic_context: the work of each later
    step is that of a real context of that length), or with *context* "walk"
    built from a random prompt by GraniteEngine.prefill (ctx - 1 decode steps,
    untimed)."""
    from .granite import GraniteConfig, GraniteEngine, synthetic_weights

    cfg = GraniteConfig()
    t0 = time.perf_counter()
    w = synthetic_weights(cfg, seed=0, device=DEV)
    eng = GraniteEngine(cfg, w, rows=rows, device=DEV, max_steps=ctx + steps + 32)
    if context == "walk":
        g = torch.Generator().manual_seed(5)
        eng.prefill([torch.randint(0, cfg.vocab, (ctx + 1,), generator=g).tolist()
                     for _ in range(rows)])
    else:
        eng.synthetic_context(ctx)
    for _ in range(4):
        eng.replay()
    torch.cuda.synchronize()
    print(f"[bench] c5 weights + engine + capture + context ({context}) "
          f"{time.perf_counter() - t0:.1f}s", flush=True)
    t1 = time.perf_counter()
    for _ in range(steps):
        eng.replay()
    torch.cuda.synchronize()
    seconds = time.perf_counter() - t1
    eng.check_errors()
    touched = len(set(eng.ridx.reshape(-1).tolist()))
    wbytes = eng.weight_bytes_per_step(touched)
    positions = range(ctx + 4, ctx + 4 + steps)
    sbytes = sum(eng.state_bytes_per_step([p] * rows) for p in positions) / steps
    step_s = seconds / steps
    out = {"config": f"c5 step b{rows} ctx{ctx}", "context": context,
           "tok_s": round(rows * steps / seconds, 1),
           "ms_per_step": round(step_s * 1e3, 4), "steps": steps,
           "bytes_per_step": int(wbytes + sbytes), "experts_touched_sample": touched,
           "GB/s": round((wbytes + sbytes) / step_s / 1e9, 1),
           "frac": round((wbytes + sbytes) / step_s / HBM_PEAK, 4)}
    print(json.dumps(out), flush=True)
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--config", default="all",
                    choices=("c4", "c4b16", "c5", "all", "c4-step", "c5-step", "gemm"))
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--rows", type=int, default=1, help="c4-step / c5-step: sequences")
    ap.add_argument("--steps", type=int, default=256, help="c4-step / c5-step: timed steps")
    ap.add_argument("--context", choices=("drawn", "walk"), default="drawn",
                    help="c5-step: the contexts drawn into the caches and states (default) or "
                         "built by prefill from random prompts (about 53 s at 8,192 tokens)")
    ap.add_argument("--ctx", type=int, default=8192, help="c5-step: context length")
    ap.add_argument("--path", choices=("auto", "small", "mfma"), default="auto",
                    help="c4-step: the small-batch kernels (rows <= 4, the default there) or "
                         "the batched MFMA path")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("hybrid kernel bench: no GPU visible")
    if args.config == "c4-step":
        bench_c4_step(args.rows, args.steps,
                      small=None if args.path == "auto" else args.path == "small")
        return 0
    if args.config == "c5-step":
        bench_c5_step(args.rows, args.steps, ctx=args.ctx, context=args.context)
        return 0
    if args.config == "gemm":
        run_gemm(args.reps)
        return 0
    for c in (("c4", "c4b16", "c5") if args.config == "all" else (args.config,)):
        run(c, args.reps)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
