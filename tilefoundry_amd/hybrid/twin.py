"""Runtime twins of the hybrid models' authored modules, on the gfx950 kernels.

The reference pairs every authored ``@func`` with a runtime twin of the same
name and signature, weights included (``src/tilefoundry/runtime/decorator.py:
24-229``: the twin's function set must equal the authored one, and ``load``
binds each weight by its canonical name after checking shape and dtype).  This
module keeps that surface for the two hybrid models:

* Qwen3.5-35B-A3B (workload C4) -- ``examples/qwen3_5_35b_a3b-tilelang/
  runtime_model.py:113-300`` twins the authored ``model.py`` (the example's
  ``build()`` tree: folded ``1 + gamma`` norms, ``(in, out)`` projections).
  ``Qwen3_5LinearAttention``, ``Qwen3_5FullAttention``, ``Qwen3_5Router``,
  ``Qwen3_5MoE``, the two layer kinds and ``Qwen3_5Decoder`` carry the authored
  functions (``conv_step``, ``l2_normalise``, ``delta_step``,
  ``linear_attention``, ``partial_rope``, ``partial_rope_kv``,
  ``full_attention``, ``routing``, ``post_norm``, ``routed_experts``,
  ``shared_expert``, ``experts``, ``residual_add``, ``embed``,
  ``final_rms_norm``, ``lm_head``) and the orchestration (``forward``,
  ``decode_hidden``, ``init_caches``, ``append_cache``,
  ``prepare_inputs_for_generation``, tests/models/qwen3_5_35b_a3b/
  model.py:466-709).  Arithmetic is the example's torch twin's
  (``kernels/torch_ref.py:22-40``): f32 activations and state, every matmul on
  the bf16 cast of its input with one rounding of the f32 sum -- the C4 engine's.
* Granite-4.0-H-small (workload C5) -- ``examples/granite_4_0_h_small-cuda/
  model.py:131-720``: ``GraniteMamba`` (``in_projection``, ``conv_step``,
  ``ssm_step``, ``gated_out``, ``mamba_mixer``), ``GraniteAttention`` (``qkv``,
  ``attend``, ``full_attention``), ``GraniteRouter``, ``GraniteMoE``
  (``post_norm``, ``routed_experts``, ``shared_mlp``, ``experts``), the layers'
  scaled ``residual_add`` and ``Granite4_0_H_Small`` with its orchestration, at
  the HIR's bf16 rounding with the authored bf16 weights (the C5 engine runs the
  same arithmetic on fp8-e4m3 weights; the authored signature declares bf16).

Ids cross the boundary as int64 (``Tensor[(S, K), "i64"]``); the kernels take
int32 inside.  Like the reference twins (``runtime.md:270-277``), a function
does not mutate its inputs: state comes in and fresh state goes out.  Every
arithmetic step runs in the HIP library; torch here only moves, casts between
storage types exactly (bf16 -> f32), and lays out data.  Where an authored f32
intermediate is handed back (``post_norm``, ``final_rms_norm``, the cached
``k_rope``), the twin hands back the bf16 value the fused kernels produce at
that point (the next matmul casts to bf16 anyway), so those outputs sit within
one bf16 rounding of the torch twin's.
"""
from __future__ import annotations

import torch

from .. import _lib
from .._lib import lib, ptr
from .granite import GraniteConfig
from .qwen3_5 import Qwen35Config, ctypes_addr

BF = torch.bfloat16
F32 = torch.float32
I32 = torch.int32
I64 = torch.int64


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def operand_order(x: torch.Tensor) -> torch.Tensor:
    """[M][K] bf16 rows (M <= 32) -> the skinny GEMMs' operand order (flat, 32 x K,
    rows past M zero): block 2s + h holds x[16h + l % 16][32s + 8 (l / 16) ..]."""
    M, K = x.shape
    full = torch.zeros(32, K, dtype=BF, device=x.device)
    full[:M] = x
    return full.view(2, 16, K // 32, 4, 8).permute(2, 0, 3, 1, 4).reshape(-1).contiguous()


def from_operand_order(flat: torch.Tensor, M: int, K: int) -> torch.Tensor:
    return flat.view(K // 32, 2, 4, 16, 8).permute(1, 3, 0, 2, 4).reshape(32, K)[:M]


class _Derived:
    """Kernel layouts of canonical weights, remembered by tensor identity (the
    reference twin's ``_Fused``, examples/qwen3_1_7b-tilelang/fast/twin.py:80-102)."""

    def __init__(self):
        self._cache: dict = {}

    def get(self, kind, make, *ts):
        key = (kind,) + tuple((t.data_ptr(), tuple(t.shape), tuple(t.stride())) for t in ts)
        hit = self._cache.get(key)
        if hit is None:
            hit = (make(), ts)                  # keep the sources alive so ids stay unique
            self._cache[key] = hit
        return hit[0]


class _Ops:
    """The library calls the twins share."""

    def __init__(self):
        self.L = lib()
        self.derived = _Derived()
        self._work: dict = {}

    def work(self, dev) -> torch.Tensor:
        w = self._work.get(str(dev))
        if w is None:
            w = torch.zeros(1 << 21, device=dev, dtype=F32)
            self._work[str(dev)] = w
        return w

    def packed(self, kind, rows_fn, *ts) -> torch.Tensor:
        """tfd_pack_skinny_bf16 of the [N][K] bf16 rows `rows_fn()` builds from *ts*."""

        def make():
            rows = rows_fn().to(BF).contiguous()
            N, K = rows.shape
            out = torch.empty(-(-N // 16) * 16 * K, dtype=BF, device=rows.device)
            self.L.tfd_pack_skinny_bf16(ptr(rows), K, N, K, ptr(out), _stream(rows))
            return out

        return self.derived.get(kind, make, *ts)

    def to_bf16(self, x: torch.Tensor) -> torch.Tensor:
        """Round f32 values to bf16 (the HIR's cast; tfd_round_bf16); bf16 passes."""
        if x.dtype == BF:
            return x.contiguous()
        xf = x.to(F32).contiguous()
        out = torch.empty(xf.shape, dtype=BF, device=x.device)
        self.L.tfd_round_bf16(ptr(xf), ptr(out), xf.numel(), _stream(xf))
        return out

    def to_f32(self, x: torch.Tensor) -> torch.Tensor:
        """bf16 -> f32 is exact (tfd_bf16_to_f32_rows); f32 passes."""
        if x.dtype == F32:
            return x.contiguous()
        xb = x.to(BF).contiguous()
        n = xb.numel()
        out = torch.empty(xb.shape, dtype=F32, device=x.device)
        self.L.tfd_bf16_to_f32_rows(ptr(xb), n, ptr(out), n, 1, n, _stream(xb))
        return out

    def gemm(self, x_op, packed, M, K, N, epi, out, ldo, resid=None, ldr=0):
        self.L.tfd_gemm_skinny_bf16(ptr(x_op), ptr(packed), M, K, N, epi, ptr(resid), ldr,
                                    ptr(out), ldo, ptr(self.work(x_op.device)),
                                    self.work(x_op.device).numel(), _stream(x_op))

    def rmsnorm_f32(self, x: torch.Tensor, gamma, eps, packed: bool):
        """C4's norm of f32 rows: bf16(x * rsqrt(mean x^2 + eps) * gamma), as rows
        [R][n] bf16 or in operand order (tfd_rmsnorm_f32_rows)."""
        R, n = x.shape
        xf = self.to_f32(x)
        dev = x.device
        if packed:
            out = torch.empty(32 * n, dtype=BF, device=dev)
            self.L.tfd_rmsnorm_f32_rows(ptr(xf), n, ptr(gamma), None, 0, ptr(out), R, n, eps,
                                        _stream(xf))
        else:
            out = torch.empty(R, n, dtype=BF, device=dev)
            self.L.tfd_rmsnorm_f32_rows(ptr(xf), n, ptr(gamma), ptr(out), n, None, R, n, eps,
                                        _stream(xf))
        return out

    def rmsnorm_tf(self, x: torch.Tensor, gamma, eps, packed: bool):
        """C5's tf.rms_norm of bf16 rows (tfd_tf_rmsnorm_rows_bf16)."""
        R, n = x.shape
        xb = self.to_bf16(x)
        dev = x.device
        if packed:
            out = torch.empty(32 * n, dtype=BF, device=dev)
            self.L.tfd_tf_rmsnorm_rows_bf16(ptr(xb), n, ptr(gamma), None, 0, ptr(out), R, n, eps,
                                            _stream(xb))
        else:
            out = torch.empty(R, n, dtype=BF, device=dev)
            self.L.tfd_tf_rmsnorm_rows_bf16(ptr(xb), n, ptr(gamma), ptr(out), n, None, R, n, eps,
                                            _stream(xb))
        return out


def _check_err(err: torch.Tensor, what: str):
    e = int(err.item())
    if e:
        raise RuntimeError(f"{what}: kernels flagged error bits {e:#x}")


def _rows(x: torch.Tensor, n: int) -> torch.Tensor:
    """(R, S=1, n) or (R, n) activations as [R][n]."""
    return x.reshape(-1, n)


class _PagedContext:
    """A prior context [R][C][HKV][D] staged in a paged pool (16-position pages in
    a seeded order, so every access goes through the page table) with the
    position C of this token free for the kernel to append."""

    def __init__(self, k_past, v_past, kv_heads, head_dim, dev, seed, split_len=64):
        R, C = int(k_past.shape[0]), int(k_past.shape[1])
        self.R, self.C = R, C
        cap = -(-(C + 1) // split_len) * split_len
        self.max_pages = cap // _lib.PAGE_SIZE
        self.num_pages = R * self.max_pages
        g = torch.Generator().manual_seed(seed + C)
        self.table = torch.randperm(self.num_pages, generator=g).view(R, self.max_pages).to(I32)
        self.table = self.table.to(dev)
        self.kpool = torch.zeros(self.num_pages, kv_heads, _lib.PAGE_SIZE, head_dim, dtype=BF,
                                 device=dev)
        self.vpool = torch.zeros_like(self.kpool)
        if C:
            p = torch.arange(C, device=dev)
            for b in range(R):
                page, row = self.table[b].long()[p // _lib.PAGE_SIZE], p % _lib.PAGE_SIZE
                self.kpool[page, :, row] = k_past[b].to(BF)
                self.vpool[page, :, row] = v_past[b].to(BF)
        self.nsplit = cap // split_len
        self.split_len = split_len
        self.stride = self.max_pages * _lib.PAGE_SIZE
        self.pos = torch.full((R,), C, dtype=I32, device=dev)

    def row_at(self, pool, b, p):
        page = int(self.table[b, p // _lib.PAGE_SIZE])
        return pool[page, :, p % _lib.PAGE_SIZE]

    def gqa_args(self, qkv, ldq, heads, kv_heads, head_dim, scale, eps, out, policy, err):
        a = _lib.TfdGqaArgs()
        a.qkv, a.ldq = ptr(qkv), ldq
        a.pos, a.page_table, a.max_pages = ptr(self.pos), ptr(self.table), self.max_pages
        a.k_pool, a.v_pool, a.num_pages = ptr(self.kpool), ptr(self.vpool), self.num_pages
        a.rows, a.heads, a.kv_heads, a.head_dim = self.R, heads, kv_heads, head_dim
        a.scale, a.eps = float(scale), float(eps)
        dev = qkv.device
        self._ws = (torch.zeros(self.R * heads * self.stride, dtype=F32, device=dev),
                    torch.zeros(self.R * heads * self.nsplit * 2, dtype=F32, device=dev),
                    torch.zeros(self.R * heads * self.nsplit * head_dim, dtype=F32, device=dev),
                    torch.zeros(self.R * kv_heads, dtype=I32, device=dev))
        a.scores, a.score_stride = ptr(self._ws[0]), self.stride
        a.stats, a.part, a.counters = ptr(self._ws[1]), ptr(self._ws[2]), ptr(self._ws[3])
        a.nsplit, a.split_len = self.nsplit, self.split_len
        a.out, a.policy, a.err = ptr(out), policy, ptr(err)
        return a


def _validate(declared: dict, weights: dict):
    """``KeyError`` for a missing weight, ``ValueError`` for a wrong shape or dtype
    (src/tilefoundry/ir/core/module.py:144-159)."""
    for name, (shape, dt) in declared.items():
        if name not in weights:
            raise KeyError(f"weight {name!r} is declared but not supplied")
        t = weights[name]
        if tuple(t.shape) != tuple(shape):
            raise ValueError(f"weight {name!r}: declared shape {tuple(shape)}, got "
                             f"{tuple(t.shape)}")
        if t.dtype != dt:
            raise ValueError(f"weight {name!r}: declared dtype {dt}, got {t.dtype}")


# ===========================================================================
# Qwen3.5-35B-A3B (C4)
# ===========================================================================
class Qwen3_5LinearAttention:
    """``Qwen3_5LinearAttention`` (model.py:121-230): the gated DeltaNet mixer."""

    def __init__(self, cfg: Qwen35Config, ops: _Ops):
        self.cfg, self.ops = cfg, ops

    def conv_step(self, conv_state, entry, conv_w):
        """(1, CONV, 3), (1, CONV, 1), (CONV, 4) -> silu(window . w): (1, CONV) f32."""
        c, o = self.cfg, self.ops
        R = int(conv_state.shape[0])
        win = o.to_f32(conv_state)
        ent = o.to_f32(entry.reshape(R, c.conv_dim))
        out = torch.empty(R, c.conv_dim, dtype=F32, device=win.device)
        a = _lib.TfdConvStepArgs(window=ptr(win), entry=ptr(ent), lde=c.conv_dim,
                                 conv_w=ptr(conv_w.to(BF).contiguous()), conv_b=None,
                                 out=ptr(out), ldo=c.conv_dim, rows=R, channels=c.conv_dim,
                                 kernel=c.conv_kernel, policy=_lib.POLICY_F32)
        o.L.tfd_conv_step_rows(ctypes_addr(a), _stream(win))
        return out

    def l2_normalise(self, x):
        """x * rsqrt(sum(x^2) + 1e-6) over the last axis (model.py:138-146)."""
        xf = self.ops.to_f32(x)
        out = torch.empty_like(xf)
        d = xf.shape[-1]
        self.ops.L.tfd_l2norm_f32(ptr(xf), ptr(out), xf.numel() // d, d, 1e-6, _stream(xf))
        return out

    def delta_step(self, recurrent_state, q, k, v, g, beta):
        """One token of the gated delta rule (model.py:148-172) -> (read (1, HV, DV),
        updated (1, HV, DK, DV)), f32."""
        c, o = self.cfg, self.ops
        R = int(recurrent_state.shape[0])
        hv, dk, dv = c.lin_value_heads, c.lin_key_dim, c.lin_value_dim
        st = o.to_f32(recurrent_state)
        upd = torch.empty_like(st)
        read = torch.empty(R, hv, dv, dtype=F32, device=st.device)
        qf, kf, vf = (o.to_f32(t) for t in (q, k, v))
        gf, bf = o.to_f32(g), o.to_f32(beta)
        a = _lib.TfdDeltaStepArgs(state_in=ptr(st), state_out=ptr(upd), q=ptr(qf), k=ptr(kf),
                                  v=ptr(vf), g=ptr(gf), beta=ptr(bf), read=ptr(read),
                                  qscale=dk ** -0.5, rows=R, heads=hv, head_k_dim=dk,
                                  head_v_dim=dv)
        o.L.tfd_delta_step_f32(ctypes_addr(a), _stream(st))
        return read, upd

    def linear_attention(self, hidden, gamma_in, w_in_qkv, w_in_z, w_in_b, w_in_a, conv_w,
                         a_log, dt_bias, conv_state, recurrent_state, gamma_gdn, w_out):
        """input norm + ``Qwen3_5MoeGatedDeltaNet`` at one token (model.py:174-230)
        -> (out (1, 1, H), entry (1, CONV, 1), updated (1, HV, DK, DV)), f32."""
        c, o = self.cfg, self.ops
        H = c.hidden
        x = _rows(hidden, H)
        R, dev = x.shape[0], hidden.device
        xn = o.rmsnorm_f32(x, gamma_in, c.eps, packed=True)
        w_in = o.packed("gdn_in", lambda: torch.cat([w_in_qkv[0].t(), w_in_z[0].t(),
                                                     w_in_b[0].t(), w_in_a[0].t()]),
                        w_in_qkv, w_in_z, w_in_b, w_in_a)
        N = c.gdn_in
        proj = torch.empty(R, N, dtype=F32, device=dev)
        o.gemm(xn, w_in, R, H, N, _lib.EPI_LOGITS, proj, N)
        conv_in = o.to_f32(conv_state).clone()
        conv_out = torch.empty_like(conv_in)
        state = o.to_f32(recurrent_state).clone()
        mix = torch.zeros(32 * c.value_dim, dtype=BF, device=dev)
        a = _lib.TfdGdnArgs()
        a.proj, a.proj_ld, a.conv_in, a.conv_out = ptr(proj), N, ptr(conv_in), ptr(conv_out)
        a.state = ptr(state)
        a.conv_w, a.a_log, a.dt_bias = ptr(conv_w), ptr(a_log), ptr(dt_bias)
        a.gamma, a.out = ptr(gamma_gdn), ptr(mix)
        a.rows, a.key_heads, a.value_heads = R, c.lin_key_heads, c.lin_value_heads
        a.head_k_dim, a.head_v_dim, a.conv_kernel = c.lin_key_dim, c.lin_value_dim, c.conv_kernel
        a.l2_eps, a.rms_eps = 1e-6, c.eps
        o.L.tfd_gdn_step(ctypes_addr(a), _stream(proj))
        w_o = o.packed("gdn_out", lambda: w_out[0].t(), w_out)
        out = torch.empty(R, H, dtype=F32, device=dev)
        o.gemm(mix, w_o, R, c.value_dim, H, _lib.EPI_LOGITS, out, H)
        entry = proj[:, :c.conv_dim].reshape(R, c.conv_dim, 1).clone()
        return out.reshape(R, 1, H), entry, state


class Qwen3_5FullAttention:
    """``Qwen3_5FullAttention`` (model.py:232-346): gated GQA with partial RoPE."""

    def __init__(self, cfg: Qwen35Config, ops: _Ops, page_seed: int = 0):
        self.cfg, self.ops, self.page_seed = cfg, ops, page_seed

    def _rope(self, x, heads, cos_cache, sin_cache, pos_ids):
        c, o = self.cfg, self.ops
        D = c.head_dim
        xf = o.to_f32(x)
        R = xf.numel() // (heads * D)
        out = torch.empty_like(xf)
        cos_t, sin_t = cos_cache.to(BF).contiguous(), sin_cache.to(BF).contiguous()
        pos = pos_ids.reshape(-1).to(I32).to(xf.device)
        if pos.numel() != R:
            pos = pos[:1].expand(R).contiguous()
        a = _lib.TfdPartialRopeArgs(x=ptr(xf), ldx=heads * D, out=ptr(out), ldo=heads * D,
                                    pos=ptr(pos), cos_table=ptr(cos_t), sin_table=ptr(sin_t),
                                    rope_rows=int(cos_t.shape[0]), rows=R, heads=heads,
                                    head_dim=D, rot=c.rot_dim)
        o.L.tfd_partial_rope_f32(ctypes_addr(a), _stream(xf))
        return out

    def partial_rope(self, x, cos_cache, sin_cache, pos_ids):
        """(1, S, HQ, D) rotated on its first rot dims (model.py:235-248)."""
        return self._rope(x, self.cfg.heads, cos_cache, sin_cache, pos_ids)

    def partial_rope_kv(self, x, cos_cache, sin_cache, pos_ids):
        """(1, S, HKV, D) rotated on its first rot dims (model.py:250-262)."""
        return self._rope(x, self.cfg.kv_heads, cos_cache, sin_cache, pos_ids)

    def full_attention(self, hidden, gamma_in, w_qg, w_k, w_v, gamma_q, gamma_k, cos_cache,
                       sin_cache, pos_ids, k_cache, v_cache, scale, w_o):
        """input norm + ``Qwen3_5MoeAttention`` at one token (model.py:264-346) ->
        (out (1, 1, H), k_rope (1, 1, HKV, D), v (1, 1, HKV, D)), f32; k_rope as
        the cache keeps it (bf16 values)."""
        c, o = self.cfg, self.ops
        H, HQ, HKV, D = c.hidden, c.heads, c.kv_heads, c.head_dim
        x = _rows(hidden, H)
        R, dev = x.shape[0], hidden.device
        xn = o.rmsnorm_f32(x, gamma_in, c.eps, packed=True)
        w_in = o.packed("attn_in", lambda: torch.cat([w_qg[0].t(), w_k[0].t(), w_v[0].t()]),
                        w_qg, w_k, w_v)
        N = c.attn_in
        proj = torch.empty(R, N, dtype=F32, device=dev)
        o.gemm(xn, w_in, R, H, N, _lib.EPI_LOGITS, proj, N)
        ctx = _PagedContext(k_cache.reshape(R, -1, HKV, D), v_cache.reshape(R, -1, HKV, D), HKV,
                            D, dev, self.page_seed)
        # the rope row this token reads, at the position the kernel appends it
        p = int(pos_ids.reshape(-1)[0])
        cos_t = torch.zeros(ctx.C + 1, c.rot_dim, dtype=BF, device=dev)
        sin_t = torch.zeros_like(cos_t)
        cos_t[ctx.C] = cos_cache.to(BF).reshape(-1, c.rot_dim)[p]
        sin_t[ctx.C] = sin_cache.to(BF).reshape(-1, c.rot_dim)[p]
        mix = torch.zeros(32 * HQ * D, dtype=BF, device=dev)
        err = torch.zeros(1, dtype=I32, device=dev)
        sc = float(scale.reshape(-1)[0]) if torch.is_tensor(scale) else float(scale)
        a = ctx.gqa_args(proj, N, HQ, HKV, D, sc, c.eps, mix, _lib.POLICY_F32, err)
        a.gamma_q, a.gamma_k, a.cos_table, a.sin_table = ptr(gamma_q), ptr(gamma_k), \
            ptr(cos_t), ptr(sin_t)
        a.rope_rows, a.rot_dim = ctx.C + 1, c.rot_dim
        o.L.tfd_gqa_decode(ctypes_addr(a), _stream(proj))
        w_out = o.packed("attn_out", lambda: w_o[0].t(), w_o)
        out = torch.empty(R, H, dtype=F32, device=dev)
        o.gemm(mix, w_out, R, HQ * D, H, _lib.EPI_LOGITS, out, H)
        _check_err(err, "full_attention")
        k_rope = torch.stack([ctx.row_at(ctx.kpool, b, ctx.C) for b in range(R)]).float()
        v = proj[:, HQ * 2 * D + HKV * D:HQ * 2 * D + 2 * HKV * D].reshape(R, 1, HKV, D).clone()
        return out.reshape(R, 1, H), k_rope.reshape(R, 1, HKV, D), v


class Qwen3_5Router:
    """``Qwen3_5Router.routing`` (model.py:348-366): softmax over every expert,
    the top k, renormalised -> (weights (S, K) f32, indices (S, K) int64)."""

    def __init__(self, cfg: Qwen35Config, ops: _Ops):
        self.cfg, self.ops = cfg, ops

    def routing(self, tokens, w_router):
        c, o = self.cfg, self.ops
        H, E, K = c.hidden, c.experts, c.top_k
        x = _rows(tokens, H)
        R, dev = x.shape[0], x.device
        x_op = operand_order(o.to_bf16(x))
        w = o.packed("router", lambda: w_router.t(), w_router)
        logits = torch.empty(R, E, dtype=F32, device=dev)
        o.gemm(x_op, w, R, H, E, _lib.EPI_LOGITS, logits, E)
        weights = torch.empty(R, K, dtype=F32, device=dev)
        idx = torch.empty(R, K, dtype=I32, device=dev)
        o.L.tfd_route_topk(ptr(logits), E, R, E, K, _lib.ROUTE_SOFTMAX_TOPK, ptr(weights),
                           ptr(idx), _stream(logits))
        return weights, idx.to(I64)


def _moe_call(ops, cfg, x_bf16, weights_f32, idx_i32, w_gate, w_up, w_down, shared_in,
              shared_out, shared_scale, fp8, policy, inter, shared_inter, experts=None):
    """tfd_moe_experts with the routing given -> f32 [R][H]."""
    R, H = x_bf16.shape
    k = idx_i32.shape[1]
    E = cfg.experts if experts is None else experts
    dev = x_bf16.device
    ld = max(inter, shared_inter)
    hidden = torch.zeros(R, k + 1, ld, dtype=BF, device=dev)
    sscale = torch.zeros(R, dtype=F32, device=dev)
    partial = torch.zeros(R, k + 1, H, dtype=F32, device=dev)
    groups = torch.zeros(_lib.moe_group_words(E, R), dtype=I32, device=dev)
    out = torch.zeros(R, H, dtype=F32, device=dev)
    err = torch.zeros(1, dtype=I32, device=dev)
    a = _lib.TfdMoeArgs()
    a.x, a.weights, a.idx = ptr(x_bf16), ptr(weights_f32), ptr(idx_i32)
    a.w_gate, a.w_up, a.w_down = ptr(w_gate), ptr(w_up), ptr(w_down)
    a.w_shared_in, a.w_shared_out = ptr(shared_in), ptr(shared_out)
    a.w_shared_scale = ptr(shared_scale)
    a.hidden, a.shared_scale, a.partial = ptr(hidden), ptr(sscale), ptr(partial)
    a.groups, a.out = ptr(groups), ptr(out)
    a.rows, a.k, a.experts, a.hidden_size = R, k, E, H
    a.inter, a.shared_inter, a.hidden_ld = inter, shared_inter, ld
    a.fp8, a.policy, a.err = fp8, policy, ptr(err)
    a.accumulate, a.route = 0, _lib.MOE_ROUTE_GIVEN
    ops.L.tfd_moe_experts(ctypes_addr(a), _stream(x_bf16))
    _check_err(err, "experts")
    return out


def _only_shared(ops, cfg, x_bf16, shared_in, shared_out, shared_scale, policy):
    """The shared expert alone: the call with k zero-weighted stand-in experts of zero
    weights (their products are exact zeros, so the sum is the shared expert's)."""
    R, H = x_bf16.shape
    dev, k, I = x_bf16.device, cfg.top_k, cfg.moe_inter
    z = ops.derived.get(("zero_experts", str(dev), k, I, H),
                        lambda: (torch.zeros(k, I, H, dtype=BF, device=dev),
                                 torch.zeros(k, H, I, dtype=BF, device=dev)))
    idx = torch.arange(k, dtype=I32, device=dev).repeat(R, 1).contiguous()
    wts = torch.zeros(R, k, dtype=F32, device=dev)
    return _moe_call(ops, cfg, x_bf16, wts, idx, z[0], z[0], z[1], shared_in, shared_out,
                     shared_scale, 0, policy, I, cfg.shared_inter, experts=k)


class Qwen3_5MoE:
    """``Qwen3_5MoE`` (model.py:369-463): post norm, router, routed + shared experts."""

    def __init__(self, cfg: Qwen35Config, ops: _Ops):
        self.cfg, self.ops = cfg, ops
        self.router = Qwen3_5Router(cfg, ops)
        self.weights: dict | None = None

    def post_norm(self, hidden, gamma_post):
        """``post_attention_layernorm`` (model.py:373-380) -> (S, H), the bf16 value
        the experts' matmuls read, as f32."""
        c, o = self.cfg, self.ops
        return o.to_f32(o.rmsnorm_f32(_rows(hidden, c.hidden), gamma_post, c.eps, packed=False))

    def _shared(self, w_shared_gate, w_shared_up, w_shared_down, w_shared_scale):
        o = self.ops
        sin = o.derived.get("shared_in", lambda: torch.cat([w_shared_gate.t(),
                                                            w_shared_up.t()]).to(BF).contiguous(),
                            w_shared_gate, w_shared_up)
        sout = o.derived.get("shared_out", lambda: w_shared_down.t().to(BF).contiguous(),
                             w_shared_down)
        sscale = w_shared_scale.reshape(-1).to(BF).contiguous()
        return sin, sout, sscale

    def experts(self, tokens, weights, indices, w_gate, w_up, w_down, w_shared_gate, w_shared_up,
                w_shared_down, w_shared_scale):
        """Routed + shared experts, no residual (model.py:437-456) -> (1, S, H) f32."""
        c, o = self.cfg, self.ops
        x = o.to_bf16(_rows(tokens, c.hidden))
        sin, sout, sscale = self._shared(w_shared_gate, w_shared_up, w_shared_down,
                                         w_shared_scale)
        out = _moe_call(o, c, x, o.to_f32(weights), indices.to(I32).contiguous(), w_gate, w_up,
                        w_down, sin, sout, sscale, 0, _lib.POLICY_F32, c.moe_inter,
                        c.shared_inter)
        return out.reshape(1, -1, c.hidden)

    def routed_experts(self, tokens, weights, indices, w_gate, w_up, w_down):
        """The picked experts' SwiGLU mixed by the routing weights (model.py:382-418)
        -> (S, H) f32: ``experts`` with a shared expert of zero weights (it adds an
        exact 0)."""
        c, o = self.cfg, self.ops
        H, IS = c.hidden, c.shared_inter
        dev = tokens.device
        z = o.derived.get(("zero_shared", str(dev)),
                          lambda: (torch.zeros(2 * IS, H, dtype=BF, device=dev),
                                   torch.zeros(H, IS, dtype=BF, device=dev),
                                   torch.zeros(H, dtype=BF, device=dev)))
        x = o.to_bf16(_rows(tokens, H))
        return _moe_call(o, c, x, o.to_f32(weights), indices.to(I32).contiguous(), w_gate, w_up,
                         w_down, z[0], z[1], z[2], 0, _lib.POLICY_F32, c.moe_inter, IS)

    def shared_expert(self, tokens, w_shared_gate, w_shared_up, w_shared_down, w_shared_scale):
        """The dense SwiGLU every token goes through, times its sigmoid gate
        (model.py:420-435) -> (S, H) f32."""
        c, o = self.cfg, self.ops
        x = o.to_bf16(_rows(tokens, c.hidden))
        sin, sout, sscale = self._shared(w_shared_gate, w_shared_up, w_shared_down,
                                         w_shared_scale)
        return _only_shared(o, c, x, sin, sout, sscale, _lib.POLICY_F32)

    def forward(self, hidden):
        """One decode step of the block: post-norm, route, then the experts
        (model.py:458-463)."""
        w = self._bound()
        tokens = self.post_norm(hidden, w["gamma_post"])
        weights, indices = self.router.routing(tokens, w["router.w_router"])
        return self.experts(tokens, weights, indices, w["w_gate"], w["w_up"], w["w_down"],
                            w["w_shared_gate"], w["w_shared_up"], w["w_shared_down"],
                            w["w_shared_scale"])

    def _bound(self):
        if self.weights is None:
            raise TypeError("this module is not loaded: call load(weights) on the decoder")
        return self.weights


class _Qwen35Layer:
    """The two decoder-layer kinds (model.py:466-516): mixer + residual, MoE +
    residual."""

    def __init__(self, cfg, ops, kind, page_seed):
        self.kind = kind
        self.mixer = (Qwen3_5FullAttention(cfg, ops, page_seed) if kind == "full_attention"
                      else Qwen3_5LinearAttention(cfg, ops))
        self.moe = Qwen3_5MoE(cfg, ops)
        self.cfg, self.ops = cfg, ops
        self.weights: dict | None = None

    def residual_add(self, a, b):
        """a + b, f32 (model.py:493-500)."""
        o = self.ops
        acc = o.to_f32(a).clone()
        n = self.cfg.hidden
        add = o.to_f32(b)
        R = acc.numel() // n
        o.L.tfd_add_f32_rows(ptr(acc), n, ptr(add), n, R, n, _stream(acc))
        return acc.reshape(a.shape)

    def _mixer(self, hidden, *args):
        w = self.weights
        if self.kind == "full_attention":
            cos, sin, pos_ids, k_cache, v_cache, scale = args
            return self.mixer.full_attention(hidden, w["gamma_in"], w["w_qg"], w["w_k"],
                                             w["w_v"], w["gamma_q"], w["gamma_k"], cos, sin,
                                             pos_ids, k_cache, v_cache, scale, w["w_o"])
        conv_state, recurrent_state = args
        return self.mixer.linear_attention(hidden, w["gamma_in"], w["w_in_qkv"], w["w_in_z"],
                                           w["w_in_b"], w["w_in_a"], w["conv_w"], w["a_log"],
                                           w["dt_bias"], conv_state, recurrent_state,
                                           w["gamma_gdn"], w["w_out"])

    def forward(self, hidden, mixer_args):
        """``_layer_forward`` (model.py:466-485)."""
        mixed, *state = self._mixer(hidden, *mixer_args)
        attended = self.residual_add(hidden, mixed)
        expert_out = self.moe.forward(attended)
        return self.residual_add(attended, expert_out), tuple(state)


def qwen35_declared(cfg: Qwen35Config) -> dict:
    """Canonical name -> (shape, dtype) of every weight the decoder twin binds: the
    example's declared parameters after its converters (model.py:174-188, 264-279,
    354-358, 373-448, 603-633)."""
    H, E, I, IS = cfg.hidden, cfg.experts, cfg.moe_inter, cfg.shared_inter
    HQ, HKV, D = cfg.heads, cfg.kv_heads, cfg.head_dim
    out = {"table": (cfg.vocab, H), "gamma_final": (H,), "w_head": (H, cfg.vocab)}
    for i in range(cfg.layers):
        m, e = f"layer{i}.mixer.", f"layer{i}.moe."
        if cfg.is_full(i):
            out.update({m + "gamma_in": (H,), m + "w_qg": (1, H, HQ * D * 2),
                        m + "w_k": (1, H, HKV * D), m + "w_v": (1, H, HKV * D),
                        m + "gamma_q": (D,), m + "gamma_k": (D,), m + "w_o": (1, HQ * D, H)})
        else:
            out.update({m + "gamma_in": (H,), m + "w_in_qkv": (1, H, cfg.conv_dim),
                        m + "w_in_z": (1, H, cfg.value_dim),
                        m + "w_in_b": (1, H, cfg.lin_value_heads),
                        m + "w_in_a": (1, H, cfg.lin_value_heads),
                        m + "conv_w": (cfg.conv_dim, cfg.conv_kernel),
                        m + "a_log": (cfg.lin_value_heads,), m + "dt_bias": (cfg.lin_value_heads,),
                        m + "gamma_gdn": (cfg.lin_value_dim,), m + "w_out": (1, cfg.value_dim, H)})
        out.update({e + "gamma_post": (H,), e + "w_gate": (E, I, H), e + "w_up": (E, I, H),
                    e + "w_down": (E, H, I), e + "w_shared_gate": (H, IS),
                    e + "w_shared_up": (H, IS), e + "w_shared_down": (IS, H),
                    e + "w_shared_scale": (H, 1), e + "router.w_router": (H, E)})
    return {k: (v, BF) for k, v in out.items()}


def qwen35_canonical(cfg: Qwen35Config, w: dict) -> dict:
    """The engine's row-layout weights (``hybrid.qwen3_5``) under the twin's
    canonical names and declared layouts -- the same draw, relaid."""
    H, IS = cfg.hidden, cfg.shared_inter
    HQ, HKV, D = cfg.heads, cfg.kv_heads, cfg.head_dim
    out = {"table": w["embed"], "gamma_final": w["gamma_final"],
           "w_head": w["head"].t().contiguous()}
    for i in range(cfg.layers):
        p, m, e = f"layer{i}.", f"layer{i}.mixer.", f"layer{i}.moe."
        rows = w[p + "w_in"]
        out[m + "gamma_in"] = w[p + "gamma_in"]
        if cfg.is_full(i):
            q = HQ * 2 * D
            out[m + "w_qg"] = rows[:q].t().contiguous()[None]
            out[m + "w_k"] = rows[q:q + HKV * D].t().contiguous()[None]
            out[m + "w_v"] = rows[q + HKV * D:q + 2 * HKV * D].t().contiguous()[None]
            out[m + "gamma_q"], out[m + "gamma_k"] = w[p + "gamma_q"], w[p + "gamma_k"]
            out[m + "w_o"] = w[p + "w_out"].t().contiguous()[None]
        else:
            conv, val, hv = cfg.conv_dim, cfg.value_dim, cfg.lin_value_heads
            out[m + "w_in_qkv"] = rows[:conv].t().contiguous()[None]
            out[m + "w_in_z"] = rows[conv:conv + val].t().contiguous()[None]
            out[m + "w_in_b"] = rows[conv + val:conv + val + hv].t().contiguous()[None]
            out[m + "w_in_a"] = rows[conv + val + hv:conv + val + 2 * hv].t().contiguous()[None]
            for n in ("conv_w", "a_log", "dt_bias", "gamma_gdn"):
                out[m + n] = w[p + n]
            out[m + "w_out"] = w[p + "w_out"].t().contiguous()[None]
        out[e + "gamma_post"] = w[p + "gamma_post"]
        for n in ("w_gate", "w_up", "w_down"):
            out[e + n] = w[p + n]
        si = w[p + "w_shared_in"]
        out[e + "w_shared_gate"] = si[:IS].t().contiguous()
        out[e + "w_shared_up"] = si[IS:].t().contiguous()
        out[e + "w_shared_down"] = w[p + "w_shared_out"].t().contiguous()
        out[e + "w_shared_scale"] = w[p + "w_shared_scale"].reshape(H, 1)
        out[e + "router.w_router"] = w[p + "w_router"].t().contiguous()
    return out


class Qwen3_5Decoder:
    """``Qwen3_5_35B_A3B`` / the example's ``Qwen3_5Decoder``: root functions and,
    once loaded, the orchestration (model.py:589-709) driven with activations
    only while weights are bound by name."""

    def __init__(self, cfg: Qwen35Config, page_seed: int = 0):
        self.cfg = cfg
        self.ops = _Ops()
        self.layer_types = ["full_attention" if cfg.is_full(i) else "linear_attention"
                            for i in range(cfg.layers)]
        self.layers = [_Qwen35Layer(cfg, self.ops, kind, page_seed) for kind in self.layer_types]
        self.weights: dict | None = None

    # ------------------------------------------------------------------ @funcs
    def embed(self, table, token_ids):
        """The table row of the token, as f32 (model.py:603-610)."""
        H, V = self.cfg.hidden, self.cfg.vocab
        dev = table.device
        ids = token_ids.reshape(-1).to(device=dev, dtype=I64).contiguous()
        R = ids.numel()
        rows = torch.empty(R, H, dtype=BF, device=dev)
        err = torch.zeros(1, dtype=I32, device=dev)
        self.ops.L.tfd_embed_rows_bf16(ptr(table.contiguous()), ptr(ids), ptr(rows), H, R, H, V,
                                       ptr(err), _stream(rows))
        if int(err.item()):
            raise IndexError(f"token id outside [0, {V})")
        return self.ops.to_f32(rows).reshape(R, 1, H)

    def final_rms_norm(self, hidden, gamma_final):
        """The last norm (model.py:612-618), as the bf16 value the head reads."""
        c, o = self.cfg, self.ops
        return o.to_f32(o.rmsnorm_f32(_rows(hidden, c.hidden), gamma_final, c.eps,
                                      packed=False)).reshape(hidden.shape)

    def lm_head(self, hidden, w_head):
        """(1, S, H) @ (H, V) -> (1, V) f32 logits of the bf16 product (model.py:620-634)."""
        c, o = self.cfg, self.ops
        x = _rows(hidden, c.hidden)
        R = x.shape[0]
        w = o.packed("head", lambda: w_head.t(), w_head)
        out = torch.empty(R, c.vocab, dtype=F32, device=x.device)
        o.gemm(operand_order(o.to_bf16(x)), w, R, c.hidden, c.vocab, _lib.EPI_LOGITS, out,
               c.vocab)
        return out

    # ---------------------------------------------------------- orchestration
    def load(self, weights: dict) -> "Qwen3_5Decoder":
        """Bind weights by canonical name (shape / dtype checked like Module.load)."""
        _validate(qwen35_declared(self.cfg), weights)
        self.weights = weights
        for i, layer in enumerate(self.layers):
            m, e = f"layer{i}.mixer.", f"layer{i}.moe."
            layer.weights = {k[len(m):]: v for k, v in weights.items() if k.startswith(m)}
            layer.moe.weights = {k[len(e):]: v for k, v in weights.items() if k.startswith(e)}
        return self

    def _bound(self, name):
        if self.weights is None:
            raise TypeError("Qwen3_5Decoder is not loaded: call load(weights) first")
        return self.weights[name]

    def decode_hidden(self, hidden, layer_args, caches):
        """Every layer, then the final norm (model.py:636-652)."""
        n = len(self.layers)
        if len(layer_args) != n or len(caches) != n:
            raise ValueError(f"decoder has {n} layers but was given {len(layer_args)} argument "
                             f"tuples and {len(caches)} caches")
        states = []
        for layer, args, cache in zip(self.layers, layer_args, caches):
            # the cache goes where the mixer declares its state (_with_cache, :557-571):
            # after (cos, sin, pos_ids) for attention, first for the linear mixer
            spliced = (*args[:3], *cache, *args[3:]) if layer.kind == "full_attention" \
                else (*cache, *args)
            hidden, state = layer.forward(hidden, spliced)
            states.append(state)
        return self.final_rms_norm(hidden, self._bound("gamma_final")), tuple(states)

    def forward(self, token_ids, layer_args, caches):
        """Token ids in, logits and the fresh per-layer state out (model.py:654-662)."""
        hidden = self.embed(self._bound("table"), token_ids)
        normed, states = self.decode_hidden(hidden, layer_args, caches)
        return self.lm_head(normed, self._bound("w_head")), states

    def init_caches(self, device="cuda:0"):
        """Zero conv windows and recurrent states, empty KV caches (model.py:664-686)."""
        c = self.cfg
        entries = []
        for kind in self.layer_types:
            if kind == "linear_attention":
                entries.append((torch.zeros(1, c.conv_dim, c.conv_kernel - 1, device=device),
                                torch.zeros(1, c.lin_value_heads, c.lin_key_dim,
                                            c.lin_value_dim, device=device)))
            else:
                empty = torch.zeros(1, 0, c.kv_heads, c.head_dim, device=device)
                entries.append((empty, empty))
        return tuple(entries)

    def append_cache(self, caches, fresh):
        """The window slides by its new column, the matrix is replaced, K/V grow
        (advance_state, model.py:573-586)."""
        out = []
        for kind, state, new in zip(self.layer_types, caches, fresh):
            if kind == "linear_attention":
                window, _ = state
                column, updated = new
                out.append((torch.cat([window, column.to(window.dtype)], dim=2)
                            [:, :, -(self.cfg.conv_kernel - 1):], updated))
            else:
                out.append(tuple(torch.cat([old, nw.to(old.dtype)], dim=1)
                                 for old, nw in zip(state, new)))
        return tuple(out)

    def prepare_inputs_for_generation(self, input_ids, step, caches, device="cuda:0"):
        """The token, the rope row at `step` and the scale for each attention layer
        (model.py:696-709)."""
        c = self.cfg
        token_ids = input_ids[step].reshape(1).to(device=device, dtype=I64)
        inv = 1.0 / c.rope_theta ** (torch.arange(0, c.rot_dim, 2, dtype=F32) / c.rot_dim)
        ph = torch.cat((step * inv, step * inv))[None]
        cos, sin = ph.cos().to(BF).to(device), ph.sin().to(BF).to(device)
        pos_ids = torch.zeros(1, device=device, dtype=I32)
        scale = torch.full((1, 1, 1, 1), c.head_dim ** -0.5, device=device, dtype=F32)
        layer_args = tuple((cos, sin, pos_ids, scale) if kind == "full_attention" else ()
                           for kind in self.layer_types)
        return token_ids, layer_args, caches


# ===========================================================================
# Granite-4.0-H-small (C5)
# ===========================================================================
class GraniteMamba:
    """``GraniteMamba`` (examples/granite_4_0_h_small-cuda/model.py:131-270)."""

    def __init__(self, cfg: GraniteConfig, ops: _Ops):
        self.cfg, self.ops = cfg, ops

    def in_projection(self, hidden, gamma_in, w_in):
        """tf.rms_norm then in_proj (model.py:141-151) -> (1, PROJ) bf16."""
        c, o = self.cfg, self.ops
        x = _rows(hidden, c.hidden)
        R = x.shape[0]
        xn = o.rmsnorm_tf(x, gamma_in, c.eps, packed=True)
        w = o.packed("m_in", lambda: w_in, w_in)
        out = torch.empty(R, c.mamba_in, dtype=BF, device=x.device)
        o.gemm(xn, w, R, c.hidden, c.mamba_in, _lib.EPI_STORE, out, c.mamba_in)
        return out

    def conv_step(self, conv_state, entry, conv_w, conv_b):
        """(1, CONVD, 3), (1, CONVD, 1) -> silu(window . w + b), bf16 ops (model.py:153-168)."""
        c, o = self.cfg, self.ops
        R = int(conv_state.shape[0])
        win = o.to_bf16(conv_state)
        ent = o.to_bf16(entry.reshape(R, c.conv_dim))
        out = torch.empty(R, c.conv_dim, dtype=BF, device=win.device)
        a = _lib.TfdConvStepArgs(window=ptr(win), entry=ptr(ent), lde=c.conv_dim,
                                 conv_w=ptr(conv_w.to(BF).contiguous()),
                                 conv_b=ptr(conv_b.to(BF).contiguous()), out=ptr(out),
                                 ldo=c.conv_dim, rows=R, channels=c.conv_dim,
                                 kernel=c.conv_kernel, policy=_lib.POLICY_BF16)
        o.L.tfd_conv_step_rows(ctypes_addr(a), _stream(win))
        return out

    def ssm_step(self, ssm_state, x, b_vec, c_vec, dt_raw, a_log, dt_bias, d_skip):
        """One token of the selective state update (model.py:169-221) -> (y (1, NH,
        PD) bf16, updated (1, NH, PD, NS) f32)."""
        c, o = self.cfg, self.ops
        R = int(ssm_state.shape[0])
        nh, pd, ns = c.mamba_heads, c.mamba_head_dim, c.d_state
        st = o.to_f32(ssm_state)
        upd = torch.empty_like(st)
        xb, bb, cb, db = (o.to_bf16(t) for t in (x, b_vec, c_vec, dt_raw))
        y = torch.empty(R, nh * pd, dtype=BF, device=st.device)
        a = _lib.TfdSsmStepArgs(state_in=ptr(st), state_out=ptr(upd), x=ptr(xb), ldx=nh * pd,
                                b_vec=ptr(bb), ldb=ns, c_vec=ptr(cb), ldc=ns, dt_raw=ptr(db),
                                lddt=nh, a_log=ptr(a_log), dt_bias=ptr(dt_bias),
                                d_skip=ptr(d_skip), y=ptr(y), ldy=nh * pd, rows=R, heads=nh,
                                head_dim=pd, state_dim=ns)
        o.L.tfd_ssm_step_bf16(ctypes_addr(a), _stream(st))
        return y.reshape(R, nh, pd), upd

    def gated_out(self, y, gate, gamma_ssm, w_out):
        """RMSNormGated then out_proj (model.py:222-237) -> (1, 1, H) bf16."""
        c, o = self.cfg, self.ops
        n = c.d_inner
        yb, gb = o.to_bf16(_rows(y, n)), o.to_bf16(_rows(gate, n))
        R = yb.shape[0]
        normed = torch.empty(R, n, dtype=BF, device=yb.device)
        a = _lib.TfdGatedNormArgs(y=ptr(yb), ldy=n, gate=ptr(gb), ldg=n, gamma=ptr(gamma_ssm),
                                  out=ptr(normed), ldo=n, rows=R, n=n, eps=c.eps)
        o.L.tfd_gated_rmsnorm_bf16(ctypes_addr(a), _stream(yb))
        w = o.packed("m_out", lambda: w_out, w_out)
        out = torch.empty(R, c.hidden, dtype=BF, device=yb.device)
        o.gemm(operand_order(normed), w, R, n, c.hidden, _lib.EPI_STORE, out, c.hidden)
        return out.reshape(R, 1, c.hidden)

    def mamba_mixer(self, hidden, gamma_in, w_in, conv_w, conv_b, a_log, dt_bias, d_skip,
                    conv_state, ssm_state, gamma_ssm, w_out):
        """The whole mixer (model.py:239-270) -> (out (1, 1, H) bf16, entry (1, CONVD,
        1) bf16, updated ssm state f32), through the fused tfd_mamba_step."""
        c, o = self.cfg, self.ops
        proj = self.in_projection(hidden, gamma_in, w_in)
        R, dev = proj.shape[0], proj.device
        conv_in = o.to_bf16(conv_state).clone()
        conv_out = torch.empty_like(conv_in)
        state = o.to_f32(ssm_state).clone()
        mix = torch.zeros(32 * c.d_inner, dtype=BF, device=dev)
        gated = torch.zeros(R, c.d_inner, dtype=F32, device=dev)
        ssq = torch.zeros(R, c.mamba_heads, dtype=F32, device=dev)
        a = _lib.TfdMambaArgs()
        a.proj, a.proj_ld, a.conv_in, a.conv_out = ptr(proj), c.mamba_in, ptr(conv_in), \
            ptr(conv_out)
        a.state = ptr(state)
        a.conv_w, a.conv_b = ptr(conv_w), ptr(conv_b)
        a.a_log, a.dt_bias, a.d_skip = ptr(a_log), ptr(dt_bias), ptr(d_skip)
        a.gamma, a.gated, a.ssq, a.out = ptr(gamma_ssm), ptr(gated), ptr(ssq), ptr(mix)
        a.rows, a.heads, a.head_dim, a.state_dim = R, c.mamba_heads, c.mamba_head_dim, c.d_state
        a.groups, a.conv_kernel, a.eps = 1, c.conv_kernel, c.eps
        o.L.tfd_mamba_step(ctypes_addr(a), _stream(proj))
        w = o.packed("m_out", lambda: w_out, w_out)
        out = torch.empty(R, c.hidden, dtype=BF, device=dev)
        o.gemm(mix, w, R, c.d_inner, c.hidden, _lib.EPI_STORE, out, c.hidden)
        entry = proj[:, c.d_inner:c.d_inner + c.conv_dim].reshape(R, c.conv_dim, 1).clone()
        return out.reshape(R, 1, c.hidden), entry, state


class GraniteAttention:
    """``GraniteAttention`` (model.py:273-366): GQA with no position embedding over a
    fixed-capacity cache."""

    def __init__(self, cfg: GraniteConfig, ops: _Ops, page_seed: int = 0):
        self.cfg, self.ops, self.page_seed = cfg, ops, page_seed

    def _proj_rows(self, hidden, gamma_in, w_q, w_k, w_v):
        c, o = self.cfg, self.ops
        x = _rows(hidden, c.hidden)
        R = x.shape[0]
        xn = o.rmsnorm_tf(x, gamma_in, c.eps, packed=True)
        w = o.packed("a_in", lambda: torch.cat([w_q, w_k, w_v]), w_q, w_k, w_v)
        out = torch.empty(R, c.attn_in, dtype=BF, device=x.device)
        o.gemm(xn, w, R, c.hidden, c.attn_in, _lib.EPI_STORE, out, c.attn_in)
        return out

    def qkv(self, hidden, gamma_in, w_q, w_k, w_v):
        """tf.rms_norm then the three projections (model.py:281-305)."""
        c = self.cfg
        HQ, HKV, D = c.heads, c.kv_heads, c.head_dim
        p = self._proj_rows(hidden, gamma_in, w_q, w_k, w_v)
        R = p.shape[0]
        return (p[:, :HQ * D].reshape(R, 1, HQ, D).clone(),
                p[:, HQ * D:(HQ + HKV) * D].reshape(R, 1, HKV, D).clone(),
                p[:, (HQ + HKV) * D:].reshape(R, 1, HKV, D).clone())

    def _attend_rows(self, qkv_rows, k_cache, v_cache, cur):
        """Attention over positions 0..cur of the caches, the token's own k/v in
        qkv_rows (tfd_gqa_decode appends them at cur) -> o_proj's input."""
        c, o = self.cfg, self.ops
        HQ, HKV, D = c.heads, c.kv_heads, c.head_dim
        R, dev = qkv_rows.shape[0], qkv_rows.device
        ctx = _PagedContext(k_cache[:, :cur], v_cache[:, :cur], HKV, D, dev, self.page_seed,
                            split_len=256)
        mix = torch.zeros(32 * HQ * D, dtype=BF, device=dev)
        err = torch.zeros(1, dtype=I32, device=dev)
        a = ctx.gqa_args(qkv_rows, c.attn_in, HQ, HKV, D, c.attention_multiplier, c.eps, mix,
                         _lib.POLICY_BF16, err)
        o.L.tfd_gqa_decode(ctypes_addr(a), _stream(qkv_rows))
        _check_err(err, "attend")
        return mix

    def _o_proj(self, mix, w_o, R):
        c, o = self.cfg, self.ops
        w = o.packed("a_out", lambda: w_o, w_o)
        out = torch.empty(R, c.hidden, dtype=BF, device=mix.device)
        o.gemm(mix, w, R, c.heads * c.head_dim, c.hidden, _lib.EPI_STORE, out, c.hidden)
        return out.reshape(R, 1, c.hidden)

    def attend(self, q, k_cache, v_cache, cur_pos, mask, w_o):
        """Attention over the live positions 0..cur_pos of the caches (the token's
        own entry already written there), then o_proj (model.py:307-344).  The
        kernel reads `cur_pos` and stops there, as the authored comment allows;
        `mask` says the same thing and is not read."""
        c = self.cfg
        HQ, HKV, D = c.heads, c.kv_heads, c.head_dim
        R = int(q.shape[0])
        cur = int(cur_pos.reshape(-1)[0])
        rows = torch.cat([self.ops.to_bf16(q.reshape(R, HQ * D)),
                          k_cache[:, cur].reshape(R, HKV * D).to(BF),
                          v_cache[:, cur].reshape(R, HKV * D).to(BF)], dim=1).contiguous()
        return self._o_proj(self._attend_rows(rows, k_cache, v_cache, cur), w_o, R)

    def full_attention(self, hidden, gamma_in, w_q, w_k, w_v, k_cache, v_cache, cur_pos, mask,
                       w_o):
        """qkv, cache_update at cur_pos, attend (model.py:346-366) -> (out, k_next,
        v_next): the caches come back with this token's entry written."""
        c = self.cfg
        HQ, HKV, D = c.heads, c.kv_heads, c.head_dim
        rows = self._proj_rows(hidden, gamma_in, w_q, w_k, w_v)
        R = rows.shape[0]
        cur = int(cur_pos.reshape(-1)[0])
        if not 0 <= cur < k_cache.shape[1]:
            raise ValueError(f"cur_pos {cur} outside the cache capacity {k_cache.shape[1]}")
        out = self._o_proj(self._attend_rows(rows, k_cache, v_cache, cur), w_o, R)
        k_next, v_next = k_cache.clone(), v_cache.clone()
        k_next[:, cur] = rows[:, HQ * D:(HQ + HKV) * D].reshape(R, HKV, D).to(k_next.dtype)
        v_next[:, cur] = rows[:, (HQ + HKV) * D:].reshape(R, HKV, D).to(v_next.dtype)
        return out, k_next, v_next


class GraniteRouter:
    """``GraniteRouter.routing`` (model.py:369-386): the top k logits, softmax over
    them -> (weights (S, K) bf16, indices (S, K) int64)."""

    def __init__(self, cfg: GraniteConfig, ops: _Ops):
        self.cfg, self.ops = cfg, ops

    def routing(self, tokens, w_router):
        c, o = self.cfg, self.ops
        H, E, K = c.hidden, c.experts, c.top_k
        x = _rows(tokens, H)
        R = x.shape[0]
        w = o.packed("g_router", lambda: w_router, w_router)
        logits = torch.empty(R, E, dtype=F32, device=x.device)
        o.gemm(operand_order(o.to_bf16(x)), w, R, H, E, _lib.EPI_LOGITS, logits, E)
        weights = torch.empty(R, K, dtype=F32, device=x.device)
        idx = torch.empty(R, K, dtype=I32, device=x.device)
        o.L.tfd_route_topk(ptr(logits), E, R, E, K, _lib.ROUTE_TOPK_SOFTMAX, ptr(weights),
                           ptr(idx), _stream(logits))
        return weights.to(BF), idx.to(I64)           # bf16 values: the cast is exact


class GraniteMoE:
    """``GraniteMoE`` (model.py:389-477)."""

    def __init__(self, cfg: GraniteConfig, ops: _Ops):
        self.cfg, self.ops = cfg, ops
        self.router = GraniteRouter(cfg, ops)
        self.weights: dict | None = None

    def post_norm(self, hidden, gamma_post):
        """tf.rms_norm (model.py:396-403) -> (S, H) bf16."""
        c, o = self.cfg, self.ops
        return o.rmsnorm_tf(_rows(hidden, c.hidden), gamma_post, c.eps, packed=False)

    def _call(self, tokens, weights, indices, w_gate, w_up, w_down, w_shared_in, w_shared_out):
        c, o = self.cfg, self.ops
        x = o.to_bf16(_rows(tokens, c.hidden))
        out = _moe_call(o, c, x, o.to_f32(weights), indices.to(I32).contiguous(), w_gate, w_up,
                        w_down, w_shared_in, w_shared_out, None, 0, _lib.POLICY_BF16,
                        c.moe_inter, c.shared_inter)
        return out.to(BF)                              # bf16 values: exact

    def experts(self, tokens, weights, indices, w_gate, w_up, w_down, w_shared_in,
                w_shared_out):
        """Routed experts + shared MLP, summed (model.py:456-471) -> (1, S, H) bf16."""
        out = self._call(tokens, weights, indices, w_gate, w_up, w_down, w_shared_in,
                         w_shared_out)
        return out.reshape(1, -1, self.cfg.hidden)

    def routed_experts(self, tokens, weights, indices, w_gate, w_up, w_down):
        """The picked experts mixed by the routing weights (model.py:405-440) -> (S, H)
        bf16: ``experts`` with a shared MLP of zero weights (it adds an exact 0)."""
        c = self.cfg
        dev = tokens.device
        z = self.ops.derived.get(("g_zero_shared", str(dev)),
                                 lambda: (torch.zeros(2 * c.shared_inter, c.hidden, dtype=BF,
                                                      device=dev),
                                          torch.zeros(c.hidden, c.shared_inter, dtype=BF,
                                                      device=dev)))
        return self._call(tokens, weights, indices, w_gate, w_up, w_down, z[0], z[1])

    def shared_mlp(self, tokens, w_shared_in, w_shared_out):
        """``GraniteMoeHybridMLP`` (model.py:442-454) -> (S, H) bf16."""
        c, o = self.cfg, self.ops
        x = o.to_bf16(_rows(tokens, c.hidden))
        return _only_shared(o, c, x, w_shared_in, w_shared_out, None, _lib.POLICY_BF16).to(BF)

    def forward(self, hidden):
        """post-norm, route, then the experts (model.py:473-477)."""
        w = self.weights
        if w is None:
            raise TypeError("this module is not loaded: call load(weights) on the decoder")
        tokens = self.post_norm(hidden, w["gamma_post"])
        weights, indices = self.router.routing(tokens, w["router.w_router"])
        return self.experts(tokens, weights, indices, w["w_gate"], w["w_up"], w["w_down"],
                            w["w_shared_in"], w["w_shared_out"])


class _GraniteLayer:
    """``GraniteMambaDecoderLayer`` / ``GraniteAttentionDecoderLayer``
    (model.py:480-523): mixer + scaled residual, MoE + scaled residual."""

    def __init__(self, cfg, ops, kind, page_seed):
        self.kind = kind
        self.mixer = (GraniteAttention(cfg, ops, page_seed) if kind == "full_attention"
                      else GraniteMamba(cfg, ops))
        self.moe = GraniteMoE(cfg, ops)
        self.cfg, self.ops = cfg, ops
        self.weights: dict | None = None

    def residual_add(self, a, b):
        """a + b * residual_multiplier at bf16 (model.py:501-510)."""
        c, o = self.cfg, self.ops
        ab, bb = o.to_bf16(a), o.to_bf16(b)
        n = c.hidden
        R = ab.numel() // n
        out = torch.empty(R, n, dtype=BF, device=ab.device)
        o.L.tfd_scaled_add_rows(ptr(ab), n, ptr(bb), n, 0, c.residual_multiplier, ptr(out), n,
                                R, n, _stream(ab))
        return out.reshape(a.shape)

    def _mixer(self, hidden, *args):
        w = self.weights
        if self.kind == "full_attention":
            k_cache, v_cache, cur_pos, mask = args
            return self.mixer.full_attention(hidden, w["gamma_in"], w["w_q"], w["w_k"], w["w_v"],
                                             k_cache, v_cache, cur_pos, mask, w["w_o"])
        conv_state, ssm_state = args
        return self.mixer.mamba_mixer(hidden, w["gamma_in"], w["w_in"], w["conv_w"],
                                      w["conv_b"], w["a_log"], w["dt_bias"], w["d_skip"],
                                      conv_state, ssm_state, w["gamma_ssm"], w["w_out"])

    def forward(self, hidden, mixer_args):
        mixed, *state = self._mixer(hidden, *mixer_args)
        attended = self.residual_add(hidden, mixed)
        expert_out = self.moe.forward(attended)
        return self.residual_add(attended, expert_out), tuple(state)


def granite_declared(cfg: GraniteConfig) -> dict:
    """Canonical name -> (shape, dtype) of the authored bf16 weights
    (model.py:141-470, 614-645; names as hf_alias.py:44-91 maps them)."""
    H, E, I, IS = cfg.hidden, cfg.experts, cfg.moe_inter, cfg.shared_inter
    HQ, HKV, D = cfg.heads, cfg.kv_heads, cfg.head_dim
    out = {"table": (cfg.vocab, H), "gamma_final": (H,)}
    for i in range(cfg.layers):
        m, e = f"layer{i}.mixer.", f"layer{i}.moe."
        if cfg.is_attention(i):
            out.update({m + "gamma_in": (H,), m + "w_q": (HQ * D, H), m + "w_k": (HKV * D, H),
                        m + "w_v": (HKV * D, H), m + "w_o": (H, HQ * D)})
        else:
            nh = cfg.mamba_heads
            out.update({m + "gamma_in": (H,), m + "w_in": (cfg.mamba_in, H),
                        m + "conv_w": (cfg.conv_dim, cfg.conv_kernel), m + "conv_b": (cfg.conv_dim,),
                        m + "a_log": (nh,), m + "dt_bias": (nh,), m + "d_skip": (nh,),
                        m + "gamma_ssm": (cfg.d_inner,), m + "w_out": (H, cfg.d_inner)})
        out.update({e + "gamma_post": (H,), e + "w_gate": (E, I, H), e + "w_up": (E, I, H),
                    e + "w_down": (E, H, I), e + "w_shared_in": (2 * IS, H),
                    e + "w_shared_out": (H, IS), e + "router.w_router": (E, H)})
    return {k: (v, BF) for k, v in out.items()}


def granite_canonical(cfg: GraniteConfig, w: dict) -> dict:
    """The engine's fp8 weights (``hybrid.granite``) dequantised to the authored bf16
    declaration under the twin's canonical names: W = bf16(e4m3(code) * scale[row])."""
    H, E, I = cfg.hidden, cfg.experts, cfg.moe_inter
    HQ, HKV, D = cfg.heads, cfg.kv_heads, cfg.head_dim

    def deq(codes, scale):
        return (codes.view(torch.float8_e4m3fn).float() * scale.float()[:, None]).to(BF)

    out = {"table": w["embed"], "gamma_final": w["gamma_final"]}
    for i in range(cfg.layers):
        p, m, e = f"layer{i}.", f"layer{i}.mixer.", f"layer{i}.moe."
        out[m + "gamma_in"] = w[p + "gamma_in"]
        w_in = deq(w[p + "w_in"], w[p + "w_in_scale"])
        out_w = deq(w[p + "w_out"], w[p + "w_out_scale"])
        if cfg.is_attention(i):
            out[m + "w_q"] = w_in[:HQ * D].contiguous()
            out[m + "w_k"] = w_in[HQ * D:(HQ + HKV) * D].contiguous()
            out[m + "w_v"] = w_in[(HQ + HKV) * D:].contiguous()
            out[m + "w_o"] = out_w
        else:
            out[m + "w_in"] = w_in
            for n in ("conv_w", "conv_b", "a_log", "dt_bias", "d_skip", "gamma_ssm"):
                out[m + n] = w[p + n]
            out[m + "w_out"] = out_w
        out[e + "gamma_post"] = w[p + "gamma_post"]
        out[e + "w_gate"] = deq(w[p + "w_gate"], w[p + "s_gate"]).view(E, I, H)
        out[e + "w_up"] = deq(w[p + "w_up"], w[p + "s_up"]).view(E, I, H)
        out[e + "w_down"] = deq(w[p + "w_down"], w[p + "s_down"]).view(E, H, I)
        out[e + "w_shared_in"] = deq(w[p + "w_shared_in"], w[p + "w_shared_in_scale"])
        out[e + "w_shared_out"] = deq(w[p + "w_shared_out"], w[p + "w_shared_out_scale"])
        out[e + "router.w_router"] = deq(w[p + "w_router"], w[p + "w_router_scale"])
    return out


class Granite4_0_H_Small:
    """``Granite4_0_H_Small`` (model.py:601-720): root functions and, once loaded, the
    orchestration over a fixed KV capacity."""

    def __init__(self, cfg: GraniteConfig, capacity: int = 4096, page_seed: int = 0):
        self.cfg, self.capacity = cfg, capacity
        self.ops = _Ops()
        self.layer_types = ["full_attention" if cfg.is_attention(i) else "linear_attention"
                            for i in range(cfg.layers)]
        self.layers = [_GraniteLayer(cfg, self.ops, kind, page_seed) for kind in self.layer_types]
        self.weights: dict | None = None

    def embed(self, table, token_ids):
        """The table row times embedding_multiplier, bf16 (model.py:614-624)."""
        c, o = self.cfg, self.ops
        H, V = c.hidden, c.vocab
        dev = table.device
        ids = token_ids.reshape(-1).to(device=dev, dtype=I64).contiguous()
        R = ids.numel()
        rows = torch.empty(R, H, dtype=BF, device=dev)
        err = torch.zeros(1, dtype=I32, device=dev)
        o.L.tfd_embed_rows_bf16(ptr(table.contiguous()), ptr(ids), ptr(rows), H, R, H, V,
                                ptr(err), _stream(rows))
        if int(err.item()):
            raise IndexError(f"token id outside [0, {V})")
        out = torch.empty_like(rows)
        o.L.tfd_scaled_add_rows(None, 0, ptr(rows), H, 0, c.embedding_multiplier, ptr(out), H,
                                R, H, _stream(rows))
        return out.reshape(R, 1, H)

    def final_rms_norm(self, hidden, gamma_final):
        """tf.rms_norm after the last layer (model.py:626-632)."""
        c, o = self.cfg, self.ops
        return o.rmsnorm_tf(_rows(hidden, c.hidden), gamma_final, c.eps,
                            packed=False).reshape(hidden.shape)

    def lm_head(self, hidden, table):
        """hidden @ table^T / logits_scaling, bf16 (model.py:634-645) -> (1, V)."""
        c, o = self.cfg, self.ops
        x = _rows(hidden, c.hidden)
        R = x.shape[0]
        w = o.packed("g_head", lambda: table, table)
        out = torch.empty(R, c.vocab, dtype=F32, device=x.device)
        work = o.work(x.device)
        o.L.tfd_gemm_skinny_bf16_logits_div(ptr(operand_order(o.to_bf16(x))), ptr(w), R,
                                            c.hidden, c.vocab, c.logits_scaling, ptr(out),
                                            c.vocab, ptr(work), work.numel(), _stream(x))
        return out.to(BF)                              # bf16 values: exact

    def load(self, weights: dict) -> "Granite4_0_H_Small":
        _validate(granite_declared(self.cfg), weights)
        self.weights = weights
        for i, layer in enumerate(self.layers):
            m, e = f"layer{i}.mixer.", f"layer{i}.moe."
            layer.weights = {k[len(m):]: v for k, v in weights.items() if k.startswith(m)}
            layer.moe.weights = {k[len(e):]: v for k, v in weights.items() if k.startswith(e)}
        return self

    def _bound(self, name):
        if self.weights is None:
            raise TypeError("Granite4_0_H_Small is not loaded: call load(weights) first")
        return self.weights[name]

    def decode_hidden(self, hidden, layer_args, caches):
        """Every layer, then the final norm (model.py:647-664)."""
        n = len(self.layers)
        if len(layer_args) != n or len(caches) != n:
            raise ValueError(f"decoder has {n} layers but was given {len(layer_args)} argument "
                             f"tuples and {len(caches)} caches")
        states = []
        for layer, args, cache in zip(self.layers, layer_args, caches):
            hidden, state = layer.forward(hidden, (*cache, *args))   # the state comes first
            states.append(state)
        return self.final_rms_norm(hidden, self._bound("gamma_final")), tuple(states)

    def forward(self, token_ids, layer_args, caches):
        hidden = self.embed(self._bound("table"), token_ids)
        normed, states = self.decode_hidden(hidden, layer_args, caches)
        return self.lm_head(normed, self._bound("table")), states

    def init_caches(self, device="cuda:0"):
        """Zero windows and states; zeroed full-capacity K/V (model.py:676-698)."""
        c = self.cfg
        entries = []
        for kind in self.layer_types:
            if kind == "linear_attention":
                entries.append((torch.zeros(1, c.conv_dim, c.conv_kernel - 1, dtype=BF,
                                            device=device),
                                torch.zeros(1, c.mamba_heads, c.mamba_head_dim, c.d_state,
                                            device=device)))
            else:
                empty = torch.zeros(1, self.capacity, c.kv_heads, c.head_dim, dtype=BF,
                                    device=device)
                entries.append((empty, empty.clone()))
        return tuple(entries)

    def append_cache(self, caches, fresh):
        """The window slides, the matrix is replaced; attention caches come back
        whole (advance_state, model.py:556-571)."""
        out = []
        for kind, state, new in zip(self.layer_types, caches, fresh):
            if kind == "linear_attention":
                window, _ = state
                column, updated = new
                out.append((torch.cat([window, column.to(window.dtype)], dim=2)
                            [:, :, -(self.cfg.conv_kernel - 1):], updated))
            else:
                out.append(tuple(new))
        return tuple(out)

    def prepare_inputs_for_generation(self, input_ids, step, caches, device="cuda:0"):
        """The token, cur_pos and the additive mask for each attention layer
        (model.py:707-720, attention_mask :584-598)."""
        token_ids = input_ids[step].reshape(1).to(device=device, dtype=I64)
        cur_pos = torch.full((1,), step, device=device, dtype=I32)
        live = torch.arange(self.capacity, device=device) <= step
        mask = torch.where(live, torch.zeros((), dtype=BF, device=device),
                           torch.full((), -1.0e30, dtype=BF, device=device)).reshape(1, 1, -1)
        layer_args = tuple(() if kind == "linear_attention" else (cur_pos, mask)
                           for kind in self.layer_types)
        return token_ids, layer_args, caches
