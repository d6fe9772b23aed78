"""Granite-4.0-H-style hybrid decode on the GPU (workload C5).

The decode step of ``examples/granite_4_0_h_small-cuda/model.py``
(``Granite4_0_H_Small``: Mamba2 and GQA layers, each followed by a top-10 MoE
with a shared MLP) at the arithmetic of the authored HIR: a bf16 residual
stream, every bf16 op rounded as written, f32 where the HIR casts.  The linear
weights are fp8-e4m3fn with one f32 scale per output row (the workload's
per-channel fp8); the tied embedding / head table stays bf16.  Per layer:

* input RMSNorm (the HIR's ``tf.rms_norm``: one rounding after gamma, in operand
  order) -> fp8 in-projection -> Mamba2 step
  (``tfd_mamba_step``) or GQA decode (``tfd_gqa_decode``, no RoPE) -> fp8
  out-projection whose epilogue adds ``bf16(b * residual_multiplier)`` into the
  stream (``tfd_gemm_skinny_fp8_resid_scaled``);
* post RMSNorm in both layouts at once (``tfd_tf_rmsnorm_rows_bf16``) -> fp8 router
  -> routed experts + shared MLP (``tfd_moe_experts``: top-10-then-softmax routing
  in its first launch, then fp8, expert-grouped, its last launch adding the
  scaled output into the stream);

then the final norm, the head over the tied table divided by ``logits_scaling``
(``tfd_gemm_skinny_bf16_logits_div``, model.py:636-645), the greedy pick and the
next token's embedding times ``embedding_multiplier``.  Sequences (up to 32) step
together; a step is recorded into two HIP graphs (the conv windows ping-pong).
Weights are synthetic (random init on the device).
"""
from __future__ import annotations

from dataclasses import dataclass
from time import perf_counter

import torch

from .. import _lib
from .._lib import lib, ptr
from ..sampling import Picker, Sampling
from .qwen3_5 import attention_splits, ctypes_addr

BF = torch.bfloat16
F32 = torch.float32
I32 = torch.int32


@dataclass(frozen=True)
class GraniteConfig:
    """Workload C5's shape; attention layers at the
    published ``layer_types`` positions (examples/granite_4_0_h_small-cuda/
    config.json), multipliers as published there."""

    hidden: int = 4096
    layers: int = 40
    attention_layers: tuple = (5, 15, 25, 35)
    mamba_heads: int = 64
    mamba_head_dim: int = 64
    d_state: int = 128
    conv_kernel: int = 4
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    experts: int = 72
    top_k: int = 10
    moe_inter: int = 768
    shared_inter: int = 1536
    vocab: int = 100352
    eps: float = 1e-5
    embedding_multiplier: float = 12.0
    residual_multiplier: float = 0.22
    attention_multiplier: float = 0.0078125
    logits_scaling: float = 16.0

    def is_attention(self, i: int) -> bool:
        return i in self.attention_layers

    @property
    def d_inner(self) -> int:
        return self.mamba_heads * self.mamba_head_dim

    @property
    def conv_dim(self) -> int:
        return self.d_inner + 2 * self.d_state

    @property
    def mamba_in(self) -> int:
        """Rows of in_proj: gate, conv channels (x|B|C), dt."""
        return self.d_inner + self.conv_dim + self.mamba_heads

    @property
    def attn_in(self) -> int:
        return (self.heads + 2 * self.kv_heads) * self.head_dim


def _fp8(N, K, g, device, std):
    """e4m3fn codes of N(0, 1) draws and a per-row scale near `std`."""
    codes = torch.randn(N, K, generator=g, device=device).to(torch.float8_e4m3fn).view(torch.uint8)
    scale = std * (0.9 + 0.2 * torch.rand(N, generator=g, device=device))
    return codes, scale


def synthetic_weights(cfg: GraniteConfig, seed: int = 0, device: str = "cuda:0",
                      std: float = 0.02) -> dict[str, torch.Tensor]:
    """Random-init weights: every linear weight fp8 codes + f32 row scales with
    values near N(0, std); norm scales 1 + N(0, std); the bf16 table N(0, std);
    conv, A_log, dt_bias, D small normal draws."""
    g = torch.Generator(device=device).manual_seed(seed)

    def rn(*shape, s=std):
        return (torch.randn(*shape, generator=g, device=device) * s).to(BF)

    def gamma(n):
        return (1 + torch.randn(n, generator=g, device=device) * std).to(BF)

    H, E, I, IS = cfg.hidden, cfg.experts, cfg.moe_inter, cfg.shared_inter
    w = {"embed": rn(cfg.vocab, H), "gamma_final": gamma(H)}

    def lin(name, N, K):
        w[name], w[name + "_scale"] = _fp8(N, K, g, device, std)

    for i in range(cfg.layers):
        p = f"layer{i}."
        w[p + "gamma_in"] = gamma(H)
        if cfg.is_attention(i):
            lin(p + "w_in", cfg.attn_in, H)
            lin(p + "w_out", H, cfg.heads * cfg.head_dim)
        else:
            lin(p + "w_in", cfg.mamba_in, H)
            w[p + "conv_w"] = rn(cfg.conv_dim, cfg.conv_kernel, s=0.5)
            w[p + "conv_b"] = rn(cfg.conv_dim, s=0.1)
            w[p + "a_log"] = rn(cfg.mamba_heads, s=0.5)
            w[p + "dt_bias"] = rn(cfg.mamba_heads, s=0.5)
            w[p + "d_skip"] = rn(cfg.mamba_heads, s=1.0)
            w[p + "gamma_ssm"] = gamma(cfg.d_inner)
            lin(p + "w_out", H, cfg.d_inner)
        w[p + "gamma_post"] = gamma(H)
        lin(p + "w_router", E, H)
        w[p + "w_gate"], w[p + "s_gate"] = _fp8(E * I, H, g, device, std)
        w[p + "w_up"], w[p + "s_up"] = _fp8(E * I, H, g, device, std)
        w[p + "w_down"], w[p + "s_down"] = _fp8(E * H, I, g, device, std)
        lin(p + "w_shared_in", 2 * IS, H)
        lin(p + "w_shared_out", H, IS)
    return w


U8 = torch.uint8


def declared_shapes(cfg: GraniteConfig) -> dict[str, tuple[tuple[int, ...], torch.dtype]]:
    """Every weight the engine reads: shape and dtype (fp8 linears as uint8
    e4m3fn codes ``[N][K]`` with f32 row scales ``[N]``)."""
    H, E, I, IS = cfg.hidden, cfg.experts, cfg.moe_inter, cfg.shared_inter
    out = {"embed": ((cfg.vocab, H), BF), "gamma_final": ((H,), BF)}

    def lin(p, name, N, K, scale=None):
        out[p + name] = ((N, K), U8)
        out[p + (scale or name + "_scale")] = ((N,), F32)

    for i in range(cfg.layers):
        p = f"layer{i}."
        out[p + "gamma_in"] = ((H,), BF)
        out[p + "gamma_post"] = ((H,), BF)
        if cfg.is_attention(i):
            lin(p, "w_in", cfg.attn_in, H)
            lin(p, "w_out", H, cfg.heads * cfg.head_dim)
        else:
            lin(p, "w_in", cfg.mamba_in, H)
            out[p + "conv_w"] = ((cfg.conv_dim, cfg.conv_kernel), BF)
            out[p + "conv_b"] = ((cfg.conv_dim,), BF)
            for n in ("a_log", "dt_bias", "d_skip"):
                out[p + n] = ((cfg.mamba_heads,), BF)
            out[p + "gamma_ssm"] = ((cfg.d_inner,), BF)
            lin(p, "w_out", H, cfg.d_inner)
        lin(p, "w_router", E, H)
        lin(p, "w_gate", E * I, H, "s_gate")
        lin(p, "w_up", E * I, H, "s_up")
        lin(p, "w_down", E * H, I, "s_down")
        lin(p, "w_shared_in", 2 * IS, H)
        lin(p, "w_shared_out", H, IS)
    return out


def validate(cfg: GraniteConfig, weights: dict[str, torch.Tensor]) -> None:
    """``KeyError`` for a missing weight, ``ValueError`` for a wrong shape or
    dtype -- the kernels take raw pointers and trust both."""
    for name, (shape, dt) in declared_shapes(cfg).items():
        if name not in weights:
            raise KeyError(f"weight {name!r} is declared but not supplied")
        t = weights[name]
        if tuple(t.shape) != shape:
            raise ValueError(f"weight {name!r}: declared shape {shape}, got {tuple(t.shape)}")
        if t.dtype != dt:
            raise ValueError(f"weight {name!r}: declared dtype {dt}, got {t.dtype}")


class GraniteEngine:
    """A Granite-style hybrid decoder stepping `rows` sequences together.

    ``weights`` is checked against ``declared_shapes(cfg)`` and copied to the
    device (contiguous) where it is not there already."""

    def __init__(self, cfg: GraniteConfig, weights: dict[str, torch.Tensor], *, rows: int,
                 device: str = "cuda:0", max_steps: int = 1024, page_seed: int = 0,
                 split_len: int | None = None, graph: bool = True, record_routes: bool = False,
                 sampling: Sampling | None = None):
        if not 1 <= rows <= 32:
            raise ValueError("rows: 1..32 sequences")
        self.cfg, self.B, self.device = cfg, rows, device
        self._lib = lib()
        self.sampling = sampling                # the token choice (None: greedy)
        self.nsteps = max_steps
        self.split_len = split_len
        # up to 16 sequences: the fp8 experts packed for the matrix-core pair
        # (tfd_moe_experts_packed, 98 us against 128 us per layer at batch 8);
        # more: row-major, the lane-sum kernels.  (At C4's bf16 widths the
        # lane-sum kernels already stream at 0.75-0.8 of HBM, and the pair's down
        # has only hidden / 16 = 128 blocks there: that engine keeps them.)
        self.moe_packed = _lib.moe_packed_fits(rows, cfg.top_k, cfg.hidden, cfg.moe_inter,
                                               cfg.shared_inter)
        # up to 8 sequences at the 4,096 hidden size: the router with the post
        # norm as its prologue (tfd_proj8_norm; 7.5 us against 9.7 for the norm
        # launch and the skinny GEMM, the same bits)
        self.router_norm = rows <= _lib.PROJ8_ROWS and cfg.hidden == _lib.PROJ8_K
        self._pack(weights)
        self._buffers(page_seed)
        # record_routes: each layer's top-k expert indices are copied into
        # routes[layer] as the step runs (a device copy inside the step's graph);
        # generate() keeps one [layers][rows][k] snapshot per step in
        # route_history, for tests that follow the engine's routing at near-ties
        self.routes = (torch.zeros(cfg.layers, rows, cfg.top_k, dtype=I32, device=device)
                       if record_routes else None)
        self.route_history = None
        self.graphs = None
        self._cur = 0
        if graph:
            self._capture()

    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def _packed8(self, codes: torch.Tensor) -> torch.Tensor:
        N, K = codes.shape
        out = torch.empty(-(-N // 16) * 16 * K, dtype=torch.uint8, device=self.device)
        self._lib.tfd_pack_skinny_fp8(ptr(codes), K, N, K, ptr(out), self._stream())
        return out

    def _pack(self, w):
        cfg = self.cfg
        validate(cfg, w)
        w = {n: w[n].to(self.device).contiguous() for n in declared_shapes(cfg)}
        self.layers = []
        for i in range(cfg.layers):
            p = f"layer{i}."
            d = {k[len(p):]: v for k, v in w.items() if k.startswith(p)}
            for name in ("w_in", "w_out", "w_router"):
                d[name] = self._packed8(d[name])
            if self.moe_packed:
                for name in ("w_gate", "w_up", "w_down", "w_shared_in", "w_shared_out"):
                    d[name] = self._packed8(d[name])
            self.layers.append(d)
        self.embed = w["embed"]
        self.gamma_final = w["gamma_final"]
        N, K = self.embed.shape
        self.head = torch.empty(-(-N // 16) * 16 * K, dtype=BF, device=self.device)
        self._lib.tfd_pack_skinny_bf16(ptr(self.embed), K, N, K, ptr(self.head), self._stream())
        torch.cuda.synchronize(self.device)

    def _buffers(self, page_seed):
        cfg, B, dev = self.cfg, self.B, self.device
        H, V, k = cfg.hidden, cfg.vocab, cfg.top_k

        def z(*shape, dtype=F32):
            return torch.zeros(*shape, dtype=dtype, device=dev)

        self.hidden = z(B, H, dtype=BF)
        self.emb = z(B, H, dtype=BF)
        self.xn = z(32 * H, dtype=BF)
        self.xm = z(B, H, dtype=BF)
        self.nproj = max(cfg.mamba_in, cfg.attn_in)
        self.nproj += (-self.nproj) % 8
        self.proj = z(B, self.nproj, dtype=BF)
        self.mix = z(32 * max(cfg.d_inner, cfg.heads * cfg.head_dim), dtype=BF)
        self.rlog = z(B, cfg.experts)
        self.rw = z(B, k)
        self.ridx = z(B, k, dtype=I32)
        ld = max(cfg.moe_inter, cfg.shared_inter)
        self.moe_hidden = z(B, k + 1, ld, dtype=BF)
        self.moe_sscale = z(B)
        self.moe_partial = None if self.moe_packed else z(B, k + 1, H)
        self.moe_groups = z(_lib.moe_group_words(cfg.experts, B), dtype=I32)
        self.moe_ld = ld
        self.state, self.conv = {}, {}
        for i in range(cfg.layers):
            if not cfg.is_attention(i):
                self.state[i] = z(B, cfg.mamba_heads, cfg.mamba_head_dim, cfg.d_state)
                self.conv[i] = (z(B, cfg.conv_dim, cfg.conv_kernel - 1, dtype=BF),
                                z(B, cfg.conv_dim, cfg.conv_kernel - 1, dtype=BF))
        self.gated = z(B, cfg.d_inner)
        self.ssq = z(B, cfg.mamba_heads)
        self.max_pages = -(-self.nsteps // 16)
        self.num_pages = B * self.max_pages
        gen = torch.Generator().manual_seed(page_seed)
        self.page_table = torch.randperm(self.num_pages, generator=gen).view(
            B, self.max_pages).to(I32).to(dev)
        self.kpool, self.vpool = {}, {}
        for i in range(cfg.layers):
            if cfg.is_attention(i):
                shape = (self.num_pages, cfg.kv_heads, 16, cfg.head_dim)
                self.kpool[i] = z(*shape, dtype=BF)
                self.vpool[i] = z(*shape, dtype=BF)
        if self.split_len is None:              # lengths follow each row's position
            self.nsplit = attention_splits(B, cfg.kv_heads, self.max_pages * 16)
        else:
            self.nsplit = -(-self.max_pages * 16 // self.split_len)
        self.stride = self.max_pages * 16
        self.scores = z(B * cfg.heads * self.stride)
        self.stats = z(B * cfg.heads * self.nsplit * 2)
        self.part = z(B * cfg.heads * self.nsplit * cfg.head_dim)
        self.counters = z(B * cfg.kv_heads, dtype=I32)
        self.logits = z(B, V)
        self.pick = z(B, dtype=I32)
        self.picker = Picker(self.sampling, B, V, dev)
        self.ids = z(B, dtype=torch.int64)
        self.pos = z(B, dtype=I32)
        self.inp = z(B, self.nsteps, dtype=I32)
        self.plen = z(B, dtype=I32)
        self.sam = z(B, self.nsteps, dtype=I32)
        self.err = z(1, dtype=I32)
        self.work = z(1 << 21)

    # ------------------------------------------------------------------ step
    def _gemm8(self, x, w, scale, K, N, epi, out, ldo, s):
        self._lib.tfd_gemm_skinny_fp8(ptr(x), ptr(w), ptr(scale), self.B, K, N, epi, None, 0,
                                      ptr(out), ldo, s)

    def _gemm8_residual(self, x, w, scale, K, s):
        """hidden = bf16(hidden + bf16((x @ w^T) * residual_multiplier)): the mixer's
        out-projection and the residual add (model.py:502-508) in one launch."""
        H = self.cfg.hidden
        self._lib.tfd_gemm_skinny_fp8_resid_scaled(ptr(x), ptr(w), ptr(scale), self.B, K, H,
                                                   ptr(self.hidden), H,
                                                   self.cfg.residual_multiplier,
                                                   ptr(self.hidden), H, s)

    def _mamba(self, i, w, s, cur):
        cfg = self.cfg
        a = _lib.TfdMambaArgs()
        cin, cout = self.conv[i][cur], self.conv[i][1 - cur]
        a.proj, a.proj_ld, a.conv_in, a.conv_out = ptr(self.proj), self.nproj, ptr(cin), ptr(cout)
        a.state = ptr(self.state[i])
        a.conv_w, a.conv_b = ptr(w["conv_w"]), ptr(w["conv_b"])
        a.a_log, a.dt_bias, a.d_skip = ptr(w["a_log"]), ptr(w["dt_bias"]), ptr(w["d_skip"])
        a.gamma, a.gated, a.ssq, a.out = ptr(w["gamma_ssm"]), ptr(self.gated), ptr(self.ssq), \
            ptr(self.mix)
        a.rows, a.heads, a.head_dim, a.state_dim = self.B, cfg.mamba_heads, cfg.mamba_head_dim, \
            cfg.d_state
        a.groups, a.conv_kernel, a.eps = 1, cfg.conv_kernel, cfg.eps
        self._lib.tfd_mamba_step(ctypes_addr(a), s)

    def _attn(self, i, s):
        cfg = self.cfg
        a = _lib.TfdGqaArgs()
        a.qkv, a.ldq = ptr(self.proj), self.nproj
        a.pos, a.page_table, a.max_pages = ptr(self.pos), ptr(self.page_table), self.max_pages
        a.k_pool, a.v_pool, a.num_pages = ptr(self.kpool[i]), ptr(self.vpool[i]), self.num_pages
        a.rows, a.heads, a.kv_heads, a.head_dim = self.B, cfg.heads, cfg.kv_heads, cfg.head_dim
        a.scale, a.eps = cfg.attention_multiplier, cfg.eps
        a.scores, a.score_stride, a.stats, a.part = ptr(self.scores), self.stride, \
            ptr(self.stats), ptr(self.part)
        a.counters, a.nsplit, a.split_len = ptr(self.counters), self.nsplit, self.split_len or 0
        a.out, a.policy, a.err = ptr(self.mix), _lib.POLICY_BF16, ptr(self.err)
        self._lib.tfd_gqa_decode(ctypes_addr(a), s)

    def _moe(self, w, s):
        cfg = self.cfg
        a = _lib.TfdMoeArgs()
        a.x, a.weights, a.idx = ptr(self.xm), ptr(self.rw), ptr(self.ridx)
        a.w_gate, a.w_up, a.w_down = ptr(w["w_gate"]), ptr(w["w_up"]), ptr(w["w_down"])
        a.s_gate, a.s_up, a.s_down = ptr(w["s_gate"]), ptr(w["s_up"]), ptr(w["s_down"])
        a.w_shared_in, a.w_shared_out = ptr(w["w_shared_in"]), ptr(w["w_shared_out"])
        a.s_shared_in, a.s_shared_out = ptr(w["w_shared_in_scale"]), ptr(w["w_shared_out_scale"])
        a.hidden, a.shared_scale = ptr(self.moe_hidden), ptr(self.moe_sscale)
        a.partial = None if self.moe_partial is None else ptr(self.moe_partial)
        # the experts' output goes straight into the residual stream, scaled
        a.groups, a.out = ptr(self.moe_groups), None
        a.resid, a.resid_mult = ptr(self.hidden), cfg.residual_multiplier
        a.rows, a.k, a.experts, a.hidden_size = self.B, cfg.top_k, cfg.experts, cfg.hidden
        a.inter, a.shared_inter, a.hidden_ld = cfg.moe_inter, cfg.shared_inter, self.moe_ld
        a.fp8, a.policy, a.err = 1, _lib.POLICY_BF16, ptr(self.err)
        a.logits, a.ldl, a.route = ptr(self.rlog), cfg.experts, _lib.MOE_ROUTE_TOPK_SOFTMAX
        if self.moe_packed:
            self._lib.tfd_moe_experts_packed(ctypes_addr(a), s)
        else:
            self._lib.tfd_moe_experts(ctypes_addr(a), s)

    def _layer(self, i, s, cur):
        cfg, L, w, B, H = self.cfg, self._lib, self.layers[i], self.B, self.cfg.hidden
        L.tfd_tf_rmsnorm_rows_bf16(ptr(self.hidden), H, ptr(w["gamma_in"]), None, 0,
                                   ptr(self.xn), B, H, cfg.eps, s)
        if cfg.is_attention(i):
            self._gemm8(self.xn, w["w_in"], w["w_in_scale"], H, cfg.attn_in, _lib.EPI_STORE,
                        self.proj, self.nproj, s)
            self._attn(i, s)
            self._gemm8_residual(self.mix, w["w_out"], w["w_out_scale"],
                                 cfg.heads * cfg.head_dim, s)
        else:
            self._gemm8(self.xn, w["w_in"], w["w_in_scale"], H, cfg.mamba_in, _lib.EPI_STORE,
                        self.proj, self.nproj, s)
            self._mamba(i, w, s, cur)
            self._gemm8_residual(self.mix, w["w_out"], w["w_out_scale"], cfg.d_inner, s)
        if self.router_norm:
            # the post norm as the router's prologue, which also writes the
            # experts' row-major input (one launch instead of two)
            a = _lib.TfdProj8NormArgs()
            a.x, a.ldx, a.gamma, a.eps = ptr(self.hidden), H, ptr(w["gamma_post"]), cfg.eps
            a.x_rows, a.ldxr = ptr(self.xm), H
            a.w, a.scale = ptr(w["w_router"]), ptr(w["w_router_scale"])
            a.rows, a.K, a.N = B, H, cfg.experts
            a.out, a.ldo, a.epilogue = ptr(self.rlog), cfg.experts, _lib.EPI_LOGITS
            L.tfd_proj8_norm(ctypes_addr(a), s)
        else:
            # post norm: row-major for the experts, operand order for the router
            L.tfd_tf_rmsnorm_rows_bf16(ptr(self.hidden), H, ptr(w["gamma_post"]), ptr(self.xm),
                                       H, ptr(self.xn), B, H, cfg.eps, s)
            self._gemm8(self.xn, w["w_router"], w["w_router_scale"], H, cfg.experts,
                        _lib.EPI_LOGITS, self.rlog, cfg.experts, s)
        self._moe(w, s)                    # routes inside the call, adds into the stream
        if self.routes is not None:
            self.routes[i].copy_(self.ridx)

    def _step(self, cur):
        s = self._stream()
        cfg, L, B, H, V = self.cfg, self._lib, self.B, self.cfg.hidden, self.cfg.vocab
        L.tfd_scaled_add_rows(None, 0, ptr(self.emb), H, 0, cfg.embedding_multiplier,
                              ptr(self.hidden), H, B, H, s)
        for i in range(cfg.layers):
            self._layer(i, s, cur)
        L.tfd_tf_rmsnorm_rows_bf16(ptr(self.hidden), H, ptr(self.gamma_final), None, 0,
                                   ptr(self.xn), B, H, cfg.eps, s)
        L.tfd_gemm_skinny_bf16_logits_div(ptr(self.xn), ptr(self.head), B, H, V,
                                          cfg.logits_scaling, ptr(self.logits), V,
                                          ptr(self.work), self.work.numel(), s)
        self.picker(self.logits, V, self.pick, self.pos, s)
        L.tfd_finalize_rows(ptr(self.pick), B, ptr(self.inp), self.nsteps, ptr(self.plen),
                            ptr(self.ids), ptr(self.pos), ptr(self.sam), self.nsteps,
                            self.nsteps, ptr(self.embed), ptr(self.emb), H, H, V, ptr(self.err),
                            s)

    def _capture(self):
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            self._load_prompts([[0]] * self.B)
            for cur in (0, 1):
                self._step(cur)
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        self.graphs = []
        for cur in (0, 1):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self._step(cur)
            self.graphs.append(g)
        torch.cuda.synchronize(self.device)
        self._reset()

    def replay(self):
        if self.graphs is not None:
            self.graphs[self._cur].replay()
        else:
            self._step(self._cur)
        self._cur ^= 1

    # ------------------------------------------------------------- generation
    def _reset(self):
        self.pos.zero_()
        self.sam.zero_()
        self.err.zero_()
        self.counters.zero_()
        for i in self.state:
            self.state[i].zero_()
            self.conv[i][0].zero_()
            self.conv[i][1].zero_()
        self._cur = 0

    def _load_prompts(self, prompts):
        self._reset()
        self.inp.zero_()
        self.plen.copy_(torch.tensor([len(p) for p in prompts], dtype=I32))
        for b, p in enumerate(prompts):
            self.inp[b, :len(p)] = torch.tensor(p, dtype=I32).to(self.device)
        self.ids.copy_(torch.tensor([p[0] for p in prompts], dtype=torch.int64))
        self._lib.tfd_embed_rows_bf16(ptr(self.embed), ptr(self.ids), ptr(self.emb),
                                      self.cfg.hidden, self.B, self.cfg.hidden, self.cfg.vocab,
                                      ptr(self.err), self._stream())

    def prefill(self, prompts: list[list[int]]):
        """Bring every sequence to its prompt's last token: the prompts (all of one
        length) are walked through the decode step, one position per step, so
        that the next step decodes each last prompt token.  The recurrent state
        of the mixers has no batched form here (each position's state is the
        previous one's update), so this is the walk ``generate`` makes, taken out
        of it."""
        if len(prompts) != self.B or any(len(p) < 1 for p in prompts):
            raise ValueError(f"need {self.B} non-empty prompts")
        if len({len(p) for p in prompts}) != 1:
            raise ValueError("prefill: the prompts must have one length (the walk moves "
                             "every sequence one position per step)")
        if len(prompts[0]) > self.nsteps:
            raise ValueError(f"prompt {len(prompts[0])} exceeds {self.nsteps} steps")
        self._load_prompts(prompts)
        for _ in range(len(prompts[0]) - 1):
            self.replay()

    def synthetic_context(self, ctx: int, seed: int = 0):
        """Stand in for a walked `ctx`-token context without walking it: every
        sequence's first `ctx` cache rows, conv windows and SSM states are drawn at
        random, and decoding continues at position `ctx` from a random token.  The
        work of every later step is that of a real `ctx`-token context."""
        if ctx + 1 > self.nsteps:
            raise ValueError(f"context {ctx} exceeds this engine's {self.nsteps} positions")
        self._reset()
        g = torch.Generator(device=self.device).manual_seed(seed)
        for i in self.kpool:
            self.kpool[i].copy_(torch.randn(self.kpool[i].shape, generator=g,
                                            device=self.device).to(BF))
            self.vpool[i].copy_(torch.randn(self.vpool[i].shape, generator=g,
                                            device=self.device).to(BF))
        for i in self.state:
            self.state[i].copy_(torch.randn(self.state[i].shape, generator=g,
                                            device=self.device) * 0.1)
            self.conv[i][0].copy_(torch.randn(self.conv[i][0].shape, generator=g,
                                              device=self.device).to(BF))
        self.pos.fill_(ctx)
        self.plen.fill_(1)
        ids = torch.randint(0, self.cfg.vocab, (self.B,), generator=g, device=self.device)
        self.ids.copy_(ids)
        self._lib.tfd_embed_rows_bf16(ptr(self.embed), ptr(self.ids), ptr(self.emb),
                                      self.cfg.hidden, self.B, self.cfg.hidden, self.cfg.vocab,
                                      ptr(self.err), self._stream())

    def check_errors(self):
        e = int(self.err.item())
        if e:
            raise RuntimeError(f"hybrid decode kernels raised error bits {e:#x}")

    def generate(self, prompts: list[list[int]], max_new: int, record_logits: bool = False):
        """Walk every prompt and continue for *max_new* tokens per sequence
        (greedy, or drawn as the engine's ``sampling`` says; the walk untimed)
        -> (tokens per sequence, seconds, logits per step)."""
        if len(prompts) != self.B or any(len(p) < 1 for p in prompts):
            raise ValueError(f"need {self.B} non-empty prompts")
        longest = max(len(p) for p in prompts)
        if longest + max_new > self.nsteps:
            raise ValueError(f"prompt {longest} + {max_new} exceeds {self.nsteps} steps")
        self._load_prompts(prompts)
        steps = longest - 1 + max_new
        hist = [] if record_logits else None
        rhist = [] if self.routes is not None else None
        torch.cuda.synchronize(self.device)
        for _ in range(longest - 1):
            self.replay()
            if hist is not None:
                hist.append(self.logits.clone())
            if rhist is not None:
                rhist.append(self.routes.clone())
        torch.cuda.synchronize(self.device)
        t0 = perf_counter()
        for _ in range(longest - 1, steps):
            self.replay()
            if hist is not None:
                hist.append(self.logits.clone())
            if rhist is not None:
                rhist.append(self.routes.clone())
        torch.cuda.synchronize(self.device)
        seconds = perf_counter() - t0
        self.check_errors()
        if rhist is not None:
            self.route_history = torch.stack(rhist).cpu()
        sam = self.sam.cpu()
        tokens = [sam[b, len(p) - 1: len(p) - 1 + max_new].tolist()
                  for b, p in enumerate(prompts)]
        return tokens, seconds, (torch.stack(hist).cpu() if hist is not None else None)

    # ------------------------------------------------------------ accounting
    def weight_bytes_per_step(self, experts_touched: float) -> float:
        """fp8 weights (1 byte each, 4 bytes per row scale) once, the experts picked
        (their union per layer) once, the bf16 head table once."""
        cfg, H = self.cfg, self.cfg.hidden

        def lin(n, k):
            return n * k + 4 * n

        total = 2 * cfg.vocab * H + 2 * H
        for i in range(cfg.layers):
            if cfg.is_attention(i):
                total += lin(cfg.attn_in, H) + lin(H, cfg.heads * cfg.head_dim)
            else:
                total += (lin(cfg.mamba_in, H) + lin(H, cfg.d_inner) +
                          2 * (cfg.conv_dim * (cfg.conv_kernel + 1) + 3 * cfg.mamba_heads +
                               cfg.d_inner))
            total += 2 * 2 * H + lin(cfg.experts, H)
            total += lin(2 * cfg.shared_inter, H) + lin(H, cfg.shared_inter)
            total += experts_touched * (2 * lin(cfg.moe_inter, H) + lin(H, cfg.moe_inter))
        return total

    def state_bytes_per_step(self, positions) -> float:
        cfg = self.cfg
        mamba = sum(1 for i in range(cfg.layers) if not cfg.is_attention(i))
        attn = cfg.layers - mamba
        per_row = mamba * (2 * 4 * cfg.mamba_heads * cfg.mamba_head_dim * cfg.d_state +
                           2 * 2 * cfg.conv_dim * (cfg.conv_kernel - 1))
        kv = sum(attn * 2 * 2 * cfg.kv_heads * cfg.head_dim * (p + 1) for p in positions)
        return self.B * per_row + kv
