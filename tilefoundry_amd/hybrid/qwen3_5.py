"""Qwen3.5-35B-A3B-style hybrid decode on the GPU (workload C4).

The decode step of ``examples/qwen3_5_35b_a3b-tilelang/runtime_model.py`` (its
``Qwen3_5Decoder`` over ``Qwen3_5LinearAttnLayer`` / ``Qwen3_5FullAttnLayer``),
with the arithmetic of the example's plain-torch twin
(``kernels/torch_ref.py:22-40``): the residual stream is f32, every matmul casts
its input to bf16 and rounds its f32 sum once.  Per layer:

* input norm (f32 in, one bf16 rounding, operand order) -> in-projection
  (skinny GEMM, f32 out) -> gated-DeltaNet step (``tfd_gdn_step``) or the
  full-attention step (``tfd_gqa_decode``) -> out-projection, whose epilogue
  adds it into the f32 residual stream;
* post norm -> router projection -> routed + shared experts
  (``tfd_moe_experts``: softmax/top-8 routing in its first launch, then
  expert-grouped), whose mix adds into the stream;

then the final norm, the head, the greedy pick and the next token's embedding
(``tfd_argmax_rows``, ``tfd_finalize_rows``).  Layer i is full attention when
i % 4 == 3 (3 GDN layers, then one GQA layer).  Sequences (up to 32) step
together, each with its own position, conv window, recurrent state and KV pages;
a step is recorded into a HIP graph (two, alternating, because the conv windows
ping-pong between two buffers) and replayed.

Weights are synthetic (random init on the device; there is no checkpoint here)
in the kernels' row layouts: every projection ``[out][in]`` (the reference's
``(in, out)`` transposed), packed once for the skinny GEMM; experts
``[E][I][H]`` / ``[E][H][I]``.
"""
from __future__ import annotations

from dataclasses import dataclass
from time import perf_counter

import torch

from .. import _lib
from .._lib import lib, ptr
from ..sampling import Picker, Sampling

BF = torch.bfloat16
F32 = torch.float32
I32 = torch.int32


@dataclass(frozen=True)
class Qwen35Config:
    """The published Qwen3.5-35B-A3B decoder shape."""

    hidden: int = 2048
    layers: int = 40
    full_every: int = 4
    lin_key_heads: int = 16
    lin_value_heads: int = 32
    lin_key_dim: int = 128
    lin_value_dim: int = 128
    conv_kernel: int = 4
    heads: int = 16
    kv_heads: int = 2
    head_dim: int = 256
    rot_dim: int = 64
    rope_theta: float = 1.0e7
    experts: int = 256
    top_k: int = 8
    moe_inter: int = 512
    shared_inter: int = 512
    vocab: int = 248320
    eps: float = 1e-6

    def is_full(self, i: int) -> bool:
        return i % self.full_every == self.full_every - 1

    @property
    def key_dim(self) -> int:
        return self.lin_key_heads * self.lin_key_dim

    @property
    def value_dim(self) -> int:
        return self.lin_value_heads * self.lin_value_dim

    @property
    def conv_dim(self) -> int:
        return 2 * self.key_dim + self.value_dim

    @property
    def gdn_in(self) -> int:
        """Rows of the GDN in-projection: conv channels (q|k|v), z, b, a."""
        return self.conv_dim + self.value_dim + 2 * self.lin_value_heads

    @property
    def attn_in(self) -> int:
        """Rows of the attention in-projection: q then gate per head, k, v."""
        return self.heads * 2 * self.head_dim + 2 * self.kv_heads * self.head_dim


def rope_tables(cfg: Qwen35Config, rows: int):
    """bf16 cos/sin [rows][rot] of rotate-half RoPE, ``cat(freqs, freqs)``
    (torch_ref.py:157-181)."""
    inv = 1.0 / cfg.rope_theta ** (torch.arange(0, cfg.rot_dim, 2, dtype=torch.float64) /
                                   cfg.rot_dim)
    f = torch.arange(rows, dtype=torch.float64)[:, None] * inv[None]
    emb = torch.cat((f, f), dim=-1)
    return emb.cos().to(BF), emb.sin().to(BF)


def synthetic_weights(cfg: Qwen35Config, seed: int = 0, device: str = "cuda:0",
                      std: float = 0.02) -> dict[str, torch.Tensor]:
    """Random-init weights in the kernels' layouts: matrices N(0, std) (router
    logits then come out near N(0, 1) at hidden 2048), norm scales 1 + N(0, std),
    a_log and dt_bias N(0, 0.5).  Drawn on `device` from a seeded generator."""
    g = torch.Generator(device=device).manual_seed(seed)

    def rn(*shape, s=std):
        return (torch.randn(*shape, generator=g, device=device) * s).to(BF)

    def gamma(n):
        return (1 + torch.randn(n, generator=g, device=device) * std).to(BF)

    H, E, I, IS = cfg.hidden, cfg.experts, cfg.moe_inter, cfg.shared_inter
    w = {"embed": rn(cfg.vocab, H), "gamma_final": gamma(H), "head": rn(cfg.vocab, H)}
    for i in range(cfg.layers):
        p = f"layer{i}."
        w[p + "gamma_in"] = gamma(H)
        if cfg.is_full(i):
            w[p + "w_in"] = rn(cfg.attn_in, H)
            w[p + "gamma_q"] = gamma(cfg.head_dim)
            w[p + "gamma_k"] = gamma(cfg.head_dim)
            w[p + "w_out"] = rn(H, cfg.heads * cfg.head_dim)
        else:
            w[p + "w_in"] = rn(cfg.gdn_in, H)
            w[p + "conv_w"] = rn(cfg.conv_dim, cfg.conv_kernel, s=0.5)
            w[p + "a_log"] = rn(cfg.lin_value_heads, s=0.5)
            w[p + "dt_bias"] = rn(cfg.lin_value_heads, s=0.5)
            w[p + "gamma_gdn"] = gamma(cfg.lin_value_dim)
            w[p + "w_out"] = rn(H, cfg.value_dim)
        w[p + "gamma_post"] = gamma(H)
        w[p + "w_router"] = rn(E, H)
        w[p + "w_gate"] = rn(E, I, H)
        w[p + "w_up"] = rn(E, I, H)
        w[p + "w_down"] = rn(E, H, I)
        w[p + "w_shared_in"] = rn(2 * IS, H)     # gate rows, then up rows
        w[p + "w_shared_out"] = rn(H, IS)
        w[p + "w_shared_scale"] = rn(H)
    return w


def declared_shapes(cfg: Qwen35Config) -> dict[str, tuple[int, ...]]:
    """Every weight the engine reads and its shape (all bf16, row layouts)."""
    H, E, I, IS = cfg.hidden, cfg.experts, cfg.moe_inter, cfg.shared_inter
    out = {"embed": (cfg.vocab, H), "gamma_final": (H,), "head": (cfg.vocab, H)}
    for i in range(cfg.layers):
        p = f"layer{i}."
        per = {"gamma_in": (H,), "gamma_post": (H,), "w_router": (E, H), "w_gate": (E, I, H),
               "w_up": (E, I, H), "w_down": (E, H, I), "w_shared_in": (2 * IS, H),
               "w_shared_out": (H, IS), "w_shared_scale": (H,)}
        if cfg.is_full(i):
            per.update(w_in=(cfg.attn_in, H), gamma_q=(cfg.head_dim,), gamma_k=(cfg.head_dim,),
                       w_out=(H, cfg.heads * cfg.head_dim))
        else:
            per.update(w_in=(cfg.gdn_in, H), conv_w=(cfg.conv_dim, cfg.conv_kernel),
                       a_log=(cfg.lin_value_heads,), dt_bias=(cfg.lin_value_heads,),
                       gamma_gdn=(cfg.lin_value_dim,), w_out=(H, cfg.value_dim))
        out.update({p + n: s for n, s in per.items()})
    return out


def validate(cfg: Qwen35Config, weights: dict[str, torch.Tensor]) -> None:
    """``KeyError`` for a missing weight, ``ValueError`` for a wrong shape or
    dtype -- the kernels take raw pointers and trust both."""
    for name, shape in declared_shapes(cfg).items():
        if name not in weights:
            raise KeyError(f"weight {name!r} is declared but not supplied")
        t = weights[name]
        if tuple(t.shape) != shape:
            raise ValueError(f"weight {name!r}: declared shape {shape}, got {tuple(t.shape)}")
        if t.dtype != BF:
            raise ValueError(f"weight {name!r}: declared dtype {BF}, got {t.dtype}")


class Qwen35Engine:
    """A Qwen3.5-style hybrid decoder stepping `rows` sequences together.

    ``weights`` is checked against ``declared_shapes(cfg)`` and copied to the
    device (contiguous) where it is not there already."""

    def __init__(self, cfg: Qwen35Config, weights: dict[str, torch.Tensor], *, rows: int,
                 device: str = "cuda:0", max_steps: int = 2112, page_seed: int = 0,
                 split_len: int | None = None, graph: bool = True, small: bool | None = None,
                 record_routes: bool = False,
                 sampling: Sampling | None = None):
        if not 1 <= rows <= 32:
            raise ValueError("rows: 1..32 sequences")
        self.cfg, self.B, self.device = cfg, rows, device
        self._lib = lib()
        self.sampling = sampling                # the token choice (None: greedy)
        # the small-batch path (rows <= 4): row GEMVs on row-major weights with
        # the norms as prologues, the delta rule over value columns, the
        # experts in two launches (tfd_rowgemv_bf16, tfd_gdn_step_cols,
        # tfd_moe_experts_small); otherwise MFMA GEMMs over packed weights
        self.small = rows <= _lib.SMALL_ROWS if small is None else bool(small)
        if self.small and rows > _lib.SMALL_ROWS:
            raise ValueError(f"small: rows <= {_lib.SMALL_ROWS}")
        self.nsteps = max_steps
        self.split_len = split_len
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

    # ----------------------------------------------------------------- set-up
    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def _packed(self, w: torch.Tensor) -> torch.Tensor:
        N, K = w.shape
        out = torch.empty(-(-N // 16) * 16 * K, dtype=BF, device=self.device)
        self._lib.tfd_pack_skinny_bf16(ptr(w), K, N, K, ptr(out), self._stream())
        return out

    def _pack(self, w):
        cfg = self.cfg
        validate(cfg, w)
        w = {n: w[n].to(self.device).contiguous() for n in declared_shapes(cfg)}
        self.layers = []
        for i in range(cfg.layers):
            p = f"layer{i}."
            d = {k[len(p):]: v for k, v in w.items() if k.startswith(p)}
            if not self.small:
                d["w_in"] = self._packed(d["w_in"])
                d["w_out"] = self._packed(d["w_out"])
                d["w_router"] = self._packed(d["w_router"])
            self.layers.append(d)
        self.embed = w["embed"]
        self.gamma_final = w["gamma_final"]
        self.head = w["head"] if self.small else self._packed(w["head"])
        torch.cuda.synchronize(self.device)

    def _buffers(self, page_seed):
        cfg, B, dev = self.cfg, self.B, self.device
        H, V, k = cfg.hidden, cfg.vocab, cfg.top_k

        def z(*shape, dtype=F32):
            return torch.zeros(*shape, dtype=dtype, device=dev)

        self.hidden = z(B, H)
        self.emb = z(B, H, dtype=BF)
        self.xn = z(32 * H, dtype=BF)                       # operand order
        self.xm = z(B, H, dtype=BF)                         # MoE input rows
        self.nproj = max(cfg.gdn_in, cfg.attn_in)
        self.proj = z(B, self.nproj)
        self.mix = z(32 * max(cfg.value_dim, cfg.heads * cfg.head_dim), dtype=BF)
        self.read = z(B, cfg.value_dim)                     # small path: GDN read-out
        self.rlog = z(B, cfg.experts)
        self.rw = z(B, k)
        self.ridx = z(B, k, dtype=I32)
        ld = max(cfg.moe_inter, cfg.shared_inter)
        self.moe_hidden = z(B, k + 1, ld, dtype=BF)
        self.moe_sscale = z(B)
        self.moe_partial = z(B, k + 1, H)
        self.moe_groups = z(_lib.moe_group_words(cfg.experts, B), dtype=I32)
        self.moe_ld = ld
        # GDN state and conv windows (two buffers each, ping-pong by step)
        self.state, self.conv = {}, {}
        for i in range(cfg.layers):
            if not cfg.is_full(i):
                self.state[i] = z(B, cfg.lin_value_heads, cfg.lin_key_dim, cfg.lin_value_dim)
                self.conv[i] = (z(B, cfg.conv_dim, cfg.conv_kernel - 1),
                                z(B, cfg.conv_dim, cfg.conv_kernel - 1))
        # paged KV of the full-attention layers
        self.max_pages = -(-self.nsteps // 16)
        self.num_pages = B * self.max_pages
        gen = torch.Generator().manual_seed(page_seed)
        self.page_table = torch.randperm(self.num_pages, generator=gen).view(
            B, self.max_pages).to(I32).to(dev)
        self.kpool, self.vpool = {}, {}
        for i in range(cfg.layers):
            if cfg.is_full(i):
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
        cos, sin = rope_tables(cfg, self.max_pages * 16)
        self.cos, self.sin = cos.to(dev), sin.to(dev)
        # head, pick, token feed
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
    def _gemm(self, x, w, K, N, out, ldo, s, resid=None):
        """out = bf16-valued f32 of x @ w^T, or resid + that (f32, in place)."""
        epi = _lib.EPI_LOGITS if resid is None else _lib.EPI_RESID_F32
        self._lib.tfd_gemm_skinny_bf16(ptr(x), ptr(w), self.B, K, N, epi,
                                       None if resid is None else ptr(resid),
                                       0 if resid is None else ldo, ptr(out), ldo,
                                       ptr(self.work), self.work.numel(), s)

    def _gdn(self, i, w, s, cur):
        a = self._gdn_args(i, w, cur)          # kept alive across the call
        self._lib.tfd_gdn_step(ctypes_addr(a), s)

    def _gdn_args(self, i, w, cur):
        cfg = self.cfg
        a = _lib.TfdGdnArgs()
        cin, cout = self.conv[i][cur], self.conv[i][1 - cur]
        a.proj, a.proj_ld, a.conv_in, a.conv_out = ptr(self.proj), self.nproj, ptr(cin), ptr(cout)
        a.state = ptr(self.state[i])
        a.conv_w, a.a_log, a.dt_bias = ptr(w["conv_w"]), ptr(w["a_log"]), ptr(w["dt_bias"])
        a.gamma, a.out = ptr(w["gamma_gdn"]), ptr(self.mix)
        a.rows, a.key_heads, a.value_heads = self.B, cfg.lin_key_heads, cfg.lin_value_heads
        a.head_k_dim, a.head_v_dim, a.conv_kernel = cfg.lin_key_dim, cfg.lin_value_dim, \
            cfg.conv_kernel
        a.l2_eps, a.rms_eps = 1e-6, cfg.eps
        return a

    def _attn(self, i, w, s):
        cfg = self.cfg
        a = _lib.TfdGqaArgs()
        a.qkv, a.ldq = ptr(self.proj), self.nproj
        a.gamma_q, a.gamma_k = ptr(w["gamma_q"]), ptr(w["gamma_k"])
        a.cos_table, a.sin_table = ptr(self.cos), ptr(self.sin)
        a.rope_rows, a.rot_dim = self.cos.shape[0], cfg.rot_dim
        a.pos, a.page_table, a.max_pages = ptr(self.pos), ptr(self.page_table), self.max_pages
        a.k_pool, a.v_pool, a.num_pages = ptr(self.kpool[i]), ptr(self.vpool[i]), self.num_pages
        a.rows, a.heads, a.kv_heads, a.head_dim = self.B, cfg.heads, cfg.kv_heads, cfg.head_dim
        a.scale, a.eps = cfg.head_dim ** -0.5, cfg.eps
        a.scores, a.score_stride, a.stats, a.part = ptr(self.scores), self.stride, \
            ptr(self.stats), ptr(self.part)
        a.counters, a.nsplit, a.split_len = ptr(self.counters), self.nsplit, self.split_len or 0
        a.out, a.policy, a.err = ptr(self.mix), _lib.POLICY_F32, ptr(self.err)
        self._lib.tfd_gqa_decode(ctypes_addr(a), s)

    def _moe(self, w, s):
        a = self._moe_args(w)                  # kept alive across the call
        self._lib.tfd_moe_experts(ctypes_addr(a), s)

    def _moe_args(self, w):
        cfg = self.cfg
        a = _lib.TfdMoeArgs()
        a.x, a.weights, a.idx = ptr(self.xm), ptr(self.rw), ptr(self.ridx)
        a.w_gate, a.w_up, a.w_down = ptr(w["w_gate"]), ptr(w["w_up"]), ptr(w["w_down"])
        a.w_shared_in, a.w_shared_out = ptr(w["w_shared_in"]), ptr(w["w_shared_out"])
        a.w_shared_scale = ptr(w["w_shared_scale"])
        a.hidden, a.shared_scale, a.partial = ptr(self.moe_hidden), ptr(self.moe_sscale), \
            ptr(self.moe_partial)
        a.groups, a.out = ptr(self.moe_groups), ptr(self.hidden)
        a.rows, a.k, a.experts, a.hidden_size = self.B, cfg.top_k, cfg.experts, cfg.hidden
        a.inter, a.shared_inter, a.hidden_ld = cfg.moe_inter, cfg.shared_inter, self.moe_ld
        a.fp8, a.policy, a.err = 0, _lib.POLICY_F32, ptr(self.err)
        a.accumulate = 1                               # residual add into the stream
        a.logits, a.ldl, a.route = ptr(self.rlog), cfg.experts, _lib.MOE_ROUTE_SOFTMAX_TOPK
        return a

    def _rowgemv(self, x, ldx, kind, w, K, N, out, ldo, s, *, gamma=None, gate=None, ldg=0,
                 resid=False, x_rows=None):
        a = _lib.TfdRowGemvArgs()
        a.x, a.ldx, a.x_kind = x, ldx, kind
        a.gamma = None if gamma is None else ptr(gamma)
        a.gate, a.ldg, a.head_dim, a.eps = gate, ldg, self.cfg.lin_value_dim, self.cfg.eps
        a.w, a.K, a.N = ptr(w), K, N
        a.out, a.ldo = ptr(out), ldo
        a.epilogue = _lib.EPI_RESID_F32 if resid else _lib.EPI_LOGITS
        a.x_rows, a.ldxr = (None, 0) if x_rows is None else (ptr(x_rows), x_rows.shape[-1])
        a.rows = self.B
        self._lib.tfd_rowgemv_bf16(ctypes_addr(a), s)

    def _layer_small(self, i, s, cur):
        cfg, w, H = self.cfg, self.layers[i], self.cfg.hidden
        full = cfg.is_full(i)
        self._rowgemv(ptr(self.hidden), H, _lib.ROWX_NORM_F32, w["w_in"], H,
                      cfg.attn_in if full else cfg.gdn_in, self.proj, self.nproj, s,
                      gamma=w["gamma_in"])
        if full:
            self._attn(i, w, s)
            self._rowgemv(ptr(self.mix), 0, _lib.ROWX_OPERAND, w["w_out"],
                          cfg.heads * cfg.head_dim, H, self.hidden, H, s, resid=True)
        else:
            a = self._gdn_args(i, w, cur)
            self._lib.tfd_gdn_step_cols(ctypes_addr(a), ptr(self.read), cfg.value_dim, s)
            self._rowgemv(ptr(self.read), cfg.value_dim, _lib.ROWX_GATED_F32, w["w_out"],
                          cfg.value_dim, H, self.hidden, H, s, gamma=w["gamma_gdn"],
                          gate=ptr(self.proj) + 4 * cfg.conv_dim, ldg=self.nproj, resid=True)
        self._rowgemv(ptr(self.hidden), H, _lib.ROWX_NORM_F32, w["w_router"], H, cfg.experts,
                      self.rlog, cfg.experts, s, gamma=w["gamma_post"], x_rows=self.xm)
        m = self._moe_args(w)                          # routes in its first launch
        self._lib.tfd_moe_experts_small(ctypes_addr(m), s)
        if self.routes is not None:
            self.routes[i].copy_(self.ridx)

    def _layer(self, i, s, cur):
        if self.small:
            self._layer_small(i, s, cur)
            return
        cfg, L, w, B, H = self.cfg, self._lib, self.layers[i], self.B, self.cfg.hidden
        L.tfd_rmsnorm_f32_rows(ptr(self.hidden), H, ptr(w["gamma_in"]), None, 0, ptr(self.xn),
                               B, H, cfg.eps, s)
        # the out-projection adds itself into the residual stream
        if cfg.is_full(i):
            self._gemm(self.xn, w["w_in"], H, cfg.attn_in, self.proj, self.nproj, s)
            self._attn(i, w, s)
            self._gemm(self.mix, w["w_out"], cfg.heads * cfg.head_dim, H, self.hidden, H, s,
                       resid=self.hidden)
        else:
            self._gemm(self.xn, w["w_in"], H, cfg.gdn_in, self.proj, self.nproj, s)
            self._gdn(i, w, s, cur)
            self._gemm(self.mix, w["w_out"], cfg.value_dim, H, self.hidden, H, s,
                       resid=self.hidden)
        L.tfd_rmsnorm_f32_rows(ptr(self.hidden), H, ptr(w["gamma_post"]), ptr(self.xm), H,
                               ptr(self.xn), B, H, cfg.eps, s)
        self._gemm(self.xn, w["w_router"], H, cfg.experts, self.rlog, cfg.experts, s)
        self._moe(w, s)                    # routes, then accumulates into the stream
        if self.routes is not None:
            self.routes[i].copy_(self.ridx)

    def _step(self, cur):
        s = self._stream()
        cfg, L, B, H, V = self.cfg, self._lib, self.B, self.cfg.hidden, self.cfg.vocab
        L.tfd_bf16_to_f32_rows(ptr(self.emb), H, ptr(self.hidden), H, B, H, s)
        for i in range(cfg.layers):
            self._layer(i, s, cur)
        if self.small:
            self._rowgemv(ptr(self.hidden), H, _lib.ROWX_NORM_F32, self.head, H, V, self.logits,
                          V, s, gamma=self.gamma_final)
        else:
            L.tfd_rmsnorm_f32_rows(ptr(self.hidden), H, ptr(self.gamma_final), None, 0,
                                   ptr(self.xn), B, H, cfg.eps, s)
            self._gemm(self.xn, self.head, H, V, self.logits, V, s)
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

    def check_errors(self):
        e = int(self.err.item())
        if e:
            raise RuntimeError(f"hybrid decode kernels raised error bits {e:#x}")

    def generate(self, prompts: list[list[int]], max_new: int, record_logits: bool = False):
        """Walk every prompt and continue for *max_new* tokens per sequence
        (greedy, or drawn as the engine's ``sampling`` says; the prompt walk is
        untimed).  -> (tokens per sequence, seconds of the timed steps, logits
        [steps][rows][V] when recorded)."""
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
        """Algorithmic weight bytes of one step: every dense weight once, the
        experts the step's sequences picked (their union per layer) once."""
        cfg = self.cfg
        H = cfg.hidden
        total = 2 * cfg.vocab * H + 2 * H                     # head, final gamma, + one embedding row
        for i in range(cfg.layers):
            if cfg.is_full(i):
                total += 2 * (cfg.attn_in * H + H * cfg.heads * cfg.head_dim + 2 * cfg.head_dim)
            else:
                total += 2 * (cfg.gdn_in * H + H * cfg.value_dim + cfg.conv_dim * cfg.conv_kernel
                              + 2 * cfg.lin_value_heads + cfg.lin_value_dim)
            total += 2 * (2 * H + cfg.experts * H + 3 * cfg.shared_inter * H + H)
            total += experts_touched * 2 * 3 * cfg.moe_inter * H
        return total

    def state_bytes_per_step(self, positions) -> float:
        """Recurrent state read and written, conv windows, KV read and written."""
        cfg = self.cfg
        gdn = sum(1 for i in range(cfg.layers) if not cfg.is_full(i))
        full = cfg.layers - gdn
        per_row = gdn * (2 * 4 * cfg.lin_value_heads * cfg.lin_key_dim * cfg.lin_value_dim +
                         2 * 4 * cfg.conv_dim * (cfg.conv_kernel - 1))
        kv = sum(full * 2 * 2 * cfg.kv_heads * cfg.head_dim * (p + 1) for p in positions)
        return self.B * per_row + kv


# The attention's grid is (splits, kv heads, rows): about two blocks per compute
# unit (256 on the MI355X) keeps every split long enough to stream its cache
# rows back to back.  Split lengths then follow each row's position (split_len
# 0 in tfd_gqa_decode), from 64 up to 512 positions.  One layer's two launches,
# measured: C5 (8 rows, 8 kv heads, 8,192 positions) 97.5 us at 512-position
# splits against 108.3 at 256 and 159.8 at 128; 16 Qwen3.5 rows (2 kv heads,
# 2,080 positions) 56.1 us at 128 against 75.7 at 64 and 68.4 at 256.
SPLIT_BLOCKS = 512
MAX_SPLIT_LEN = 512


def attention_splits(rows: int, kv_heads: int, cap: int) -> int:
    """Splits per (row, kv head) over a cache of *cap* positions, their lengths
    derived from each row's position."""
    least = -(-cap // MAX_SPLIT_LEN)                   # 512 positions at most
    return max(least, min(-(-cap // 64), -(-SPLIT_BLOCKS // (rows * kv_heads))))


def ctypes_addr(struct) -> int:
    import ctypes
    return ctypes.addressof(struct)
