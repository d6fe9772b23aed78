"""Batched decode: up to 32 sequences advance one token per step (workload C3).

The batch-1 engine's structure (``engine.py``; the reference's
``examples/qwen3_1_7b-tilelang/fast/engine.py:69-301``) with a batch axis:

* each sequence has its own position, prompt, picks and page-table row over one
  shared page pool per layer (``[B * pages][HKV][16][D]`` bf16, a seeded
  permutation so every sequence's pages are scattered through the pool);
* the projections are skinny GEMMs on the matrix cores
  (``tfd_gemm_skinny_bf16``: M = batch rows, 16x16x32 bf16 MFMA), the norms run
  row by row, and attention runs per (split, kv head, sequence);
* the whole step -- every layer, the head, the per-sequence pick and the next
  embeddings -- is recorded once into a HIP graph and replayed; the last kernel
  feeds each sequence its next prompt token while its prompt lasts and its pick
  after, so prompts of different lengths walk and continue without host round trips.
"""
from __future__ import annotations

from time import perf_counter

import torch

from .. import _lib
from .._lib import lib, ptr
from ..sampling import Picker, Sampling
from .config import Qwen3Config
from .engine import bf16_scale, scatter_cache
from .prefill import attention_splits
from .weights import head_rows, pack_layer, validate

MAX_BATCH = 32


def _round_up(n: int, m: int) -> int:
    return (n + m - 1) // m * m


class BatchGenerated:
    """Per-sequence continuations of one batched run and its timing."""

    def __init__(self, tokens, seconds, prefill_seconds, steps, logits=None):
        self.tokens: list[list[int]] = tokens
        self.seconds = seconds
        self.prefill_seconds = prefill_seconds
        self.steps = steps                    # timed steps (each advances every sequence)
        self.logits = logits                  # [steps, B, V] f32 when recorded

    @property
    def tokens_per_second(self) -> float:
        n = sum(len(t) for t in self.tokens)
        return n / self.seconds if self.seconds > 0 else float("inf")


class BatchEngine:
    """A loaded Qwen3 dense decoder stepping `batch` sequences together."""

    def __init__(self, cfg: Qwen3Config, weights: dict[str, torch.Tensor], *, batch: int,
                 device: str = "cuda:0", max_new: int = 256, prompt_room: int = 4096,
                 page_seed: int | None = 0, graph: bool = True, split_tiles: int | None = None,
                 splits: int | None = None, sampling: Sampling | None = None):
        """*split_tiles*: 64-position tiles per attention split (default: split
        lengths that follow each sequence's position, over *splits* splits per
        sequence and kv head, by default ``prefill.attention_splits``).
        *sampling*: the token choice (``tilefoundry_amd.sampling.Sampling``;
        None: greedy)."""
        if cfg.dtype != torch.bfloat16:
            raise ValueError(f"the HIP engine runs bf16 weights; config has {cfg.dtype}")
        if not 1 <= batch <= MAX_BATCH:
            raise ValueError(f"batch must lie in [1, {MAX_BATCH}], got {batch}")
        validate(cfg, weights)
        self.cfg, self.B = cfg, batch
        self.device = torch.device(device)
        self.L = cfg.num_hidden_layers
        self.H, self.V = cfg.hidden_size, cfg.vocab_size
        self.HQ, self.HKV, self.D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        self.I = cfg.intermediate_size
        self.QD = self.HQ * self.D
        self.qkv_n = cfg.qkv_size
        self.eps = float(cfg.rms_norm_eps)
        self.scale = bf16_scale(self.D)
        self.nsteps = max_new + prompt_room
        self.cap = _round_up(self.nsteps, _lib.ATTN_SPLIT)
        self.max_pages = self.cap // _lib.PAGE_SIZE
        tiles = self.cap // _lib.ATTN_SPLIT
        if split_tiles is None:
            if splits is not None and not 1 <= splits <= tiles:
                raise ValueError(f"splits must lie in [1, {tiles}], got {splits}")
            self.nsplit = splits or attention_splits(batch, self.HKV, self.cap)
            self.split_tiles = 0              # derived from each sequence's position
            self.score_stride = self.cap
        else:
            if split_tiles < 1 or splits is not None:
                raise ValueError(f"split_tiles must be positive and given without splits, "
                                 f"got {split_tiles} / {splits}")
            self.split_tiles = split_tiles
            self.nsplit = -(-tiles // self.split_tiles)
            self.score_stride = self.nsplit * self.split_tiles * _lib.ATTN_SPLIT
        if self.cap > cfg.max_position_embeddings:
            raise ValueError(f"capacity {self.cap} exceeds the rope table "
                             f"({cfg.max_position_embeddings} positions)")
        self._lib = lib()
        self.sampling = sampling
        self._pack(weights, page_seed)
        self._buffers()
        self.graph = None
        if graph:
            self._capture()

    # ---------------------------------------------------------------- setup
    def _pack(self, weights, page_seed):
        dev = self.device
        self.layers = []
        for i in range(self.L):
            layer = pack_layer(weights, i, dev)
            for n in ("w_qkv", "w_o", "w_gu", "w_down"):
                layer[n] = self._mfma_order(layer[n])
            self.layers.append(layer)
        self.w_embed, head = head_rows(weights, dev)
        self.w_head = self._mfma_order(head)
        self.gamma_final = weights["gamma_final"].to(dev).contiguous()
        d = self.D
        inv = 1.0 / (self.cfg.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
        ph = torch.outer(torch.arange(self.cap, dtype=torch.float32), inv)
        ph = torch.cat((ph, ph), dim=-1)
        self.cos = ph.cos().to(torch.bfloat16).to(dev).contiguous()
        self.sin = ph.sin().to(torch.bfloat16).to(dev).contiguous()
        self.num_pages = self.B * self.max_pages
        if page_seed is None:
            table = torch.arange(self.num_pages, dtype=torch.int32)
        else:
            g = torch.Generator().manual_seed(page_seed)
            table = torch.randperm(self.num_pages, generator=g).to(torch.int32)
        self.page_table = table.view(self.B, self.max_pages).to(dev).contiguous()

    def _mfma_order(self, w: torch.Tensor) -> torch.Tensor:
        """[N][K] row-major weights -> the skinny GEMM's 1 KiB operand blocks."""
        N, K = w.shape
        out = torch.empty(-(-N // 16) * 16, K, device=w.device, dtype=w.dtype)
        self._lib.tfd_pack_skinny_bf16(ptr(w), K, N, K, ptr(out),
                                       torch.cuda.current_stream(w.device).cuda_stream)
        torch.cuda.synchronize(w.device)
        return out

    def _buffers(self):
        dev, bf, f32, i32 = self.device, torch.bfloat16, torch.float32, torch.int32
        B = self.B

        def z(*shape, dtype=bf):
            return torch.zeros(*shape, device=dev, dtype=dtype)

        self.hid_rows = z(self.L + 1, B, self.H)      # [0]: the step's input embeddings
        self.hid = self.hid_rows[0]
        # GEMM inputs in operand order (32 rows x K, see tfd_rmsnorm_rows_bf16)
        self.xn = z(32 * self.H)
        self.qkv = z(B, self.qkv_n)
        self.attn = z(32 * self.QD)
        self.h1 = z(B, self.H)
        self.hmid = z(32 * self.I)
        self.kpool = z(self.L, self.num_pages, self.HKV, _lib.PAGE_SIZE, self.D)
        self.vpool = z(self.L, self.num_pages, self.HKV, _lib.PAGE_SIZE, self.D)
        self.scores = z(B, self.HQ, self.score_stride, dtype=f32)
        self.smax = z(B, self.nsplit, self.HQ, dtype=f32)
        self.snew = z(B, self.HQ, dtype=f32)
        self.psum = z(B, self.nsplit, self.HQ, dtype=f32)
        self.pout = z(B, self.nsplit, self.HQ, self.D, dtype=f32)
        self.counters = z(B, self.HKV, dtype=i32)
        self.logits = z(B, self.V, dtype=f32)
        self.pick = z(B, dtype=i32)
        self.picker = Picker(self.sampling, B, self.V, self.device)
        self.pos = z(B, dtype=i32)
        self.ids = z(B, dtype=torch.int64)
        self.inp = z(B, self.nsteps, dtype=i32)
        self.sam = z(B, self.nsteps, dtype=i32)
        self.plen = z(B, dtype=i32)
        self.err = z(1, dtype=i32)
        # skinny-GEMM work: tile counters (kept at zero by the library) and the
        # f32 partial tiles of GEMMs that split K; 8 MiB covers every projection
        self.work = z(1 << 21, dtype=f32)

    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    # ---------------------------------------------------------------- the step
    def _gemm(self, x, w, K, N, epi, resid, out, ldo, s):
        """out = epi(x @ w^T) for the batch's rows (model.py:160-171 and friends)."""
        self._lib.tfd_gemm_skinny_bf16(ptr(x), ptr(w), self.B, K, N, epi,
                                       None if resid is None else ptr(resid),
                                       0 if resid is None else resid.shape[-1], ptr(out), ldo,
                                       ptr(self.work), self.work.numel(), s)

    def _layer(self, i: int, s: int):
        """One decoder layer (model.py:236-266) for every sequence."""
        L, w = self._lib, self.layers[i]
        B, H, I, D = self.B, self.H, self.I, self.D
        x_in, x_out = self.hid_rows[i], self.hid_rows[i + 1]
        L.tfd_rmsnorm_rows_bf16(ptr(x_in), H, ptr(w["gamma_in"]), ptr(self.xn), 0, B, H,
                                self.eps, 1, s)
        self._gemm(self.xn, w["w_qkv"], H, self.qkv_n, _lib.EPI_STORE, None, self.qkv,
                   self.qkv_n, s)
        L.tfd_attn_rope_scores_paged_batched(
            ptr(self.qkv), self.qkv_n, ptr(w["gamma_q"]), ptr(w["gamma_k"]), ptr(self.cos),
            ptr(self.sin), self.cap, ptr(self.pos), ptr(self.page_table), self.max_pages,
            ptr(self.kpool[i]), ptr(self.vpool[i]), self.num_pages, B, self.HQ, self.HKV, D,
            self.scale, self.eps, ptr(self.scores), self.score_stride, ptr(self.smax),
            ptr(self.snew), self.nsplit, self.split_tiles, ptr(self.err), s)
        L.tfd_attn_pv_combine_paged_batched(
            ptr(self.qkv), self.qkv_n, ptr(self.pos), ptr(self.page_table), self.max_pages,
            ptr(self.vpool[i]), self.num_pages, B, self.HQ, self.HKV, D, ptr(self.scores),
            self.score_stride, ptr(self.smax), ptr(self.snew), ptr(self.psum), ptr(self.pout),
            self.nsplit, self.split_tiles, ptr(self.counters), ptr(self.attn),
            ptr(self.err), s)
        self._gemm(self.attn, w["w_o"], self.QD, H, _lib.EPI_RESID, x_in, self.h1, H,
                   s)
        L.tfd_rmsnorm_rows_bf16(ptr(self.h1), H, ptr(w["gamma_post"]), ptr(self.xn), 0, B, H,
                                self.eps, 1, s)
        self._gemm(self.xn, w["w_gu"], H, 2 * I, _lib.EPI_SWIGLU, None, self.hmid, 0, s)
        self._gemm(self.hmid, w["w_down"], I, H, _lib.EPI_RESID, self.h1, x_out, H, s)

    def _step(self):
        s = self._stream()
        for i in range(self.L):
            self._layer(i, s)
        L, B, H = self._lib, self.B, self.H
        L.tfd_rmsnorm_rows_bf16(ptr(self.hid_rows[self.L]), H, ptr(self.gamma_final),
                                ptr(self.xn), 0, B, H, self.eps, 1, s)
        self._gemm(self.xn, self.w_head, H, self.V, _lib.EPI_LOGITS, None, self.logits,
                   self.V, s)
        self.picker(self.logits, self.V, self.pick, self.pos, s)
        L.tfd_finalize_rows(ptr(self.pick), B, ptr(self.inp), self.nsteps, ptr(self.plen),
                            ptr(self.ids), ptr(self.pos), ptr(self.sam), self.nsteps,
                            self.nsteps, ptr(self.w_embed), ptr(self.hid), H, H, self.V,
                            ptr(self.err), s)

    def _capture(self):
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            self._load_prompts([[0]] * self.B)
            for _ in range(3):
                self._step()
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._step()
        torch.cuda.synchronize(self.device)
        self._reset()

    def replay(self):
        if self.graph is not None:
            self.graph.replay()
        else:
            self._step()

    def run_steps(self, n: int):
        for _ in range(n):
            self.replay()

    # ------------------------------------------------------------- generation
    def _reset(self):
        self.pos.zero_()
        self.sam.zero_()
        self.err.zero_()

    def _load_prompts(self, prompts: list[list[int]]):
        self._reset()
        self.inp.zero_()
        lens = []
        for b, p in enumerate(prompts):
            self.inp[b, :len(p)] = torch.tensor(p, dtype=torch.int32).to(self.device)
            lens.append(len(p))
        self.plen.copy_(torch.tensor(lens, dtype=torch.int32))
        self.ids.copy_(torch.tensor([p[0] for p in prompts], dtype=torch.int64))
        self._lib.tfd_embed_rows_bf16(ptr(self.w_embed), ptr(self.ids), ptr(self.hid), self.H,
                                      self.B, self.H, self.V, ptr(self.err), self._stream())

    def place_context(self, k_caches, v_caches, tokens: list[int]):
        """Stand in for walked contexts without walking them: sequence b's cache
        rows 0 .. P_b - 1 of layer i become ``k_caches[i][b]`` /
        ``v_caches[i][b]`` ([P_b][HKV][D] bf16, through its page-table row), and
        the next step decodes ``tokens[b]`` at position P_b (the oracle's
        ``forward`` with the same caches, model.py:307-317)."""
        if len(tokens) != self.B or len(k_caches) != self.L or len(v_caches) != self.L:
            raise ValueError(f"place_context: {self.B} sequences x {self.L} layers of caches")
        lens = [int(c.shape[0]) for c in k_caches[0]]
        if max(lens) + 1 > self.nsteps:
            raise ValueError(f"place_context: a position past this engine's {self.nsteps}")
        if any(not 0 <= int(t) < self.V for t in tokens):
            raise ValueError(f"place_context: token ids must lie in [0, {self.V})")
        self._reset()
        self.inp.zero_()
        for b, (P, t) in enumerate(zip(lens, tokens)):
            self.inp[b, P] = int(t)
        self.plen.copy_(torch.tensor([P + 1 for P in lens], dtype=torch.int32))
        self.pos.copy_(torch.tensor(lens, dtype=torch.int32))
        self.ids.copy_(torch.tensor([int(t) for t in tokens], dtype=torch.int64))
        for b in range(self.B):
            scatter_cache(self.kpool, self.vpool, self.page_table[b],
                          [k_caches[i][b] for i in range(self.L)],
                          [v_caches[i][b] for i in range(self.L)])
        self._lib.tfd_embed_rows_bf16(ptr(self.w_embed), ptr(self.ids), ptr(self.hid), self.H,
                                      self.B, self.H, self.V, ptr(self.err), self._stream())

    def prefill(self, prompts: list[list[int]]):
        """Fill sequence b's cache at positions 0 .. len(prompts[b]) - 2 in batched
        passes (``qwen3.prefill``, through b's page-table row), so that the next
        step decodes every prompt's last token at its own position."""
        if len(prompts) != self.B or any(len(p) < 1 for p in prompts):
            raise ValueError(f"need {self.B} non-empty prompts")
        if getattr(self, "_prefiller", None) is None:
            from .prefill import Prefill
            self._prefiller = Prefill(self, packed=True)
        self._load_prompts(prompts)
        for b, p in enumerate(prompts):
            if len(p) > 1:
                self._prefiller.run(list(p[:-1]), 0, seq=b)
        self.pos.copy_(torch.tensor([len(p) - 1 for p in prompts], dtype=torch.int32))
        self.ids.copy_(torch.tensor([p[-1] for p in prompts], dtype=torch.int64))
        self._lib.tfd_embed_rows_bf16(ptr(self.w_embed), ptr(self.ids), ptr(self.hid), self.H,
                                      self.B, self.H, self.V, ptr(self.err), self._stream())

    def check_errors(self):
        e = int(self.err.item())
        if e:
            names = [n for bit, n in ((1, "token id"), (2, "position"), (4, "page-table entry"),
                                      (8, "step")) if e & bit]
            raise RuntimeError(f"decode kernels flagged an out-of-range {', '.join(names)}")

    def generate(self, prompts: list[list[int]], max_new: int, record_logits: bool = False,
                 prefill: bool = False) -> BatchGenerated:
        """Walk every prompt, then continue for *max_new* tokens per sequence
        (greedy, or drawn as the engine's ``sampling`` says).  Sequence b's
        continuation starts after its own prompt; all sequences step together,
        so the step count is max(prompt) - 1 + max_new,
        and the timing covers the steps after the longest prompt.  With
        *prefill*, every prompt but its last token goes through ``prefill`` and
        all sequences decode their last prompt token in the first step: max_new
        steps, all timed."""
        if len(prompts) != self.B:
            raise ValueError(f"engine holds {self.B} sequences, got {len(prompts)} prompts")
        if any(len(p) < 1 for p in prompts):
            raise ValueError("every sequence needs a prompt of at least one token")
        longest = max(len(p) for p in prompts)
        if longest + max_new > self.nsteps:
            raise ValueError(f"prompt {longest} + {max_new} new exceeds this engine's "
                             f"{self.nsteps} steps")
        if any(not 0 <= int(t) < self.V for p in prompts for t in p):
            raise ValueError(f"prompt ids must lie in [0, {self.V})")
        torch.cuda.synchronize(self.device)
        t_pre = perf_counter()
        if prefill:
            self.prefill(prompts)
            starts = [0] * self.B                      # step of each sequence's first pick
        else:
            self._load_prompts(prompts)
            starts = [len(p) - 1 for p in prompts]
        torch.cuda.synchronize(self.device)
        t_pre = perf_counter() - t_pre
        steps = max(starts) + max_new
        warm = max(starts)
        hist = (torch.empty(steps, self.B, self.V, device=self.device, dtype=torch.float32)
                if record_logits else None)
        torch.cuda.synchronize(self.device)
        t0 = perf_counter()
        for k in range(warm):
            self.replay()
            if hist is not None:
                hist[k].copy_(self.logits)
        torch.cuda.synchronize(self.device)
        t1 = perf_counter()
        for k in range(warm, steps):
            self.replay()
            if hist is not None:
                hist[k].copy_(self.logits)
        torch.cuda.synchronize(self.device)
        t2 = perf_counter()
        self.check_errors()
        sam = self.sam.cpu()
        tokens = [sam[b, len(p) - 1: len(p) - 1 + max_new].tolist()
                  for b, p in enumerate(prompts)]
        logits = None
        if hist is not None:
            h = hist.cpu()
            # logits at each sequence's own picks: step starts[b] + j
            logits = [h[st: st + max_new, b] for b, st in enumerate(starts)]
        return BatchGenerated(tokens, t2 - t1, t1 - t0 + t_pre, max_new, logits)

    # ------------------------------------------------------------ accounting
    def weight_bytes_per_step(self) -> int:
        return self.cfg.weight_bytes_per_step()

    def kv_bytes_at(self, positions) -> int:
        """KV bytes one step touches with sequences at *positions*."""
        return sum(self.cfg.kv_bytes_per_position() * (p + 1) for p in positions)
