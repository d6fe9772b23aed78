"""One captured batch-1 decode step over a paged KV cache, replayed per token.

The same shape as the reference's fast engine
(``examples/qwen3_1_7b-tilelang/fast/engine.py:69-301``): a fixed-capacity cache
whose write position advances, the position in a one-element device tensor, and
the whole step -- every layer, the head, the greedy pick and the next token's
embedding -- recorded once into a HIP graph (``torch.cuda.graph``) and replayed.
The last kernel writes the pick back as the next input, or the next prompt
token while the prompt lasts, so walking the prompt and continuing past it need
no host round trip.

What differs, MI355X-first:

* the KV cache is paged: per layer a pool ``[pages][HKV][16][D]`` bf16 and a
  device page table; a position's row is ``table[p // 16] * 16 + p % 16``;
* six kernels per layer instead of eight, the norms folded into the
  projections that consume them (see ``csrc/qwen3_decode.hip``);
* every kernel is hand-written HIP for gfx950 reached through the C ABI in
  ``include/tf_decode.h``; there is no torch compute on the step.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from time import perf_counter

import torch

from .. import _lib
from .._lib import lib, ptr
from .config import Qwen3Config
from .weights import head_rows, pack_layer, validate


@dataclass(frozen=True)
class Generated:
    """A continuation and the timing of the part that produced it (engine.py:55-66)."""

    tokens: list[int]
    seconds: float
    prefill_seconds: float
    prompt_steps: int
    logits: torch.Tensor | None = None   # [len(tokens), V] f32, when recorded

    @property
    def tokens_per_second(self) -> float:
        return len(self.tokens) / self.seconds if self.seconds > 0 else float("inf")


def scatter_cache(kpool, vpool, page_table, k_caches, v_caches):
    """Write contiguous caches into paged pools: position p of a sequence is row
    p % 16 of page ``page_table[p // 16]`` (per layer i, pools [L][pages][HKV]
    [16][D], caches [P][HKV][D])."""
    for i, (kc, vc) in enumerate(zip(k_caches, v_caches)):
        P = int(kc.shape[0])
        if P == 0:
            continue
        pos = torch.arange(P, device=kpool.device)
        pages = page_table[pos // _lib.PAGE_SIZE].long()
        rows = pos % _lib.PAGE_SIZE
        kpool[i][pages, :, rows] = kc.to(kpool.device, kpool.dtype)
        vpool[i][pages, :, rows] = vc.to(vpool.device, vpool.dtype)


def _round_up(n: int, m: int) -> int:
    return (n + m - 1) // m * m


def bf16_scale(head_dim: int) -> float:
    """``head_dim ** -0.5`` as the bf16 value the reference feeds (model.py:384-386)."""
    return torch.tensor(head_dim ** -0.5, dtype=torch.bfloat16).item()


class Engine:
    """A loaded Qwen3 dense decoder and one captured decode step over it."""

    def __init__(self, cfg: Qwen3Config, weights: dict[str, torch.Tensor], *,
                 device: str = "cuda:0", max_new: int = 2048, prompt_room: int = 512,
                 page_seed: int | None = 0, graph: bool = True,
                 lm_head_blocks: int = 2048, mode: str | None = None):
        """*mode*: ``"persistent"`` runs whole steps in one cooperative launch
        (``tfd_decode_persistent``); ``"xcd"`` does the same with each layer split
        over the device's 8 XCDs (``tfd_decode_xcd``: the Qwen3-1.7B shape on a
        256-CU device); ``"graph"`` replays a captured graph of the
        per-phase launches; ``"direct"`` issues those launches each step.  The
        default is ``"graph"`` (``"direct"`` when *graph* is False)."""
        if cfg.dtype != torch.bfloat16:
            raise ValueError(f"the HIP engine runs bf16 weights; config has {cfg.dtype}")
        validate(cfg, weights)
        self.cfg = cfg
        self.device = torch.device(device)
        self.L = cfg.num_hidden_layers
        self.H, self.V = cfg.hidden_size, cfg.vocab_size
        self.HQ, self.HKV, self.D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        self.I = cfg.intermediate_size
        self.eps = float(cfg.rms_norm_eps)
        self.scale = bf16_scale(self.D)

        self.nsteps = max_new + prompt_room
        self.cap = _round_up(self.nsteps, _lib.ATTN_SPLIT)
        self.max_pages = self.cap // _lib.PAGE_SIZE
        self.nsplit = self.cap // _lib.ATTN_SPLIT
        if self.cap > cfg.max_position_embeddings:
            raise ValueError(f"capacity {self.cap} exceeds the rope table "
                             f"({cfg.max_position_embeddings} positions)")
        self.nb = lm_head_blocks
        self.mode = mode or ("graph" if graph else "direct")
        if self.mode not in ("persistent", "xcd", "graph", "direct"):
            raise ValueError(f"mode {self.mode!r}")
        self._lib = lib()
        self._pack(weights, page_seed)
        self._buffers()
        self.graph = None
        if self.mode in ("persistent", "xcd"):
            self._persistent_args()
        if self.mode == "xcd":
            self._xcd_args()
        elif self.mode == "graph":
            self._capture()

    # ---------------------------------------------------------------- weights
    def _pack(self, weights, page_seed):
        dev = self.device
        self.layers = [pack_layer(weights, i, dev) for i in range(self.L)]
        self.w_embed, self.w_head = head_rows(weights, dev)
        self.gamma_final = weights["gamma_final"].to(dev).contiguous()
        # the rope tables exactly as _generation_rope builds them (model.py:107-120)
        d = self.D
        inv = 1.0 / (self.cfg.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
        ph = torch.outer(torch.arange(self.cap, dtype=torch.float32), inv)
        ph = torch.cat((ph, ph), dim=-1)
        self.cos = ph.cos().to(torch.bfloat16).to(dev).contiguous()
        self.sin = ph.sin().to(torch.bfloat16).to(dev).contiguous()
        # a page table: a seeded permutation of the pool, so every read goes
        # through the indirection (page_seed=None keeps pages in order)
        if page_seed is None:
            table = torch.arange(self.max_pages, dtype=torch.int32)
        else:
            g = torch.Generator().manual_seed(page_seed)
            table = torch.randperm(self.max_pages, generator=g).to(torch.int32)
        self.page_table = table.to(dev)

    # ---------------------------------------------------------------- buffers
    def _buffers(self):
        dev, bf, f32, i32 = self.device, torch.bfloat16, torch.float32, torch.int32

        def z(*shape, dtype=bf):
            return torch.zeros(*shape, device=dev, dtype=dtype)

        # one activation row per layer: every address is written once per step
        # (the persistent kernel reads them through the caches)
        self.hid_rows = z(self.L + 1, self.H)     # row 0: the step's input embedding
        self.hid = self.hid_rows[0]
        self.h1_rows = z(self.L, self.H)
        self.qkv_rows = z(self.L, self.cfg.qkv_size)
        self.attn_rows = z(self.L, self.HQ * self.D)
        self.hmid_rows = z(self.L, self.I)
        self.kpool = z(self.L, self.max_pages, self.HKV, _lib.PAGE_SIZE, self.D)
        self.vpool = z(self.L, self.max_pages, self.HKV, _lib.PAGE_SIZE, self.D)
        self.scores = z(self.HQ, self.cap, dtype=f32)
        self.smax = z(self.nsplit, self.HQ, dtype=f32)
        self.snew = z(self.HQ, dtype=f32)
        self.psum = z(self.nsplit, self.HQ, dtype=f32)
        self.pout = z(self.nsplit, self.HQ, self.D, dtype=f32)
        self.counters = z(self.HKV, dtype=i32)
        self.logits = z(self.V, dtype=f32)
        self.grid = int(self._lib.tfd_decode_persistent_grid())
        self.bv = z(max(self.nb, self.grid), dtype=f32)
        self.bi = z(max(self.nb, self.grid), dtype=i32)
        self.pos = z(1, dtype=i32)
        self.ids = z(1, dtype=torch.int64)
        self.inp = z(self.nsteps, dtype=i32)
        self.sam = z(self.nsteps, dtype=i32)
        self.plen = z(1, dtype=i32)
        self.err = z(1, dtype=i32)

    # ---------------------------------------------------------------- the step
    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def _layer(self, i: int, s: int):
        """One decoder layer (model.py:236-266) as six launches."""
        L, w = self._lib, self.layers[i]
        H, I, D = self.H, self.I, self.D
        kp, vp = self.kpool[i], self.vpool[i]
        x_in, x_out = self.hid_rows[i], self.hid_rows[i + 1]
        h1, qkv, attn, hmid = self.h1_rows[i], self.qkv_rows[i], self.attn_rows[i], self.hmid_rows[i]
        L.tfd_gemv_bf16(ptr(x_in), ptr(w["gamma_in"]), ptr(w["w_qkv"]), None, ptr(qkv),
                        H, self.cfg.qkv_size, _lib.PRO_NORM, _lib.EPI_STORE, self.eps, s)
        L.tfd_attn_rope_scores_paged(
            ptr(qkv), ptr(w["gamma_q"]), ptr(w["gamma_k"]), ptr(self.cos), ptr(self.sin),
            self.cap, ptr(self.pos), ptr(self.pos), ptr(self.page_table), self.max_pages,
            ptr(kp), ptr(vp), self.max_pages, self.HQ, self.HKV, D, self.scale, self.eps,
            ptr(self.scores), self.cap, ptr(self.smax), ptr(self.snew), self.nsplit,
            ptr(self.err), s)
        L.tfd_attn_pv_combine_paged(
            ptr(qkv), ptr(self.pos), ptr(self.page_table), self.max_pages, ptr(vp),
            self.max_pages, self.HQ, self.HKV, D, ptr(self.scores), self.cap, ptr(self.smax),
            ptr(self.snew), ptr(self.psum), ptr(self.pout), self.nsplit, ptr(self.counters),
            ptr(attn), ptr(self.err), s)
        L.tfd_gemv_bf16(ptr(attn), None, ptr(w["w_o"]), ptr(x_in), ptr(h1),
                        self.HQ * D, H, _lib.PRO_PLAIN, _lib.EPI_RESID, self.eps, s)
        L.tfd_gemv_bf16(ptr(h1), ptr(w["gamma_post"]), ptr(w["w_gu"]), None, ptr(hmid),
                        H, 2 * I, _lib.PRO_NORM, _lib.EPI_SWIGLU, self.eps, s)
        L.tfd_gemv_bf16(ptr(hmid), None, ptr(w["w_down"]), ptr(h1), ptr(x_out),
                        I, H, _lib.PRO_PLAIN, _lib.EPI_RESID, self.eps, s)

    def _step(self, record: list | None = None):
        """One decode step: every layer, then head + pick + next embedding."""
        s = self._stream()
        if record is not None:
            record.append(self.hid.clone())
        for i in range(self.L):
            self._layer(i, s)
            if record is not None:
                record.append(self.hid_rows[i + 1].clone())
        self._lib.tfd_lm_head_argmax_bf16(ptr(self.hid_rows[self.L]), ptr(self.gamma_final),
                                          ptr(self.w_head),
                                          ptr(self.logits), ptr(self.bv), ptr(self.bi), self.H,
                                          self.V, self.nb, self.eps, s)
        self._lib.tfd_argmax_finalize(ptr(self.bv), ptr(self.bi), self.nb, ptr(self.inp),
                                      ptr(self.plen), ptr(self.ids), ptr(self.pos),
                                      ptr(self.sam), self.nsteps, ptr(self.w_embed),
                                      ptr(self.hid), self.H, self.V, ptr(self.err), s)

    def _embed_current(self):
        self._lib.tfd_embed_bf16(ptr(self.w_embed), ptr(self.ids), ptr(self.hid), self.H, self.V,
                                 ptr(self.err), self._stream())

    def _capture(self):
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            self._load_prompt([0])
            for _ in range(3):
                self._step()
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._step()
        torch.cuda.synchronize(self.device)
        self._reset()

    def _persistent_args(self):
        """The layer table (device), the flag-in-data exchange buffers and the
        argument block of the persistent kernel."""
        layers = (_lib.TfdLayer * self.L)()
        for i, w in enumerate(self.layers):
            layers[i] = _lib.TfdLayer(
                ptr(w["w_qkv"]), ptr(w["w_o"]), ptr(w["w_gu"]), ptr(w["w_down"]),
                ptr(w["gamma_in"]), ptr(w["gamma_post"]), ptr(w["gamma_q"]), ptr(w["gamma_k"]),
                ptr(self.kpool[i]), ptr(self.vpool[i]))
        raw = torch.frombuffer(bytearray(bytes(layers)), dtype=torch.uint8)
        self.layer_table = raw.to(self.device)
        # exchange buffers: one 8-byte word per bf16 pair or f32 (payload, tag)
        words = {"x_hid": self.H // 2, "x_h1": self.H // 2, "x_qkv": self.cfg.qkv_size // 2,
                 "x_attn": self.HQ * self.D // 2, "x_mid": self.I // 2,
                 "x_smax": self.nsplit * self.HQ, "x_psum": self.nsplit * self.HQ,
                 "x_pout": self.nsplit * self.HQ * self.D, "x_best": 2 * self.grid}
        self.xbuf = {k: torch.zeros(2 * n, device=self.device, dtype=torch.int32)
                     for k, n in words.items()}
        self.epoch = 0
        self.args = _lib.TfdDecodeArgs(
            layers=ptr(self.layer_table), n_layers=self.L, hidden=self.H, heads=self.HQ,
            kv_heads=self.HKV, head_dim=self.D, intermediate=self.I, vocab=self.V,
            eps=self.eps, scale=self.scale, w_embed=ptr(self.w_embed), w_head=ptr(self.w_head),
            gamma_final=ptr(self.gamma_final), cos_table=ptr(self.cos), sin_table=ptr(self.sin),
            rope_rows=self.cap, page_table=ptr(self.page_table), max_pages=self.max_pages,
            num_pages=self.max_pages, **{k: ptr(t) for k, t in self.xbuf.items()}, epoch=0,
            scores=ptr(self.scores), score_stride=self.cap, score_new=ptr(self.snew),
            nsplit=self.nsplit, logits=ptr(self.logits), ids=ptr(self.ids), pos=ptr(self.pos),
            inp=ptr(self.inp), prompt_len=ptr(self.plen), sam=ptr(self.sam), nsteps=self.nsteps,
            err=ptr(self.err))

    def _xcd_args(self):
        """The per-XCD exchange arenas of ``tfd_decode_xcd`` (TfdXcdArgs)."""
        X, H = _lib.XCDS, self.H
        words = {"hid": X * H // 2, "h1": X * H // 2, "opart": X * H, "dpart": X * H,
                 "smax": X * self.nsplit * self.HQ, "psum": X * self.nsplit * self.HQ,
                 "pout": X * self.nsplit * self.HQ * self.D}
        self.xcd_buf = {k: torch.zeros(2 * n, device=self.device, dtype=torch.int32)
                        for k, n in words.items()}
        self.xcd_args = _lib.TfdXcdArgs(**{k: ptr(t) for k, t in self.xcd_buf.items()})

    def _launch_persistent(self, n: int):
        """One launch of *n* steps; advances the exchange-buffer epoch past them."""
        tags = n * _lib.tags_per_step(self.L)
        if self.epoch + tags >= 0xFFFFFFFF:
            for t in self.xbuf.values():
                t.zero_()
            for t in getattr(self, "xcd_buf", {}).values():
                t.zero_()
            self.epoch = 0
        self.args.epoch = self.epoch
        if self.mode == "xcd":
            self._lib.tfd_decode_xcd(ctypes.byref(self.args), ctypes.byref(self.xcd_args), n,
                                     self._stream())
        else:
            self._lib.tfd_decode_persistent(ctypes.byref(self.args), n, 0, self._stream())
        self.epoch += tags

    def phase_timeline(self, prompt_ids: list[int], steps: int) -> torch.Tensor:
        """Device clock stamps of *steps* persistent steps after walking
        *prompt_ids*: ``[steps, blocks, 7 * layers + 2, 2]`` microseconds since
        block 0 began the first step -- per layer the qkv, attention scores, P.V
        and merge, o, gate/up and down phases, then the head and the pick; for
        each, when the block had its input and when its output was out."""
        if self.mode not in ("persistent", "xcd"):
            raise ValueError("the phase timeline belongs to the persistent kernels")
        n = _lib.timeline_stamps(self.L)
        buf = torch.zeros(steps * self.grid * n, device=self.device, dtype=torch.int64)
        self._load_prompt(prompt_ids)
        self.run_steps(len(prompt_ids) - 1)
        torch.cuda.synchronize(self.device)
        self.args.timeline, self.args.timeline_steps = ptr(buf), steps
        try:
            self.run_steps(steps)
            torch.cuda.synchronize(self.device)
        finally:
            self.args.timeline, self.args.timeline_steps = None, 0
        st = buf.view(steps, self.grid, n).double().cpu()
        st = (st - st[0, 0, 0]) * 0.01                          # 100 MHz clock -> us
        return st.view(steps, self.grid, n // 2, 2)

    def run_steps(self, n: int):
        """*n* decode steps: one persistent launch, or n replays / direct steps."""
        if n <= 0:
            return
        if self.mode in ("persistent", "xcd"):
            self._launch_persistent(n)
        else:
            for _ in range(n):
                self.replay()

    def replay(self):
        """One decode step."""
        if self.mode in ("persistent", "xcd"):
            self._launch_persistent(1)
        elif self.graph is not None:
            self.graph.replay()
        else:
            self._step()

    # ------------------------------------------------------------- generation
    def _reset(self):
        self.pos.zero_()
        self.sam.zero_()
        self.err.zero_()

    def _load_prompt(self, prompt_ids: list[int]):
        pl = len(prompt_ids)
        self._reset()
        self.inp.zero_()
        self.inp[:pl] = torch.tensor(prompt_ids, dtype=torch.int32).to(self.device)
        self.plen.fill_(pl)
        self.ids.fill_(int(prompt_ids[0]))
        self._embed_current()

    def check_errors(self):
        """Raise if a kernel flagged an out-of-range index since the last reset."""
        e = int(self.err.item())
        if e:
            if e & _lib.ERR_PLACEMENT:
                raise RuntimeError("the XCD-partitioned decode kernel read an XCC id outside "
                                   "0..7 (not an 8-XCD device); its results are void")
            if e & _lib.ERR_SYNC:
                raise RuntimeError("the persistent decode kernel gave up waiting for another "
                                   "block's data (bounded wait exceeded); its results are void")
            names = [n for bit, n in ((1, "token id"), (2, "position"), (4, "page-table entry"),
                                      (8, "step")) if e & bit]
            raise RuntimeError(f"decode kernels flagged an out-of-range {', '.join(names)}")

    def prefill(self, prompt_ids: list[int]):
        """Load *prompt_ids* and fill the cache of all but its last token in
        batched passes (``qwen3.prefill``: up to 32 positions per pass through every
        layer), leaving the engine at the last prompt position: the next decode step
        consumes the last prompt token and picks the first new one, exactly where
        walking the prompt step by step would leave it."""
        pl = len(prompt_ids)
        self._load_prompt(prompt_ids)
        if pl < 2:
            return
        if getattr(self, "_prefiller", None) is None:
            from .prefill import Prefill
            self._prefiller = Prefill(self)
        self._prefiller.run(list(prompt_ids[:-1]), 0)
        self.pos.fill_(pl - 1)
        self.ids.fill_(int(prompt_ids[-1]))
        self._embed_current()

    def generate(self, prompt_ids: list[int], max_new: int,
                 record_logits: bool = False, prefill: bool = False) -> Generated:
        """Walk *prompt_ids* (or, with *prefill*, fill its cache in batched
        passes), then continue for *max_new* greedy tokens (engine.py:239-271); the
        timing covers the continuation only."""
        pl = len(prompt_ids)
        if pl < 1:
            raise ValueError("decode needs a prompt of at least one token")
        if pl + max_new > self.nsteps:
            raise ValueError(f"prompt {pl} + {max_new} new exceeds this engine's "
                             f"{self.nsteps} steps")
        if any(not 0 <= int(t) < self.V for t in prompt_ids):
            raise ValueError(f"prompt ids must lie in [0, {self.V})")
        hist = (torch.empty(max_new, self.V, device=self.device, dtype=torch.float32)
                if record_logits else None)
        torch.cuda.synchronize(self.device)
        t0 = perf_counter()
        if prefill:
            self.prefill(prompt_ids)
        else:
            self._load_prompt(prompt_ids)
            self.run_steps(pl - 1)
        torch.cuda.synchronize(self.device)
        t1 = perf_counter()
        if hist is None:
            self.run_steps(max_new)
        else:
            for k in range(max_new):
                self.replay()
                hist[k].copy_(self.logits)
        torch.cuda.synchronize(self.device)
        t2 = perf_counter()
        self.check_errors()
        out = self.sam[pl - 1: pl - 1 + max_new].tolist()
        return Generated(out, t2 - t1, t1 - t0, pl, None if hist is None else hist.cpu())

    def place_context(self, k_caches, v_caches, token: int):
        """Stand in for a walked context without walking it: layer i's cache
        rows 0 .. P-1 become ``k_caches[i]`` / ``v_caches[i]`` ([P][HKV][D] bf16,
        written through the page table), and the next step decodes *token* at
        position P -- the step the oracle's ``forward`` takes with the same caches
        (model.py:307-317).  Run it with ``run_steps(1)``; ``logits`` then hold
        its logits."""
        P = int(k_caches[0].shape[0])
        if len(k_caches) != self.L or len(v_caches) != self.L:
            raise ValueError(f"place_context: need {self.L} layers of caches")
        if P + 1 > self.nsteps:
            raise ValueError(f"place_context: position {P} past this engine's {self.nsteps}")
        if not 0 <= int(token) < self.V:
            raise ValueError(f"place_context: token {token} outside [0, {self.V})")
        self._reset()
        self.inp.zero_()
        self.inp[P] = int(token)
        self.plen.fill_(P + 1)
        self.ids.fill_(int(token))
        self.pos.fill_(P)
        scatter_cache(self.kpool, self.vpool, self.page_table, k_caches, v_caches)
        self._embed_current()

    def walk(self, seq: list[int], start: int, steps: int):
        """Teacher-forced: feed *seq* token by token, untimed, and record the
        steps at positions start .. start + steps - 1 -> (the engine's pick at
        each, its logits [steps][V] f32 on the host).  The pick at position p
        predicts seq[p + 1]; *seq* needs start + steps tokens."""
        if start < 0 or steps < 1 or start + steps > len(seq):
            raise ValueError(f"walk: start {start} + steps {steps} past {len(seq)} tokens")
        if len(seq) > self.nsteps:
            raise ValueError(f"walk: {len(seq)} tokens exceed this engine's {self.nsteps} steps")
        self._load_prompt(seq)
        self.run_steps(start)
        hist = torch.empty(steps, self.V, device=self.device, dtype=torch.float32)
        for k in range(steps):
            self.replay()
            hist[k].copy_(self.logits)
        torch.cuda.synchronize(self.device)
        self.check_errors()
        return self.sam[start:start + steps].tolist(), hist.cpu()

    def logits_for(self, prompt_ids: list[int]) -> torch.Tensor:
        """The logits after consuming every token of *prompt_ids* (f32 copy)."""
        self._load_prompt(prompt_ids)
        self.run_steps(len(prompt_ids))
        torch.cuda.synchronize(self.device)
        self.check_errors()
        return self.logits.clone()

    def trace(self, prompt_ids: list[int]) -> list[torch.Tensor]:
        """Hidden state entering the stack and leaving each layer, at the last
        prompt position (engine.py:273-287)."""
        self._load_prompt(prompt_ids)
        self.run_steps(len(prompt_ids) - 1)
        rec: list[torch.Tensor] = []
        self._step(record=rec)
        torch.cuda.synchronize(self.device)
        return rec

    # ------------------------------------------------------------ accounting
    def weight_bytes_per_step(self) -> int:
        return self.cfg.weight_bytes_per_step()

    def kv_bytes_at(self, pos: int) -> int:
        """KV bytes a step at position *pos* touches: reads of pos prior
        positions plus the write of its own, every layer."""
        return self.cfg.kv_bytes_per_position() * (pos + 1)
