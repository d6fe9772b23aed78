"""Prompt prefill: up to 32 prompt positions through every layer in one pass.

The reference's engine walks a prompt one token per replayed decode step
(``examples/qwen3_1_7b-tilelang/fast/engine.py:261-262``); its placed fixture
``tests/fixtures/placed/qwen3_1_7b_pd.py:55-230`` (``layer_prefill``) is the
batched form: the prompt rows go through the norm, one q/k/v GEMM, q/k norm +
RoPE, the cache update for every row, causal attention and the MLP GEMMs
together.  Here a chunk of R <= 32 prompt rows runs each layer as the batched
decode step does (``batch_engine.py``: MFMA skinny GEMMs, row norms, paged
attention per (split, kv head, row)), with every row a position of the same
sequence: row r sits at position c0 + r and all rows share the sequence's page
table, so row r attends to the cache rows 0 .. c0 + r - 1 the earlier rows
wrote plus its own key -- the causal attention of the prompt, each position
valued exactly as a decode step at that position values it (the HIR's rounding
points; only f32 summation orders differ).

Rows of one chunk append their keys and values to the same cache the later
rows read, so the scores launch runs twice per layer: the first launch's
appends (every row's split 0 writes its own position) are complete when the
second one reads the cache, and the second launch writes the same bits again.

Prefill fills the cache for positions start .. start + n - 1 and leaves the
hidden states of those rows unused: the last prompt token is then decoded as
before, by the decode step, which produces the first new token.

The same pass serves a batch engine (``batch_engine.py``): its sequences share
one pool of pages, each with its own page-table row, and a prompt is prefilled
one sequence at a time through that sequence's row.
"""
from __future__ import annotations

import torch

from .. import _lib
from .._lib import lib, ptr

MAX_ROWS = 32

# The batched attention's grid is (splits, kv heads, rows): about two blocks per
# compute unit (256 on the MI355X) keeps every split long enough that its tiles
# stream back to back.  At batch 32 over 4,159 positions, measured per layer:
# scores + P.V 98.8 us with 2 splits, 99.8 with 3, 102.8 with 4, 111.7 with 17.
SPLIT_BLOCKS = 512


def attention_splits(rows: int, kv_heads: int, cap: int) -> int:
    """Splits per (row, kv head) of the batched attention for *rows* rows; their
    length follows each row's position (``split_tiles`` 0)."""
    tiles = -(-cap // _lib.ATTN_SPLIT)
    return max(1, min(tiles, -(-SPLIT_BLOCKS // (rows * kv_heads))))


class Prefill:
    """The batched prompt pass over an engine's weights, pools and page table.

    *engine* is a ``qwen3.engine.Engine`` (or anything with its attributes:
    ``layers``, ``kpool``/``vpool`` [L][pages][HKV][16][D], ``page_table``
    ([max_pages], or [sequences][max_pages] with ``num_pages`` pages in the
    pool), ``cos``/``sin``, ``cap``).  With *packed* False the projections are
    re-laid once into the skinny GEMMs' operand blocks (one more copy of the
    layer weights in HBM); a batch engine's layers are already in that order."""

    def __init__(self, engine, packed: bool = False):
        e = engine
        self.e = e
        self._lib = lib()
        self.dev = e.device
        self.L, self.H, self.I, self.D = e.L, e.H, e.I, e.D
        self.HQ, self.HKV = e.HQ, e.HKV
        self.QD = self.HQ * self.D
        self.qkv_n = e.cfg.qkv_size
        self.eps, self.scale = e.eps, e.scale
        self.max_pages = e.max_pages
        self.num_pages = getattr(e, "num_pages", e.max_pages)
        self.rows = e.page_table.reshape(-1, self.max_pages)      # [sequences][max_pages]
        self.nsplit = attention_splits(MAX_ROWS, self.HKV, e.cap)
        self.split_tiles = 0                  # derived from each row's position
        self.score_stride = -(-e.cap // _lib.ATTN_SPLIT) * _lib.ATTN_SPLIT
        s = torch.cuda.current_stream(self.dev).cuda_stream
        self.layers = []
        for w in e.layers:
            lw = dict(w)
            if not packed:
                for n in ("w_qkv", "w_o", "w_gu", "w_down"):
                    lw[n] = self._mfma_order(w[n], s)
            self.layers.append(lw)
        torch.cuda.synchronize(self.dev)
        self._buffers()

    def _mfma_order(self, w, s):
        N, K = w.shape
        out = torch.empty(-(-N // 16) * 16, K, device=w.device, dtype=w.dtype)
        self._lib.tfd_pack_skinny_bf16(ptr(w), K, N, K, ptr(out), s)
        return out

    def _buffers(self):
        dev, bf, f32, i32 = self.dev, torch.bfloat16, torch.float32, torch.int32
        R = MAX_ROWS

        def z(*shape, dtype=bf):
            return torch.zeros(*shape, device=dev, dtype=dtype)

        self.hid = [z(R, self.H), z(R, self.H)]       # ping-pong layer input / output
        self.xn = z(32 * self.H)
        self.qkv = z(R, self.qkv_n)
        self.attn = z(32 * self.QD)
        self.h1 = z(R, self.H)
        self.hmid = z(32 * self.I)
        self.scores = z(R, self.HQ, self.score_stride, dtype=f32)
        self.smax = z(R, self.nsplit, self.HQ, dtype=f32)
        self.snew = z(R, self.HQ, dtype=f32)
        self.psum = z(R, self.nsplit, self.HQ, dtype=f32)
        self.pout = z(R, self.nsplit, self.HQ, self.D, dtype=f32)
        self.counters = z(R, self.HKV, dtype=i32)
        self.pos = z(R, dtype=i32)
        self.ids = z(R, dtype=torch.int64)
        self.table = self.rows[:1].expand(R, -1).contiguous()
        self.work = z(1 << 21, dtype=f32)

    def _gemm(self, x, w, R, K, N, epi, resid, out, ldo, s):
        self._lib.tfd_gemm_skinny_bf16(ptr(x), ptr(w), R, K, N, epi,
                                       None if resid is None else ptr(resid),
                                       0 if resid is None else resid.shape[-1], ptr(out), ldo,
                                       ptr(self.work), self.work.numel(), s)

    def _layer(self, i, R, s):
        """One decoder layer (model.py:236-266) for R prompt rows."""
        L, w, e = self._lib, self.layers[i], self.e
        H, I, D = self.H, self.I, self.D
        x_in, x_out = self.hid[i % 2], self.hid[(i + 1) % 2]
        L.tfd_rmsnorm_rows_bf16(ptr(x_in), H, ptr(w["gamma_in"]), ptr(self.xn), 0, R, H,
                                self.eps, 1, s)
        self._gemm(self.xn, w["w_qkv"], R, H, self.qkv_n, _lib.EPI_STORE, None, self.qkv,
                   self.qkv_n, s)
        for _ in range(2):      # the first launch's appends complete before the second reads
            L.tfd_attn_rope_scores_paged_batched(
                ptr(self.qkv), self.qkv_n, ptr(w["gamma_q"]), ptr(w["gamma_k"]), ptr(e.cos),
                ptr(e.sin), e.cap, ptr(self.pos), ptr(self.table), self.max_pages,
                ptr(e.kpool[i]), ptr(e.vpool[i]), self.num_pages, R, self.HQ, self.HKV, D,
                self.scale, self.eps, ptr(self.scores), self.score_stride, ptr(self.smax),
                ptr(self.snew), self.nsplit, self.split_tiles, ptr(e.err), s)
        L.tfd_attn_pv_combine_paged_batched(
            ptr(self.qkv), self.qkv_n, ptr(self.pos), ptr(self.table), self.max_pages,
            ptr(e.vpool[i]), self.num_pages, R, self.HQ, self.HKV, D, ptr(self.scores),
            self.score_stride, ptr(self.smax), ptr(self.snew), ptr(self.psum), ptr(self.pout),
            self.nsplit, self.split_tiles, ptr(self.counters), ptr(self.attn), ptr(e.err), s)
        self._gemm(self.attn, w["w_o"], R, self.QD, H, _lib.EPI_RESID, x_in, self.h1, H, s)
        L.tfd_rmsnorm_rows_bf16(ptr(self.h1), H, ptr(w["gamma_post"]), ptr(self.xn), 0, R, H,
                                self.eps, 1, s)
        self._gemm(self.xn, w["w_gu"], R, H, 2 * I, _lib.EPI_SWIGLU, None, self.hmid, 0, s)
        self._gemm(self.hmid, w["w_down"], R, I, H, _lib.EPI_RESID, self.h1, x_out, H, s)

    def run(self, tokens: list[int], start: int = 0, seq: int = 0):
        """Fill every layer's cache at positions start .. start + len(tokens) - 1
        of sequence *seq* (its page-table row) from those tokens (chunks of up to
        32 rows)."""
        e = self.e
        if start < 0 or start + len(tokens) > e.cap:
            raise ValueError(f"prefill: positions {start}..{start + len(tokens) - 1} outside the "
                             f"cache ({e.cap} positions)")
        if any(not 0 <= int(t) < e.V for t in tokens):
            raise ValueError(f"prefill: token ids must lie in [0, {e.V})")
        if not 0 <= seq < self.rows.shape[0]:
            raise ValueError(f"prefill: sequence {seq} outside [0, {self.rows.shape[0]})")
        self.table.copy_(self.rows[seq:seq + 1].expand(MAX_ROWS, -1))
        s = torch.cuda.current_stream(self.dev).cuda_stream
        for c0 in range(0, len(tokens), MAX_ROWS):
            chunk = tokens[c0:c0 + MAX_ROWS]
            R = len(chunk)
            self.ids[:R].copy_(torch.tensor(chunk, dtype=torch.int64))
            self.pos[:R].copy_(torch.arange(start + c0, start + c0 + R, dtype=torch.int32))
            self._lib.tfd_embed_rows_bf16(ptr(e.w_embed), ptr(self.ids), ptr(self.hid[0]),
                                          self.H, R, self.H, e.V, ptr(e.err), s)
            for i in range(self.L):
                self._layer(i, R, s)
