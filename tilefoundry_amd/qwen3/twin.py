"""Runtime twin of the authored Qwen3 modules, on the gfx950 kernels.

The reference pairs every authored ``@func`` with a runtime twin of the same
signature (``src/tilefoundry/runtime/decorator.py:24-229``,
``docs/spec/runtime.md:73-117``); ``examples/qwen3_1_7b-tilelang/fast/twin.py:112-236``
is the Qwen3 one.  This module keeps that surface -- the same function names,
the same argument order with weights included, the same return values -- so a
comparison can run twin and oracle function by function on one draw.

* ``LayerTwin`` mirrors ``Qwen3_1_7B_DecoderLayer``: ``input_rms_norm``,
  ``self_attention``, ``mlp``, ``decoder_layer`` (model.py:125-266).
* ``RootTwin`` mirrors ``Qwen3_1_7B``: ``embed``, ``final_rms_norm``, ``lm_head``
  (model.py:279-305), and, once loaded with weights, the orchestration methods
  ``forward / decode_hidden / append_cache / init_caches /
  prepare_inputs_for_generation`` (model.py:307-387), which callers drive with
  activations only while weights are filled by name (decorator.py:53-77).

Like the reference twin, ``self_attention`` takes the prior cache as a tensor
and returns this step's own key and value; internally it stages that context in
a paged pool (a seeded page permutation) and runs the same kernels as the engine.
All arithmetic is in the HIP library; torch here only moves and reshapes data.
"""
from __future__ import annotations

import torch

from .. import _lib
from .._lib import lib, ptr
from .config import Qwen3Config
from .weights import LAYER_NAMES, rows, validate


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


class _Packed:
    """Row-major packings of the canonical weights, remembered by tensor identity
    (the reference twin's ``_Fused``, fast/twin.py:80-102)."""

    def __init__(self):
        self._cache: dict = {}

    def get(self, kind: str, *ts: torch.Tensor) -> torch.Tensor:
        key = (kind,) + tuple((t.data_ptr(), tuple(t.shape), tuple(t.stride())) for t in ts)
        got = self._cache.get(key)
        if got is None:
            if kind == "rows":
                got = torch.cat([rows(t) for t in ts], dim=0).contiguous()
            elif kind == "gu":
                gate, up = rows(ts[0]), rows(ts[1])
                got = torch.stack([gate, up], 1).reshape(2 * gate.shape[0], -1).contiguous()
            else:
                raise KeyError(kind)
            self._cache[key] = (got, ts)   # keep sources alive so ids stay unique
            return got
        return got[0]


class LayerTwin:
    """One decoder layer in the authored signatures (model.py:123-266)."""

    def __init__(self, cfg: Qwen3Config, page_seed: int = 0):
        if cfg.dtype != torch.bfloat16:
            raise ValueError("the HIP twin runs bf16")
        self.cfg = cfg
        self.page_seed = page_seed
        self._packed = _Packed()
        self._lib = lib()

    # ------------------------------------------------------------------ @funcs
    def input_rms_norm(self, hidden, gamma_in):
        """``input_rms_norm`` (model.py:125-137)."""
        h = self.cfg.hidden_size
        out = torch.empty(h, device=hidden.device, dtype=hidden.dtype)
        self._lib.tfd_rmsnorm_bf16(ptr(hidden.contiguous()), ptr(gamma_in), ptr(out), h,
                                   float(self.cfg.rms_norm_eps), _stream(hidden))
        return out.reshape(1, 1, h)

    def self_attention(self, hidden, gamma_in, w_q, w_k, w_v, gamma_q, gamma_k, cos_cache,
                       sin_cache, pos_ids, k_cache, v_cache, scale, w_o):
        """``self_attention`` (model.py:139-216): returns (out, k_rope, v)."""
        out, k_new, v_new, _ = self._attention(hidden, gamma_in, w_q, w_k, w_v, gamma_q, gamma_k,
                                               cos_cache, sin_cache, pos_ids, k_cache, v_cache,
                                               scale, w_o, resid=None)
        return out, k_new, v_new

    def mlp(self, hidden, gamma_post, w_gate, w_up, w_down):
        """``mlp`` (model.py:218-234)."""
        return self._mlp(hidden, gamma_post, w_gate, w_up, w_down, resid=None)

    def decoder_layer(self, hidden, gamma_in, w_q, w_k, w_v, gamma_q, gamma_k, cos_cache,
                      sin_cache, pos_ids, k_cache, v_cache, scale, w_o, gamma_post, w_gate, w_up,
                      w_down):
        """``decoder_layer`` (model.py:236-266): h1 = hidden + attn; out = h1 + mlp(h1).
        The residual adds run in the projections' epilogues, as in the engine."""
        h1, k_new, v_new, _ = self._attention(hidden, gamma_in, w_q, w_k, w_v, gamma_q, gamma_k,
                                              cos_cache, sin_cache, pos_ids, k_cache, v_cache,
                                              scale, w_o, resid=hidden)
        return self._mlp(h1, gamma_post, w_gate, w_up, w_down, resid=h1), k_new, v_new

    # --------------------------------------------------------------- internals
    def _attention(self, hidden, gamma_in, w_q, w_k, w_v, gamma_q, gamma_k, cos_cache, sin_cache,
                   pos_ids, k_cache, v_cache, scale, w_o, resid):
        cfg, L = self.cfg, self._lib
        dev = hidden.device
        s = _stream(hidden)
        H, HQ, HKV, D = cfg.hidden_size, cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        ctx = int(k_cache.shape[1])
        cap = (ctx + 1 + _lib.ATTN_SPLIT - 1) // _lib.ATTN_SPLIT * _lib.ATTN_SPLIT
        max_pages, nsplit = cap // _lib.PAGE_SIZE, cap // _lib.ATTN_SPLIT
        eps = float(cfg.rms_norm_eps)

        qkv = torch.empty(cfg.qkv_size, device=dev, dtype=torch.bfloat16)
        w_qkv = self._packed.get("rows", w_q, w_k, w_v)
        L.tfd_gemv_bf16(ptr(hidden.contiguous()), ptr(gamma_in), ptr(w_qkv), None, ptr(qkv), H,
                        cfg.qkv_size, _lib.PRO_NORM, _lib.EPI_STORE, eps, s)

        # stage the prior context in a paged pool, pages in a seeded random order
        g = torch.Generator().manual_seed(self.page_seed + ctx)
        table = torch.randperm(max_pages, generator=g).to(torch.int32).to(dev)
        kpool = torch.zeros(max_pages, HKV, _lib.PAGE_SIZE, D, device=dev, dtype=torch.bfloat16)
        vpool = torch.zeros_like(kpool)
        if ctx:
            p = torch.arange(ctx, device=dev)
            page, row = table.long()[p // _lib.PAGE_SIZE], p % _lib.PAGE_SIZE
            kpool[page, :, row] = k_cache[0].to(torch.bfloat16)
            vpool[page, :, row] = v_cache[0].to(torch.bfloat16)
        cache_len = torch.tensor([ctx], device=dev, dtype=torch.int32)
        rope_pos = pos_ids.reshape(-1)[:1].to(device=dev, dtype=torch.int32)
        err = torch.zeros(1, device=dev, dtype=torch.int32)
        scores = torch.empty(HQ, cap, device=dev, dtype=torch.float32)
        smax = torch.empty(nsplit, HQ, device=dev, dtype=torch.float32)
        snew = torch.empty(HQ, device=dev, dtype=torch.float32)
        psum = torch.empty(nsplit, HQ, device=dev, dtype=torch.float32)
        pout = torch.empty(nsplit, HQ, D, device=dev, dtype=torch.float32)
        counters = torch.zeros(HKV, device=dev, dtype=torch.int32)
        attn = torch.empty(HQ * D, device=dev, dtype=torch.bfloat16)
        sc = float(scale.reshape(-1)[0].item())
        cos_t, sin_t = cos_cache.contiguous(), sin_cache.contiguous()
        L.tfd_attn_rope_scores_paged(
            ptr(qkv), ptr(gamma_q), ptr(gamma_k), ptr(cos_t), ptr(sin_t), int(cos_t.shape[0]),
            ptr(rope_pos), ptr(cache_len), ptr(table), max_pages, ptr(kpool), ptr(vpool),
            max_pages, HQ, HKV, D, sc, eps, ptr(scores), cap, ptr(smax), ptr(snew), nsplit,
            ptr(err), s)
        L.tfd_attn_pv_combine_paged(
            ptr(qkv), ptr(cache_len), ptr(table), max_pages, ptr(vpool), max_pages, HQ, HKV, D,
            ptr(scores), cap, ptr(smax), ptr(snew), ptr(psum), ptr(pout), nsplit, ptr(counters),
            ptr(attn), ptr(err), s)
        out = torch.empty(H, device=dev, dtype=torch.bfloat16)
        w_o_rows = self._packed.get("rows", w_o)
        if resid is None:
            L.tfd_gemv_bf16(ptr(attn), None, ptr(w_o_rows), None, ptr(out), HQ * D, H,
                            _lib.PRO_PLAIN, _lib.EPI_STORE, eps, s)
        else:
            L.tfd_gemv_bf16(ptr(attn), None, ptr(w_o_rows), ptr(resid.contiguous()), ptr(out),
                            HQ * D, H, _lib.PRO_PLAIN, _lib.EPI_RESID, eps, s)
        e = int(err.item())
        if e:
            raise RuntimeError(f"attention kernels flagged error bits {e:#x}")
        page, row = int(table[ctx // _lib.PAGE_SIZE]), ctx % _lib.PAGE_SIZE
        k_new = kpool[page, :, row].reshape(1, 1, HKV, D).clone()
        v_new = vpool[page, :, row].reshape(1, 1, HKV, D).clone()
        return out.reshape(1, 1, H), k_new, v_new, attn

    def _mlp(self, hidden, gamma_post, w_gate, w_up, w_down, resid):
        cfg, L = self.cfg, self._lib
        dev, s = hidden.device, _stream(hidden)
        H, I = cfg.hidden_size, cfg.intermediate_size
        eps = float(cfg.rms_norm_eps)
        hmid = torch.empty(I, device=dev, dtype=torch.bfloat16)
        L.tfd_gemv_bf16(ptr(hidden.contiguous()), ptr(gamma_post),
                        ptr(self._packed.get("gu", w_gate, w_up)), None, ptr(hmid), H, 2 * I,
                        _lib.PRO_NORM, _lib.EPI_SWIGLU, eps, s)
        out = torch.empty(H, device=dev, dtype=torch.bfloat16)
        w_down_rows = self._packed.get("rows", w_down)
        if resid is None:
            L.tfd_gemv_bf16(ptr(hmid), None, ptr(w_down_rows), None, ptr(out), I, H,
                            _lib.PRO_PLAIN, _lib.EPI_STORE, eps, s)
        else:
            L.tfd_gemv_bf16(ptr(hmid), None, ptr(w_down_rows), ptr(resid.contiguous()),
                            ptr(out), I, H, _lib.PRO_PLAIN, _lib.EPI_RESID, eps, s)
        return out.reshape(1, 1, H)


class RootTwin:
    """``Qwen3_1_7B`` (model.py:269-387): root @funcs plus, once loaded, the
    orchestration methods driven with activations only."""

    def __init__(self, cfg: Qwen3Config, page_seed: int = 0):
        self.cfg = cfg
        self.layer = LayerTwin(cfg, page_seed)
        self._lib = lib()
        self.weights: dict[str, torch.Tensor] | None = None

    # ------------------------------------------------------------------ @funcs
    def embed(self, w_embed, token_ids):
        """``embed`` (model.py:279-287)."""
        h, v = self.cfg.hidden_size, self.cfg.vocab_size
        out = torch.empty(h, device=w_embed.device, dtype=w_embed.dtype)
        err = torch.zeros(1, device=w_embed.device, dtype=torch.int32)
        ids = token_ids.reshape(1).to(device=w_embed.device, dtype=torch.int64)
        self._lib.tfd_embed_bf16(ptr(w_embed.contiguous()), ptr(ids), ptr(out), h, v, ptr(err),
                                 _stream(w_embed))
        if int(err.item()):
            raise IndexError(f"token id {int(ids.item())} outside [0, {v})")
        return out.reshape(1, 1, h)

    def final_rms_norm(self, hidden, gamma_final):
        """``final_rms_norm`` (model.py:289-298)."""
        return self.layer.input_rms_norm(hidden, gamma_final)

    def lm_head(self, hidden, w_head):
        """``lm_head`` (model.py:300-305): bf16 logits ``(1, V)``."""
        h, v = self.cfg.hidden_size, self.cfg.vocab_size
        head = self.layer._packed.get("rows", w_head)
        out = torch.empty(v, device=hidden.device, dtype=torch.bfloat16)
        self._lib.tfd_gemv_bf16(ptr(hidden.contiguous()), None, ptr(head), None, ptr(out), h, v,
                                _lib.PRO_PLAIN, _lib.EPI_STORE, 0.0, _stream(hidden))
        return out.reshape(1, v)

    # ---------------------------------------------------------- orchestration
    def load(self, weights: dict[str, torch.Tensor]) -> "RootTwin":
        """Bind weights by canonical name (shape/dtype checked like Module.load)."""
        validate(self.cfg, weights)
        self.weights = weights
        return self

    def _bound(self, name):
        if self.weights is None:
            raise TypeError("RootTwin is not loaded: call load(weights) first")
        return self.weights[name]

    def forward(self, token_ids, cos_cache, sin_cache, pos_ids, scale, caches):
        """``forward`` (model.py:307-317)."""
        hidden = self.embed(self._bound("w_embed"), token_ids)
        normed, entries = self.decode_hidden(hidden, cos_cache, sin_cache, pos_ids, scale, caches)
        return self.lm_head(normed, self._bound("w_head")), entries

    def decode_hidden(self, hidden, cos_cache, sin_cache, pos_ids, scale, caches):
        """``decode_hidden`` (model.py:319-337)."""
        n = self.cfg.num_hidden_layers
        if len(caches) != n:
            raise ValueError(f"decoder has {n} layers but was given {len(caches)} caches")
        entries = []
        for i, (k_cache, v_cache) in enumerate(caches):
            w = [self._bound(f"layer{i}.{name}") for name in LAYER_NAMES]
            g_in, w_q, w_k, w_v, g_q, g_k, w_o, g_post, w_gate, w_up, w_down = w
            hidden, k_new, v_new = self.layer.decoder_layer(
                hidden, g_in, w_q, w_k, w_v, g_q, g_k, cos_cache, sin_cache, pos_ids, k_cache,
                v_cache, scale, w_o, g_post, w_gate, w_up, w_down)
            entries.append((k_new, v_new))
        return self.final_rms_norm(hidden, self._bound("gamma_final")), tuple(entries)

    @staticmethod
    def append_cache(caches, fresh):
        """``append_cache`` (model.py:339-352)."""
        return tuple((torch.cat([kc, kn], dim=1), torch.cat([vc, vn], dim=1))
                     for (kc, vc), (kn, vn) in zip(caches, fresh))

    def init_caches(self, device="cuda:0"):
        """``init_caches`` (model.py:354-374)."""
        c = self.cfg
        empty = (1, 0, c.num_key_value_heads, c.head_dim)
        return tuple((torch.zeros(empty, device=device, dtype=c.dtype),
                      torch.zeros(empty, device=device, dtype=c.dtype))
                     for _ in range(c.num_hidden_layers))

    def prepare_inputs_for_generation(self, input_ids, step, caches, device="cuda:0"):
        """``prepare_inputs_for_generation`` (model.py:376-387)."""
        c = self.cfg
        token_ids = input_ids[step].reshape(1).to(device=device, dtype=torch.int64)
        d = c.head_dim
        inv = 1.0 / (c.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
        ph = torch.outer(torch.arange(c.max_position_embeddings, dtype=torch.float32), inv)
        ph = torch.cat((ph, ph), dim=-1)
        cos, sin = ph.cos().to(c.dtype).to(device), ph.sin().to(c.dtype).to(device)
        pos_ids = torch.tensor([step], device=device, dtype=torch.int32)
        scale = torch.full((1, 1, 1, 1), d ** -0.5, device=device, dtype=c.dtype)
        return token_ids, cos, sin, pos_ids, scale, caches
