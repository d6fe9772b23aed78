"""The Qwen3 dense decode step as the reference evaluator computes it (CPU torch).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Every function restates one ``@func`` or orchestration method of
``examples/qwen3_1_7b-tilelang/ref_src/model.py``; the line numbers are given on
each.  An op is written as the torch call the evaluator's handler for that op
makes, at the dtype the HIR declares:

* ``tf.cast``      -> ``Tensor.to``                    (``ir/hir/tensor/cast.py:43-46``)
* binary ops       -> ``torch.add/mul/sub/div/maximum``, never promoting
                      (``ir/hir/math/binary.py:130-139, 192-214``)
* ``tf.reduce``    -> ``mean/sum/amax`` in the input dtype; an empty ``max``
                      gives the dtype's least value (``ir/hir/tensor/reduce.py:108-147``)
* ``tf.rsqrt/exp`` -> ``torch.rsqrt/exp``              (``ir/hir/math/unary.py:73-90``)
* ``tf.matmul``    -> ``torch.matmul``                 (``ir/hir/nn/matmul.py:188-192``)
* ``tf.rope``      -> f32 rotate-half, cast back       (``ir/hir/nn/rope.py:147-173``)
* ``tf.silu``      -> ``torch.nn.functional.silu``     (``ir/hir/nn/silu.py:39-41``)
* ``tf.index_select`` -> ``torch.index_select``        (``ir/hir/tensor/index_select.py:141-149``)
* ``tf.repeat_interleave`` -> ``torch.repeat_interleave`` (``ir/hir/tensor/repeat_interleave.py:70-74``)

Weights are passed as a flat dict in the reference's canonical names and
layouts (``ref_src/hf_alias.py:25-43``): top-level ``w_embed (V,H)``,
``gamma_final (H,)``, ``w_head (H,V)``; per layer ``layer{i}.gamma_in``,
``.w_q (1,H,HQ*D)``, ``.w_k``, ``.w_v (1,H,HKV*D)``, ``.gamma_q``, ``.gamma_k (D,)``,
``.w_o (1,HQ*D,H)``, ``.gamma_post``, ``.w_gate``, ``.w_up (1,H,I)``,
``.w_down (1,I,H)``.
"""
from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass
from functools import lru_cache

import torch


class _Sums:
    """How the oracle evaluates the HIR's f32-accumulated reductions (matmul and
    ``reduce_sum``).  The default is torch's own kernels, as the evaluator runs
    them.  ``exact_sums()`` switches to sums taken in f64 and rounded once to
    the declared dtype: the same HIR semantics with a different (correctly
    rounded) summation, used to measure how far any f32 summation order moves
    the results -- the noise floor a correct implementation must stay within."""

    exact = False
    #: ``exact_products()``: attention's elementwise products are not rounded
    #: to the model dtype before their sum (see ``_prod_sum``)
    products = False

    def matmul(self, a, b):
        if self.exact:
            return torch.matmul(a.double(), b.double()).to(a.dtype)
        return torch.matmul(a, b)

    def sum(self, x, dim, keepdim=False):
        if self.exact:
            return x.double().sum(dim=dim, keepdim=keepdim).to(x.dtype)
        return x.sum(dim=dim, keepdim=keepdim)


_ops = _Sums()


@contextmanager
def exact_sums():
    """Evaluate every matmul and attention sum exactly (f64) inside the block."""
    prev = _ops.exact
    _ops.exact = True
    try:
        yield
    finally:
        _ops.exact = prev


@contextmanager
def exact_products():
    """Inside the block, attention's q.k and p.v products enter their sums
    unrounded (taken in f32, where every bf16 x bf16 product is exact) instead of
    rounded to the model dtype one by one; the sums are rounded to the model
    dtype as before, and every other op keeps its HIR rounding.  This is the
    arithmetic of a matrix-core product -- the reference's fast path computes
    both attention products with ``T.gemm``
    (``examples/qwen3_1_7b-tilelang/fast/kernels.py:418-501``) -- and the XCD
    decode kernel's."""
    prev = _ops.products
    _ops.products = True
    try:
        yield
    finally:
        _ops.products = prev


def _prod_sum(a, b, dim, keepdim=False):
    """``_ops.sum(a * b, dim)`` of the HIR (bf16 products, each rounded, summed
    in f32 and rounded once); under ``exact_products()`` the products are exact
    and only the sum is rounded to the operands' dtype."""
    if not _ops.products:
        return _ops.sum(a * b, dim=dim, keepdim=keepdim)
    wide = torch.float64 if _ops.exact else torch.float32
    return (a.to(wide) * b.to(wide)).sum(dim=dim, keepdim=keepdim).to(a.dtype)


@dataclass(frozen=True)
class Qwen3Dims:
    """The published fields a Qwen3 dense decoder is built from (``ref_src/config.json``)."""

    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    intermediate: int
    vocab: int
    layers: int
    eps: float = 1e-6
    rope_theta: float = 1.0e6
    max_positions: int = 40960
    dtype: torch.dtype = torch.bfloat16

    @property
    def group(self) -> int:
        return self.heads // self.kv_heads


#: Workload C1: tiny Qwen3-style decoder, fp32.
C1 = Qwen3Dims(hidden=256, heads=4, kv_heads=2, head_dim=64, intermediate=768,
               vocab=4096, layers=2, dtype=torch.float32)
#: Workload C2: the Qwen3-1.7B architecture, bf16.
C2 = Qwen3Dims(hidden=2048, heads=16, kv_heads=8, head_dim=128, intermediate=6144,
               vocab=151936, layers=28, dtype=torch.bfloat16)


# ----------------------------------------------------------------- rope tables
@lru_cache(maxsize=8)
def generation_rope(dims: Qwen3Dims, rows: int | None = None):
    """``_generation_rope`` (``ref_src/model.py:107-120``): cos/sin ``(rows, D)``.

    Inverse frequencies in f32, the f32 outer product with the position ramp,
    duplicated halves, ``cos``/``sin`` in f32, then cast to the model dtype.
    """
    d = dims.head_dim
    rows = dims.max_positions if rows is None else rows
    inverse = 1.0 / (dims.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    phases = torch.outer(torch.arange(rows, dtype=torch.float32), inverse)
    phases = torch.cat((phases, phases), dim=-1)
    return phases.cos().to(dims.dtype), phases.sin().to(dims.dtype)


def _rope(x, cos_cache, sin_cache, pos_ids, out_dtype):
    """``tf.rope`` eval (``ir/hir/nn/rope.py:147-173``) for one operand."""
    xf = x.float()
    pos = pos_ids.reshape(-1).long()
    cos = cos_cache[pos].float()[None, :, None, :]
    sin = sin_cache[pos].float()[None, :, None, :]
    half = xf.shape[-1] // 2
    rotated = torch.cat((-xf[..., half:], xf[..., :half]), dim=-1)
    return (xf * cos + rotated * sin).to(out_dtype)


def _head_rms(x, gamma, eps, dt):
    """The per-head RMS written out in ``self_attention`` (``model.py:172-178``)."""
    x32 = x.to(torch.float32)
    var = (x32 * x32).mean(dim=-1, keepdim=True)
    return (x32 * torch.rsqrt(var + eps)).to(dt) * gamma


# --------------------------------------------------------------- layer @funcs
def input_rms_norm(dims: Qwen3Dims, hidden, gamma_in):
    """``Qwen3_1_7B_DecoderLayer.input_rms_norm`` (``model.py:125-137``).

    The normalised activation is rounded to the model dtype *before* the learned
    scale multiplies it (the Qwen3RMSNorm order).
    """
    x32 = hidden.to(torch.float32)
    variance = (x32 * x32).mean(dim=-1, keepdim=True)
    normed = (x32 * torch.rsqrt(variance + dims.eps)).to(dims.dtype)
    return normed * gamma_in


def self_attention(dims: Qwen3Dims, hidden, gamma_in, w_q, w_k, w_v, gamma_q, gamma_k,
                   cos_cache, sin_cache, pos_ids, k_cache, v_cache, scale, w_o):
    """``self_attention`` (``model.py:139-216``): fused norm, QKV, q/k norm, RoPE,
    GQA over the prior cache plus this token, o_proj.

    Returns ``(out, k_rope, v)`` -- this token's own entry, for the caller to append.
    """
    dt = dims.dtype
    hq, hkv, d, g = dims.heads, dims.kv_heads, dims.head_dim, dims.group
    ctx = k_cache.shape[1]
    hidden_norm = input_rms_norm(dims, hidden, gamma_in)
    q = _ops.matmul(hidden_norm, w_q).reshape(1, 1, hq, d)
    k = _ops.matmul(hidden_norm, w_k).reshape(1, 1, hkv, d)
    v = _ops.matmul(hidden_norm, w_v).reshape(1, 1, hkv, d)
    q_n = _head_rms(q, gamma_q, dims.eps, dt)
    q_rope = _rope(q_n, cos_cache, sin_cache, pos_ids, dt)
    k_n = _head_rms(k, gamma_k, dims.eps, dt)
    k_rope = _rope(k_n, cos_cache, sin_cache, pos_ids, dt)

    q_s = q_rope.reshape(1, 1, hq, d) * scale
    k_ctx = torch.repeat_interleave(k_cache, g, dim=2).permute(0, 2, 1, 3).reshape(1, 1, hq, ctx, d)
    v_ctx = torch.repeat_interleave(v_cache, g, dim=2).permute(0, 2, 1, 3).reshape(1, 1, hq, ctx, d)
    k_new = torch.repeat_interleave(k_rope, g, dim=2)
    v_new = torch.repeat_interleave(v, g, dim=2)

    q_e = q_s.reshape(1, 1, hq, 1, d)
    score_ctx = _prod_sum(q_e, k_ctx, dim=-1, keepdim=True)            # (1,1,hq,ctx,1)
    score_new = _prod_sum(q_s, k_new, dim=-1, keepdim=True)            # (1,1,hq,1)
    if ctx == 0:
        # reduce.py:124-133: an empty max is the dtype's least representable value
        ctx_max = torch.full((1, 1, hq, 1), float("-inf"), dtype=dt)
    else:
        ctx_max = score_ctx.amax(dim=-2)                           # (1,1,hq,1)
    peak = torch.maximum(ctx_max, score_new)
    peak_e = peak.reshape(1, 1, hq, 1, 1)
    p_ctx = torch.exp(score_ctx - peak_e)
    p_new = torch.exp(score_new - peak)
    total = _ops.sum(p_ctx, dim=-2) + p_new
    weighted = _prod_sum(p_ctx, v_ctx, dim=-2) + p_new * v_new
    attn = weighted / total
    out = _ops.matmul(attn.reshape(1, 1, hq * d), w_o)
    return out, k_rope, v


def mlp(dims: Qwen3Dims, hidden, gamma_post, w_gate, w_up, w_down):
    """``mlp`` (``model.py:218-234``): fused post-attention norm + dense SwiGLU."""
    hidden_norm = input_rms_norm(dims, hidden, gamma_post)
    gate = _ops.matmul(hidden_norm, w_gate)
    up = _ops.matmul(hidden_norm, w_up)
    act = torch.nn.functional.silu(gate)
    return _ops.matmul(act * up, w_down)


def decoder_layer(dims: Qwen3Dims, hidden, gamma_in, w_q, w_k, w_v, gamma_q, gamma_k,
                  cos_cache, sin_cache, pos_ids, k_cache, v_cache, scale, w_o,
                  gamma_post, w_gate, w_up, w_down):
    """``decoder_layer`` (``model.py:236-266``): attention + residual, mlp + residual."""
    attn_out, k_new, v_new = self_attention(
        dims, hidden, gamma_in, w_q, w_k, w_v, gamma_q, gamma_k,
        cos_cache, sin_cache, pos_ids, k_cache, v_cache, scale, w_o)
    h1 = hidden + attn_out
    return h1 + mlp(dims, h1, gamma_post, w_gate, w_up, w_down), k_new, v_new


# ---------------------------------------------------------------- root @funcs
def embed(dims: Qwen3Dims, w_embed, token_ids):
    """``Qwen3_1_7B.embed`` (``model.py:279-287``)."""
    return torch.index_select(w_embed, 0, token_ids).reshape(1, 1, dims.hidden)


def final_rms_norm(dims: Qwen3Dims, hidden, gamma_final):
    """``final_rms_norm`` (``model.py:289-298``)."""
    return input_rms_norm(dims, hidden, gamma_final)


def lm_head(dims: Qwen3Dims, hidden, w_head):
    """``lm_head`` (``model.py:300-305``): logits in the model dtype."""
    return _ops.matmul(hidden.reshape(1, dims.hidden), w_head)


_LAYER_WEIGHTS = ("gamma_in", "w_q", "w_k", "w_v", "gamma_q", "gamma_k", "w_o",
                  "gamma_post", "w_gate", "w_up", "w_down")


class Qwen3Oracle:
    """The root module with weights bound, driving the orchestration methods
    ``forward / decode_hidden / append_cache / init_caches /
    prepare_inputs_for_generation`` (``model.py:307-387``)."""

    def __init__(self, dims: Qwen3Dims, weights: dict[str, torch.Tensor]):
        self.dims = dims
        self.w = weights

    def _layer(self, i):
        return [self.w[f"layer{i}.{n}"] for n in _LAYER_WEIGHTS]

    def forward(self, token_ids, cos_cache, sin_cache, pos_ids, scale, caches, record=None):
        """``forward`` (``model.py:307-317``): logits and each layer's fresh entry."""
        hidden = embed(self.dims, self.w["w_embed"], token_ids)
        normed, entries = self.decode_hidden(hidden, cos_cache, sin_cache, pos_ids, scale,
                                             caches, record=record)
        return lm_head(self.dims, normed, self.w["w_head"]), entries

    def decode_hidden(self, hidden, cos_cache, sin_cache, pos_ids, scale, caches, record=None):
        """``decode_hidden`` (``model.py:319-337``)."""
        if len(caches) != self.dims.layers:
            raise ValueError(f"decoder has {self.dims.layers} layers but was given "
                             f"{len(caches)} caches")
        entries = []
        if record is not None:
            record.append(hidden.clone())
        for i, (k_cache, v_cache) in enumerate(caches):
            g_in, w_q, w_k, w_v, g_q, g_k, w_o, g_post, w_gate, w_up, w_down = self._layer(i)
            hidden, k_new, v_new = decoder_layer(
                self.dims, hidden, g_in, w_q, w_k, w_v, g_q, g_k, cos_cache, sin_cache,
                pos_ids, k_cache, v_cache, scale, w_o, g_post, w_gate, w_up, w_down)
            entries.append((k_new, v_new))
            if record is not None:
                record.append(hidden.clone())
        return final_rms_norm(self.dims, hidden, self.w["gamma_final"]), tuple(entries)

    @staticmethod
    def append_cache(caches, fresh):
        """``append_cache`` (``model.py:339-352``)."""
        return tuple((torch.cat([kc, kn], dim=1), torch.cat([vc, vn], dim=1))
                     for (kc, vc), (kn, vn) in zip(caches, fresh))

    def init_caches(self):
        """``init_caches`` (``model.py:354-374``): zero-length caches."""
        d = self.dims
        empty = (1, 0, d.kv_heads, d.head_dim)
        return tuple((torch.zeros(empty, dtype=d.dtype), torch.zeros(empty, dtype=d.dtype))
                     for _ in range(d.layers))

    def prepare_inputs_for_generation(self, input_ids, step, caches):
        """``prepare_inputs_for_generation`` (``model.py:376-387``)."""
        d = self.dims
        token_ids = input_ids[step].reshape(1).to(torch.int64)
        cos_cache, sin_cache = generation_rope(d)
        pos_ids = torch.tensor([step], dtype=torch.int32)
        scale = torch.full((1, 1, 1, 1), d.head_dim ** -0.5, dtype=d.dtype)
        return token_ids, cos_cache, sin_cache, pos_ids, scale, caches


def greedy(logits) -> int:
    """``greedy`` (``ref_src/generation.py:24-26``): ``torch.argmax`` -> first maximal index."""
    return int(torch.argmax(logits).item())


@dataclass
class OracleRun:
    tokens: list[int]          # the continuation (greedy picks)
    logits: list[torch.Tensor]  # logits (f32 copy) at each pick, in order
    margins: list[float]       # top-1 minus top-2 logit at each pick


def decode(oracle: Qwen3Oracle, prompt_ids: list[int], max_new: int,
           keep_logits: bool = True) -> OracleRun:
    """The greedy loop of ``ref_src/generation.py:41-85`` over token ids.

    Every prompt position is one forward; the last prompt step's logits give the
    first pick; each pick is fed back.  Unlike the reference loop, the logits of
    every pick are kept (for the comparison) and the top-2 margin is recorded.
    """
    if not prompt_ids:
        raise ValueError("decode needs a prompt of at least one token")
    pl = len(prompt_ids)
    input_ids = torch.zeros(pl + max_new, dtype=torch.int64)
    input_ids[:pl] = torch.tensor(prompt_ids, dtype=torch.int64)
    caches = oracle.init_caches()
    logits = None
    with torch.no_grad():
        for step in range(pl):
            args = oracle.prepare_inputs_for_generation(input_ids, step, caches)
            logits, fresh = oracle.forward(*args)
            caches = oracle.append_cache(caches, fresh)
        out, kept, margins = [], [], []
        for step in range(max_new):
            token = greedy(logits)
            top2 = torch.topk(logits.float().reshape(-1), 2).values
            margins.append(float(top2[0] - top2[1]))
            if keep_logits:
                kept.append(logits.float().reshape(-1).clone())
            out.append(token)
            if step + 1 == max_new:
                break
            input_ids[pl + step] = token
            args = oracle.prepare_inputs_for_generation(input_ids, pl + step, caches)
            logits, fresh = oracle.forward(*args)
            caches = oracle.append_cache(caches, fresh)
    return OracleRun(out, kept, margins)
