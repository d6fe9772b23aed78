"""Weights for the Qwen3 decoder: canonical names, synthetic draws, validation, packing.

Canonical names and layouts are the reference's (``ref_src/model.py:123-305`` as
bound by ``ref_src/hf_alias.py:25-43``): a flat dict with top-level ``w_embed``
``(V, H)``, ``gamma_final (H,)``, ``w_head (H, V)`` and per layer
``layer{i}.{name}`` with ``w_q (1, H, HQ*D)``, ``w_k``/``w_v (1, H, HKV*D)``,
``w_o (1, HQ*D, H)``, ``w_gate``/``w_up (1, H, I)``, ``w_down (1, I, H)`` and the
norm scales ``gamma_in``/``gamma_post (H,)``, ``gamma_q``/``gamma_k (D,)``.

The projections are drawn in Hugging Face's ``(out, in)`` orientation and the
canonical ``(1, in, out)`` entries are transposed *views* of them, so the packed
device layout (row-major ``[out][in]``) costs no CPU copy and the tied head is the
embedding table itself.
"""
from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import torch

from .config import Qwen3Config

LAYER_NAMES = ("gamma_in", "w_q", "w_k", "w_v", "gamma_q", "gamma_k", "w_o", "gamma_post",
               "w_gate", "w_up", "w_down")

_CHUNK = 1 << 22


def declared_shapes(cfg: Qwen3Config) -> dict[str, tuple[int, ...]]:
    """Every canonical weight and its declared shape (model.py:139-305)."""
    h, d, i = cfg.hidden_size, cfg.head_dim, cfg.intermediate_size
    out = {"w_embed": (cfg.vocab_size, h), "gamma_final": (h,), "w_head": (h, cfg.vocab_size)}
    per = {"gamma_in": (h,), "w_q": (1, h, cfg.q_size), "w_k": (1, h, cfg.kv_size),
           "w_v": (1, h, cfg.kv_size), "gamma_q": (d,), "gamma_k": (d,),
           "w_o": (1, cfg.q_size, h), "gamma_post": (h,), "w_gate": (1, h, i),
           "w_up": (1, h, i), "w_down": (1, i, h)}
    for layer in range(cfg.num_hidden_layers):
        for name, shape in per.items():
            out[f"layer{layer}.{name}"] = shape
    return out


def validate(cfg: Qwen3Config, weights: dict[str, torch.Tensor]) -> None:
    """Name, shape and dtype check, as ``Module.load`` / ``_validate_declared``
    do (``ir/core/module.py:144-159``): ``KeyError`` for a missing weight,
    ``ValueError`` for a wrong shape or dtype."""
    for name, shape in declared_shapes(cfg).items():
        if name not in weights:
            raise KeyError(f"weight {name!r} is declared but not supplied")
        t = weights[name]
        if tuple(t.shape) != shape:
            raise ValueError(f"weight {name!r}: declared shape {shape}, got {tuple(t.shape)}")
        if t.dtype != cfg.dtype:
            raise ValueError(f"weight {name!r}: declared dtype {cfg.dtype}, got {t.dtype}")


def _normal(shape, seed: int, key: int, sigma: float, pool) -> torch.Tensor:
    """N(0, sigma^2) f32 draws, in fixed 4M-element chunks each seeded by
    (seed, key, chunk) -- the result does not depend on the thread count."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)

    def fill(c):
        lo = c * _CHUNK
        hi = min(n, lo + _CHUNK)
        rng = np.random.Generator(np.random.PCG64(np.random.SeedSequence([seed, key, c])))
        out[lo:hi] = rng.standard_normal(hi - lo, dtype=np.float32)

    list(pool.map(fill, range((n + _CHUNK - 1) // _CHUNK)))
    t = torch.from_numpy(out).reshape(shape)
    return t.mul_(sigma)


def synthetic_weights(cfg: Qwen3Config, seed: int = 0, sigma: float = 0.02,
                      norms: str = "random") -> dict[str, torch.Tensor]:
    """Random-init weights of the architecture, on the CPU, in canonical names.

    Every parameter is N(0, sigma^2) -- the reference's own test convention
    (``tests/models/decode_oracle.py:213-233`` draws *every* parameter, norm
    scales included).  ``norms="ones"`` sets the norm scales to 1 instead (the
    Hugging Face initialisation), which gives attention sharper softmaxes; tests
    use both.  The head is tied: ``w_head`` is ``w_embed.T``.
    """
    h, d, i, v = cfg.hidden_size, cfg.head_dim, cfg.intermediate_size, cfg.vocab_size
    dt = cfg.dtype
    threads = min(16, os.cpu_count() or 1)
    w: dict[str, torch.Tensor] = {}
    key = 0

    def draw(shape):
        nonlocal key
        key += 1
        return _normal(shape, seed, key, sigma, pool).to(dt)

    def norm(n):
        t = draw((n,))
        return torch.ones(n, dtype=dt) if norms == "ones" else t

    with ThreadPoolExecutor(threads) as pool:
        w["w_embed"] = draw((v, h))
        for layer in range(cfg.num_hidden_layers):
            p = f"layer{layer}."
            w[p + "gamma_in"] = norm(h)
            w[p + "w_q"] = draw((cfg.q_size, h)).t().unsqueeze(0)
            w[p + "w_k"] = draw((cfg.kv_size, h)).t().unsqueeze(0)
            w[p + "w_v"] = draw((cfg.kv_size, h)).t().unsqueeze(0)
            w[p + "gamma_q"] = norm(d)
            w[p + "gamma_k"] = norm(d)
            w[p + "w_o"] = draw((h, cfg.q_size)).t().unsqueeze(0)
            w[p + "gamma_post"] = norm(h)
            w[p + "w_gate"] = draw((i, h)).t().unsqueeze(0)
            w[p + "w_up"] = draw((i, h)).t().unsqueeze(0)
            w[p + "w_down"] = draw((h, i)).t().unsqueeze(0)
        w["gamma_final"] = norm(h)
    w["w_head"] = w["w_embed"].t()
    return w


def rows(t: torch.Tensor) -> torch.Tensor:
    """A canonical ``(1, in, out)`` / ``(in, out)`` weight as row-major ``[out][in]``."""
    return t.reshape(t.shape[-2], t.shape[-1]).t()


def pack_layer(weights: dict[str, torch.Tensor], layer: int, device) -> dict[str, torch.Tensor]:
    """One layer in the device layout the kernels read.

    * ``w_qkv`` ``[HQ*D + 2*HKV*D][H]``: q rows, then k, then v (one GEMV).
    * ``w_o`` ``[H][HQ*D]``.
    * ``w_gu`` ``[2*I][H]`` with gate and up rows interleaved (gate_i at 2i,
      up_i at 2i+1), so one wave owns both halves of an activation.
    * ``w_down`` ``[H][I]``.
    """
    p = f"layer{layer}."
    g = lambda n: weights[p + n]  # noqa: E731
    qkv = torch.cat([rows(g("w_q")), rows(g("w_k")), rows(g("w_v"))], dim=0)
    gate, up = rows(g("w_gate")), rows(g("w_up"))
    gu = torch.stack([gate, up], dim=1).reshape(2 * gate.shape[0], gate.shape[1])
    out = {
        "w_qkv": qkv.to(device).contiguous(),
        "w_o": rows(g("w_o")).to(device).contiguous(),
        "w_gu": gu.to(device).contiguous(),
        "w_down": rows(g("w_down")).to(device).contiguous(),
    }
    for n in ("gamma_in", "gamma_post", "gamma_q", "gamma_k"):
        out[n] = g(n).to(device).contiguous()
    return out


def head_rows(weights: dict[str, torch.Tensor], device) -> tuple[torch.Tensor, torch.Tensor]:
    """(embedding table, head rows ``[V][H]``) on the device; one tensor when tied."""
    emb = weights["w_embed"].to(device).contiguous()
    head = weights["w_head"]
    if head.t().data_ptr() == weights["w_embed"].data_ptr() and head.t().is_contiguous():
        return emb, emb
    return emb, rows(head).to(device).contiguous()
