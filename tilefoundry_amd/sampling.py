"""The step's token choice over f32 logit rows: greedy or sampled, on the device.

Greedy is the first maximal logit (``tfd_argmax_rows``; ref_src/generation.py:24-26).
Sampling is ``tfd_sample_rows`` (include/tf_decode.h), the reference's two samplers:

* ``Sampling(top_k=k, top_p=p, temperature=t)`` with k in 1..64: the top k, softmax
  at temperature t, the nucleus p inside them, one draw
  (examples/qwen3_5_35b_a3b-tilelang/run.py:145-180; that runtime's published
  defaults are t 1.0, k 20, p 0.95);
* ``Sampling(top_k=0, temperature=t)``: softmax(logits / t) over the whole
  vocabulary, by Gumbel-max (examples/granite_4_0_h_small-cuda/kernels/
  granite.cu:716-800; its run.py defaults to t 1.0).

The engines pass each sequence's position as the draw's counter, so the captured
step draws anew on every replay and a run is reproducible from ``seed``.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import lib, ptr


@dataclass(frozen=True)
class Sampling:
    """Sampling settings (see the module docstring); ``None`` in their place is greedy."""

    temperature: float = 1.0
    top_k: int = 0
    top_p: float = 1.0
    seed: int = 0

    def __post_init__(self):
        if not self.temperature > 0:
            raise ValueError(f"temperature must be positive, got {self.temperature}")
        if not 0 <= self.top_k <= _lib.SAMPLE_MAX_K:
            raise ValueError(f"top_k must lie in [0, {_lib.SAMPLE_MAX_K}] (0: the whole "
                             f"vocabulary), got {self.top_k}")
        if not 0 < self.top_p <= 1:
            raise ValueError(f"top_p must lie in (0, 1], got {self.top_p}")
        if self.top_k == 0 and self.top_p < 1:
            raise ValueError("top_p < 1 needs top_k >= 1: the nucleus is taken inside the top k")
        if not 0 <= self.seed < 1 << 64:
            raise ValueError(f"seed must be a 64-bit unsigned integer, got {self.seed}")


class Picker:
    """Launches the pick of one step: rows x vocab f32 logits (row stride ldl) ->
    pick (int32 per row), reading each row's counter on the device."""

    def __init__(self, sampling: Sampling | None, rows: int, vocab: int, device):
        self.sampling = sampling
        self.rows, self.vocab = rows, vocab
        L = lib()
        if sampling is None:
            self.work = torch.zeros(rows * _lib.ARGMAX_WORK, dtype=torch.int32, device=device)
            self.nbytes = 0
            return
        if vocab > _lib.SAMPLE_MAX_VOCAB:
            raise ValueError(f"sampling takes vocabularies up to {_lib.SAMPLE_MAX_VOCAB}, "
                             f"got {vocab}")
        self.nbytes = int(L.tfd_sample_work_bytes(rows, vocab, sampling.top_k))
        self.work = torch.zeros(max(self.nbytes, 8), dtype=torch.uint8, device=device)
        self.args = _lib.TfdSampling(sampling.temperature, sampling.top_k, sampling.top_p,
                                     sampling.seed)

    def __call__(self, logits, ldl: int, pick, counter, stream: int) -> None:
        L = lib()
        if self.sampling is None:
            L.tfd_argmax_rows(ptr(logits), ldl, self.rows, self.vocab, ptr(pick),
                              ptr(self.work), stream)
        else:
            L.tfd_sample_rows(ptr(logits), ldl, self.rows, self.vocab, ctypes.byref(self.args),
                              ptr(counter), ptr(pick), ptr(self.work), self.nbytes, stream)
