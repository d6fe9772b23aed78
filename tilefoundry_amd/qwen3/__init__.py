"""Qwen3 dense decoder (workloads C1-C3) on the gfx950 kernels."""
from .config import QWEN3_1_7B, TINY, Qwen3Config
from .weights import declared_shapes, synthetic_weights, validate

__all__ = ["Qwen3Config", "QWEN3_1_7B", "TINY", "declared_shapes", "synthetic_weights",
           "validate"]
