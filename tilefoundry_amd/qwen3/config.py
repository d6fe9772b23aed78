"""Qwen3 dense decoder dimensions, read the way the reference reads them.

The reference builds its model from the checkpoint's own ``config.json`` through
Hugging Face's ``Qwen3Config`` (``examples/qwen3_1_7b-tilelang/ref_src/model.py:67-73``;
"a published dimension is published, never derived").  ``from_json`` does the
same from the dict, and the presets restate the benchmark's configs C1 and C2.
"""
from __future__ import annotations

import json
from dataclasses import dataclass, replace
from pathlib import Path

import torch


@dataclass(frozen=True)
class Qwen3Config:
    hidden_size: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    intermediate_size: int
    vocab_size: int
    num_hidden_layers: int
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1.0e6
    max_position_embeddings: int = 40960
    tie_word_embeddings: bool = True
    dtype: torch.dtype = torch.bfloat16

    @property
    def group(self) -> int:
        return self.num_attention_heads // self.num_key_value_heads

    @property
    def q_size(self) -> int:
        return self.num_attention_heads * self.head_dim

    @property
    def kv_size(self) -> int:
        return self.num_key_value_heads * self.head_dim

    @property
    def qkv_size(self) -> int:
        return self.q_size + 2 * self.kv_size

    def layer_params(self) -> int:
        """Parameters of one decoder layer, norms included."""
        h, i = self.hidden_size, self.intermediate_size
        return (h * self.qkv_size + self.q_size * h + 3 * h * i
                + 2 * h + 2 * self.head_dim)

    def weight_bytes_per_step(self) -> int:
        """Bytes of weights one batch-1 decode step reads: every layer, the head,
        the final norm scale and the one embedding row gathered."""
        el = torch.tensor([], dtype=self.dtype).element_size()
        head = self.vocab_size * self.hidden_size
        return el * (self.num_hidden_layers * self.layer_params() + head
                     + self.hidden_size + self.hidden_size)

    def kv_bytes_per_position(self) -> int:
        """K and V bytes one cached position holds across all layers."""
        el = torch.tensor([], dtype=self.dtype).element_size()
        return el * 2 * self.num_hidden_layers * self.kv_size

    @staticmethod
    def from_json(path_or_dict) -> "Qwen3Config":
        d = path_or_dict
        if not isinstance(d, dict):
            d = json.loads(Path(d).read_text(encoding="utf-8"))
        rope = d.get("rope_parameters") or {}
        theta = rope.get("rope_theta", d.get("rope_theta", 1.0e6))
        dt = str(d.get("torch_dtype", d.get("dtype", "bfloat16"))).removeprefix("torch.")
        return Qwen3Config(
            hidden_size=d["hidden_size"],
            num_attention_heads=d["num_attention_heads"],
            num_key_value_heads=d["num_key_value_heads"],
            head_dim=d.get("head_dim", d["hidden_size"] // d["num_attention_heads"]),
            intermediate_size=d["intermediate_size"],
            vocab_size=d["vocab_size"],
            num_hidden_layers=d["num_hidden_layers"],
            rms_norm_eps=d.get("rms_norm_eps", 1e-6),
            rope_theta=float(theta),
            max_position_embeddings=d.get("max_position_embeddings", 40960),
            tie_word_embeddings=d.get("tie_word_embeddings", True),
            dtype={"bfloat16": torch.bfloat16, "float16": torch.float16,
                   "float32": torch.float32}[dt],
        )

    def with_(self, **kw) -> "Qwen3Config":
        return replace(self, **kw)


#: Workload C1 -- tiny Qwen3-style decoder (fp32, CPU plumbing).
TINY = Qwen3Config(hidden_size=256, num_attention_heads=4, num_key_value_heads=2, head_dim=64,
                   intermediate_size=768, vocab_size=4096, num_hidden_layers=2,
                   dtype=torch.float32)
#: Workload C2 -- the Qwen3-1.7B architecture (ref_src/config.json), bf16.
QWEN3_1_7B = Qwen3Config(hidden_size=2048, num_attention_heads=16, num_key_value_heads=8,
                         head_dim=128, intermediate_size=6144, vocab_size=151936,
                         num_hidden_layers=28)
