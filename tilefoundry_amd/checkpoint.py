"""Published safetensors checkpoints as the engines' weight dicts.

The reference binds a checkpoint directory through ``SafetensorsResource``
(``src/tilefoundry/runtime/resource.py:183-286``: a sharded directory with
``model.safetensors.index.json``, or one unsharded ``model.safetensors``; one
mmap'd handle per shard) and an alias table per model mapping the model's
canonical weight names to the published keys, with a converter where the stored
form differs from the declared one:

* Qwen3 (C1-C3): ``examples/qwen3_1_7b-tilelang/ref_src/hf_alias.py:25-43`` --
  every ``nn.Linear`` ``(out, in)`` weight read as ``(1, in, out)``, the head as
  ``(in, out)``; the engine then packs q|k|v and gate|up itself
  (``fast/engine.py:110-133`` does the same packing).
* Qwen3.5 (C4): ``examples/qwen3_5_35b_a3b-tilelang/model.py:931-992`` (keys
  under ``model.language_model.``, fused expert tensors) and its converters
  (``model.py:230-291``): every ``Qwen3_5MoeRMSNorm`` gamma is stored as a
  delta from one, ``gamma = bf16(stored + 1)``, except the gated norm's
  (``linear_attn.norm.weight``), which is flat; the depthwise conv weight drops
  its singleton axis.
* Granite-4.0-H (C5): ``examples/granite_4_0_h_small-cuda/hf_alias.py:44-91`` --
  each expert block's fused ``input_linear`` holds the gate rows then the up
  rows, the conv weight drops its singleton axis, the layer norms sit on the
  layer.  The workload runs fp8-e4m3 weights with one f32 scale per output row:
  a checkpoint that stores fp8 codes with ``weight_scale`` tensors is taken as
  is, a bf16 one is quantised per row at load (scale = max|row| / 448).

Every loader returns what the matching engine takes: ``load_qwen3`` the canonical
dict of ``tilefoundry_amd.qwen3.weights`` (checked by ``validate``), the hybrid
loaders the engines' own row-layout dicts.  Tensors stay on the CPU, read
through the shard mmaps, until the engine copies them to the device.
"""
from __future__ import annotations

import json
from pathlib import Path

import torch

from .hybrid.granite import GraniteConfig
from .hybrid.qwen3_5 import Qwen35Config
from .qwen3.config import Qwen3Config
from .qwen3.weights import validate

BF = torch.bfloat16
FP8_MAX = 448.0                     # largest finite e4m3fn value


class SafetensorsDir:
    """A checkpoint directory: sharded (``model.safetensors.index.json``) or a
    single ``model.safetensors``; each shard is opened once, mmap'd."""

    def __init__(self, path):
        from safetensors import safe_open

        self.path = Path(path)
        self._open = safe_open
        index = self.path / "model.safetensors.index.json"
        if index.is_file():
            self._map = dict(json.loads(index.read_text(encoding="utf-8"))["weight_map"])
        else:
            single = self.path / "model.safetensors"
            if not single.is_file():
                raise FileNotFoundError(f"{self.path} holds neither model.safetensors.index.json "
                                        "nor model.safetensors")
            with safe_open(str(single), framework="pt", device="cpu") as h:
                self._map = dict.fromkeys(h.keys(), "model.safetensors")
        self._handles: dict[str, object] = {}

    def __contains__(self, key: str) -> bool:
        return key in self._map

    def keys(self):
        return self._map.keys()

    def get(self, key: str) -> torch.Tensor:
        try:
            shard = self._map[key]
        except KeyError:
            raise KeyError(f"{self.path}: no tensor named {key!r}") from None
        h = self._handles.get(shard)
        if h is None:
            h = self._open(str(self.path / shard), framework="pt", device="cpu")
            self._handles[shard] = h
        return h.get_tensor(key)

    def config(self) -> dict:
        return json.loads((self.path / "config.json").read_text(encoding="utf-8"))


# ---------------------------------------------------------------------------
# Qwen3
# ---------------------------------------------------------------------------
#: canonical layer weight -> (published key under ``model.layers.{i}.``, is a projection)
QWEN3_LAYER_KEYS = {
    "gamma_in": ("input_layernorm.weight", False),
    "gamma_post": ("post_attention_layernorm.weight", False),
    "gamma_q": ("self_attn.q_norm.weight", False),
    "gamma_k": ("self_attn.k_norm.weight", False),
    "w_q": ("self_attn.q_proj.weight", True),
    "w_k": ("self_attn.k_proj.weight", True),
    "w_v": ("self_attn.v_proj.weight", True),
    "w_o": ("self_attn.o_proj.weight", True),
    "w_gate": ("mlp.gate_proj.weight", True),
    "w_up": ("mlp.up_proj.weight", True),
    "w_down": ("mlp.down_proj.weight", True),
}


def qwen3_alias(cfg: Qwen3Config) -> dict[str, str]:
    """Canonical name -> published key (ref_src/hf_alias.py:25-43)."""
    out = {"w_embed": "model.embed_tokens.weight", "gamma_final": "model.norm.weight",
           "w_head": "lm_head.weight"}
    for i in range(cfg.num_hidden_layers):
        for name, (key, _) in QWEN3_LAYER_KEYS.items():
            out[f"layer{i}.{name}"] = f"model.layers.{i}.{key}"
    return out


def load_qwen3(path) -> tuple[Qwen3Config, dict[str, torch.Tensor]]:
    """(config, canonical weights) of a published Qwen3 checkpoint directory.

    Projections come back as ``(1, in, out)`` transposed views of the stored
    ``(out, in)`` tensors and the head as ``(in, out)``; with tied embeddings and
    no ``lm_head.weight`` the head is the embedding table's transpose.  Raises
    ``KeyError`` for a missing weight and ``ValueError`` for a wrong shape or
    dtype, as the reference's load does (``ir/core/module.py:144-159``)."""
    ck = SafetensorsDir(path)
    cfg = Qwen3Config.from_json(ck.config())
    w = {"w_embed": ck.get("model.embed_tokens.weight"),
         "gamma_final": ck.get("model.norm.weight")}
    for i in range(cfg.num_hidden_layers):
        for name, (key, projection) in QWEN3_LAYER_KEYS.items():
            t = ck.get(f"model.layers.{i}.{key}")
            w[f"layer{i}.{name}"] = t.t().unsqueeze(0) if projection else t
    if "lm_head.weight" in ck:
        w["w_head"] = ck.get("lm_head.weight").t()
    elif cfg.tie_word_embeddings:
        w["w_head"] = w["w_embed"].t()
    else:
        raise KeyError(f"{path}: no lm_head.weight and the embeddings are not tied")
    validate(cfg, w)
    return cfg, w


# ---------------------------------------------------------------------------
# Qwen3.5 (MoE, gated DeltaNet + full attention)
# ---------------------------------------------------------------------------
def qwen3_5_config(d: dict) -> Qwen35Config:
    """The text decoder's shape from a published ``config.json`` (the
    multimodal one nests it under ``text_config``)."""
    t = d.get("text_config", d)
    types = t.get("layer_types")
    layers = t["num_hidden_layers"]
    every = t.get("full_attention_interval")
    if types is not None:
        fulls = [i for i, k in enumerate(types) if k == "full_attention"]
        every = fulls[0] + 1 if fulls else 0
        if not fulls or fulls != list(range(every - 1, layers, every)):
            raise ValueError(f"layer_types {types} are not one full-attention layer every "
                             "N layers, the only layout the engine steps")
    rope = t.get("rope_parameters") or {}
    head_dim = t["head_dim"]
    rot = int(round(head_dim * rope.get("partial_rotary_factor",
                                         t.get("partial_rotary_factor", 0.25))))
    return Qwen35Config(
        hidden=t["hidden_size"], layers=layers, full_every=every,
        lin_key_heads=t["linear_num_key_heads"], lin_value_heads=t["linear_num_value_heads"],
        lin_key_dim=t["linear_key_head_dim"], lin_value_dim=t["linear_value_head_dim"],
        conv_kernel=t["linear_conv_kernel_dim"], heads=t["num_attention_heads"],
        kv_heads=t["num_key_value_heads"], head_dim=head_dim, rot_dim=rot,
        rope_theta=float(rope.get("rope_theta", t.get("rope_theta", 1.0e7))),
        experts=t["num_experts"], top_k=t["num_experts_per_tok"],
        moe_inter=t["moe_intermediate_size"], shared_inter=t["shared_expert_intermediate_size"],
        vocab=t["vocab_size"], eps=float(t.get("rms_norm_eps", 1e-6)))


def _plus_one(t: torch.Tensor) -> torch.Tensor:
    """``Qwen3_5MoeRMSNorm`` stores gamma - 1 (it computes ``x * (1 + w)``); the
    engine's norm is ``x * gamma``: bf16(stored + 1), as model.py:236-239 does."""
    return (t.to(BF) + torch.ones_like(t, dtype=BF))


def load_qwen3_5(path, cfg: Qwen35Config | None = None) -> tuple[Qwen35Config,
                                                                  dict[str, torch.Tensor]]:
    """(config, engine weights) of a published Qwen3.5-MoE checkpoint: keys
    under ``model.language_model.`` (or ``model.`` for a text-only export),
    fused expert tensors (``mlp.experts.gate_up_proj`` ``(E, 2I, H)``,
    ``mlp.experts.down_proj`` ``(E, H, I)``) or one tensor per expert."""
    ck = SafetensorsDir(path)
    cfg = cfg or qwen3_5_config(ck.config())
    pre = "model.language_model." if "model.language_model.embed_tokens.weight" in ck else "model."
    g = ck.get
    E, I, IS = cfg.experts, cfg.moe_inter, cfg.shared_inter
    d = ck.config()
    tied = bool(d.get("text_config", d).get("tie_word_embeddings",
                                            d.get("tie_word_embeddings", False)))
    if "lm_head.weight" in ck:
        head = g("lm_head.weight")
    elif tied:
        head = g(pre + "embed_tokens.weight")
    else:
        raise KeyError(f"{path}: no lm_head.weight and the embeddings are not tied")
    w = {"embed": g(pre + "embed_tokens.weight"),
         "gamma_final": _plus_one(g(pre + "norm.weight")), "head": head}
    for i in range(cfg.layers):
        p, k = f"layer{i}.", f"{pre}layers.{i}."
        w[p + "gamma_in"] = _plus_one(g(k + "input_layernorm.weight"))
        w[p + "gamma_post"] = _plus_one(g(k + "post_attention_layernorm.weight"))
        if cfg.is_full(i):
            a = k + "self_attn."
            w[p + "w_in"] = torch.cat([g(a + "q_proj.weight"), g(a + "k_proj.weight"),
                                       g(a + "v_proj.weight")], dim=0)
            w[p + "gamma_q"] = _plus_one(g(a + "q_norm.weight"))
            w[p + "gamma_k"] = _plus_one(g(a + "k_norm.weight"))
            w[p + "w_out"] = g(a + "o_proj.weight")
        else:
            a = k + "linear_attn."
            w[p + "w_in"] = torch.cat([g(a + "in_proj_qkv.weight"), g(a + "in_proj_z.weight"),
                                       g(a + "in_proj_b.weight"), g(a + "in_proj_a.weight")],
                                      dim=0)
            w[p + "conv_w"] = g(a + "conv1d.weight").squeeze(1)
            w[p + "a_log"] = g(a + "A_log")
            w[p + "dt_bias"] = g(a + "dt_bias")
            w[p + "gamma_gdn"] = g(a + "norm.weight")          # the gated norm: flat
            w[p + "w_out"] = g(a + "out_proj.weight")
        m = k + "mlp."
        w[p + "w_router"] = g(m + "gate.weight")
        if m + "experts.gate_up_proj" in ck:
            gu = g(m + "experts.gate_up_proj")
            w[p + "w_gate"], w[p + "w_up"] = gu[:, :I], gu[:, I:]
            w[p + "w_down"] = g(m + "experts.down_proj")
        else:
            e = m + "experts.{}."
            w[p + "w_gate"] = torch.stack([g(e.format(j) + "gate_proj.weight") for j in range(E)])
            w[p + "w_up"] = torch.stack([g(e.format(j) + "up_proj.weight") for j in range(E)])
            w[p + "w_down"] = torch.stack([g(e.format(j) + "down_proj.weight") for j in range(E)])
        s = m + "shared_expert."
        w[p + "w_shared_in"] = torch.cat([g(s + "gate_proj.weight"), g(s + "up_proj.weight")], 0)
        w[p + "w_shared_out"] = g(s + "down_proj.weight")
        w[p + "w_shared_scale"] = g(m + "shared_expert_gate.weight").reshape(-1)
        assert w[p + "w_gate"].shape == (E, I, cfg.hidden), (p, w[p + "w_gate"].shape)
        assert w[p + "w_shared_in"].shape == (2 * IS, cfg.hidden)
    return cfg, {n: t.to(BF) for n, t in w.items()}


# ---------------------------------------------------------------------------
# Granite-4.0-H (Mamba2 + GQA, top-k MoE with a shared MLP; fp8 linears)
# ---------------------------------------------------------------------------
def granite_config(d: dict) -> GraniteConfig:
    """The decoder's shape and multipliers from a published ``config.json``
    (layer types as published, ``mamba`` / ``attention``, or as transformers
    rewrites them, ``linear_attention`` / ``full_attention``)."""
    types = ["attention" if k in ("attention", "full_attention") else k for k in d["layer_types"]]
    d_head = d["mamba_d_head"]
    heads = d.get("mamba_n_heads", d["mamba_expand"] * d["hidden_size"] // d_head)
    if d.get("mamba_n_groups", 1) != 1:
        raise ValueError("the engine steps Mamba2 with one B/C group")
    return GraniteConfig(
        hidden=d["hidden_size"], layers=d["num_hidden_layers"],
        attention_layers=tuple(i for i, k in enumerate(types) if k == "attention"),
        mamba_heads=heads, mamba_head_dim=d_head, d_state=d["mamba_d_state"],
        conv_kernel=d["mamba_d_conv"], heads=d["num_attention_heads"],
        kv_heads=d["num_key_value_heads"],
        head_dim=d.get("head_dim", d["hidden_size"] // d["num_attention_heads"]),
        experts=d["num_local_experts"], top_k=d["num_experts_per_tok"],
        moe_inter=d["intermediate_size"], shared_inter=d["shared_intermediate_size"],
        vocab=d["vocab_size"], eps=float(d["rms_norm_eps"]),
        embedding_multiplier=float(d["embedding_multiplier"]),
        residual_multiplier=float(d["residual_multiplier"]),
        attention_multiplier=float(d["attention_multiplier"]),
        logits_scaling=float(d["logits_scaling"]))


def quantize_rows_fp8(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-output-row e4m3fn codes (uint8 ``[N][K]``) and f32 scales ``[N]`` of a
    ``[N][K]`` matrix: scale = max|row| / 448 (1 for an all-zero row), codes =
    e4m3fn(row / scale) rounded to nearest even, so dequantisation is
    ``f32(code) * scale``."""
    w = w.float()
    amax = w.abs().amax(dim=1)
    scale = torch.where(amax > 0, amax / FP8_MAX, torch.ones_like(amax))
    codes = (w / scale[:, None]).to(torch.float8_e4m3fn).view(torch.uint8)
    return codes.contiguous(), scale.contiguous()


def _fp8_linear(ck: SafetensorsDir, key: str) -> tuple[torch.Tensor, torch.Tensor]:
    """(codes, row scales) of a stored linear weight ``key`` (``...weight``):
    fp8 with a ``weight_scale`` beside it as stored, anything else quantised."""
    t = ck.get(key)
    t = t.reshape(-1, t.shape[-1])                 # expert tensors: one row per (expert, out)
    skey = key[: -len("weight")] + "weight_scale"
    if t.dtype == torch.float8_e4m3fn and skey in ck:
        scale = ck.get(skey).float().reshape(-1)
        if scale.numel() != t.shape[0]:
            raise ValueError(f"{skey}: {scale.numel()} scales for {t.shape[0]} rows "
                             "(the engine takes one scale per output row)")
        return t.view(torch.uint8).contiguous(), scale.contiguous()
    if t.dtype == torch.float8_e4m3fn:
        raise ValueError(f"{key}: fp8 weight without {skey}")
    return quantize_rows_fp8(t)


def load_granite(path, cfg: GraniteConfig | None = None) -> tuple[GraniteConfig,
                                                                  dict[str, torch.Tensor]]:
    """(config, engine weights) of a published Granite-4.0-H checkpoint
    (hf_alias.py:44-91); the expert tensors ``block_sparse_moe.input_linear``
    ``(E, 2I, H)`` and ``output_linear`` ``(E, H, I)`` become the engine's
    ``[E*I][H]`` / ``[E*H][I]`` row matrices, one scale per row."""
    ck = SafetensorsDir(path)
    cfg = cfg or granite_config(ck.config())
    g = ck.get
    E, I, H = cfg.experts, cfg.moe_inter, cfg.hidden
    w = {"embed": g("model.embed_tokens.weight").to(BF),
         "gamma_final": g("model.norm.weight").to(BF)}

    def lin(name, key):
        w[name], w[name + "_scale"] = _fp8_linear(ck, key)

    for i in range(cfg.layers):
        p, k = f"layer{i}.", f"model.layers.{i}."
        w[p + "gamma_in"] = g(k + "input_layernorm.weight").to(BF)
        w[p + "gamma_post"] = g(k + "post_attention_layernorm.weight").to(BF)
        if cfg.is_attention(i):
            a = k + "self_attn."
            parts = [_fp8_linear(ck, a + n + "_proj.weight") for n in "qkv"]
            w[p + "w_in"] = torch.cat([c for c, _ in parts], dim=0)
            w[p + "w_in_scale"] = torch.cat([s for _, s in parts], dim=0)
            lin(p + "w_out", a + "o_proj.weight")
        else:
            a = k + "mamba."
            lin(p + "w_in", a + "in_proj.weight")
            w[p + "conv_w"] = g(a + "conv1d.weight").squeeze(1).to(BF)
            w[p + "conv_b"] = g(a + "conv1d.bias").to(BF)
            w[p + "a_log"] = g(a + "A_log").to(BF)
            w[p + "dt_bias"] = g(a + "dt_bias").to(BF)
            w[p + "d_skip"] = g(a + "D").to(BF)
            w[p + "gamma_ssm"] = g(a + "norm.weight").to(BF)
            lin(p + "w_out", a + "out_proj.weight")
        m = k + "block_sparse_moe."
        lin(p + "w_router", m + "router.layer.weight")
        gu_codes, gu_scale = _fp8_linear(ck, m + "input_linear.weight")   # rows e*2I + r
        gu_codes, gu_scale = gu_codes.view(E, 2 * I, H), gu_scale.view(E, 2 * I)
        w[p + "w_gate"] = gu_codes[:, :I].reshape(E * I, H).contiguous()
        w[p + "s_gate"] = gu_scale[:, :I].reshape(-1).contiguous()
        w[p + "w_up"] = gu_codes[:, I:].reshape(E * I, H).contiguous()
        w[p + "s_up"] = gu_scale[:, I:].reshape(-1).contiguous()
        w[p + "w_down"], w[p + "s_down"] = _fp8_linear(ck, m + "output_linear.weight")
        lin(p + "w_shared_in", k + "shared_mlp.input_linear.weight")
        lin(p + "w_shared_out", k + "shared_mlp.output_linear.weight")
    return cfg, w


__all__ = ["SafetensorsDir", "QWEN3_LAYER_KEYS", "qwen3_alias", "load_qwen3", "qwen3_5_config",
           "load_qwen3_5", "granite_config", "quantize_rows_fp8", "load_granite"]
