"""Whole-step pins of the hybrid oracles (``GraniteOracle.step``,
``Qwen35Oracle.step``) against Hugging Face's own models, on the CPU.

The per-function pins (``test_oracle_hybrid.py``) leave open how a whole step
composes its pieces: the published multipliers (embedding x12, residual x0.22,
attention 1/128, logits / 16), which layers are which type, the shared-expert
gate, the residual stream, the final norm and the head.  Here a tiny
``GraniteMoeHybridForCausalLM`` / ``Qwen3_5MoeForCausalLM`` (transformers 5.15,
built offline from a config, weights copied from the same synthetic dict the
oracle reads; Granite's fp8 codes dequantised to f32) runs the prompt as one
full sequence -- chunked Mamba2 scan, chunked gated-delta rule, causal-mask
attention: different algorithms from the oracle's one-token recurrences -- and
its logits at every position are compared with the oracle stepping token by
token.  With ``unrounded()`` both are f32 mathematics and agree to f32
accumulation noise; with the oracle's bf16 rounding on, the gap is bf16 noise.
A dropped multiplier, a swapped layer type or a missing gate moves the logits
by O(1) (checked by planting each in the oracle's config or weights)."""
import dataclasses

import pytest
import torch

from oracle import hybrid_ref as H
from tilefoundry_amd.hybrid import granite as G
from tilefoundry_amd.hybrid import qwen3_5 as Q

hf_g = pytest.importorskip("transformers.models.granitemoehybrid.modeling_granitemoehybrid")
hf_q = pytest.importorskip("transformers.models.qwen3_5_moe.modeling_qwen3_5_moe")

T = 7          # positions compared per sequence
B = 2          # sequences stepped together by the oracle


def _copy(param, value):
    with torch.no_grad():
        assert param.shape == value.shape, (param.shape, value.shape)
        param.copy_(value.float())


# ---------------------------------------------------------------------------
# Granite-4.0-H (C5)
# ---------------------------------------------------------------------------
GRANITE_TINY = G.GraniteConfig(hidden=64, layers=4, attention_layers=(1,), mamba_heads=4,
                               mamba_head_dim=16, d_state=16, heads=4, kv_heads=2, head_dim=16,
                               experts=6, top_k=2, moe_inter=32, shared_inter=48, vocab=96)


def granite_hf(cfg, w):
    from transformers.models.granitemoehybrid.configuration_granitemoehybrid import (
        GraniteMoeHybridConfig)
    assert cfg.heads * cfg.head_dim == cfg.hidden
    hc = GraniteMoeHybridConfig(
        vocab_size=cfg.vocab, hidden_size=cfg.hidden, intermediate_size=cfg.moe_inter,
        num_hidden_layers=cfg.layers, num_attention_heads=cfg.heads,
        num_key_value_heads=cfg.kv_heads, rms_norm_eps=cfg.eps, tie_word_embeddings=True,
        embedding_multiplier=cfg.embedding_multiplier, logits_scaling=cfg.logits_scaling,
        residual_multiplier=cfg.residual_multiplier,
        attention_multiplier=cfg.attention_multiplier, num_local_experts=cfg.experts,
        num_experts_per_tok=cfg.top_k, shared_intermediate_size=cfg.shared_inter,
        position_embedding_type=None, max_position_embeddings=64,
        layer_types=["attention" if cfg.is_attention(i) else "mamba" for i in range(cfg.layers)],
        mamba_n_heads=cfg.mamba_heads, mamba_n_groups=1, mamba_d_state=cfg.d_state,
        mamba_d_head=cfg.mamba_head_dim, mamba_d_conv=cfg.conv_kernel,
        mamba_expand=cfg.d_inner // cfg.hidden, mamba_chunk_size=4, mamba_conv_bias=True,
        mamba_proj_bias=False)
    m = hf_g.GraniteMoeHybridForCausalLM(hc).float().eval()
    deq = lambda n: H.fp8_dequant(w[n], w[n + "_scale"] if n + "_scale" in w else
                                  w[n.replace("w_", "s_")])
    E, I, Hd = cfg.experts, cfg.moe_inter, cfg.hidden
    _copy(m.model.embed_tokens.weight, w["embed"])
    _copy(m.model.norm.weight, w["gamma_final"])
    for i, layer in enumerate(m.model.layers):
        p = f"layer{i}."
        _copy(layer.input_layernorm.weight, w[p + "gamma_in"])
        _copy(layer.post_attention_layernorm.weight, w[p + "gamma_post"])
        if cfg.is_attention(i):
            qkv = deq(p + "w_in")
            a = layer.self_attn
            nq, nk = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
            _copy(a.q_proj.weight, qkv[:nq])
            _copy(a.k_proj.weight, qkv[nq:nq + nk])
            _copy(a.v_proj.weight, qkv[nq + nk:nq + 2 * nk])
            _copy(a.o_proj.weight, deq(p + "w_out"))
        else:
            mb = layer.mamba
            _copy(mb.in_proj.weight, deq(p + "w_in"))
            _copy(mb.conv1d.weight, w[p + "conv_w"][:, None, :])
            _copy(mb.conv1d.bias, w[p + "conv_b"])
            _copy(mb.A_log, w[p + "a_log"])
            _copy(mb.dt_bias, w[p + "dt_bias"])
            _copy(mb.D, w[p + "d_skip"])
            _copy(mb.norm.weight, w[p + "gamma_ssm"])
            _copy(mb.out_proj.weight, deq(p + "w_out"))
        moe = layer.block_sparse_moe
        _copy(moe.router.weight, deq(p + "w_router"))
        gate = H.fp8_dequant(w[p + "w_gate"], w[p + "s_gate"]).view(E, I, Hd)
        up = H.fp8_dequant(w[p + "w_up"], w[p + "s_up"]).view(E, I, Hd)
        _copy(moe.experts.gate_up_proj, torch.cat((gate, up), dim=1))
        _copy(moe.experts.down_proj, H.fp8_dequant(w[p + "w_down"], w[p + "s_down"]).view(E, Hd, I))
        _copy(layer.shared_mlp.input_linear.weight, deq(p + "w_shared_in"))
        _copy(layer.shared_mlp.output_linear.weight, deq(p + "w_shared_out"))
    return m


def granite_weights(cfg, seed=0):
    """The engine's synthetic draw with wider weights, and attention q/k/v rows
    scaled up so the scores reach O(1) after the 1/128 multiplier (every term
    of the step then moves the logits)."""
    w = G.synthetic_weights(cfg, seed=seed, device="cpu", std=0.08)
    for i in cfg.attention_layers:
        w[f"layer{i}.w_in_scale"] = w[f"layer{i}.w_in_scale"] * 12.0
    return w


def _granite_oracle_logits(cfg, w, ids):
    orc = H.GraniteOracle(cfg, w, ids.shape[0])
    return torch.stack([orc.step(ids[:, t].tolist()) for t in range(ids.shape[1])], dim=1)


def _rel(a, b):
    return ((a - b).abs().max() / b.abs().max()).item()


@pytest.fixture(scope="module")
def granite_case():
    cfg = GRANITE_TINY
    w = granite_weights(cfg)
    ids = torch.randint(0, cfg.vocab, (B, T), generator=torch.Generator().manual_seed(1))
    m = granite_hf(cfg, w)
    with torch.no_grad():
        want = m(input_ids=ids).logits
    return cfg, w, ids, want


def test_granite_oracle_step_matches_hf_model_in_f32(granite_case):
    cfg, w, ids, want = granite_case
    with H.unrounded():
        got = _granite_oracle_logits(cfg, w, ids)
    err = _rel(got, want)
    print("granite f32 rel err", err, "max |logit|", want.abs().max().item())
    assert err < 2e-4, err


def test_granite_oracle_step_with_bf16_rounding_is_near_hf(granite_case):
    cfg, w, ids, want = granite_case
    got = _granite_oracle_logits(cfg, w, ids)
    err = _rel(got, want)
    print("granite bf16 rel err", err)
    assert err < 5e-2, err


@pytest.mark.parametrize("plant", ["embedding_multiplier", "residual_multiplier",
                                   "attention_multiplier", "logits_scaling", "layer_type"])
def test_granite_pin_fails_on_a_planted_mistake(granite_case, plant):
    cfg, w, ids, want = granite_case
    if plant == "layer_type":
        bad = dataclasses.replace(cfg, attention_layers=(2,))
        w = dict(w)
        for n in [k for k in w if k.startswith("layer1.") or k.startswith("layer2.")]:
            del w[n]
        ref = granite_weights(cfg)
        for n, v in ref.items():          # layer 1 and 2 swap their mixers' weights
            if n.startswith("layer1."):
                w["layer2." + n[7:]] = v
            elif n.startswith("layer2."):
                w["layer1." + n[7:]] = v
    else:
        bad = dataclasses.replace(cfg, **{plant: getattr(cfg, plant) * 2.0})
    with H.unrounded():
        got = _granite_oracle_logits(bad, w, ids)
    assert _rel(got, want) > 1e-2, plant


# ---------------------------------------------------------------------------
# Qwen3.5-35B-A3B (C4)
# ---------------------------------------------------------------------------
QWEN35_TINY = Q.Qwen35Config(hidden=64, layers=4, lin_key_heads=2, lin_value_heads=4,
                             lin_key_dim=16, lin_value_dim=16, heads=4, kv_heads=2, head_dim=32,
                             rot_dim=8, experts=8, top_k=2, moe_inter=32, shared_inter=48,
                             vocab=96)


def qwen35_hf(cfg, w):
    from transformers.models.qwen3_5_moe.configuration_qwen3_5_moe import Qwen3_5MoeTextConfig
    hc = Qwen3_5MoeTextConfig(
        vocab_size=cfg.vocab, hidden_size=cfg.hidden, num_hidden_layers=cfg.layers,
        num_attention_heads=cfg.heads, num_key_value_heads=cfg.kv_heads, head_dim=cfg.head_dim,
        rms_norm_eps=cfg.eps, tie_word_embeddings=False, max_position_embeddings=64,
        rope_parameters={"rope_type": "default", "rope_theta": cfg.rope_theta,
                         "partial_rotary_factor": cfg.rot_dim / cfg.head_dim},
        linear_conv_kernel_dim=cfg.conv_kernel, linear_key_head_dim=cfg.lin_key_dim,
        linear_value_head_dim=cfg.lin_value_dim, linear_num_key_heads=cfg.lin_key_heads,
        linear_num_value_heads=cfg.lin_value_heads, moe_intermediate_size=cfg.moe_inter,
        shared_expert_intermediate_size=cfg.shared_inter, num_experts_per_tok=cfg.top_k,
        num_experts=cfg.experts,
        layer_types=["full_attention" if cfg.is_full(i) else "linear_attention"
                     for i in range(cfg.layers)])
    m = hf_q.Qwen3_5MoeForCausalLM(hc).float().eval()
    one = lambda g: g.float() - 1.0        # HF's RMSNorm multiplies by (1 + weight)
    IS = cfg.shared_inter
    _copy(m.model.embed_tokens.weight, w["embed"])
    _copy(m.model.norm.weight, one(w["gamma_final"]))
    _copy(m.lm_head.weight, w["head"])
    for i, layer in enumerate(m.model.layers):
        p = f"layer{i}."
        _copy(layer.input_layernorm.weight, one(w[p + "gamma_in"]))
        _copy(layer.post_attention_layernorm.weight, one(w[p + "gamma_post"]))
        win = w[p + "w_in"]
        if cfg.is_full(i):
            a = layer.self_attn
            nq, nk = cfg.heads * 2 * cfg.head_dim, cfg.kv_heads * cfg.head_dim
            _copy(a.q_proj.weight, win[:nq])
            _copy(a.k_proj.weight, win[nq:nq + nk])
            _copy(a.v_proj.weight, win[nq + nk:nq + 2 * nk])
            _copy(a.q_norm.weight, one(w[p + "gamma_q"]))
            _copy(a.k_norm.weight, one(w[p + "gamma_k"]))
            _copy(a.o_proj.weight, w[p + "w_out"])
        else:
            g = layer.linear_attn
            c, v, hv = cfg.conv_dim, cfg.value_dim, cfg.lin_value_heads
            _copy(g.in_proj_qkv.weight, win[:c])
            _copy(g.in_proj_z.weight, win[c:c + v])
            _copy(g.in_proj_b.weight, win[c + v:c + v + hv])
            _copy(g.in_proj_a.weight, win[c + v + hv:c + v + 2 * hv])
            _copy(g.conv1d.weight, w[p + "conv_w"][:, None, :])
            _copy(g.A_log, w[p + "a_log"])
            _copy(g.dt_bias, w[p + "dt_bias"])
            _copy(g.norm.weight, w[p + "gamma_gdn"])
            _copy(g.out_proj.weight, w[p + "w_out"])
        moe = layer.mlp
        _copy(moe.gate.weight, w[p + "w_router"])
        _copy(moe.experts.gate_up_proj, torch.cat((w[p + "w_gate"], w[p + "w_up"]), dim=1))
        _copy(moe.experts.down_proj, w[p + "w_down"])
        _copy(moe.shared_expert.gate_proj.weight, w[p + "w_shared_in"][:IS])
        _copy(moe.shared_expert.up_proj.weight, w[p + "w_shared_in"][IS:])
        _copy(moe.shared_expert.down_proj.weight, w[p + "w_shared_out"])
        _copy(moe.shared_expert_gate.weight, w[p + "w_shared_scale"][None])
    return m


def _qwen35_oracle_logits(cfg, w, ids):
    orc = H.Qwen35Oracle(cfg, w, ids.shape[0], max_pos=64)
    return torch.stack([orc.step(ids[:, t].tolist(), [t] * ids.shape[0])
                        for t in range(ids.shape[1])], dim=1)


@pytest.fixture(scope="module")
def qwen35_case():
    cfg = QWEN35_TINY
    w = Q.synthetic_weights(cfg, seed=2, device="cpu", std=0.1)
    ids = torch.randint(0, cfg.vocab, (B, T), generator=torch.Generator().manual_seed(3))
    m = qwen35_hf(cfg, w)
    with torch.no_grad():
        want = m(input_ids=ids).logits
    return cfg, w, ids, want


def test_qwen35_oracle_step_matches_hf_model_in_f32(qwen35_case):
    cfg, w, ids, want = qwen35_case
    with H.unrounded():
        got = _qwen35_oracle_logits(cfg, w, ids)
    err = _rel(got, want)
    print("qwen3.5 f32 rel err", err, "max |logit|", want.abs().max().item())
    assert err < 2e-4, err


def test_qwen35_oracle_step_with_bf16_rounding_is_near_hf(qwen35_case):
    cfg, w, ids, want = qwen35_case
    got = _qwen35_oracle_logits(cfg, w, ids)
    err = _rel(got, want)
    print("qwen3.5 bf16 rel err", err)
    assert err < 5e-2, err


@pytest.mark.parametrize("plant", ["layer_type", "shared_gate", "rope_theta"])
def test_qwen35_pin_fails_on_a_planted_mistake(qwen35_case, plant):
    cfg, w, ids, want = qwen35_case
    w = dict(w)
    if plant == "layer_type":
        bad = dataclasses.replace(cfg, full_every=2)      # layers 1 and 3 full attention
        ref = Q.synthetic_weights(bad, seed=2, device="cpu", std=0.1)
        w.update({k: v for k, v in ref.items() if k.startswith("layer1.")})
    elif plant == "shared_gate":
        bad = cfg
        for i in range(cfg.layers):
            w[f"layer{i}.w_shared_scale"] = torch.zeros_like(w[f"layer{i}.w_shared_scale"])
    else:
        bad = dataclasses.replace(cfg, rope_theta=cfg.rope_theta / 1e4)
    with H.unrounded():
        got = _qwen35_oracle_logits(bad, w, ids)
    assert _rel(got, want) > 1e-3, plant
