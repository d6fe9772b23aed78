"""Checkpoint loading (``tilefoundry_amd.checkpoint``) on the CPU.

The published key names and layouts come from Hugging Face itself: each test
builds the model class the checkpoint belongs to (transformers 5.15, offline,
from a tiny config), copies known weights into it, writes it with
``save_pretrained`` -- the writer that produced the published checkpoints, legacy
key names included (Granite's ``block_sparse_moe.input_linear``) -- and loads the
directory back.  What must come back:

* Qwen3: the canonical dict ``synthetic_weights`` draws, bit for bit, from a
  single file and from a sharded directory with an index; tied and untied
  heads; ``KeyError`` / ``ValueError`` on a missing weight, a wrong shape or a
  wrong dtype (``ir/core/module.py:144-159``).
* Qwen3.5: the engine's synthetic dict bit for bit, through HF's ``1 + gamma``
  storage of every RMSNorm gamma but the gated one.
* Granite: fp8 codes and row scales bit for bit from a checkpoint that stores
  them (``weight_scale`` beside each fp8 weight), and from a bf16 checkpoint the
  per-row quantisation, whose dequantised values are within half an e4m3 step of
  the stored weights.
"""
import json

import pytest
import torch
from safetensors.torch import save_file

from tilefoundry_amd import checkpoint as C
from tilefoundry_amd.hybrid import granite as G
from tilefoundry_amd.hybrid import qwen3_5 as Q
from tilefoundry_amd.qwen3 import TINY, synthetic_weights
from tilefoundry_amd.qwen3.weights import rows

transformers = pytest.importorskip("transformers")


def _qwen3_hf(cfg, w, tied=True):
    hc = transformers.Qwen3Config(
        vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size,
        intermediate_size=cfg.intermediate_size, num_hidden_layers=cfg.num_hidden_layers,
        num_attention_heads=cfg.num_attention_heads, num_key_value_heads=cfg.num_key_value_heads,
        head_dim=cfg.head_dim, rms_norm_eps=cfg.rms_norm_eps, tie_word_embeddings=tied,
        rope_parameters={"rope_type": "default", "rope_theta": cfg.rope_theta},
        max_position_embeddings=cfg.max_position_embeddings)
    m = transformers.Qwen3ForCausalLM(hc).to(torch.bfloat16)
    sd = {"model.embed_tokens.weight": w["w_embed"], "model.norm.weight": w["gamma_final"]}
    if not tied:
        sd["lm_head.weight"] = rows(w["w_head"])
    for i in range(cfg.num_hidden_layers):
        for name, (key, proj) in C.QWEN3_LAYER_KEYS.items():
            t = w[f"layer{i}.{name}"]
            sd[f"model.layers.{i}.{key}"] = rows(t) if proj else t
    missing, unexpected = m.load_state_dict({k: v.contiguous() for k, v in sd.items()},
                                            strict=False)
    assert not unexpected and set(missing) <= {"lm_head.weight"}, (missing, unexpected)
    return m


@pytest.fixture(scope="module")
def qwen3_case():
    cfg = TINY.with_(dtype=torch.bfloat16)
    return cfg, synthetic_weights(cfg, seed=5)


def _same(a, b):
    assert set(a) == set(b), set(a) ^ set(b)
    for n in a:
        assert a[n].shape == b[n].shape and a[n].dtype == b[n].dtype, n
        assert torch.equal(a[n], b[n]), n


@pytest.mark.parametrize("shards", ["single", "sharded"])
def test_qwen3_checkpoint_reproduces_the_weights(tmp_path, qwen3_case, shards):
    cfg, w = qwen3_case
    _qwen3_hf(cfg, w).save_pretrained(tmp_path, max_shard_size="40KB" if shards == "sharded"
                                      else "10GB")
    assert (tmp_path / "model.safetensors.index.json").is_file() == (shards == "sharded")
    got_cfg, got = C.load_qwen3(tmp_path)
    assert got_cfg == cfg
    _same(got, w)
    # the tied head is the table itself, as synthetic_weights draws it
    assert got["w_head"].data_ptr() == got["w_embed"].data_ptr()


def test_qwen3_untied_head(tmp_path, qwen3_case):
    cfg, w = qwen3_case
    w = dict(w)
    w["w_head"] = synthetic_weights(cfg, seed=6)["w_embed"].t()
    _qwen3_hf(cfg, w, tied=False).save_pretrained(tmp_path)
    got_cfg, got = C.load_qwen3(tmp_path)
    assert not got_cfg.tie_word_embeddings
    assert torch.equal(got["w_head"], w["w_head"])


def _qwen3_raw(tmp_path, cfg, w, edit):
    """A hand-written single-file checkpoint with one entry edited."""
    sd = {"model.embed_tokens.weight": w["w_embed"], "model.norm.weight": w["gamma_final"]}
    for i in range(cfg.num_hidden_layers):
        for name, (key, proj) in C.QWEN3_LAYER_KEYS.items():
            t = w[f"layer{i}.{name}"]
            sd[f"model.layers.{i}.{key}"] = rows(t) if proj else t
    edit(sd)
    save_file({k: v.contiguous() for k, v in sd.items()}, str(tmp_path / "model.safetensors"))
    (tmp_path / "config.json").write_text(json.dumps({
        "hidden_size": cfg.hidden_size, "num_attention_heads": cfg.num_attention_heads,
        "num_key_value_heads": cfg.num_key_value_heads, "head_dim": cfg.head_dim,
        "intermediate_size": cfg.intermediate_size, "vocab_size": cfg.vocab_size,
        "num_hidden_layers": cfg.num_hidden_layers, "rms_norm_eps": cfg.rms_norm_eps,
        "rope_theta": cfg.rope_theta, "tie_word_embeddings": True, "torch_dtype": "bfloat16"}))


def test_qwen3_rejects_a_missing_a_misshapen_and_a_mistyped_weight(tmp_path, qwen3_case):
    cfg, w = qwen3_case
    key = "model.layers.1.mlp.up_proj.weight"
    cases = {
        "missing": (lambda sd: sd.pop(key), KeyError),
        "shape": (lambda sd: sd.__setitem__(key, sd[key][:-1]), ValueError),
        "dtype": (lambda sd: sd.__setitem__(key, sd[key].float()), ValueError),
    }
    for name, (edit, err) in cases.items():
        d = tmp_path / name
        d.mkdir()
        _qwen3_raw(d, cfg, w, edit)
        with pytest.raises(err):
            C.load_qwen3(d)
    d = tmp_path / "empty"
    d.mkdir()
    with pytest.raises(FileNotFoundError):
        C.load_qwen3(d)


def test_qwen3_5_checkpoint_reproduces_the_engine_weights(tmp_path):
    from tests.test_oracle_hybrid_models import QWEN35_TINY, qwen35_hf

    cfg = QWEN35_TINY
    w = Q.synthetic_weights(cfg, seed=2, device="cpu", std=0.1)
    qwen35_hf(cfg, w).to(torch.bfloat16).save_pretrained(tmp_path)
    got_cfg, got = C.load_qwen3_5(tmp_path)
    assert got_cfg == cfg
    _same(got, w)


def _without_head(tmp_path, tie: bool):
    """A Qwen3.5 checkpoint with lm_head.weight removed and tie_word_embeddings
    set to *tie*."""
    import json

    from safetensors import safe_open
    from tests.test_oracle_hybrid_models import QWEN35_TINY, qwen35_hf

    cfg = QWEN35_TINY
    w = Q.synthetic_weights(cfg, seed=2, device="cpu", std=0.1)
    qwen35_hf(cfg, w).to(torch.bfloat16).save_pretrained(tmp_path)
    for path in tmp_path.glob("*.safetensors"):
        with safe_open(str(path), "pt") as f:
            sd = {k: f.get_tensor(k) for k in f.keys() if k != "lm_head.weight"}
        save_file(sd, str(path))
    index = tmp_path / "model.safetensors.index.json"
    if index.exists():
        d = json.loads(index.read_text())
        d["weight_map"].pop("lm_head.weight", None)
        index.write_text(json.dumps(d))
    conf = tmp_path / "config.json"
    d = json.loads(conf.read_text())
    if "text_config" in d:
        d["text_config"]["tie_word_embeddings"] = tie
    d["tie_word_embeddings"] = tie
    conf.write_text(json.dumps(d))
    return cfg, w


def test_qwen3_5_missing_head_is_refused_unless_tied(tmp_path):
    """Qwen3.5-MoE does not tie its embeddings: a checkpoint without
    lm_head.weight is an error, unless its config says the embeddings are tied
    (then the head is the embedding table)."""
    (tmp_path / "untied").mkdir()
    _without_head(tmp_path / "untied", tie=False)
    with pytest.raises(KeyError, match="not tied"):
        C.load_qwen3_5(tmp_path / "untied")
    (tmp_path / "tied").mkdir()
    _, w = _without_head(tmp_path / "tied", tie=True)
    _, got = C.load_qwen3_5(tmp_path / "tied")
    assert torch.equal(got["head"], got["embed"])


def test_qwen3_5_gamma_converter_is_one_plus_the_stored_delta():
    stored = torch.tensor([-0.5, -0.0078125, 0.0, 0.25, 0.9921875], dtype=torch.bfloat16)
    assert torch.equal(C._plus_one(stored),
                       torch.tensor([0.5, 0.9921875, 1.0, 1.25, 1.9921875], dtype=torch.bfloat16))


def _granite_saved(tmp_path, cfg, w):
    from tests.test_oracle_hybrid_models import granite_hf

    granite_hf(cfg, w).to(torch.bfloat16).save_pretrained(tmp_path)


def test_granite_fp8_checkpoint_reproduces_the_engine_weights(tmp_path):
    """A checkpoint holding fp8 codes with their row scales (the stored form of
    an fp8 export): every linear comes back as the same codes and scales."""
    from tests.test_oracle_hybrid_models import GRANITE_TINY, granite_weights

    cfg = GRANITE_TINY
    w = granite_weights(cfg)
    _granite_saved(tmp_path, cfg, w)
    # replace every linear weight by its fp8 codes and scales
    path = tmp_path / "model.safetensors"
    from safetensors import safe_open
    with safe_open(str(path), "pt") as f:
        sd = {k: f.get_tensor(k) for k in f.keys()}
    E, I, Hd = cfg.experts, cfg.moe_inter, cfg.hidden
    nq, nk = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim

    def put(key, codes, scale):
        sd[key] = codes.view(torch.float8_e4m3fn)
        sd[key[: -len("weight")] + "weight_scale"] = scale.float().reshape(-1, 1)

    for i in range(cfg.layers):
        p, k = f"layer{i}.", f"model.layers.{i}."
        if cfg.is_attention(i):
            c, s = w[p + "w_in"], w[p + "w_in_scale"]
            put(k + "self_attn.q_proj.weight", c[:nq], s[:nq])
            put(k + "self_attn.k_proj.weight", c[nq:nq + nk], s[nq:nq + nk])
            put(k + "self_attn.v_proj.weight", c[nq + nk:], s[nq + nk:])
            put(k + "self_attn.o_proj.weight", w[p + "w_out"], w[p + "w_out_scale"])
        else:
            put(k + "mamba.in_proj.weight", w[p + "w_in"], w[p + "w_in_scale"])
            put(k + "mamba.out_proj.weight", w[p + "w_out"], w[p + "w_out_scale"])
        put(k + "block_sparse_moe.router.layer.weight", w[p + "w_router"], w[p + "w_router_scale"])
        gu = torch.cat((w[p + "w_gate"].view(E, I, Hd), w[p + "w_up"].view(E, I, Hd)), dim=1)
        gs = torch.cat((w[p + "s_gate"].view(E, I), w[p + "s_up"].view(E, I)), dim=1)
        put(k + "block_sparse_moe.input_linear.weight", gu, gs)
        put(k + "block_sparse_moe.output_linear.weight", w[p + "w_down"].view(E, Hd, I),
            w[p + "s_down"])
        put(k + "shared_mlp.input_linear.weight", w[p + "w_shared_in"], w[p + "w_shared_in_scale"])
        put(k + "shared_mlp.output_linear.weight", w[p + "w_shared_out"],
            w[p + "w_shared_out_scale"])
    save_file(sd, str(path))
    got_cfg, got = C.load_granite(tmp_path)
    assert got_cfg == cfg
    _same(got, {n: (t.float() if n.endswith("_scale") or n.split(".")[-1].startswith("s_")
                    else t) for n, t in w.items()})


def test_granite_bf16_checkpoint_is_quantised_per_row(tmp_path):
    from oracle import hybrid_ref as H
    from tests.test_oracle_hybrid_models import GRANITE_TINY, granite_weights

    cfg = GRANITE_TINY
    w = granite_weights(cfg)
    _granite_saved(tmp_path, cfg, w)
    got_cfg, got = C.load_granite(tmp_path)
    assert got_cfg == cfg
    assert set(got) == set(w)
    for n, t in w.items():
        if t.dtype != torch.uint8:
            if not (n.endswith("_scale") or n.split(".")[-1].startswith("s_")):
                assert torch.equal(got[n], t), n
            continue
        sname = n + "_scale" if n + "_scale" in w else n.replace("w_", "s_")
        want = H.fp8_dequant(t, w[sname]).to(torch.bfloat16).float()   # what the file stores
        have = H.fp8_dequant(got[n], got[sname])
        # e4m3 keeps 3 mantissa bits: half a step is 1/16 of the value's binade
        assert (have - want).abs().le(want.abs() / 16 + got[sname][:, None] * 2 ** -9).all(), n
        assert got[sname].dtype == torch.float32 and got[n].shape == t.shape


def test_quantize_rows_fp8_uses_the_full_e4m3_range():
    w = torch.tensor([[0.0, 1.0, -2.0, 0.5], [0.0, 0.0, 0.0, 0.0], [3.0, -448.0, 1e-3, 7.0]])
    codes, scale = C.quantize_rows_fp8(w)
    assert torch.equal(scale, torch.tensor([2.0 / 448, 1.0, 1.0]))
    back = codes.view(torch.float8_e4m3fn).float() * scale[:, None]
    assert back[:, :2].abs().max(dim=1).values.tolist()[1] == 0.0
    assert back[0].abs().max() == 2.0 and back[2, 1] == -448.0
