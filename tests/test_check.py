"""The ``check`` comparator (``tilefoundry_amd.check``) against the contract of
the reference's (``src/tilefoundry/runtime/measure.py:61-378``,
``cli/check.py:91-165, 532-648``): its eight functions, bounds, reported
quantities and refusals.

Each function is pinned on inputs whose answer the mathematics fixes (adjacent
floats are one ulp apart, orthogonal vectors have cosine 0, a zero reference
gives an absolute L2 distance, NaN fails every bound), and every refusal on the
case it exists for.  The command line runs on files here and, on the GPU, runs
a Qwen3, a Qwen3.5 and a Granite twin function against the oracle's output.
"""
import json
import math

import pytest
import torch
from safetensors.torch import save_file

from tilefoundry_amd import check as K


def _m(req, a, b=None):
    return req.measure(torch.as_tensor(a), None if b is None else torch.as_tensor(b))


def test_rel_l2_and_its_zero_reference():
    r = _m(K.RelL2(max=0.25), [3.75, 5.0], [3.0, 4.0])        # |(0.75, 1)| / |(3, 4)|
    assert r.values["rel_l2"] == 0.25 and r.passed
    r = _m(K.RelL2(max=5.0), [3.0, 4.0], [0.0, 0.0])
    assert r.values == {"absolute_l2": 5.0} and r.note and r.passed
    # one f32 -> bf16 rounding: every element within 2^-9 of itself
    x = torch.randn(4096, generator=torch.Generator().manual_seed(0))
    r = K.RelL2(max=2 ** -9).measure(x.to(torch.bfloat16).float(), x)
    assert r.passed and r.values["rel_l2"] > 2 ** -12


def test_cosine_fixed_points():
    assert _m(K.Cosine(min=0.0), [1.0, 0.0], [0.0, 2.0]).values["cosine"] == 0.0
    assert _m(K.Cosine(min=1.0 - 1e-12), [2.0, 4.0], [1.0, 2.0]).passed
    assert _m(K.Cosine(min=-1.0), [0.0, 2.0], [0.0, -3.0]).values["cosine"] == -1.0
    both = _m(K.Cosine(min=1.0), [0.0, 0.0], [0.0, 0.0])
    assert both.passed and both.note
    one = _m(K.Cosine(min=-1.0), [0.0, 0.0], [1.0, 0.0])
    assert not one.passed and one.values["cosine"] == 0.0


def test_ulp_counts_representable_values():
    one = torch.tensor([1.0])
    nxt = torch.nextafter(one, torch.tensor([2.0]))
    assert _m(K.Ulp(max=1), nxt, one).values["max_ulp"] == 1
    tiny = torch.tensor([1e-45])                       # the smallest f32 subnormal
    assert _m(K.Ulp(max=2), tiny, -tiny).values["max_ulp"] == 2
    assert _m(K.Ulp(max=0), torch.tensor([0.0]), torch.tensor([-0.0])).passed
    b = torch.tensor([1.0], dtype=torch.bfloat16)
    assert _m(K.Ulp(max=1), torch.tensor([1.0078125], dtype=torch.bfloat16), b).values[
        "max_ulp"] == 1
    # across zero in f64: the two smallest subnormals of either sign are 2 apart
    d = torch.tensor([5e-324], dtype=torch.float64)
    assert _m(K.Ulp(max=2), d, -d).values["max_ulp"] == 2
    # 2^k and its predecessor are one apart whatever the binade
    for dtype in (torch.float16, torch.bfloat16, torch.float32, torch.float64):
        p = torch.tensor([-8.0], dtype=dtype)
        q = torch.nextafter(p.float(), torch.tensor([0.0])).to(dtype) if dtype in (
            torch.float16, torch.bfloat16) else torch.nextafter(p, torch.zeros_like(p))
        if dtype in (torch.float16, torch.bfloat16):
            # the f32 neighbour rounds back onto p in a narrower type; step by the bits
            q = (p.view(torch.int16) - 1).view(dtype)
        assert _m(K.Ulp(max=1), q, p).values["max_ulp"] == 1, dtype
    with pytest.raises(ValueError, match="float output"):
        _m(K.Ulp(max=1), torch.tensor([1]), torch.tensor([1]))


def test_max_abs_max_rel_and_allclose():
    assert _m(K.MaxAbs(max=0.5), [1.0, 2.5], [1.0, 2.0]).values["max_abs"] == 0.5
    r = _m(K.MaxRel(max=1.0), [0.0, 3.0], [0.0, 2.0])
    assert r.values["max_rel"] == 0.5 and r.passed
    assert _m(K.MaxRel(max=1e9), [1e-3], [0.0]).values["max_rel"] == math.inf
    assert not _m(K.MaxRel(max=1e9), [float("nan")], [1.0]).passed
    ok = _m(K.AllClose(atol=0.1, rtol=0.1), [1.05, 10.9], [1.0, 10.0])
    assert ok.passed and ok.values["max_violation"] == 0.0
    bad = _m(K.AllClose(atol=0.1, rtol=0.0), [1.0, 2.5], [1.0, 2.0])
    assert not bad.passed and bad.values["max_violation"] == pytest.approx(0.4)
    nan = _m(K.AllClose(atol=1.0, rtol=1.0), [float("nan")], [1.0])
    assert not nan.passed


def test_equal_and_nan_inf():
    r = _m(K.Equal(), torch.tensor([1, 2, 3]), torch.tensor([1, 5, 3]))
    assert r.values == {"mismatched": 1.0, "elements": 3.0} and not r.passed
    # floats compare by bit pattern: the same NaN is equal, +0 and -0 are not
    assert _m(K.Equal(), [float("nan")], [float("nan")]).passed
    assert not _m(K.Equal(), [0.0], [-0.0]).passed
    r = K.NanInf().measure(torch.tensor([1.0, float("nan"), float("inf"), -float("inf")]))
    assert r.values == {"nan": 1.0, "inf": 2.0} and not r.passed


def test_a_requirement_carries_every_bound():
    with pytest.raises(ValueError, match="bounded by exactly"):
        K.Requirement("allclose", (("atol", 1.0),))
    with pytest.raises(ValueError, match="not a comparison function"):
        K.Requirement("close_enough")
    assert K.AllClose(atol=1, rtol=2).bounds == {"atol": 1.0, "rtol": 2.0}


def test_refusals():
    t = torch.ones(3)
    ids = torch.tensor([1, 2])
    with pytest.raises(ValueError, match="no default bound"):
        K.compare(t, t, expect={})
    with pytest.raises(ValueError, match="did not produce"):
        K.compare(t, t, expect={"output": [K.NanInf()], "output[0]": [K.NanInf()]})
    with pytest.raises(ValueError, match="with equal"):
        K.compare(ids, ids, expect={"output": [K.RelL2(max=1.0)]})
    assert K.compare(ids, ids, expect={"output": [K.Equal()]}).passed
    with pytest.raises(ValueError, match="there is none"):
        K.compare(t, None, expect={"output": [K.RelL2(max=1.0)]})
    assert K.compare(t, None, expect={"output": [K.NanInf()]}).passed
    with pytest.raises(ValueError, match="do not line up"):
        K.compare((t, t), (t,), expect={"output[0]": [K.NanInf()], "output[1]": [K.NanInf()]})
    with pytest.raises(ValueError, match="differs in form"):
        K.compare(t, t.double(), expect={"output": [K.MaxAbs(max=0.0)]})
    with pytest.raises(TypeError):
        K.compare([t], [t], expect={"output": [K.NanInf()]})


def test_nested_outputs_are_addressed_by_position():
    t = torch.zeros(2)
    got = [p for p, _ in K.leaves((t, (t, (t,)), t))]
    assert got == ["output[0]", "output[1][0]", "output[1][1][0]", "output[2]"]


def test_check_runs_both_sides_on_the_same_inputs():
    seen = []

    def cand(x, y):
        seen.append(("c", x, y))
        return (x + y, (x * y).to(torch.int64))

    def ref(x, y):
        seen.append(("r", x, y))
        return (x + y + 1e-4, (x * y).to(torch.int64))

    x, y = torch.arange(4.0), torch.full((4,), 2.0)
    rep = K.check(cand, ref, (x, y), expect={"output[0]": [K.MaxAbs(max=1e-3)],
                                             "output[1]": [K.Equal()]})
    assert rep.passed and [s[0] for s in seen] == ["c", "r"]
    assert seen[0][1] is seen[1][1]
    # a requirement set that cannot hold is refused before the reference runs
    seen.clear()
    with pytest.raises(ValueError):
        K.check(cand, ref, (x, y), expect={"output[0]": [K.MaxAbs(max=1.0)]})
    assert [s[0] for s in seen] == ["c"]


@pytest.mark.parametrize("stated, msg", [
    ([], "no comparison stated"),
    ([("fn", "rel_l2")], "no output before it"),
    ([("out", "output"), ("max", 1.0)], "no --fn before it"),
    ([("out", "output"), ("fn", "cosine"), ("max", 1.0)], "does not bound"),
    ([("out", "output"), ("fn", "rel_l2"), ("max", 1.0), ("max", 2.0)], "twice"),
    ([("out", "output"), ("fn", "allclose"), ("atol", 1.0)], "missing --rtol"),
    ([("out", "output")], "names no --fn"),
    ([("out", "output"), ("fn", "nan_inf"), ("out", "output")], "more than once"),
])
def test_expectations_reader_refuses(stated, msg):
    with pytest.raises(ValueError, match=msg):
        K.expectations(stated)


def test_expectations_reader_builds_in_order():
    got = K.expectations([("out", "output[0]"), ("fn", "allclose"), ("rtol", 0.01),
                          ("atol", 0.001), ("fn", "nan_inf"), ("out", "output[1]"),
                          ("fn", "equal")])
    assert got == {"output[0]": (K.AllClose(atol=0.001, rtol=0.01), K.NanInf()),
                   "output[1]": (K.Equal(),)}


def test_command_line_on_files(tmp_path, capsys):
    g = torch.Generator().manual_seed(1)
    x = torch.randn(64, 32, generator=g)
    want = tmp_path / "want.safetensors"
    got = tmp_path / "got.safetensors"
    save_file({"a": x.to(torch.bfloat16)}, str(want))
    save_file({"a": (x * (1 + 1e-3)).to(torch.bfloat16)}, str(got))
    base = ["--candidate", str(got), "--expected", str(want), "--out", "output"]
    assert K.main(base + ["--fn", "rel_l2", "--max", "4e-3", "--fn", "cosine",
                          "--min", "0.9999"]) == 0
    assert "output: bfloat16 [64, 32]" in capsys.readouterr().out
    assert K.main(base + ["--fn", "rel_l2", "--max", "1e-5", "--json"]) == 1
    rep = json.loads(capsys.readouterr().out)
    assert not rep["passed"]
    fn = rep["outputs"][0]["fns"][0]
    assert fn["fn"] == "rel_l2" and fn["max"] == 1e-5 and not fn["passed"] and "rel_l2" in fn
    assert K.main(base + ["--fn", "rel_l2"]) == 2          # a bound has no default
    assert "no default" in capsys.readouterr().err
    assert K.main(["--candidate", str(got), "--out", "output", "--fn", "nan_inf"]) == 0
    assert K.main(["qwen3_7:embed", "--out", "output", "--fn", "nan_inf"]) == 2
    assert "qwen3_5:<selector>" in capsys.readouterr().err


@pytest.mark.gpu
def test_command_line_runs_a_qwen3_twin_function_against_the_oracle(gpu_device, tmp_path,
                                                                     capsys):
    """``qwen3:layer1.mlp`` of a self-written checkpoint, the HIP twin against
    the oracle's ``mlp`` on the same weights and hidden state."""
    from oracle import qwen3_hir as O
    from tests.test_checkpoint import _qwen3_hf
    from tilefoundry_amd.qwen3 import TINY, synthetic_weights

    cfg = TINY.with_(dtype=torch.bfloat16)
    w = synthetic_weights(cfg, seed=4)
    _qwen3_hf(cfg, w).save_pretrained(tmp_path)
    hidden = torch.randn(1, 1, cfg.hidden_size, generator=torch.Generator().manual_seed(2))
    hidden = hidden.to(torch.bfloat16)
    dims = O.Qwen3Dims(hidden=cfg.hidden_size, heads=cfg.num_attention_heads,
                       kv_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim,
                       intermediate=cfg.intermediate_size, vocab=cfg.vocab_size,
                       layers=cfg.num_hidden_layers, dtype=cfg.dtype)
    with torch.no_grad():
        want = O.mlp(dims, hidden, *[w[f"layer1.{n}"] for n in
                                     ("gamma_post", "w_gate", "w_up", "w_down")])
    save_file({"hidden": hidden}, str(tmp_path / "hidden.safetensors"))
    save_file({"out": want.contiguous()}, str(tmp_path / "want.safetensors"))
    print("[check] qwen3:layer1.mlp", flush=True)
    capsys.readouterr()
    rc = K.main(["qwen3:layer1.mlp", "--ckpt", str(tmp_path), "--device", gpu_device,
                 "--input", str(tmp_path / "hidden.safetensors"),
                 "--expected", str(tmp_path / "want.safetensors"),
                 "--out", "output", "--fn", "rel_l2", "--max", "8e-3", "--fn", "cosine",
                 "--min", "0.9999", "--fn", "nan_inf"])
    out = capsys.readouterr().out
    print(out)
    assert rc == 0, out


@pytest.mark.gpu
def test_command_line_runs_a_qwen3_5_twin_function_against_the_oracle(gpu_device, tmp_path,
                                                                       capsys):
    """``qwen3_5:layer0.mixer.linear_attention`` (a gated-DeltaNet layer) of a
    four-layer Qwen3.5 checkpoint at the model's widths: its three outputs -- the
    mixer output, the conv window entry and the updated f32 state -- against the
    oracle's gated-DeltaNet step on the checkpoint's weights."""
    from oracle import hybrid_ref as H
    from tests.test_oracle_hybrid_models import qwen35_hf
    from tilefoundry_amd.checkpoint import load_qwen3_5
    from tilefoundry_amd.hybrid.qwen3_5 import Qwen35Config
    from tilefoundry_amd.hybrid.qwen3_5 import synthetic_weights

    cfg = Qwen35Config(layers=4, experts=8, vocab=4096)
    qwen35_hf(cfg, synthetic_weights(cfg, seed=7, device="cpu")).to(
        torch.bfloat16).save_pretrained(tmp_path)
    _, w = load_qwen3_5(tmp_path)
    f = lambda t: t.float()                                       # noqa: E731
    g = torch.Generator().manual_seed(8)
    hidden = torch.randn(1, 1, cfg.hidden, generator=g)
    conv = H.bf(torch.randn(1, cfg.conv_dim, 3, generator=g))
    state = torch.randn(1, cfg.lin_value_heads, cfg.lin_key_dim, cfg.lin_value_dim,
                        generator=g) * 0.05
    xn = H.bf(H._rms_flat(hidden[0], f(w["layer0.gamma_in"]), cfg.eps))
    proj = H.bf(H.mm_rows(f(w["layer0.w_in"]), xn))
    gated, _, want_state = H.gdn_step(
        proj, conv, state, f(w["layer0.conv_w"]), f(w["layer0.a_log"]), f(w["layer0.dt_bias"]),
        f(w["layer0.gamma_gdn"]), hk=cfg.lin_key_heads, hv=cfg.lin_value_heads,
        dk=cfg.lin_key_dim, dv=cfg.lin_value_dim, rms_eps=cfg.eps)
    want_out = H.bf(H.mm_rows(f(w["layer0.w_out"]), H.bf(gated)))[None]
    want_entry = proj[:, :cfg.conv_dim, None]
    for name, t in (("hidden", hidden), ("conv", conv), ("state", state)):
        save_file({"t": t.contiguous()}, str(tmp_path / f"{name}.safetensors"))
    # the twin hands back (out f32, entry f32, state f32) as authored
    save_file({"0": want_out.float().contiguous(), "1": want_entry.float().contiguous(),
               "2": want_state.float().contiguous()}, str(tmp_path / "want.safetensors"))
    print("[check] qwen3_5:layer0.mixer.linear_attention", flush=True)
    capsys.readouterr()
    rc = K.main(["qwen3_5:layer0.mixer.linear_attention", "--ckpt", str(tmp_path),
                 "--device", gpu_device,
                 *[a for n in ("hidden", "conv", "state")
                   for a in ("--input", str(tmp_path / f"{n}.safetensors"))],
                 "--expected", str(tmp_path / "want.safetensors"),
                 "--out", "output[0]", "--fn", "rel_l2", "--max", "2e-2", "--fn", "cosine",
                 "--min", "0.999",
                 "--out", "output[1]", "--fn", "rel_l2", "--max", "1e-2",
                 "--out", "output[2]", "--fn", "rel_l2", "--max", "1e-3", "--fn", "nan_inf"])
    out = capsys.readouterr().out
    print(out)
    assert rc == 0, out


@pytest.mark.gpu
def test_command_line_runs_a_granite_twin_function_against_the_oracle(gpu_device, tmp_path,
                                                                       capsys):
    """``granite:layer0.moe.routing`` of a two-layer Granite checkpoint (hidden
    1,024, 24 experts, top 10): the expert ids judged by ``equal`` (a discrete
    output) and their softmax weights to the bf16 bar, against the oracle's
    router on the checkpoint's (fp8-quantised, dequantised) router weights."""
    from oracle import hybrid_ref as H
    from tests.test_oracle_hybrid_models import granite_hf
    from tilefoundry_amd.checkpoint import load_granite
    from tilefoundry_amd.hybrid import twin as T
    from tilefoundry_amd.hybrid.granite import GraniteConfig
    from tilefoundry_amd.hybrid.granite import synthetic_weights

    cfg = GraniteConfig(hidden=1024, layers=2, attention_layers=(1,), mamba_heads=16, heads=8,
                        kv_heads=2, experts=24, top_k=10, moe_inter=256, shared_inter=512,
                        vocab=4096)
    granite_hf(cfg, synthetic_weights(cfg, seed=9, device="cpu")).to(
        torch.bfloat16).save_pretrained(tmp_path)
    got_cfg, w = load_granite(tmp_path)
    can = T.granite_canonical(got_cfg, w)
    router = can["layer0.moe.router.w_router"].float().cpu()
    tokens = H.bf(torch.randn(3, cfg.hidden, generator=torch.Generator().manual_seed(10)))
    want_w, want_i = H.route_topk_softmax(H.bf(H.mm_rows(router, tokens)), cfg.top_k)
    save_file({"t": tokens.to(torch.bfloat16).contiguous()}, str(tmp_path / "tokens.safetensors"))
    save_file({"0": want_w.to(torch.bfloat16).contiguous(), "1": want_i.contiguous()},
              str(tmp_path / "want.safetensors"))
    print("[check] granite:layer0.moe.routing", flush=True)
    capsys.readouterr()
    rc = K.main(["granite:layer0.moe.routing", "--ckpt", str(tmp_path), "--device", gpu_device,
                 "--input", str(tmp_path / "tokens.safetensors"),
                 "--expected", str(tmp_path / "want.safetensors"),
                 "--out", "output[0]", "--fn", "max_rel", "--max", str(2 ** -7),
                 "--out", "output[1]", "--fn", "equal"])
    out = capsys.readouterr().out
    print(out)
    assert rc == 0, out
