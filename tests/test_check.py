"""The ``check`` comparator (``tilefoundry_amd.check``) against the reference's
contract (``src/tilefoundry/runtime/measure.py:61-378``, ``cli/check.py:91-165``).

Each predicate is pinned on inputs whose answer the mathematics fixes (adjacent
floats are one ulp apart, orthogonal vectors have cosine 0, a zero reference has
an absolute L2 distance, NaN fails every bound), and every refusal rule on the
case it exists for.  The command line runs on files here and, on the GPU, runs a
Qwen3 twin function against the oracle's output.
"""
import json
import math

import pytest
import torch
from safetensors.torch import save_file

from tilefoundry_amd import check as K


def _m(pred, a, b=None):
    return pred.measure(torch.as_tensor(a), None if b is None else torch.as_tensor(b))


def test_rel_l2_and_its_zero_reference():
    r = _m(K.RelL2(max=0.25), [3.75, 5.0], [3.0, 4.0])        # |(0.75, 1)| / |(3, 4)|
    assert r.values["rel_l2"] == 0.25 and r.passed
    r = _m(K.RelL2(max=0.5), [0.3, 0.4], [0.0, 0.0])
    assert r.values == {"absolute_l2": pytest.approx(0.5)} and r.note and r.passed
    # one f32 -> bf16 rounding: every element within 2^-9 of itself
    x = torch.randn(4096, generator=torch.Generator().manual_seed(0))
    r = K.RelL2(max=2 ** -9).measure(x.to(torch.bfloat16).float(), x)
    assert r.passed and r.values["rel_l2"] > 2 ** -12


def test_cosine_fixed_points():
    assert _m(K.Cosine(min=0.0), [1.0, 0.0], [0.0, 2.0]).values["cosine"] == 0.0
    assert _m(K.Cosine(min=1.0 - 1e-7), [2.0, 4.0], [1.0, 2.0]).passed
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
    with pytest.raises(ValueError, match="float output"):
        _m(K.Ulp(max=1), torch.tensor([1]), torch.tensor([1]))


def test_max_abs_max_rel_and_allclose():
    assert _m(K.MaxAbs(max=0.5), [1.0, 2.5], [1.0, 2.0]).values["max_abs"] == 0.5
    r = _m(K.MaxRel(max=1.0), [0.0, 3.0], [0.0, 2.0])
    assert r.values["max_rel"] == 0.5 and r.passed
    assert _m(K.MaxRel(max=1e9), [1e-3], [0.0]).values["max_rel"] == math.inf
    ok = _m(K.AllClose(atol=0.1, rtol=0.1), [1.05, 10.9], [1.0, 10.0])
    assert ok.passed and ok.values["max_violation"] == 0.0
    bad = _m(K.AllClose(atol=0.1, rtol=0.0), [1.0, 2.5], [1.0, 2.0])
    assert not bad.passed and bad.values["max_violation"] == pytest.approx(0.4)
    nan = _m(K.AllClose(atol=1.0, rtol=1.0), [float("nan")], [1.0])
    assert not nan.passed


def test_equal_and_nan_inf():
    r = _m(K.Equal(), torch.tensor([1, 2, 3]), torch.tensor([1, 5, 3]))
    assert r.values == {"mismatched": 1.0, "elements": 3.0} and not r.passed
    r = K.NanInf().measure(torch.tensor([1.0, float("nan"), float("inf"), -float("inf")]))
    assert r.values == {"nan": 1.0, "inf": 2.0} and not r.passed


def test_refusals():
    t = torch.ones(3)
    ids = torch.tensor([1, 2])
    with pytest.raises(ValueError, match="no comparison requested"):
        K.compare(t, t, expect={})
    with pytest.raises(ValueError, match="name no output"):
        K.compare(t, t, expect={"output": [K.NanInf()], "output[0]": [K.NanInf()]})
    with pytest.raises(ValueError, match="Use equal"):
        K.compare(ids, ids, expect={"output": [K.RelL2(max=1.0)]})
    assert K.compare(ids, ids, expect={"output": [K.Equal()]}).passed
    with pytest.raises(ValueError, match="no reference"):
        K.compare(t, None, expect={"output": [K.RelL2(max=1.0)]})
    assert K.compare(t, None, expect={"output": [K.NanInf()]}).passed
    with pytest.raises(ValueError, match="structures differ"):
        K.compare((t, t), (t,), expect={"output[0]": [K.NanInf()], "output[1]": [K.NanInf()]})
    with pytest.raises(ValueError, match="shape/dtype"):
        K.compare(t, t.double(), expect={"output": [K.MaxAbs(max=0.0)]})
    with pytest.raises(TypeError):
        K.compare([t], [t], expect={"output": [K.NanInf()]})


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


@pytest.mark.parametrize("stated, msg", [
    ([], "no comparison"),
    ([("fn", "rel_l2")], "before any --out"),
    ([("out", "output"), ("max", 1.0)], "before any --fn"),
    ([("out", "output"), ("fn", "cosine"), ("max", 1.0)], "takes"),
    ([("out", "output"), ("fn", "rel_l2"), ("max", 1.0), ("max", 2.0)], "twice"),
    ([("out", "output"), ("fn", "allclose"), ("atol", 1.0)], "needs"),
    ([("out", "output")], "states no --fn"),
    ([("out", "output"), ("fn", "nan_inf"), ("out", "output")], "given twice"),
])
def test_expectations_parser_refuses(stated, msg):
    with pytest.raises(ValueError, match=msg):
        K.expectations(stated)


def test_expectations_parser_builds_in_order():
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
    assert "PASS  output" in capsys.readouterr().out
    assert K.main(base + ["--fn", "rel_l2", "--max", "1e-5", "--json"]) == 1
    rep = json.loads(capsys.readouterr().out)
    assert not rep["passed"] and rep["outputs"][0]["results"][0]["fn"] == "rel_l2"
    assert K.main(base + ["--fn", "rel_l2"]) == 2          # a bound has no default
    assert "no default" in capsys.readouterr().err
    assert K.main(["--candidate", str(got), "--out", "output", "--fn", "nan_inf"]) == 0


@pytest.mark.gpu
def test_command_line_runs_a_twin_function_against_the_oracle(gpu_device, tmp_path, capsys):
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
