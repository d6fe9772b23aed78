"""The oracle against the committed golden fixtures (tests/golden/make_golden.py).

c1_tiny_fp32.json was written only after the oracle and Hugging Face's
Qwen3ForCausalLM produced the same 32 greedy tokens from the same weights; this
test recomputes the oracle and requires the same tokens and logits.
"""
import json
from pathlib import Path

import torch

from oracle import qwen3_hir as O
from tilefoundry_amd.qwen3 import TINY, synthetic_weights

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_c1_oracle_reproduces_fixture():
    fx = json.loads((GOLDEN / "c1_tiny_fp32.json").read_text())
    assert fx["tokens"] == fx["hf_tokens"]
    w = synthetic_weights(TINY, seed=0)
    g = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, O.C1.vocab, (128,), generator=g).tolist()
    assert prompt == fx["prompt"]
    run = O.decode(O.Qwen3Oracle(O.C1, w), prompt, 32)
    assert run.tokens == fx["tokens"]
    for k, top in enumerate(fx["top16"]):
        for idx, val in top:
            assert abs(float(run.logits[k][idx]) - val) <= 1e-6 * max(1.0, abs(val))


def test_c2_fixture_is_self_consistent():
    """The C2 fixture's recorded picks are the argmax of its recorded top-8."""
    path = GOLDEN / "c2_qwen3_1p7b.json"
    fx = json.loads(path.read_text())
    for norms in ("random", "ones"):
        run = fx[norms]
        assert len(run["tokens"]) == 64
        for tok, top in zip(run["tokens"], run["top8"]):
            best = max(v for _, v in top)
            first = min(i for i, v in top if v == best)
            assert tok == first


def test_c2_order_noise_fixture():
    """The exact-sum fixtures agree with the oracle's own logits to within the
    recorded noise, and the noise is what summation order alone can produce:
    small against the logits, nonzero, and the same picks."""
    import numpy as np

    noise = json.loads((GOLDEN / "c2_order_noise.json").read_text())
    fx = json.loads((GOLDEN / "c2_qwen3_1p7b.json").read_text())
    for norms in ("random", "ones"):
        for k in (0, 63):
            def load(name):
                raw = np.load(GOLDEN / name).astype(np.int16)
                return torch.from_numpy(raw).view(torch.bfloat16).float()
            orc = load(f"c2_{norms}_logits_step{k}.npy")
            ex = load(f"c2_{norms}_exact_step{k}.npy")
            d = float((orc - ex).abs().max())
            assert d == noise[norms][f"step{k}"]["max_abs"]
            assert 0 < d <= 0.05 * float(orc.abs().max())
            # the exact evaluation picks the same token unless the step is a near-tie
            assert int(torch.argmax(ex)) == fx[norms]["tokens"][k] or \
                fx[norms]["margins"][k] <= 2 * d
