"""The Granite-style hybrid decode engine (workload C5: fp8 weights, Mamba2 +
GQA, top-k-then-softmax MoE) against the oracle's whole-step composition on the
GPU, at the model's real widths with three layers (Mamba2, GQA, Mamba2) and a
4,096-token vocabulary so the CPU oracle runs in seconds: 12 experts (top 4),
and the workload's 72 (top 10) at batch 1 and 8.  Teacher-forced on the engine's
own tokens and, at router near-ties, on its routing (tests/_hybrid_steps.py):
every step's logits within 5e-2 of max |logit| (the workload's fp8 bound), greedy
picks equal where the oracle's top-2 margin exceeds twice the step's error.
C5's residual stream is bf16 with every op rounded (the HIR policy), so the
engine's router inputs sit a bf16 ulp from the oracle's wherever a rounding went
the other way; a router logit, a 4,096-long sum of them, then moves by up to a
few ulps, and routing is followed for swaps within 4 ulps of the k-th logit (2
for C4's f32 stream).  The widest swap of each run is printed."""
import pytest
import torch

from oracle import hybrid_ref as H
from tests._hybrid_steps import check_steps, feed_of
from tilefoundry_amd.hybrid.granite import GraniteConfig, GraniteEngine, synthetic_weights

pytestmark = pytest.mark.gpu


def _run(dev, cfg, rows, *, seed, prompts, new):
    w = synthetic_weights(cfg, seed=seed, device=dev)
    eng = GraniteEngine(cfg, w, rows=rows, device=dev, max_steps=64, split_len=16,
                        record_routes=True)
    tokens, _, logits = eng.generate(prompts, new, record_logits=True)
    steps = max(len(p) for p in prompts) - 1 + new
    assert logits.shape[0] == steps
    feed = feed_of(eng, prompts, steps)
    assert all(tokens[b] == feed[b][len(p):len(p) + new] for b, p in enumerate(prompts))
    orc = H.GraniteOracle(cfg, {k: v.cpu() for k, v in w.items()}, rows)
    orc.route_slack = 4.0
    return check_steps(orc, lambda t, tok, r: orc.step(tok, routes=r), logits,
                       eng.route_history, feed, prompts, 5e-2)


@pytest.mark.parametrize("rows", [1, 2])
def test_granite_engine_matches_oracle_steps(gpu_device, rows):
    cfg = GraniteConfig(layers=3, attention_layers=(1,), experts=12, top_k=4, vocab=4096)
    g = torch.Generator().manual_seed(10 + rows)
    prompts = [torch.randint(0, cfg.vocab, (3 + b,), generator=g).tolist() for b in range(rows)]
    _run(gpu_device, cfg, rows, seed=5, prompts=prompts, new=3)


@pytest.mark.parametrize("rows", [1, 8])
def test_granite_engine_at_full_expert_width(gpu_device, rows):
    """The workload's MoE width: 72 fp8 experts, top 10 then softmax, plus the
    shared MLP, at batch 1 and the workload's batch 8, over 8 generated steps;
    routing followed at near-ties (the count is printed), the logits bound the
    workload's at every step."""
    cfg = GraniteConfig(layers=3, attention_layers=(1,), experts=72, top_k=10, vocab=4096)
    g = torch.Generator().manual_seed(40 + rows)
    prompts = [torch.randint(0, cfg.vocab, (3 + b % 3,), generator=g).tolist()
               for b in range(rows)]
    _, picks, _ = _run(gpu_device, cfg, rows, seed=13, prompts=prompts, new=8)
    assert picks >= rows * 2


def test_granite_prefill_is_the_walk(gpu_device):
    """GraniteEngine.prefill walks equal-length prompts to their last token: the
    greedy continuation after it equals generate's (which walks the same
    prompts), and unequal lengths are refused."""
    cfg = GraniteConfig(layers=3, attention_layers=(1,), experts=12, top_k=4, vocab=4096)
    w = synthetic_weights(cfg, seed=5, device=gpu_device)
    eng = GraniteEngine(cfg, w, rows=2, device=gpu_device, max_steps=64, split_len=16)
    g = torch.Generator().manual_seed(9)
    prompts = [torch.randint(0, cfg.vocab, (7,), generator=g).tolist() for _ in range(2)]
    tokens, _, _ = eng.generate(prompts, 6)
    eng.prefill(prompts)
    for _ in range(6):
        eng.replay()
    eng.check_errors()
    sam = eng.sam.cpu()
    assert [sam[b, 6:12].tolist() for b in range(2)] == tokens
    with pytest.raises(ValueError, match="one length"):
        eng.prefill([prompts[0], prompts[1][:5]])
