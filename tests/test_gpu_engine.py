"""The captured decode engine against the oracle's greedy loop.

Parity bar of the decode path: greedy tokens identical for the first 64 steps;
logits within max |delta| <= 2e-2 of the oracle's max |logit| (bf16).  The small
configs here are config 1's shape at bf16 and the Qwen3-1.7B layer shape at two
layers; the full-depth model is checked against committed golden fixtures in
test_gpu_golden.py.
"""
import math

import pytest
import torch

from oracle import qwen3_hir as O
from tests._parity import oracle_arith, report
from tilefoundry_amd.qwen3 import QWEN3_1_7B, TINY, synthetic_weights
from tilefoundry_amd.qwen3.engine import Engine

pytestmark = pytest.mark.gpu


def _dims(cfg):
    return O.Qwen3Dims(hidden=cfg.hidden_size, heads=cfg.num_attention_heads,
                       kv_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim,
                       intermediate=cfg.intermediate_size, vocab=cfg.vocab_size,
                       layers=cfg.num_hidden_layers, dtype=cfg.dtype)


def _prompt(n, vocab, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, vocab, (n,), generator=g).tolist()


def _ulp_at(v: float) -> float:
    return 2.0 ** (math.floor(math.log2(abs(v))) - 7) if v else 2.0 ** -133


def _first_divergence(a, b):
    for k, (x, y) in enumerate(zip(a, b)):
        if x != y:
            return k
    return None


def _check_run(eng_run, orc_run, steps, strict=True):
    """Free-running greedy parity.  strict: all *steps* tokens identical.
    Otherwise the first divergence must be explained by the logit error at that
    step: the oracle's gap between its pick and the engine's is at most twice
    the largest |engine - oracle| logit difference (both logits moved by at most
    that much; with bf16 logits such near-ties are decided by f32 summation
    order)."""
    k = _first_divergence(eng_run.tokens[:steps], orc_run.tokens[:steps])
    upto = steps if k is None else k + 1
    for j in range(upto):
        r = report(eng_run.logits[j], orc_run.logits[j])
        assert r["max_rel"] <= 2e-2, (j, r)
    if k is None:
        return None
    ol, el = orc_run.logits[k], eng_run.logits[k]
    mine, theirs = eng_run.tokens[k], orc_run.tokens[k]
    gap = float(ol[theirs] - ol[mine])
    eps = float((el - ol).abs().max())
    detail = (f"diverged at step {k}: engine {mine} (oracle logit {float(ol[mine])}, engine "
              f"{float(el[mine])}) vs oracle {theirs} (oracle logit {float(ol[theirs])}, "
              f"engine {float(el[theirs])}); oracle margin {orc_run.margins[k]}, max|dlogit| {eps}")
    assert not strict, detail
    assert gap <= 2 * eps + 1e-12, detail
    return k


def _teacher_forced(eng, prompt, orc_run, steps):
    """Feed the oracle's own continuation: the engine's pick at every position
    must equal the oracle's, except where the oracle's margin between the two
    picks is within twice that step's largest |engine - oracle| logit
    difference (both logits moved by at most that much).  Returns the number of
    such near-tie picks, which is at most the number of steps whose oracle
    top-2 margin is within twice the step's error."""
    seq = list(prompt) + orc_run.tokens[:steps - 1]
    picks, logits = eng.walk(seq, len(prompt) - 1, steps)
    near_ties = close = 0
    for k in range(steps):
        ol = orc_run.logits[k]
        eps = float((logits[k] - ol).abs().max())
        assert eps <= 2e-2 * float(ol.abs().max()), (k, eps)
        close += orc_run.margins[k] <= 2 * eps
        if picks[k] == orc_run.tokens[k]:
            continue
        gap = float(ol[orc_run.tokens[k]] - ol[picks[k]])
        assert gap <= 2 * eps + 1e-12, (k, picks[k], orc_run.tokens[k], gap, eps)
        near_ties += 1
    assert near_ties <= close
    return near_ties


SMALL = TINY.with_(dtype=torch.bfloat16)


@pytest.mark.parametrize("norms", ["ones", "random"])
def test_small_bf16_greedy_64(gpu_device, norms):
    w = synthetic_weights(SMALL, seed=0, norms=norms)
    prompt = _prompt(16, SMALL.vocab_size)
    orc = O.decode(O.Qwen3Oracle(_dims(SMALL), w), prompt, 64)
    eng = Engine(SMALL, w, device=gpu_device, max_new=64, prompt_room=16)
    run = eng.generate(prompt, 64, record_logits=True)
    _check_run(run, orc, 64)
    assert _teacher_forced(eng, prompt, orc, 64) == 0


def test_qwen3_layer_shape_two_layers_greedy_64(gpu_device):
    cfg = QWEN3_1_7B.with_(num_hidden_layers=2)
    w = synthetic_weights(cfg, seed=0, norms="ones")
    prompt = _prompt(8, cfg.vocab_size)
    orc = O.decode(O.Qwen3Oracle(_dims(cfg), w), prompt, 64)
    eng = Engine(cfg, w, device=gpu_device, max_new=64, prompt_room=8)
    run = eng.generate(prompt, 64, record_logits=True)
    k = _check_run(run, orc, 64, strict=False)
    ties = _teacher_forced(eng, prompt, orc, 64)
    print(f"free-running identical for {64 if k is None else k} steps; teacher-forced "
          f"near-tie picks: {ties}; oracle margins min {min(orc.margins):.4g}")


def test_paging_and_graph_do_not_change_results(gpu_device):
    """Any page permutation, and graph replay vs direct launches, give the same
    bits (paged result == contiguous result, mha_decode_paged.py:100-116)."""
    w = synthetic_weights(SMALL, seed=2, norms="ones")
    prompt = _prompt(20, SMALL.vocab_size, seed=3)
    runs = []
    for page_seed, graph in ((None, True), (7, True), (11, False)):
        eng = Engine(SMALL, w, device=gpu_device, max_new=80, prompt_room=20,
                     page_seed=page_seed, graph=graph)
        runs.append(eng.generate(prompt, 80, record_logits=True))
    for r in runs[1:]:
        assert r.tokens == runs[0].tokens
        assert torch.equal(r.logits, runs[0].logits)


def test_generate_is_repeatable_and_logits_for_matches(gpu_device):
    w = synthetic_weights(SMALL, seed=4, norms="ones")
    eng = Engine(SMALL, w, device=gpu_device, max_new=32, prompt_room=12)
    prompt = _prompt(12, SMALL.vocab_size, seed=5)
    a = eng.generate(prompt, 32, record_logits=True)
    b = eng.generate(prompt, 32, record_logits=True)
    assert a.tokens == b.tokens and torch.equal(a.logits, b.logits)
    lg = eng.logits_for(prompt)
    assert torch.equal(lg.cpu(), a.logits[0])


def test_capacity_and_prompt_checks(gpu_device):
    w = synthetic_weights(SMALL, seed=4, norms="ones")
    eng = Engine(SMALL, w, device=gpu_device, max_new=8, prompt_room=4, graph=False)
    with pytest.raises(ValueError):
        eng.generate([1, 2, 3, 4, 5], 8)           # 5 + 8 > 12 steps
    with pytest.raises(ValueError):
        eng.generate([], 4)
    with pytest.raises(ValueError):
        eng.generate([SMALL.vocab_size], 4)        # id out of range


@pytest.mark.parametrize("shape", ["small", "qwen3_2layer"])
def test_persistent_kernel_equals_per_phase_launches(gpu_device, shape):
    """The persistent kernel runs the same phase code on the same partition as
    the per-phase launches: tokens and logits must be bit-identical, and one
    launch of n steps must equal n launches of one step."""
    cfg = SMALL if shape == "small" else QWEN3_1_7B.with_(num_hidden_layers=2)
    w = synthetic_weights(cfg, seed=6, norms="ones")
    prompt = _prompt(12, cfg.vocab_size, seed=9)
    ref = Engine(cfg, w, device=gpu_device, max_new=48, prompt_room=12, mode="graph")
    per = Engine(cfg, w, device=gpu_device, max_new=48, prompt_room=12, mode="persistent")
    a = ref.generate(prompt, 48, record_logits=True)
    b = per.generate(prompt, 48, record_logits=True)
    assert a.tokens == b.tokens
    assert torch.equal(a.logits, b.logits)
    c = per.generate(prompt, 48)                    # two launches: prompt walk, continuation
    assert c.tokens == a.tokens
    assert torch.equal(per.logits, ref.logits)


def test_xcd_kernel_matches_oracle_at_the_layer_shape(gpu_device):
    """The XCD-partitioned persistent kernel (two layers of the Qwen3-1.7B shape)
    against the oracle's greedy loop in the kernel's arithmetic (attention's
    products exact): logits within the bf16 bar, free-running tokens identical
    until a near-tie the measured error explains, teacher-forced picks bounded by
    each step's error."""
    cfg = QWEN3_1_7B.with_(num_hidden_layers=2)
    w = synthetic_weights(cfg, seed=0, norms="ones")
    prompt = _prompt(8, cfg.vocab_size)
    with oracle_arith("xcd"):
        orc = O.decode(O.Qwen3Oracle(_dims(cfg), w), prompt, 64)
    eng = Engine(cfg, w, device=gpu_device, max_new=64, prompt_room=8, mode="xcd")
    run = eng.generate(prompt, 64, record_logits=True)
    k = _check_run(run, orc, 64, strict=False)
    ties = _teacher_forced(eng, prompt, orc, 64)
    print(f"xcd: free-running identical for {64 if k is None else k} steps; teacher-forced "
          f"near-tie picks {ties}")


def test_xcd_kernel_tracks_the_persistent_kernel(gpu_device):
    """Same weights and prompt: the XCD kernel differs from the chip-wide one in
    the f32 order of the o and down sums and in taking attention's products
    exactly (the chip-wide kernel rounds each one, as the HIR does), so the
    logits agree to the north-star bar (2e-2 of max |logit|; cosine >= 0.999,
    the two arithmetics being a bf16 rounding per product apart) and the tokens
    agree wherever no near-tie is hit; one launch of n steps equals n launches of
    one step bit for bit."""
    cfg = QWEN3_1_7B.with_(num_hidden_layers=2)
    w = synthetic_weights(cfg, seed=6, norms="ones")
    prompt = _prompt(12, cfg.vocab_size, seed=9)
    ref = Engine(cfg, w, device=gpu_device, max_new=48, prompt_room=12, mode="persistent")
    xcd = Engine(cfg, w, device=gpu_device, max_new=48, prompt_room=12, mode="xcd")
    a = ref.generate(prompt, 48, record_logits=True)
    b = xcd.generate(prompt, 48, record_logits=True)
    k = _first_divergence(a.tokens, b.tokens)
    upto = 48 if k is None else k + 1
    for j in range(upto):
        r = report(b.logits[j], a.logits[j])
        assert r["max_rel"] <= 2e-2 and r["cos"] >= 0.999, (j, r)
    c = xcd.generate(prompt, 48)                    # two launches: prompt walk, continuation
    assert c.tokens == b.tokens
    one = [xcd.generate(prompt, 1)]
    assert one[0].tokens == b.tokens[:1]


def test_xcd_kernel_paging_changes_no_bit(gpu_device):
    """The XCD kernel looks up its first K/V tiles' pages once per step: a permuted
    page table gives the bits of the identity layout, through contexts that cross
    16-token pages and 64-position splits, in one launch and in launches of a step."""
    cfg = QWEN3_1_7B.with_(num_hidden_layers=2)
    w = synthetic_weights(cfg, seed=8, norms="ones")
    prompt = _prompt(40, cfg.vocab_size, seed=12)
    runs = []
    for page_seed in (None, 7, 13):
        eng = Engine(cfg, w, device=gpu_device, max_new=96, prompt_room=40, mode="xcd",
                     page_seed=page_seed)
        runs.append(eng.generate(prompt, 96, record_logits=True))
    for r in runs[1:]:
        assert r.tokens == runs[0].tokens
        assert torch.equal(r.logits, runs[0].logits)


def test_xcd_kernel_is_independent_of_where_a_launch_starts(gpu_device):
    """The dispatcher's first XCD moves with the workgroups dispatched before a
    launch.  Single-workgroup kernels launched in between rotate it through
    every offset; each block takes its XCD from the hardware and its rank from
    block / 8, so every run plays the same partition and returns the same bits."""
    cfg = QWEN3_1_7B.with_(num_hidden_layers=2)
    w = synthetic_weights(cfg, seed=6, norms="ones")
    prompt = _prompt(12, cfg.vocab_size, seed=9)
    xcd = Engine(cfg, w, device=gpu_device, max_new=16, prompt_room=12, mode="xcd")
    base = xcd.generate(prompt, 16, record_logits=True)
    one = torch.zeros(1, device=gpu_device)
    for shift in range(1, 8):
        for _ in range(shift):
            one.add_(1.0)                           # one workgroup
        run = xcd.generate(prompt, 16, record_logits=True)
        assert run.tokens == base.tokens, shift
        assert torch.equal(run.logits, base.logits), shift
