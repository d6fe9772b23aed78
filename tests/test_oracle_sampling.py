"""Pins of the sampling oracle (oracle/sampling.py), on the CPU.

* the hash: mix64 reproduces splitmix64's published first outputs for seed
  1234567; the uniforms it yields are uniform (moments, no repeats);
* the top-k order: value first (NaN last, -0 as +0), then the lower index --
  against Python's own sort of (value, index) tuples, on rows full of ties;
* the top-k / temperature / nucleus / draw chain: with top_k 1 every draw is the
  first maximum; over a fine grid of uniforms the picks' frequencies are the
  kept, renormalised probabilities computed independently with torch as
  run.py:166-179 computes them (softmax of the top k over T, the mask
  (cumsum - probs) < top_p with the first kept);
* the Gumbel path: over many rows' draws the frequencies approach softmax(v / T).
"""
import math

import numpy as np
import pytest
import torch

from oracle import sampling as S


def test_mix64_is_splitmix64():
    assert S.splitmix64_stream(1234567, 5) == [
        6457827717110365317, 3203168211198807973, 9817491932198370423,
        4593380528125082431, 16408922859458223821]


def test_uniforms_are_uniform():
    u = np.array([S.draw_uniform(7, r, c) for r in range(40) for c in range(500)], np.float64)
    assert abs(u.mean() - 0.5) < 0.01 and abs(u.var() - 1 / 12) < 0.005
    assert len(set(u.tolist())) > 0.99 * len(u)
    g = S.gumbel_uniforms(7, 3, 11, 100_000).astype(np.float64)
    assert g.min() > 0 and g.max() < 1
    assert abs(g.mean() - 0.5) < 0.005 and abs(g.var() - 1 / 12) < 0.002
    # the vectorised form is the scalar hash, bit for bit
    for i in (0, 1, 99_999):
        assert g[i] == ((S.rand24(7, 3, 11, i) >> 1) + 0.5) / 8388608.0


def test_topk_order_against_a_tuple_sort():
    rng = np.random.default_rng(0)
    for _ in range(20):
        row = rng.integers(-3, 4, size=300).astype(np.float32) * np.float32(0.5)
        row[rng.integers(0, 300, size=5)] = np.nan
        row[rng.integers(0, 300, size=5)] = -0.0
        def rank(i):
            v = float(row[i])
            return (0 if math.isnan(v) else 1, 0.0 if math.isnan(v) else v + 0.0, -i)
        want = sorted(range(len(row)), key=rank, reverse=True)[:64]
        assert S.topk_indices(row, 64).tolist() == want


def test_top1_is_the_first_maximum():
    rng = np.random.default_rng(1)
    row = rng.integers(0, 5, size=1000).astype(np.float32)
    first = int(np.argmax(row))
    for u in np.linspace(0, 0.999999, 50, dtype=np.float32):
        assert S.sample_topk(row, 0.7, 1, 0.5, u)[0] == first


@pytest.mark.parametrize("temperature,top_k,top_p", [(1.0, 20, 0.95), (0.7, 8, 1.0),
                                                     (1.6, 50, 0.5), (1.0, 64, 0.05)])
def test_draw_frequencies_are_runpy_probabilities(temperature, top_k, top_p):
    rng = np.random.default_rng(top_k)
    row = (rng.standard_normal(3000) * 2).astype(np.float32)
    # run.py:166-179 with torch
    values, ids = torch.topk(torch.from_numpy(row).float(), top_k)
    if temperature != 1.0:
        values = values / max(temperature, 1e-6)
    probs = torch.softmax(values, dim=-1)
    if top_p < 1.0:
        keep = (torch.cumsum(probs, dim=-1) - probs) < top_p
        keep[0] = True
        probs = probs * keep
    probs = probs / probs.sum()
    want = {int(i): float(p) for i, p in zip(ids, probs) if p > 0}
    n = 20000
    got = {}
    for u in (np.arange(n, dtype=np.float64) + 0.5) / n:
        k = S.sample_topk(row, temperature, top_k, top_p, np.float32(u))[0]
        got[k] = got.get(k, 0) + 1
    assert set(got) <= set(want)
    for k, p in want.items():
        assert abs(got.get(k, 0) / n - p) <= 2.0 / n + 1e-5, (k, got.get(k, 0) / n, p)


def test_gumbel_frequencies_are_softmax():
    row = np.array([0.0, 1.0, -0.5, 2.0, 0.3, -3.0, 1.5, 0.9], np.float32)
    for temperature in (1.0, 0.5, 2.0):
        want = torch.softmax(torch.from_numpy(row) / temperature, 0).numpy()
        n = 20000
        counts = np.zeros(len(row))
        for r in range(n):
            counts[S.sample_gumbel(row, temperature, seed=5, row_id=r, ctr=3)[0]] += 1
        assert np.abs(counts / n - want).max() < 0.012, (temperature, counts / n, want)
