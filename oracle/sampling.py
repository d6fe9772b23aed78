"""Token sampling as tfd_sample_rows computes it (CPU, numpy).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Two samplers of the reference, restated with this library's random numbers:

* ``sample_topk``: ``sample`` of ``examples/qwen3_5_35b_a3b-tilelang/run.py:145-180``
  -- the top k logits, divided by the temperature, softmax over the k, the
  nucleus (``(cumsum(probs) - probs) < top_p``, the first always kept), the
  kept probabilities renormalised, one categorical draw -- with the draw taken
  as the inverse CDF at a given uniform ``u`` instead of ``torch.multinomial``;
* ``sample_gumbel``: ``sample_stage1_kernel`` of
  ``examples/granite_4_0_h_small-cuda/kernels/granite.cu:716-800`` -- softmax
  over the whole row at a temperature by Gumbel-max: the argmax of
  ``v / T - log(-log(u_i))``.

The uniforms come from a counter-based hash of (seed, row, counter, element):
``rand24`` is splitmix64's output function (Steele, Lea and Flood, OOPSLA 2014)
chained over the four.  The arithmetic is float32 in the order the kernel takes
it (sequential sums), so picks agree with the GPU's except where ``u`` falls on
a boundary within float32 rounding (``exp`` and ``log`` may differ by an ulp);
``sample_topk`` and ``sample_gumbel`` return the distance to the nearest
boundary so a test can tell those draws apart.
"""
from __future__ import annotations

import numpy as np

MASK64 = (1 << 64) - 1
DRAW_ELEM = 0xFFFFFFFF


def mix64(z: int) -> int:
    """splitmix64's output function (a bijection of 64-bit integers)."""
    z &= MASK64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    return z ^ (z >> 31)


def splitmix64_stream(seed: int, n: int) -> list[int]:
    """The splitmix64 generator's first n outputs (state += golden gamma, then
    the output function): used to pin ``mix64`` against its published outputs."""
    out, s = [], seed & MASK64
    for _ in range(n):
        s = (s + 0x9E3779B97F4A7C15) & MASK64
        out.append(mix64(s))
    return out


def rand24(seed: int, row: int, ctr: int, elem: int) -> int:
    """24 random bits of (seed, row, counter, element), as the kernel's rand24."""
    h = mix64((mix64((mix64(seed) + (row & 0xFFFFFFFF)) & MASK64)
               + (((ctr & 0xFFFFFFFF) << 32) | (elem & 0xFFFFFFFF))) & MASK64)
    return h >> 40


def draw_uniform(seed: int, row: int, ctr: int) -> np.float32:
    """The top-k path's uniform in [0, 1)."""
    return np.float32(rand24(seed, row, ctr, DRAW_ELEM)) * np.float32(1.0 / 16777216.0)


def gumbel_uniforms(seed: int, row: int, ctr: int, n: int) -> np.ndarray:
    """The Gumbel path's uniforms in (0, 1) for elements 0 .. n-1: the top 23 of
    rand24's bits, (b + 0.5) / 2^23 (vectorised restatement of rand24)."""
    m = np.uint64(MASK64)
    with np.errstate(over="ignore"):
        def vmix(z):
            z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
            z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
            return z ^ (z >> np.uint64(31))
        base = np.uint64((mix64((mix64(seed) + (row & 0xFFFFFFFF)) & MASK64)))
        elems = np.arange(n, dtype=np.uint64) | np.uint64((ctr & 0xFFFFFFFF) << 32)
        h = vmix((base + elems) & m)
    bits = (h >> np.uint64(41)).astype(np.float32)       # 23 bits: b + 0.5 exact in f32
    return (bits + np.float32(0.5)) * np.float32(1.0 / 8388608.0)


def logit_keys(row: np.ndarray) -> np.ndarray:
    """The kernel's 64-bit key of every logit: value order (NaN lowest, -0 as +0),
    then the lower index first; larger keys rank first."""
    b = np.asarray(row, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (b & np.uint64(0x7FFFFFFF)) > np.uint64(0x7F800000)
    b = np.where(b == np.uint64(0x80000000), np.uint64(0), b)
    neg = (b & np.uint64(0x80000000)) != 0
    ordv = np.where(neg, (~b) & np.uint64(0xFFFFFFFF), b | np.uint64(0x80000000))
    ordv = np.where(nan, np.uint64(0), ordv)
    idx = np.arange(len(row), dtype=np.uint64)
    return (ordv << np.uint64(32)) | (np.uint64(0xFFFFFFFF) - idx)


def topk_indices(row: np.ndarray, k: int) -> np.ndarray:
    """The k highest-ranked logits' indices, best first."""
    keys = logit_keys(row)
    order = np.argsort(keys)[::-1][:k]
    return order.astype(np.int64)


def sample_topk(row: np.ndarray, temperature: float, top_k: int, top_p: float,
                u: np.float32) -> tuple[int, float]:
    """run.py's top-k / temperature / softmax / nucleus / draw at uniform u.
    -> (pick, the draw's distance to the nearest cumulative boundary, relative
    to the kept mass)."""
    row = np.asarray(row, dtype=np.float32)
    ids = topk_indices(row, min(top_k, len(row)))
    t = np.float32(temperature)
    x = [np.float32(row[i]) / t if temperature != 1.0 else np.float32(row[i]) for i in ids]
    m = x[0]
    e, s = [], np.float32(0)
    for xi in x:
        ei = np.float32(np.exp(np.float32(xi - m))) if xi == xi else np.float32(0)
        e.append(ei)
        s = np.float32(s + ei)
    if not (s > 0):
        return int(ids[0]), float("inf")
    p, kept, before, last = [], np.float32(0), np.float32(0), 0
    for i, ei in enumerate(e):
        pi = np.float32(ei / s)
        keep = i == 0 or top_p >= 1.0 or before < np.float32(top_p)
        before = np.float32(before + pi)
        p.append(pi if keep else np.float32(0))
        if keep:
            kept = np.float32(kept + pi)
            last = i
    target = np.float32(np.float32(u) * kept)
    acc, at = np.float32(0), last
    for i in range(last + 1):
        acc = np.float32(acc + p[i])
        if p[i] > 0 and target < acc:
            at = i
            break
    # distance from the target to the nearest boundary (for draws a rounding
    # of exp or of a sum could move across one)
    acc2, dist = np.float32(0), float("inf")
    for i in range(last + 1):
        acc2 = np.float32(acc2 + p[i])
        dist = min(dist, abs(float(acc2) - float(target)) / float(kept))
    return int(ids[at]), dist


def sample_gumbel(row: np.ndarray, temperature: float, seed: int, row_id: int,
                  ctr: int) -> tuple[int, float]:
    """Gumbel-max over the whole row -> (pick, margin between the best and the
    second-best perturbed value, relative to the best's magnitude)."""
    row = np.asarray(row, dtype=np.float32)
    u = gumbel_uniforms(seed, row_id, ctr, len(row))
    v = row / np.float32(temperature) if temperature != 1.0 else row
    g = (v - np.log(-np.log(u))).astype(np.float32)
    g = np.where(np.isnan(g), np.float32(-np.inf), g)
    best = int(np.argmax(g))                       # the first maximum
    if not np.isfinite(g[best]) and np.isnan(row).all():
        return 0, float("inf")
    top2 = np.sort(g)[-2:] if len(g) > 1 else np.array([g[best], -np.inf], np.float32)
    margin = float(top2[-1] - top2[-2]) / max(1.0, abs(float(top2[-1])))
    return best, margin
