"""Regenerate the committed golden fixtures (CPU, minutes at C2 size).

    python tests/golden/make_golden.py [c1] [c2] [c2x] [c2xs] [c2xp]

c1_tiny_fp32.json   workload C1: tiny Qwen3 (2 layers, hidden 256, 4q/2kv,
                    head_dim 64, I 768, V 4096), fp32, every parameter N(0, 0.02)
                    from seed 0, a 128-token uniform-random prompt (seed 0), 32
                    greedy tokens.  Produced by the oracle AND by Hugging Face
                    Qwen3ForCausalLM (full-sequence forward, same weights); the
                    script refuses to write unless the two agree.
c2_qwen3_1p7b.json  workload C2 shape (28 layers, bf16), the bench's
                    synthetic weights (seed 0) and 32-token prompt (seed 0): the
                    oracle's first 64 greedy tokens, their top-2 margins and each
                    step's top-8 (index, logit); for both norm-scale draws.
c2_*_logits.npy     full bf16 logits (raw uint16) of steps 0 and 63.
c2_*_exact_step*.npy  (target c2x) the same two steps teacher-forced on the
                    recorded tokens, with every matmul and attention sum taken
                    exactly (oracle.exact_sums: the HIR's rounding points, f64
                    sums).  c2_order_noise.json records how far the oracle's own
                    f32 sums sit from these: the noise floor of f32 summation
                    order at this depth, which bounds what any correct
                    implementation can be asked to match.
c2_*_exact_steps.npz  (target c2xs) the exact-sum logits at steps 0, 8, ...,
                    56 and 63 of the same teacher-forced walk (keys step<k>).
c2_*_exactprod_steps.npz  (target c2xp) the same steps of the same walk in the
                    exact-products arithmetic (oracle.exact_products: attention's
                    q.k and p.v products not rounded before their sums, the XCD
                    kernel's), with exact sums; c2_order_noise_exactprod.json
                    records how far that arithmetic's own f32 sums sit from it at
                    steps 0 and 63.

The fixtures are data (inputs and expected outputs), regenerated from seeds.
"""
from __future__ import annotations

import json
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
HERE = Path(__file__).resolve().parent

from oracle import qwen3_hir as O  # noqa: E402
from tilefoundry_amd.qwen3 import QWEN3_1_7B, TINY, synthetic_weights  # noqa: E402


def prompt_ids(n: int, vocab: int, seed: int = 0) -> list[int]:
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, vocab, (n,), generator=g).tolist()


def hf_greedy(dims, w, prompt, n):
    from tests.test_oracle_pins import _hf_model

    model = _hf_model(dims, w)
    seq = list(prompt)
    with torch.no_grad():
        for _ in range(n):
            logits = model(torch.tensor(seq).unsqueeze(0)).logits[0, -1]
            seq.append(int(torch.argmax(logits)))
    return seq[len(prompt):]


def make_c1():
    dims = O.C1
    w = synthetic_weights(TINY, seed=0)
    prompt = prompt_ids(128, dims.vocab)
    run = O.decode(O.Qwen3Oracle(dims, w), prompt, 32)
    hf = hf_greedy(dims, w, prompt, 32)
    if hf != run.tokens:
        raise SystemExit(f"oracle and HF disagree: {run.tokens} vs {hf}")
    top = [[[int(i), float(v)] for v, i in zip(*torch.topk(lg, 16))] for lg in run.logits]
    out = {"config": "C1 tiny Qwen3 fp32; all parameters N(0,0.02) seed 0; prompt 128 ids seed 0",
           "prompt": prompt, "tokens": run.tokens, "hf_tokens": hf, "margins": run.margins,
           "top16": top}
    (HERE / "c1_tiny_fp32.json").write_text(json.dumps(out))
    print("c1: tokens", run.tokens[:8], "...")


def make_c2():
    dims = O.C2
    prompt = prompt_ids(32, dims.vocab)
    out = {"config": "C2 Qwen3-1.7B-arch bf16; N(0,0.02) seed 0; prompt 32 ids seed 0",
           "prompt": prompt}
    for norms in ("random", "ones"):
        t0 = time.time()
        w = synthetic_weights(QWEN3_1_7B, seed=0, norms=norms)
        run = O.decode(O.Qwen3Oracle(dims, w), prompt, 64)
        top = [[[int(i), float(v)] for v, i in zip(*torch.topk(lg, 8))] for lg in run.logits]
        out[norms] = {"tokens": run.tokens, "margins": run.margins, "top8": top}
        for k in (0, 63):
            raw = run.logits[k].to(torch.bfloat16).view(torch.int16).numpy().astype(np.uint16)
            np.save(HERE / f"c2_{norms}_logits_step{k}.npy", raw)
        print(f"c2 {norms}: {time.time() - t0:.0f}s tokens {run.tokens[:8]}...", flush=True)
        del w
    (HERE / "c2_qwen3_1p7b.json").write_text(json.dumps(out))


def forced_logits(oracle, seq, at):
    """Logits after consuming seq[:k + 1] for each k in *at* (one pass over seq)."""
    input_ids = torch.tensor(seq, dtype=torch.int64)
    caches = oracle.init_caches()
    out = {}
    with torch.no_grad():
        for step in range(max(at) + 1):
            args = oracle.prepare_inputs_for_generation(input_ids, step, caches)
            logits, fresh = oracle.forward(*args)
            caches = oracle.append_cache(caches, fresh)
            if step in at:
                out[step] = logits.float().reshape(-1).clone()
    return out


def make_c2x():
    fx = json.loads((HERE / "c2_qwen3_1p7b.json").read_text())
    prompt = fx["prompt"]
    pl = len(prompt)
    noise = {}
    for norms in ("random", "ones"):
        t0 = time.time()
        w = synthetic_weights(QWEN3_1_7B, seed=0, norms=norms)
        seq = prompt + fx[norms]["tokens"][:63]
        with O.exact_sums():
            ex = forced_logits(O.Qwen3Oracle(O.C2, w), seq, {pl - 1, pl - 1 + 63})
        noise[norms] = {}
        for k in (0, 63):
            lg = ex[pl - 1 + k]
            raw = lg.to(torch.bfloat16).view(torch.int16).numpy().astype(np.uint16)
            np.save(HERE / f"c2_{norms}_exact_step{k}.npy", raw)
            ref = np.load(HERE / f"c2_{norms}_logits_step{k}.npy").astype(np.int16)
            orc = torch.from_numpy(ref).view(torch.bfloat16).float()
            d = (orc - lg).abs()
            noise[norms][f"step{k}"] = {"max_abs": float(d.max()), "mean_abs": float(d.mean()),
                                       "max_logit": float(orc.abs().max())}
        print(f"c2x {norms}: {time.time() - t0:.0f}s {noise[norms]}", flush=True)
        del w
    (HERE / "c2_order_noise.json").write_text(json.dumps(noise, indent=1))


EXACT_STEPS = (0, 8, 16, 24, 32, 40, 48, 56, 63)


def make_c2xs():
    """c2_*_exact_steps.npz: the exact-sum logits (as make_c2x) at every 8th of
    the 64 steps and the last, raw bf16 bits under keys step<k>; steps 0 and 63
    must reproduce c2_*_exact_step{0,63}.npy bit for bit."""
    fx = json.loads((HERE / "c2_qwen3_1p7b.json").read_text())
    prompt = fx["prompt"]
    pl = len(prompt)
    for norms in ("random", "ones"):
        t0 = time.time()
        w = synthetic_weights(QWEN3_1_7B, seed=0, norms=norms)
        seq = prompt + fx[norms]["tokens"][:63]
        with O.exact_sums():
            ex = forced_logits(O.Qwen3Oracle(O.C2, w), seq, {pl - 1 + k for k in EXACT_STEPS})
        arrays = {}
        for k in EXACT_STEPS:
            arrays[f"step{k}"] = (ex[pl - 1 + k].to(torch.bfloat16).view(torch.int16).numpy()
                                  .astype(np.uint16))
        for k in (0, 63):
            same = np.load(HERE / f"c2_{norms}_exact_step{k}.npy")
            assert np.array_equal(same, arrays[f"step{k}"]), (norms, k)
        np.savez_compressed(HERE / f"c2_{norms}_exact_steps.npz", **arrays)
        print(f"c2xs {norms}: {time.time() - t0:.0f}s", flush=True)
        del w


def make_c2xp():
    """c2_*_exactprod_steps.npz and c2_order_noise_exactprod.json: the walk of
    make_c2xs in the exact-products arithmetic, with exact sums (the reference
    values) and with the oracle's f32 sums at steps 0 and 63 (their distance from
    the reference values is that arithmetic's summation-order noise)."""
    fx = json.loads((HERE / "c2_qwen3_1p7b.json").read_text())
    prompt = fx["prompt"]
    pl = len(prompt)
    noise = {}
    for norms in ("random", "ones"):
        t0 = time.time()
        w = synthetic_weights(QWEN3_1_7B, seed=0, norms=norms)
        seq = prompt + fx[norms]["tokens"][:63]
        with O.exact_products():
            with O.exact_sums():
                ex = forced_logits(O.Qwen3Oracle(O.C2, w), seq,
                                   {pl - 1 + k for k in EXACT_STEPS})
            f32 = forced_logits(O.Qwen3Oracle(O.C2, w), seq, {pl - 1, pl - 1 + 63})
        arrays = {}
        for k in EXACT_STEPS:
            arrays[f"step{k}"] = (ex[pl - 1 + k].to(torch.bfloat16).view(torch.int16).numpy()
                                  .astype(np.uint16))
        np.savez_compressed(HERE / f"c2_{norms}_exactprod_steps.npz", **arrays)
        noise[norms] = {}
        for k in (0, 63):
            ref = ex[pl - 1 + k].to(torch.bfloat16).float()
            orc = f32[pl - 1 + k].to(torch.bfloat16).float()
            d = (orc - ref).abs()
            noise[norms][f"step{k}"] = {"max_abs": float(d.max()), "mean_abs": float(d.mean()),
                                       "max_logit": float(ref.abs().max())}
        print(f"c2xp {norms}: {time.time() - t0:.0f}s {noise[norms]}", flush=True)
        del w
    (HERE / "c2_order_noise_exactprod.json").write_text(json.dumps(noise, indent=1))


if __name__ == "__main__":
    which = sys.argv[1:] or ["c1", "c2", "c2x"]
    if "c2xp" in which:
        make_c2xp()
    if "c2xs" in which:
        make_c2xs()
    if "c1" in which:
        make_c1()
    if "c2" in which:
        make_c2()
    if "c2x" in which:
        make_c2x()
