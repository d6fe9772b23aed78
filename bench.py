"""Decode throughput of the Qwen3-1.7B-architecture model at batch 1 (workload C2).

    python bench.py [--gpus 1] [--steps 2048] [--warmup 64] [--mode xcd|persistent|graph]

A step is one decode token: every layer, the head, the greedy pick.  The
workload is C2: bf16 weights drawn N(0, 0.02) from seed 0
(every parameter, norm scales included), tied embeddings, a 32-token
uniform-random prompt (seed 0), a 16-token-page KV cache, and 2048 greedy new
tokens (positions 31..2078).  `--steps N` times the LAST N tokens of that run
(N = 2048, the default, times all of them; the first 2048 - N are decoded
untimed first), so every timed step works at the context depth the workload
gives it.  Weights are resident in HBM before the timed region starts.

Modes: "xcd" (default) runs all the timed steps in one launch of the
XCD-partitioned persistent decode kernel; "persistent" in one launch of the
chip-wide persistent kernel; "graph" replays a captured graph of per-phase
launches once per token.

Prints one JSON line: the metric; the whole-step HBM roofline fraction from
algorithmic bytes (weights once + the KV each step touches); the dominant
kernel's roofline -- in the persistent modes the decode kernel itself: the
algorithmic bytes of the timed launch over its duration, HIP events on the
launch stream around it (rocprofv3's trace of the same command lists that
launch as its last dispatch of the kernel); in graph mode the gate/up GEMV --
with the HBM traffic that rocprofv3's counters measured for it when a profile
is committed; and the CPU oracle timed on the host.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK = 8.0e12          # MI355X HBM3E, bytes/s
REFERENCE_TOKS = 612.5     # the reference's published rate for this metric (H200)
METRIC = "decode tok/s bs=1 Qwen3-1.7B-arch bf16; achieved HBM TB/s vs 8 TB/s peak"


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def time_gate_up(eng, rounds: int) -> float:
    """Average duration (s) of the gate/up GEMV launch, rotating over every
    layer's weights (1.4 GB, past the 256 MB last-level cache), HIP events on
    the launch stream."""
    import torch

    from tilefoundry_amd import _lib
    from tilefoundry_amd._lib import ptr

    stream = torch.cuda.current_stream(eng.device)
    s = stream.cuda_stream
    L = eng._lib

    def launch(i):
        w = eng.layers[i]
        L.tfd_gemv_bf16(ptr(eng.h1_rows[i]), ptr(w["gamma_post"]), ptr(w["w_gu"]), None,
                        ptr(eng.hmid_rows[i]),
                        eng.H, 2 * eng.I, _lib.PRO_NORM, _lib.EPI_SWIGLU, eng.eps, s)

    for i in range(eng.L):
        launch(i)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(rounds):
        for i in range(eng.L):
            launch(i)
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / 1e3 / (rounds * eng.L)


class LaunchClock:
    """HIP events on the launch stream around the persistent launches of *eng*
    made while ``armed`` (the timed region's), with the algorithmic bytes of
    each (weights once per step + the KV every step reads and writes at its
    position)."""

    def __init__(self, eng):
        import torch

        self.eng, self.torch = eng, torch
        self.records = []          # (start event, end event, bytes)
        self.pos = 0
        self.armed = False
        launch, load = eng._launch_persistent, eng._load_prompt

        def timed_launch(n):
            w = eng.weight_bytes_per_step()
            nbytes = sum(w + eng.kv_bytes_at(p) for p in range(self.pos, self.pos + n))
            self.pos += n
            if not self.armed:
                launch(n)
                return
            stream = torch.cuda.current_stream(eng.device)
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            launch(n)
            b.record(stream)
            self.records.append((a, b, nbytes))

        def timed_load(prompt_ids):
            self.pos = 0
            load(prompt_ids)

        eng._launch_persistent = timed_launch
        eng._load_prompt = timed_load

    def summary(self):
        self.torch.cuda.synchronize(self.eng.device)
        secs = [a.elapsed_time(b) / 1e3 for a, b, _ in self.records]
        nbytes = [n for _, _, n in self.records]
        k = len(secs)
        return k, sum(nbytes) / k, sum(secs) / k


def traffic_for(kernel: str, positions, algorithmic_bytes: float):
    """(HBM bytes of the timed launch, where the figure comes from) from the
    committed rocprofv3 counter summary (profiles/hbm_traffic.json: FETCH_SIZE
    and WRITE_SIZE of one profiled launch, each scaled by what the same counter
    reads for a plain copy of known size), or (None, None) when none is
    committed for *kernel*.  When the committed launch covered the same
    positions as this run's timed launch (the same command), its measured
    bytes are the figure; otherwise its ratio of HBM bytes to algorithmic bytes
    is applied to this launch's algorithmic bytes, and the source says so."""
    path = ROOT / "profiles" / "hbm_traffic.json"
    if not path.exists():
        return None, None
    try:
        entries = json.loads(path.read_text()).get(kernel)
        if isinstance(entries, dict):
            entries = [entries]
        # the committed launch over the same positions, else the first one
        entry = next((e for e in entries
                      if list(e.get("timed_positions", [])) == list(positions)), entries[0])
        hbm, alg = float(entry["hbm_bytes"]), float(entry["algorithmic_bytes"])
        counted = entry.get("launch", "a committed counter run")
        if list(entry.get("timed_positions", [])) == list(positions):
            return round(hbm), f"rocprofv3 FETCH_SIZE + WRITE_SIZE of this launch ({counted})"
        ratio = hbm / alg
        return (round(ratio * algorithmic_bytes),
                f"committed counter ratio {ratio:.4f} (HBM bytes per algorithmic byte, counted "
                f"on {counted}) times this launch's algorithmic bytes")
    except (ValueError, KeyError, TypeError, ZeroDivisionError, AttributeError, IndexError):
        return None, None


def copy_probe(nbytes: int = 1 << 30) -> int:
    """A plain device copy of *nbytes* (three launches): the calibration kernel
    for the FETCH_SIZE / WRITE_SIZE counters."""
    import torch

    src = torch.ones(nbytes // 4, dtype=torch.int32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes": nbytes, "launches": 3}), flush=True)
    return 0


def cpu_baseline(weights, prompt, budget_s: float) -> dict:
    """The CPU oracle (a restatement of the authored HIR run the way the
    reference evaluator runs it) on this host's cores: decode steps over the
    same weights and prompt until *budget_s* of work is done."""
    import torch

    from oracle import qwen3_hir as O

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    orc = O.Qwen3Oracle(O.C2, weights)
    caches = orc.init_caches()
    ids = torch.tensor(prompt, dtype=torch.int64)
    O.generation_rope(O.C2)
    steps, t0 = 0, time.perf_counter()
    with torch.no_grad():
        while steps < len(prompt):
            args = orc.prepare_inputs_for_generation(ids, steps, caches)
            _, fresh = orc.forward(*args)
            caches = orc.append_cache(caches, fresh)
            steps += 1
            if time.perf_counter() - t0 >= budget_s:
                break
    dt = time.perf_counter() - t0
    return {"value": round(steps / dt, 4), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{steps} decode steps (positions 0..{steps - 1} of the 32-token prompt, "
                      f"same weights) of the oracle in torch on {threads} threads of "
                      f"'{cpu_model()}', {dt:.1f} s"}


def bench_c3(args) -> int:
    """Workload C3: the same model at batch 32, every sequence with a
    4096-token random context (built untimed: by default prefilled one
    sequence at a time, 32 positions per pass; `--c3-context walk` walks the
    contexts with batched decode steps instead), then `--steps` (default 256)
    timed steps of 32 tokens each."""
    import torch

    from tilefoundry_amd import _lib
    from tilefoundry_amd._lib import ptr
    from tilefoundry_amd.qwen3 import QWEN3_1_7B, synthetic_weights
    from tilefoundry_amd.qwen3.batch_engine import BatchEngine

    cfg = QWEN3_1_7B
    batch, ctx = 32, 4096
    steps = args.steps if args.steps_given else 256
    t0 = time.perf_counter()
    weights = synthetic_weights(cfg, seed=0)
    eng = BatchEngine(cfg, weights, batch=batch, device="cuda:0", max_new=steps,
                      prompt_room=ctx, splits=args.c3_splits)
    prompts = []
    for b in range(batch):
        g = torch.Generator().manual_seed(1000 + b)
        prompts.append(torch.randint(0, cfg.vocab_size, (ctx,), generator=g).tolist())
    t1 = time.perf_counter()
    if args.c3_context == "prefill":
        eng.prefill(prompts)                    # the contexts, untimed
    else:
        eng._load_prompts(prompts)
        eng.run_steps(ctx - 1)
    torch.cuda.synchronize()
    print(f"[bench] c3 setup {t1 - t0:.1f}s, contexts ({args.c3_context}, {batch} x {ctx - 1} "
          f"positions) {time.perf_counter() - t1:.1f}s", file=sys.stderr, flush=True)
    stream = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start = time.perf_counter()
    a.record(stream)
    eng.run_steps(steps)
    b.record(stream)
    torch.cuda.synchronize()
    seconds = time.perf_counter() - start
    eng.check_errors()
    tok_s = batch * steps / seconds
    positions = range(ctx - 1, ctx - 1 + steps)
    w_bytes = cfg.weight_bytes_per_step()
    kv = sum(eng.kv_bytes_at([p] * batch) for p in positions) / steps
    step_bytes = w_bytes + kv
    step_bw = step_bytes * steps / seconds

    # the dominant kernels: attention over the 32 caches, timed on their own for
    # layer 0 at the final positions (they rewrite the same new K/V row each time)
    L, s = eng._lib, stream.cuda_stream
    w = eng.layers[0]
    rounds = args.kernel_rounds
    pos_now = int(eng.pos[0].item())
    kv_read = batch * pos_now * cfg.num_key_value_heads * cfg.head_dim * 2   # K (or V) bytes

    def scores():
        L.tfd_attn_rope_scores_paged_batched(
            ptr(eng.qkv), eng.qkv_n, ptr(w["gamma_q"]), ptr(w["gamma_k"]), ptr(eng.cos),
            ptr(eng.sin), eng.cap, ptr(eng.pos), ptr(eng.page_table), eng.max_pages,
            ptr(eng.kpool[0]), ptr(eng.vpool[0]), eng.num_pages, batch, eng.HQ, eng.HKV, eng.D,
            eng.scale, eng.eps, ptr(eng.scores), eng.score_stride, ptr(eng.smax),
            ptr(eng.snew), eng.nsplit, eng.split_tiles, ptr(eng.err), s)

    def pv():
        L.tfd_attn_pv_combine_paged_batched(
            ptr(eng.qkv), eng.qkv_n, ptr(eng.pos), ptr(eng.page_table), eng.max_pages,
            ptr(eng.vpool[0]), eng.num_pages, batch, eng.HQ, eng.HKV, eng.D, ptr(eng.scores),
            eng.score_stride, ptr(eng.smax), ptr(eng.snew), ptr(eng.psum), ptr(eng.pout),
            eng.nsplit, eng.split_tiles, ptr(eng.counters), ptr(eng.attn), ptr(eng.err), s)

    def time_it(fn):
        fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(rounds):
            fn()
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_time(e1) / 1e3 / rounds

    sc_s, pv_s = time_it(scores), time_it(pv)
    # tiles per split at the final position (split_tiles 0: derived from it)
    tiles_now = (pos_now + 63) // 64
    split_tiles = eng.split_tiles or (tiles_now + eng.nsplit - 1) // eng.nsplit
    att_bw = 2 * kv_read / (sc_s + pv_s)
    line = {
        "metric": "decode tok/s bs=32 Qwen3-1.7B-arch bf16, 4096-token contexts "
                  "(config C3); achieved HBM TB/s vs 8 TB/s peak",
        "value": round(tok_s, 1), "unit": "tok/s", "n_gpus": 1, "steps": steps, "warmup": 0,
        "ms_per_step": round(1e3 * seconds / steps, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random-init N(0,0.02) weights seed 0, 32 random 4096-id contexts)",
        "config": {"workload": "C3: Qwen3-1.7B-arch bf16 decode, batch 32, 4096-token contexts, "
                               f"{steps} new tokens per sequence, 16-token KV pages",
                   "batch": batch, "context": ctx, "new_tokens": steps,
                   "context_built_by": args.c3_context},
        "step_roofline": {"bound": "hbm", "bytes_per_step": int(step_bytes),
                          "achieved": round(step_bw / 1e9, 1), "peak": HBM_PEAK / 1e9,
                          "unit": "GB/s", "frac": round(step_bw / HBM_PEAK, 4),
                          "roofline_tok_s": round(batch * HBM_PEAK / step_bytes, 1)},
        "roofline": {"bound": "hbm", "kernel": "attn_rope_scores + attn_pv_combine (batched, "
                                               "one layer)",
                     "achieved": round(att_bw / 1e9, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                     "frac": round(att_bw / HBM_PEAK, 4), "traffic": None,
                     "bytes_per_launch": kv_read, "scores_us": round(sc_s * 1e6, 2),
                     "pv_us": round(pv_s * 1e6, 2), "splits": eng.nsplit,
                     "split_positions": 64 * split_tiles},
    }
    print(json.dumps(line), flush=True)
    return 0


# What each of the XCD kernel's 14 per-layer stamps marks, per role (the
# attention ranks are blocks 0..127, rank = block / 8 < 16; the streaming
# ranks the rest)
TIMELINE_STAMPS = {
    "attention": ["layer start", "tiles, q/k scales, o slab requested", "qkv staged",
                  "scores done", "(P.V start)", "P.V partials out", "(merge start)",
                  "merged outputs out", "o input staged", "o partials out", "h1 staged",
                  "gate/up out", "SwiGLU staged", "down partials out, down sums published"],
    "streaming": ["layer start", "qkv out", "gate/up rows + down slab requested", "", "", "",
                  "", "", "o input staged", "o partials out", "o sums published, h1 staged",
                  "gate/up out", "SwiGLU staged", "down partials out, layer output staged"],
}


def timeline(ctxs) -> int:
    """Per-role device-clock stamps of the XCD kernel on the C2 model: one
    step after walking a random prompt of each context length; for each stamp,
    min / median / max over the role's blocks of (stamp - the layer's earliest
    start) in us, averaged over layers 2 .. L-2; then the head's stamps."""
    import torch

    from tilefoundry_amd.qwen3 import QWEN3_1_7B, synthetic_weights
    from tilefoundry_amd.qwen3.engine import Engine

    cfg = QWEN3_1_7B
    weights = synthetic_weights(cfg, seed=0)
    eng = Engine(cfg, weights, device="cuda:0", max_new=max(ctxs) + 8, prompt_room=8,
                 mode="xcd")
    L, per = cfg.num_hidden_layers, 14
    n_attn = 16 * 8
    for ctx in ctxs:
        g = torch.Generator().manual_seed(0)
        prompt = torch.randint(0, cfg.vocab_size, (ctx,), generator=g).tolist()
        st = eng.phase_timeline(prompt, 3)[1:]                # drop the first step
        S, B = st.shape[0], st.shape[1]
        step_us = (st[-1, :, -1, 1].median() - st[0, :, -1, 1].median()).item() / (S - 1)
        s = st[0].reshape(B, -1)
        print(f"== ctx {ctx}: step {step_us:.1f} us", flush=True)
        for role, sel in (("attention", slice(0, n_attn)), ("streaming", slice(n_attn, B))):
            print(f"  {role} ranks: stamp  min  median  max", flush=True)
            for k in range(per):
                if not TIMELINE_STAMPS[role][k]:
                    continue
                v = [(s[sel, l * per + k] - s[:, l * per].min()) for l in range(2, L - 1)]
                mn = sum(x.min().item() for x in v) / len(v)
                md = sum(x.median().item() for x in v) / len(v)
                mx = sum(x.max().item() for x in v) / len(v)
                print(f"    {k:2d} {mn:6.2f} {md:6.2f} {mx:6.2f}  {TIMELINE_STAMPS[role][k]}",
                      flush=True)
        h = s[:, L * per:]
        t0 = s[:, L * per - 1].median()
        names = ["head start", "head done", "(pick start)", "pick done"]
        print("  head (us after the last layer's median end, median / max): " + ", ".join(
            f"{names[k]} {(h[:, k] - t0).median().item():.1f} / {(h[:, k] - t0).max().item():.1f}"
            for k in range(h.shape[1])), flush=True)
    return 0


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2048)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--cpu-budget", type=float, default=20.0,
                    help="seconds of CPU-oracle work for the cpu_baseline leg (0 skips it)")
    ap.add_argument("--kernel-rounds", type=int, default=20)
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a 1 GiB device copy (counter calibration) and exit")
    ap.add_argument("--mode", default="xcd", choices=("persistent", "xcd", "graph"),
                    help="persistent: one cooperative launch per run of steps; xcd: the same "
                         "with each layer split over the 8 XCDs; graph: a captured graph of "
                         "per-phase launches replayed per token")
    ap.add_argument("--timeline", default=None, metavar="CTX[,CTX...]",
                    help="only print the XCD kernel's per-role phase timeline on the C2 model "
                         "at these context lengths and exit")
    ap.add_argument("--c3-context", default="prefill", choices=("prefill", "walk"),
                    help="c3: build the 4096-token contexts by prefill (default) or by "
                         "walking them with batched decode steps")
    ap.add_argument("--c3-splits", type=int, default=None, metavar="N",
                    help="c3: attention splits per (sequence, kv head), each split's length "
                         "following its sequence's position (default: the engine's choice)")
    ap.add_argument("--config", default="c2", choices=("c2", "c3"),
                    help="c2: the headline batch-1 workload; c3: batch 32 over 4096-token "
                         "contexts")
    args = ap.parse_args(argv)
    args.steps_given = any(a == "--steps" or a.startswith("--steps=") for a in (argv or sys.argv))
    if args.copy_probe:
        return copy_probe()
    if args.timeline:
        return timeline([int(c) for c in args.timeline.split(",")])
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (every box here "
              "has one MI355X); run with --gpus 1", file=sys.stderr)
        return 2

    if args.config == "c3":
        return bench_c3(args)

    import torch

    from tilefoundry_amd.qwen3 import QWEN3_1_7B, synthetic_weights
    from tilefoundry_amd.qwen3.engine import Engine

    cfg = QWEN3_1_7B
    t0 = time.perf_counter()
    weights = synthetic_weights(cfg, seed=0)
    g = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, cfg.vocab_size, (32,), generator=g).tolist()
    run_len = max(args.steps, 2048)            # new tokens of the whole run
    skip = run_len - args.steps                 # decoded untimed before the timed ones
    eng = Engine(cfg, weights, device="cuda:0", max_new=run_len, prompt_room=len(prompt),
                 mode=args.mode)
    clock = LaunchClock(eng) if args.mode in ("persistent", "xcd") else None
    print(f"[bench] weights + engine + capture {time.perf_counter() - t0:.1f}s", file=sys.stderr,
          flush=True)

    # untimed warmup: a short generation from the same prompt
    if args.warmup:
        eng.generate(prompt, min(args.warmup, run_len))
    # the timed region: walk the prompt and the first `skip` new tokens
    # (untimed), then exactly --steps steps
    pl = len(prompt)
    eng._load_prompt(prompt)
    eng.run_steps(pl - 1 + skip)
    torch.cuda.synchronize()
    if clock is not None:
        clock.armed = True
    start = time.perf_counter()
    eng.run_steps(args.steps)
    torch.cuda.synchronize()
    seconds = time.perf_counter() - start
    if clock is not None:
        clock.armed = False
    eng.check_errors()
    first_pos = pl - 1 + skip
    tokens = eng.sam[first_pos: first_pos + args.steps].tolist()

    # algorithmic bytes: weights once per step + K/V of every position read and the new one written
    w_bytes = cfg.weight_bytes_per_step()
    kv_bytes = sum(eng.kv_bytes_at(p) for p in range(first_pos, first_pos + args.steps))
    step_bytes = w_bytes + kv_bytes / args.steps
    tok_s = args.steps / seconds
    step_bw = step_bytes * tok_s

    if clock is not None:
        launches, bytes_per_launch, launch_s = clock.summary()
        kernel = "k_decode_persistent<4,12,128,2>" if args.mode == "persistent" else "k_decode_xcd"
        traffic, traffic_source = traffic_for(
            kernel, [first_pos, first_pos + args.steps - 1], bytes_per_launch)
        bw = bytes_per_launch / launch_s
        roofline = {"bound": "hbm", "kernel": f"{kernel} (whole decode steps per launch)",
                    "achieved": round(bw / 1e9, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                    "frac": round(bw / HBM_PEAK, 4),
                    "traffic": traffic, "traffic_source": traffic_source,
                    "bytes_per_launch": int(bytes_per_launch),
                    "avg_launch_ms": round(launch_s * 1e3, 3), "launches": launches}
    else:
        gu_s = time_gate_up(eng, args.kernel_rounds)
        gu_bytes = 2 * cfg.intermediate_size * cfg.hidden_size * 2 + 2 * cfg.hidden_size * 2 \
            + cfg.intermediate_size * 2
        gu_bw = gu_bytes / gu_s
        roofline = {"bound": "hbm", "kernel": "k_gemv<4,4,norm,swiglu> (gate/up, 12288x2048)",
                    "achieved": round(gu_bw / 1e9, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                    "frac": round(gu_bw / HBM_PEAK, 4), "traffic": None,
                    "bytes_per_launch": gu_bytes, "avg_us": round(gu_s * 1e6, 3)}

    line = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * seconds / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(tok_s / REFERENCE_TOKS, 3),
        "dtype": "bf16",
        "data": "synthetic (random-init N(0,0.02) weights seed 0, random 32-token prompt)",
        "config": {"workload": "C2: Qwen3-1.7B-arch bf16 decode, batch 1, 32-token prompt, "
                               f"{run_len} greedy new tokens, 16-token KV pages; timed: new "
                               f"tokens {skip + 1}..{run_len} (positions {first_pos}.."
                               f"{first_pos + args.steps - 1})",
                   "mode": args.mode,
                   "batch": 1, "prompt": pl, "new_tokens": run_len,
                   "timed_positions": [first_pos, first_pos + args.steps - 1],
                   "layers": cfg.num_hidden_layers, "hidden": cfg.hidden_size,
                   "vocab": cfg.vocab_size},
        "step_roofline": {"bound": "hbm", "bytes_per_step": int(step_bytes),
                          "achieved": round(step_bw / 1e9, 1), "peak": HBM_PEAK / 1e9,
                          "unit": "GB/s", "frac": round(step_bw / HBM_PEAK, 4),
                          "roofline_tok_s": round(HBM_PEAK / step_bytes, 1)},
        "roofline": roofline,
        "first_tokens": tokens[:8],
    }
    if args.cpu_budget > 0:
        line["cpu_baseline"] = cpu_baseline(weights, prompt, args.cpu_budget)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
