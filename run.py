"""Continue a prompt on an MI355X with the HIP decode engines, and report the rate.

    python run.py --prompt "..." --max-new-tokens 2048 --ckpt /path/to/Qwen3-1.7B
    python run.py --synthetic c2 --random-prompt 32 --max-new-tokens 2048

The command line of ``examples/qwen3_1_7b-tilelang/run.py:61-97`` (``--prompt``,
``--max-new-tokens``, ``--ckpt``, ``--device``) and its report: the continuation,
then the rate over exactly the steps that produced it, with the prompt walk
reported apart.  A published checkpoint directory is read through
``tilefoundry_amd.checkpoint`` (the reference's alias tables and converters) and
its own tokenizer; ``config.json``'s ``model_type`` picks the engine (Qwen3,
Qwen3.5-MoE or Granite-4.0-H).  Without a checkpoint, ``--synthetic`` builds
random-init weights of a benchmark configuration (C1/C2 for Qwen3, C4, C5) and
the prompt comes as ids (``--prompt-ids``) or a seeded random draw
(``--random-prompt``); the continuation is then printed as ids.

Tokens are greedy unless ``--sample`` is given: then they are drawn on the device
(``tilefoundry_amd.sampling``) with the reference runtimes' defaults -- Qwen3.5's
published top-k 20 / top-p 0.95 at temperature 1.0
(``examples/qwen3_5_35b_a3b-tilelang/run.py:145-180``), Granite's softmax over
the whole vocabulary at temperature 1.0 (``examples/granite_4_0_h_small-cuda/
run.py:21-28``) -- which ``--temperature``, ``--top-k`` (0: the whole
vocabulary), ``--top-p`` and ``--sample-seed`` override.  Qwen3 (greedy only in
its reference) samples through the batched engine with one sequence.
"""
from __future__ import annotations

import argparse
import os
import sys
from pathlib import Path
from time import perf_counter

HERE = Path(__file__).resolve().parent
if str(HERE) not in sys.path:
    sys.path.insert(0, str(HERE))

NEED_GIB = {"qwen3": 12.0, "qwen3_5": 90.0, "granite": 40.0}


def pick_device(want: str | None, need_gib: float) -> str:
    """The emptiest visible GPU with room for the model, unless one is named."""
    if want:
        return want
    import torch

    if not torch.cuda.is_available():
        raise SystemExit("no GPU is visible: the engines are HIP kernels and have no CPU path")
    best = None
    for i in range(torch.cuda.device_count()):
        try:
            free, _ = torch.cuda.mem_get_info(i)
        except RuntimeError:
            continue
        gib = free / 2**30
        if gib >= need_gib and (best is None or gib > best[1]):
            best = (i, gib)
    if best is None:
        raise SystemExit(f"no visible GPU has {need_gib:.0f} GiB free "
                         f"(HIP_VISIBLE_DEVICES={os.environ.get('HIP_VISIBLE_DEVICES', 'unset')})")
    return f"cuda:{best[0]}"


def model_of(args) -> str:
    if args.model:
        return args.model
    if args.ckpt is None:
        return "qwen3"
    import json

    kind = json.loads((args.ckpt / "config.json").read_text(encoding="utf-8")).get("model_type", "")
    if kind.startswith("qwen3_5"):
        return "qwen3_5"
    if kind.startswith("granitemoehybrid"):
        return "granite"
    if kind.startswith("qwen3"):
        return "qwen3"
    raise SystemExit(f"{args.ckpt}: model_type {kind!r} is none of qwen3, qwen3_5_moe, "
                     "granitemoehybrid")


def prompt_of(args, tokenizer, vocab: int) -> list[int]:
    if args.prompt is not None:
        if tokenizer is None:
            raise SystemExit("a text prompt needs --ckpt with its tokenizer; "
                             "use --prompt-ids or --random-prompt with --synthetic")
        enc = tokenizer.encode(args.prompt)
        ids = list(getattr(enc, "ids", enc))
    elif args.prompt_ids is not None:
        ids = [int(t) for t in args.prompt_ids.split(",") if t.strip()]
    else:
        import torch

        g = torch.Generator().manual_seed(args.seed)
        ids = torch.randint(0, vocab, (args.random_prompt,), generator=g).tolist()
    if not ids:
        raise SystemExit("decode needs a prompt that encodes to at least one token")
    if any(not 0 <= t < vocab for t in ids):
        raise SystemExit(f"prompt ids must lie in [0, {vocab})")
    return ids


def xcd_fits(cfg, device) -> bool:
    """The XCD-partitioned kernel's shape and device (8 XCDs x 32 CUs)."""
    import torch

    shape = (cfg.hidden_size, cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim,
             cfg.intermediate_size) == (2048, 16, 8, 128, 6144)
    return shape and torch.cuda.get_device_properties(device).multi_processor_count == 256


#: --sample's defaults per model (the reference runtimes' own)
SAMPLE_DEFAULTS = {"qwen3": (1.0, 20, 0.95), "qwen3_5": (1.0, 20, 0.95),
                   "granite": (1.0, 0, 1.0)}


def sampling_of(args, model: str):
    """The Sampling the flags ask for, or None (greedy)."""
    if not args.sample:
        return None
    from tilefoundry_amd.sampling import Sampling

    t, k, p = SAMPLE_DEFAULTS[model]
    return Sampling(temperature=t if args.temperature is None else args.temperature,
                    top_k=k if args.top_k is None else args.top_k,
                    top_p=p if args.top_p is None else args.top_p, seed=args.sample_seed)


def build(args, model: str, device: str):
    """(make(prompt_len) -> engine, run(engine, prompt) -> (tokens, seconds of the
    continuation, seconds of the prompt walk), vocab, step mode)."""
    import torch

    sampling = sampling_of(args, model)
    if model == "qwen3":
        from tilefoundry_amd.qwen3 import QWEN3_1_7B, TINY, synthetic_weights
        from tilefoundry_amd.qwen3.engine import Engine

        if args.ckpt is not None:
            from tilefoundry_amd.checkpoint import load_qwen3

            cfg, w = load_qwen3(args.ckpt)
        else:
            # C1 is the reference's small CPU case; the engine computes in bf16
            cfg = QWEN3_1_7B if args.synthetic == "c2" else TINY.with_(dtype=torch.bfloat16)
            w = synthetic_weights(cfg, seed=args.seed)
        room = args.prompt_room
        if sampling is not None:
            from tilefoundry_amd.qwen3.batch_engine import BatchEngine

            def make_batch(prompt_len):
                return BatchEngine(cfg, w, batch=1, device=device, max_new=args.max_new_tokens,
                                   prompt_room=max(room, prompt_len + 8), sampling=sampling)

            def run_batch(eng, prompt):
                r = eng.generate([prompt], args.max_new_tokens, prefill=args.prefill)
                return r.tokens[0], r.seconds, r.prefill_seconds

            return make_batch, run_batch, cfg.vocab_size, "batch, sampled"
        mode = args.mode or ("xcd" if xcd_fits(cfg, device) else "persistent")

        def make(prompt_len):
            return Engine(cfg, w, device=device, max_new=args.max_new_tokens,
                          prompt_room=max(room, prompt_len + 8), mode=mode)

        def run(eng, prompt):
            r = eng.generate(prompt, args.max_new_tokens, prefill=args.prefill)
            return r.tokens, r.seconds, r.prefill_seconds

        return make, run, cfg.vocab_size, mode
    if model == "qwen3_5":
        from tilefoundry_amd.hybrid.qwen3_5 import Qwen35Config, Qwen35Engine, synthetic_weights

        if args.ckpt is not None:
            from tilefoundry_amd.checkpoint import load_qwen3_5

            cfg, w = load_qwen3_5(args.ckpt)
        else:
            cfg = Qwen35Config()
            w = synthetic_weights(cfg, seed=args.seed, device=device)
        engine_cls = Qwen35Engine
    else:
        from tilefoundry_amd.hybrid.granite import GraniteConfig, GraniteEngine, synthetic_weights

        if args.ckpt is not None:
            from tilefoundry_amd.checkpoint import load_granite

            cfg, w = load_granite(args.ckpt)
        else:
            cfg = GraniteConfig()
            w = synthetic_weights(cfg, seed=args.seed, device=device)
        engine_cls = GraniteEngine

    def make(prompt_len):
        return engine_cls(cfg, w, rows=1, device=device,
                          max_steps=prompt_len + args.max_new_tokens + 8, sampling=sampling)

    def run(eng, prompt):
        t0 = perf_counter()
        tokens, seconds, _ = eng.generate([prompt], args.max_new_tokens)
        return tokens[0], seconds, perf_counter() - t0 - seconds

    return make, run, cfg.vocab, "graph" if sampling is None else "graph, sampled"


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    src = ap.add_mutually_exclusive_group(required=True)
    src.add_argument("--ckpt", type=Path, help="published checkpoint directory")
    src.add_argument("--synthetic", choices=("c1", "c2", "c4", "c5"),
                     help="random-init weights of a benchmark configuration instead")
    prm = ap.add_mutually_exclusive_group(required=True)
    prm.add_argument("--prompt", help="prompt to continue (needs the checkpoint's tokenizer)")
    prm.add_argument("--prompt-ids", help="prompt as comma-separated token ids")
    prm.add_argument("--random-prompt", type=int, metavar="N", help="N seeded random token ids")
    ap.add_argument("--max-new-tokens", type=int, default=2048, metavar="TOKENS")
    ap.add_argument("--device", default=None, help="runtime device (default: an idle one)")
    ap.add_argument("--model", choices=("qwen3", "qwen3_5", "granite"), default=None,
                    help="engine (default: the checkpoint's model_type; c4/c5 imply theirs)")
    ap.add_argument("--mode", choices=("xcd", "persistent", "graph"), default=None,
                    help="Qwen3 step: XCD-partitioned or chip-wide persistent kernel, or a "
                         "graph of per-phase launches (default: xcd where it fits)")
    ap.add_argument("--prompt-room", type=int, default=64,
                    help="Qwen3: prompt positions the engine reserves")
    ap.add_argument("--seed", type=int, default=0, help="weights / random prompt seed")
    ap.add_argument("--prefill", action="store_true",
                    help="Qwen3: fill the prompt's cache in batched passes (32 positions per "
                         "pass) instead of walking it one decode step per token")
    ap.add_argument("--sample", action="store_true",
                    help="draw tokens instead of taking the largest logit (the model's "
                         "reference defaults unless the flags below say otherwise)")
    ap.add_argument("--temperature", type=float, default=None, help="--sample: temperature")
    ap.add_argument("--top-k", type=int, default=None,
                    help="--sample: candidates (1..64; 0: the whole vocabulary)")
    ap.add_argument("--top-p", type=float, default=None,
                    help="--sample: nucleus mass inside the top k")
    ap.add_argument("--sample-seed", type=int, default=0, help="--sample: seed of the draws")
    args = ap.parse_args(argv)
    if not args.sample and any(v is not None for v in (args.temperature, args.top_k,
                                                       args.top_p)):
        raise SystemExit("--temperature / --top-k / --top-p need --sample")
    if args.max_new_tokens < 1:
        raise SystemExit("--max-new-tokens must be at least 1")
    if args.synthetic in ("c4", "c5"):
        args.model = args.model or {"c4": "qwen3_5", "c5": "granite"}[args.synthetic]
    model = model_of(args)

    tokenizer = None
    if args.ckpt is not None and args.prompt is not None:
        from transformers import AutoTokenizer

        tokenizer = AutoTokenizer.from_pretrained(str(args.ckpt))
    device = pick_device(args.device, NEED_GIB[model])
    t0 = perf_counter()
    make, run, vocab, mode = build(args, model, device)
    prompt = prompt_of(args, tokenizer, vocab)
    eng = make(len(prompt))
    load = perf_counter() - t0

    tokens, seconds, prefill = run(eng, prompt)
    text = tokenizer.decode(tokens) if tokenizer is not None else " ".join(map(str, tokens))
    print(text)
    print()
    print(f"{len(tokens) / seconds:.1f} tok/s ({len(tokens)} tokens in {seconds:.3f}s, "
          f"{1e3 * seconds / len(tokens):.3f} ms/token)")
    print(f"  device {device}  |  {model} ({mode})  |  prompt {len(prompt)} tokens, "
          f"prefill {1e3 * prefill:.1f}ms  |  load {load:.1f}s  |  "
          f"{len(text)} characters generated")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
