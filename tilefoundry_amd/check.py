"""``check``: hold what an implementation produced against a reference.

The reference's comparator (``src/tilefoundry/runtime/measure.py:61-378``, its
command line ``src/tilefoundry/cli/check.py:91-165``) is a contract, and this
module keeps it: the same eight predicates with the same definitions and bound
names, and the same refusals --

* there is no default bound: every output needs at least one predicate, and
  every predicate every one of its bounds;
* the expectations must name exactly the outputs produced (a nested tuple of
  tensors flattens to ``output``, ``output[0]``, ``output[1][0]`` ...);
* a discrete (integer / bool) output admits only ``equal``: one wrong token id
  is a total failure, never a small deviation;
* without a reference only ``nan_inf`` can be measured;
* candidate and reference must flatten to the same paths, shapes and dtypes.

``check(candidate, reference, inputs, expect=...)`` runs both callables on the
same inputs; ``compare`` measures outputs already produced.  The command line
(``python -m tilefoundry_amd.check``) runs one function of the Qwen3 twin
(``tilefoundry_amd.qwen3.twin``, the HIP path) on input files -- or compares two
output files -- against ``--expected`` files with ``--out / --fn / --<bound>``
stated in the reference's order.
"""
from __future__ import annotations

import argparse
import json
import math
import sys
from dataclasses import dataclass
from pathlib import Path
from typing import Callable, ClassVar, Mapping, Sequence

import torch

_TINY = 1e-12
_INT_OF = {torch.bfloat16: torch.int16, torch.float16: torch.int16, torch.float32: torch.int32,
           torch.float64: torch.int64}


@dataclass(frozen=True)
class Predicate:
    """One comparison and the bound(s) it holds an output to."""

    name: ClassVar[str] = ""
    bounds: ClassVar[tuple[str, ...]] = ()
    needs_reference: ClassVar[bool] = True
    discrete: ClassVar[bool] = False          # meaningful on an integer output
    guidance: ClassVar[str] = ""

    def measure(self, got: torch.Tensor, want: torch.Tensor | None) -> "Result":
        raise NotImplementedError

    def result(self, values: Mapping[str, float], ok: bool, note: str | None = None) -> "Result":
        return Result(self, dict(values), bool(ok), note)


@dataclass(frozen=True)
class Result:
    predicate: Predicate
    values: Mapping[str, float]
    passed: bool
    note: str | None = None


def _f(t: torch.Tensor) -> torch.Tensor:
    return t.detach().float().cpu()


@dataclass(frozen=True)
class AllClose(Predicate):
    atol: float
    rtol: float
    name = "allclose"
    bounds = ("atol", "rtol")
    guidance = "per element, |a - b| <= atol + rtol |b|: the one bad element an aggregate hides"

    def measure(self, got, want):
        a, b = _f(got), _f(want)
        excess = ((a - b).abs() - (self.atol + self.rtol * b.abs())).max().item()
        return self.result({"max_violation": excess if math.isnan(excess) else max(excess, 0.0)},
                           excess <= 0.0)


@dataclass(frozen=True)
class RelL2(Predicate):
    max: float
    name = "rel_l2"
    bounds = ("max",)
    guidance = "||a - b|| / ||b||: aggregate magnitude"

    def measure(self, got, want):
        a, b = _f(got), _f(want)
        dist, ref = (a - b).norm().item(), b.norm().item()
        if ref <= _TINY:
            return self.result({"absolute_l2": dist}, dist <= self.max,
                               "the reference is all zero: an absolute L2 distance")
        return self.result({"rel_l2": dist / ref}, dist / ref <= self.max)


@dataclass(frozen=True)
class Cosine(Predicate):
    min: float
    name = "cosine"
    bounds = ("min",)
    guidance = "cosine of the angle: aggregate direction, catches a systematic bias"

    def measure(self, got, want):
        a, b = _f(got).reshape(-1), _f(want).reshape(-1)
        na, nb = a.norm().item(), b.norm().item()
        if na <= _TINY and nb <= _TINY:
            return self.result({"cosine": 1.0}, 1.0 >= self.min, "both sides are all zero")
        if na <= _TINY or nb <= _TINY:
            return self.result({"cosine": 0.0}, False, "one side is all zero, the other not")
        c = (torch.dot(a, b) / (a.norm() * b.norm())).item()
        return self.result({"cosine": c}, c >= self.min)


@dataclass(frozen=True)
class Equal(Predicate):
    name = "equal"
    discrete = True
    guidance = "bitwise; for discrete outputs, where one wrong value is total failure"

    def measure(self, got, want):
        bad = int((got.detach().cpu() != want.detach().cpu()).sum().item())
        return self.result({"mismatched": float(bad), "elements": float(got.numel())}, bad == 0)


def ordered_bits(t: torch.Tensor) -> torch.Tensor:
    """A float tensor's bit patterns as int64, ordered as the floats are (the
    difference of two is the count of representable values between them)."""
    try:
        raw = t.detach().cpu().contiguous().view(_INT_OF[t.dtype]).to(torch.int64)
    except KeyError:
        raise ValueError(f"check: ulp is defined on a float output, not on {t.dtype}") from None
    sign = 1 << (8 * t.element_size() - 1)
    return torch.where(raw >= 0, raw, -(raw + sign))


@dataclass(frozen=True)
class Ulp(Predicate):
    max: float
    name = "ulp"
    bounds = ("max",)
    guidance = "distance in units of last place, at the output's own dtype"

    def measure(self, got, want):
        d = (ordered_bits(got) - ordered_bits(want)).abs().max().item()
        return self.result({"max_ulp": float(d)}, d <= self.max)


@dataclass(frozen=True)
class MaxAbs(Predicate):
    max: float
    name = "max_abs"
    bounds = ("max",)
    guidance = "largest absolute difference"

    def measure(self, got, want):
        d = (_f(got) - _f(want)).abs().max().item()
        return self.result({"max_abs": d}, d <= self.max)


@dataclass(frozen=True)
class MaxRel(Predicate):
    max: float
    name = "max_rel"
    bounds = ("max",)
    guidance = "largest |a - b| / |b| (0 where both are 0, inf where only b is)"

    def measure(self, got, want):
        a, b = _f(got), _f(want)
        diff, mag = (a - b).abs(), b.abs()
        rel = torch.where(mag > 0, diff / mag.clamp_min(_TINY),
                          torch.where(diff == 0, torch.zeros_like(diff),
                                      torch.full_like(diff, float("inf"))))
        r = rel.max().item()
        return self.result({"max_rel": r}, r <= self.max)


@dataclass(frozen=True)
class NanInf(Predicate):
    name = "nan_inf"
    needs_reference = False
    guidance = "no NaN and no Inf; the one predicate that needs no reference"

    def measure(self, got, want=None):
        t = got.detach().cpu()
        nan, inf = int(torch.isnan(t).sum().item()), int(torch.isinf(t).sum().item())
        return self.result({"nan": float(nan), "inf": float(inf)}, nan == 0 and inf == 0)


PREDICATES: dict[str, type[Predicate]] = {
    p.name: p for p in (AllClose, RelL2, Cosine, Equal, Ulp, MaxAbs, MaxRel, NanInf)}
BOUNDS = sorted({b for p in PREDICATES.values() for b in p.bounds})


@dataclass(frozen=True)
class OutputCheck:
    path: str
    shape: tuple[int, ...]
    dtype: str
    ref_norm: float | None
    results: tuple[Result, ...]

    @property
    def passed(self) -> bool:
        return all(r.passed for r in self.results)


@dataclass(frozen=True)
class Report:
    outputs: tuple[OutputCheck, ...]

    @property
    def passed(self) -> bool:
        return all(o.passed for o in self.outputs)

    def lines(self) -> list[str]:
        out = []
        for o in self.outputs:
            out.append(f"{'PASS' if o.passed else 'FAIL'}  {o.path}  {o.dtype}{list(o.shape)}"
                       + ("" if o.ref_norm is None else f"  |ref| {o.ref_norm:.6g}"))
            for r in o.results:
                vals = ", ".join(f"{k} {v:.6g}" for k, v in r.values.items())
                bound = ", ".join(f"{b} {getattr(r.predicate, b)}" for b in r.predicate.bounds)
                out.append(f"    {'ok  ' if r.passed else 'FAIL'} {r.predicate.name}: {vals}"
                           + (f"  (bound {bound})" if bound else "")
                           + (f"  -- {r.note}" if r.note else ""))
        return out

    def as_json(self) -> dict:
        return {"passed": self.passed, "outputs": [
            {"path": o.path, "shape": list(o.shape), "dtype": o.dtype, "ref_norm": o.ref_norm,
             "passed": o.passed,
             "results": [{"fn": r.predicate.name, "passed": r.passed, "values": dict(r.values),
                          "bounds": {b: getattr(r.predicate, b) for b in r.predicate.bounds},
                          "note": r.note} for r in o.results]} for o in self.outputs]}


def flatten(x, path: str = "output") -> list[tuple[str, torch.Tensor]]:
    """A tensor or nested tuple of tensors as ``[(path, tensor)]``."""
    if isinstance(x, torch.Tensor):
        return [(path, x)]
    if isinstance(x, tuple):
        return [leaf for i, item in enumerate(x) for leaf in flatten(item, f"{path}[{i}]")]
    raise TypeError(f"check: {path} must be a torch.Tensor or a tuple of them, "
                    f"got {type(x).__name__}")


def _cover(paths: Sequence[str], expect: Mapping[str, Sequence[Predicate]],
           has_reference: bool) -> None:
    unknown = sorted(set(expect) - set(paths))
    if unknown:
        raise ValueError(f"check: {unknown} name no output; this run produced {list(paths)}")
    for path in paths:
        stated = tuple(expect.get(path) or ())
        if not stated:
            raise ValueError(
                f"check: no comparison requested for output {path!r}.  Every output needs at "
                "least one predicate; there is no default, because a default bound that cannot "
                "be met trains you to ignore FAIL (one f32 -> bf16 rounding alone is rel_l2 "
                "1.66e-3)")
        if not has_reference:
            two_sided = sorted({p.name for p in stated if p.needs_reference})
            if two_sided:
                alone = sorted(n for n, p in PREDICATES.items() if not p.needs_reference)
                raise ValueError(f"check: {path!r} asks for {two_sided} with no reference to "
                                 f"compare against; without one only {alone} can be measured")


def _admit(path: str, t: torch.Tensor, predicates: Sequence[Predicate]) -> None:
    if t.dtype.is_floating_point:
        return
    for p in predicates:
        if not p.discrete:
            raise ValueError(
                f"check: {path} is {t.dtype}; {p.name} is not meaningful on a discrete output "
                "(one wrong value is both a tiny numerical deviation and a completely wrong "
                "result).  Use equal.")


def compare(produced, expected, *, expect: Mapping[str, Sequence[Predicate]]) -> Report:
    """Measure outputs already produced (``expected`` may be None)."""
    got = flatten(produced)
    if not got:
        raise ValueError("check: the candidate produced no tensor, so nothing was compared")
    paths = [p for p, _ in got]
    _cover(paths, expect, expected is not None)
    ref: dict[str, torch.Tensor] = {}
    if expected is not None:
        want = flatten(expected)
        if paths != [p for p, _ in want]:
            raise ValueError(f"check: candidate/reference output structures differ: {paths} vs "
                             f"{[p for p, _ in want]}")
        for (path, a), (_, b) in zip(got, want):
            if a.shape != b.shape or a.dtype != b.dtype:
                raise ValueError(f"check: {path} shape/dtype mismatch: candidate "
                                 f"{tuple(a.shape)}/{a.dtype} vs reference "
                                 f"{tuple(b.shape)}/{b.dtype}")
            ref[path] = b
    outs = []
    for path, a in got:
        preds = tuple(expect[path])
        _admit(path, a, preds)
        b = ref.get(path)
        outs.append(OutputCheck(path, tuple(a.shape), str(a.dtype).removeprefix("torch."),
                                None if b is None else _f(b).norm().item(),
                                tuple(p.measure(a, b) for p in preds)))
    return Report(tuple(outs))


def check(candidate: Callable, reference: Callable | None, inputs: tuple, *,
          expect: Mapping[str, Sequence[Predicate]]) -> Report:
    """Run *candidate* (and *reference*, when there is one) on the same inputs and
    measure every output against the predicates *expect* states for it."""
    produced = candidate(*inputs)
    got_paths = [p for p, _ in flatten(produced)]
    _cover(got_paths, expect, reference is not None)
    return compare(produced, None if reference is None else reference(*inputs), expect=expect)


# ---------------------------------------------------------------------------
# the command line
# ---------------------------------------------------------------------------
class _Ordered(argparse.Action):
    """Record --out / --fn / --<bound> in the order given."""

    def __call__(self, parser, ns, values, option_string=None):
        seq = getattr(ns, "stated", None) or []
        seq.append((self.dest, values))
        ns.stated = seq


def expectations(stated: Sequence[tuple[str, object]] | None) -> dict[str, tuple[Predicate, ...]]:
    """The ``--out`` / ``--fn`` / bound sequence as each output's predicates."""
    if not stated:
        raise ValueError("no comparison requested: every output needs --out PATH and at least "
                         "one --fn (see --help for the functions)")
    grouped: dict[str, list[tuple[str, dict[str, float]]]] = {}
    current = None
    fn = None
    for flag, value in stated:
        if flag == "out":
            if value in grouped:
                raise ValueError(f"--out {value!r} was given twice; state its functions together")
            current, fn = value, None
            grouped[current] = []
        elif flag == "fn":
            if current is None:
                raise ValueError(f"--fn {value} came before any --out; name the output first")
            fn = (value, {})
            grouped[current].append(fn)
        else:
            if fn is None:
                raise ValueError(f"--{flag} came before any --fn; name the function it bounds")
            name, bounds = fn
            if flag not in PREDICATES[name].bounds:
                raise ValueError(f"--fn {name} takes {list(PREDICATES[name].bounds) or 'no bounds'}"
                                 f", not --{flag}")
            if flag in bounds:
                raise ValueError(f"--{flag} was given twice for one --fn {name}")
            bounds[flag] = float(value)
    built = {}
    for path, fns in grouped.items():
        if not fns:
            raise ValueError(f"--out {path!r} states no --fn; there is no default bound")
        made = []
        for name, bounds in fns:
            missing = [b for b in PREDICATES[name].bounds if b not in bounds]
            if missing:
                raise ValueError(f"--fn {name} needs {['--' + b for b in missing]}; a bound has "
                                 "no default")
            made.append(PREDICATES[name](**bounds))
        built[path] = tuple(made)
    return built


def guidance() -> str:
    width = max(len(n) for n in PREDICATES)
    lines = ["comparison -- every output needs at least one --fn, and every --fn its bounds:",
             ""]
    for name in sorted(PREDICATES):
        p = PREDICATES[name]
        b = " ".join(f"--{x} X" for x in p.bounds)
        lines.append(f"  --fn {name:<{width}} {b:<18} {p.guidance}")
    lines += ["", "a bf16 result rounds once per f32 -> bf16 landing, at most 2^-9 = 1.95e-3 of "
              "the value each: take rtol ~ 2^-9 * sqrt(n) for the longest serial chain of n "
              "landings; atol covers the elements near zero."]
    return "\n".join(lines)


def load_tensors(path: str) -> list[torch.Tensor]:
    """Tensors of a file: ``.npy`` (one; bf16 stored as its int16 bits is not
    recognisable, so store bf16 in ``.safetensors`` or ``.pt``), ``.safetensors``
    (every tensor, in key order), ``.pt`` (a tensor or tuple, weights-only load)."""
    p = Path(path)
    if p.suffix == ".npy":
        import numpy as np

        return [torch.from_numpy(np.load(p, allow_pickle=False))]
    if p.suffix == ".safetensors":
        from safetensors.torch import load_file

        d = load_file(str(p))
        return [d[k] for k in sorted(d)]
    if p.suffix == ".pt":
        obj = torch.load(p, map_location="cpu", weights_only=True)
        return [obj] if isinstance(obj, torch.Tensor) else list(obj)
    raise ValueError(f"{path}: not .npy, .safetensors or .pt")


def _pack(leaves: list[torch.Tensor]):
    return leaves[0] if len(leaves) == 1 else tuple(leaves)


def _twin_call(source: str, ckpt: str | None, inputs: list[torch.Tensor], device: str):
    """Run one function of the Qwen3 twin: ``qwen3:<fn>`` for a root function
    (embed, final_rms_norm, lm_head) or ``qwen3:layer<i>.<fn>`` (input_rms_norm,
    self_attention, mlp, decoder_layer).  Weight parameters are bound by
    canonical name from the checkpoint; the inputs fill the activations, in the
    function's own parameter order."""
    import inspect

    from .checkpoint import load_qwen3
    from .qwen3.twin import RootTwin

    model, _, selector = source.partition(":")
    if model != "qwen3":
        raise ValueError(f"{source}: the command line runs the Qwen3 twin (qwen3:<selector>)")
    if ckpt is None:
        raise ValueError(f"{source}: the twin's weights come from --ckpt")
    cfg, weights = load_qwen3(ckpt)
    root = RootTwin(cfg)
    head, _, fn = selector.rpartition(".")
    if head:
        if not (head.startswith("layer") and head[5:].isdigit()
                and int(head[5:]) < cfg.num_hidden_layers):
            raise ValueError(f"{source}: {head!r} is no layer of this {cfg.num_hidden_layers}-layer "
                             "checkpoint")
        target, prefix = root.layer, head + "."
        allowed = ("input_rms_norm", "self_attention", "mlp", "decoder_layer")
    else:
        target, prefix = root, ""
        allowed = ("embed", "final_rms_norm", "lm_head")
    if fn not in allowed:
        raise ValueError(f"{source}: {fn!r} is none of {allowed}")
    params = list(inspect.signature(getattr(target, fn)).parameters)
    acts = iter(t.to(device) for t in inputs)
    args = []
    for name in params:
        if prefix + name in weights or name in weights:
            args.append(weights.get(prefix + name, weights.get(name)).to(device).contiguous())
        else:
            try:
                args.append(next(acts))
            except StopIteration:
                raise ValueError(f"{source}: too few --input files for its activations "
                                 f"(parameter {name!r})") from None
    if next(acts, None) is not None:
        raise ValueError(f"{source}: more --input files than activations")
    return getattr(target, fn)(*args)


def main(argv: Sequence[str] | None = None) -> int:
    ap = argparse.ArgumentParser(prog="python -m tilefoundry_amd.check",
                                 description=__doc__, epilog=guidance(),
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("source", nargs="?", help="qwen3:<selector> (a twin function to run); "
                    "omit it to compare --candidate files")
    ap.add_argument("--input", action="append", default=[], metavar="PATH",
                    help="an activation file; repeat per input, in parameter order")
    ap.add_argument("--candidate", action="append", default=[], metavar="PATH",
                    help="an output file, instead of running a source")
    ap.add_argument("--ckpt", metavar="DIR", help="checkpoint directory for the twin's weights")
    ap.add_argument("--expected", action="append", default=[], metavar="PATH",
                    help="the reference's output file(s)")
    ap.add_argument("--device", default="cuda:0")
    ap.add_argument("--out", action=_Ordered, metavar="OUTPUT",
                    help="the output the following --fn apply to: output, output[0], ...")
    ap.add_argument("--fn", action=_Ordered, choices=sorted(PREDICATES))
    for b in BOUNDS:
        ap.add_argument(f"--{b}", action=_Ordered, type=float, help=argparse.SUPPRESS)
    ap.add_argument("--json", action="store_true", help="machine-readable report")
    args = ap.parse_args(argv)
    try:
        expect = expectations(getattr(args, "stated", None))
        if (args.source is None) == (not args.candidate):
            raise ValueError("give a source to run or --candidate files, not both or neither")
        if args.source is not None:
            produced = _twin_call(args.source, args.ckpt,
                                  [t for f in args.input for t in load_tensors(f)], args.device)
        else:
            produced = _pack([t for f in args.candidate for t in load_tensors(f)])
        expected = (_pack([t for f in args.expected for t in load_tensors(f)])
                    if args.expected else None)
        report = compare(produced, expected, expect=expect)
    except (ValueError, TypeError) as e:
        print(f"check: {e}", file=sys.stderr)
        return 2
    print(json.dumps(report.as_json(), indent=1) if args.json else "\n".join(report.lines()))
    return 0 if report.passed else 1


if __name__ == "__main__":
    raise SystemExit(main())
