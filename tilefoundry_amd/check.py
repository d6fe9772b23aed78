"""``check``: measure what an implementation produced against a reference,
under bounds the caller states.

What is kept from the reference (``src/tilefoundry/runtime/measure.py:61-378``
and the command line ``src/tilefoundry/cli/check.py:91-165, 532-648``) is its
contract, not its code:

* eight comparison functions and their bounds -- ``allclose`` (atol, rtol),
  ``rel_l2`` (max), ``cosine`` (min), ``equal``, ``ulp`` (max), ``max_abs``
  (max), ``max_rel`` (max), ``nan_inf`` -- and the quantities each reports
  (``max_violation``; ``rel_l2``, or ``absolute_l2`` against an all-zero
  reference; ``cosine``; ``mismatched`` and ``elements``; ``max_ulp``;
  ``max_abs``; ``max_rel``; ``nan`` and ``inf``);
* the refusals: no bound has a default, so every output names at least one
  function and every function all of its bounds; the stated outputs are
  exactly the ones produced (a nested tuple of tensors is addressed as
  ``output``, ``output[0]``, ``output[1][0]`` ...); an integer or bool output
  is judged by ``equal`` alone; without a reference only ``nan_inf`` can be
  measured; candidate and reference must have the same structure, shapes and
  dtypes;
* on the command line, ``--out`` / ``--fn`` / ``--<bound>`` read in the order
  written: a function belongs to the output named before it, a bound to the
  function named before it.

This module's own design: each comparison function is one row of a table
(its bounds, whether it needs a reference, whether it may judge integers, and
a measuring function that works on float64 arrays); a requirement is a
function name with its bound values; a report is a list of per-output
verdicts.  The command line runs a function of a runtime twin on the HIP path
-- ``qwen3:<selector>``, ``qwen3_5:<selector>`` or ``granite:<selector>`` with
the weights of a checkpoint directory -- or compares output files, against
``--expected`` files.
"""
from __future__ import annotations

import argparse
import inspect
import json
import math
import sys
from dataclasses import dataclass, field
from pathlib import Path
from typing import Callable, Mapping, Sequence

import numpy as np
import torch

_ZERO_NORM = 1e-12      # a norm at or below this is taken for an all-zero vector


# ---------------------------------------------------------------------------
# measurements: each takes the candidate and reference as float64 arrays (the
# reference None for a one-sided function) and returns (values, passed, note)
# ---------------------------------------------------------------------------
def _max_or_nan(x: np.ndarray) -> float:
    """The largest element, NaN when any element is NaN, 0 for an empty array."""
    if x.size == 0:
        return 0.0
    return float(np.max(x))          # np.max propagates NaN


def _allclose(a, b, atol, rtol):
    excess = _max_or_nan(np.abs(a - b) - (atol + rtol * np.abs(b)))
    shown = excess if math.isnan(excess) else max(excess, 0.0)
    return {"max_violation": shown}, excess <= 0.0, None


def _rel_l2(a, b, max):
    dist, ref = float(np.linalg.norm(a - b)), float(np.linalg.norm(b))
    if ref <= _ZERO_NORM:
        return ({"absolute_l2": dist}, dist <= max,
                "the reference is all zero, so this is the absolute L2 distance")
    return {"rel_l2": dist / ref}, dist / ref <= max, None


def _cosine(a, b, min):
    na, nb = float(np.linalg.norm(a)), float(np.linalg.norm(b))
    if na <= _ZERO_NORM and nb <= _ZERO_NORM:
        return {"cosine": 1.0}, 1.0 >= min, "candidate and reference are both all zero"
    if na <= _ZERO_NORM or nb <= _ZERO_NORM:
        return {"cosine": 0.0}, False, "exactly one of candidate and reference is all zero"
    c = float(np.dot(a.ravel(), b.ravel()) / (na * nb))
    return {"cosine": c}, c >= min, None


def _max_abs(a, b, max):
    d = _max_or_nan(np.abs(a - b))
    return {"max_abs": d}, d <= max, None


def _max_rel(a, b, max):
    diff, mag = np.abs(a - b), np.abs(b)
    rel = np.zeros_like(diff)
    nz = mag > 0
    np.divide(diff, mag, out=rel, where=nz)
    # against a zero reference element: no error if the candidate is zero too,
    # otherwise an unbounded one
    rel[~nz & (diff != 0)] = math.inf
    rel[np.isnan(diff)] = math.nan
    r = _max_or_nan(rel)
    return {"max_rel": r}, r <= max, None


def _nan_inf(a, b):
    nans, infs = int(np.isnan(a).sum()), int(np.isinf(a).sum())
    return {"nan": float(nans), "inf": float(infs)}, nans == 0 and infs == 0, None


_INT_VIEW = {torch.bfloat16: torch.int16, torch.float16: torch.int16,
             torch.float32: torch.int32, torch.float64: torch.int64}


def order_keys(t: torch.Tensor) -> np.ndarray:
    """Integers that sort as the floats of *t* do, one apart for adjacent
    representable values (+0 and -0 share a key): from the unsigned bit pattern
    u, u itself for a clear sign bit and 2^(w-1) - u otherwise."""
    view = _INT_VIEW.get(t.dtype)
    if view is None:
        raise ValueError(f"check: ulp counts representable values of a float output; this one "
                         f"holds {t.dtype}")
    width = 8 * t.element_size()
    u = t.detach().cpu().contiguous().view(view).numpy().astype(np.int64)
    if width < 64:
        u &= (1 << width) - 1                       # the unsigned pattern
        top = 1 << (width - 1)
        return np.where(u < top, u, top - u)
    # 64-bit: the signed view already orders the positive half; mirror the rest
    return np.where(u >= 0, u, np.int64(-(2 ** 63)) - u)


@dataclass(frozen=True)
class _Fn:
    name: str
    bounds: tuple[str, ...]
    two_sided: bool          # needs a reference
    integers: bool           # may judge an integer / bool output
    about: str
    run: Callable


_FUNCTIONS = {f.name: f for f in (
    _Fn("allclose", ("atol", "rtol"), True, False,
        "every element within atol + rtol |reference|: finds the single outlier",
        _allclose),
    _Fn("rel_l2", ("max",), True, False, "L2 distance over the reference's L2 norm", _rel_l2),
    _Fn("cosine", ("min",), True, False,
        "cosine of the angle between the two: a drift of direction, such as a bias",
        _cosine),
    _Fn("equal", (), True, True,
        "identical values (floats: identical bit patterns); for ids, picks and indices",
        None),
    _Fn("ulp", ("max",), True, False,
        "the most representable values between an element and its reference, at the "
        "output's own dtype", None),
    _Fn("max_abs", ("max",), True, False, "the largest elementwise difference", _max_abs),
    _Fn("max_rel", ("max",), True, False,
        "the largest |difference| / |reference| (0 where both are 0, inf where only the "
        "reference is)", _max_rel),
    _Fn("nan_inf", (), False, False, "no NaN and no infinity; needs no reference", _nan_inf),
)}
PREDICATES = _FUNCTIONS
BOUNDS = sorted({b for f in _FUNCTIONS.values() for b in f.bounds})


def _as_f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().to("cpu", torch.float64).numpy()


@dataclass(frozen=True)
class Outcome:
    """What one requirement measured on one output."""

    fn: str
    bounds: Mapping[str, float]
    values: Mapping[str, float]
    passed: bool
    note: str | None = None


@dataclass(frozen=True)
class Requirement:
    """A comparison function with every one of its bounds."""

    fn: str
    bound_values: tuple[tuple[str, float], ...] = ()

    def __post_init__(self):
        spec = _FUNCTIONS.get(self.fn)
        if spec is None:
            raise ValueError(f"check: {self.fn!r} is not a comparison function "
                             f"(there are {sorted(_FUNCTIONS)})")
        given = dict(self.bound_values)
        if set(given) != set(spec.bounds):
            raise ValueError(f"check: {self.fn} is bounded by exactly {list(spec.bounds)}; "
                             f"got {sorted(given)}")

    @property
    def spec(self) -> _Fn:
        return _FUNCTIONS[self.fn]

    @property
    def bounds(self) -> dict[str, float]:
        return dict(self.bound_values)

    def measure(self, candidate: torch.Tensor, reference: torch.Tensor | None = None) -> Outcome:
        spec = self.spec
        if spec.two_sided and reference is None:
            raise ValueError(f"check: {self.fn} compares against a reference, and none was given")
        if self.fn == "equal":
            values, ok, note = _equal(candidate, reference)
        elif self.fn == "ulp":
            gap = np.abs(order_keys(candidate) - order_keys(reference))
            d = int(gap.max()) if gap.size else 0
            values, ok, note = {"max_ulp": float(d)}, d <= self.bounds["max"], None
        else:
            a = _as_f64(candidate)
            b = None if reference is None else _as_f64(reference)
            values, ok, note = spec.run(a, b, **self.bounds)
        return Outcome(self.fn, self.bounds, values, bool(ok), note)


def _equal(candidate, reference):
    a, b = candidate.detach().cpu(), reference.detach().cpu()
    if a.dtype.is_floating_point:
        view = _INT_VIEW.get(a.dtype)
        if view is not None:
            a, b = a.contiguous().view(view), b.contiguous().view(view)
    bad = int((a != b).sum().item())
    return {"mismatched": float(bad), "elements": float(a.numel())}, bad == 0, None


# the requirements under the reference's names
def AllClose(atol: float, rtol: float) -> Requirement:
    return Requirement("allclose", (("atol", float(atol)), ("rtol", float(rtol))))


def RelL2(max: float) -> Requirement:
    return Requirement("rel_l2", (("max", float(max)),))


def Cosine(min: float) -> Requirement:
    return Requirement("cosine", (("min", float(min)),))


def Equal() -> Requirement:
    return Requirement("equal")


def Ulp(max: float) -> Requirement:
    return Requirement("ulp", (("max", float(max)),))


def MaxAbs(max: float) -> Requirement:
    return Requirement("max_abs", (("max", float(max)),))


def MaxRel(max: float) -> Requirement:
    return Requirement("max_rel", (("max", float(max)),))


def NanInf() -> Requirement:
    return Requirement("nan_inf")


# ---------------------------------------------------------------------------
# outputs and reports
# ---------------------------------------------------------------------------
def leaves(x, root: str = "output") -> list[tuple[str, torch.Tensor]]:
    """The tensors of a tensor or nested tuple, depth first, with their paths."""
    out, stack = [], [(root, x)]
    while stack:
        path, item = stack.pop()
        if isinstance(item, torch.Tensor):
            out.append((path, item))
        elif isinstance(item, tuple):
            stack.extend((f"{path}[{i}]", sub) for i, sub in reversed(list(enumerate(item))))
        else:
            raise TypeError(f"check: {path} is a {type(item).__name__}; an output is a tensor "
                            "or a tuple of tensors")
    return out


@dataclass(frozen=True)
class Verdict:
    """One output: its description and every requirement's outcome."""

    path: str
    shape: tuple[int, ...]
    dtype: str
    ref_norm: float | None
    outcomes: tuple[Outcome, ...]

    @property
    def passed(self) -> bool:
        return all(o.passed for o in self.outcomes)


@dataclass(frozen=True)
class Report:
    verdicts: tuple[Verdict, ...] = field(default_factory=tuple)

    @property
    def passed(self) -> bool:
        return all(v.passed for v in self.verdicts)

    @property
    def outputs(self) -> tuple[Verdict, ...]:
        return self.verdicts

    def text(self) -> str:
        rows = []
        for v in self.verdicts:
            ref = "" if v.ref_norm is None else f", reference norm {v.ref_norm:.6g}"
            rows.append(f"{v.path}: {v.dtype} {list(v.shape)}{ref} -- "
                        f"{'PASS' if v.passed else 'FAIL'}")
            for o in v.outcomes:
                got = "  ".join(f"{k} = {val:.6g}" for k, val in o.values.items())
                lim = ", ".join(f"{k} {val:g}" for k, val in o.bounds.items())
                rows.append(f"    {o.fn:<9} {got}" + (f"   [{lim}]" if lim else "")
                            + ("   ok" if o.passed else "   FAILED")
                            + (f"   ({o.note})" if o.note else ""))
        return "\n".join(rows)

    def as_json(self) -> dict:
        return {"passed": self.passed, "outputs": [
            {"path": v.path, "shape": list(v.shape), "dtype": v.dtype,
             **({} if v.ref_norm is None else {"ref_norm": v.ref_norm}), "passed": v.passed,
             "fns": [{"fn": o.fn, **o.bounds, **o.values, "passed": o.passed,
                      **({} if o.note is None else {"note": o.note})} for o in v.outcomes]}
            for v in self.verdicts]}


def _refuse_uncovered(paths: Sequence[str], expect: Mapping[str, Sequence[Requirement]],
                      one_sided: bool) -> None:
    stray = [p for p in expect if p not in paths]
    if stray:
        raise ValueError(f"check: the requirements name {sorted(stray)}, which this run did not "
                         f"produce (it produced {list(paths)})")
    for p in paths:
        reqs = list(expect.get(p) or ())
        if not reqs:
            raise ValueError(f"check: nothing is required of {p}; there is no default bound -- "
                             "name at least one comparison for every output (a single f32 -> "
                             "bf16 rounding already moves rel_l2 by about 1.7e-3)")
        if one_sided:
            needing = sorted({r.fn for r in reqs if r.spec.two_sided})
            if needing:
                alone = sorted(n for n, f in _FUNCTIONS.items() if not f.two_sided)
                raise ValueError(f"check: {p} asks for {needing}, which need a reference, and "
                                 f"there is none; alone, only {alone} can be measured")


def _refuse_inapplicable(path: str, t: torch.Tensor, reqs: Sequence[Requirement]) -> None:
    if t.dtype.is_floating_point:
        return
    wrong = [r.fn for r in reqs if not r.spec.integers]
    if wrong:
        raise ValueError(f"check: {path} holds {t.dtype} values; {wrong} would treat a wrong id "
                         "as a small numerical error.  Judge integer and bool outputs with "
                         "equal")


def compare(produced, expected, *, expect: Mapping[str, Sequence[Requirement]]) -> Report:
    """Measure outputs already produced against *expected* (None: no reference)."""
    got = leaves(produced)
    if not got:
        raise ValueError("check: the output holds no tensor to measure")
    paths = [p for p, _ in got]
    _refuse_uncovered(paths, expect, expected is None)
    refs: dict[str, torch.Tensor] = {}
    if expected is not None:
        want = leaves(expected)
        if [p for p, _ in want] != paths:
            raise ValueError(f"check: the candidate's outputs {paths} and the reference's "
                             f"{[p for p, _ in want]} do not line up")
        for (p, a), (_, b) in zip(got, want):
            if a.shape != b.shape or a.dtype != b.dtype:
                raise ValueError(f"check: {p} differs in form: the candidate's is "
                                 f"{a.dtype} {tuple(a.shape)}, the reference's "
                                 f"{b.dtype} {tuple(b.shape)}")
            refs[p] = b
    verdicts = []
    for p, a in got:
        reqs = tuple(expect[p])
        _refuse_inapplicable(p, a, reqs)
        b = refs.get(p)
        verdicts.append(Verdict(p, tuple(a.shape), str(a.dtype).replace("torch.", ""),
                                None if b is None else float(np.linalg.norm(_as_f64(b))),
                                tuple(r.measure(a, b) for r in reqs)))
    return Report(tuple(verdicts))


def check(candidate: Callable, reference: Callable | None, inputs: tuple, *,
          expect: Mapping[str, Sequence[Requirement]]) -> Report:
    """Call *candidate* and, if given, *reference* on the same *inputs*, and
    measure each output of the candidate against its requirements in *expect*."""
    produced = candidate(*inputs)
    # refuse a bad requirement set before spending a reference run on it
    _refuse_uncovered([p for p, _ in leaves(produced)], expect, reference is None)
    return compare(produced, None if reference is None else reference(*inputs), expect=expect)


# ---------------------------------------------------------------------------
# the ordered --out / --fn / --<bound> sequence
# ---------------------------------------------------------------------------
class _Reader:
    """Reads ``(flag, value)`` pairs in the order the command line gave them."""

    def __init__(self):
        self.by_output: dict[str, list[tuple[str, dict[str, float]]]] = {}
        self.output: str | None = None
        self.fn: tuple[str, dict[str, float]] | None = None

    def take(self, flag: str, value) -> None:
        if flag == "out":
            if value in self.by_output:
                raise ValueError(f"--out {value} appears more than once: give all of its "
                                 "comparisons after one --out")
            self.output, self.fn = value, None
            self.by_output[value] = []
        elif flag == "fn":
            if self.output is None:
                raise ValueError(f"--fn {value} has no output before it: write --out OUTPUT "
                                 "first")
            self.fn = (value, {})
            self.by_output[self.output].append(self.fn)
        else:
            if self.fn is None:
                raise ValueError(f"--{flag} has no --fn before it to bound")
            name, given = self.fn
            allowed = _FUNCTIONS[name].bounds
            if flag not in allowed:
                raise ValueError(f"--{flag} does not bound --fn {name} (its bounds: "
                                 f"{', '.join('--' + b for b in allowed) or 'none'})")
            if flag in given:
                raise ValueError(f"--{flag} is given twice for the same --fn {name}")
            given[flag] = float(value)

    def requirements(self) -> dict[str, tuple[Requirement, ...]]:
        out = {}
        for path, fns in self.by_output.items():
            if not fns:
                raise ValueError(f"--out {path} names no --fn: every output needs a "
                                 "comparison, and there is no default")
            reqs = []
            for name, given in fns:
                lacking = [f"--{b}" for b in _FUNCTIONS[name].bounds if b not in given]
                if lacking:
                    raise ValueError(f"--fn {name} is missing {', '.join(lacking)}: its bounds "
                                     "have no default")
                reqs.append(Requirement(name, tuple((b, given[b])
                                                    for b in _FUNCTIONS[name].bounds)))
            out[path] = tuple(reqs)
        return out


def expectations(stated: Sequence[tuple[str, object]] | None) -> dict[str, tuple[Requirement, ...]]:
    """Requirements per output from the command line's ordered flags."""
    if not stated:
        raise ValueError("no comparison stated: name each output with --out and give it at "
                         "least one --fn (the functions are listed under --help)")
    reader = _Reader()
    for flag, value in stated:
        reader.take(flag, value)
    return reader.requirements()


def guidance() -> str:
    lines = ["comparison functions (every output needs at least one; bounds have no default):"]
    for name in sorted(_FUNCTIONS):
        f = _FUNCTIONS[name]
        flags = " ".join(f"--{b} X" for b in f.bounds) or "(no bound)"
        lines.append(f"  --fn {name}  {flags}\n      {f.about}")
    lines.append("a bf16 output is rounded at most 2^-9 (1.95e-3) of its value each time an "
                 "f32 value lands in bf16; for a chain of n such landings take rtol near "
                 "2^-9 * sqrt(n), and atol for the elements near zero.")
    return "\n".join(lines)


# ---------------------------------------------------------------------------
# files and twins
# ---------------------------------------------------------------------------
def load_tensors(path: str) -> list[torch.Tensor]:
    """The tensors a file holds: ``.npy`` (one tensor), ``.safetensors`` (every
    tensor, by key), ``.pt`` (a tensor or a sequence; weights-only load).  bf16
    has no numpy dtype: store it in ``.safetensors`` or ``.pt``."""
    p = Path(path)
    kind = p.suffix
    if kind == ".npy":
        return [torch.from_numpy(np.load(p, allow_pickle=False))]
    if kind == ".safetensors":
        from safetensors.torch import load_file

        d = load_file(str(p))
        return [d[k] for k in sorted(d)]
    if kind == ".pt":
        obj = torch.load(p, map_location="cpu", weights_only=True)
        return [obj] if isinstance(obj, torch.Tensor) else list(obj)
    raise ValueError(f"{path}: expected a .npy, .safetensors or .pt file")


def _bundle(ts: list[torch.Tensor]):
    return ts[0] if len(ts) == 1 else tuple(ts)


def _bind(fn, weights: Mapping[str, torch.Tensor], prefix: str,
          inputs: list[torch.Tensor], device: str, source: str) -> list:
    """The arguments of *fn*: a parameter named like a weight under *prefix*
    gets that weight, every other one the next input file's tensor."""
    args, pending = [], list(inputs)
    for name in inspect.signature(fn).parameters:
        key = prefix + name
        if key in weights:
            args.append(weights[key].to(device).contiguous())
        elif pending:
            args.append(pending.pop(0).to(device))
        else:
            raise ValueError(f"{source}: parameter {name!r} is no weight and there is no "
                             "--input left for it")
    if pending:
        raise ValueError(f"{source}: {len(pending)} --input tensor(s) left over after every "
                         "activation parameter was filled")
    return args


def _layer_index(part: str, n_layers: int, source: str) -> int:
    if not (part.startswith("layer") and part[5:].isdigit()):
        raise ValueError(f"{source}: {part!r} should be layer<i>")
    i = int(part[5:])
    if i >= n_layers:
        raise ValueError(f"{source}: the checkpoint has {n_layers} layers, no layer {i}")
    return i


def _qwen3_target(selector: str, ckpt: str, source: str):
    from .checkpoint import load_qwen3
    from .qwen3.twin import RootTwin

    cfg, weights = load_qwen3(ckpt)
    root = RootTwin(cfg)
    parts = selector.split(".")
    if len(parts) == 1:
        if parts[0] not in ("embed", "final_rms_norm", "lm_head"):
            raise ValueError(f"{source}: the Qwen3 root functions are embed, final_rms_norm and "
                             "lm_head")
        return getattr(root, parts[0]), weights, ""
    if len(parts) == 2:
        i = _layer_index(parts[0], cfg.num_hidden_layers, source)
        if parts[1] not in ("input_rms_norm", "self_attention", "mlp", "decoder_layer"):
            raise ValueError(f"{source}: a Qwen3 layer's functions are input_rms_norm, "
                             "self_attention, mlp and decoder_layer")
        # the layer twin is one object; its weights are bound per call by name
        return getattr(root.layer, parts[1]), weights, f"layer{i}."
    raise ValueError(f"{source}: write qwen3:<fn> or qwen3:layer<i>.<fn>")


def _hybrid_target(model: str, selector: str, ckpt: str, source: str):
    from .hybrid import twin as T

    if model == "qwen3_5":
        from .checkpoint import load_qwen3_5

        cfg, w = load_qwen3_5(ckpt)
        weights = T.qwen35_canonical(cfg, w)
        dec = T.Qwen3_5Decoder(cfg).load(weights)
    else:
        from .checkpoint import load_granite

        cfg, w = load_granite(ckpt)
        weights = T.granite_canonical(cfg, w)
        dec = T.Granite4_0_H_Small(cfg).load(weights)
    parts = selector.split(".")
    if len(parts) == 1:
        fn = getattr(dec, parts[0], None) if parts[0] in ("embed", "final_rms_norm",
                                                          "lm_head") else None
        if fn is None:
            raise ValueError(f"{source}: the root functions are embed, final_rms_norm and "
                             "lm_head")
        return fn, weights, ""
    i = _layer_index(parts[0], len(dec.layers), source)
    layer = dec.layers[i]
    if len(parts) == 2 and parts[1] == "residual_add":
        return layer.residual_add, weights, f"layer{i}."
    if len(parts) == 3 and parts[1] in ("mixer", "moe"):
        owner, prefix = getattr(layer, parts[1]), f"layer{i}.{parts[1]}."
        if parts[1] == "moe" and parts[2] == "routing":
            owner, prefix = owner.router, prefix + "router."
        fn = getattr(owner, parts[2], None)
        if parts[2].startswith("_") or not callable(fn) or parts[2] in ("forward", "load"):
            raise ValueError(f"{source}: layer {i}'s {parts[1]} ({type(owner).__name__}) has no "
                             f"authored function {parts[2]!r}")
        return fn, weights, prefix
    raise ValueError(f"{source}: write {model}:<fn>, {model}:layer<i>.residual_add or "
                     f"{model}:layer<i>.mixer.<fn> / .moe.<fn>")


def run_twin(source: str, ckpt: str | None, inputs: list[torch.Tensor], device: str):
    """Run one function of a runtime twin (the HIP path) with weights bound
    by canonical name from the checkpoint at *ckpt* and the activations from
    *inputs*, in the function's parameter order."""
    model, sep, selector = source.partition(":")
    if not sep or model not in ("qwen3", "qwen3_5", "granite") or not selector:
        raise ValueError(f"{source}: the source is qwen3:<selector>, qwen3_5:<selector> or "
                         "granite:<selector>")
    if ckpt is None:
        raise ValueError(f"{source}: the twin's weights come from a checkpoint: give --ckpt DIR")
    if model == "qwen3":
        fn, weights, prefix = _qwen3_target(selector, ckpt, source)
    else:
        fn, weights, prefix = _hybrid_target(model, selector, ckpt, source)
    with torch.no_grad():
        return fn(*_bind(fn, weights, prefix, inputs, device, source))


class _InOrder(argparse.Action):
    """Keep --out / --fn / --<bound> as one sequence in the order written."""

    def __call__(self, parser, namespace, values, option_string=None):
        seq = list(getattr(namespace, "stated", None) or [])
        seq.append((self.dest, values))
        namespace.stated = seq


def main(argv: Sequence[str] | None = None) -> int:
    ap = argparse.ArgumentParser(prog="python -m tilefoundry_amd.check",
                                 description=__doc__, epilog=guidance(),
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("source", nargs="?",
                    help="qwen3:<selector>, qwen3_5:<selector> or granite:<selector> -- a twin "
                         "function to run; leave it out to judge --candidate files")
    ap.add_argument("--input", action="append", default=[], metavar="PATH",
                    help="an activation file, one per activation parameter, in order")
    ap.add_argument("--candidate", action="append", default=[], metavar="PATH",
                    help="an output file to judge instead of running a source")
    ap.add_argument("--ckpt", metavar="DIR", help="the checkpoint the twin's weights come from")
    ap.add_argument("--expected", action="append", default=[], metavar="PATH",
                    help="the reference's output file(s)")
    ap.add_argument("--device", default="cuda:0")
    ap.add_argument("--out", action=_InOrder, metavar="OUTPUT",
                    help="the output the --fn flags after it judge: output, output[0], ...")
    ap.add_argument("--fn", action=_InOrder, choices=sorted(_FUNCTIONS))
    for b in BOUNDS:
        ap.add_argument(f"--{b}", action=_InOrder, type=float, help=argparse.SUPPRESS)
    ap.add_argument("--json", action="store_true", help="print the report as JSON")
    args = ap.parse_args(argv)
    try:
        expect = expectations(getattr(args, "stated", None))
        if bool(args.source) == bool(args.candidate):
            raise ValueError("give either a source to run or --candidate files (exactly one)")
        if args.source:
            produced = run_twin(args.source, args.ckpt,
                                [t for f in args.input for t in load_tensors(f)], args.device)
        else:
            produced = _bundle([t for f in args.candidate for t in load_tensors(f)])
        expected = (_bundle([t for f in args.expected for t in load_tensors(f)])
                    if args.expected else None)
        report = compare(produced, expected, expect=expect)
    except (ValueError, TypeError) as e:
        print(f"check: {e}" if not str(e).startswith("check:") else str(e), file=sys.stderr)
        return 2
    print(json.dumps(report.as_json(), indent=1) if args.json else report.text())
    return 0 if report.passed else 1


if __name__ == "__main__":
    raise SystemExit(main())
