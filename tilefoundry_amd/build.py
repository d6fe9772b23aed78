"""Build the gfx950 decode library in-tree: ``python -m tilefoundry_amd.build``.

One ``hipcc`` invocation per shared library, no JIT and no cache outside the
tree, so the built ``.so`` sits next to the sources and travels with the repo.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / "csrc"
INCLUDE = ROOT / "include"
LIB = HERE / "libtfdecode_gfx950.so"
ARCH = "gfx950"

#: Sources linked into the library; every header under csrc/ and include/ is a
#: dependency of all of them.
SOURCES = ["qwen3_decode.hip", "qwen3_xcd.hip", "qwen3_batch.hip", "hybrid.hip",
           "gqa_hybrid.hip", "twin_ops.hip", "hybrid_small.hip", "sample.hip"]

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # Elementwise epilogues mirror separate torch ops: no contraction into FMA.
    # Dot products spell their FMAs out explicitly.
    "-ffp-contract=off",
    # Packed-FP32 instructions stay off for all device code on this pool.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return str(Path(rocm) / "bin" / "hipcc")


def build(verbose: bool = False) -> Path:
    """Compile every source into ``libtfdecode_gfx950.so`` (always recompiles):
    one object per source, compiled side by side (no device code crosses a
    source file, so no relocatable device code is needed), then one link."""
    tmp = LIB.with_suffix(".so.tmp")
    objdir = HERE / "_build"
    objdir.mkdir(exist_ok=True)
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    jobs = []
    for src in SOURCES:
        obj = objdir / (Path(src).stem + ".o")
        cmd = [hipcc(), *compile_flags, "-c", str(CSRC / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        jobs.append((obj, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                                           text=True)))
    objs, errors = [], []
    for obj, proc in jobs:
        _, err = proc.communicate()
        if proc.returncode != 0:
            errors.append(f"{obj.name}: hipcc failed ({proc.returncode}):\n{err[-4000:]}")
        objs.append(str(obj))
    if errors:
        raise RuntimeError("\n".join(errors))
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed ({proc.returncode}):\n{proc.stderr[-4000:]}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
