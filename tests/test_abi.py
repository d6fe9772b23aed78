"""The C ABI: the built library exports every entry include/*.h declares, the
ctypes binding covers them, and the ctypes structs have the C layout.
No GPU work is done here (only tfd_abi_version is called)."""
import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from tilefoundry_amd import _lib
from tilefoundry_amd.build import LIB

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "tf_decode.h"
HEADERS = sorted((ROOT / "include").glob("*.h"))


def declared_functions() -> list[str]:
    names = set()
    for header in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names |= set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(tfd_\w+)\s*\(", text, re.M))
    return sorted(names)


def test_header_declares_entries():
    names = declared_functions()
    assert "tfd_gemv_bf16" in names and "tfd_decode_persistent" in names
    assert "tfd_gdn_step" in names and "tfd_gemm_skinny_fp8" in names
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)


def test_header_constants_match_binding():
    """Every plain #define of the header has the value the binding uses."""
    defines = {}
    for header in HEADERS:
        defines.update(re.findall(r"^#define TFD_(\w+) (\d+)", header.read_text(), re.M))
    names = {"ABI_VERSION", "PRO_PLAIN", "PRO_NORM", "EPI_STORE", "EPI_RESID", "EPI_SWIGLU",
             "EPI_LOGITS", "ERR_TOKEN_RANGE", "ERR_POS_RANGE", "ERR_PAGE_RANGE",
             "ERR_STEP_RANGE", "ERR_SYNC", "ERR_PLACEMENT", "PAGE_SIZE", "ATTN_SPLIT", "SKINNY_COUNTERS", "EPI_RESID_F32",
             "ROUTE_SOFTMAX_TOPK", "ROUTE_TOPK_SOFTMAX", "POLICY_F32", "POLICY_BF16",
             "MOE_ROUTE_GIVEN", "MOE_ROUTE_SOFTMAX_TOPK", "MOE_ROUTE_TOPK_SOFTMAX",
             "SAMPLE_MAX_K", "SAMPLE_MAX_VOCAB"}
    assert names <= set(defines), names - set(defines)
    for name in names:
        assert getattr(_lib, name) == int(defines[name]), name


@pytest.mark.skipif(not Path(LIB).exists(), reason="library not built")
def test_library_exports_every_declared_entry():
    dll = ctypes.CDLL(str(LIB))
    for name in declared_functions():
        assert hasattr(dll, name), name
    dll.tfd_abi_version.restype = ctypes.c_int
    assert dll.tfd_abi_version() == _lib.ABI_VERSION


STRUCTS = {"TfdDecodeArgs": _lib.TfdDecodeArgs, "TfdLayer": _lib.TfdLayer,
           "TfdMoeArgs": _lib.TfdMoeArgs, "TfdGdnArgs": _lib.TfdGdnArgs,
           "TfdMambaArgs": _lib.TfdMambaArgs, "TfdGqaArgs": _lib.TfdGqaArgs,
           "TfdXcdArgs": _lib.TfdXcdArgs, "TfdConvStepArgs": _lib.TfdConvStepArgs,
           "TfdDeltaStepArgs": _lib.TfdDeltaStepArgs, "TfdPartialRopeArgs": _lib.TfdPartialRopeArgs,
           "TfdSsmStepArgs": _lib.TfdSsmStepArgs, "TfdGatedNormArgs": _lib.TfdGatedNormArgs,
           "TfdRowGemvArgs": _lib.TfdRowGemvArgs, "TfdProj8NormArgs": _lib.TfdProj8NormArgs,
           "TfdSampling": _lib.TfdSampling}


@pytest.mark.skipif(shutil.which("gcc") is None, reason="no C compiler")
def test_ctypes_structs_match_c_layout(tmp_path):
    lines = ['#include <stdio.h>', '#include <stddef.h>',
             *[f'#include "{h}"' for h in HEADERS], 'int main(void) {']
    for name, cls in STRUCTS.items():
        lines.append(f'  printf("{name} %zu\\n", sizeof({name}));')
        for f, _ in cls._fields_:
            lines.append(f'  printf("{name}.{f} %zu\\n", offsetof({name}, {f}));')
    lines.append("  return 0; }")
    src = tmp_path / "probe.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", str(src), "-o", str(exe)], check=True)
    out = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True,
                                                        text=True, check=True).stdout.splitlines())
    for name, cls in STRUCTS.items():
        assert int(out[name]) == ctypes.sizeof(cls), name
        for f, _ in cls._fields_:
            assert int(out[f"{name}.{f}"]) == getattr(cls, f).offset, f"{name}.{f}"
