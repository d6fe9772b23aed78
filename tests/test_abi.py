"""The C ABI: the built library exports every entry include/tf_decode.h declares,
the ctypes binding covers them, and the ctypes structs have the C layout.
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


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(tfd_\w+)\s*\(", text, re.M)))


def test_header_declares_entries():
    names = declared_functions()
    assert "tfd_gemv_bf16" in names and "tfd_decode_persistent" in names
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)


def test_header_constants_match_binding():
    """Every plain #define of the header has the value the binding uses."""
    defines = dict(re.findall(r"^#define TFD_(\w+) (\d+)", HEADER.read_text(), re.M))
    names = {"ABI_VERSION", "PRO_PLAIN", "PRO_NORM", "EPI_STORE", "EPI_RESID", "EPI_SWIGLU",
             "EPI_LOGITS", "ERR_TOKEN_RANGE", "ERR_POS_RANGE", "ERR_PAGE_RANGE",
             "ERR_STEP_RANGE", "ERR_SYNC", "PAGE_SIZE", "ATTN_SPLIT", "SKINNY_COUNTERS"}
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


@pytest.mark.skipif(shutil.which("gcc") is None, reason="no C compiler")
def test_ctypes_structs_match_c_layout(tmp_path):
    fields = [f for f, _ in _lib.TfdDecodeArgs._fields_]
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"',
             'int main(void) {',
             '  printf("TfdLayer %zu\\n", sizeof(TfdLayer));',
             '  printf("TfdDecodeArgs %zu\\n", sizeof(TfdDecodeArgs));']
    for f in fields:
        lines.append(f'  printf("{f} %zu\\n", offsetof(TfdDecodeArgs, {f}));')
    lines.append("  return 0; }")
    src = tmp_path / "probe.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", str(src), "-o", str(exe)], check=True)
    out = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True,
                                                        text=True, check=True).stdout.splitlines())
    assert int(out["TfdLayer"]) == ctypes.sizeof(_lib.TfdLayer)
    assert int(out["TfdDecodeArgs"]) == ctypes.sizeof(_lib.TfdDecodeArgs)
    for f in fields:
        assert int(out[f]) == getattr(_lib.TfdDecodeArgs, f).offset, f
