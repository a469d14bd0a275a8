"""The C-ABI library loads and exports every symbol include/*.h declares (no compute, no GPU)."""
import ctypes
import glob
import os
import re

from conftest import ROOT


def declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        src = re.sub(r"//[^\n]*", "", src)
        src = re.sub(r"typedef[^;]*;", "", src, flags=re.S)
        for m in re.finditer(r"\b(e2\w*)\s*\(", src):
            names.add(m.group(1))
    return names


def test_headers_declare_entry_points():
    names = declared_symbols()
    assert "e2mi_i8_gemm" in names and "e2mi_quantize" in names


def test_library_exports_every_declared_symbol():
    import e2mi
    lib = ctypes.CDLL(e2mi.LIB_PATH)
    missing = [n for n in sorted(declared_symbols()) if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_python_mirror_binds_every_declared_symbol():
    import e2mi
    missing = sorted(declared_symbols() - set(e2mi.SIGNATURES))
    assert not missing, f"declared in include/ but not bound in e2mi.py: {missing}"


def test_errors_are_reported_without_a_gpu():
    import e2mi
    lib = e2mi.load()
    # bad geometry is rejected before any HIP call
    assert lib.e2mi_quantize(None, None, None, None, 4, 100, 100, 128) == -1
    assert "quantize" in e2mi.last_error()
    assert lib.e2mi_interleave_gate_up(None, None, None, None, None, None, 100, 8) == -1
