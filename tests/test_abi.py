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
    # the attention's softmax needs a positive, finite logit scale
    for bad in (0.0, -0.5, float("inf"), float("nan")):
        assert lib.e2mi_attention(None, None, None, None, None, 1, 128, 3, 1, 256, bad, None, None, None) == -1
        assert "scale" in e2mi.last_error()
        assert lib.e2mi_attention_packed_window(None, None, None, None, 8, None, None, None, 1, 8, 3, 1, 256,
                                                bad, 0, None, None, None, None, 0) == -1
        assert "scale" in e2mi.last_error()


def _exports(path):
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", path], check=True, capture_output=True,
                         text=True).stdout
    return {f[2] for f in (l.split() for l in out.splitlines()) if len(f) == 3 and f[1] in "TWDBR"}


def test_backend_library_exports_only_engine_names():
    """lib/libe2mi_backend.so is what links into the reference: every e2mi_* entry point and no
    e2_* name, which the reference's own library defines (e2_free, e2_last_error, e2_text_embed*,
    the dispatch functions)."""
    import e2mi
    path = os.path.join(os.path.dirname(e2mi.LIB_PATH), "libe2mi_backend.so")
    names = _exports(path)
    want = {n for n in declared_symbols() if n.startswith("e2mi_")}
    assert want - names == set(), sorted(want - names)
    stray = sorted(n for n in names if not n.startswith("e2mi_"))
    assert not stray, f"backend library exports non-engine names: {stray}"
    # the full library does export the model API a caller of include/e2.h uses
    assert {"e2_free", "e2_last_error", "e2_text_embed_batch"} <= _exports(e2mi.LIB_PATH)


def test_integration_adapter_compiles_and_links(tmp_path):
    """The reference-side adapter shown in the integration guide builds against include/e2mi.h
    alone and resolves every symbol from lib/libe2mi_backend.so."""
    import subprocess
    import e2mi
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    sec = text[text.index("## 1."):text.index("## 2.")]
    code = re.search(r"```c\n(.*?)```", sec, flags=re.S).group(1)
    assert '#include "e2mi.h"' in code and '"e2.h"' not in code
    src = tmp_path / "e2mi_adapter.c"
    src.write_text(code)
    libdir = os.path.dirname(e2mi.LIB_PATH)
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Wextra", "-Werror", "-fPIC", "-shared",
                    "-I" + os.path.join(ROOT, "include"), str(src), "-L" + libdir, "-le2mi_backend",
                    "-Wl,--no-undefined", "-o", str(tmp_path / "adapter.so")], check=True)
