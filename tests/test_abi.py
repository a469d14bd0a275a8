"""The C-ABI library loads and exports every symbol include/*.h declares (no compute, no GPU)."""
import ctypes
import glob
import os
import re

import pytest

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


# the two entries that take this repository's model container: exported by lib/libe2mi.so only
MODEL_ENTRIES = {"e2mi_create", "e2mi_create_rows"}
REF = "/root/reference"


def test_backend_library_exports_only_engine_names():
    """lib/libe2mi_backend.so is what links into the reference: every e2mi_* entry point except the
    two that take this repository's model container, and no e2_* name, which the reference's own
    library defines (e2_free, e2_last_error, e2_text_embed*, the dispatch functions)."""
    import e2mi
    path = os.path.join(os.path.dirname(e2mi.LIB_PATH), "libe2mi_backend.so")
    names = _exports(path)
    want = {n for n in declared_symbols() if n.startswith("e2mi_")} - MODEL_ENTRIES
    assert want - names == set(), sorted(want - names)
    assert not names & MODEL_ENTRIES, sorted(names & MODEL_ENTRIES)
    assert {"e2mi_create_tensors", "e2mi_create_e8cq"} <= names
    stray = sorted(n for n in names if not n.startswith("e2mi_"))
    assert not stray, f"backend library exports non-engine names: {stray}"
    # the full library does export the model API a caller of include/e2.h uses
    assert {"e2_free", "e2_last_error", "e2_text_embed_batch", "e2mi_create"} <= _exports(e2mi.LIB_PATH)


def _gcc(args, tmp_path, src_text=None, name="t.c"):
    import subprocess
    src = tmp_path / name
    if src_text is not None:
        src.write_text(src_text)
    return subprocess.run(["gcc", "-std=gnu11", "-Wall", "-Wextra", "-Werror", "-fPIC", "-c",
                           "-o", str(tmp_path / (name + ".o"))] + args + [str(src)],
                          capture_output=True, text=True)


def _ref_includes():
    if not os.path.isdir(os.path.join(REF, "src")):
        pytest.skip("the reference tree is absent on this host")
    return ["-I" + os.path.join(REF, "src"), "-I" + os.path.join(REF, "include"),
            "-I" + os.path.join(ROOT, "include")]


def test_integration_adapter_compiles_against_the_reference(tmp_path):
    """The reference-side adapter (e2.c_amd/integration/e2hip_mi.c: e2_hip_mi_create(e2_model *m)
    walking the reference's own model) builds against the reference's headers and include/e2mi.h
    with -Wall -Wextra -Werror, and resolves every symbol from lib/libe2mi_backend.so."""
    import subprocess
    import e2mi
    inc = _ref_includes()
    adapter = os.path.join(ROOT, "e2.c_amd", "integration", "e2hip_mi.c")
    r = subprocess.run(["gcc", "-std=gnu11", "-Wall", "-Wextra", "-Werror", "-fPIC", "-shared"] + inc +
                       ["-o", str(tmp_path / "adapter.so"), adapter, "-L" + os.path.dirname(e2mi.LIB_PATH),
                        "-le2mi_backend"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    und = subprocess.run(["nm", "-u", str(tmp_path / "adapter.so")], capture_output=True, text=True).stdout
    assert "e2mi_create_tensors" in und


def test_reference_model_cannot_reach_the_model_entry(tmp_path):
    """A reference e2_model handed to e2mi_create is a compile error: the engine's entry takes this
    repository's e2mi_model, a different struct tag from the reference's e2_model (src/model.h:113)."""
    inc = _ref_includes()
    bad = ('#include "model.h"\n#include "e2mi.h"\n'
           "e2mi_engine *f(e2_model *m) { return e2mi_create(m); }\n")
    r = _gcc(inc, tmp_path, bad, "bad.c")
    assert r.returncode != 0 and "incompatible pointer type" in r.stderr, r.stderr
    good = ('#include "model.h"\n#include "e2mi.h"\n'
            "e2mi_engine *f(const e2mi_tensor *t, int n) { return e2mi_create_tensors(t, n, 1, 0, 0, 0); }\n")
    r = _gcc(inc, tmp_path, good, "good.c")
    assert r.returncode == 0, r.stderr
