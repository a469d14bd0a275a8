"""The library's host code under AddressSanitizer and UndefinedBehaviorSanitizer, as the reference's
CI runs its CPU code (.github/workflows/cpu.yml:19-23): tests/sanitize/host_checks.cpp links
model.cpp (the E8CQ reader over corrupted caches, the writer, the caller-held tensor list),
plan.cpp (packed rows and attention work lists into arrays of exactly the documented sizes, over
random masks) and dispatch.cpp, built with g++ for the host only. Any sanitizer report fails."""
import os
import shutil
import subprocess

import pytest

from conftest import ROOT

SRC = [os.path.join(ROOT, "tests", "sanitize", "host_checks.cpp")] + [
    os.path.join(ROOT, "e2.c_amd", "csrc", f) for f in ("model.cpp", "plan.cpp", "dispatch.cpp")]


def test_host_code_under_asan_ubsan(tmp_path):
    if not shutil.which("g++"):
        pytest.skip("no g++ on this host")
    exe = str(tmp_path / "host_checks")
    flags = ["-std=c++20", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
             "-fno-sanitize-recover=undefined", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
             "-I" + os.path.join(ROOT, "include")]
    r = subprocess.run(["g++"] + flags + SRC + ["-o", exe, "-pthread"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    env.pop("LD_PRELOAD", None)
    r = subprocess.run([exe, str(tmp_path)], capture_output=True, text=True, timeout=600, env=env)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-6000:]
    assert "AddressSanitizer" not in out and "runtime error" not in out and "LeakSanitizer" not in out, out[-6000:]
    assert "host checks: ok" in out
