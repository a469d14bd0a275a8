"""Error paths under forced runtime failures (the reference's tests/test_oom.c, which wraps malloc at
link time, CMakeLists.txt:370-374): lib/libe2mi_fault.so is the library's own objects linked with
hipMalloc, hipHostMalloc, hipStreamCreateWithFlags, hipGraphInstantiate and hipGraphLaunch wrapped
(tests/fault/fault_shim.cpp); a countdown makes the n-th call of a kind fail on the host, before the
runtime does anything, so no kernel is affected.

- every device or pinned allocation that engine creation makes, failed in turn: creation returns
  NULL with a message and gives back every byte it had taken;
- a stream that cannot be created: creation fails;
- a graph that cannot be instantiated or launched: the call fails with a message, and the next call
  on the same engine gives the embeddings an unfaulted engine gives."""
import ctypes as C
import os

import numpy as np
import pytest

from model_util import random_batch

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FAULT_SO = os.path.join(ROOT, "e2.c_amd", "lib", "libe2mi_fault.so")
F_ALLOC, F_STREAM, F_INSTANTIATE, F_LAUNCH = 0, 1, 2, 3


@pytest.fixture(scope="module")
def flib(gpu):
    import e2mi
    assert os.path.exists(FAULT_SO), "lib/libe2mi_fault.so is built with the library (make -C e2.c_amd)"
    L = C.CDLL(FAULT_SO)
    P, I = C.c_void_p, C.c_int
    L.e2_config_baseline.argtypes = [C.POINTER(e2mi.E2Config)]
    L.e2_model_synthetic.restype = P
    L.e2_model_synthetic.argtypes = [C.POINTER(e2mi.E2Config), C.c_uint64]
    L.e2_free.argtypes = [P]
    L.e2mi_create_rows.restype = P
    L.e2mi_create_rows.argtypes = [P, I]
    L.e2mi_destroy.argtypes = [P]
    L.e2mi_text_embed_batch.argtypes = [P, P, P, I, I, P]
    L.e2mi_last_error.restype = C.c_char_p
    L.e2mi_fault_arm.argtypes = [I, I]
    L.e2mi_fault_calls.restype = C.c_long
    L.e2mi_fault_calls.argtypes = [I]
    cfg = e2mi.E2Config()
    L.e2_config_baseline(C.byref(cfg))
    cfg.n_layers, cfg.vocab, cfg.max_seq = 1, 1000, 512
    m = L.e2_model_synthetic(C.byref(cfg), 77)
    assert m
    # the unfaulted library on the same synthetic model: the embeddings to come back to
    want_model = e2mi.Model.synthetic(e2mi.baseline_config(n_layers=1, vocab=1000, max_seq=512), 77)
    yield L, m, e2mi.Engine(want_model, max_rows=1024)
    L.e2_free(m)


def _embed(L, g, ids, valid):
    out = np.full((ids.shape[0], 768), 7.0, np.float32)
    rc = L.e2mi_text_embed_batch(g, ids.ctypes.data, valid.ctypes.data, ids.shape[0], ids.shape[1],
                                 out.ctypes.data)
    return rc, out


def test_every_creation_allocation_can_fail(flib):
    import torch
    L, m, _ = flib
    L.e2mi_fault_arm(F_ALLOC, -1)
    g = L.e2mi_create_rows(m, 1024)
    assert g
    L.e2mi_destroy(g)
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    c0 = L.e2mi_fault_calls(F_ALLOC)
    g = L.e2mi_create_rows(m, 1024)
    n = L.e2mi_fault_calls(F_ALLOC) - c0
    assert g and n > 20, n
    L.e2mi_destroy(g)
    for k in range(n):
        L.e2mi_fault_arm(F_ALLOC, k)
        g = L.e2mi_create_rows(m, 1024)
        L.e2mi_fault_arm(F_ALLOC, -1)
        assert not g, f"creation survived the failure of allocation {k}"
        msg = L.e2mi_last_error().decode()
        assert msg and ("alloc" in msg.lower() or "memory" in msg.lower() or "malloc" in msg.lower()), (k, msg)
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    assert abs(free1 - free0) < (32 << 20), f"{(free0 - free1) >> 20} MiB not given back"


def test_stream_creation_failure(flib):
    L, m, _ = flib
    L.e2mi_fault_arm(F_STREAM, 0)
    g = L.e2mi_create_rows(m, 1024)
    L.e2mi_fault_arm(F_STREAM, -1)
    assert not g and L.e2mi_last_error().decode()


@pytest.mark.parametrize("kind,text", [(F_INSTANTIATE, "instantiate"), (F_LAUNCH, "launch")])
def test_graph_failure_then_recovery(flib, rng, kind, text):
    L, m, want_eng = flib
    ids, valid = random_batch(rng, 3, 96, 1000, min_len=20)
    want = want_eng.embed_batch(ids, valid)
    g = L.e2mi_create_rows(m, 1024)
    assert g
    try:
        if kind == F_LAUNCH:  # a recorded graph first: the first call of a shape records it
            rc, out = _embed(L, g, ids, valid)
            assert rc == 0 and np.array_equal(out, want)
        L.e2mi_fault_arm(kind, 0)
        rc, out = _embed(L, g, ids, valid)
        L.e2mi_fault_arm(kind, -1)
        assert rc == -1 and text in L.e2mi_last_error().decode(), L.e2mi_last_error()
        for _ in range(2):
            rc, out = _embed(L, g, ids, valid)
            assert rc == 0 and np.array_equal(out, want)
    finally:
        L.e2mi_destroy(g)
