"""The library the reference links (lib/libe2mi_backend.so: the engine's objects, only e2mi_* names
exported) run through its own C entry points, as the reference-side adapter calls them: an engine
made by e2mi_create_e8cq from an E8CQ cache (the file E2_Q8_WRITE makes, e2.c:276-292) gives the
embeddings of the engine built in memory from the same model, bit for bit, at both geometries."""
import ctypes as C
import os

import numpy as np
import pytest

from model_util import random_batch, reference_small_config, small_config

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def backend(gpu):
    import e2mi
    lib = C.CDLL(os.path.join(os.path.dirname(e2mi.LIB_PATH), "libe2mi_backend.so"))
    lib.e2mi_create_e8cq.restype = C.c_void_p
    lib.e2mi_create_e8cq.argtypes = [C.c_char_p, C.c_int, C.c_int, C.c_int, C.c_int]
    lib.e2mi_last_error.restype = C.c_char_p
    lib.e2mi_text_embed_batch.restype = C.c_int
    lib.e2mi_text_embed_batch.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int,
                                          C.c_void_p]
    lib.e2mi_destroy.restype = None
    lib.e2mi_destroy.argtypes = [C.c_void_p]
    return lib


def _embed(lib, h, ids, valid, dim):
    out = np.empty((ids.shape[0], dim), np.float32)
    rc = lib.e2mi_text_embed_batch(h, ids.ctypes.data, valid.ctypes.data, ids.shape[0], ids.shape[1],
                                   out.ctypes.data)
    assert rc == 0, lib.e2mi_last_error().decode()
    return out


@pytest.mark.parametrize("geometry", [0, 1])
def test_backend_e8cq_engine_matches_model_engine(backend, rng, tmp_path, geometry):
    import e2mi
    if geometry == 0:
        cfg, L, S = small_config(e2mi, n_layers=2), 2, 300
    else:
        cfg, L, S = reference_small_config(e2mi, n_layers=6), 6, 700
    m = e2mi.Model.synthetic(cfg, 31 + geometry)
    p = str(tmp_path / "w.e8cq")
    m.save_e8cq(p)
    want_eng = e2mi.Engine(m, max_rows=4096)
    h = backend.e2mi_create_e8cq(p.encode(), geometry, L, 1000, 4096)
    assert h, backend.e2mi_last_error().decode()
    try:
        for B in (3, 1):
            ids, valid = random_batch(rng, B, S, 1000, min_len=40)
            got = _embed(backend, h, ids, valid, want_eng.dim)
            assert np.array_equal(got, want_eng.embed_batch(ids, valid)), (geometry, B)
    finally:
        backend.e2mi_destroy(h)


def test_backend_e8cq_refusals(backend, tmp_path):
    import e2mi
    m = e2mi.Model.synthetic(small_config(e2mi, n_layers=2), 5)
    p = str(tmp_path / "w.e8cq")
    m.save_e8cq(p)
    # the file holds 2 layers and a 1000-token table: other shapes are refused, not read past
    assert not backend.e2mi_create_e8cq(p.encode(), 0, 3, 1000, 0)
    assert backend.e2mi_last_error()
    assert not backend.e2mi_create_e8cq(p.encode(), 0, 2, 999, 0)
    assert not backend.e2mi_create_e8cq(p.encode(), 2, 2, 1000, 0)
    assert b"geometry" in backend.e2mi_last_error()
    assert not backend.e2mi_create_e8cq(str(tmp_path / "missing.e8cq").encode(), 0, 2, 1000, 0)
