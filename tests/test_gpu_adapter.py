"""The model-level drop-in for e2_hip_create(e2_model *m) (include/e2hip.h:31-35, hip.c:112-167).

The reference-side adapter e2.c_amd/integration/e2hip_mi.c, compiled against the reference's own
headers by oracle/Makefile into oracle/_ref/libe2hipmi.so, walks the reference's live e2_model and
makes the engine with e2mi_create_tensors. One process holds both sides: the reference's text tower
(oracle/_ref/libreftext.so, its e2_model built by oracle/ref_text.c from an E8CQ cache) and the
engine (e2.c_amd/lib/libe2mi_backend.so, e2mi_* names only).

- The adapter's engine against the reference's own e2_text_embed_batch (text.c:997-1027) on the same
  e2_model: every row at cosine >= 0.9999 after one layer, within 1e-3 (1 - cosine) after two (the
  bars of the reference recipe cross-check, test_oracle_reftext.py), and the head_dim-512 layer 5
  alone (layers 0-4 made identities in the reference's model before the adapter walks it). The
  reference's attention is forced to f32 (E2_ATTN_TEXT=f32, dispatch.c:139-142): the engine's f16
  MFMA attention computes the f32 attention's arithmetic; the reference's own rule would pick its
  int8 attention for long unpadded sequences, a different arithmetic (dispatch.c:47-52). A padded
  batch runs under the reference's unforced rule too (it keeps f32 attention there).
- The adapter's engine against e2mi_create_e8cq on the same cache: bit for bit (the cache's token
  table is rounded to bf16 first, the precision the reference holds it in, e2.c:316-317).
- e2mi_create_tensors over the product model's own buffers against e2mi_create_e8cq: bit for bit.
"""
import ctypes as C
import os

import numpy as np
import pytest

from conftest import ROOT
from model_util import bf16_round, random_batch, reference_small_config

pytestmark = pytest.mark.gpu

ADAPTER_SO = os.path.join(ROOT, "oracle", "_ref", "libe2hipmi.so")
VOCAB = 1000
E2_VOCAB = 262144
BAR_ONE = 1e-4
BAR_TWO = 1e-3


def _bf16_table_cache(src, dst):
    """Copy of E8CQ cache `src` with the f32 token table rounded to bf16 (kept f32)."""
    blob = bytearray(open(src, "rb").read())
    n, io = np.frombuffer(blob, np.uint32, 2, 8)
    for i in range(int(n)):
        e = io + 152 * i
        name = bytes(blob[e:e + 96]).split(b"\0")[0]
        if name == b"language_model.embed_tokens.weight":
            nbytes, off = np.frombuffer(blob, np.uint64, 2, e + 136)
            t = np.frombuffer(blob, np.float32, int(nbytes) // 4, int(off))
            blob[int(off):int(off) + int(nbytes)] = bf16_round(t).tobytes()
            break
    else:
        raise AssertionError("no token table in the cache")
    open(dst, "wb").write(bytes(blob))


@pytest.fixture(scope="module")
def sides(gpu, tmp_path_factory):
    if not os.path.exists(ADAPTER_SO):
        pytest.skip("oracle/_ref/libe2hipmi.so not built (needs the reference tree at build time)")
    import e2mi
    lib = C.CDLL(ADAPTER_SO)
    lib.e2_hip_mi_create.restype = C.c_void_p
    lib.e2_hip_mi_create.argtypes = [C.c_void_p]
    lib.e2_hip_mi_last_error.restype = C.c_char_p
    lib.e2mi_text_embed_batch.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p]
    lib.e2mi_destroy.restype = None
    lib.e2mi_destroy.argtypes = [C.c_void_p]
    lib.e2mi_create_e8cq.restype = C.c_void_p
    lib.e2mi_create_e8cq.argtypes = [C.c_char_p, C.c_int, C.c_int, C.c_int, C.c_int]
    lib.rt_model.restype = C.c_void_p
    lib.rt_attn_text.argtypes = [C.c_int]
    lib.rt_attn_text.restype = None
    m = e2mi.Model.synthetic(reference_small_config(e2mi, n_layers=6, vocab=VOCAB), 4242)
    d = tmp_path_factory.mktemp("adapter")
    raw, path = str(d / "raw.e8cq"), str(d / "bf16.e8cq")
    m.save_e8cq(raw)
    _bf16_table_cache(raw, path)
    return lib, m, raw, path


def _embed(lib, h, ids, valid):
    out = np.empty((ids.shape[0], 768), np.float32)
    rc = lib.e2mi_text_embed_batch(h, ids.ctypes.data, valid.ctypes.data, ids.shape[0], ids.shape[1],
                                   out.ctypes.data)
    assert rc == 0, lib.e2_hip_mi_last_error().decode()
    return out


def _dist(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    c = (a * b).sum(1) / (np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1))
    return float(1 - c.min())


def _batches(rng):
    ids = rng.integers(0, VOCAB, (2, 300)).astype(np.int32)
    full = np.ones((2, 300), np.uint8)
    tail = full.copy()
    tail[1, 230:] = 0
    return [("full300", ids, full), ("tail300", ids, tail),
            ("window700",) + tuple(a[None] for a in (rng.integers(0, VOCAB, 700).astype(np.int32),
                                                     np.ones(700, np.uint8))),
            ("padded64",) + random_batch(rng, 3, 64, VOCAB, min_len=20)]


def _adapter_engine(lib, n_layers, path, identity=(), attn_f32=True):
    from oracle.binding import RefText
    rt = RefText(path, n_layers, VOCAB, nthreads=8)
    for l in identity:
        rt.identity_layer(l)
    lib.rt_attn_text(0 if attn_f32 else -1)
    h = lib.e2_hip_mi_create(lib.rt_model())
    assert h, lib.e2_hip_mi_last_error().decode()
    return rt, h


@pytest.mark.parametrize("n_layers", [1, 2])
def test_adapter_engine_matches_reference_text_tower(sides, rng, n_layers):
    lib, _, _, path = sides
    rt, h = _adapter_engine(lib, n_layers, path)
    try:
        bar = BAR_ONE if n_layers == 1 else BAR_TWO
        for name, ids, valid in _batches(rng):
            want = rt.embed_batch(ids, valid)
            d = _dist(_embed(lib, h, ids, valid), want)
            print(f"layers {n_layers} {name}: 1 - cos {d:.2e}", flush=True)
            assert d < bar, (n_layers, name, d)
    finally:
        lib.e2mi_destroy(h)
        lib.rt_attn_text(-1)
        rt.close()


def test_adapter_engine_full_attention_layer(sides, rng):
    """Layer 5 (head_dim 512, one kv head, RoPE theta 1e6, no window) alone: layers 0-4 are made
    identities in the reference's e2_model, and the adapter uploads that model as it is."""
    lib, _, _, path = sides
    rt, h = _adapter_engine(lib, 6, path, identity=range(5))
    try:
        for name, ids, valid in _batches(rng)[:2]:
            d = _dist(_embed(lib, h, ids, valid), rt.embed_batch(ids, valid))
            print(f"layer 5 {name}: 1 - cos {d:.2e}", flush=True)
            assert d < BAR_ONE, (name, d)
    finally:
        lib.e2mi_destroy(h)
        lib.rt_attn_text(-1)
        rt.close()


def test_adapter_engine_under_the_reference_rule(sides, rng):
    """The reference's unforced attention rule keeps f32 attention for sequences shorter than its int8
    threshold (dispatch.c:47-52, text.c:873-876), so the same bar holds without the override."""
    lib, _, _, path = sides
    rt, h = _adapter_engine(lib, 1, path, attn_f32=False)
    try:
        thr = next(s for s in range(32, 2049) if rt.attn_i8(s))
        ids, valid = random_batch(rng, 4, max(32, thr) - 1, VOCAB, min_len=8)
        d = _dist(_embed(lib, h, ids, valid), rt.embed_batch(ids, valid))
        assert d < BAR_ONE, d
    finally:
        lib.e2mi_destroy(h)
        rt.close()


def test_adapter_engine_equals_cache_engine(sides, rng):
    """Same weights through the two reference-side routes (the live e2_model, the E8CQ cache):
    bit-identical embeddings. The adapter hands over the reference's full 262144-row bf16 table; the
    cache holds VOCAB rows of the same values."""
    lib, _, _, path = sides
    rt, h = _adapter_engine(lib, 6, path)
    hc = lib.e2mi_create_e8cq(path.encode(), 1, 6, VOCAB, 0)
    assert hc, lib.e2_hip_mi_last_error().decode()
    try:
        for name, ids, valid in _batches(rng):
            assert np.array_equal(_embed(lib, h, ids, valid), _embed(lib, hc, ids, valid)), name
    finally:
        lib.e2mi_destroy(h)
        lib.e2mi_destroy(hc)
        lib.rt_attn_text(-1)
        rt.close()


def test_tensor_entry_equals_cache_entry(sides, rng):
    """e2mi_create_tensors over the product model's own buffers (f32 table, borrowed views) against
    e2mi_create_e8cq on that model's cache, and with a bf16 table handed over against the
    bf16-rounded cache: bit for bit."""
    import e2mi
    lib, m, raw, path = sides
    cfg = m.config
    ids, valid = random_batch(rng, 3, 300, VOCAB, min_len=40)
    for cache, table in ((raw, None), (path, "bf16")):
        tb = None
        if table:
            t = bf16_round(m.tensor("language_model.embed_tokens.weight"))
            tb = np.ascontiguousarray((t.view(np.uint32) >> 16).astype(np.uint16))
        eng = e2mi.Engine.from_tensors(e2mi.model_tensors(m, tb), cfg, 1)
        hc = lib.e2mi_create_e8cq(cache.encode(), 1, cfg.n_layers, VOCAB, 0)
        assert hc
        try:
            assert np.array_equal(eng.embed_batch(ids, valid), _embed(lib, hc, ids, valid)), cache
        finally:
            lib.e2mi_destroy(hc)
