"""Model container: synthetic weights, tensor views, and the E8CQ packed cache format
(q8cache.c v1) — round trip, cross-read with the reference's own writer/reader (oracle/_ref), and
refusal of corrupted files (test_q8cache.c:113-248 style)."""
import ctypes as C
import os
import struct

import numpy as np
import pytest

from model_util import NORMS, Q8, lname, small_config


@pytest.fixture(scope="module")
def e2mi_mod():
    import e2mi
    e2mi.load()
    return e2mi


@pytest.fixture(scope="module")
def model(e2mi_mod):
    return e2mi_mod.Model.synthetic(small_config(e2mi_mod), 1004)


def test_baseline_config(e2mi_mod):
    c = e2mi_mod.baseline_config()
    assert (c.n_layers, c.hidden, c.ffn, c.n_heads, c.n_kv_heads, c.head_dim, c.vocab) == \
        (24, 768, 1152, 3, 1, 256, 262144)
    assert abs(c.embed_scale - np.sqrt(768)) < 1e-5 and c.attn_scale == 1.0 and c.rms_eps == np.float32(1e-6)


def test_synthetic_is_deterministic_and_in_range(e2mi_mod, model, oracle):
    m2 = e2mi_mod.Model.synthetic(small_config(e2mi_mod), 1004)
    m3 = e2mi_mod.Model.synthetic(small_config(e2mi_mod), 1005)
    wq, sc, bsq, N, K = model.tensor(lname(1, Q8[4]))
    assert (N, K) == (1152, 768)
    assert np.array_equal(wq, m2.tensor(lname(1, Q8[4]))[0])
    assert not np.array_equal(wq, m3.tensor(lname(1, Q8[4]))[0])
    w = oracle.q8w_unpack(wq, N, K)
    assert w.min() >= -127 and w.max() <= 127 and abs(float(w.mean())) < 1
    assert sc.min() >= 0.001 and sc.max() <= 0.02
    # bsq is the per-128-block row sum (int8.c:57-61)
    assert np.array_equal(bsq[:, :N], w.reshape(N, K // 128, 128).sum(-1).T.astype(np.int32))
    g = model.tensor(lname(0, NORMS[0]))
    assert g.shape == (768,) and abs(g.mean() - 1) < 0.02 and 0.03 < g.std() < 0.07
    t = model.tensor("language_model.embed_tokens.weight")
    assert t.shape == (1000, 768) and abs(t.std() - 0.02) < 0.001


def test_e8cq_round_trip(e2mi_mod, model, tmp_path):
    p = str(tmp_path / "m.e8cq")
    model.save_e8cq(p)
    m2 = e2mi_mod.Model.load_e8cq(p, small_config(e2mi_mod))
    for l in range(2):
        for s in Q8:
            a, b = model.tensor(lname(l, s)), m2.tensor(lname(l, s))
            assert all(np.array_equal(x, y) for x, y in zip(a[:3], b[:3]))
        for s in NORMS:
            assert np.array_equal(model.tensor(lname(l, s)), m2.tensor(lname(l, s)))
    assert not [f for f in os.listdir(tmp_path) if ".tmp." in f]   # atomic commit leaves no temp


def _ref_q8c(ref):
    L = ref.lib
    L.q8c_write_open.argtypes = [C.c_char_p]
    L.q8c_put_q8w.argtypes = [C.c_char_p, C.c_void_p]
    L.q8c_defer.argtypes = [C.c_char_p, C.c_int, C.c_int, C.POINTER(C.c_int64), C.c_void_p, C.c_size_t]
    L.q8c_read_open.argtypes = [C.c_char_p]
    L.q8c_get_q8w.argtypes = [C.c_char_p, C.c_void_p]
    L.q8c_error.restype = C.c_char_p
    return L


def test_e8cq_cross_read_with_reference(e2mi_mod, model, ref, tmp_path):
    from oracle.binding import Q8W
    L = _ref_q8c(ref)
    # ours -> the reference's validating reader (q8cache.c:242-385)
    p1 = str(tmp_path / "ours.e8cq")
    model.save_e8cq(p1)
    assert L.q8c_read_open(p1.encode()) == 0, L.q8c_error()
    try:
        for l in range(2):
            for s in Q8:
                q = Q8W()
                assert L.q8c_get_q8w(lname(l, s).encode(), C.byref(q)) == 0
                wq, sc, bsq, N, K = model.tensor(lname(l, s))
                assert (q.N, q.K, q.nblocks, q.Npad) == (N, K, K // 128, (N + 7) & ~7)
                got = np.ctypeslib.as_array(C.cast(q.w, C.POINTER(C.c_int8)), (wq.size,))
                assert np.array_equal(got, wq)
                assert np.array_equal(np.ctypeslib.as_array(C.cast(q.scale, C.POINTER(C.c_float)), (N,)), sc)
    finally:
        L.q8c_read_close()
    # the reference's writer (q8cache.c:61-222) -> our loader
    p2 = str(tmp_path / "ref.e8cq")
    assert L.q8c_write_open(p2.encode()) == 0
    keep = []
    for l in range(2):
        for s in Q8:
            wq, sc, bsq, N, K = model.tensor(lname(l, s))
            keep += [wq, sc, bsq]
            q = Q8W(wq.ctypes.data, bsq.ctypes.data, sc.ctypes.data, N, K, K // 128, (N + 7) & ~7,
                    -1e31, 1e31, 0)
            assert L.q8c_put_q8w(lname(l, s).encode(), C.byref(q)) == 0
        for s in NORMS:
            g = np.ascontiguousarray(model.tensor(lname(l, s)), np.float32)
            keep.append(g)
            dims = (C.c_int64 * 4)(g.size, 0, 0, 0)
            assert L.q8c_defer(lname(l, s).encode(), 2, 1, dims, g.ctypes.data, g.nbytes) == 0
    for name in ("language_model.embed_tokens.weight", "language_model.norm.weight"):
        t = np.ascontiguousarray(model.tensor(name), np.float32)
        keep.append(t)
        dims = (C.c_int64 * 4)(*(list(t.shape) + [0] * (4 - t.ndim)))
        assert L.q8c_defer(name.encode(), 2, t.ndim, dims, t.ctypes.data, t.nbytes) == 0
    assert L.q8c_write_close() == 0
    m2 = e2mi_mod.Model.load_e8cq(p2, small_config(e2mi_mod))
    for l in range(2):
        for s in Q8:
            assert np.array_equal(model.tensor(lname(l, s))[0], m2.tensor(lname(l, s))[0])
        for s in NORMS:
            assert np.array_equal(model.tensor(lname(l, s)), m2.tensor(lname(l, s)))


def _corrupt(src, dst, off, data):
    b = bytearray(open(src, "rb").read())
    b[off:off + len(data)] = data
    open(dst, "wb").write(bytes(b))


def test_e8cq_corruption_refused(e2mi_mod, model, tmp_path):
    p = str(tmp_path / "good.e8cq")
    model.save_e8cq(p)
    raw = open(p, "rb").read()
    magic, ver, n, io = struct.unpack_from("<4I", raw, 0)
    first = io  # first index entry: name[96] kind ndim dims[4] nbytes off
    kind_off, nb_off, off_off = first + 96, first + 136, first + 144
    cases = {
        "magic": (0, b"XXXX"),
        "version": (4, struct.pack("<I", 2)),
        "index misaligned": (12, struct.pack("<I", io + 4)),
        "index past end": (12, struct.pack("<I", len(raw) + 16)),
        "entry count": (8, struct.pack("<I", n + 10 ** 6)),
        "unterminated name": (first, b"A" * 96),
        "empty name": (first, b"\0"),
        "kind": (kind_off, struct.pack("<I", 9)),
        "blob misaligned": (off_off, struct.pack("<Q", struct.unpack_from("<Q", raw, off_off)[0] + 4)),
        "blob outside": (off_off, struct.pack("<Q", io)),
        "size mismatch": (nb_off, struct.pack("<Q", struct.unpack_from("<Q", raw, nb_off)[0] - 16)),
        "truncated": None,
    }
    for name, mod in cases.items():
        bad = str(tmp_path / f"bad_{name.replace(' ', '_')}.e8cq")
        if mod is None:
            open(bad, "wb").write(raw[: len(raw) // 2])
        else:
            _corrupt(p, bad, *mod)
        with pytest.raises(e2mi_mod.E2MIError):
            e2mi_mod.Model.load_e8cq(bad, small_config(e2mi_mod))
    # a cache of another geometry is refused by shape
    with pytest.raises(e2mi_mod.E2MIError, match="missing or mis-shaped"):
        e2mi_mod.Model.load_e8cq(p, small_config(e2mi_mod, n_layers=3))
    with pytest.raises(e2mi_mod.E2MIError, match="mis-shaped"):
        e2mi_mod.Model.load_e8cq(p, small_config(e2mi_mod, vocab=999))


def test_bad_configs_refused(e2mi_mod):
    for over in (dict(head_dim=128), dict(hidden=700), dict(n_heads=3, n_kv_heads=2), dict(max_seq=4096),
                 dict(attn_scale=0.0), dict(attn_scale=-1.0), dict(attn_scale=float("inf")),
                 dict(n_heads=16, n_kv_heads=1)):
        with pytest.raises(e2mi_mod.E2MIError):
            e2mi_mod.Model.synthetic(e2mi_mod.baseline_config(n_layers=1, vocab=10, **over), 1)


def test_reference_config(e2mi_mod):
    """The reference checkpoint's text geometry (e2.c:294-301, model.h:12-16, text.c:467-478)."""
    c = e2mi_mod.reference_config()
    assert (c.n_layers, c.hidden, c.ffn, c.n_heads, c.n_kv_heads, c.head_dim, c.vocab, c.max_seq) == \
        (24, 512, 2048, 4, 2, 256, 262144, 2048)
    assert (c.ple_dim, c.out_dim, c.window, c.full_period, c.full_head_dim, c.full_kv_heads) == \
        (512, 768, 512, 6, 512, 1)
    assert c.rope_theta == 1e4 and c.rope_theta_full == 1e6
    assert c.embed_scale == np.float32(np.sqrt(512)) and c.ple_scale == np.float32(1 / np.sqrt(512))
    # full-attention layers 5, 11, 17, 23 (text.c:267)
    assert [l for l in range(24) if c.layer_geom(l)[0] == 512] == [5, 11, 17, 23]
    b = e2mi_mod.baseline_config()
    assert (b.ple_dim, b.out_dim, b.window, b.full_period) == (0, 0, 0, 0)


def test_reference_geometry_tensors_and_e8cq(e2mi_mod, tmp_path):
    """The reference geometry's extra tensors (names of e2.c:316-381, shapes per layer type), the
    BASELINE tensors unchanged by the extras' seeds, and an E8CQ round trip that checks them."""
    cfg = e2mi_mod.reference_config(n_layers=6, vocab=100)
    m = e2mi_mod.Model.synthetic(cfg, 9)
    shapes = {"language_model.ple.per_layer_model_projection.weight": (6 * 512, 512),
              "language_model.embedding_projection.weight": (768, 512)}
    for name, nk in shapes.items():
        assert m.tensor(name)[3:5] == nk
    assert m.tensor("language_model.ple.per_layer_projection_norm.weight").shape == (512,)
    for l, (qd, kvd) in ((0, (1024, 512)), (5, (2048, 512))):
        assert m.tensor(lname(l, Q8[0]))[3:5] == (qd, 512)
        assert m.tensor(lname(l, Q8[1]))[3:5] == (kvd, 512)
        assert m.tensor(lname(l, Q8[3]))[3:5] == (512, qd)
        assert m.tensor(lname(l, "self_attn.q_norm.weight")).shape == (qd // 4,)
        assert m.tensor(lname(l, "ple_block.per_layer_input_gate.weight"))[3:5] == (512, 512)
        assert m.tensor(lname(l, "ple_block.per_layer_projection.weight"))[3:5] == (512, 512)
        assert m.tensor(lname(l, "layer_scalar")).shape == (1,)
    p = str(tmp_path / "ref.e8cq")
    m.save_e8cq(p)
    m2 = e2mi_mod.Model.load_e8cq(p, cfg)
    for name in list(shapes) + [lname(5, "ple_block.per_layer_projection.weight")]:
        assert all(np.array_equal(x, y) for x, y in zip(m.tensor(name)[:3], m2.tensor(name)[:3]))
    assert np.array_equal(m.tensor(lname(3, "layer_scalar")), m2.tensor(lname(3, "layer_scalar")))
    # a cache without the PLE tensors is refused for this geometry, accepted for the BASELINE one
    b = e2mi_mod.Model.synthetic(e2mi_mod.baseline_config(n_layers=1, vocab=100), 9)
    pb = str(tmp_path / "b.e8cq")
    b.save_e8cq(pb)
    with pytest.raises(e2mi_mod.E2MIError, match="missing or mis-shaped"):
        e2mi_mod.Model.load_e8cq(pb, e2mi_mod.reference_config(n_layers=1, vocab=100, hidden=768, ffn=1152,
                                                                 n_heads=3, n_kv_heads=1, full_period=0))
    # the extras draw from their own streams: the shared tensors match a BASELINE-extras-free model
    plain = e2mi_mod.Model.synthetic(e2mi_mod.reference_config(n_layers=6, vocab=100, ple_dim=0, out_dim=0), 9)
    assert np.array_equal(plain.tensor(lname(2, Q8[4]))[0], m.tensor(lname(2, Q8[4]))[0])


def test_tensor_entry_refusals(e2mi_mod):
    """e2mi_create_tensors checks the caller's tensors before any device work: a missing tensor, a
    mis-shaped or duplicated one, a bad kind, a null pointer or an unknown geometry is refused with a
    message (no GPU needed: nothing reaches the device)."""
    from model_util import reference_small_config
    e2mi = e2mi_mod
    m = e2mi.Model.synthetic(reference_small_config(e2mi, n_layers=1, vocab=64), 3)
    cfg = m.config
    t = e2mi.model_tensors(m)
    lib = e2mi.load()
    q = next(i for i in range(len(t)) if t[i].kind == 3)

    def refused(arr, n, what, geometry=1):
        assert not lib.e2mi_create_tensors(arr, n, geometry, cfg.n_layers, cfg.vocab, 0)
        assert what in e2mi.last_error(), e2mi.last_error()

    refused(t, len(t) - 1, "missing")
    t[q].N += 8
    t[q].Npad += 8
    refused(t, len(t), "mis-shaped")
    t[q].N -= 8
    refused(t, len(t), "Npad")
    t[q].Npad -= 8
    t[q].kind = 7
    refused(t, len(t), "kind")
    t[q].kind = 3
    scale = t[q].scale
    t[q].scale = None
    refused(t, len(t), "no scales")
    t[q].scale = scale
    dup = (e2mi.E2MITensor * (len(t) + 1))(*t, t[0])
    refused(dup, len(dup), "twice")
    refused(t, len(t), "geometry", geometry=5)
    refused(None, 0, "no tensors")
    # the complete list passes the checks; without a gfx950 device the engine itself then fails
    t2 = e2mi.model_tensors(m)
    if not lib.e2mi_create_tensors(t2, len(t2), 1, cfg.n_layers, cfg.vocab, 0):
        assert "create_tensors" not in e2mi.last_error(), e2mi.last_error()
