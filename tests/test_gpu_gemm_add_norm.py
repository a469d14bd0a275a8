"""The projection with the norm_add in its epilogue (e2mi_i8_gemm_add_norm_quant and
e2mi_i8_gemm_add_norm_scale_quant, gemm_an.hip) against the two launches each replaces,
e2mi_i8_gemm then e2mi_add_norm_quant / e2mi_add_norm_scale_quant (the encoder's O and down
projections and the norm_add after each, text.c:944-953; the reference checkpoint's 512-wide
projections and its PLE layers' scaled norm_add, text.c:955-961).

Bars: every output bit-identical with the two launches (the same per-128 fold, the same row
arithmetic), which test_gpu_gemm.py and test_gpu_rowops.py pin to the oracle; the projection y also
bit-exact with the oracle's GEMM directly on a small case. Row counts cover one 16-row unit, ragged
last units, fewer units than CUs, one to five units per workgroup and several chunks per workgroup;
K = 768 (O) and 1152 (down); 512-wide rows at K = 512 to 2048, plain and scaled."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
EPS = 1e-6
D = 768


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _np(t):
    return t.cpu().numpy()


def _case(rng, M, K, N=D):
    qa = rng.integers(-127, 128, (M, K), dtype=np.int8)
    as_ = rng.uniform(0.001, 0.05, (M, K // 128)).astype(np.float32)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    ws = rng.uniform(0.001, 0.02, N).astype(np.float32)
    res = rng.standard_normal((M, N)).astype(np.float32)
    ga = (1 + 0.05 * rng.standard_normal(N)).astype(np.float32)
    gn = (1 + 0.05 * rng.standard_normal(N)).astype(np.float32)
    return qa, as_, w, ws, res, ga, gn


def _same(a, b, what):
    a, b = _np(a), _np(b)
    assert a.shape == b.shape, what
    bad = np.flatnonzero(a.reshape(-1).view(np.uint8 if a.dtype == np.int8 else np.uint32) !=
                         b.reshape(-1).view(np.uint8 if b.dtype == np.int8 else np.uint32))
    assert bad.size == 0, f"{what}: {bad.size} elements differ, first at {np.unravel_index(bad[0], a.shape)}"


def _both(gpu, rng, M, K, gamma_next=True, want_xn=True, quant=True, inplace=False, N=D, post_scale=None):
    """post_scale None: the plain norm_add; else the scaled one (x itself quantized without gamma_next)"""
    import e2mi
    qa, as_, w, ws, res, ga, gn = _case(rng, M, K, N)
    W = e2mi.DeviceWeight.from_rowmajor(w, ws)
    tqa, tas, tga = _t(qa, gpu), _t(as_, gpu), _t(ga, gpu)
    tgn = _t(gn, gpu) if gamma_next else None
    # the two launches
    y0 = e2mi.i8_gemm(tqa, tas, W)
    r0 = _t(res, gpu)
    if post_scale is None:
        x0, xn0, q0, qs0 = e2mi.add_norm_quant(y0, r0, tga, tgn, EPS, x_out=r0 if inplace else None,
                                               want_xn=want_xn, quant=quant)
    else:
        x0, xn0, q0, qs0 = e2mi.add_norm_scale_quant(y0, r0, tga, post_scale, tgn, EPS,
                                                     x_out=r0 if inplace else None, want_xn=want_xn, quant=quant)
    # the fused one
    r1 = _t(res, gpu)
    if post_scale is None:
        x1, xn1, q1, qs1, y1 = e2mi.i8_gemm_add_norm_quant(tqa, tas, W, r1, tga, tgn, EPS,
                                                           x_out=r1 if inplace else None, want_xn=want_xn,
                                                           quant=quant, want_y=True)
    else:
        x1, xn1, q1, qs1, y1 = e2mi.i8_gemm_add_norm_scale_quant(tqa, tas, W, r1, tga, post_scale, tgn, EPS,
                                                                 x_out=r1 if inplace else None, want_xn=want_xn,
                                                                 quant=quant, want_y=True)
    _same(y1, y0, "y")
    _same(x1, x0, "x")
    if gamma_next and want_xn:
        _same(xn1, xn0, "xn")
    if quant and (gamma_next or post_scale is not None):
        _same(q1, q0, "q")
        _same(qs1, qs0, "qs")
    return qa, as_, w, ws, y1


@pytest.mark.parametrize("M,K", [(1, 768), (16, 768), (50, 1152), (333, 768), (1000, 1152), (4100, 768),
                                 (17408, 768), (17408, 1152), (17264, 768), (44000, 768)])
def test_fused_equals_two_launches(gpu, rng, M, K):
    _both(gpu, rng, M, K)


@pytest.mark.parametrize("variant", ["x_only", "no_xn", "no_q", "inplace"])
def test_fused_output_variants(gpu, rng, variant):
    kw = {"x_only": dict(gamma_next=False), "no_xn": dict(want_xn=False), "no_q": dict(quant=False),
          "inplace": dict(inplace=True)}[variant]
    _both(gpu, rng, 2100, 768, **kw)


@pytest.mark.parametrize("M,K", [(1, 512), (50, 1024), (2100, 2048), (17408, 1024), (17408, 2048)])
def test_fused_512_equals_two_launches(gpu, rng, M, K):
    _both(gpu, rng, M, K, N=512)


@pytest.mark.parametrize("M,K,gamma_next", [(333, 2048, False), (17408, 2048, False), (17408, 512, True),
                                            (5, 512, True)])
def test_fused_scaled_equals_two_launches(gpu, rng, M, K, gamma_next):
    """the PLE layers' norm_adds: after the down projection x itself quantized (scale 1), after the
    PLE projection scaled by the layer scalar and normed for the next layer"""
    _both(gpu, rng, M, K, N=512, gamma_next=gamma_next, post_scale=1.0 if not gamma_next else 0.7373)
    _both(gpu, rng, 300, K, N=512, gamma_next=gamma_next, post_scale=0.2, inplace=True)


def test_fused_fast_fold(gpu, rng):
    import e2mi
    prev = e2mi.load().e2mi_gemm_set_fold(1)
    try:
        _both(gpu, rng, 3000, 1152)
    finally:
        e2mi.load().e2mi_gemm_set_fold(prev)


def test_fused_projection_vs_oracle(gpu, oracle, rng):
    qa, as_, w, ws, y = _both(gpu, rng, 96, 1152)
    yo = oracle.i8_gemm(qa, as_, w, ws)
    assert np.array_equal(_np(y).view(np.uint32), np.asarray(yo, np.float32).view(np.uint32))


def test_fused_refuses(gpu, rng):
    import e2mi
    qa, as_, w, ws, res, ga, gn = _case(rng, 64, 768)
    Wb = e2mi.DeviceWeight.from_rowmajor(w, ws, bias=np.zeros(D, np.float32))
    with pytest.raises(RuntimeError, match="bias"):
        e2mi.i8_gemm_add_norm_quant(_t(qa, gpu), _t(as_, gpu), Wb, _t(res, gpu), _t(ga, gpu), _t(gn, gpu))
    W2 = e2mi.DeviceWeight.from_rowmajor(np.zeros((256, 768), np.int8), np.ones(256, np.float32))
    with pytest.raises(RuntimeError, match="N = 512 or 768"):
        e2mi.i8_gemm_add_norm_quant(_t(qa, gpu), _t(as_, gpu), W2, _t(res[:, :256], gpu), _t(ga[:256], gpu),
                                    _t(gn[:256], gpu))
    W7 = e2mi.DeviceWeight.from_rowmajor(w, ws)
    with pytest.raises(RuntimeError, match="512-wide"):
        e2mi.i8_gemm_add_norm_scale_quant(_t(qa, gpu), _t(as_, gpu), W7, _t(res, gpu), _t(ga, gpu), 1.0, None)


def test_engine_fused_equals_unfused(gpu, rng, monkeypatch):
    """The engine with the fused O/down + norm_add launches (default) against E2MI_NOFUSE_AN=1 (the
    GEMM, then the row kernel): the same embeddings bit for bit, through the host entry (packed and
    padded rows) and the device entry (planned on the device: the kernel reads the device row
    count and its row ranges follow it, over batches of several row counts)."""
    import sys
    import torch
    sys.path.insert(0, __file__.rsplit("/", 1)[0])
    from model_util import random_batch, small_config
    import e2mi
    m = e2mi.Model.synthetic(small_config(e2mi, n_layers=2), 77)
    fused = e2mi.Engine(m, max_rows=32768)
    monkeypatch.setenv("E2MI_NOFUSE_AN", "1")
    plain = e2mi.Engine(m, max_rows=32768)
    monkeypatch.delenv("E2MI_NOFUSE_AN")
    # the last batch has more rows than one round of the CUs covers: the engine runs the separate
    # kernels there (both entries)
    for B, S, lo in [(4, 128, 40), (9, 300, 1), (16, 256, 200), (2, 512, 500), (50, 512, 480)]:
        ids, valid = random_batch(rng, B, S, 1000, min_len=lo)
        a, b = fused.embed_batch(ids, valid), plain.embed_batch(ids, valid)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (B, S)
        tid, tv = torch.from_numpy(ids).to(gpu), torch.from_numpy(valid).to(gpu)
        oa = torch.empty((B, 768), device=gpu)
        ob = torch.empty((B, 768), device=gpu)
        fused.embed_batch_device(tid, tv, oa)
        plain.embed_batch_device(tid, tv, ob)
        torch.cuda.synchronize()
        assert np.array_equal(_np(oa).view(np.uint32), a.view(np.uint32)), (B, S, "device entry")
        assert np.array_equal(_np(ob).view(np.uint32), a.view(np.uint32)), (B, S, "device entry, unfused")
    for e in (fused, plain):
        e.set_packing(False)
    ids, valid = random_batch(rng, 5, 200, 1000, min_len=20)
    a, b = fused.embed_batch(ids, valid), plain.embed_batch(ids, valid)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), "padded rows"


def test_engine_fused_equals_unfused_reference_geometry(gpu, rng, monkeypatch):
    """The reference checkpoint's geometry (hidden 512, PLE, window, a head_dim-512 layer): the O,
    down and PLE projections with their norm_adds fused (the down's quantizing x itself, the PLE
    projection's scaled by the layer scalar) give the same embeddings bit for bit as
    E2MI_NOFUSE_AN=1, through the host and the device entry."""
    import sys
    import torch
    sys.path.insert(0, __file__.rsplit("/", 1)[0])
    from model_util import random_batch, reference_small_config
    import e2mi
    m = e2mi.Model.synthetic(reference_small_config(e2mi, n_layers=6), 78)
    fused = e2mi.Engine(m, max_rows=4096)
    monkeypatch.setenv("E2MI_NOFUSE_AN", "1")
    plain = e2mi.Engine(m, max_rows=4096)
    monkeypatch.delenv("E2MI_NOFUSE_AN")
    for B, S, lo in [(4, 256, 60), (3, 1024, 600), (16, 128, 1)]:
        ids, valid = random_batch(rng, B, S, 1000, min_len=lo)
        a, b = fused.embed_batch(ids, valid), plain.embed_batch(ids, valid)
        assert a.shape == (B, 768)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (B, S)
        tid, tv = torch.from_numpy(ids).to(gpu), torch.from_numpy(valid).to(gpu)
        oa = torch.empty((B, 768), device=gpu)
        fused.embed_batch_device(tid, tv, oa)
        torch.cuda.synchronize()
        assert np.array_equal(_np(oa).view(np.uint32), a.view(np.uint32)), (B, S, "device entry")
