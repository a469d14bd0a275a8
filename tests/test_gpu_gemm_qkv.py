"""The fused q|k|v GEMM (e2mi_i8_gemm_qkv): the projection of text.c:836-838 with the q/k/v RMSNorm
and RoPE of text.c:853-854 in its epilogue, against the same two stages run separately
(e2mi_i8_gemm then e2mi_qkv_norm_rope / _packed, each pinned to the oracle elsewhere) and against
the oracle's composition directly.

The fused epilogue adds a row's squares in another order (its 256 columns spread over two waves
and 32 lanes), so its inverse rms can differ from the row kernel's by an ulp: the f32 outputs are
held to 2e-6 relative of the separate stages (1e-6 absolute, where RoPE's difference cancels) and
1e-5 of the oracle, and the f16 outputs to one f16 rounding step on at most 1 % of the elements.
Covered: the padded layout (positions m % S, V^T
per sequence), packed rows with their own positions (V^T over all rows), row counts that leave a
partial 128-row tile, the BASELINE heads (3 q + 1 kv) and the reference checkpoint's sliding
layers (4 q + 2 kv), and the row order the weight must be stored in."""
import numpy as np
import pytest

from conftest import assert_f32_close

pytestmark = pytest.mark.gpu

EPS = 1e-6
D = 256


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _np(t):
    return t.cpu().numpy()


def _setup(rng, oracle, M, H, KV, K=768):
    N = (H + 2 * KV) * D
    x = rng.standard_normal((M, K)).astype(np.float32)
    qa, as_ = oracle.quantize(x)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    ws = rng.uniform(0.001, 0.02, N).astype(np.float32)
    gq = (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)
    gk = (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)
    return qa, as_, w, ws, gq, gk


def _f16_close(got, want, what):
    """f16 outputs: equal, or one f16 rounding step apart, on at most 1 % of the elements."""
    g = got.view(np.uint16).astype(np.int32)
    w = want.view(np.uint16).astype(np.int32)
    d = np.abs(g - w)
    assert d.max() <= 1, f"{what}: f16 outputs {d.max()} steps apart"
    assert (d > 0).mean() <= 0.01, f"{what}: {(d > 0).mean():.4f} of the f16 outputs differ"


@pytest.mark.parametrize("H,KV,B,S", [(3, 1, 4, 128), (3, 1, 2, 300), (4, 2, 3, 256)])
def test_fused_qkv_padded_layout(gpu, oracle, rng, H, KV, B, S):
    import e2mi
    M = B * S
    qa, as_, w, ws, gq, gk = _setup(rng, oracle, M, H, KV)
    order = e2mi.qkv_pair_order(np.arange(w.shape[0]))
    Wf = e2mi.DeviceWeight.from_rowmajor(np.ascontiguousarray(w[order]), np.ascontiguousarray(ws[order]))
    W = e2mi.DeviceWeight.from_rowmajor(w, ws)
    cs, sn = oracle.rope_table(S, D, 10000.0)
    qd, sd = _t(qa, gpu), _t(as_, gpu)
    args = (_t(gq, gpu), _t(gk, gpu), _t(cs, gpu), _t(sn, gpu))
    fused = e2mi.i8_gemm_qkv(qd, sd, Wf, H, KV, *args, S=S, want_f32=True)
    qkv = e2mi.i8_gemm(qd, sd, W)
    sep = e2mi.qkv_norm_rope(qkv, S, H, KV, *args, EPS, want_f32=True)
    for name, a, b in zip(("q32", "k32", "v32"), fused[3:], sep[3:]):
        assert_f32_close(_np(a), _np(b), rtol=2e-6, atol=1e-6, what=name)
    for name, a, b in zip(("q16", "k16", "vt16"), fused[:3], sep[:3]):
        _f16_close(_np(a), _np(b), name)
    # the oracle's composition, per sequence
    y = _np(qkv)
    q32, k32, v32 = (_np(t) for t in fused[3:])
    for b in range(B):
        rows = slice(b * S, (b + 1) * S)
        qo = oracle.rmsnorm(np.ascontiguousarray(y[rows, :H * D]).reshape(-1, D), gq, EPS)
        qo = oracle.rope_rows(qo, H, cs, sn).reshape(S, H * D)
        ko = oracle.rmsnorm(np.ascontiguousarray(y[rows, H * D:(H + KV) * D]).reshape(-1, D), gk, EPS)
        ko = oracle.rope_rows(ko, KV, cs, sn).reshape(S, KV * D)
        vo = oracle.rmsnorm(np.ascontiguousarray(y[rows, (H + KV) * D:]).reshape(-1, D), None, EPS).reshape(S, KV * D)
        assert_f32_close(q32[rows], qo, rtol=1e-5, atol=2e-6, what="q vs oracle")
        assert_f32_close(k32[rows], ko, rtol=1e-5, atol=2e-6, what="k vs oracle")
        assert_f32_close(v32[rows], vo, rtol=1e-5, atol=2e-6, what="v vs oracle")
    # V^T per sequence is the f16 of v32
    vt = _np(fused[2]).astype(np.float32)             # [B][KV][D][S]
    assert np.array_equal(vt, v32.astype(np.float16).astype(np.float32).reshape(B, S, KV, D).transpose(0, 2, 3, 1))


@pytest.mark.parametrize("H,KV,M", [(3, 1, 512), (3, 1, 300), (4, 2, 777)])
def test_fused_qkv_packed_rows(gpu, oracle, rng, H, KV, M):
    """Packed batches: each row's RoPE position from pos (sequences of assorted lengths laid out
    back to back), V^T over all M rows."""
    import e2mi
    qa, as_, w, ws, gq, gk = _setup(rng, oracle, M, H, KV)
    pos = []
    while len(pos) < M:
        L = int(rng.integers(1, 200))
        pos += list(range(L))
    pos = np.asarray(pos[:M], np.int32)
    order = e2mi.qkv_pair_order(np.arange(w.shape[0]))
    Wf = e2mi.DeviceWeight.from_rowmajor(np.ascontiguousarray(w[order]), np.ascontiguousarray(ws[order]))
    W = e2mi.DeviceWeight.from_rowmajor(w, ws)
    cs, sn = oracle.rope_table(512, D, 10000.0)
    qd, sd, pd = _t(qa, gpu), _t(as_, gpu), _t(pos, gpu)
    args = (_t(gq, gpu), _t(gk, gpu), _t(cs, gpu), _t(sn, gpu))
    fused = e2mi.i8_gemm_qkv(qd, sd, Wf, H, KV, *args, pos=pd, want_f32=True)
    sep = e2mi.qkv_norm_rope_packed(e2mi.i8_gemm(qd, sd, W), pd, H, KV, *args, EPS, want_f32=True)
    for name, a, b in zip(("q32", "k32", "v32"), fused[3:], sep[3:]):
        assert_f32_close(_np(a), _np(b), rtol=2e-6, atol=1e-6, what=name)
    for name, a, b in zip(("q16", "k16"), fused[:2], sep[:2]):
        _f16_close(_np(a), _np(b), name)
    _f16_close(_np(fused[2]).reshape(KV, D, M), _np(sep[2]), "vt16")


def test_fused_qkv_needs_pair_order(gpu, oracle, rng):
    """The same weight without the pair order gives different q (the epilogue pairs the wrong
    dimensions): the order is part of the entry point's contract."""
    import e2mi
    H, KV, S = 3, 1, 128
    qa, as_, w, ws, gq, gk = _setup(rng, oracle, S, H, KV)
    cs, sn = oracle.rope_table(S, D, 10000.0)
    args = (_t(gq, gpu), _t(gk, gpu), _t(cs, gpu), _t(sn, gpu))
    W = e2mi.DeviceWeight.from_rowmajor(w, ws)
    qd, sd = _t(qa, gpu), _t(as_, gpu)
    wrong = e2mi.i8_gemm_qkv(qd, sd, W, H, KV, *args, S=S, want_f32=True)
    sep = e2mi.qkv_norm_rope(e2mi.i8_gemm(qd, sd, W), S, H, KV, *args, EPS, want_f32=True)
    assert np.abs(_np(wrong[3]) - _np(sep[3])).max() > 0.1


def test_fused_qkv_rejects_bad_geometry(gpu, oracle, rng):
    import e2mi
    H, KV, S = 3, 1, 128
    qa, as_, w, ws, gq, gk = _setup(rng, oracle, 2 * S, H, KV)
    W = e2mi.DeviceWeight.from_rowmajor(w, ws)
    cs, sn = oracle.rope_table(S, D, 10000.0)
    args = (_t(gq, gpu), _t(gk, gpu), _t(cs, gpu), _t(sn, gpu))
    with pytest.raises(e2mi.E2MIError):
        e2mi.i8_gemm_qkv(_t(qa, gpu), _t(as_, gpu), W, 4, KV, *args, S=S)     # N != (H + 2 KV) * 256
    with pytest.raises(e2mi.E2MIError):
        e2mi.i8_gemm_qkv(_t(qa[:200], gpu), _t(as_[:200], gpu), W, H, KV, *args, S=S)  # M % S
