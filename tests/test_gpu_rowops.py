"""Row kernels (RMSNorm family + quantize, embedding, q/k/v norm + RoPE, GeGLU, pooling) vs the
oracle. Bars: f32 within 1e-5 relative of the oracle (IEEE arithmetic, different summation order);
quantized bytes exact for the kernel's own f32 values, and within one step of the oracle's bytes
only at a rounding boundary (the test_gpu_ffn.c:114-120 rule)."""
import numpy as np
import pytest

from conftest import assert_f32_close

pytestmark = pytest.mark.gpu
EPS = 1e-6


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _np(t):
    return t.cpu().numpy()


def _bytes_rule(q_gpu, x_oracle, oracle):
    qo, so = oracle.quantize(np.ascontiguousarray(x_oracle, np.float32))
    d = np.abs(q_gpu.astype(int) - qo.astype(int))
    scaled = x_oracle / np.repeat(so, 128, axis=1)
    near = np.abs(scaled - (np.floor(scaled) + 0.5)) < 0.002
    assert np.all((d == 0) | ((d == 1) & near)), f"{int((d > 1).sum())} bytes off by >1"


@pytest.mark.parametrize("M,D", [(1, 768), (333, 768), (64, 1152), (17, 256)])
def test_norm_quant(gpu, oracle, rng, M, D):
    import e2mi
    x = (rng.standard_normal((M, D)) * rng.uniform(0.1, 30, (M, 1))).astype(np.float32)
    g = (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)
    xn, q, qs = e2mi.norm_quant(_t(x, gpu), _t(g, gpu), EPS)
    xo = oracle.rmsnorm(x, g, EPS)
    assert_f32_close(_np(xn), xo, rtol=1e-5, atol=1e-6, what="rmsnorm")
    qg, sg = oracle.quantize(_np(xn))
    assert np.array_equal(_np(q), qg) and np.array_equal(_np(qs).view(np.uint32), sg.view(np.uint32))
    _bytes_rule(_np(q), xo, oracle)


@pytest.mark.parametrize("M,D", [(2048, 768), (5, 768)])
def test_add_norm_quant(gpu, oracle, rng, M, D):
    import e2mi
    src = (rng.standard_normal((M, D)) * 20).astype(np.float32)
    res = rng.standard_normal((M, D)).astype(np.float32)
    ga = (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)
    gn = (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)
    x, xn, q, qs = e2mi.add_norm_quant(_t(src, gpu), _t(res, gpu), _t(ga, gpu), _t(gn, gpu), EPS)
    xo = oracle.norm_add(src, res, ga, EPS)
    assert_f32_close(_np(x), xo, rtol=1e-5, atol=1e-5, what="norm_add")
    xno, _ = oracle.norm_split(_np(x), gn, EPS)      # norm_split of the kernel's own x
    assert_f32_close(_np(xn), xno, rtol=1e-5, atol=1e-6, what="norm_split")
    qg, sg = oracle.quantize(_np(xn))
    assert np.array_equal(_np(q), qg) and np.array_equal(_np(qs), sg)
    # in place: x_out aliasing res (the encoder's residual stream)
    import torch
    rt = _t(res, gpu)
    e2mi.add_norm_quant(_t(src, gpu), rt, _t(ga, gpu), None, EPS, x_out=rt)
    assert_f32_close(_np(rt), xo, rtol=1e-5, atol=1e-5, what="in-place norm_add")


def test_embed_norm_quant(gpu, oracle, rng):
    import e2mi
    V, D, M = 1000, 768, 300
    table = (0.02 * rng.standard_normal((V, D))).astype(np.float32)
    ids = rng.integers(0, V, M).astype(np.int32)
    g = (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)
    scale = np.float32(np.sqrt(768.0))
    x, q, qs = e2mi.embed_norm_quant(_t(table, gpu), _t(ids, gpu), float(scale), _t(g, gpu), EPS)
    xo = table[ids] * scale
    assert np.array_equal(_np(x), xo)  # one f32 multiply: exact
    _bytes_rule(_np(q), oracle.rmsnorm(xo, g, EPS), oracle)


@pytest.mark.parametrize("B,S", [(2, 64), (3, 100)])
def test_qkv_norm_rope(gpu, oracle, rng, B, S):
    import e2mi
    H, KV, D = 3, 1, 256
    M = B * S
    qkv = (rng.standard_normal((M, (H + 2 * KV) * D)) * 15).astype(np.float32)
    gq = (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)
    gk = (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)
    cs, sn = oracle.rope_table(S, D, 10000.0)
    q16, k16, vt16, q32, k32, v32 = e2mi.qkv_norm_rope(_t(qkv, gpu), S, H, KV, _t(gq, gpu), _t(gk, gpu),
                                                       _t(cs, gpu), _t(sn, gpu), EPS)
    for b in range(B):
        rows = slice(b * S, (b + 1) * S)
        qo = oracle.rmsnorm(qkv[rows, :H * D].reshape(-1, D), gq, EPS)
        qo = oracle.rope_rows(qo, H, cs, sn).reshape(S, H * D)
        ko = oracle.rmsnorm(qkv[rows, H * D:(H + KV) * D].reshape(-1, D), gk, EPS)
        ko = oracle.rope_rows(ko, KV, cs, sn).reshape(S, KV * D)
        vo = oracle.rmsnorm(qkv[rows, (H + KV) * D:].reshape(-1, D), None, EPS).reshape(S, KV * D)
        assert_f32_close(_np(q32)[rows], qo, rtol=1e-5, atol=2e-6, what="q")
        assert_f32_close(_np(k32)[rows], ko, rtol=1e-5, atol=2e-6, what="k")
        assert_f32_close(_np(v32)[rows], vo, rtol=1e-5, atol=2e-6, what="v")
    import torch
    assert torch.equal(q16, q32.half()) and torch.equal(k16, k32.half())
    vt = vt16.float().cpu().numpy()                   # [B][KV][D][S]
    assert np.array_equal(vt, _np(v32.half().float()).reshape(B, S, KV, D).transpose(0, 2, 3, 1))


@pytest.mark.parametrize("M", [1, 300])
def test_gelu_mul_quant(gpu, oracle, rng, M):
    import e2mi
    D = 1152
    gate = (rng.standard_normal((M, D)) * 3).astype(np.float32)
    up = (rng.standard_normal((M, D)) * 3).astype(np.float32)
    gt = _t(gate, gpu)
    q, qs = e2mi.gelu_mul_quant(gt, _t(up, gpu))
    go, qo, so = oracle.gelu_mul_quant(gate, up)
    assert_f32_close(_np(gt), go, rtol=1e-5, atol=1e-6, what="gelu*up")
    qg, sg = oracle.quantize(_np(gt))
    assert np.array_equal(_np(q), qg) and np.array_equal(_np(qs), sg)
    _bytes_rule(_np(q), go, oracle)


@pytest.mark.parametrize("D", [768, 1280])
def test_pool_l2(gpu, oracle, rng, D):
    """(D = 1280: the widest hidden/out_dim the model container accepts.)"""
    import e2mi
    B, S = 5, 200
    x = rng.standard_normal((B * S, D)).astype(np.float32)
    valid = (rng.random(B * S) > 0.3).astype(np.uint8)
    valid[2 * S:3 * S] = 0                             # an all-invalid sequence -> exact zeros
    valid[4 * S:4 * S + 1] = 1
    valid[4 * S + 1:5 * S] = 0                         # a single valid row
    out = _np(e2mi.pool_l2(_t(x, gpu), _t(valid, gpu), B, S))
    for b in range(B):
        vb = valid[b * S:(b + 1) * S]
        want = oracle.meanpool_l2(np.ascontiguousarray(x[b * S:(b + 1) * S]), vb)
        if vb.any():
            assert_f32_close(out[b], want, rtol=1e-5, atol=1e-7, what=f"pool {b}")
            assert abs(np.linalg.norm(out[b]) - 1) < 1e-5
        else:
            assert np.all(out[b] == 0)
