"""HIP quantizer and int8 MFMA GEMM vs the oracle (through the C ABI, on a gfx950 device).

Bars (include/e2mi.h): quantized bytes and scales bit-exact for the same f32
input; int32 block accumulators bit-exact; f32 GEMM output bit-exact with the reference's AVX-512
fold order (the oracle is pinned to it in test_oracle_ref.py), so also within 1e-4.
"""
import numpy as np
import pytest

from conftest import assert_f32_close

pytestmark = pytest.mark.gpu


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _np(t):
    return t.cpu().numpy()


def _acts(rng, M, K):
    x = rng.standard_normal((M, K)).astype(np.float32) * rng.uniform(0.01, 50, (M, 1)).astype(np.float32)
    x[:, rng.integers(0, K, 2)] *= 30
    x[0] = 0
    if M > 3:
        x[3, :128] = np.arange(128, dtype=np.float32) - 63.5
    return x


@pytest.mark.parametrize("M,K", [(1, 128), (128, 768), (333, 1152), (2048, 768)])
@pytest.mark.parametrize("block", [128, "K"])
def test_quantize_bit_exact(gpu, oracle, rng, M, K, block):
    import e2mi
    blk = K if block == "K" else block
    x = _acts(rng, M, K)
    q, s = e2mi.quantize(_t(x, gpu), block=blk)
    qo, so = oracle.quantize(x, block=blk)
    assert np.array_equal(_np(q), qo)
    assert np.array_equal(_np(s).view(np.uint32), so.view(np.uint32))


def test_quantize_strided_rows(gpu, oracle, rng):
    import e2mi
    import torch
    x = _acts(rng, 64, 1024)
    xt = _t(x, gpu)[:, :768]                      # ldx = 1024 > K = 768
    q, s = e2mi.quantize(xt)
    qo, so = oracle.quantize(np.ascontiguousarray(x[:, :768]))
    assert np.array_equal(_np(q), qo) and np.array_equal(_np(s), so)


def _gemm_case(rng, M, N, K):
    qa = rng.integers(-127, 128, (M, K), dtype=np.int8)
    as_ = rng.uniform(0.001, 0.05, (M, K // 128)).astype(np.float32)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    ws = rng.uniform(0.001, 0.02, N).astype(np.float32)
    return qa, as_, w, ws


@pytest.mark.parametrize("M,N,K", [(128, 1152, 768), (1, 8, 128), (77, 200, 384),
                                   (513, 1280, 768), (1000, 768, 1152)])
def test_gemm_bit_exact(gpu, oracle, rng, M, N, K):
    import e2mi
    qa, as_, w, ws = _gemm_case(rng, M, N, K)
    W = e2mi.DeviceWeight.from_rowmajor(w, ws)
    y, acc = e2mi.i8_gemm_acc(_t(qa, gpu), _t(as_, gpu), W)
    assert np.array_equal(_np(acc), oracle.i8_gemm_acc(qa, w))
    yo = oracle.i8_gemm(qa, as_, w, ws)
    assert np.array_equal(_np(y).view(np.uint32), yo.view(np.uint32))
    y2 = e2mi.i8_gemm(_t(qa, gpu), _t(as_, gpu), W)   # the production kernel, no dump
    assert np.array_equal(_np(y2).view(np.uint32), yo.view(np.uint32))


def test_gemm_config1_bias_and_packed_upload(gpu, oracle, rng):
    """A f32 128x768 ~N(0,1) quantized per block, W int8 1152x768 uniform,
    ws ~U(0.001,0.02), bias ~N(0,0.01); weights uploaded in the reference's packed layout."""
    import e2mi
    M, N, K = 128, 1152, 768
    a = rng.standard_normal((M, K)).astype(np.float32)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    ws = rng.uniform(0.001, 0.02, N).astype(np.float32)
    bias = (0.01 * rng.standard_normal(N)).astype(np.float32)
    wq, _ = oracle.q8w_pack(w)
    W = e2mi.DeviceWeight.from_packed(wq, ws, N, K, bias=bias)
    q, s = e2mi.quantize(_t(a, gpu))
    y = e2mi.i8_gemm(q, s, W)
    qo, so = oracle.quantize(a)
    assert np.array_equal(_np(q), qo)
    yo = oracle.i8_gemm(qo, so, w, ws, bias=bias)
    assert np.array_equal(_np(y).view(np.uint32), yo.view(np.uint32))
    # and the int8 result tracks the fp32 product (test_int8.c:135 bar)
    yf = a @ (w.astype(np.float32) * ws[:, None]).T + bias
    cos = float((_np(y) * yf).sum() / np.linalg.norm(_np(y)) / np.linalg.norm(yf))
    assert cos > 0.9995


def test_gemm_column_range_and_clamp(gpu, oracle, rng):
    import e2mi
    import torch
    M, N, K = 40, 96, 256
    qa, as_, w, ws = _gemm_case(rng, M, N, K)
    W = e2mi.DeviceWeight.from_rowmajor(w, ws)
    W.set_clamp(-0.5, 0.5)
    y = torch.full((M, N), 7.0, device=gpu)
    e2mi.i8_gemm(_t(qa, gpu), _t(as_, gpu), W, n0=24, n1=72, y=y)
    yo = oracle.i8_gemm(qa, as_, w, ws, lo=-0.5, hi=0.5)
    got = _np(y)
    assert np.all(got[:, :24] == 7.0) and np.all(got[:, 72:] == 7.0)   # untouched columns
    assert np.array_equal(got[:, 24:72].view(np.uint32), yo[:, 24:72].view(np.uint32))


@pytest.mark.parametrize("M,N,K", [(128, 1152, 768), (300, 768, 1152), (64, 128, 128)])
def test_gemm_requant_epilogue(gpu, oracle, rng, M, N, K):
    import e2mi
    qa, as_, w, ws = _gemm_case(rng, M, N, K)
    W = e2mi.DeviceWeight.from_rowmajor(w, ws)
    yq, ys = e2mi.i8_gemm_q(_t(qa, gpu), _t(as_, gpu), W)
    yo = oracle.i8_gemm(qa, as_, w, ws)
    qo, so = oracle.quantize(yo)          # bit-exact f32, so bit-exact requantization
    assert np.array_equal(_np(yq), qo)
    assert np.array_equal(_np(ys).view(np.uint32), so.view(np.uint32))


@pytest.mark.parametrize("M", [64, 2048, 100])
def test_gemm_geglu_epilogue(gpu, oracle, rng, M):
    """gate|up GEMM + GELU-tanh * up + per-128 quantization in one kernel (config 2's FFN core)."""
    import e2mi
    F, K = 1152, 768
    qa = rng.integers(-127, 128, (M, K), dtype=np.int8)
    as_ = rng.uniform(0.001, 0.01, (M, K // 128)).astype(np.float32)
    wg = rng.integers(-127, 128, (F, K), dtype=np.int8)
    wu = rng.integers(-127, 128, (F, K), dtype=np.int8)
    sg = rng.uniform(0.001, 0.02, F).astype(np.float32)
    su = rng.uniform(0.001, 0.02, F).astype(np.float32)
    wi, si = e2mi.interleave_gate_up(wg, sg, wu, su)
    W = e2mi.DeviceWeight.from_rowmajor(wi, si)
    q, qs, g = e2mi.i8_gemm_geglu(_t(qa, gpu), _t(as_, gpu), W)
    gate = oracle.i8_gemm(qa, as_, wg, sg)
    up = oracle.i8_gemm(qa, as_, wu, su)
    go, qo, so = oracle.gelu_mul_quant(gate, up)
    g = _np(g)
    # the reference's own bar for this stage: |got - want| / (1 + |want|) < 1e-4 (test_gpu_ffn.c:104);
    # for very negative gate values both reference formulas cancel in 1 + tanh, the kernel does not
    assert_f32_close(g, go, rtol=1e-4, atol=1e-4, what="gelu*up")
    # bytes: exact for the kernel's own f32 values; within one step of the oracle's only where the
    # scaled value sits at a rounding boundary (test_gpu_ffn.c:114-120 rule)
    qg, sgk = oracle.quantize(g)
    assert np.array_equal(_np(q), qg)
    assert np.array_equal(_np(qs).view(np.uint32), sgk.view(np.uint32))
    d = np.abs(_np(q).astype(int) - qo.astype(int))
    scaled = go / np.repeat(so, 128, axis=1)
    near = np.abs(scaled - (np.floor(scaled) + 0.5)) < 0.002
    assert np.all((d == 0) | ((d == 1) & near))
    assert_f32_close(_np(qs), so, rtol=1e-4, what="scales")


@pytest.mark.parametrize("M,N,K", [(128, 1152, 768), (77, 200, 384), (300, 768, 1152), (1, 8, 128)])
def test_gemm_per_token_bit_exact(gpu, oracle, rng, M, N, K):
    """Per-token activation scales (BASELINE configs 1 and 5; the reference built with one block per
    row, int8.h:61-70 E2_I8_BLOCK = K): int32 over the whole K, one fold, bit-exact."""
    import e2mi
    qa = rng.integers(-127, 128, (M, K), dtype=np.int8)
    as_ = rng.uniform(0.001, 0.05, (M, 1)).astype(np.float32)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    ws = rng.uniform(0.001, 0.02, N).astype(np.float32)
    bias = (0.01 * rng.standard_normal(N)).astype(np.float32)
    W = e2mi.DeviceWeight.from_rowmajor(w, ws, bias=bias)
    y = e2mi.i8_gemm_tok(_t(qa, gpu), _t(as_, gpu), W)
    yo = oracle.i8_gemm(qa, as_, w, ws, bias=bias, block=K)
    assert np.array_equal(_np(y).view(np.uint32), yo.view(np.uint32))


def test_gemm_per_token_config1_quantized(gpu, oracle, rng):
    """BASELINE config 1 as written: A f32 [128 x 768] ~N(0,1) quantized per token, W uniform int8,
    ws ~U(0.001,0.02), bias ~N(0,0.01); quantizer and GEMM bit-exact, and close to the fp32 product."""
    import e2mi
    M, N, K = 128, 1152, 768
    a = rng.standard_normal((M, K)).astype(np.float32)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    ws = rng.uniform(0.001, 0.02, N).astype(np.float32)
    bias = (0.01 * rng.standard_normal(N)).astype(np.float32)
    W = e2mi.DeviceWeight.from_rowmajor(w, ws, bias=bias)
    q, s = e2mi.quantize(_t(a, gpu), block=K)
    y = e2mi.i8_gemm_tok(q, s, W)
    qo, so = oracle.quantize(a, block=K)
    assert np.array_equal(_np(q), qo) and np.array_equal(_np(s).view(np.uint32), so.view(np.uint32))
    yo = oracle.i8_gemm(qo, so, w, ws, bias=bias, block=K)
    assert np.array_equal(_np(y).view(np.uint32), yo.view(np.uint32))
    yf = a @ (w.astype(np.float32) * ws[:, None]).T + bias
    cos = float((_np(y) * yf).sum() / np.linalg.norm(_np(y)) / np.linalg.norm(yf))
    assert cos > 0.999


def test_gemm_per_token_column_range_clamp_and_requant(gpu, oracle, rng):
    import e2mi
    import torch
    M, N, K = 40, 256, 256
    qa = rng.integers(-127, 128, (M, K), dtype=np.int8)
    as_ = rng.uniform(0.001, 0.05, (M, 1)).astype(np.float32)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    ws = rng.uniform(0.001, 0.02, N).astype(np.float32)
    W = e2mi.DeviceWeight.from_rowmajor(w, ws)
    yq, ys = e2mi.i8_gemm_tok_q(_t(qa, gpu), _t(as_, gpu), W)
    qo, so = oracle.quantize(oracle.i8_gemm(qa, as_, w, ws, block=K))
    assert np.array_equal(_np(yq), qo) and np.array_equal(_np(ys).view(np.uint32), so.view(np.uint32))
    W.set_clamp(-0.5, 0.5)
    y = torch.full((M, N), 7.0, device=gpu)
    e2mi.i8_gemm_tok(_t(qa, gpu), _t(as_, gpu), W, n0=24, n1=200, y=y)
    yo = oracle.i8_gemm(qa, as_, w, ws, block=K, lo=-0.5, hi=0.5)
    got = _np(y)
    assert np.all(got[:, :24] == 7.0) and np.all(got[:, 200:] == 7.0)
    assert np.array_equal(got[:, 24:200].view(np.uint32), yo[:, 24:200].view(np.uint32))


@pytest.mark.parametrize("M,N,K,n0,n1", [(300, 1152, 768, 0, 1152), (77, 200, 512, 0, 200),
                                         (515, 384, 1152, 4, 380), (130, 77, 768, 0, 77),
                                         (64, 256, 768, 3, 250), (257, 1280, 640, 128, 1280),
                                         (1, 128, 1152, 0, 128), (700, 512, 768, 128, 512)])
def test_gemm_per_token_no_post_bit_exact(gpu, oracle, rng, M, N, K, n0, n1):
    """Per-token GEMM without bias or clamp, at shapes that take each per-token f32 kernel: the
    overlapped-epilogue one (N a multiple of 128, K = 768 or 1152) and the general one (any other
    N, column offset or K); columns outside [n0, n1) untouched."""
    import e2mi
    import torch
    qa = rng.integers(-127, 128, (M, K), dtype=np.int8)
    as_ = rng.uniform(0.001, 0.05, (M, 1)).astype(np.float32)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    ws = rng.uniform(0.001, 0.02, N).astype(np.float32)
    W = e2mi.DeviceWeight.from_rowmajor(w, ws)
    y = torch.full((M, N), 7.0, device=gpu)
    e2mi.i8_gemm_tok(_t(qa, gpu), _t(as_, gpu), W, n0=n0, n1=n1, y=y)
    yo = oracle.i8_gemm(qa, as_, w, ws, block=K)
    got = _np(y)
    assert np.all(got[:, :n0] == 7.0) and np.all(got[:, n1:] == 7.0)
    assert np.array_equal(got[:, n0:n1].view(np.uint32), yo[:, n0:n1].view(np.uint32))
