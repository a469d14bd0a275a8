"""Pin the oracle against the reference's own kernels, compiled from its sources (oracle/_ref).

Bit-exact: the per-block quantizer (AVX-512, AVX-VNNI and scalar builds), the weight quantizer and
packer, the int8 GEMM with the AVX-512 fold order, and the scalar GEMM's mul+add fold.
Tolerance: the fp32 helpers, which the reference builds with rsqrt/rcp approximations.
"""
import os

import numpy as np
import pytest

from conftest import assert_f32_close


def _acts(rng, M, K, outliers=True):
    x = rng.standard_normal((M, K)).astype(np.float32)
    x *= rng.uniform(0.01, 100, (M, 1)).astype(np.float32)
    if outliers:
        x[:, rng.integers(0, K, 3)] *= 30          # test_int8.c-style outlier columns
    x[0] = 0.0                                      # zero row: scale 1, bytes 0
    if M > 2:
        x[2, :128] = 0.0                            # one zero block
    if M > 3:                                       # exact rounding ties at scale 1/127 steps
        x[3, :128] = np.arange(128, dtype=np.float32) - 63.5
    return x


@pytest.mark.parametrize("which", ["avx512", "vnni", "scalar"])
@pytest.mark.parametrize("M,K", [(1, 128), (37, 768), (16, 1152), (9, 2048)])
def test_quantizer_bit_exact(oracle, ref, rng, which, M, K):
    x = _acts(rng, M, K)
    q1, s1 = oracle.quantize(x)
    q2, s2 = ref.quantize(x, which)
    assert np.array_equal(q1, q2)
    assert np.array_equal(s1.view(np.uint32), s2.view(np.uint32))


def test_weight_quantizer_bit_exact(oracle, ref, rng):
    for N, K in [(40, 256), (13, 768), (1152, 768)]:
        w = (rng.standard_normal((N, K)) * rng.uniform(0.001, 1, (N, 1))).astype(np.float32)
        w[0] = 0
        a, b = oracle.q8w_from_f32(w), ref.q8w_from_f32(w)
        for x, y in zip(a, b):
            assert np.array_equal(x.view(np.uint8), y.view(np.uint8))


def test_pack_unpack_layout(oracle, rng):
    N, K = 45, 384
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    wq, bsq = oracle.q8w_pack(w)
    # closed form of int8.h:17 and int8.c:57-61
    kq = K // 4
    for n in (0, 7, 8, 44):
        for k in (0, 3, 4, 127, 383):
            assert wq[(n >> 3) * kq * 32 + (k >> 2) * 32 + (n & 7) * 4 + (k & 3)] == w[n, k]
    assert np.array_equal(oracle.q8w_unpack(wq, N, K), w)
    assert np.array_equal(bsq[:, :N], w.reshape(N, K // 128, 128).sum(-1).T.astype(np.int32))


@pytest.mark.parametrize("M,N,K", [(128, 1152, 768), (37, 77, 384), (8, 40, 1152), (3, 16, 128)])
def test_gemm_avx512_fold_bit_exact(oracle, ref, rng, M, N, K):
    qa = rng.integers(-127, 128, (M, K), dtype=np.int8)
    as_ = rng.uniform(0.001, 0.05, (M, K // 128)).astype(np.float32)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    ws = rng.uniform(0.001, 0.02, N).astype(np.float32)
    wq, bsq = oracle.q8w_pack(w)
    y_or = oracle.i8_gemm(qa, as_, w, ws)
    y_ref = ref.gemm(qa, as_, wq, ws, bsq, N, K, "avx512")
    assert np.array_equal(y_or.view(np.uint32), y_ref.view(np.uint32))
    # the threaded VNNI port used by the recipe and the CPU baseline is the same arithmetic
    assert np.array_equal(oracle.i8_gemm_mt(qa, as_, w, ws).view(np.uint32), y_or.view(np.uint32))
    # the N-split is bit-identical (test_scalar_kernels.c:149-158)
    n0 = 16 if N > 32 else 0
    y_split = ref.gemm(qa, as_, wq, ws, bsq, N, K, "avx512", n0=n0, n1=N)
    assert np.array_equal(y_split[:, n0:].view(np.uint32), y_or[:, n0:].view(np.uint32))
    # the scalar reference folds with mul+add: restated exactly too
    y_s = ref.gemm(qa, as_, wq, ws, bsq, N, K, "scalar")
    assert np.array_equal(oracle.i8_gemm_scalar(qa, as_, w, ws).view(np.uint32), y_s.view(np.uint32))


def test_gemm_int32_accumulators_brute_force(oracle, rng):
    M, N, K = 5, 9, 256
    qa = rng.integers(-128, 128, (M, K), dtype=np.int8)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    acc = oracle.i8_gemm_acc(qa, w)
    want = np.einsum("mbk,nbk->bmn", qa.reshape(M, 2, 128).astype(np.int64),
                     w.reshape(N, 2, 128).astype(np.int64))
    assert np.array_equal(acc, want)
    # extreme operands stay exact: |acc| <= 128*128*128 < 2^24
    acc2 = oracle.i8_gemm_acc(np.full((1, 128), -128, np.int8), np.full((1, 128), -127, np.int8))
    assert acc2[0, 0, 0] == 128 * 128 * 127


def test_fp32_helpers_match_reference(oracle, ref, rng):
    k = ref.kernels()
    R, D, eps = 7, 768, 1e-6
    x = rng.standard_normal((R, D)).astype(np.float32) * 3
    g = (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)
    a = x.copy()
    k.rmsnorm(a.ctypes.data, R, D, g.ctypes.data, eps)
    assert_f32_close(oracle.rmsnorm(x, g, eps), a, rtol=2e-6, what="rmsnorm")
    a, res = x.copy(), np.empty_like(x)
    k.norm_split(a.ctypes.data, res.ctypes.data, R, D, g.ctypes.data, eps)
    ox, ores = oracle.norm_split(x, g, eps)
    assert_f32_close(ox, a, rtol=2e-6, what="norm_split")
    assert np.array_equal(ores, res)
    src = rng.standard_normal((R, D)).astype(np.float32)
    out = np.empty_like(x)
    k.norm_add(out.ctypes.data, src.ctypes.data, x.ctypes.data, R, D, g.ctypes.data, eps)
    assert_f32_close(oracle.norm_add(src, x, g, eps), out, rtol=2e-6, atol=1e-5, what="norm_add")
    v = np.linspace(-12, 12, 4096).astype(np.float32)
    gv = v.copy()
    k.gelu_tanh(gv.ctypes.data, gv.size)
    og = np.array([oracle.lib.or_gelu_tanh(float(t)) for t in v], np.float32)
    assert np.max(np.abs(og - gv)) < 3e-6 * 12
    s = rng.standard_normal(513).astype(np.float32) * 8
    sr = s.copy()
    k.softmax(sr.ctypes.data, sr.size)
    sd = np.exp(s.astype(np.float64) - s.max())
    sd /= sd.sum()
    # the reference's own bar vs double (test_softmax.c:33), for both float implementations
    assert np.max(np.abs(oracle.softmax(s) - sd)) < 3e-7 * 4
    assert np.max(np.abs(sr - sd)) < 3e-7 * 4
    valid = (rng.random(50) > 0.3).astype(np.uint8)
    xm = rng.standard_normal((50, 768)).astype(np.float32)
    assert_f32_close(oracle.meanpool_l2(xm, valid), ref.meanpool_l2(xm, valid), rtol=1e-6,
                     atol=1e-7, what="pool")


@pytest.mark.parametrize("K", [768, 1152])
def test_per_row_build_bit_exact(oracle, rng, K):
    """The reference built with one activation block per row (E2_I8_BLOCK = K, int8.h:61-70):
    its quantizer and GEMM against the oracle's block = K restatement, bit for bit. These builds
    are the CPU baseline of the per-token GEMM sweep."""
    from oracle.binding import Ref
    if not os.path.exists(Ref.per_row_path(K)):
        pytest.skip("oracle/_ref per-row builds absent (the reference tree is absent on this host)")
    ref = Ref.per_row(K)
    M, N = 37, 77
    x = _acts(rng, M, K)
    q1, s1 = oracle.quantize(x, block=K)
    q2, s2 = ref.quantize(x)
    assert s2.shape == (M, 1)
    assert np.array_equal(q1, q2)
    assert np.array_equal(s1.view(np.uint32), s2.view(np.uint32))
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    ws = rng.uniform(0.001, 0.02, N).astype(np.float32)
    wq, _ = oracle.q8w_pack(w)
    bsq = w.astype(np.int32).sum(1)[None, :]
    y_ref = ref.gemm(q1, s1, wq, ws, bsq, N, K, "avx512")
    y_or = oracle.i8_gemm(q1, s1, w, ws, block=K)
    assert np.array_equal(y_or.view(np.uint32), y_ref.view(np.uint32))
    # and it differs from the per-128 build's result (the block is really K)
    y128 = oracle.i8_gemm(*oracle.quantize(x), w, ws)
    assert not np.array_equal(y128, y_or)


@pytest.mark.parametrize("K,N", [(768, 1152), (1152, 768)])
def test_pool_harness_matches_oracle(oracle, rng, K, N):
    """The CPU baseline's harness (oracle/ref_gemm_pool.c: the reference's e2_i8_gemm_avx512 on its
    own pool, columns claimed in tiles) computes the per-token GEMM the oracle restates, bit for bit,
    on a partial column tile and a row count the reference pads to 8."""
    from oracle.binding import Q8W, RefGemmPool
    if not RefGemmPool.available(K):
        pytest.skip("oracle/_ref not built")
    import bench
    if "avx512_vnni" not in bench.cpu_flags():
        pytest.skip("no AVX-512 VNNI on this host")
    M = 136
    pool = RefGemmPool(K, nthreads=4)
    try:
        qa = rng.integers(-127, 128, (M, K), dtype=np.int8)
        qb = (qa.view(np.uint8) ^ 0x80).view(np.int8).copy()
        as_ = rng.uniform(0.001, 0.05, (M, 1)).astype(np.float32)
        w, ws, wq = bench.packed_weight(rng, N, K)
        bsq = np.zeros(N + 32, np.int32)
        bsq[:N] = w.astype(np.int32).sum(1)
        wsp = np.zeros(N + 32, np.float32)
        wsp[:N] = ws
        wqp = np.concatenate([wq, np.zeros(4 * K * 8, np.int8)])
        q = Q8W(wqp.ctypes.data, bsq.ctypes.data, wsp.ctypes.data, N, K, 1, N, -1e31, 1e31, 1)
        y = np.zeros((M, N), np.float32)
        pool.gemm(0, y, qb, as_, q)
        yo = oracle.i8_gemm(qa, as_, w, ws, block=K)
        assert np.array_equal(y.view(np.uint32), yo.view(np.uint32))
    finally:
        pool.close()
