"""Oracle functions pinned by mathematics (closed forms and double-precision evaluation)."""
import numpy as np
import pytest


def test_rope_table_closed_form(oracle):
    """The table the oracle (and the product's host code) builds: cos/sin(p / theta^(2i/D)),
    duplicated over both halves (text.c:483-506), against float64."""
    S, D = 64, 256
    cs, sn = oracle.rope_table(S, D, 10000.0)
    i = np.arange(D // 2)
    f = np.arange(S)[:, None] / (10000.0 ** (2 * i / D))[None, :]
    # the angle is p * inv in float32 (text.c:500-501): its rounding error grows like p * 2^-24
    tol = 2e-6 + np.arange(S)[:, None] * 1.2e-7
    assert np.all(np.abs(cs[:, :D // 2] - np.cos(f)) <= tol) and np.array_equal(cs[:, D // 2:], cs[:, :D // 2])
    assert np.all(np.abs(sn[:, :D // 2] - np.sin(f)) <= tol) and np.array_equal(sn[:, D // 2:], sn[:, :D // 2])
    # a plausible slip (rotating by theta^(i/D) instead of theta^(2i/D)) is far outside the bound
    f_bad = np.arange(S)[:, None] / (10000.0 ** (i / D))[None, :]
    assert np.abs(cs[:, :D // 2] - np.cos(f_bad)).max() > 0.1


def test_gelu_accuracy_vs_double(oracle):
    v = np.linspace(-10, 10, 2001)
    want = 0.5 * v * (1 + np.tanh(np.sqrt(2 / np.pi) * (v + 0.044715 * v ** 3)))
    got = np.array([oracle.lib.or_gelu_tanh(float(t)) for t in v])
    assert np.max(np.abs(got - want)) < 3e-6 * 10  # test_softmax.c:52 bar, scaled by |v|




def test_rope_rows_rotation(oracle, rng):
    """rotate-half on one row == a 2-D rotation of each (i, i+D/2) pair by the table's angle."""
    S, D = 8, 256
    cs, sn = oracle.rope_table(S, D, 10000.0)
    x = rng.standard_normal((S, D)).astype(np.float32)
    y = oracle.rope_rows(x, 1, cs, sn)
    a, b = x[:, :D // 2].astype(np.float64), x[:, D // 2:].astype(np.float64)
    c, s = cs[:, :D // 2].astype(np.float64), sn[:, :D // 2].astype(np.float64)
    assert np.allclose(y[:, :D // 2], a * c - b * s, atol=1e-5)
    assert np.allclose(y[:, D // 2:], b * c + a * s, atol=1e-5)
    # rotation preserves each pair's norm
    assert np.allclose(np.hypot(y[:, :D // 2], y[:, D // 2:]), np.hypot(a, b), rtol=1e-5)


def test_attention_oracle_vs_float64(oracle, rng):
    """The row-wise oracle against a float64 brute force with masking (text.c:534-572)."""
    S, H, KV, D = 40, 3, 1, 256
    q = rng.standard_normal((S, H * D)).astype(np.float32)
    k = rng.standard_normal((S, KV * D)).astype(np.float32)
    v = rng.standard_normal((S, KV * D)).astype(np.float32)
    valid = (rng.random(S) > 0.25).astype(np.uint8)
    got = oracle.attention(q, k, v, valid, H, KV, D, scale=0.0625)
    want = np.zeros((S, H * D))
    vk = valid.astype(bool)
    for h in range(H):
        qh = q[:, h * D:(h + 1) * D].astype(np.float64)
        lg = qh @ k.astype(np.float64).T * 0.0625
        lg[:, ~vk] = -np.inf
        p = np.exp(lg - lg.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        want[:, h * D:(h + 1) * D] = p @ v.astype(np.float64)
    want[~vk] = 0
    assert np.abs(got - want).max() < 2e-5 * np.abs(want).max()


def test_meanpool_l2_closed_form(oracle, rng):
    x = rng.standard_normal((30, 768)).astype(np.float32)
    valid = (rng.random(30) > 0.5).astype(np.uint8)
    m = x[valid.astype(bool)].astype(np.float64).mean(0)
    assert np.allclose(oracle.meanpool_l2(x, valid), m / np.linalg.norm(m), atol=1e-6)
    assert np.all(oracle.meanpool_l2(x, np.zeros(30, np.uint8)) == 0)


def test_norms_closed_form(oracle, rng):
    x = (rng.standard_normal((4, 768)) * 5).astype(np.float32)
    g = (1 + 0.05 * rng.standard_normal(768)).astype(np.float32)
    xd = x.astype(np.float64)
    want = xd / np.sqrt((xd ** 2).mean(1, keepdims=True) + 1e-6) * g
    assert np.allclose(oracle.rmsnorm(x, g, 1e-6), want, rtol=2e-6, atol=1e-6)
    res = rng.standard_normal((4, 768)).astype(np.float32)
    assert np.allclose(oracle.norm_add(x, res, g, 1e-6), want + res, rtol=2e-6, atol=2e-6)
    xs, r = oracle.norm_split(x, g, 1e-6)
    assert np.array_equal(r, x) and np.allclose(xs, want, rtol=2e-6, atol=1e-6)


def _ref_test_inputs(S, H, KV, D):
    """The inputs of the reference's attention test (test_text_attention.c:47-53)."""
    GD, KD = H * D, KV * D
    i = np.arange(S * GD, dtype=np.float32)
    q = (np.sin(i * np.float32(0.031)) * np.float32(0.12)).astype(np.float32).reshape(S, GD)
    i = np.arange(S * KD, dtype=np.float32)
    k = (np.cos(i * np.float32(0.017)) * np.float32(0.12)).astype(np.float32).reshape(S, KD)
    v = np.sin(i * np.float32(0.007)).astype(np.float32).reshape(S, KD)
    return q, k, v


def _attention_f64(q, k, v, H, KV, D):
    S = q.shape[0]
    out = np.zeros((S, H * D))
    for h in range(H):
        kv = h // (H // KV)
        s = q[:, h * D:(h + 1) * D].astype(np.float64) @ k[:, kv * D:(kv + 1) * D].astype(np.float64).T
        p = np.exp(s - s.max(1, keepdims=True))
        out[:, h * D:(h + 1) * D] = (p / p.sum(1, keepdims=True)) @ v[:, kv * D:(kv + 1) * D]
    return out


def test_attention_i8_oracle_within_reference_bar(oracle, rng):
    """The int8 attention restatement (text.c:638-700) against a float64 brute force within the
    reference's own bar for its int8 path, 2e-2 (test_text_attention.c:69-71), on the reference
    test's inputs and on random ones, at lengths with partial 128-key blocks. A mistake in the
    quantization points (a dropped scale, a transposed operand, the wrong softmax axis) is far
    outside it."""
    H, KV, D = 3, 1, 256
    for S in (128, 197, 300):
        q, k, v = _ref_test_inputs(S, H, KV, D)
        got = oracle.attention_i8(q, k, v, H, KV, D)
        assert np.abs(got - _attention_f64(q, k, v, H, KV, D)).max() < 2e-2
    H, KV = 4, 2
    q = (rng.standard_normal((150, H * D)) * 0.1).astype(np.float32)
    k = (rng.standard_normal((150, KV * D)) * 0.1).astype(np.float32)
    v = rng.standard_normal((150, KV * D)).astype(np.float32)
    assert np.abs(oracle.attention_i8(q, k, v, H, KV, D) - _attention_f64(q, k, v, H, KV, D)).max() < 2e-2
    # peaked attention (logit std ~2): per-(row, head) cosine with float64 >= 0.999, while
    # normalizing over the query axis instead of the key axis drops it below 0.9
    q = (rng.standard_normal((150, H * D)) * 0.35).astype(np.float32)
    k = (rng.standard_normal((150, KV * D)) * 0.35).astype(np.float32)
    want = _attention_f64(q, k, v, H, KV, D)
    got = oracle.attention_i8(q, k, v, H, KV, D)
    bad = np.zeros_like(want)
    for h in range(H):
        kv = h // (H // KV)
        sc = q[:, h * D:(h + 1) * D].astype(np.float64) @ k[:, kv * D:(kv + 1) * D].astype(np.float64).T
        pb = np.exp(sc - sc.max(0, keepdims=True))
        bad[:, h * D:(h + 1) * D] = (pb / pb.sum(0, keepdims=True)) @ v[:, kv * D:(kv + 1) * D]

    def cos(a, b):
        a, b = a.reshape(-1, D), b.reshape(-1, D)
        return (a * b).sum(1) / (np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1))
    assert cos(got, want).min() >= 0.999 and cos(bad, want).min() < 0.9


def _q_f32(x):
    """The reference quantizer's arithmetic for one block/row (int8.c:41-42, kernels_i8_avx512_vnni.c:
    321-363 as compiled): scale amax * RN(1/127), bytes rne(x * RN(127 / amax))."""
    amax = np.float32(np.abs(x).max())
    inv127 = np.frombuffer(np.uint32(0x3C010204).tobytes(), np.float32)[0]
    sc = np.float32(amax * inv127) if amax > 0 else np.float32(1)
    inv = np.float32(np.float32(127) / amax) if amax > 0 else np.float32(1)
    return np.rint((x * inv).astype(np.float32)).astype(np.int32), sc


def test_attention_i8_oracle_uniform_closed_form(oracle, rng):
    """K = 0: every score is 0, the softmax is uniform (p = RN(1/S) on every key), each 128-key block
    of P quantizes to 127 with scale RN(p RN(1/127)), and ctx[d] = sum over key blocks (in order) of
    fma(127 * sum_j v8[j][d], RN(ps * vs[d]), .), with V^T quantized per dim over the sequence."""
    H, KV, D = 3, 1, 256
    for S in (128, 200):
        q = rng.standard_normal((S, H * D)).astype(np.float32)
        k = np.zeros((S, KV * D), np.float32)
        v = rng.standard_normal((S, KV * D)).astype(np.float32)
        got = oracle.attention_i8(q, k, v, H, KV, D).astype(np.float64)
        p = np.float32(np.float32(1) / np.float32(S))
        qp, ps = _q_f32(np.full(128, p, np.float32))
        assert np.all(qp == 127)
        want = np.zeros(D)
        for d in range(D):
            v8, vs = _q_f32(v[:, d])
            f = 0.0
            for b0 in range(0, S, 128):
                acc = 127 * int(v8[b0:b0 + 128].sum())
                f = float(np.float32(acc * float(np.float32(ps * vs)) + f))
            want[d] = f
        for h in range(H):
            assert np.allclose(got[:, h * D:(h + 1) * D], want[None, :], rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("K,block", [(768, 128), (768, 768), (1152, 1152), (1152, 128)])
def test_threaded_gemm_equals_scalar_fold(oracle, rng, K, block):
    """The oracle's threaded VNNI GEMM (the every-row checker at M = 65536) gives the scalar
    restatement's bits for blocks of 128 and for one block per row, partial row and column tiles
    included."""
    M, N = 37, 200
    qa = rng.integers(-127, 128, (M, K), dtype=np.int8)
    as_ = rng.uniform(0.001, 0.05, (M, K // block)).astype(np.float32)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    ws = rng.uniform(0.001, 0.02, N).astype(np.float32)
    a = oracle.i8_gemm(qa, as_, w, ws, block=block)
    b = oracle.i8_gemm_mt(qa, as_, w, ws, block=block, nthreads=4)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
