"""Oracle functions pinned by mathematics (closed forms and double-precision evaluation)."""
import numpy as np


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
