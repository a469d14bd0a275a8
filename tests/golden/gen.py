"""Deterministic, platform-independent inputs for the golden vectors.

Everything derives from the reference's LCG `s = s*1664525 + 1013904223 (mod 2^32)`
(tests/test_scalar_kernels.c:26-28, tools/kernel_bench.c:33-38) using only integer arithmetic and
correctly rounded IEEE operations (+, *, /, sqrt), so the same seed gives the same bytes on any
host: no libm transcendental is involved. Normals are Irwin-Hall sums of four uniforms (mean 0,
variance 1), which is what the configs' N(0, s) draws are approximated by here.
"""
import hashlib

import numpy as np

_A, _C, _M32 = 1664525, 1013904223, 0xFFFFFFFF


def lcg_u32(seed, n):
    """The first n outputs s_1..s_n of the LCG started at s_0 = seed (vectorised jump-ahead)."""
    n = int(n)
    out = np.empty(n, np.uint64)
    blk = 1024
    s = int(seed) & _M32
    first = np.empty(min(blk, n), np.uint64)
    for i in range(first.size):
        s = (s * _A + _C) & _M32
        first[i] = s
    out[: first.size] = first
    if n <= blk:
        return out.astype(np.uint32)
    # s_{i+blk} = Ab * s_i + Cb (mod 2^32)
    Ab, Cb = 1, 0
    for _ in range(blk):
        Ab, Cb = (Ab * _A) & _M32, (Cb * _A + _C) & _M32
    Ab, Cb = np.uint64(Ab), np.uint64(Cb)
    mask = np.uint64(_M32)
    for off in range(blk, n, blk):
        m = min(blk, n - off)
        out[off: off + m] = (out[off - blk: off - blk + m] * Ab + Cb) & mask
    return out.astype(np.uint32)


def uniform(seed, n):
    """U[0,1) in float64 with 24 random bits (exact)."""
    return (lcg_u32(seed, n) >> np.uint32(8)).astype(np.float64) * (1.0 / 16777216.0)


def normal(seed, shape, std=1.0, mean=0.0):
    n = int(np.prod(shape))
    u = uniform(seed, 4 * n).reshape(n, 4)
    z = (((u[:, 0] + u[:, 1]) + (u[:, 2] + u[:, 3])) - 2.0) * np.sqrt(3.0)
    return (z * std + mean).astype(np.float32).reshape(shape)


def int8_uniform(seed, shape):
    """Uniform over [-127, 127] (the configs' weight bytes)."""
    n = int(np.prod(shape))
    v = ((lcg_u32(seed, n) >> np.uint32(8)) % np.uint32(255)).astype(np.int16) - 127
    return v.astype(np.int8).reshape(shape)


def scales(seed, n, lo=0.001, hi=0.02):
    return (lo + (hi - lo) * uniform(seed, n)).astype(np.float32)


def student_t3(seed, shape, outlier_frac=0.001, outlier_scale=50.0):
    """Student-t(nu=3) = z / sqrt(chi2_3 / 3), with ceil(frac*K) seeded channels scaled x50."""
    M, K = shape
    z = normal(seed, (M, K)).astype(np.float64)
    c = normal(seed + 1, (M, K, 3)).astype(np.float64)
    chi = (c * c).sum(-1) / 3.0
    x = z / np.sqrt(np.maximum(chi, 1e-6))
    n_out = int(np.ceil(outlier_frac * K))
    cols = (lcg_u32(seed + 2, n_out) % np.uint32(K)).astype(np.int64)
    x[:, cols] *= outlier_scale
    return x.astype(np.float32)


def edge_activations(M=9, K=256):
    """Rows that exercise the quantizer's special cases: an all-zero row (scale 1, bytes 0), a zero
    block, exact rounding ties, a single huge element, denormal-sized values and a negative-only
    block."""
    x = normal(77, (M, K), std=2.0)
    x[0] = 0.0
    x[1, :128] = 0.0
    x[2, :128] = np.arange(128, dtype=np.float32) - 63.5
    x[3, 5] = 3.0e4
    x[4, 128:] = 1.0e-30
    x[5, :128] = -np.abs(x[5, :128])
    x[6] = np.float32(127.0) * (np.arange(K) % 3 - 1)
    return x


def digest(a):
    """sha256 of an array's bytes (dtype and shape fixed by the caller)."""
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def pack_q8w(w):
    """The reference's quad-interleaved layout (src/int8.h:14-22) and per-block row sums
    (src/int8.c:57-61), written from the closed form."""
    N, K = w.shape
    Npad, kq = (N + 7) & ~7, K // 4
    wp = np.zeros((Npad, K), np.int8)
    wp[:N] = w
    # [Npad/8][K/4][8][4]
    wq = wp.reshape(Npad // 8, 8, kq, 4).transpose(0, 2, 1, 3).reshape(-1).copy()
    bsq = wp.reshape(Npad, K // 128, 128).astype(np.int32).sum(-1).T.copy()
    return wq, bsq


# ----------------------------------------------------------------------------- the cases
def c1_inputs():
    """A [128 x 768] ~N(0,1), W int8 [1152 x 768], ws ~U(0.001,0.02),
    bias ~N(0,0.01)."""
    return {
        "a": normal(1001, (128, 768)),
        "w": int8_uniform(1002, (1152, 768)),
        "ws": scales(1003, 1152),
        "bias": normal(1004, (1152,), std=0.01),
    }


def c5_inputs(K=1152, N=768, M=64):
    """A slice of the C5 sweep's operands: Student-t activations with an outlier channel."""
    return {
        "a": student_t3(5001, (M, K)),
        "w": int8_uniform(5002, (N, K)),
        "ws": scales(5003, N),
    }


def weight_inputs(N=40, K=256):
    """f32 weights for the weight quantizer (int8.c:19-88), one zero row."""
    w = normal(3001, (N, K)) * (0.001 + uniform(3002, N).astype(np.float32)[:, None])
    w[0] = 0.0
    return w.astype(np.float32)


def fp32_inputs():
    R, D = 4, 768
    return {
        "x": normal(4001, (R, D), std=3.0),
        "src": normal(4002, (R, D)),
        "gamma": normal(4003, (D,), std=0.05, mean=1.0),
        "gelu_x": np.linspace(-12, 12, 2048).astype(np.float32),
        "soft_x": normal(4004, (513,), std=8.0),
        "pool_x": normal(4005, (50, 768)),
        "pool_valid": (uniform(4006, 50) > 0.3).astype(np.uint8),
        "eps": np.float32(1e-6),
    }
