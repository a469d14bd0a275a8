"""Fused f16-MFMA attention vs the oracle's row-wise fp32 attention (text.c:534-572).

The oracle gets the same f16-rounded q/k/v, so the comparison isolates the kernel's own
arithmetic (f16 probabilities in the PV product, exp approximation, summation order). Bars:
per-row cosine >= 0.9999 and max |err| <= 2e-3 * max |ctx|; the quantized
context is bit-exact for the kernel's own f32 context."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _np(t):
    return t.cpu().numpy()


def _case(rng, B, S, H, KV, D=256, lengths=None, holes=False):
    q = rng.standard_normal((B * S, H * D)).astype(np.float32)
    k = rng.standard_normal((B * S, KV * D)).astype(np.float32)
    v = rng.standard_normal((B * S, KV * D)).astype(np.float32)
    valid = np.ones(B * S, np.uint8)
    if lengths is not None:
        for b, L in enumerate(lengths):
            valid[b * S + L:(b + 1) * S] = 0
    if holes:
        valid[rng.random(B * S) < 0.1] = 0
    return q, k, v, valid


@pytest.mark.parametrize("B,S,lengths,holes,scale", [
    (2, 512, [512, 300], False, 1.0),     # config-3 geometry, trailing padding
    (3, 100, [100, 37, 1], False, 1.0),   # S not a multiple of the 32-key tile, a 1-token sequence
    (2, 77, None, True, 1.0),             # holes inside the sequence (the row-wise path)
    (2, 256, [256, 0], False, 1.0 / 16),  # an all-padding sequence, a flatter softmax
])
def test_attention_vs_oracle(gpu, oracle, rng, B, S, lengths, holes, scale):
    import e2mi
    import torch
    H, KV, D = 3, 1, 256
    q, k, v, valid = _case(rng, B, S, H, KV, D, lengths, holes)
    q16, k16, v16 = (_t(a, gpu).half() for a in (q, k, v))
    vt16 = v16.reshape(B, S, KV, D).permute(0, 2, 3, 1).contiguous()
    cq, cs, c32 = e2mi.attention(q16, k16, vt16, _t(valid, gpu), B, S, H, KV, scale=scale)
    got = _np(c32)
    qf, kf, vf = (_np(t.float()) for t in (q16, k16, v16))
    for b in range(B):
        r = slice(b * S, (b + 1) * S)
        want = oracle.attention(np.ascontiguousarray(qf[r]), np.ascontiguousarray(kf[r]),
                                np.ascontiguousarray(vf[r]), np.ascontiguousarray(valid[r]), H, KV, D,
                                scale=scale)
        g = got[r]
        vb = valid[r].astype(bool)
        assert np.all(g[~vb] == 0), "invalid query rows must have a zero context"
        if vb.any():
            gv, wv = g[vb].reshape(-1, D).astype(np.float64), want[vb].reshape(-1, D).astype(np.float64)
            cos = (gv * wv).sum(1) / (np.linalg.norm(gv, axis=1) * np.linalg.norm(wv, axis=1))
            assert cos.min() >= 0.9999, f"seq {b}: min row cosine {cos.min()}"
            assert np.abs(gv - wv).max() <= 2e-3 * np.abs(wv).max()
    qo, so = oracle.quantize(got)
    assert np.array_equal(_np(cq), qo) and np.array_equal(_np(cs), so)
