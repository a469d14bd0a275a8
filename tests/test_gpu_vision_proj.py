"""The vision tower's int8 projections (vision.c:985-1110) on the device GEMMs: per-128 activation
blocks (the text tower's E2_I8_BLOCK), P <= 2520 patches (model.h:27), hidden 768, MLP 3072
(model.h:20-25). Per layer: q|k|v 768 -> 3 x 768 from one quantization (vgemm3), o 768 -> 768,
gate|up 768 -> 2 x 3072 with gelu_tanh(gate) * up quantized per 128 (vgemm2 + vgelu_up_quant), down
3072 -> 768 from those bytes (vgemm_ready); the patch projection 768 -> 768 once per image.

Bars as for the text GEMMs: quantized bytes and f32 outputs bit-exact with the oracle (itself
bit-exact with the reference's e2_i8_gemm_avx512), the GeGLU stage within the reference's GELU bar
(test_gpu_ffn.c:104) with bytes exact for the kernel's own f32 values.
"""
import numpy as np
import pytest

from conftest import assert_f32_close

pytestmark = pytest.mark.gpu

P_MAX, D, INTER = 2520, 768, 3072


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _np(t):
    return t.cpu().numpy()


def _rows(rng, M):
    return np.unique(np.concatenate([np.arange(min(M, 40)), np.arange(max(0, M - 40), M), rng.integers(0, M, 128)]))


@pytest.mark.parametrize("P", [P_MAX, 577])
def test_vision_qkv_o_down_patch_bit_exact(gpu, oracle, rng, P):
    """The f32-output projections at the vision shapes: activations quantized per 128 on the device
    (bit-exact with the reference quantizer), then the GEMM, bit-exact on sampled rows."""
    import e2mi
    x = (rng.standard_normal((P, D)) * 2).astype(np.float32)
    q, s = e2mi.quantize(_t(x, gpu))
    rows = _rows(rng, P)
    qo, so = oracle.quantize(x[rows])
    assert np.array_equal(_np(q)[rows], qo) and np.array_equal(_np(s)[rows].view(np.uint32), so.view(np.uint32))
    for N, K in ((3 * D, D), (D, D), (D, INTER)):
        if K == D:
            qa, as_ = q, s
            qa_np, as_np = _np(q), _np(s)
        else:
            qa_np = rng.integers(-127, 128, (P, K), dtype=np.int8)
            as_np = rng.uniform(0.001, 0.05, (P, K // 128)).astype(np.float32)
            qa, as_ = _t(qa_np, gpu), _t(as_np, gpu)
        w = rng.integers(-127, 128, (N, K), dtype=np.int8)
        ws = rng.uniform(0.001, 0.02, N).astype(np.float32)
        W = e2mi.DeviceWeight.from_rowmajor(w, ws)
        y = _np(e2mi.i8_gemm(qa, as_, W))
        yo = oracle.i8_gemm(qa_np[rows], as_np[rows], w, ws)
        assert np.array_equal(y[rows].view(np.uint32), yo.view(np.uint32)), (N, K)


@pytest.mark.parametrize("P", [P_MAX, 300])
def test_vision_gate_up_geglu(gpu, oracle, rng, P):
    """gate|up 768 -> 2 x 3072 with the GeGLU epilogue (vision.c:1099-1103 + vgelu_up_quant)."""
    import e2mi
    qa = rng.integers(-127, 128, (P, D), dtype=np.int8)
    as_ = rng.uniform(0.001, 0.01, (P, D // 128)).astype(np.float32)
    wg = rng.integers(-127, 128, (INTER, D), dtype=np.int8)
    wu = rng.integers(-127, 128, (INTER, D), dtype=np.int8)
    sg = rng.uniform(0.001, 0.02, INTER).astype(np.float32)
    su = rng.uniform(0.001, 0.02, INTER).astype(np.float32)
    wi, si = e2mi.interleave_gate_up(wg, sg, wu, su)
    W = e2mi.DeviceWeight.from_rowmajor(wi, si)
    q, qs, g = e2mi.i8_gemm_geglu(_t(qa, gpu), _t(as_, gpu), W)
    rows = _rows(rng, P)
    gate = oracle.i8_gemm(qa[rows], as_[rows], wg, sg)
    up = oracle.i8_gemm(qa[rows], as_[rows], wu, su)
    go, _, _ = oracle.gelu_mul_quant(gate, up)
    gk = _np(g)[rows]
    assert_f32_close(gk, go, rtol=1e-4, atol=1e-4, what="gelu*up")
    qg, sgk = oracle.quantize(gk)
    assert np.array_equal(_np(q)[rows], qg)
    assert np.array_equal(_np(qs)[rows].view(np.uint32), sgk.view(np.uint32))
