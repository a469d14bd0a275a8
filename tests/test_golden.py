"""The oracle and the HIP path against golden vectors written by the reference's own kernels.

tests/golden/vectors.npz holds outputs of the reference's quantizer (AVX-512, AVX-VNNI and scalar
builds), weight quantizer, AVX-512 and scalar int8 GEMMs and fp32 helpers, compiled from its
sources (tests/golden/make_golden.py). Inputs are regenerated here from the seeds in
tests/golden/gen.py. These tests need neither the reference tree nor oracle/_ref, so they run on
any host; the `gpu` ones check the device path against the same vectors.

Bars: bytes, scales and f32 GEMM outputs bit-exact; fp32 helpers within the tolerances the
reference itself builds them to (rcp/rsqrt approximations: tests/test_softmax.c:33,52).
"""
import os
import sys

import numpy as np
import pytest

from conftest import assert_f32_close

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, HERE)
import gen  # noqa: E402


@pytest.fixture(scope="module")
def golden():
    with np.load(os.path.join(HERE, "vectors.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="module")
def c1():
    return gen.c1_inputs()


@pytest.fixture(scope="module")
def c5():
    return gen.c5_inputs()


def _same_bits(a, b):
    return np.array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8))


def test_inputs_regenerate(golden, c1, c5):
    """The seeded inputs are the ones the vectors were written for (no drift in gen.py)."""
    assert list(golden["c1_in"]) == [gen.digest(c1[k]) for k in ("a", "w", "ws", "bias")]
    assert list(golden["c5_in"]) == [gen.digest(c5[k]) for k in ("a", "w", "ws")]
    assert str(golden["edge_in"]) == gen.digest(gen.edge_activations())
    assert str(golden["wq_in"]) == gen.digest(gen.weight_inputs())
    f = gen.fp32_inputs()
    assert list(golden["fp_in"]) == [gen.digest(f[k]) for k in sorted(f)]


# ------------------------------------------------------------------------- oracle (CPU)
def test_oracle_quantizer(oracle, golden, c1, c5):
    q, s = oracle.quantize(c1["a"])
    assert gen.digest(q) == str(golden["c1_q_digest"]), np.argwhere(q[:4] != golden["c1_q_head"])[:5]
    assert _same_bits(s, golden["c1_s"])
    q, s = oracle.quantize(c5["a"])
    assert gen.digest(q) == str(golden["c5_q_digest"])
    assert _same_bits(s, golden["c5_s"])
    q, s = oracle.quantize(gen.edge_activations())
    assert np.array_equal(q, golden["edge_q"])
    assert _same_bits(s, golden["edge_s"])


def test_oracle_weight_quantizer(oracle, golden):
    wq, sc, bsq = oracle.q8w_from_f32(gen.weight_inputs())
    assert _same_bits(wq, golden["wq_w"])
    assert _same_bits(sc, golden["wq_scale"])
    assert _same_bits(bsq, golden["wq_bsq"])


@pytest.mark.parametrize("case", ["c1", "c5"])
def test_oracle_gemm(oracle, golden, c1, c5, case):
    d = c1 if case == "c1" else c5
    q, s = oracle.quantize(d["a"])
    y = oracle.i8_gemm(q, s, d["w"], d["ws"])
    head = golden[f"{case}_y_head"]
    assert _same_bits(y[: head.shape[0]], head)
    assert gen.digest(y) == str(golden[f"{case}_y_digest"])
    if case == "c1":
        ys = oracle.i8_gemm_scalar(q, s, d["w"], d["ws"])
        assert _same_bits(ys[:4], golden["c1_yscalar_head"])
        assert gen.digest(ys) == str(golden["c1_yscalar_digest"])


def test_oracle_fp32_helpers(oracle, golden):
    f = gen.fp32_inputs()
    eps = float(f["eps"])
    assert_f32_close(oracle.rmsnorm(f["x"], f["gamma"], eps), golden["fp_rmsnorm"], rtol=2e-6,
                     what="rmsnorm")
    ox, ores = oracle.norm_split(f["x"], f["gamma"], eps)
    assert_f32_close(ox, golden["fp_norm_split"], rtol=2e-6, what="norm_split")
    assert np.array_equal(ores, f["x"])
    assert_f32_close(oracle.norm_add(f["src"], f["x"], f["gamma"], eps), golden["fp_norm_add"],
                     rtol=2e-6, atol=1e-5, what="norm_add")
    og = np.array([oracle.lib.or_gelu_tanh(float(t)) for t in f["gelu_x"]], np.float32)
    assert np.max(np.abs(og - golden["fp_gelu"])) < 3e-6 * 12
    # both float softmaxes are within 3e-7 of exact (test_softmax.c:33), so within 2x of each other
    assert np.max(np.abs(oracle.softmax(f["soft_x"]) - golden["fp_softmax"])) < 2 * 4 * 3e-7
    assert_f32_close(oracle.meanpool_l2(f["pool_x"], f["pool_valid"]), golden["fp_pool"],
                     rtol=1e-6, atol=1e-7, what="pool")


# ---------------------------------------------------------------------------- HIP path
def _dev(a, gpu):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


@pytest.mark.gpu
def test_gpu_quantizer_golden(gpu, golden, c1, c5):
    import e2mi
    for x, qkey, skey in ((c1["a"], "c1_q_digest", "c1_s"), (c5["a"], "c5_q_digest", "c5_s")):
        q, s = e2mi.quantize(_dev(x, gpu))
        assert gen.digest(q.cpu().numpy()) == str(golden[qkey])
        assert _same_bits(s.cpu().numpy(), golden[skey])
    q, s = e2mi.quantize(_dev(gen.edge_activations(), gpu))
    assert np.array_equal(q.cpu().numpy(), golden["edge_q"])
    assert _same_bits(s.cpu().numpy(), golden["edge_s"])


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["c1", "c5"])
def test_gpu_gemm_golden(gpu, golden, c1, c5, case):
    """Device quantizer + f32-epilogue GEMM on the packed (reference-layout) weights, bit-exact with
    the reference's AVX-512 kernel."""
    import e2mi
    d = c1 if case == "c1" else c5
    wq, _ = gen.pack_q8w(d["w"])
    N, K = d["w"].shape
    w = e2mi.DeviceWeight.from_packed(wq, d["ws"], N, K)
    q, s = e2mi.quantize(_dev(d["a"], gpu))
    y = e2mi.i8_gemm(q, s, w).cpu().numpy()
    head = golden[f"{case}_y_head"]
    assert _same_bits(y[: head.shape[0]], head)
    assert gen.digest(y) == str(golden[f"{case}_y_digest"])
