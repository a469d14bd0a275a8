"""Write tests/golden/vectors.npz: outputs of the reference's own kernels on the seeded inputs of
tests/golden/gen.py.

The reference kernels come from oracle/_ref/libe2ref.so, which oracle/Makefile compiles from the
reference's sources (src/int8.c, src/kernels_i8_avx512_vnni.c, src/kernels_i8_vnni.c,
src/kernels.c, src/kernels_avx512.c ...) with the reference's own flags. Only data is written:
small arrays in full, large ones as sha256 digests plus their first rows. Re-run after changing
gen.py:

    make -C oracle ref && python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, HERE)

import gen  # noqa: E402
from oracle.binding import Ref  # noqa: E402


def main():
    ref = Ref()
    out = {}

    # quantizer + GEMM at BASELINE config 1 (and the scalar reference GEMM)
    c1 = gen.c1_inputs()
    out["c1_in"] = np.array([gen.digest(c1[k]) for k in ("a", "w", "ws", "bias")])
    q, s = ref.quantize(c1["a"], "avx512")
    for which in ("vnni", "scalar"):
        q2, s2 = ref.quantize(c1["a"], which)
        assert np.array_equal(q, q2) and np.array_equal(s.view(np.uint32), s2.view(np.uint32))
    out["c1_q_digest"] = np.array(gen.digest(q))
    out["c1_q_head"] = q[:4].copy()
    out["c1_s"] = s
    wq, bsq = gen.pack_q8w(c1["w"])
    N, K = c1["w"].shape
    y = ref.gemm(q, s, wq, c1["ws"], bsq, N, K, "avx512")
    out["c1_y_digest"] = np.array(gen.digest(y))
    out["c1_y_head"] = y[:4].copy()
    ys = ref.gemm(q, s, wq, c1["ws"], bsq, N, K, "scalar")
    out["c1_yscalar_digest"] = np.array(gen.digest(ys))
    out["c1_yscalar_head"] = ys[:4].copy()

    # a slice of the C5 sweep: heavy-tailed activations, K = 1152
    c5 = gen.c5_inputs()
    out["c5_in"] = np.array([gen.digest(c5[k]) for k in ("a", "w", "ws")])
    q, s = ref.quantize(c5["a"], "avx512")
    out["c5_q_digest"] = np.array(gen.digest(q))
    out["c5_s"] = s
    wq, bsq = gen.pack_q8w(c5["w"])
    N, K = c5["w"].shape
    y = ref.gemm(q, s, wq, c5["ws"], bsq, N, K, "avx512")
    out["c5_y_digest"] = np.array(gen.digest(y))
    out["c5_y_head"] = y[:2].copy()

    # quantizer special cases, all three builds of the reference quantizer
    xe = gen.edge_activations()
    out["edge_in"] = np.array(gen.digest(xe))
    q, s = ref.quantize(xe, "avx512")
    for which in ("vnni", "scalar"):
        q2, s2 = ref.quantize(xe, which)
        assert np.array_equal(q, q2) and np.array_equal(s.view(np.uint32), s2.view(np.uint32))
    out["edge_q"], out["edge_s"] = q, s

    # weight quantizer + packer (int8.c:19-88 as built)
    wf = gen.weight_inputs()
    out["wq_in"] = np.array(gen.digest(wf))
    out["wq_w"], out["wq_scale"], out["wq_bsq"] = ref.q8w_from_f32(wf)

    # fp32 helpers through the reference's kernel table (kernels.h:22-66, avx512 row)
    f = gen.fp32_inputs()
    out["fp_in"] = np.array([gen.digest(f[k]) for k in sorted(f)])
    k = ref.kernels()
    R, D = f["x"].shape
    eps = float(f["eps"])
    a = f["x"].copy()
    k.rmsnorm(a.ctypes.data, R, D, f["gamma"].ctypes.data, eps)
    out["fp_rmsnorm"] = a
    a, res = f["x"].copy(), np.empty_like(f["x"])
    k.norm_split(a.ctypes.data, res.ctypes.data, R, D, f["gamma"].ctypes.data, eps)
    out["fp_norm_split"] = a
    o = np.empty_like(f["x"])
    k.norm_add(o.ctypes.data, f["src"].ctypes.data, f["x"].ctypes.data, R, D,
               f["gamma"].ctypes.data, eps)
    out["fp_norm_add"] = o
    g = f["gelu_x"].copy()
    k.gelu_tanh(g.ctypes.data, g.size)
    out["fp_gelu"] = g
    sm = f["soft_x"].copy()
    k.softmax(sm.ctypes.data, sm.size)
    out["fp_softmax"] = sm
    out["fp_pool"] = ref.meanpool_l2(f["pool_x"], f["pool_valid"])

    dst = os.path.join(HERE, "vectors.npz")
    np.savez_compressed(dst, **out)
    print(f"wrote {dst} ({os.path.getsize(dst)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
