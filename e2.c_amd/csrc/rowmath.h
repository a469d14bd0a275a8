// rowmath.h — the per-row arithmetic of the RMSNorm family, shared by the row kernels (rowops.hip)
// and the GEMM whose epilogue runs the norm_add (gemm_an.hip), so both give the same bits.
//
// A row is held by one wave, lane l holding float4 chunks l, l + 64, ... (elements 4 (l + 64 i) ..
// + 3); sums of squares are taken per lane over its chunks in order, then over the wave.
#pragma once

#include "common.h"

namespace e2mi {

__device__ inline float4 ld4(const float *p) { return *(const float4 *)p; }
__device__ inline void st4(float *p, float4 v) { *(float4 *)p = v; }
__device__ inline float sumsq4(float4 v) { return v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w; }
__device__ inline float amax4(float4 v) {
    return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
}
// 1 / sqrt(ss / D + eps), every step correctly rounded (kernels.c:76-87)
__device__ inline float rms_inv(float ss, int D, float eps) {
    return __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, (float)D) + eps));
}
// (v * inv) * g, each product rounded
__device__ inline float4 scale4(float4 v, float inv, float4 g) {
    return make_float4(__fmul_rn(__fmul_rn(v.x, inv), g.x), __fmul_rn(__fmul_rn(v.y, inv), g.y),
                       __fmul_rn(__fmul_rn(v.z, inv), g.z), __fmul_rn(__fmul_rn(v.w, inv), g.w));
}

}  // namespace e2mi
