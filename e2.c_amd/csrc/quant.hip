// quant.hip — per-(row, 128-block) symmetric int8 activation quantizer for gfx950.
//
// Same contract as the reference's e2_i8_quantize (src/kernels.h:70-72; arithmetic of
// src/kernels_i8_avx512_vnni.c:312-366 as compiled): per block amax, scale = amax*RN(1/127),
// inv = 127/amax, q = rne(x*inv). Bytes are stored signed (include/e2hip.h:19-21), scales in the
// reference's [M][nb] layout. HBM-bound: each 128-element block is one half-wave's float4 loads,
// a 5-step xor-shuffle max, and one 4-byte store per lane.
#include "common.h"

namespace e2mi {

// block == 128: a half-wave per (row, block); 8 blocks per 256-thread workgroup.
__global__ __launch_bounds__(256) void k_quant128(int8_t *__restrict__ q, float *__restrict__ sc,
                                                  const float *__restrict__ x, int M, int K,
                                                  int ldx, int ldq, const int *rows) {
    const int nb = K / kQBlock;
    const long item = (long)blockIdx.x * 8 + (threadIdx.x >> 5);
    if (item >= (long)M * nb) return;
    const int m = (int)(item / nb), b = (int)(item % nb), l = threadIdx.x & 31;
    if (rows && m >= *rows) return;
    const float4 v = *(const float4 *)(x + (size_t)m * ldx + b * kQBlock + l * 4);
    float a = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    a = group_max<32>(a);
    const QScale s = qscale(a);
    *(uint32_t *)(q + (size_t)m * ldq + b * kQBlock + l * 4) =
        pack4(qbyte(v.x, s.inv), qbyte(v.y, s.inv), qbyte(v.z, s.inv), qbyte(v.w, s.inv));
    if (l == 0) sc[(size_t)m * nb + b] = s.sc;
}

// block == K (the per-token variant, the reference rebuilt with -DE2_I8_BLOCK=K): one wave per row.
__global__ __launch_bounds__(256) void k_quant_row(int8_t *__restrict__ q, float *__restrict__ sc,
                                                   const float *__restrict__ x, int M, int K,
                                                   int ldx, int ldq, const int *rows) {
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
    if (m >= M || (rows && m >= *rows)) return;
    const float *xr = x + (size_t)m * ldx;
    float a = 0.f;
    for (int k = l * 4; k < K; k += 256) {
        const float4 v = *(const float4 *)(xr + k);
        a = fmaxf(a, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    a = group_max<64>(a);
    const QScale s = qscale(a);
    for (int k = l * 4; k < K; k += 256) {
        const float4 v = *(const float4 *)(xr + k);
        *(uint32_t *)(q + (size_t)m * ldq + k) =
            pack4(qbyte(v.x, s.inv), qbyte(v.y, s.inv), qbyte(v.z, s.inv), qbyte(v.w, s.inv));
    }
    if (l == 0) sc[m] = s.sc;
}

// per-128 blocks with one wave per row (K <= 256 NCH): chunk i of lane l holds elements
// 4 (l + 64 i) .. + 3, i.e. block 2 i + l / 32, so each block's maximum is one half-wave reduction;
// 16-byte loads, 4-byte stores of whole 128-byte block rows per half-wave
template <int NCH>
__global__ __launch_bounds__(256) void k_quant128_r(int8_t *__restrict__ q, float *__restrict__ sc,
                                                    const float *__restrict__ x, int M, int K,
                                                    int ldx, int ldq, const int *rows) {
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
    if (m >= M || (rows && m >= *rows)) return;
    const float *xr = x + (size_t)m * ldx;
    const int nb = K / kQBlock;
    float4 v[NCH];
#pragma unroll
    for (int i = 0; i < NCH; i++) {
        const int k = l * 4 + 256 * i;
        v[i] = k < K ? *(const float4 *)(xr + k) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int i = 0; i < NCH; i++) {
        const int k = l * 4 + 256 * i;
        float a = fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w)));
        a = group_max<32>(a);
        if (k < K) {
            const QScale s = qscale(a);
            *(uint32_t *)(q + (size_t)m * ldq + k) =
                pack4(qbyte(v[i].x, s.inv), qbyte(v[i].y, s.inv), qbyte(v[i].z, s.inv), qbyte(v[i].w, s.inv));
            if ((l & 31) == 0) sc[(size_t)m * nb + 2 * i + (l >> 5)] = s.sc;
        }
    }
}

// the same with the row held in registers (K <= 256 NCH): one read of x instead of two
template <int NCH>
__global__ __launch_bounds__(256) void k_quant_row_r(int8_t *__restrict__ q, float *__restrict__ sc,
                                                     const float *__restrict__ x, int M, int K,
                                                     int ldx, int ldq, const int *rows) {
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
    if (m >= M || (rows && m >= *rows)) return;
    const float *xr = x + (size_t)m * ldx;
    float4 v[NCH];
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < NCH; i++) {
        const int k = l * 4 + 256 * i;
        v[i] = k < K ? *(const float4 *)(xr + k) : make_float4(0.f, 0.f, 0.f, 0.f);
        a = fmaxf(a, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    }
    a = group_max<64>(a);
    const QScale s = qscale(a);
#pragma unroll
    for (int i = 0; i < NCH; i++) {
        const int k = l * 4 + 256 * i;
        if (k < K)
            *(uint32_t *)(q + (size_t)m * ldq + k) =
                pack4(qbyte(v[i].x, s.inv), qbyte(v[i].y, s.inv), qbyte(v[i].z, s.inv), qbyte(v[i].w, s.inv));
    }
    if (l == 0) sc[m] = s.sc;
}

int launch_quantize(hipStream_t s, int8_t *q, int ldq, float *scales, const float *x, int M,
                    int K, int ldx, int block) {
    if (M <= 0 || K <= 0 || K % 128 || ldx < K || ldq < K || ldx % 4 || ldq % 4) {
        set_error("quantize: bad geometry M=%d K=%d ldx=%d ldq=%d (K %% 128 == 0, ld >= K, ld %% 4 == 0)",
                  M, K, ldx, ldq);
        return -1;
    }
    if (!q || !scales || !x || !aligned16(x) || ((uintptr_t)q & 3)) {
        set_error("quantize: null or misaligned pointer (x 16-B, q 4-B aligned)");
        return -1;
    }
    const int *rows = device_rows().ptr;
    if (block == kQBlock) {
        const long items = (long)M * (K / kQBlock);
        const dim3 g((unsigned)((M + 3) / 4));
        if (K <= 768)
            hipLaunchKernelGGL(k_quant128_r<3>, g, dim3(256), 0, s, q, scales, x, M, K, ldx, ldq, rows);
        else if (K <= 1280)
            hipLaunchKernelGGL(k_quant128_r<5>, g, dim3(256), 0, s, q, scales, x, M, K, ldx, ldq, rows);
        else
            hipLaunchKernelGGL(k_quant128, dim3((unsigned)((items + 7) / 8)), dim3(256), 0, s, q,
                               scales, x, M, K, ldx, ldq, rows);
    } else if (block == K) {
        const dim3 g((unsigned)((M + 3) / 4));
        if (K <= 768)
            hipLaunchKernelGGL(k_quant_row_r<3>, g, dim3(256), 0, s, q, scales, x, M, K, ldx, ldq, rows);
        else if (K <= 1280)
            hipLaunchKernelGGL(k_quant_row_r<5>, g, dim3(256), 0, s, q, scales, x, M, K, ldx, ldq, rows);
        else
            hipLaunchKernelGGL(k_quant_row, g, dim3(256), 0, s, q, scales, x, M, K, ldx, ldq, rows);
    } else {
        set_error("quantize: block must be 128 or K (got %d, K=%d)", block, K);
        return -1;
    }
    return check_hip(hipGetLastError(), "quantize launch");
}

}  // namespace e2mi
