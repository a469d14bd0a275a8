// weights.hip — device weight upload and the quad-interleaved -> row-major re-layout.
//
// The reference stores int8 weights as [Npad/8][K/4][8][4] (src/int8.h:14-22): one 32-byte vector
// holds a k-quad of 8 output rows, the shape vpdpbusd wants. MFMA fragments want each output row's
// K bytes contiguous, so the packed blob (from the reference's loader or an E8CQ cache blob,
// q8cache.c:163-181) is uploaded once and re-laid out on the device: one thread per k-quad, a
// 4-byte gather from the packed blob and a 4-byte store into the row-major copy.
#include <stdlib.h>
#include <string.h>

#include "common.h"
#include "model_internal.h"

namespace e2mi {

// row n of the packed blob lands in destination row (n / grp) * gstride + goff + n % grp: the
// identity for a plain upload, an offset for q|k|v concatenation, and the per-32 gate|up
// interleave the GeGLU epilogue reads
__global__ void k_unpack_quads(int8_t *__restrict__ dst, int ld, const int8_t *__restrict__ src,
                               int N, int K, int grp, int gstride, int goff, int pair_order) {
    const int kq_n = (K + 3) / 4;
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long)N * kq_n) return;
    const int n = (int)(i / kq_n), kq = (int)(i % kq_n);
    const uint32_t v = *(const uint32_t *)(src + ((size_t)(n >> 3) * kq_n + kq) * 32 + (n & 7) * 4);
    size_t row = (size_t)(n / grp) * gstride + goff + n % grp;
    if (pair_order) row = (row & ~(size_t)0xC0) | ((row & 0x40) << 1) | ((row & 0x80) >> 1);
    *(uint32_t *)(dst + row * ld + kq * 4) = v;
}

int upload_packed_rows(int8_t *dst, int ld, const int8_t *wq, int N, int K, int grp, int gstride,
                       int goff, hipStream_t s, bool pair_order) {
    const size_t bytes = (size_t)((N + 7) / 8) * ((K + 3) / 4) * 32;
    int8_t *staging = nullptr;
    if (check_hip(hipMalloc(&staging, bytes), "hipMalloc staging")) return -1;
    int rc = check_hip(hipMemcpyAsync(staging, wq, bytes, hipMemcpyHostToDevice, s), "upload packed");
    if (!rc) {
        const long n = (long)N * ((K + 3) / 4);
        hipLaunchKernelGGL(k_unpack_quads, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, dst,
                           ld, staging, N, K, grp, gstride, goff, pair_order ? 1 : 0);
        rc = check_hip(hipGetLastError(), "unpack launch");
    }
    // the staging blob must outlive the kernel
    if (!rc) rc = check_hip(hipStreamSynchronize(s), "unpack sync");
    (void)hipFree(staging);
    return rc;
}

static int alloc_q8w(e2mi_q8w *out, int N, int K, const float *scale, const float *bias,
                     hipStream_t s) {
    memset(out, 0, sizeof *out);
    out->N = N;
    out->K = K;
    out->ld = (K + 15) & ~15;
    out->out_min = -1e31f;
    out->out_max = 1e31f;
    E2MI_HIP(hipMalloc(&out->w, (size_t)N * out->ld));
    if (check_hip(hipMalloc(&out->scale, sizeof(float) * N), "hipMalloc scale")) {
        (void)hipFree(out->w);
        memset(out, 0, sizeof *out);
        return -1;
    }
    if (bias && check_hip(hipMalloc(&out->bias, sizeof(float) * N), "hipMalloc bias")) {
        (void)hipFree(out->w);
        (void)hipFree(out->scale);
        memset(out, 0, sizeof *out);
        return -1;
    }
    if (check_hip(hipMemcpyAsync(out->scale, scale, sizeof(float) * N, hipMemcpyHostToDevice, s),
                  "upload scale") ||
        (bias && check_hip(hipMemcpyAsync(out->bias, bias, sizeof(float) * N,
                                          hipMemcpyHostToDevice, s),
                           "upload bias"))) {
        e2mi_q8w_free(out);
        return -1;
    }
    return 0;
}

static int check_dims(int N, int K, const void *w, const float *scale, const char *who) {
    if (!w || !scale || N <= 0 || K <= 0 || K % 128) {
        set_error("%s: need non-null weights/scales, N > 0 and K a positive multiple of 128 (N=%d K=%d)",
                  who, N, K);
        return -1;
    }
    return 0;
}

}  // namespace e2mi

using namespace e2mi;

extern "C" int e2mi_q8w_upload_packed(e2mi_q8w *out, const int8_t *wq, const float *scale,
                                      const float *bias, int N, int K, e2mi_stream stream) {
    if (!out || check_dims(N, K, wq, scale, "q8w_upload_packed")) return -1;
    hipStream_t s = (hipStream_t)stream;
    if (alloc_q8w(out, N, K, scale, bias, s)) return -1;
    const int rc = upload_packed_rows(out->w, out->ld, wq, N, K, N, 0, 0, s);
    if (rc) e2mi_q8w_free(out);
    return rc;
}

extern "C" int e2mi_q8w_upload_rowmajor(e2mi_q8w *out, const int8_t *w, const float *scale,
                                        const float *bias, int N, int K, e2mi_stream stream) {
    if (!out || check_dims(N, K, w, scale, "q8w_upload_rowmajor")) return -1;
    hipStream_t s = (hipStream_t)stream;
    if (alloc_q8w(out, N, K, scale, bias, s)) return -1;
    if (check_hip(hipMemcpy2DAsync(out->w, out->ld, w, K, K, N, hipMemcpyHostToDevice, s),
                  "upload weights") ||
        check_hip(hipStreamSynchronize(s), "upload sync")) {
        e2mi_q8w_free(out);
        return -1;
    }
    return 0;
}

extern "C" void e2mi_q8w_free(e2mi_q8w *w) {
    if (!w) return;
    if (w->w) (void)hipFree(w->w);
    if (w->scale) (void)hipFree(w->scale);
    if (w->bias) (void)hipFree(w->bias);
    memset(w, 0, sizeof *w);
}

extern "C" int e2mi_interleave_gate_up(int8_t *w_out, float *s_out, const int8_t *gate,
                                       const float *sgate, const int8_t *up, const float *sup,
                                       int F, int K) {
    if (!w_out || !s_out || !gate || !sgate || !up || !sup || F <= 0 || F % 128 || K <= 0) {
        set_error("interleave_gate_up: null pointer or F not a positive multiple of 128 (F=%d)", F);
        return -1;
    }
    for (int b = 0; b < F / 32; b++)
        for (int i = 0; i < 32; i++) {
            const int src = b * 32 + i;
            memcpy(w_out + (size_t)(b * 64 + i) * K, gate + (size_t)src * K, (size_t)K);
            memcpy(w_out + (size_t)(b * 64 + 32 + i) * K, up + (size_t)src * K, (size_t)K);
            s_out[b * 64 + i] = sgate[src];
            s_out[b * 64 + 32 + i] = sup[src];
        }
    return 0;
}
