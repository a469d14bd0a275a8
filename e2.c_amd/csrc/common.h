// common.h — shared definitions of the gfx950 int8 encoder backend (device and host side).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/e2mi.h"

namespace e2mi {

// One activation/weight quantization block (reference src/int8.h:61-70, E2_I8_BLOCK).
constexpr int kQBlock = 128;

// RN(1/127): the constant the reference's amax/127.0f folds into under -freciprocal-math
// (kernels_i8_avx512_vnni.c:341 as compiled with CMakeLists.txt:110).
__host__ __device__ inline float inv127() { return __builtin_bit_cast(float, 0x3c010204u); }

// ---- error reporting (the e2_hip_last_error convention, reference src/gpu/hip/hip.c:27-49)
void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
int check_hip(hipError_t e, const char *what);
#define E2MI_HIP(call)                                                                     \
    do {                                                                                   \
        if (::e2mi::check_hip((call), #call)) return -1;                                   \
    } while (0)

inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// ---- the row count of a forward planned on the device (the engine's device entry): while the
// engine enqueues such a forward, the row kernels, the quantizer, the q/k/v norm kernel and the
// per-128 GEMMs launched from that thread read their row count from `ptr` (an int in device memory
// that the planner writes, times `mul`), and the host row count they are given only sizes their
// grids. Rows past the device count are never read by the rows before them, so the count prunes
// work only. `est` (> 0) is the host's estimate of that count, from which the GEMMs choose their
// tile shape (the same results either way). Unset (null) for every other launch.
struct DeviceRows {
    const int *ptr = nullptr;
    int mul = 1;
    int est = 0;
};
DeviceRows device_rows();
class DeviceRowsScope {
  public:
    DeviceRowsScope(const int *ptr, int mul = 1, int est = 0);
    ~DeviceRowsScope();
    DeviceRowsScope(const DeviceRowsScope &) = delete;
    DeviceRowsScope &operator=(const DeviceRowsScope &) = delete;

  private:
    DeviceRows prev_;
};

// compute units of the current device (256 on the MI355X), cached after the first query
int num_cus();

}  // namespace e2mi

// ---- device helpers
#if defined(__HIPCC__)
namespace e2mi {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// GELU-tanh (the GeGLU epilogues' gelu, text.c:424-468) through the identity
// 0.5 v (1 + tanh z) = v / (1 + e^(-2z)): one v_exp_f32 and one v_rcp_f32 (about 1 ulp) instead of
// the library tanhf and an IEEE division, with no cancellation for negative v (1 + tanh z is never
// formed); e^(-2z) -> inf gives exactly 0 (the reciprocal of inf is 0) and -> 0 gives v
__device__ inline float gelu_tanh(float v) {
    const float c = 0.7978845608028654f;
    const float z = c * (v + 0.044715f * v * v * v);
    return v * __builtin_amdgcn_rcpf(1.f + __expf(-2.f * z));
}

// The quantizer's per-block arithmetic: scale = amax * RN(1/127), inv = 127 / amax (correctly
// rounded division), q = rne(x * inv) saturated to [-128,127] like the SIMD pack.
struct QScale {
    float sc, inv;
};
__device__ inline QScale qscale(float amax) {
    QScale r;
    if (amax > 0.f) {
        r.sc = __fmul_rn(amax, inv127());
        r.inv = __fdiv_rn(127.0f, amax);
    } else {
        r.sc = 1.0f;
        r.inv = 1.0f;
    }
    return r;
}
__device__ inline int qbyte(float x, float inv) {
    float r = __builtin_rintf(__fmul_rn(x, inv));
    r = fminf(fmaxf(r, -128.f), 127.f);
    return (int)r;
}
// q = rne(x * inv) via the 1.5*2^23 trick: x*inv is rounded to f32 first (as the reference's
// mulps does), then adding 12582912 rounds it to an integer with ties to even; |x*inv| <= 127.00002
// for |x| <= amax, so the integer lands in [-127, 127] and is the low byte of the sum's bits.
__device__ inline uint32_t qbits(float x, float inv) {
    return __builtin_bit_cast(uint32_t, __fadd_rn(__fmul_rn(x, inv), 12582912.0f));
}
__device__ inline uint32_t pack4_magic(float a, float b, float c, float d, float inv) {
    const uint32_t lo = __builtin_amdgcn_perm(qbits(b, inv), qbits(a, inv), 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm(qbits(d, inv), qbits(c, inv), 0x0c0c0400u);
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}
__device__ inline uint32_t pack4(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
           ((uint32_t)(d & 0xff) << 24);
}

// The value of lane l ^ O (O a power of two below 64), by VALU operations only. Within a 16-lane
// row by DPP (xor 1 and 2 by quad permutes, 4 by the row shifts either way and a select, 8 by a
// rotation of the row by half); xor 16 and 32 by gfx950's lane swaps of a register with itself:
// v_permlane16_swap exchanges the odd 16-lane rows of its first operand with the even rows of its
// second, v_permlane32_swap the upper 32 lanes of the first with the lower 32 of the second, so the
// partner of a lane with bit O clear is in the second result and of one with it set in the first.
template <int O>
__device__ inline float xor_lane(float v) {
    const int x = __builtin_bit_cast(int, v);
    int r;
    if constexpr (O == 1) {
        r = __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, true);  // quad_perm [1, 0, 3, 2]
    } else if constexpr (O == 2) {
        r = __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, true);  // quad_perm [2, 3, 0, 1]
    } else if constexpr (O == 4) {
        const int up = __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true);  // row_shr:4, lane - 4
        const int dn = __builtin_amdgcn_update_dpp(0, x, 0x104, 0xF, 0xF, true);  // row_shl:4, lane + 4
        r = (threadIdx.x & 4) ? up : dn;
    } else if constexpr (O == 8) {
        r = __builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, true);  // row_ror:8
    } else if constexpr (O == 16) {
        const auto p = __builtin_amdgcn_permlane16_swap(x, x, false, false);
        r = (threadIdx.x & 16) ? (int)p[0] : (int)p[1];
    } else {
        static_assert(O == 32, "xor of 1 .. 32");
        const auto p = __builtin_amdgcn_permlane32_swap(x, x, false, false);
        r = (threadIdx.x & 32) ? (int)p[0] : (int)p[1];
    }
    return __builtin_bit_cast(float, r);
}
template <int O, int W>
__device__ inline float xor_max(float v) {
    if constexpr (O == 0) return v;
    else return xor_max<O / 2, W>(fmaxf(v, xor_lane<O>(v)));
}
template <int O, int W>
__device__ inline float xor_sum(float v) {
    if constexpr (O == 0) return v;
    else return xor_sum<O / 2, W>(v + xor_lane<O>(v));
}
// max / sum over the 2^k lanes of a lane group (width <= 64) by the xor butterfly, partners W/2
// apart first; every lane gets the same result (each step's two operands commute)
template <int W>
__device__ inline float group_max(float v) {
    return xor_max<W / 2, W>(v);
}
template <int W>
__device__ inline float group_sum(float v) {
    return xor_sum<W / 2, W>(v);
}

// Workgroups are dispatched round-robin over the 8 XCDs; remap so each XCD walks a contiguous
// range of logical tiles (consecutive N tiles of one M block share that XCD's L2).
__device__ inline int xcd_swizzle(int pid, int total) {
    constexpr int kXcd = 8;
    if (total % kXcd) return pid;
    return (pid % kXcd) * (total / kXcd) + pid / kXcd;
}

// The same direct-to-LDS loads as inline assembly, for the pipelined kernels (GEMM, attention). The compiler's
// wait-count pass cannot tell which LDS bytes a builtin direct-to-LDS load writes, so after one it
// waits for all of them (s_waitcnt vmcnt(0)) before the next LDS read, draining a multi-stage load
// pipeline every K step. Loads issued here are invisible to that pass: the kernel orders them
// itself (explicit vmcnt waits + barriers), and issues no other vector-memory load the compiler
// would wait for inside the loop. M0 carries the LDS destination (no other code in the kernel uses
// M0); one wait state separates its write from the load.
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
__device__ inline v4u rsrc_words(const void *base, uint32_t bytes) {
    const uint64_t a = (uint64_t)base;
    v4u r;
    r.x = __builtin_amdgcn_readfirstlane((uint32_t)a);
    r.y = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32) & 0xffffu);
    r.z = __builtin_amdgcn_readfirstlane(bytes);
    r.w = 0x00020000u;
    return r;
}
__device__ inline void dma16(v4u r, uint32_t lds, uint32_t voff, uint32_t soff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 ::"s"(lds), "v"(voff), "s"(r), "s"(soff)
                 : "memory");
}
__device__ inline void dma4(v4u r, uint32_t lds, uint32_t voff, uint32_t soff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, %3 offen lds"
                 ::"s"(lds), "v"(voff), "s"(r), "s"(soff)
                 : "memory");
}

}  // namespace e2mi
#endif
