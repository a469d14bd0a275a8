// gemm.hip — W8A8 GEMM on gfx950 int8 MFMA (v_mfma_i32_32x32x32_i8) with the fused per-block
// dequantization of the reference's e2_i8_gemm (src/int8.h:94-97; fold order of
// src/kernels_i8_avx512_vnni.c:100-122):
//
//   y[m,n] = sum_b fma((float)acc_b[m,n], RN(as[m,b] * ws[n]), .)      acc_b exact int32
//
// then one of the fused epilogues:
//   EPI_F32   y (+bias), clamped to [lo,hi], stored f32 (the reference contract)
//   EPI_I8Q   y (+bias) requantized per (row, 128 output columns) for the next GEMM: int8 + scale
//   EPI_GEGLU W rows interleaved per 256 as [128 gate | 128 up]; g = gelu_tanh(gate) * up is
//             quantized per 128 (text.c:424-468 fused into the producing GEMM), g optionally kept
//
// Tiling: BM x BN workgroup tile of 64x64 wave tiles, K walked in 128-deep steps (one quantization
// block per step, so the int32 accumulators are folded into f32 once per step). A, W and the
// step's activation scales go HBM -> LDS with buffer loads that write LDS directly (no VGPR round
// trip), NS-1 steps ahead of the MFMAs; the fragment reads are conflict-free on the 64-bank LDS
// (see swz). Two kernels share the epilogues: k_gemm folds each step after its MFMAs, k_gemm_db
// double-buffers the int32 accumulators so one step's fold overlaps the next step's MFMAs.
#include <stdlib.h>
#include <type_traits>
#include <string.h>

#include "common.h"

namespace e2mi {

enum { EPI_F32 = 0, EPI_I8Q = 1, EPI_GEGLU = 2 };

struct GemmArgs {
    const int8_t *A;
    const float *as;
    const int8_t *W;
    const float *ws;
    const float *bias;
    float *Y;        // EPI_F32 output, EPI_GEGLU optional f32 g
    int8_t *Yq;      // EPI_I8Q / EPI_GEGLU quantized output
    float *ys;       // ... and its per-128 scales [M][ldys]
    int32_t *accd;   // optional int32 accumulator dump [nb][M][N] (parity tests)
    int lda, ldw, ldy, ldyq, ldys;
    int M, N, K;
    float lo, hi;
};


// GELU-tanh through the identity 0.5 v (1 + tanh z) = v / (1 + e^(-2z)): one v_exp_f32 and one
// reciprocal instead of the library tanhf, with no cancellation for negative v (1 + tanh z is never
// formed); e^(-2z) -> inf gives exactly 0 and -> 0 gives v
__device__ inline float gelu_tanh(float v) {
    const float c = 0.7978845608028654f;
    const float z = c * (v + 0.044715f * v * v * v);
    return __fdividef(v, 1.f + __expf(-2.f * z));
}

// LDS tiles hold 128-byte K slices of consecutive rows with no padding. The LDS has 64 banks of 4
// bytes and serves a ds_read_b128 16 lanes at a time; a 128-byte row spans 32 banks, so rows of
// equal parity share a bank half. The 16-byte chunk c of row r sits at slot c ^ ((r >> 1) & 7):
// the 16 consecutive rows read by one 16-lane group then cover all 64 banks once. Each
// 1-KB direct-to-LDS load fills 8 rows of a tile: lane l writes slot l, so it fetches row l/8's
// chunk (l % 8) ^ ((row >> 1) & 7).
__device__ inline int swzk(int r) { return (r >> 1) & 7; }
__device__ inline int swz(int r, int c) { return r * 128 + ((c ^ swzk(r)) << 4); }

typedef __attribute__((address_space(3))) void lds_void;

// Buffer loads straight into LDS: the per-lane offset is a VGPR fixed for the whole K loop and the
// K step's offset a scalar, so a step costs no VALU address arithmetic. (Device functions rather
// than lambdas: the builtin is only known to the device pass.)
__device__ inline void lds_load16(__amdgpu_buffer_rsrc_t r, void *lds, uint32_t voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds, 16, voff, soff, 0, 0);
}
__device__ inline void lds_load4(__amdgpu_buffer_rsrc_t r, void *lds, uint32_t voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds, 4, voff, soff, 0, 0);
}

// The fused epilogues over a finished BM x BN tile: f holds each wave's WM x WN f32 results in the
// MFMA C layout (lane column lane % 32, rows 8 (r / 4) + 4 (lane / 32) + r % 4 of each 32x32 tile).
// POST: bit 0 adds the bias, bit 1 clamps to [lo, hi] (compile-time, so the common case of
// neither costs no VALU work per element)
template <int BM, int BN, int WM, int WN, int LDSB, int EPI, bool FAST, int POST>
__device__ inline void store_tile_impl(const GemmArgs &p, float (&f)[WM / 32][WN / 32][16],
                                       const float (&wsr)[WN / 32], int m0, int n0, int wm, int wn,
                                       int tid, unsigned char *smem) {
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int NT = (BM / WM) * (BN / WN) * 64;
    const int lane = tid & 63;
    auto post = [&](float v, float b) {
        if constexpr (POST & 1) v = v + b;
        if constexpr (POST & 2) v = fminf(fmaxf(v, p.lo), p.hi);
        return v;
    };
    if constexpr (EPI == EPI_F32) {
        // buffer stores: the lane's byte offset is computed once, every (tile, register) row step
        // is a wave-uniform SGPR offset; rows past M fall outside the descriptor's range and are
        // dropped by the hardware, columns past N are masked per lane
        const __amdgpu_buffer_rsrc_t ry =
            __builtin_amdgcn_make_buffer_rsrc(p.Y, 0, (int)min((long)p.M * p.ldy * 4, 0x7fffffffL), 0x00020000);
        const int vrow = wm * WM + (lane >> 5) * 4, vcol = wn * WN + (lane & 31);
        const int voff = ((m0 + vrow) * p.ldy + n0 + vcol) * 4;
#pragma unroll
        for (int tn = 0; tn < TN; tn++) {
            const int n = n0 + vcol + tn * 32;
            if (n >= p.N) continue;
            const float b = (POST & 1) ? p.bias[n] : 0.f;
#pragma unroll
            for (int tm = 0; tm < TM; tm++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const float v = post(FAST ? __fmul_rn(f[tm][tn][r], wsr[tn]) : f[tm][tn][r], b);
                    const int srow = __builtin_amdgcn_readfirstlane((tm * 32 + (r >> 2) * 8 + (r & 3)) * p.ldy * 4);
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), ry,
                                                          voff + tn * 128, srow, 0);
                }
        }
    } else {
        // Stage the f32 tile through LDS (the A/W staging buffers are free now), then each group of
        // threads owns whole 128-column quantization blocks of a row.
        constexpr int FP = BN + 4;  // f32 row pitch
        static_assert(BM * FP * 4 <= LDSB, "epilogue tile does not fit");
        float *sf = (float *)smem;
        {
            float *sl = sf + (wm * WM + (lane >> 5) * 4) * FP + wn * WN + (lane & 31);
#pragma unroll
            for (int tn = 0; tn < TN; tn++) {
                const float b = (POST & 1) ? p.bias[min(n0 + wn * WN + tn * 32 + (lane & 31), p.N - 1)] : 0.f;
#pragma unroll
                for (int tm = 0; tm < TM; tm++)
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const float v = post(FAST ? __fmul_rn(f[tm][tn][r], wsr[tn]) : f[tm][tn][r], b);
                        sl[(tm * 32 + (r >> 2) * 8 + (r & 3)) * FP + tn * 32] = v;
                    }
            }
        }
        __syncthreads();
        // output columns per tile and per thread: I8Q keeps BN columns, GEGLU halves them
        constexpr int OUTC = (EPI == EPI_GEGLU) ? BN / 2 : BN;
        constexpr int TPR = OUTC / 16;  // threads per row, 16 columns each
        constexpr int RPP = NT / TPR;   // rows per pass
        static_assert(OUTC % 128 == 0 && TPR <= 64, "quantization block must be tile-local");
        const int oc0 = (EPI == EPI_GEGLU) ? n0 / 2 : n0;  // first output column of this tile
        const int ldo = (EPI == EPI_GEGLU) ? p.N / 2 : p.N;
        const int t_r = tid / TPR, t_c = tid % TPR;
        for (int rr = 0; rr < BM; rr += RPP) {
            const int ml = rr + t_r, m = m0 + ml;
            float v[16];
            if constexpr (EPI == EPI_GEGLU) {
                // W rows are interleaved per 256: [128 gate | 128 up] for each output block
                const int blk = (t_c * 16) >> 7, w = (t_c * 16) & 127;
                const float *gp = sf + ml * FP + blk * 256 + w;
#pragma unroll
                for (int i = 0; i < 16; i += 4) {
                    const float4 g = *(const float4 *)(gp + i), u = *(const float4 *)(gp + 128 + i);
                    v[i] = gelu_tanh(g.x) * u.x;
                    v[i + 1] = gelu_tanh(g.y) * u.y;
                    v[i + 2] = gelu_tanh(g.z) * u.z;
                    v[i + 3] = gelu_tanh(g.w) * u.w;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 16; i += 4) {
                    const float4 x = *(const float4 *)(sf + ml * FP + t_c * 16 + i);
                    v[i] = x.x;
                    v[i + 1] = x.y;
                    v[i + 2] = x.z;
                    v[i + 3] = x.w;
                }
            }
            float a = 0.f;
#pragma unroll
            for (int i = 0; i < 16; i++) a = fmaxf(a, fabsf(v[i]));
            a = group_max<8>(a);  // 8 threads x 16 columns = one 128-column block
            const QScale s = qscale(a);
            const int oc = oc0 + t_c * 16;
            if (m < p.M && oc < ldo) {
                uint32_t w4[4];
#pragma unroll
                for (int i = 0; i < 4; i++)
                    w4[i] = pack4_magic(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3], s.inv);
                *(uint4 *)(p.Yq + (size_t)m * p.ldyq + oc) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
                if ((t_c & 7) == 0) p.ys[(size_t)m * p.ldys + (oc >> 7)] = s.sc;
                if (EPI == EPI_GEGLU && p.Y) {
#pragma unroll
                    for (int i = 0; i < 16; i += 4)
                        *(float4 *)(p.Y + (size_t)m * p.ldy + oc + i) =
                            make_float4(v[i], v[i + 1], v[i + 2], v[i + 3]);
                }
            }
        }
    }
}

template <int BM, int BN, int WM, int WN, int LDSB, int EPI, bool FAST>
__device__ inline void store_tile(const GemmArgs &p, float (&f)[WM / 32][WN / 32][16],
                                  const float (&wsr)[WN / 32], int m0, int n0, int wm, int wn,
                                  int tid, unsigned char *smem) {
    const int post = (p.bias != nullptr ? 1 : 0) | ((p.lo > -1e30f || p.hi < 1e30f) ? 2 : 0);
    if (post == 0)
        store_tile_impl<BM, BN, WM, WN, LDSB, EPI, FAST, 0>(p, f, wsr, m0, n0, wm, wn, tid, smem);
    else if (post == 1)
        store_tile_impl<BM, BN, WM, WN, LDSB, EPI, FAST, 1>(p, f, wsr, m0, n0, wm, wn, tid, smem);
    else if (post == 2)
        store_tile_impl<BM, BN, WM, WN, LDSB, EPI, FAST, 2>(p, f, wsr, m0, n0, wm, wn, tid, smem);
    else
        store_tile_impl<BM, BN, WM, WN, LDSB, EPI, FAST, 3>(p, f, wsr, m0, n0, wm, wn, tid, smem);
}

template <int BM, int BN, int WM, int WN, int NS, int EPI, bool DUMP, bool FAST>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64, (NS > 2 || BM * BN > 128 * 128) ? 1 : 2) void k_gemm(GemmArgs p) {
    constexpr int NWN = BN / WN, NWAVE = (BM / WM) * NWN, NT = NWAVE * 64;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int AI = BM / 8 / NWAVE, BI = BN / 8 / NWAVE;  // 1-KB loads per wave per step
    static_assert(AI * NWAVE * 8 == BM && BI * NWAVE * 8 == BN, "tile/threads mismatch");
    static_assert(BM <= 64 * NWAVE, "one scale per lane");
    constexpr int STAGE = (BM + BN) * 128 + 64 * NWAVE * 4;  // A | W | scales (one per lane)
    extern __shared__ __align__(16) unsigned char smem[];

    const int tiles_n = (p.N + BN - 1) / BN;
    const int pid = xcd_swizzle(blockIdx.x, gridDim.x);
    const int m0 = (pid / tiles_n) * BM, n0 = (pid % tiles_n) * BN;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / NWN, wn = wave % NWN;
    const int nb = p.K / kQBlock;

    // per-lane global byte offsets (32-bit: the host checks both operands span < 4 GiB); rows past
    // M/N are clamped, their outputs are never stored
    uint32_t oa[AI], ob[BI];
#pragma unroll
    for (int i = 0; i < AI; i++) {
        const int r = (i * NWAVE + wave) * 8 + (lane >> 3);
        oa[i] = (uint32_t)min(m0 + r, p.M - 1) * (uint32_t)p.lda + (((lane & 7) ^ swzk(r)) << 4);
    }
#pragma unroll
    for (int i = 0; i < BI; i++) {
        const int r = (i * NWAVE + wave) * 8 + (lane >> 3);
        ob[i] = (uint32_t)min(n0 + r, p.N - 1) * (uint32_t)p.ldw + (((lane & 7) ^ swzk(r)) << 4);
    }
    // scales: lane (wave, lane) fetches row wave*64+lane (waves past BM/64 fetch a clamped copy
    // into their own slot, so every wave issues the same number of loads per step)
    const uint32_t os = (uint32_t)min(m0 + wave * 64 + lane, p.M - 1) * (uint32_t)nb * 4;
    // buffer descriptors: per-lane offsets stay in VGPRs, the K step's offset is a scalar
    const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc(
        (void *)p.A, 0, (int)(uint32_t)((size_t)p.M * p.lda), 0x00020000);
    const __amdgpu_buffer_rsrc_t rW = __builtin_amdgcn_make_buffer_rsrc(
        (void *)p.W, 0, (int)(uint32_t)((size_t)p.N * p.ldw), 0x00020000);
    const __amdgpu_buffer_rsrc_t rS = __builtin_amdgcn_make_buffer_rsrc(
        (void *)p.as, 0, (int)(uint32_t)((size_t)p.M * nb * 4), 0x00020000);

    auto issue = [&](int kb, int st) {
        unsigned char *s = smem + st * STAGE;
        const int ko = kb * kQBlock;
#pragma unroll
        for (int i = 0; i < AI; i++)
            lds_load16(rA, s + (i * NWAVE + wave) * 1024, oa[i], ko);
#pragma unroll
        for (int i = 0; i < BI; i++)
            lds_load16(rW, s + BM * 128 + (i * NWAVE + wave) * 1024, ob[i], ko);
        lds_load4(rS, s + (BM + BN) * 128 + wave * 256, os, kb * 4);
    };

    float wsr[TN];
#pragma unroll
    for (int tn = 0; tn < TN; tn++)
        wsr[tn] = p.ws[min(n0 + wn * WN + tn * 32 + (lane & 31), p.N - 1)];

    v16i acc[TM][TN];
    float f[TM][TN][16];
#pragma unroll
    for (int tm = 0; tm < TM; tm++)
#pragma unroll
        for (int tn = 0; tn < TN; tn++)
#pragma unroll
            for (int r = 0; r < 16; r++) f[tm][tn][r] = 0.f;

#pragma unroll
    for (int st = 0; st < NS - 1; st++)
        if (st < nb) issue(st, st);
    const v16i zero = {};
    constexpr int L = AI + BI + 1;  // loads per wave per step
    for (int kb = 0; kb < nb; kb++) {
        // wait for this step's tiles (later steps may stay in flight), then the barrier both
        // publishes them and retires every wave's reads of the buffer refilled next
        const int rem = min(nb - 1 - kb, NS - 2);
        if (rem <= 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        else if (rem == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(L) : "memory");
        else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * L) : "memory");
        __syncthreads();
        if (kb + NS - 1 < nb) issue(kb + NS - 1, (kb + NS - 1) % NS);
        const int cur = kb % NS;
        const unsigned char *sb0 = smem + cur * STAGE;
        const float *asb = (const float *)(sb0 + (BM + BN) * 128) + wm * WM + (lane >> 5) * 4;
        {
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                const int cc = kk * 2 + (lane >> 5);
                v4i af[TM], bf[TN];
#pragma unroll
                for (int tm = 0; tm < TM; tm++)
                    af[tm] = *(const v4i *)(sb0 + swz(wm * WM + tm * 32 + (lane & 31), cc));
#pragma unroll
                for (int tn = 0; tn < TN; tn++)
                    bf[tn] = *(const v4i *)(sb0 + BM * 128 + swz(wn * WN + tn * 32 + (lane & 31), cc));
#pragma unroll
                for (int tm = 0; tm < TM; tm++)
#pragma unroll
                    for (int tn = 0; tn < TN; tn++)
                        acc[tm][tn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(
                            af[tm], bf[tn], kk == 0 ? zero : acc[tm][tn], 0, 0, 0);
            }
            // fold this block: f = fma((float)acc, RN(as*ws), f), the reference's order
#pragma unroll
            for (int tm = 0; tm < TM; tm++)
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const float4 a4 = *(const float4 *)(asb + tm * 32 + g * 8);
                    const float av[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
                    for (int tn = 0; tn < TN; tn++)
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            const int r = g * 4 + j;
                            // FAST folds only the activation scale per block and applies ws[n] once
                            // at the end (2 VALU ops per element and block instead of 3; f32 result
                            // within a few ulp of the reference's order instead of bit-exact)
                            f[tm][tn][r] = __builtin_fmaf((float)acc[tm][tn][r],
                                                          FAST ? av[j] : __fmul_rn(av[j], wsr[tn]),
                                                          f[tm][tn][r]);
                        }
                }
        }
        if constexpr (DUMP) {
#pragma unroll
            for (int tm = 0; tm < TM; tm++)
#pragma unroll
                for (int tn = 0; tn < TN; tn++)
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int m = m0 + wm * WM + tm * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                        const int n = n0 + wn * WN + tn * 32 + (lane & 31);
                        if (m < p.M && n < p.N)
                            p.accd[((size_t)kb * p.M + m) * p.N + n] = acc[tm][tn][r];
                    }
        }
    }
    __syncthreads();  // the epilogue may reuse the staging buffers
    store_tile<BM, BN, WM, WN, NS * STAGE, EPI, FAST>(p, f, wsr, m0, n0, wm, wn, tid, smem);
}

// LDS of the double-buffered kernel: NS stages of A|W, NS+1 scale slots, and at least the f32
// tile the requantizing epilogues stage (row pitch BN+4 floats)
constexpr int db_lds_bytes(int BM, int BN, int NWAVE, int NS, int EPI) {
    const int loop = NS * (BM + BN) * 128 + (NS + 1) * 64 * NWAVE * 4;
    const int epi = EPI == EPI_F32 ? 0 : BM * (BN + 4) * 4;
    return loop > epi ? loop : epi;
}

// Kernel with double-buffered int32 accumulators: the MFMAs of K step kb accumulate into one set
// while the other set, holding step kb-1, is folded into f on the VALU, one 32x32 tile after each
// of the 4 MFMA rounds. The fold of a step therefore overlaps the next step's MFMAs instead of
// waiting for them (the fold costs as many VALU cycles per element as the MFMAs take). The loads
// run NS-1 steps ahead; the activation scales of a step live in a ring of NS+1 slots so the fold
// of step kb-1 can still read them while step kb+NS-1 is being loaded.
template <int BM, int BN, int WM, int WN, int NS, int EPI, bool FAST, int OCC>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64, OCC) void k_gemm_db(GemmArgs p) {
    constexpr int NWN = BN / WN, NWAVE = (BM / WM) * NWN;
    constexpr int TM = WM / 32, TN = WN / 32, NTILE = TM * TN;
    constexpr int TPK = (NTILE + 3) / 4;                      // tiles folded per MFMA round
    constexpr int AI = BM / 8 / NWAVE, BI = BN / 8 / NWAVE;  // 1-KB loads per wave per step
    static_assert(AI * NWAVE * 8 == BM && BI * NWAVE * 8 == BN, "tile/threads mismatch");
    static_assert(BM <= 64 * NWAVE, "one scale per lane");
    constexpr int TILE = (BM + BN) * 128;  // A | W of one step
    constexpr int SSLOT = 64 * NWAVE * 4;  // one step's activation scales (one per lane)
    constexpr int RS = NS + 1;
    extern __shared__ __align__(16) unsigned char smem[];
    unsigned char *const sscale = smem + NS * TILE;

    const int tiles_n = (p.N + BN - 1) / BN;
    const int pid = xcd_swizzle(blockIdx.x, gridDim.x);
    const int m0 = (pid / tiles_n) * BM, n0 = (pid % tiles_n) * BN;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / NWN, wn = wave % NWN;
    const int nb = p.K / kQBlock;

    uint32_t oa[AI], ob[BI];
#pragma unroll
    for (int i = 0; i < AI; i++) {
        const int r = (i * NWAVE + wave) * 8 + (lane >> 3);
        oa[i] = (uint32_t)min(m0 + r, p.M - 1) * (uint32_t)p.lda + (((lane & 7) ^ swzk(r)) << 4);
    }
#pragma unroll
    for (int i = 0; i < BI; i++) {
        const int r = (i * NWAVE + wave) * 8 + (lane >> 3);
        ob[i] = (uint32_t)min(n0 + r, p.N - 1) * (uint32_t)p.ldw + (((lane & 7) ^ swzk(r)) << 4);
    }
    const uint32_t os = (uint32_t)min(m0 + wave * 64 + lane, p.M - 1) * (uint32_t)nb * 4;
    // buffer descriptors: per-lane offsets stay in VGPRs, the K step's offset is a scalar
    const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc(
        (void *)p.A, 0, (int)(uint32_t)((size_t)p.M * p.lda), 0x00020000);
    const __amdgpu_buffer_rsrc_t rW = __builtin_amdgcn_make_buffer_rsrc(
        (void *)p.W, 0, (int)(uint32_t)((size_t)p.N * p.ldw), 0x00020000);
    const __amdgpu_buffer_rsrc_t rS = __builtin_amdgcn_make_buffer_rsrc(
        (void *)p.as, 0, (int)(uint32_t)((size_t)p.M * nb * 4), 0x00020000);

    auto issue = [&](int kb) {
        unsigned char *st = smem + (kb % NS) * TILE;
        const int ko = kb * kQBlock;
#pragma unroll
        for (int i = 0; i < AI; i++)
            lds_load16(rA, st + (i * NWAVE + wave) * 1024, oa[i], ko);
#pragma unroll
        for (int i = 0; i < BI; i++)
            lds_load16(rW, st + BM * 128 + (i * NWAVE + wave) * 1024, ob[i], ko);
        lds_load4(rS, sscale + (kb % RS) * SSLOT + wave * 256, os, kb * 4);
    };

    float wsr[TN];
#pragma unroll
    for (int tn = 0; tn < TN; tn++)
        wsr[tn] = p.ws[min(n0 + wn * WN + tn * 32 + (lane & 31), p.N - 1)];

    float f[TM][TN][16];
#pragma unroll
    for (int tm = 0; tm < TM; tm++)
#pragma unroll
        for (int tn = 0; tn < TN; tn++)
#pragma unroll
            for (int r = 0; r < 16; r++) f[tm][tn][r] = 0.f;
    v16i acc0[TM][TN], acc1[TM][TN];

    // fold one 32x32 tile of step kb: f = fma((float)acc, RN(as*ws), f), the reference's order
    auto fold = [&](const v16i (&acc)[TM][TN], int t, int kb) {
        const int tm = t / TN, tn = t % TN;
        const float *asb = (const float *)(sscale + (kb % RS) * SSLOT) + wm * WM + tm * 32 + (lane >> 5) * 4;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const float4 a4 = *(const float4 *)(asb + g * 8);
            const float av[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int r = g * 4 + j;
                f[tm][tn][r] = __builtin_fmaf((float)acc[tm][tn][r],
                                              FAST ? av[j] : __fmul_rn(av[j], wsr[tn]), f[tm][tn][r]);
            }
        }
    };

#pragma unroll
    for (int st = 0; st < NS - 1; st++)
        if (st < nb) issue(st);
    constexpr int L = AI + BI + 1;  // loads per wave per step
    const v16i zero = {};
    // one K step into `cur`, folding `prev` (step kb-1) tile by tile when FOLD
    auto step = [&](auto fold_prev, int kb, v16i (&cur)[TM][TN], const v16i (&prev)[TM][TN]) {
        const int rem = min(nb - 1 - kb, NS - 2);
        if (rem <= 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        else if (rem == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(L) : "memory");
        else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * L) : "memory");
        __syncthreads();
        if (kb + NS - 1 < nb) issue(kb + NS - 1);
        const unsigned char *sb = smem + (kb % NS) * TILE;
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            const int cc = kk * 2 + (lane >> 5);
            v4i af[TM], bf[TN];
#pragma unroll
            for (int tm = 0; tm < TM; tm++)
                af[tm] = *(const v4i *)(sb + swz(wm * WM + tm * 32 + (lane & 31), cc));
#pragma unroll
            for (int tn = 0; tn < TN; tn++)
                bf[tn] = *(const v4i *)(sb + BM * 128 + swz(wn * WN + tn * 32 + (lane & 31), cc));
#pragma unroll
            for (int tm = 0; tm < TM; tm++)
#pragma unroll
                for (int tn = 0; tn < TN; tn++)
                    cur[tm][tn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[tm], bf[tn],
                                                                        kk == 0 ? zero : cur[tm][tn], 0, 0, 0);
            if constexpr (decltype(fold_prev)::value) {
#pragma unroll
                for (int t = kk * TPK; t < (kk + 1) * TPK; t++)
                    if (t < NTILE) fold(prev, t, kb - 1);
            }
        }
    };
    using no_fold = std::integral_constant<bool, false>;
    using do_fold = std::integral_constant<bool, true>;
    step(no_fold{}, 0, acc0, acc1);
    int kb = 1;
    for (; kb + 1 < nb; kb += 2) {
        step(do_fold{}, kb, acc1, acc0);
        step(do_fold{}, kb + 1, acc0, acc1);
    }
    if (kb < nb) {  // nb even: the last step (odd) lands in acc1
        step(do_fold{}, kb, acc1, acc0);
#pragma unroll
        for (int t = 0; t < NTILE; t++) fold(acc1, t, kb);
    } else {
#pragma unroll
        for (int t = 0; t < NTILE; t++) fold(acc0, t, nb - 1);
    }
    __syncthreads();  // the epilogue may reuse the staging buffers
    store_tile<BM, BN, WM, WN, db_lds_bytes(BM, BN, NWAVE, NS, EPI), EPI, FAST>(p, f, wsr, m0, n0, wm, wn,
                                                                             tid, smem);
}

template <int BM, int BN, int WM, int WN, int NS, int EPI, bool FAST, int OCC>
static int launch_db1(hipStream_t s, const GemmArgs &p) {
    constexpr int NWAVE = (BM / WM) * (BN / WN);
    constexpr size_t lds = db_lds_bytes(BM, BN, NWAVE, NS, EPI);
    static_assert(NS >= 2 && NS <= 4 && lds <= 160 * 1024, "LDS budget");
    auto kern = k_gemm_db<BM, BN, WM, WN, NS, EPI, FAST, OCC>;
    static bool attr = false;
    if (!attr) {
        if (check_hip(hipFuncSetAttribute((const void *)kern,
                                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                      "gemm lds attribute"))
            return -1;
        attr = true;
    }
    const long tiles = (long)((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
    hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(NWAVE * 64), lds, s, p);
    return check_hip(hipGetLastError(), "gemm launch");
}

template <int BM, int BN, int WM, int WN, int NS, int EPI, bool DUMP, bool FAST>
static int launch_tile1(hipStream_t s, const GemmArgs &p) {
    constexpr int NT = (BM / WM) * (BN / WN) * 64;
    constexpr int NWAVE = (BM / WM) * (BN / WN);
    constexpr size_t lds = NS * ((size_t)(BM + BN) * 128 + 64 * NWAVE * 4);
    static_assert(NS >= 2 && NS <= 4 && lds <= 160 * 1024, "LDS budget");
    auto kern = k_gemm<BM, BN, WM, WN, NS, EPI, DUMP, FAST>;
    static bool attr = false;
    if (!attr) {
        if (check_hip(hipFuncSetAttribute((const void *)kern,
                                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                      "gemm lds attribute"))
            return -1;
        attr = true;
    }
    const long tiles = (long)((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
    hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(NT), lds, s, p);
    return check_hip(hipGetLastError(), "gemm launch");
}

// E2MI_GEMM_FOLD=fast selects the 2-op fold for the whole process (read once); the default is
// the reference's bit-exact fold order
static bool fold_fast() {
    static int v = -1;
    if (v < 0) {
        const char *e = getenv("E2MI_GEMM_FOLD");
        v = (e && strcmp(e, "fast") == 0) ? 1 : 0;
    }
    return v == 1;
}

template <int BM, int BN, int WM, int WN, int NS, int EPI, bool DUMP>
static int launch_tile(hipStream_t s, const GemmArgs &p) {
    if (!DUMP && fold_fast()) return launch_tile1<BM, BN, WM, WN, NS, EPI, DUMP, true>(s, p);
    return launch_tile1<BM, BN, WM, WN, NS, EPI, DUMP, false>(s, p);
}

static int check_args(const GemmArgs &p, const char *who) {
    if (p.M <= 0 || p.N <= 0 || p.K <= 0 || p.K % kQBlock) {
        set_error("%s: bad geometry M=%d N=%d K=%d (K must be a positive multiple of 128)", who, p.M,
                  p.N, p.K);
        return -1;
    }
    if (!p.A || !p.as || !p.W || !p.ws || !aligned16(p.A) || !aligned16(p.W) || p.lda % 16 ||
        p.ldw % 16 || p.lda < p.K || p.ldw < p.K) {
        set_error("%s: operands must be non-null, 16-byte aligned, with 16-byte row pitches >= K", who);
        return -1;
    }
    if ((long)p.M * (long)p.N > (1L << 31) || (long)p.M * p.lda >= (1L << 32) ||
        (long)p.N * p.ldw >= (1L << 32) || (long)p.M * p.ldy * 4 >= (1L << 31)) {
        set_error("%s: problem too large", who);
        return -1;
    }
    return 0;
}

int launch_gemm_f32(hipStream_t s, GemmArgs p, bool dump) {
    if (check_args(p, "i8_gemm")) return -1;
    if (!p.Y || p.ldy < p.N) {
        set_error("i8_gemm: null output or ldy < N");
        return -1;
    }
    if (dump) {
        if (!p.accd) {
            set_error("i8_gemm: null accumulator dump");
            return -1;
        }
        return launch_tile<128, 128, 64, 64, 2, EPI_F32, true>(s, p);
    }
    return launch_tile<128, 128, 64, 64, 2, EPI_F32, false>(s, p);
}

int launch_gemm_i8q(hipStream_t s, GemmArgs p) {
    if (check_args(p, "i8_gemm_q")) return -1;
    if (p.N % 128 || !p.Yq || !p.ys || p.ldyq < p.N || p.ldyq % 16 || !aligned16(p.Yq) ||
        p.ldys < p.N / 128) {
        set_error("i8_gemm_q: N must be a multiple of 128 with a 16-byte aligned int8 output");
        return -1;
    }
    return launch_tile<128, 128, 64, 64, 2, EPI_I8Q, false>(s, p);
}

int launch_gemm_geglu(hipStream_t s, GemmArgs p) {
    if (check_args(p, "i8_gemm_geglu")) return -1;
    if (p.N % 256 || !p.Yq || !p.ys || p.ldyq < p.N / 2 || p.ldyq % 16 || !aligned16(p.Yq) ||
        p.ldys < p.N / 256 || (p.Y && (p.ldy < p.N / 2 || p.ldy % 4 || !aligned16(p.Y)))) {
        set_error("i8_gemm_geglu: N (gate|up interleaved) must be a multiple of 256, outputs aligned");
        return -1;
    }
    // 8 waves of 64x64 over a 128x256 tile (64 output columns per wave pair), accumulators
    // double-buffered so the fold overlaps the next step's MFMAs
    if (fold_fast()) return launch_db1<128, 256, 64, 64, 2, EPI_GEGLU, true, 2>(s, p);
    return launch_db1<128, 256, 64, 64, 2, EPI_GEGLU, false, 2>(s, p);
}

}  // namespace e2mi

// ------------------------------------------------------------------ C ABI
using namespace e2mi;

static int weight_ok(const e2mi_q8w *w, const char *who) {
    if (!w || !w->w || !w->scale || w->N <= 0 || w->K <= 0 || w->K % 128 || w->ld < w->K ||
        w->ld % 16) {
        set_error("%s: invalid weight handle", who);
        return 0;
    }
    return 1;
}

static GemmArgs make_args(const int8_t *qa, const float *as, const e2mi_q8w *w, int M, int n0,
                          int n1) {
    GemmArgs p = {};
    p.A = qa;
    p.as = as;
    p.W = w->w + (size_t)n0 * w->ld;
    p.ws = w->scale + n0;
    p.bias = w->bias ? w->bias + n0 : nullptr;
    p.lda = w->K;
    p.ldw = w->ld;
    p.M = M;
    p.N = n1 - n0;
    p.K = w->K;
    p.lo = w->out_min;
    p.hi = w->out_max;
    return p;
}

extern "C" int e2mi_i8_gemm(e2mi_stream stream, float *y, int ldy, const int8_t *qa,
                            const float *a_scales, const e2mi_q8w *w, int M, int n0, int n1) {
    if (!weight_ok(w, "i8_gemm")) return -1;
    if (n0 < 0 || n1 > w->N || n0 >= n1 || !y) {
        set_error("i8_gemm: bad column range [%d,%d) for N=%d", n0, n1, w ? w->N : 0);
        return -1;
    }
    GemmArgs p = make_args(qa, a_scales, w, M, n0, n1);
    p.Y = y + n0;
    p.ldy = ldy;
    return launch_gemm_f32((hipStream_t)stream, p, false);
}

extern "C" int e2mi_i8_gemm_acc(e2mi_stream stream, float *y, int ldy, int32_t *acc,
                                const int8_t *qa, const float *a_scales, const e2mi_q8w *w, int M,
                                int n0, int n1) {
    if (!weight_ok(w, "i8_gemm_acc")) return -1;
    if (n0 < 0 || n1 > w->N || n0 >= n1 || !y || !acc) {
        set_error("i8_gemm_acc: bad column range [%d,%d) or null output", n0, n1);
        return -1;
    }
    GemmArgs p = make_args(qa, a_scales, w, M, n0, n1);
    p.Y = y + n0;
    p.ldy = ldy;
    p.accd = acc;
    return launch_gemm_f32((hipStream_t)stream, p, true);
}

extern "C" int e2mi_i8_gemm_q(e2mi_stream stream, int8_t *yq, float *ys, const int8_t *qa,
                              const float *a_scales, const e2mi_q8w *w, int M) {
    if (!weight_ok(w, "i8_gemm_q")) return -1;
    GemmArgs p = make_args(qa, a_scales, w, M, 0, w->N);
    p.Yq = yq;
    p.ldyq = w->N;
    p.ys = ys;
    p.ldys = w->N / 128;
    return launch_gemm_i8q((hipStream_t)stream, p);
}

extern "C" int e2mi_i8_gemm_geglu(e2mi_stream stream, int8_t *q, float *qs, float *g,
                                  const int8_t *qa, const float *a_scales,
                                  const e2mi_q8w *w_gate_up, int M) {
    if (!weight_ok(w_gate_up, "i8_gemm_geglu")) return -1;
    GemmArgs p = make_args(qa, a_scales, w_gate_up, M, 0, w_gate_up->N);
    const int F = w_gate_up->N / 2;
    p.Yq = q;
    p.ldyq = F;
    p.ys = qs;
    p.ldys = F / 128;
    p.Y = g;
    p.ldy = F;
    return launch_gemm_geglu((hipStream_t)stream, p);
}
