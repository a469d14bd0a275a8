// gemm.hip — W8A8 GEMM on gfx950 int8 MFMA (v_mfma_i32_32x32x32_i8) with the fused per-block
// dequantization of the reference's e2_i8_gemm (src/int8.h:94-97; fold order of
// src/kernels_i8_avx512_vnni.c:100-122):
//
//   y[m,n] = sum_b fma((float)acc_b[m,n], RN(as[m,b] * ws[n]), .)      acc_b exact int32
//
// then one of the fused epilogues:
//   EPI_F32   y (+bias), clamped to [lo,hi], stored f32 (the reference contract)
//   EPI_I8Q   y (+bias) requantized per (row, 128 output columns) for the next GEMM: int8 + scale
//   EPI_GELUMUL g = gelu_tanh(y) * mul[m][n] (mul from memory: the PLE gate, text.c:906-913),
//             quantized per (row, 128 columns) like EPI_I8Q; g optionally stored f32
//   EPI_GEGLU W rows interleaved per 64 as [32 gate | 32 up]; g = gelu_tanh(gate) * up is
//             quantized per 128 (text.c:424-468 fused into the producing GEMM), g optionally kept
//   EPI_QKV   the q|k|v projection with the attention's row stage fused in (text.c:836-854): per
//             256-wide head, RMSNorm (q/k with their gamma, v without), RoPE on q and k, f16
//             outputs for the attention (q, k row-major, V transposed); W's rows of each head in
//             rotate-half pair order (see p_epilogue_qkv)
//
// The production kernels are persistent and software-pipelined: k_gemm_p for per-(row, 128)
// activation scales (K is walked in 128-deep steps, one quantization block per step, so the int32
// accumulators are folded into f32 once per step) and k_gemm_t for per-row (per-token) scales,
// whose accumulators run over the whole K of a tile; their designs are described above them.
// k_gemm_dump is a plain kernel that also writes every K block's int32 accumulators, the parity
// hook for the integer part.
// A and W tiles live in LDS as 128-byte K slices of consecutive rows whose fragment reads are
// conflict-free on the 64-bank LDS (see swz).
#include <stdlib.h>
#include <string.h>

#include <type_traits>
#include <utility>

#include <stddef.h>

#include "common.h"

namespace e2mi {

enum { EPI_F32 = 0, EPI_I8Q = 1, EPI_GEGLU = 2, EPI_GELUMUL = 3, EPI_QKV = 4 };

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
    const float *mul;  // EPI_GELUMUL: the multiplier of gelu(y) [M][ldmul]
    int ldmul;
    int lda, ldw, ldy, ldyq, ldys;
    int M, N, K;
    float lo, hi;
    // EPI_QKV: q/k gammas [256], RoPE tables [positions][256], each row's position (packed
    // batches) or none (row % qS), f16 outputs q [M][qH*256], k [M][qKV*256] and V^T
    // [M/qS][qKV][256][qS], optional f32 copies q, k, v [M][heads*256]
    const float *q_gamma, *k_gamma, *cs, *sn;
    const int32_t *pos;
    uint16_t *q16, *k16, *vt16;
    float *q32, *k32, *v32;
    int qH, qKV, qS;
    float eps;
    // a device row count (a multiple of 256, at most M; k_gemm_p only, which takes it as its own
    // first argument), or null: M rows
    const int *rows;
};


// LDS tiles hold 128-byte K slices of consecutive rows with no padding. The LDS has 64 banks of 4
// bytes and serves a ds_read_b128 16 lanes at a time; a 128-byte row spans 32 banks, so rows of
// equal parity share a bank half. The 16-byte chunk c of row r sits at slot c ^ ((r >> 1) & 7):
// the 16 consecutive rows read by one 16-lane group then cover all 64 banks once. Each
// 1-KB direct-to-LDS load fills 8 rows of a tile: lane l writes slot l, so it fetches row l/8's
// chunk (l % 8) ^ ((row >> 1) & 7).
__device__ inline int swzk(int r) { return (r >> 1) & 7; }
__device__ inline int swz(int r, int c) { return r * 128 + ((c ^ swzk(r)) << 4); }

// Buffer loads straight into LDS: the per-lane offset is a VGPR fixed for the whole K loop and the
// K step's offset a scalar, so a step costs no VALU address arithmetic. (Device functions rather
// than lambdas: the builtin is only known to the device pass.)
__device__ inline void lds_load16(__amdgpu_buffer_rsrc_t r, void *lds, uint32_t voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds, 16, voff, soff, 0, 0);
}
__device__ inline void lds_load4(__amdgpu_buffer_rsrc_t r, void *lds, uint32_t voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)lds, 4, voff, soff, 0, 0);
}

// The direct-to-LDS loads of the pipelined kernel (dma16, dma4, rsrc_words) are in common.h.

// The accumulator-dump kernel (e2mi_i8_gemm_acc, the parity hook for "bit-exact int32
// accumulators"): 128 x 128 tiles of 4 waves of 64 x 64, two direct-to-LDS stages, the exact fold
// after each step's MFMAs, every step's int32 accumulators written to accd [nb][M][N], f32 output
// with the optional bias and clamp. Not a throughput path.
__global__ __launch_bounds__(256, 2) void k_gemm_dump(GemmArgs p) {
    constexpr int BM = 128, BN = 128, WM = 64, WN = 64, NWN = 2, NWAVE = 4, TM = 2, TN = 2;
    constexpr int AI = BM / 8 / NWAVE, BI = BN / 8 / NWAVE;  // 1-KB loads per wave per step
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
    const uint32_t os = (uint32_t)min(m0 + wave * 64 + lane, p.M - 1) * (uint32_t)nb * 4;
    const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc(
        (void *)p.A, 0, (int)(uint32_t)((size_t)p.M * p.lda), 0x00020000);
    const __amdgpu_buffer_rsrc_t rW = __builtin_amdgcn_make_buffer_rsrc(
        (void *)p.W, 0, (int)(uint32_t)((size_t)p.N * p.ldw), 0x00020000);
    const __amdgpu_buffer_rsrc_t rS = __builtin_amdgcn_make_buffer_rsrc(
        (void *)p.as, 0, (int)(uint32_t)((size_t)p.M * nb * 4), 0x00020000);
    auto issue = [&](int kb) {
        unsigned char *s = smem + (kb & 1) * STAGE;
        const int ko = kb * kQBlock;
#pragma unroll
        for (int i = 0; i < AI; i++) lds_load16(rA, s + (i * NWAVE + wave) * 1024, oa[i], ko);
#pragma unroll
        for (int i = 0; i < BI; i++) lds_load16(rW, s + BM * 128 + (i * NWAVE + wave) * 1024, ob[i], ko);
        lds_load4(rS, s + (BM + BN) * 128 + wave * 256, os, kb * 4);
    };

    float wsr[TN];
#pragma unroll
    for (int tn = 0; tn < TN; tn++) wsr[tn] = p.ws[min(n0 + wn * WN + tn * 32 + (lane & 31), p.N - 1)];
    v16i acc[TM][TN];
    float f[TM][TN][16];
#pragma unroll
    for (int tm = 0; tm < TM; tm++)
#pragma unroll
        for (int tn = 0; tn < TN; tn++)
#pragma unroll
            for (int r = 0; r < 16; r++) f[tm][tn][r] = 0.f;
    issue(0);
    const v16i zero = {};
    for (int kb = 0; kb < nb; kb++) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (kb + 1 < nb) issue(kb + 1);
        const unsigned char *sb0 = smem + (kb & 1) * STAGE;
        const float *asb = (const float *)(sb0 + (BM + BN) * 128) + wm * WM + (lane >> 5) * 4;
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            const int cc = kk * 2 + (lane >> 5);
            v4i af[TM], bf[TN];
#pragma unroll
            for (int tm = 0; tm < TM; tm++) af[tm] = *(const v4i *)(sb0 + swz(wm * WM + tm * 32 + (lane & 31), cc));
#pragma unroll
            for (int tn = 0; tn < TN; tn++) bf[tn] = *(const v4i *)(sb0 + BM * 128 + swz(wn * WN + tn * 32 + (lane & 31), cc));
#pragma unroll
            for (int tm = 0; tm < TM; tm++)
#pragma unroll
                for (int tn = 0; tn < TN; tn++)
                    acc[tm][tn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[tm], bf[tn], kk == 0 ? zero : acc[tm][tn], 0, 0, 0);
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
                        f[tm][tn][r] = __builtin_fmaf((float)acc[tm][tn][r], __fmul_rn(av[j], wsr[tn]), f[tm][tn][r]);
                    }
            }
#pragma unroll
        for (int tm = 0; tm < TM; tm++)
#pragma unroll
            for (int tn = 0; tn < TN; tn++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int m = m0 + wm * WM + tm * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                    const int n = n0 + wn * WN + tn * 32 + (lane & 31);
                    if (m < p.M && n < p.N) p.accd[((size_t)kb * p.M + m) * p.N + n] = acc[tm][tn][r];
                }
    }
#pragma unroll
    for (int tn = 0; tn < TN; tn++) {
        const int n = n0 + wn * WN + tn * 32 + (lane & 31);
        if (n >= p.N) continue;
        const float b = p.bias ? p.bias[n] : 0.f;
#pragma unroll
        for (int tm = 0; tm < TM; tm++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + wm * WM + tm * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                if (m < p.M) p.Y[(size_t)m * p.ldy + n] = fminf(fmaxf(f[tm][tn][r] + b, p.lo), p.hi);
            }
    }
}

// fold order of all GEMM launches (e2mi_gemm_set_fold); E2MI_GEMM_FOLD=fast sets the fast one
// at the first launch
static int g_fold = -1;
static bool fold_fast() {
    if (g_fold < 0) {
        const char *e = getenv("E2MI_GEMM_FOLD");
        g_fold = (e && strcmp(e, "fast") == 0) ? 1 : 0;
    }
    return g_fold == 1;
}
bool gemm_fold_fast() { return fold_fast(); }

// ---------------------------------------------------------------------------------------------
// Persistent pipelined kernel (the production path). One 512-thread workgroup per CU walks a list
// of BM x BN output tiles; the 128-deep K steps of consecutive tiles form one flat pipeline:
//   - A, W, the step's activation scales and its tile's weight scales go HBM/L2 -> LDS by direct
//     buffer loads two steps ahead (3 A|W stages, a ring of 4 scale slots), issued two at a time
//     between the step's MFMAs;
//   - 8 waves of 32 x 128 each; the int32 accumulators are double-buffered: the MFMAs of step g
//     accumulate into one set while the other set (step g-1) is folded into f on the VALU, the
//     fold cut into 4-element units placed between the step's 16 MFMAs (sched_group_barrier),
//     since the fold costs more VALU cycles than the MFMAs take;
//   - a tile's last step is folded during the next tile's first step, then the tile's epilogue
//     runs; requantizing epilogues transpose f through wave-private rows of the step's consumed
//     A|W stage.
// The tile list (M-major) is cut into one contiguous chunk per XCD (workgroups are dispatched
// round-robin over the 8 XCDs), so the N tiles of an M block run on one XCD and share its L2.
// 8-wave workgroups (one per CU) keep 3 A|W stages (loads two steps ahead); 4-wave workgroups
// (two per CU) keep 2 (one step ahead)
constexpr int kPSlots = 4;
template <int NWAVE>
constexpr int p_stages() { return NWAVE == 8 ? 3 : 2; }

// a slot holds one step's activation scales and its tile's weight scales, one float per lane each
template <int BM, int BN, int NWAVE>
constexpr int p_lds_bytes() {
    return p_stages<NWAVE>() * (BM + BN) * 128 + kPSlots * 2 * 64 * NWAVE * 4;
}

// requantizing epilogue of one tile. Every wave owns whole rows of each 128-column quantization
// block (I8Q: its 32 x 128 tile; GEGLU: 32 rows x 64 of a block's 128 output columns, the other
// 64 in wave wn ^ 1), so the transpose from the MFMA layout to row-contiguous columns goes through
// a wave-private LDS area (8 rows at a time) with no workgroup barrier; GEGLU exchanges only the
// per-row partial maxima between the two waves of a block (one barrier). scr: 8 waves x 8 rows x
// (RW + 4) floats, then GEGLU's exchange area of 8 waves x 32 floats.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
// cache policy of the per-token kernel's output stores (epilogues with NT = true): sc0 | nt
// (non-temporal, streamed past the caches). Measured on the per-token f32 sweep at M = 65536, whose
// outputs nothing re-reads: 1124 -> 1350 TOPS (768x1280: 121.5 -> 96.6 us) against the default
// policy. The per-128 kernel keeps the default: in the encoder's forward the next kernel reads its
// outputs at once, and streaming them cost 2 % end to end. A runtime choice between the two (a
// uniform branch per store) cost the epilogues 2-5 %, so it is per kernel, at compile time.
constexpr int kStoreNT = 3;

template <int BM, int BN, int NWM, int NWN, int EPI, bool FAST, int POST, bool NT = false>
__device__ __attribute__((always_inline)) inline void p_epilogue_q(const GemmArgs &p, float (&f)[4][16],
                                                                   const float (&wsr)[4], int m0, int n0,
                                                                   int wave, int wm, int wn, int lane,
                                                                   float *scr) {
    constexpr bool GG = EPI == EPI_GEGLU, GM = EPI == EPI_GELUMUL;
    constexpr int RW = GG ? 64 : 128;  // output columns per wave row
    constexpr int FP = RW + 4;          // f32 pitch of the wave-private rows
    constexpr int CPL = RW / 8;         // output columns per lane in the transposed chunk (16 | 8)
    float *ws_ = scr + wave * 8 * FP;   // this wave's 8 rows
    float b[4] = {0.f, 0.f, 0.f, 0.f};
    if constexpr (POST & 1) {
        if (p.bias) {
#pragma unroll
            for (int tn = 0; tn < 4; tn++) b[tn] = p.bias[min(n0 + wn * 128 + tn * 32 + (lane & 31), p.N - 1)];
        }
    }
    auto post = [&](float v, int tn) {
        if constexpr (FAST) v = __fmul_rn(v, wsr[tn]);
        if constexpr (POST & 1) v = v + b[tn];
        if constexpr (POST & 2) v = fminf(fmaxf(v, p.lo), p.hi);
        return v;
    };
    const int cr = lane >> 3, cc = (lane & 7) * CPL;  // transposed chunk: row, first column
    // output column of this lane's transposed values and the row stride
    const int oc = (GG ? n0 / 2 + wn * 64 : n0 + wn * 128) + cc;
    const int ldo = GG ? p.N / 2 : p.N;
    float v[4][CPL];  // per chunk, the lane's CPL output values of row 8c + cr
    float amax[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        // registers 4c..4c+3 hold rows 8c + 4 (lane / 32) + j; column (lane % 32) of each 32-wide tile
        float *sl = ws_ + ((lane >> 5) * 4) * FP + (lane & 31);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if constexpr (GG) {
                // W columns of the wave: [gate 32 | up 32 | gate 32 | up 32]
#pragma unroll
                for (int t = 0; t < 2; t++)
                    sl[j * FP + t * 32] = gelu_tanh(post(f[2 * t][4 * c + j], 2 * t)) * post(f[2 * t + 1][4 * c + j], 2 * t + 1);
            } else {
#pragma unroll
                for (int tn = 0; tn < 4; tn++) sl[j * FP + tn * 32] = post(f[tn][4 * c + j], tn);
            }
        }
        // (LDS operations of one wave complete in order: no barrier, the reads see the writes)
        const float *rp = ws_ + cr * FP + cc;
#pragma unroll
        for (int i = 0; i < CPL; i += 4) {
            const float4 x = *(const float4 *)(rp + i);
            v[c][i] = x.x;
            v[c][i + 1] = x.y;
            v[c][i + 2] = x.z;
            v[c][i + 3] = x.w;
        }
        if constexpr (GM) {
            // g = gelu_tanh(y) * mul for the lane's CPL consecutive columns of row 8c + cr (rows
            // past M read row M - 1; their outputs are not stored)
            const int m = min(m0 + wm * 32 + 8 * c + cr, p.M - 1);
            const float *mp = p.mul + (size_t)m * p.ldmul + oc;
#pragma unroll
            for (int i = 0; i < CPL; i += 4) {
                const float4 u = oc < ldo ? *(const float4 *)(mp + i) : make_float4(0.f, 0.f, 0.f, 0.f);
                v[c][i] = gelu_tanh(v[c][i]) * u.x;
                v[c][i + 1] = gelu_tanh(v[c][i + 1]) * u.y;
                v[c][i + 2] = gelu_tanh(v[c][i + 2]) * u.z;
                v[c][i + 3] = gelu_tanh(v[c][i + 3]) * u.w;
            }
        }
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < CPL; i++) a = fmaxf(a, fabsf(v[c][i]));
        amax[c] = group_max<8>(a);  // the 8 lanes of a row hold its RW columns
    }
    if constexpr (GG) {
        // the other 64 columns of each block live in wave wn ^ 1: exchange per-row maxima
        float *xch = scr + NWM * NWN * 8 * FP;
        if ((lane & 7) == 0) {
#pragma unroll
            for (int c = 0; c < 4; c++) xch[wave * 32 + 8 * c + cr] = amax[c];
        }
        __syncthreads();
        const int other = wm * NWN + (wn ^ 1);
#pragma unroll
        for (int c = 0; c < 4; c++) amax[c] = fmaxf(amax[c], xch[other * 32 + 8 * c + cr]);
    }
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const QScale s = qscale(amax[c]);
        const int m = m0 + wm * 32 + 8 * c + cr;
        if (m < p.M && oc < ldo) {
            uint32_t w4[CPL / 4];
#pragma unroll
            for (int i = 0; i < CPL / 4; i++)
                w4[i] = pack4_magic(v[c][4 * i], v[c][4 * i + 1], v[c][4 * i + 2], v[c][4 * i + 3], s.inv);
            int8_t *dst = p.Yq + (size_t)m * p.ldyq + oc;
            float *sdst = p.ys + (size_t)m * p.ldys + (oc >> 7);
            const bool sw = (lane & 7) == 0 && (!GG || (wn & 1) == 0);
            if constexpr (NT) {
                if constexpr (CPL == 16) __builtin_nontemporal_store((u32x4){w4[0], w4[1], w4[2], w4[3]}, (u32x4 *)dst);
                else __builtin_nontemporal_store((u32x2){w4[0], w4[1]}, (u32x2 *)dst);
                if (sw) __builtin_nontemporal_store(s.sc, sdst);
            } else {
                if constexpr (CPL == 16) *(u32x4 *)dst = (u32x4){w4[0], w4[1], w4[2], w4[3]};
                else *(u32x2 *)dst = (u32x2){w4[0], w4[1]};
                if (sw) *sdst = s.sc;
            }
            if ((GG || GM) && p.Y) {
#pragma unroll
                for (int i = 0; i < CPL; i += 4)
                    *(f32x4 *)(p.Y + (size_t)m * p.ldy + oc + i) = (f32x4){v[c][i], v[c][i + 1], v[c][i + 2], v[c][i + 3]};
            }
        }
    }
}

// f32 epilogue straight from the accumulator registers: buffer stores whose row step is a scalar
// offset; rows past M fall outside the descriptor's range and are dropped, columns past N masked
template <int POST, bool FAST, bool NT = false>
__device__ __attribute__((always_inline)) inline void p_epilogue_f32(const GemmArgs &p, float (&f)[4][16],
                                                                     const float (&wsr)[4], int m0, int n0,
                                                                     int wm, int wn, int lane) {
    const __amdgpu_buffer_rsrc_t ry =
        __builtin_amdgcn_make_buffer_rsrc(p.Y, 0, (int)min((long)p.M * p.ldy * 4, 0x7fffffffL), 0x00020000);
    const int vrow = wm * 32 + (lane >> 5) * 4, vcol = wn * 128 + (lane & 31);
    const int voff = ((m0 + vrow) * p.ldy + n0 + vcol) * 4;
#pragma unroll
    for (int tn = 0; tn < 4; tn++) {
        const int n = n0 + vcol + tn * 32;
        if (n >= p.N) continue;
        const float b = ((POST & 1) && p.bias) ? p.bias[n] : 0.f;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            float v = f[tn][r];
            if constexpr (FAST) v = __fmul_rn(v, wsr[tn]);
            if constexpr (POST & 1) v = v + b;
            if constexpr (POST & 2) v = fminf(fmaxf(v, p.lo), p.hi);
            const int srow = __builtin_amdgcn_readfirstlane(((r >> 2) * 8 + (r & 3)) * p.ldy * 4);
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), ry, voff + tn * 128, srow,
                                                  NT ? kStoreNT : 0);
        }
    }
}

// the value of lane l ^ X (X <= 16, so within the lane's 32-lane half) by VALU lane exchanges
// (xor_lane: DPP, gfx950's permlane16 swap), not a ds_swizzle through the LDS unit, whose
// latency and wait the halving reductions below paid at every step
template <int X>
__device__ inline float swz_xor(float v) {
    static_assert(X >= 1 && X <= 16, "within a 32-lane half");
    return xor_lane<X>(v);
}
// one halving step of a transposing reduction over lanes: 2N partial sums -> N, the lanes with
// bit X set keeping the upper half (each gives away the half it does not keep)
template <int X, int N>
__device__ inline void halve(const float (&v)[2 * N], float (&o)[N], bool up) {
#pragma unroll
    for (int i = 0; i < N; i++) {
        const float keep = up ? v[i + N] : v[i], give = up ? v[i] : v[i + N];
        o[i] = keep + swz_xor<X>(give);
    }
}
// f16 of an f32 value that is already rounded (the register barrier keeps the compiler from
// folding the multiply that produced x into the conversion)
__device__ inline uint16_t f2h_rn(float x) {
    asm volatile("" : "+v"(x));
    return __builtin_bit_cast(uint16_t, (_Float16)x);
}
__device__ inline float rms_inv256(float ss, float eps) {
    return __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, 256.0f) + eps));
}

// The q|k|v epilogue (EPI_QKV) of a 128 x 256 tile, which is one head of 128 rows: 8 waves, wave
// (wm, wn) holding rows wm * 32 .. + 31 and W rows wn * 128 .. + 127 of the head. W's rows of each
// 256-row head are stored with bits 6 and 7 of the row index swapped, so that wave wn's column tile
// t (lane column c) is head dimension (t >> 1) * 128 + wn * 64 + (t & 1) * 32 + c: the rotate-half
// partners i and i + 128 of RoPE sit in tiles t and t + 2 of the same lane.
//  1. the row's sum of squares: per lane over its 4 tiles, over the 32 lanes of each half by a
//     transposing halving exchange (16 values -> 1 in four swizzle steps, then the pair), and over
//     the two waves of the head through LDS (one barrier);
//  2. inv = 1 / sqrt(ss / 256 + eps) (the row kernel's arithmetic), shared through LDS per wave;
//  3. q/k: x = (y * inv) * gamma, then a' = a c - b s, b' = b c + a s (products rounded, then the
//     sum; kernels.c:112-126), f16; v: y * inv, f16, stored transposed per sequence.
// scr: 3 x 8 x 32 words of the step's free A|W stage (partial sums, inverse rms, positions).
// k_gemm_p's arguments as laid out in its kernel-argument segment: the device row count's pointer
// first (preloaded into SGPRs: gemm.hip is built with -amdgpu-kernarg-preload-count=2, so the count
// is loaded at once instead of after the argument segment), then the GemmArgs.
struct PArgsLayout {
    const int *rows;
    GemmArgs p;
};
// The kernel's own GemmArgs, read through a pointer the compiler cannot follow back to the kernel's
// entry: the fields read through it are loaded (s_load) where they are used instead of being held
// in SGPRs across the K loop. The fused q|k|v kernel needs eleven pointers and five scalars in its
// epilogue only; held for the whole kernel they pushed it past the SGPR file (41 SGPRs spilled).
typedef const __attribute__((address_space(4))) GemmArgs *KernArgs;
__device__ __attribute__((always_inline)) inline KernArgs kernel_args() {
    KernArgs a = (KernArgs)((const __attribute__((address_space(4))) char *)__builtin_amdgcn_kernarg_segment_ptr() +
                            offsetof(PArgsLayout, p));
    asm volatile("" : "+s"(a));
    return a;
}

template <bool FAST>
__device__ __attribute__((always_inline)) inline void p_epilogue_qkv(KernArgs pa, float (&f)[4][16],
                                                                     const float (&wsr)[4], int m0, int n0,
                                                                     int wave, int wm, int wn, int lane,
                                                                     float *scr) {
    const KernArgs p = pa;
    if constexpr (FAST) {
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int r = 0; r < 16; r++) f[t][r] = __fmul_rn(f[t][r], wsr[t]);
    }
    const int hd = n0 >> 8, nqk = p->qH + p->qKV;
    const int hh = lane >> 5, c = lane & 31;
    // 1. register r = 4 g + j holds row 8 g + 4 hh + j of the wave's 32
    float s16[16], s8[8], s4[4], s2[2], s1[1];
#pragma unroll
    for (int r = 0; r < 16; r++) {
        float a = __fmul_rn(f[0][r], f[0][r]);
#pragma unroll
        for (int t = 1; t < 4; t++) a = a + __fmul_rn(f[t][r], f[t][r]);
        s16[r] = a;
    }
    halve<16, 8>(s16, s8, lane & 16);
    halve<8, 4>(s8, s4, lane & 8);
    halve<4, 2>(s4, s2, lane & 4);
    halve<2, 1>(s2, s1, lane & 2);
    const float part = s1[0] + swz_xor<1>(s1[0]);
    const int j = ((lane >> 4) & 1) * 8 + ((lane >> 3) & 1) * 4 + ((lane >> 2) & 1) * 2 + ((lane >> 1) & 1);
    const int rw = 8 * (j >> 2) + 4 * hh + (j & 3);
    float *xs = scr, *xi = scr + 8 * 32;
    if ((lane & 1) == 0) xs[wave * 32 + rw] = part;
    __syncthreads();
    // 2. the two waves add the same two partial sums (addition commutes: both get the same inv)
    const float inv = rms_inv256(part + xs[(wm * 2 + (wn ^ 1)) * 32 + rw], p->eps);
    if ((lane & 1) == 0) xi[wave * 32 + rw] = inv;
    // 3. four rows at a time (registers 4 g .. 4 g + 3, rows rb + 8 g + 0..3), their inv read back
    // from LDS (LDS operations of one wave complete in order: the reads see this wave's writes);
    // buffer stores whose range ends at row M drop the rows past it
    const int rb = m0 + wm * 32 + 4 * hh;
    typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
    if (hd < nqk) {
        const bool isq = hd < p->qH;
        const int hq = isq ? hd : hd - p->qH, ld = (isq ? p->qH : p->qKV) * 256;
        const float *gam = isq ? p->q_gamma : p->k_gamma;
        const __amdgpu_buffer_rsrc_t r16 =
            __builtin_amdgcn_make_buffer_rsrc(isq ? p->q16 : p->k16, 0, (int)min((long)p->M * ld * 2, 0x7fffffffL), 0x00020000);
        float *o32 = isq ? p->q32 : p->k32;
        const __amdgpu_buffer_rsrc_t r32 =
            __builtin_amdgcn_make_buffer_rsrc(o32, 0, o32 ? (int)min((long)p->M * ld * 4, 0x7fffffffL) : 0, 0x00020000);
        const int i0 = wn * 64 + c;  // tiles t = 0, 1: dimensions i0 + 32 t and i0 + 32 t + 128
        const float g00 = gam[i0], g01 = gam[i0 + 128], g10 = gam[i0 + 32], g11 = gam[i0 + 160];
        // the 16 rows' positions, then per group of 4 rows its 16 table entries, each batch of
        // loads issued before any is used (every wait here also waits for the K loop's loads in
        // flight, so one wait per batch rather than per value)
        // the wave's 32 row positions go through LDS (lane l < 32: row wm * 32 + l)
        int *xp = (int *)(scr + 2 * 8 * 32) + wave * 32;
        if (lane < 32) {
            const int m = min(m0 + wm * 32 + lane, p->M - 1);
            xp[lane] = p->pos ? p->pos[m] : m % p->qS;
        }
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int4 p4 = *(const int4 *)(xp + 8 * g + 4 * hh);
            const int pg[4] = {p4.x, p4.y, p4.z, p4.w};
            float cv[4][2], sv[4][2];
#pragma unroll
            for (int jj = 0; jj < 4; jj++)
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const size_t e = (size_t)pg[jj] * 256 + i0 + 32 * t;
                    cv[jj][t] = p->cs[e];
                    sv[jj][t] = p->sn[e];
                }
            const float4 i4 = *(const float4 *)(xi + wave * 32 + 8 * g + 4 * hh);
            const float ivg[4] = {i4.x, i4.y, i4.z, i4.w};
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const int r = 4 * g + jj, m = rb + 8 * g + jj;
                const int o = (m * ld + hq * 256 + i0) * 2;
                uint32_t lo16[2], hi16[2];
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const float a = __fmul_rn(__fmul_rn(f[t][r], ivg[jj]), t ? g10 : g00);
                    const float b = __fmul_rn(__fmul_rn(f[t + 2][r], ivg[jj]), t ? g11 : g01);
                    const float lo = __fmul_rn(a, cv[jj][t]) - __fmul_rn(b, sv[jj][t]);
                    const float hi = __fmul_rn(b, cv[jj][t]) + __fmul_rn(a, sv[jj][t]);
                    lo16[t] = f2h_rn(lo);
                    hi16[t] = f2h_rn(hi);
                    if (o32) {
                        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, lo), r32, 2 * o + 128 * t, 0, 0);
                        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, hi), r32, 2 * o + 128 * t + 512, 0, 0);
                    }
                }
                // lanes 0-31 hold row m0' = rb - 4 hh's columns i0 and i0 + 32, lanes 32-63 row m0' + 4's:
                // one lane swap between the halves gives each store one row's 64 consecutive
                // columns (a whole 128-byte line) instead of half lines of two rows
                const int o0 = ((m0 + wm * 32 + 8 * g + jj) * ld + hq * 256 + wn * 64 + lane) * 2;
                const auto sl = __builtin_amdgcn_permlane32_swap(lo16[0], lo16[1], false, false);
                const auto sh = __builtin_amdgcn_permlane32_swap(hi16[0], hi16[1], false, false);
                __builtin_amdgcn_raw_buffer_store_b16((uint16_t)sl[0], r16, o0, 0, 0);
                __builtin_amdgcn_raw_buffer_store_b16((uint16_t)sl[1], r16, o0 + 8 * ld, 0, 0);
                __builtin_amdgcn_raw_buffer_store_b16((uint16_t)sh[0], r16, o0 + 256, 0, 0);
                __builtin_amdgcn_raw_buffer_store_b16((uint16_t)sh[1], r16, o0 + 8 * ld + 256, 0, 0);
            }
        }
    } else {
        const int vh = hd - nqk, S = p->qS, ld32 = p->qKV * 256;
        const bool fast = S % 4 == 0;
        float *o32 = p->v32;
        const __amdgpu_buffer_rsrc_t r32 =
            __builtin_amdgcn_make_buffer_rsrc(o32, 0, o32 ? (int)min((long)p->M * ld32 * 4, 0x7fffffffL) : 0, 0x00020000);
        if (S % 128 == 0 && ((uintptr_t)p->vt16 & 15) == 0) {
            // the tile's 128 rows are 128 consecutive positions of one sequence, contiguous in each
            // dimension's V^T row: the f16 values go through LDS as [dimension][position] (pitch
            // 272 bytes, two passes of 128 dimensions in the consumed stage past the 3 KB of the
            // steps above), and each dimension's 256 bytes are written as 16 lane stores of 16
            // bytes (whole lines; the direct stores were 8 bytes a lane, one line each)
            constexpr int VP = 272;
            unsigned char *stg = (unsigned char *)scr + 4096;
            uint16_t *vrow = p->vt16 + (size_t)((m0 / S) * p->qKV + vh) * 256 * S + m0 % S;
            const int tid = wave * 64 + lane;
#pragma unroll
            for (int pass = 0; pass < 2; pass++) {
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const float4 i4 = *(const float4 *)(xi + wave * 32 + 8 * g + 4 * hh);
                    const float ivg[4] = {i4.x, i4.y, i4.z, i4.w};
                    const int m = rb + 8 * g;
#pragma unroll
                    for (int t = 2 * pass; t < 2 * pass + 2; t++) {
                        const int dl = wn * 64 + (t & 1) * 32 + c;
                        float x[4];
#pragma unroll
                        for (int jj = 0; jj < 4; jj++) x[jj] = __fmul_rn(f[t][4 * g + jj], ivg[jj]);
                        *(u32x2v *)(stg + dl * VP + (wm * 32 + 8 * g + 4 * hh) * 2) =
                            (u32x2v){(uint32_t)f2h_rn(x[0]) | ((uint32_t)f2h_rn(x[1]) << 16),
                                     (uint32_t)f2h_rn(x[2]) | ((uint32_t)f2h_rn(x[3]) << 16)};
                        if (o32) {
                            const int d = (t >> 1) * 128 + dl;
#pragma unroll
                            for (int jj = 0; jj < 4; jj++)
                                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, x[jj]), r32,
                                                                      ((m + jj) * ld32 + vh * 256 + d) * 4, 0, 0);
                        }
                    }
                }
                asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
                for (int rnd = 0; rnd < 4; rnd++) {
                    const int dl = rnd * 32 + (tid >> 4), ch = tid & 15, mm = m0 + 8 * ch;
                    const uint4 v = *(const uint4 *)(stg + dl * VP + ch * 16);
                    uint16_t *dst = vrow + (size_t)(128 * pass + dl) * S + 8 * ch;
                    if (mm + 8 <= p->M) {
                        *(uint4 *)dst = v;
                    } else {
                        const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                        for (int e = 0; e < 8; e++)
                            if (mm + e < p->M) dst[e] = (uint16_t)(w4[e >> 1] >> (16 * (e & 1)));
                    }
                }
                // every wave's reads of this pass before the next pass overwrites the staging
                asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            }
            return;
        }
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const float4 i4 = *(const float4 *)(xi + wave * 32 + 8 * g + 4 * hh);
            const float ivg[4] = {i4.x, i4.y, i4.z, i4.w};
            const int m = rb + 8 * g;  // rows m .. m + 3, m a multiple of 4
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int d = (t >> 1) * 128 + wn * 64 + (t & 1) * 32 + c;
                float x[4];
#pragma unroll
                for (int jj = 0; jj < 4; jj++) x[jj] = __fmul_rn(f[t][4 * g + jj], ivg[jj]);
                if (fast && m + 3 < p->M) {
                    // four consecutive positions of one sequence: one 8-byte store
                    uint16_t *dst = p->vt16 + ((size_t)((m / S) * p->qKV + vh) * 256 + d) * S + m % S;
                    *(u32x2v *)dst = (u32x2v){(uint32_t)f2h_rn(x[0]) | ((uint32_t)f2h_rn(x[1]) << 16),
                                              (uint32_t)f2h_rn(x[2]) | ((uint32_t)f2h_rn(x[3]) << 16)};
                } else {
#pragma unroll
                    for (int jj = 0; jj < 4; jj++) {
                        const int mm = m + jj;
                        if (mm < p->M)
                            p->vt16[((size_t)((mm / S) * p->qKV + vh) * 256 + d) * S + mm % S] = f2h_rn(x[jj]);
                    }
                }
                if (o32) {
#pragma unroll
                    for (int jj = 0; jj < 4; jj++)
                        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, x[jj]), r32,
                                                              ((m + jj) * ld32 + vh * 256 + d) * 4, 0, 0);
                }
            }
        }
    }
}

// 8 waves of 32 x 128 (one 32-row MFMA tile by four 32-column ones): NWM x NWN waves, BM = 32 NWM,
// BN = 128 NWN
template <int BM, int BN, int NWM, int NWN, int EPI, bool FAST, int POST, bool NT = false>
__global__ __launch_bounds__(NWM * NWN * 64, 8 / (NWM * NWN)) void k_gemm_p(const int *rows, GemmArgs p, int tiles_n,
                                                                               int tiles) {
    constexpr int NWAVE = NWM * NWN;
    static_assert(BM == 32 * NWM && BN == 128 * NWN && (NWAVE == 8 || NWAVE == 4), "8 or 4 waves of 32x128");
    constexpr int kPStages = p_stages<NWAVE>(), AHEAD = kPStages - 1;  // loads AHEAD steps ahead
    constexpr int AI = BM / 8 / NWAVE, BI = BN / 8 / NWAVE;  // 1-KB loads per wave per step
    constexpr int L = AI + BI + 2;                           // loads per wave per step
    constexpr int TILE = (BM + BN) * 128;                    // A | W of one step
    constexpr int SHALF = 64 * NWAVE * 4;                    // as of one step (one per lane)
    constexpr int SSLOT = 2 * SHALF;                         // as | ws
    constexpr bool XACT = !FAST;
    extern __shared__ __align__(16) unsigned char smem[];
    unsigned char *const sscale = smem + kPStages * TILE;

    if (rows) {
        // a forward planned on the device: its row count, a multiple of 256, from device memory; the
        // host M sized the grid and, in the q|k|v epilogue (which reads the kernel's arguments
        // again), bounds the stores of tiles that all lie below this count
        p.M = min(p.M, *rows);
        tiles = (p.M + BM - 1) / BM * tiles_n;
    }
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / NWN, wn = wave % NWN;
    const int nb = p.K / kQBlock;   // K steps per tile
    const int nsb = nb;             // activation scales per row

    // this workgroup's tiles: chunk [c0, c1) of the tile list, every per-th tile from c0 + li
    const int nx = (gridDim.x % 8 == 0) ? 8 : 1;
    const int grp = blockIdx.x % nx, li = blockIdx.x / nx, per = gridDim.x / nx;
    const int c0 = (int)((long)tiles * grp / nx), c1 = (int)((long)tiles * (grp + 1) / nx);
    const int ntile = (c1 - c0 > li) ? (c1 - c0 - li + per - 1) / per : 0;
    const int G = ntile * nb;  // K steps of this workgroup
    auto tile_m0 = [&](int j) { return ((c0 + li + j * per) / tiles_n) * BM; };
    auto tile_n0 = [&](int j) { return ((c0 + li + j * per) % tiles_n) * BN; };

    const v4u rA = rsrc_words(p.A, (uint32_t)((size_t)p.M * p.lda));
    const v4u rW = rsrc_words(p.W, (uint32_t)((size_t)p.N * p.ldw));
    const v4u rS = rsrc_words(p.as, (uint32_t)((size_t)p.M * nsb * 4));
    const v4u rV = rsrc_words(p.ws, (uint32_t)((size_t)p.N * 4));
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const lds_void *)smem);

    // loads of flat step g (tile j, block kb) into stage g % stages and slot g % 4. Load i of a wave
    // fills rows (i * NWAVE + wave) * 8 + lane / 8 of the tile, 16-byte chunk (lane % 8) ^ swzk(row);
    // with 8 or 4 waves swzk(row) = (wave % 2) * 4 + (lane / 16) % 4 for every i, so one per-lane offset
    // per operand serves all loads and the row base is a scalar. Rows past M (N) lie past the
    // buffer's range and read as zero; their outputs are never stored. The slot gets the step's
    // activation scales and its tile's ws (waves past BM/64 or BN/64 fetch a copy of the last 64).
    const int swl = ((lane & 7) ^ ((wave & 1) * 4 + ((lane >> 4) & 3))) << 4;
    const uint32_t vla = (uint32_t)(lane >> 3) * (uint32_t)p.lda + swl;
    const uint32_t vlb = (uint32_t)(lane >> 3) * (uint32_t)p.ldw + swl;
    const uint32_t vls = (uint32_t)lane * (uint32_t)nsb * 4;
    int ij = 0, ikb = 0;  // next step to issue
    // a step's 8 loads per wave (AI of A, BI of W, as, ws) in 4 parts of 2, so that issuing them is
    // spread over the step's MFMAs: issuing all at once stalls the wave on the vector-memory path
    struct Issue {
        uint32_t st, sl, ko, ks;
        int m0, n0;
    };
    auto issue_prep = [&](int g) {
        Issue is;
        is.m0 = tile_m0(ij);
        is.n0 = tile_n0(ij);
        is.st = lds0 + (uint32_t)((g % kPStages) * TILE);
        is.sl = lds0 + (uint32_t)(kPStages * TILE + (g % kPSlots) * SSLOT + wave * 256);
        is.ko = (uint32_t)(ikb * kQBlock);
        is.ks = (uint32_t)(ikb * 4);
        if (++ikb == nb) {
            ikb = 0;
            ++ij;
        }
        return is;
    };
    constexpr int WAITN = (AHEAD - 1) * L;  // loads issued after a step's own, when it starts
    auto issue_load = [&](const Issue &is, int i) {
        if (i < AI)
            dma16(rA, is.st + (i * NWAVE + wave) * 1024,
                  vla + (uint32_t)(is.m0 + (i * NWAVE + wave) * 8) * (uint32_t)p.lda, is.ko);
        else if (i < AI + BI)
            dma16(rW, is.st + BM * 128 + ((i - AI) * NWAVE + wave) * 1024,
                  vlb + (uint32_t)(is.n0 + ((i - AI) * NWAVE + wave) * 8) * (uint32_t)p.ldw, is.ko);
        else if (i == AI + BI)
            dma4(rS, is.sl, vls + (uint32_t)(is.m0 + min(wave * 64, BM - 64)) * (uint32_t)nsb * 4, is.ks);
        else
            dma4(rV, is.sl + SHALF, (uint32_t)(is.n0 + min(wave * 64, BN - 64) + lane) * 4, 0);
    };
    auto issue_part = [&](const Issue &is, int part) {
#pragma unroll
        for (int i = part * L / 4; i < (part + 1) * L / 4; i++) issue_load(is, i);
    };
    auto issue_next = [&](int g) {
        const Issue is = issue_prep(g);
#pragma unroll
        for (int q = 0; q < 4; q++) issue_part(is, q);
    };

    // the fold of "step -1" (zero accumulators) reads slot 3, which must hold finite scales; it is
    // not loaded before step 1, after that fold (the barrier of step 0 publishes the zeros)
    for (int i = tid; i < SSLOT / 16; i += NWAVE * 64)
        ((uint4 *)(sscale + (kPSlots - 1) * SSLOT))[i] = make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int a = 0; a < AHEAD; a++)
        if (G > a) issue_next(a);

    // ws of this lane's four columns, read from a slot's ws half
    float wsr[4];
    auto read_ws = [&](const unsigned char *slot) {
#pragma unroll
        for (int tn = 0; tn < 4; tn++)
            wsr[tn] = *(const float *)(slot + SHALF + (wn * 128 + tn * 32 + (lane & 31)) * 4);
    };

    float f[4][16];
#pragma unroll
    for (int tn = 0; tn < 4; tn++)
#pragma unroll
        for (int r = 0; r < 16; r++) f[tn][r] = 0.f;
    v16i acc0[4], acc1[4];
#pragma unroll
    for (int tn = 0; tn < 4; tn++) acc1[tn] = (v16i){};

    // per-lane fragment offsets inside a stage: row (lane % 32) of a 32-row tile, 16-byte chunk
    // 2 kk + lane / 32; the XOR swizzle depends only on the row within 16, so one offset per kk
    // serves every tile (W tile t adds t * 4096 as an immediate)
    int offa[4], offb[4];
#pragma unroll
    for (int kk = 0; kk < 4; kk++) {
        const int o = swz(lane & 31, kk * 2 + (lane >> 5));
        offa[kk] = wm * 32 * 128 + o;
        offb[kk] = BM * 128 + wn * 128 * 128 + o;
    }
    const int offs = (wm * 32 + (lane >> 5) * 4) * 4;

    // fold unit u (4 elements): tile tn = u % 4, registers 4q..4q+3 with q = u / 4
    auto fold_unit = [&](const v16i (&acc)[4], int u, const float *sslot) {
        const int tn = u % 4, q = u / 4;
        const float4 a4 = *(const float4 *)((const unsigned char *)sslot + offs + q * 32);
        const float av[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r = q * 4 + j;
            // the reference's order: f = fma((float)acc, RN(as * ws), f); FAST folds as only and
            // multiplies by ws once in the epilogue
            f[tn][r] = __builtin_fmaf((float)acc[tn][r], XACT ? __fmul_rn(av[j], wsr[tn]) : av[j], f[tn][r]);
        }
    };
    const v16i zero = {};
    int cj = 0, ckb = 0;  // tile / block of the step being computed
    // one K step: MFMAs of step g into cur, interleaved with the fold of prev (step g-1), and the
    // loads of step g + 2 issued 2 per K sub-step (past the end of the list they fetch rows beyond
    // the operands' range into stages no longer read, which is harmless)
    auto step = [&](int g, v16i (&cur)[4], const v16i (&prev)[4]) {
        if (g + 1 < G) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(WAITN) : "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        const bool tile_start = ckb == 0 && g > 0;  // prev is the previous tile's last step
        const Issue is_next = issue_prep(g + AHEAD);
        const unsigned char *sb = smem + (g % kPStages) * TILE;
        const unsigned char *spb = sscale + ((g + kPSlots - 1) % kPSlots) * SSLOT;
        const float *sp = (const float *)spb;
        read_ws(spb);  // the folded step's tile
        // The A fragment and the first W fragment of sub-step kk + 1 are read during sub-step kk,
        // so its first MFMA does not wait for a fresh LDS read; each fold unit's VALU work comes
        // before its MFMA and covers the remaining reads' latency (C5 sweep and encoder shapes:
        // 4-5 % faster than reading every fragment at the sub-step's start and folding after the
        // MFMA). The fused q|k|v epilogue keeps the plain order: its registers leave no room for
        // the 8 extra fragment registers.
        constexpr bool PREF = EPI != EPI_QKV;
        v4i apf[2], bpf[2];
        if constexpr (PREF) {
            apf[0] = *(const v4i *)(sb + offa[0]);
            bpf[0] = *(const v4i *)(sb + offb[0]);
        }
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            issue_part(is_next, kk);
            v4i af, bf[4];
            if constexpr (PREF) {
                af = apf[kk & 1];
                bf[0] = bpf[kk & 1];
#pragma unroll
                for (int t = 1; t < 4; t++) bf[t] = *(const v4i *)(sb + offb[kk] + t * 4096);
                if (kk < 3) {
                    apf[(kk + 1) & 1] = *(const v4i *)(sb + offa[kk + 1]);
                    bpf[(kk + 1) & 1] = *(const v4i *)(sb + offb[kk + 1]);
                }
            } else {
                af = *(const v4i *)(sb + offa[kk]);
#pragma unroll
                for (int t = 0; t < 4; t++) bf[t] = *(const v4i *)(sb + offb[kk] + t * 4096);
            }
#pragma unroll
            for (int tn = 0; tn < 4; tn++)
                cur[tn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bf[tn], kk == 0 ? zero : cur[tn], 0, 0, 0);
#pragma unroll
            for (int u = kk * 4; u < kk * 4 + 4; u++) fold_unit(prev, u, sp);
            // 5 fragment reads + 1 scale read, then per MFMA its fold unit (before it when PREF)
            __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                if constexpr (PREF) {
                    __builtin_amdgcn_sched_group_barrier(0x002, XACT ? 12 : 8, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                } else {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, XACT ? 12 : 8, 0);
                }
            }
        }
        if (tile_start) {
            // the previous tile is complete: its epilogue, then a fresh f. A requantizing epilogue
            // stages through this step's A|W stage once every wave is done with it; the stage is
            // refilled only by the next step's loads, issued after that step's barrier.
            const int pm0 = tile_m0(cj - 1), pn0 = tile_n0(cj - 1);
            if constexpr (EPI == EPI_F32) {
                p_epilogue_f32<POST, FAST, NT>(p, f, wsr, pm0, pn0, wm, wn, lane);
            } else if constexpr (EPI == EPI_QKV) {
                __syncthreads();
                p_epilogue_qkv<FAST>(kernel_args(), f, wsr, pm0, pn0, wave, wm, wn, lane,
                                     (float *)(smem + (g % kPStages) * TILE));
            } else {
                __syncthreads();
                p_epilogue_q<BM, BN, NWM, NWN, EPI, FAST, POST, NT>(p, f, wsr, pm0, pn0, wave, wm, wn, lane,
                                                                (float *)(smem + (g % kPStages) * TILE));
            }
#pragma unroll
            for (int tn = 0; tn < 4; tn++)
#pragma unroll
                for (int r = 0; r < 16; r++) f[tn][r] = 0.f;
        }
        if (++ckb == nb) {
            ckb = 0;
            ++cj;
        }
    };
    int g = 0;
    for (; g + 1 < G; g += 2) {
        step(g, acc0, acc1);
        step(g + 1, acc1, acc0);
    }
    if (g < G) step(g, acc0, acc1);
    if (G > 0) {
        // fold the last step (acc0 when G is odd) and write the last tile
        __syncthreads();
        const float *sp = (const float *)(sscale + ((G - 1) % kPSlots) * SSLOT);
        read_ws((const unsigned char *)sp);
        // (two branches: selecting one of the register arrays at run time would put it in memory)
        if (G & 1) {
#pragma unroll
            for (int u = 0; u < 16; u++) fold_unit(acc0, u, sp);
        } else {
#pragma unroll
            for (int u = 0; u < 16; u++) fold_unit(acc1, u, sp);
        }
        const int pm0 = tile_m0(ntile - 1), pn0 = tile_n0(ntile - 1);
        if constexpr (EPI == EPI_F32)
            p_epilogue_f32<POST, FAST, NT>(p, f, wsr, pm0, pn0, wm, wn, lane);
        else if constexpr (EPI == EPI_QKV)
            p_epilogue_qkv<FAST>(kernel_args(), f, wsr, pm0, pn0, wave, wm, wn, lane,
                                 (float *)(smem + ((G - 1) % kPStages) * TILE));
        else
            p_epilogue_q<BM, BN, NWM, NWN, EPI, FAST, POST, NT>(p, f, wsr, pm0, pn0, wave, wm, wn, lane,
                                                            (float *)(smem + ((G - 1) % kPStages) * TILE));
    }
    // the last steps issued loads past the end of the list: they must land before the workgroup's
    // LDS is released
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Per-token GEMM with 64 x 128 wave tiles: 8 waves (4 x 2) of a 256 x 256 output tile, two A|W
// stages of 64 KB, loads one step ahead. Per 32-deep K sub-step a wave reads 6 fragments (2 of A,
// 4 of W) for 8 MFMAs, half the LDS bytes per MFMA of the 32 x 128 wave tile, and the next
// sub-step's fragments are read while the current ones feed the MFMAs. With one scale per row the
// int32 accumulators run over the whole K of a tile (no per-step fold); the tile's last step folds
// them, f = fma((float)acc, RN(as[m] * ws[n]), 0), and runs the epilogue, one 32-row half at a time.
template <int EPI, int POST>
__global__ __launch_bounds__(512, 1) void k_gemm_t(GemmArgs p, int tiles_n, int tiles) {
    constexpr int BM = 256, BN = 256, NWM = 4, NWN = 2, NWAVE = 8, STAGES = 2;
    constexpr int AI = BM / 8 / NWAVE, BI = BN / 8 / NWAVE;  // 1-KB loads per wave per step
    constexpr int L = AI + BI + 2;                           // loads per wave per step
    constexpr int TILE = (BM + BN) * 128;                    // A | W of one step
    constexpr int SHALF = 64 * NWAVE * 4;                    // as of one step (one per lane)
    constexpr int SSLOT = 2 * SHALF;                         // as | ws
    extern __shared__ __align__(16) unsigned char smem[];
    unsigned char *const sscale = smem + STAGES * TILE;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / NWN, wn = wave % NWN;
    const int nb = p.K / kQBlock;

    const int nx = (gridDim.x % 8 == 0) ? 8 : 1;
    const int grp = blockIdx.x % nx, li = blockIdx.x / nx, per = gridDim.x / nx;
    const int c0 = (int)((long)tiles * grp / nx), c1 = (int)((long)tiles * (grp + 1) / nx);
    const int ntile = (c1 - c0 > li) ? (c1 - c0 - li + per - 1) / per : 0;
    const int G = ntile * nb;
    auto tile_m0 = [&](int j) { return ((c0 + li + j * per) / tiles_n) * BM; };
    auto tile_n0 = [&](int j) { return ((c0 + li + j * per) % tiles_n) * BN; };

    const v4u rA = rsrc_words(p.A, (uint32_t)((size_t)p.M * p.lda));
    const v4u rW = rsrc_words(p.W, (uint32_t)((size_t)p.N * p.ldw));
    const v4u rS = rsrc_words(p.as, (uint32_t)((size_t)p.M * 4));
    const v4u rV = rsrc_words(p.ws, (uint32_t)((size_t)p.N * 4));
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const lds_void *)smem);

    // load i of a wave fills rows (i * NWAVE + wave) * 8 + lane / 8 of the tile (as in k_gemm_p);
    // the slot gets the tile's activation scales (rows min(64 wave, BM - 64) + lane) and weight
    // scales, loaded with every step of the tile and read at its last
    const int swl = ((lane & 7) ^ ((wave & 1) * 4 + ((lane >> 4) & 3))) << 4;
    const uint32_t vla = (uint32_t)(lane >> 3) * (uint32_t)p.lda + swl;
    const uint32_t vlb = (uint32_t)(lane >> 3) * (uint32_t)p.ldw + swl;
    int ij = 0, ikb = 0;
    struct Issue {
        uint32_t st, sl, ko;
        int m0, n0;
    };
    auto issue_prep = [&](int g) {
        Issue is;
        is.m0 = tile_m0(ij);
        is.n0 = tile_n0(ij);
        is.st = lds0 + (uint32_t)((g % STAGES) * TILE);
        is.sl = lds0 + (uint32_t)(STAGES * TILE + (g % kPSlots) * SSLOT + wave * 256);
        is.ko = (uint32_t)(ikb * kQBlock);
        if (++ikb == nb) {
            ikb = 0;
            ++ij;
        }
        return is;
    };
    auto issue_load = [&](const Issue &is, int i) {
        if (i < AI)
            dma16(rA, is.st + (i * NWAVE + wave) * 1024,
                  vla + (uint32_t)(is.m0 + (i * NWAVE + wave) * 8) * (uint32_t)p.lda, is.ko);
        else if (i < AI + BI)
            dma16(rW, is.st + BM * 128 + ((i - AI) * NWAVE + wave) * 1024,
                  vlb + (uint32_t)(is.n0 + ((i - AI) * NWAVE + wave) * 8) * (uint32_t)p.ldw, is.ko);
        else if (i == AI + BI)
            dma4(rS, is.sl, (uint32_t)(is.m0 + min(wave * 64, BM - 64) + lane) * 4, 0);
        else
            dma4(rV, is.sl + SHALF, (uint32_t)(is.n0 + min(wave * 64, BN - 64) + lane) * 4, 0);
    };
    auto issue_part = [&](const Issue &is, int part) {
#pragma unroll
        for (int i = part * L / 4; i < (part + 1) * L / 4; i++) issue_load(is, i);
    };
    if (G > 0) {
        const Issue is = issue_prep(0);
#pragma unroll
        for (int q = 0; q < 4; q++) issue_part(is, q);
    }

    // fragment offsets inside a stage (row lane % 32 of a 32-row tile, 16-byte chunk 2 kk + lane / 32);
    // A half h adds h * 4096, W tile t adds t * 4096
    int offa[4], offb[4];
#pragma unroll
    for (int kk = 0; kk < 4; kk++) {
        const int o = swz(lane & 31, kk * 2 + (lane >> 5));
        offa[kk] = wm * 64 * 128 + o;
        offb[kk] = BM * 128 + wn * 128 * 128 + o;
    }
    v16i acc[2][4];
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int t = 0; t < 4; t++) acc[h][t] = (v16i){};

    int cj = 0, ckb = 0;
    for (int g = 0; g < G; g++) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        // the next step's loads go to the other stage, consumed by the previous step (past the end
        // of the list they fetch rows beyond the operands' range into a stage no longer read)
        const Issue is_next = issue_prep(g + 1);
        const unsigned char *sb = smem + (g % STAGES) * TILE;
        v4i af[2][2], bf[2][4];
        auto frags = [&](int kk, v4i (&a)[2], v4i (&b)[4]) {
#pragma unroll
            for (int h = 0; h < 2; h++) a[h] = *(const v4i *)(sb + offa[kk] + h * 4096);
#pragma unroll
            for (int t = 0; t < 4; t++) b[t] = *(const v4i *)(sb + offb[kk] + t * 4096);
        };
        frags(0, af[0], bf[0]);
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            const int c = kk & 1;
            if (kk < 3) frags(kk + 1, af[c ^ 1], bf[c ^ 1]);
            issue_part(is_next, kk);
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int t = 0; t < 4; t++)
                    acc[h][t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[c][h], bf[c][t], acc[h][t], 0, 0, 0);
        }
        if (++ckb == nb) {
            const unsigned char *slot = sscale + (g % kPSlots) * SSLOT;
            float wsr[4];
#pragma unroll
            for (int tn = 0; tn < 4; tn++)
                wsr[tn] = *(const float *)(slot + SHALF + (wn * 128 + tn * 32 + (lane & 31)) * 4);
            const int pm0 = tile_m0(cj), pn0 = tile_n0(cj);
            // a requantizing epilogue stages through this step's stage once every wave is done
            // with it; the stage is refilled only by the loads issued after the next barrier
            if constexpr (EPI != EPI_F32) __syncthreads();
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int wmh = wm * 2 + h;  // the 32-row wave row of the epilogue
                float f[4][16];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float4 a4 = *(const float4 *)(slot + (wmh * 32 + (lane >> 5) * 4 + q * 8) * 4);
                    const float av[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
                    for (int tn = 0; tn < 4; tn++)
#pragma unroll
                        for (int j = 0; j < 4; j++)
                            f[tn][q * 4 + j] = __builtin_fmaf((float)acc[h][tn][q * 4 + j], __fmul_rn(av[j], wsr[tn]), 0.f);
                }
#pragma unroll
                for (int t = 0; t < 4; t++) acc[h][t] = (v16i){};
                if constexpr (EPI == EPI_F32)
                    p_epilogue_f32<POST, false, true>(p, f, wsr, pm0, pn0, wmh, wn, lane);
                else
                    p_epilogue_q<BM, BN, NWM, NWN, EPI, false, POST, true>(p, f, wsr, pm0, pn0, wave, wmh, wn, lane,
                                                                     (float *)(smem + (g % STAGES) * TILE));
            }
            ckb = 0;
            ++cj;
        }
    }
    // the last step issued loads past the end of the list: they must land before the workgroup's
    // LDS is released
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// ---------------------------------------------------------------------------------------------
// Per-token GEMM with the f32 epilogue overlapped (k_gemm_tv): the per-token f32 contract at
// K = 128 NB, N a multiple of 128, no bias or clamp (the config-5 sweep). Its time is the f32
// output's HBM write, so the design keeps that write stream running while the MFMAs go on:
//   - one 512-thread workgroup per CU, 8 waves (4 x 2) of 64 x 64 over a 256 x 128 output tile,
//     two waves per SIMD; each wave holds two accumulator sets of 2 x 2 v_mfma_i32_32x32x32_i8
//     tiles (128 registers): tile j's MFMAs accumulate into one set while the previous tile's
//     epilogue is converted and stored from the other, and the other wave of the SIMD covers the
//     fragment waits (one wave per SIMD with 64 x 128 waves, two sets of 256 registers, measured
//     3-6 % slower on the sweep);
//   - the M-major tile list cut into one contiguous chunk per XCD as in k_gemm_p (N = 1152 =
//     9 x 128 divides evenly);
//   - three 48 KB A|W stages, loads two steps ahead; the barrier sits after the third of a step's
//     four 32-deep sub-steps, once the step's last fragments are in registers, so the next step's
//     first fragments are read under the fourth sub-step's MFMAs;
//   - the loop is fully unrolled per tile into slots of one MFMA each (16 per step), fenced by
//     sched_barrier: a sub-step's four fragment reads (for the next sub-step) at its first slot,
//     one of the next-but-one step's 7 direct-to-LDS loads at each of the step's first 7 slots,
//     and the previous tile's 64 output elements per lane spread over the first NB - 1 steps, one
//     conversion fma((float)acc, RN(as * ws), 0) and one non-temporal dword store each (a store
//     writes two full 128-byte rows); stores and loads share the in-order vmcnt counter, so the
//     barrier's wait counts exactly the operations issued after the awaited loads.
namespace tv {
constexpr int BM = 256, BN = 128, NW = 8, STAGES = 3, NSLOT = 3;
constexpr int TILE = (BM + BN) * 128;
constexpr int SLOT = 2048;                     // as (256 floats) | ws (128 floats) of one tile
constexpr int LDS = STAGES * TILE + NSLOT * SLOT;
constexpr int L = BM / 8 / NW + BN / 8 / NW + 1;  // loads per wave per step: 4 A, 2 W, as or ws
constexpr int NMICRO = 64;                     // epilogue elements per lane and tile
constexpr int SPS = 16;                        // MFMA slots per step
static_assert(LDS <= 160 * 1024, "LDS budget");
template <int NB>
constexpr int micro_slot(int u) { return u * (SPS * (NB - 1)) / NMICRO; }
template <int NB>
constexpr int stores_in(int s0, int s1) {
    int n = 0;
    for (int u = 0; u < NMICRO; u++) n += (micro_slot<NB>(u) >= s0 && micro_slot<NB>(u) < s1) ? 1 : 0;
    return n;
}
}  // namespace tv

template <int NB>
__global__ __launch_bounds__(512, 1) void k_gemm_tv(GemmArgs p, int tiles_n, int tiles) {
    using namespace tv;
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int hi = lane >> 5, r32 = lane & 31;

    const int nx = (gridDim.x % 8 == 0) ? 8 : 1;
    const int grp = blockIdx.x % nx, li = blockIdx.x / nx, per = gridDim.x / nx;
    const int c0 = (int)((long)tiles * grp / nx), c1 = (int)((long)tiles * (grp + 1) / nx);
    const int ntile = (c1 - c0 > li) ? (c1 - c0 - li + per - 1) / per : 0;
    const int per_m = per / tiles_n, per_n = per % tiles_n;
    struct TC {
        int mb, nt;
    };
    auto tc_next = [&](TC t) {
        t.mb += per_m;
        t.nt += per_n;
        if (t.nt >= tiles_n) {
            t.nt -= tiles_n;
            t.mb += 1;
        }
        return t;
    };
    const TC tc0 = {(c0 + li) / tiles_n, (c0 + li) % tiles_n};

    const v4u rA = rsrc_words(p.A, (uint32_t)((size_t)p.M * p.lda));
    const v4u rW = rsrc_words(p.W, (uint32_t)((size_t)p.N * p.ldw));
    const v4u rS = rsrc_words(p.as, (uint32_t)((size_t)p.M * 4));
    const v4u rV = rsrc_words(p.ws, (uint32_t)((size_t)p.N * 4));
    const __amdgpu_buffer_rsrc_t ry =
        __builtin_amdgcn_make_buffer_rsrc(p.Y, 0, (int)min((long)p.M * p.ldy * 4, 0x7fffffffL), 0x00020000);
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const lds_void *)smem);

    // load i of a wave fills rows (i * 8 + wave) * 8 + lane / 8 of its tile (A: i < 4, W: i < 6),
    // 16-byte chunk (lane % 8) ^ swzk(row), the same for every i (see k_gemm_p); load 6: waves 0-3
    // the activation scales of rows 64 wave .. + 63, waves 4-7 the weight scales of columns
    // 64 (wave % 2) .. + 63 (waves 6 and 7 repeat 4 and 5: the same bytes to the same place)
    const int swl = ((lane & 7) ^ ((wave & 1) * 4 + ((lane >> 4) & 3))) << 4;
    const uint32_t vla = (uint32_t)(lane >> 3) * (uint32_t)p.lda + swl;
    const uint32_t vlb = (uint32_t)(lane >> 3) * (uint32_t)p.ldw + swl;
    const uint32_t vl4 = (uint32_t)lane * 4;
    const uint32_t sta = 64u * (uint32_t)p.lda, stw = 64u * (uint32_t)p.ldw;  // 64 rows

    int ig = 0, ikb = 0, islot = 0;
    TC itc = tc0;
    struct Issue {
        uint32_t st, sl, ko;
        int m0, n0;
    };
    uint32_t sa = 0, sw = 0;
    auto issue_prep = [&]() {
        Issue is;
        is.m0 = itc.mb * BM;
        is.n0 = itc.nt * BN;
        is.st = lds0 + (uint32_t)((ig % STAGES) * TILE) + (uint32_t)wave * 1024u;
        is.sl = lds0 + (uint32_t)(STAGES * TILE + islot * SLOT);
        is.ko = (uint32_t)(ikb * kQBlock);
        ++ig;
        if (++ikb == NB) {
            ikb = 0;
            itc = tc_next(itc);
            islot = islot == NSLOT - 1 ? 0 : islot + 1;
        }
        return is;
    };
    auto issue_load = [&](const Issue &is, int i) {
        if (i == 0) sa = (uint32_t)(is.m0 + wave * 8) * (uint32_t)p.lda + is.ko;
        if (i == 4) sw = (uint32_t)(is.n0 + wave * 8) * (uint32_t)p.ldw + is.ko;
        if (i < 4) {
            dma16(rA, is.st + i * NW * 1024, vla, sa);
            sa += sta;
        } else if (i < 6) {
            dma16(rW, is.st + BM * 128 + (i - 4) * NW * 1024, vlb, sw);
            sw += stw;
        } else if (wave < 4) {
            dma4(rS, is.sl + wave * 256, vl4, (uint32_t)(is.m0 + wave * 64) * 4);
        } else {
            dma4(rV, is.sl + 1024 + (wave & 1) * 256, vl4, (uint32_t)(is.n0 + (wave & 1) * 64) * 4);
        }
    };

    // fragments of 32-deep sub-step kk: row r32 of a 32-row tile, 16-byte chunk 2 kk + hi
    int fo[4];
#pragma unroll
    for (int kk = 0; kk < 4; kk++) fo[kk] = swz(r32, 2 * kk + hi);
    struct Frags {
        v4i a[2], w[2];
    };
    auto read_frags = [&](int stage, int kk, Frags &f) {
        const unsigned char *sb = smem + stage * TILE + fo[kk];
#pragma unroll
        for (int h = 0; h < 2; h++) f.a[h] = *(const v4i *)(sb + (wm * 64 + h * 32) * 128);
#pragma unroll
        for (int t = 0; t < 2; t++) f.w[t] = *(const v4i *)(sb + BM * 128 + (wn * 64 + t * 32) * 128);
    };

    // epilogue of the previous tile: lane holds column 64 wn + 32 t + r32 and rows
    // 64 wm + 32 h + 8 g + 4 hi + r
    struct Epi {
        f32x4 a4[2][4];
        float w1[2];
        uint32_t vy[4];
        uint32_t srow;
        uint32_t so;
    } ep;
    auto epi_begin = [&](TC tc, int slot) {
        const unsigned char *sl = smem + STAGES * TILE + slot * SLOT;
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int g = 0; g < 4; g++)
                ep.a4[h][g] = *(const f32x4 *)(sl + (wm * 64 + h * 32 + g * 8 + hi * 4) * 4);
#pragma unroll
        for (int t = 0; t < 2; t++) ep.w1[t] = *(const float *)(sl + 1024 + (wn * 64 + t * 32 + r32) * 4);
        const int n0 = tc.nt * BN + wn * 64;
#pragma unroll
        for (int r = 0; r < 4; r++) ep.vy[r] = (uint32_t)(((wm * 64 + hi * 4 + r) * p.ldy + n0 + r32) * 4);
        ep.srow = (uint32_t)(tc.mb * BM) * (uint32_t)p.ldy * 4u;
    };
    auto micro = [&](v16i (&acc)[2][2], auto U) {
        constexpr int u = decltype(U)::value;
        constexpr int h = u / 32, g = (u / 8) % 4, t = (u / 4) % 2, r = u % 4;
        if constexpr (t == 0 && r == 0) ep.so = ep.srow + (uint32_t)((h * 32 + g * 8) * p.ldy * 4);
        const float y = __builtin_fmaf((float)acc[h][t][4 * g + r], __fmul_rn(ep.a4[h][g][r], ep.w1[t]), 0.f);
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, y), ry, ep.vy[r] + t * 128, ep.so,
                                              kStoreNT);
    };

    Frags F[2];
    const int G = ntile * NB;
    if (G > 0) {
        Issue is = issue_prep();
#pragma unroll
        for (int i = 0; i < L; i++) issue_load(is, i);
        is = issue_prep();
#pragma unroll
        for (int i = 0; i < L; i++) issue_load(is, i);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(L) : "memory");
        __syncthreads();
        read_frags(0, 0, F[0]);
    }
    const v16i zero = {};

    int g = 0;
    TC ctc = tc0, etc = tc0;
    int cslot = 0, eslot = 0;
    auto tile = [&](v16i (&cur)[2][2], v16i (&prev)[2][2], auto EON) {
        constexpr bool EPI_ON = decltype(EON)::value;
        if constexpr (EPI_ON) epi_begin(etc, eslot);
        Issue is;
        [&]<int... S>(std::integer_sequence<int, S...>) {
            (
                [&] {
                    constexpr int s = S;          // slot of the tile
                    constexpr int st = s / SPS;   // step
                    constexpr int ss = s % SPS;   // slot of the step
                    constexpr int kk = ss / 4;    // sub-step
                    constexpr int i = ss % 4;     // MFMA of the sub-step
                    constexpr int h = i / 2, t = i % 2;
                    if constexpr (ss == 0) is = issue_prep();
                    const Frags &f = F[kk % 2];
                    cur[h][t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a[h], f.w[t],
                                                                       (st == 0 && kk == 0) ? zero : cur[h][t], 0, 0, 0);
                    if constexpr (i == 0) {
                        if constexpr (kk < 3) read_frags(g % STAGES, kk + 1, F[(kk + 1) % 2]);
                        else read_frags((g + 1) % STAGES, 0, F[0]);
                    }
                    if constexpr (ss < L) issue_load(is, ss);
                    if constexpr (EPI_ON) {
                        [&]<int... U>(std::integer_sequence<int, U...>) {
                            ((micro_slot<NB>(U) == s ? micro(prev, std::integral_constant<int, U>{}) : void()), ...);
                        }(std::make_integer_sequence<int, NMICRO>{});
                    }
                    if constexpr (ss == 11) {
                        // every wave has read stage g % 3 and step g + 1's loads have landed:
                        // besides them, the queue holds the stores of slots L-1..15 of step g - 1
                        // and 0..11 of step g and the L loads of step g + 2
                        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                        constexpr int after =
                            L + (EPI_ON ? stores_in<NB>(st * SPS, st * SPS + 12) +
                                              (st > 0 ? stores_in<NB>(st * SPS - SPS - 1 + L, st * SPS) : 0)
                                        : 0);
                        static_assert(after <= 63, "vmcnt range");
                        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(after) : "memory");
                        __builtin_amdgcn_s_barrier();
                    }
                    if constexpr (ss == SPS - 1) ++g;
                    __builtin_amdgcn_sched_barrier(0);
                }(),
                ...);
        }(std::make_integer_sequence<int, SPS * NB>{});
        etc = ctc;
        eslot = cslot;
        ctc = tc_next(ctc);
        cslot = cslot == NSLOT - 1 ? 0 : cslot + 1;
    };
    static_assert(stores_in<NB>(SPS * (NB - 1), SPS * NB) == 0, "the last step of a tile stores nothing");
    auto final_epi = [&](v16i (&acc)[2][2]) {
        epi_begin(etc, eslot);
        [&]<int... U>(std::integer_sequence<int, U...>) {
            (micro(acc, std::integral_constant<int, U>{}), ...);
        }(std::make_integer_sequence<int, NMICRO>{});
    };

    v16i accA[2][2], accB[2][2];
    if (ntile > 0) {
        tile(accA, accB, std::false_type{});
        int j = 1;
        for (; j + 1 < ntile; j += 2) {
            tile(accB, accA, std::true_type{});
            tile(accA, accB, std::true_type{});
        }
        if (j < ntile) {
            tile(accB, accA, std::true_type{});
            final_epi(accB);
        } else {
            final_epi(accA);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Per-token GEMM with the requantizing epilogue overlapped (k_gemm_tq): the per-token requant
// contract (e2mi_i8_gemm_tok_q) at K = 128 NB, N a multiple of 128, no bias or clamp. The pipeline
// of k_gemm_tv (256 x 128 output tiles, one 512-thread workgroup per CU, three 48 KB A|W stages
// with loads two steps ahead, slots of one MFMA each, two accumulator sets, the previous tile's
// epilogue spread over the current tile's slots), with the waves laid out for the requantization:
//   - 8 waves of 32 x 128 (all of the tile's 128 columns, one quantization block), four MFMA tiles
//     each; a wave owns whole blocks, so a row's maximum needs no other wave;
//   - W's 128 rows of a tile are fetched into LDS in the order rho -> 4 (rho % 32) + rho / 32, so
//     MFMA tile t leaves lane c (of 32) the output column 4 c + t: every lane holds four
//     consecutive columns of each of its 16 rows, one int8 dword, and a store instruction writes
//     two rows' 128 bytes whole;
//   - epilogue of the previous tile, spread over the slots: (A) 64 conversions
//     y = fma((float)acc, RN(as * ws), 0) in place, with the lane's running row maxima; (B) the
//     rows' maxima over the 32 lanes of each half by a transposing halving exchange (each lane
//     pair ends with one row's maximum), the quantizer's scale and inverse for that row, its scale
//     stored, the 16 inverses fetched back by lane permutes; (C) 16 packs and dword stores.
// Bytes and scales equal k_gemm_t's requantizing epilogue (the same conversion, maximum and
// quantizer arithmetic).
namespace tq {
constexpr int BM = 256, BN = 128, NW = 8, STAGES = 3, NSLOT = 3;
constexpr int TILE = (BM + BN) * 128;
constexpr int SLOT = 2048;                     // as (256 floats) | ws (128 floats) of one tile
constexpr int LDS = STAGES * TILE + NSLOT * SLOT;
constexpr int L = BM / 8 / NW + BN / 8 / NW + 1;  // loads per wave per step: 4 A, 2 W, as or ws
constexpr int SPS = 16;                        // MFMA slots per step
constexpr int NA = 64, NC = 16;                // phase A conversions, phase C packs per lane
static_assert(LDS <= 160 * 1024, "LDS budget");
// slots of the phases within a tile (the epilogue of the previous tile): A over the first slots,
// B right after the last A, C in the last NC slots before the tile's last step
template <int NB>
constexpr int slot_c(int r) { return SPS * (NB - 1) - NC + r; }
template <int NB>
constexpr int slot_a(int u) { return u * (slot_c<NB>(0) - 1) / NA; }
template <int NB>
constexpr int slot_b() { return slot_a<NB>(NA - 1); }
// stores issued in slots [s0, s1): one for the scales at B, one per C slot
template <int NB>
constexpr int stores_in(int s0, int s1) {
    int n = (slot_b<NB>() >= s0 && slot_b<NB>() < s1) ? 1 : 0;
    for (int r = 0; r < NC; r++) n += (slot_c<NB>(r) >= s0 && slot_c<NB>(r) < s1) ? 1 : 0;
    return n;
}
}  // namespace tq

template <int X>
__device__ inline float swz_xor_max(float v) { return fmaxf(v, swz_xor<X>(v)); }
template <int X, int N>
__device__ inline void halve_max(const float (&v)[2 * N], float (&o)[N], bool up) {
#pragma unroll
    for (int i = 0; i < N; i++) {
        const float keep = up ? v[i + N] : v[i], give = up ? v[i] : v[i + N];
        o[i] = fmaxf(keep, swz_xor<X>(give));
    }
}

template <int NB>
__global__ __launch_bounds__(512, 1) void k_gemm_tq(GemmArgs p, int tiles_n, int tiles) {
    using namespace tq;
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hi = lane >> 5, r32 = lane & 31;

    const int nx = (gridDim.x % 8 == 0) ? 8 : 1;
    const int grp = blockIdx.x % nx, li = blockIdx.x / nx, per = gridDim.x / nx;
    const int c0 = (int)((long)tiles * grp / nx), c1 = (int)((long)tiles * (grp + 1) / nx);
    const int ntile = (c1 - c0 > li) ? (c1 - c0 - li + per - 1) / per : 0;
    const int per_m = per / tiles_n, per_n = per % tiles_n;
    struct TC {
        int mb, nt;
    };
    auto tc_next = [&](TC t) {
        t.mb += per_m;
        t.nt += per_n;
        if (t.nt >= tiles_n) {
            t.nt -= tiles_n;
            t.mb += 1;
        }
        return t;
    };
    const TC tc0 = {(c0 + li) / tiles_n, (c0 + li) % tiles_n};

    const v4u rA = rsrc_words(p.A, (uint32_t)((size_t)p.M * p.lda));
    const v4u rW = rsrc_words(p.W, (uint32_t)((size_t)p.N * p.ldw));
    const v4u rS = rsrc_words(p.as, (uint32_t)((size_t)p.M * 4));
    const v4u rV = rsrc_words(p.ws, (uint32_t)((size_t)p.N * 4));
    const __amdgpu_buffer_rsrc_t rq =
        __builtin_amdgcn_make_buffer_rsrc(p.Yq, 0, (int)min((long)p.M * p.ldyq, 0x7fffffffL), 0x00020000);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(p.ys, 0, (int)min((long)p.M * p.ldys * 4, 0x7fffffffL), 0x00020000);
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const lds_void *)smem);

    // A loads as in k_gemm_tv. W load ii (0, 1) of a wave fills LDS rows rho = 64 ii + 8 wave +
    // lane / 8 with W row 4 (rho % 32) + rho / 32 = 32 (wave % 4) + 2 ii + wave / 4 + 4 (lane / 8)
    // of the tile: the lane part 4 (lane / 8) rows, the rest a scalar row; the 16-byte chunk
    // swizzle depends on the LDS row only, as for A
    const int swl = ((lane & 7) ^ ((wave & 1) * 4 + ((lane >> 4) & 3))) << 4;
    const uint32_t vla = (uint32_t)(lane >> 3) * (uint32_t)p.lda + swl;
    const uint32_t vlb = (uint32_t)(lane >> 3) * 4u * (uint32_t)p.ldw + swl;
    const uint32_t vl4 = (uint32_t)lane * 4;
    const uint32_t sta = 64u * (uint32_t)p.lda;

    int ig = 0, ikb = 0, islot = 0;
    TC itc = tc0;
    struct Issue {
        uint32_t st, sl, ko;
        int m0, n0;
    };
    uint32_t sa = 0;
    auto issue_prep = [&]() {
        Issue is;
        is.m0 = itc.mb * BM;
        is.n0 = itc.nt * BN;
        is.st = lds0 + (uint32_t)((ig % STAGES) * TILE) + (uint32_t)wave * 1024u;
        is.sl = lds0 + (uint32_t)(STAGES * TILE + islot * SLOT);
        is.ko = (uint32_t)(ikb * kQBlock);
        ++ig;
        if (++ikb == NB) {
            ikb = 0;
            itc = tc_next(itc);
            islot = islot == NSLOT - 1 ? 0 : islot + 1;
        }
        return is;
    };
    auto issue_load = [&](const Issue &is, int i) {
        if (i == 0) sa = (uint32_t)(is.m0 + wave * 8) * (uint32_t)p.lda + is.ko;
        if (i < 4) {
            dma16(rA, is.st + i * NW * 1024, vla, sa);
            sa += sta;
        } else if (i < 6) {
            const uint32_t wr = (uint32_t)(is.n0 + 32 * (wave & 3) + 2 * (i - 4) + (wave >> 2));
            dma16(rW, is.st + BM * 128 + (i - 4) * NW * 1024, vlb, wr * (uint32_t)p.ldw + is.ko);
        } else if (wave < 4) {
            dma4(rS, is.sl + wave * 256, vl4, (uint32_t)(is.m0 + wave * 64) * 4);
        } else {
            dma4(rV, is.sl + 1024 + (wave & 1) * 256, vl4, (uint32_t)(is.n0 + (wave & 1) * 64) * 4);
        }
    };

    // fragments of 32-deep sub-step kk: row r32 of a 32-row tile, 16-byte chunk 2 kk + hi
    int fo[4];
#pragma unroll
    for (int kk = 0; kk < 4; kk++) fo[kk] = swz(r32, 2 * kk + hi);
    struct Frags {
        v4i a, w[4];
    };
    auto read_frags = [&](int stage, int kk, Frags &f) {
        const unsigned char *sb = smem + stage * TILE + fo[kk];
        f.a = *(const v4i *)(sb + (wave * 32) * 128);
#pragma unroll
        for (int t = 0; t < 4; t++) f.w[t] = *(const v4i *)(sb + BM * 128 + (t * 32) * 128);
    };

    // epilogue state of the previous tile: register r of tile t holds row
    // 32 wave + 8 (r / 4) + 4 hi + r % 4 and column 4 r32 + t
    struct Epi {
        f32x4 a4[4];  // activation scales of the lane's 16 rows
        f32x4 w4;     // weight scales of its 4 columns
        float m[16];  // running row maxima, then the rows' inverse scales
        uint32_t row0;  // first row of the wave (of the tile being written)
        uint32_t col;   // the lane's first column
    } ep;
    auto epi_begin = [&](TC tc, int slot) {
        const unsigned char *sl = smem + STAGES * TILE + slot * SLOT;
#pragma unroll
        for (int g = 0; g < 4; g++) ep.a4[g] = *(const f32x4 *)(sl + (wave * 32 + g * 8 + hi * 4) * 4);
        ep.w4 = *(const f32x4 *)(sl + 1024 + (4 * r32) * 4);
        ep.row0 = (uint32_t)(tc.mb * BM + wave * 32);
        ep.col = (uint32_t)(tc.nt * BN + 4 * r32);
    };
    // phase A, element u: tile t = u % 4 of register r = u / 4
    auto phase_a = [&](v16i (&acc)[4], auto U) {
        constexpr int u = decltype(U)::value;
        constexpr int t = u % 4, r = u / 4;
        const float y = __builtin_fmaf((float)acc[t][r], __fmul_rn(ep.a4[r >> 2][r & 3], ep.w4[t]), 0.f);
        acc[t][r] = __builtin_bit_cast(int, y);
        ep.m[r] = t == 0 ? fabsf(y) : fmaxf(ep.m[r], fabsf(y));
    };
    // phase B: per-row maxima over the half-wave, scale and inverse, the scales stored, the lane's
    // 16 rows' inverses back in ep.m
    auto phase_b = [&]() {
        float m8[8], m4[4], m2[2], m1[1];
        halve_max<16, 8>(ep.m, m8, lane & 16);
        halve_max<8, 4>(m8, m4, lane & 8);
        halve_max<4, 2>(m4, m2, lane & 4);
        halve_max<2, 1>(m2, m1, lane & 2);
        const float amax = swz_xor_max<1>(m1[0]);
        // this lane pair holds register j's row
        const int j = ((lane >> 4) & 1) * 8 + ((lane >> 3) & 1) * 4 + ((lane >> 2) & 1) * 2 + ((lane >> 1) & 1);
        const QScale qs = qscale(amax);
        const uint32_t row = ep.row0 + (uint32_t)(8 * (j >> 2) + 4 * hi + (j & 3));
        // one lane per row writes its scale; the others point past the descriptor's range
        const uint32_t so = (lane & 1) == 0 ? (row * (uint32_t)p.ldys + (ep.col - 4 * r32) / 128) * 4 : 0x80000000u;
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, qs.sc), rs, so, 0, 0);
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int src = (lane & 0x20) | (((r >> 3) & 1) << 4) | (((r >> 2) & 1) << 3) | (((r >> 1) & 1) << 2) |
                            ((r & 1) << 1);
            ep.m[r] = __shfl(qs.inv, src);
        }
    };
    // phase C, register r: the four columns' bytes, one dword store
    auto phase_c = [&](v16i (&acc)[4], auto R) {
        constexpr int r = decltype(R)::value;
        // the elements go through plain ints first: __builtin_bit_cast of a vector element lvalue
        // reads the vector's first element in this compiler (its address is the vector's)
        const int b0 = acc[0][r], b1 = acc[1][r], b2 = acc[2][r], b3 = acc[3][r];
        const uint32_t w = pack4_magic(__builtin_bit_cast(float, b0), __builtin_bit_cast(float, b1),
                                       __builtin_bit_cast(float, b2), __builtin_bit_cast(float, b3), ep.m[r]);
        const uint32_t row = ep.row0 + (uint32_t)(8 * (r >> 2) + 4 * hi + (r & 3));
        __builtin_amdgcn_raw_buffer_store_b32(w, rq, row * (uint32_t)p.ldyq + ep.col, 0, 0);
    };

    Frags F[2];
    const int G = ntile * NB;
    if (G > 0) {
        Issue is = issue_prep();
#pragma unroll
        for (int i = 0; i < L; i++) issue_load(is, i);
        is = issue_prep();
#pragma unroll
        for (int i = 0; i < L; i++) issue_load(is, i);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(L) : "memory");
        __syncthreads();
        read_frags(0, 0, F[0]);
    }
    const v16i zero = {};

    int g = 0;
    TC ctc = tc0, etc = tc0;
    int cslot = 0, eslot = 0;
    auto tile = [&](v16i (&cur)[4], v16i (&prev)[4], auto EON) {
        constexpr bool EPI_ON = decltype(EON)::value;
        if constexpr (EPI_ON) epi_begin(etc, eslot);
        Issue is;
        [&]<int... S>(std::integer_sequence<int, S...>) {
            (
                [&] {
                    constexpr int s = S;          // slot of the tile
                    constexpr int st = s / SPS;   // step
                    constexpr int ss = s % SPS;   // slot of the step
                    constexpr int kk = ss / 4;    // sub-step
                    constexpr int t = ss % 4;     // MFMA (output tile) of the sub-step
                    if constexpr (ss == 0) is = issue_prep();
                    const Frags &f = F[kk % 2];
                    cur[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.a, f.w[t], (st == 0 && kk == 0) ? zero : cur[t],
                                                                    0, 0, 0);
                    if constexpr (t == 0) {
                        if constexpr (kk < 3) read_frags(g % STAGES, kk + 1, F[(kk + 1) % 2]);
                        else read_frags((g + 1) % STAGES, 0, F[0]);
                    }
                    if constexpr (ss < L) issue_load(is, ss);
                    if constexpr (EPI_ON) {
                        [&]<int... U>(std::integer_sequence<int, U...>) {
                            ((slot_a<NB>(U) == s ? phase_a(prev, std::integral_constant<int, U>{}) : void()), ...);
                        }(std::make_integer_sequence<int, NA>{});
                        if constexpr (slot_b<NB>() == s) phase_b();
                        [&]<int... R>(std::integer_sequence<int, R...>) {
                            ((slot_c<NB>(R) == s ? phase_c(prev, std::integral_constant<int, R>{}) : void()), ...);
                        }(std::make_integer_sequence<int, NC>{});
                    }
                    if constexpr (ss == 11) {
                        // every wave has read stage g % 3 and step g + 1's loads have landed:
                        // besides them, the queue holds the stores of slots L-1..15 of step g - 1
                        // and 0..11 of step g and the L loads of step g + 2
                        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                        constexpr int after =
                            L + (EPI_ON ? stores_in<NB>(st * SPS, st * SPS + 12) +
                                              (st > 0 ? stores_in<NB>(st * SPS - SPS - 1 + L, st * SPS) : 0)
                                        : 0);
                        static_assert(after <= 63, "vmcnt range");
                        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(after) : "memory");
                        __builtin_amdgcn_s_barrier();
                    }
                    if constexpr (ss == SPS - 1) ++g;
                    __builtin_amdgcn_sched_barrier(0);
                }(),
                ...);
        }(std::make_integer_sequence<int, SPS * NB>{});
        etc = ctc;
        eslot = cslot;
        ctc = tc_next(ctc);
        cslot = cslot == NSLOT - 1 ? 0 : cslot + 1;
    };
    static_assert(stores_in<NB>(SPS * (NB - 1), SPS * NB) == 0, "the last step of a tile stores nothing");
    auto final_epi = [&](v16i (&acc)[4]) {
        epi_begin(etc, eslot);
        [&]<int... U>(std::integer_sequence<int, U...>) {
            (phase_a(acc, std::integral_constant<int, U>{}), ...);
        }(std::make_integer_sequence<int, NA>{});
        phase_b();
        [&]<int... R>(std::integer_sequence<int, R...>) {
            (phase_c(acc, std::integral_constant<int, R>{}), ...);
        }(std::make_integer_sequence<int, NC>{});
    };

    v16i accA[4], accB[4];
    if (ntile > 0) {
        tile(accA, accB, std::false_type{});
        int j = 1;
        for (; j + 1 < ntile; j += 2) {
            tile(accB, accA, std::true_type{});
            tile(accA, accB, std::true_type{});
        }
        if (j < ntile) {
            tile(accB, accA, std::true_type{});
            final_epi(accB);
        } else {
            final_epi(accA);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

int num_cus() {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
    }
    return cus;
}

template <int BM, int BN, int NWM, int NWN, int EPI, bool FAST, int POST, bool NT = false>
static int launch_p1(hipStream_t s, const GemmArgs &p) {
    constexpr size_t lds = p_lds_bytes<BM, BN, NWM * NWN>();
    static_assert(lds <= 160 * 1024, "LDS budget");
    static_assert(EPI == EPI_F32 || EPI == EPI_QKV ||
                      NWM * NWN * (8 * ((EPI == EPI_GEGLU ? 64 : 128) + 4) + 32) * 4 <= (BM + BN) * 128,
                  "epilogue scratch fits a stage");
    auto kern = k_gemm_p<BM, BN, NWM, NWN, EPI, FAST, POST, NT>;
    static bool attr = false;
    if (!attr) {
        if (check_hip(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                      "gemm lds attribute"))
            return -1;
        attr = true;
    }
    const int tiles_n = (p.N + BN - 1) / BN;
    const long tiles = (long)((p.M + BM - 1) / BM) * tiles_n;
    if (tiles > (1L << 30)) {
        set_error("gemm: too many tiles");
        return -1;
    }
    const int grid = (int)min(tiles, (long)num_cus() * (8 / (NWM * NWN)));
    hipLaunchKernelGGL(kern, dim3(grid), dim3(NWM * NWN * 64), lds, s, p.rows, p, tiles_n, (int)tiles);
    return check_hip(hipGetLastError(), "gemm launch");
}

template <int EPI, int POST>
static int launch_t1(hipStream_t s, const GemmArgs &p) {
    constexpr size_t lds = 2 * (256 + 256) * 128 + kPSlots * 2 * 64 * 8 * 4;
    static_assert(lds <= 160 * 1024, "LDS budget");
    auto kern = k_gemm_t<EPI, POST>;
    static bool attr = false;
    if (!attr) {
        if (check_hip(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                      "gemm lds attribute"))
            return -1;
        attr = true;
    }
    const int tiles_n = (p.N + 255) / 256;
    const long tiles = (long)((p.M + 255) / 256) * tiles_n;
    if (tiles > (1L << 30)) {
        set_error("gemm: too many tiles");
        return -1;
    }
    const int grid = (int)min(tiles, (long)num_cus());
    hipLaunchKernelGGL(kern, dim3(grid), dim3(512), lds, s, p, tiles_n, (int)tiles);
    return check_hip(hipGetLastError(), "gemm launch");
}

template <int NB>
static int launch_tv(hipStream_t s, const GemmArgs &p) {
    auto kern = k_gemm_tv<NB>;
    static bool attr = false;
    if (!attr) {
        if (check_hip(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, tv::LDS),
                      "gemm lds attribute"))
            return -1;
        attr = true;
    }
    const int tiles_n = p.N / tv::BN;
    const long tiles = (long)((p.M + tv::BM - 1) / tv::BM) * tiles_n;
    if (tiles > (1L << 30)) {
        set_error("gemm: too many tiles");
        return -1;
    }
    const int grid = (int)min(tiles, (long)num_cus());
    hipLaunchKernelGGL(kern, dim3(grid), dim3(512), tv::LDS, s, p, tiles_n, (int)tiles);
    return check_hip(hipGetLastError(), "gemm launch");
}
template <int NB>
static int launch_tq(hipStream_t s, const GemmArgs &p) {
    auto kern = k_gemm_tq<NB>;
    static bool attr = false;
    if (!attr) {
        if (check_hip(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, tq::LDS),
                      "gemm lds attribute"))
            return -1;
        attr = true;
    }
    const int tiles_n = p.N / tq::BN;
    const long tiles = (long)((p.M + tq::BM - 1) / tq::BM) * tiles_n;
    if (tiles > (1L << 30)) {
        set_error("gemm: too many tiles");
        return -1;
    }
    const int grid = (int)min(tiles, (long)num_cus());
    hipLaunchKernelGGL(kern, dim3(grid), dim3(512), tq::LDS, s, p, tiles_n, (int)tiles);
    return check_hip(hipGetLastError(), "gemm launch");
}
// the overlapped per-token f32 kernel: N a multiple of 128, no bias or clamp, K = 768 or 1152 (the
// unrolled instantiations); every other per-token call takes k_gemm_t
static bool use_tv(const GemmArgs &p) {
    const bool post = p.bias != nullptr || p.lo > -1e30f || p.hi < 1e30f;
    return !post && p.N % tv::BN == 0 && (p.K == 6 * kQBlock || p.K == 9 * kQBlock);
}

// E2MI_TQ=0 keeps the per-token requantizing calls on k_gemm_t (A/B measurements)
static bool use_tq() {
    static int on = -1;
    if (on < 0) {
        const char *e = getenv("E2MI_TQ");
        on = (e && e[0] == '0') ? 0 : 1;
    }
    return on == 1;
}

template <int EPI>
static int launch_t(hipStream_t s, const GemmArgs &p) {
    if (EPI == EPI_F32 && use_tv(p)) return p.K == 6 * kQBlock ? launch_tv<6>(s, p) : launch_tv<9>(s, p);
    if (EPI == EPI_I8Q && use_tv(p) && use_tq()) return p.K == 6 * kQBlock ? launch_tq<6>(s, p) : launch_tq<9>(s, p);
    const bool post = p.bias != nullptr || p.lo > -1e30f || p.hi < 1e30f;
    return post ? launch_t1<EPI, 3>(s, p) : launch_t1<EPI, 0>(s, p);
}

// f32 outputs of 128 MB or more go out with non-temporal stores: at M = 65536 the default
// policy's write-allocation of a 200-335 MB output evicts the A and W tiles every step re-reads
// from L2, and the loads then queue behind the writes (C5 768x1280: 155-163 -> 135-142 us).
// Smaller outputs keep the default: in the encoder's forward the next kernel reads them at once,
// from the caches. The requantizing epilogue's int8 outputs (84 MB at C5) measured slower
// streamed and keep the default.
constexpr size_t kStreamOutBytes = (size_t)128 << 20;
template <int BM, int BN, int NWM, int NWN, int EPI, bool FAST, int POST>
static int launch_p2(hipStream_t s, const GemmArgs &p) {
    if constexpr (EPI == EPI_F32 && BM == 256) {
        if ((size_t)p.M * (size_t)p.N * 4 >= kStreamOutBytes) return launch_p1<BM, BN, NWM, NWN, EPI, FAST, POST, true>(s, p);
    }
    return launch_p1<BM, BN, NWM, NWN, EPI, FAST, POST>(s, p);
}
// POST: bit 0 adds a bias, bit 1 clamps to [lo, hi]; only "none" and "both" are instantiated (the
// bias pointer may be null and an absent clamp is +-1e31)
template <int BM, int BN, int NWM, int NWN, int EPI>
static int launch_p(hipStream_t s, const GemmArgs &p) {
    const bool post = p.bias != nullptr || p.lo > -1e30f || p.hi < 1e30f;
    if (fold_fast())
        return post ? launch_p2<BM, BN, NWM, NWN, EPI, true, 3>(s, p) : launch_p2<BM, BN, NWM, NWN, EPI, true, 0>(s, p);
    return post ? launch_p2<BM, BN, NWM, NWN, EPI, false, 3>(s, p) : launch_p2<BM, BN, NWM, NWN, EPI, false, 0>(s, p);
}

static int launch_dump(hipStream_t s, const GemmArgs &p) {
    constexpr size_t lds = 2 * ((size_t)(128 + 128) * 128 + 64 * 4 * 4);
    static bool attr = false;
    if (!attr) {
        if (check_hip(hipFuncSetAttribute((const void *)k_gemm_dump, hipFuncAttributeMaxDynamicSharedMemorySize,
                                          (int)lds),
                      "gemm lds attribute"))
            return -1;
        attr = true;
    }
    const long tiles = (long)((p.M + 127) / 128) * ((p.N + 127) / 128);
    hipLaunchKernelGGL(k_gemm_dump, dim3((unsigned)tiles), dim3(256), lds, s, p);
    return check_hip(hipGetLastError(), "gemm launch");
}

static int check_args(const GemmArgs &p, const char *who, bool rows_ok = true) {
    if (p.rows && !rows_ok) {
        set_error("%s: a device row count is taken by the per-128 GEMMs only", who);
        return -1;
    }
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

// 128 x 128 tiles of 4 waves, two workgroups per CU, instead of 256 x 128 tiles of 8 waves, one
// per CU, where they take fewer rounds of the device: with fewer 256 x 128 tiles than CUs (the
// vision tower's 2520-patch projections, small batches), and where the 256 x 128 tiles need a last
// round that only a few CUs work on (the reference geometry's N = 512 projections at 17408 rows:
// 272 tiles, two rounds for 1.06 rounds of work). In units of one 256 x 128 tile's time on a CU:
// 256 x 128 tiles take ceil(tiles / CUs) rounds; 128 x 128 tiles take one unit per full round of
// two workgroups on every CU, and a last partial round of at most one workgroup per CU about 0.6
// (a 128 x 128 workgroup alone on its CU).
bool gemm_half_tiles(int M, int N) {
    const long C = num_cus();
    const long t256 = (long)((M + 255) / 256) * ((N + 127) / 128);
    if (t256 < C) return true;
    const long t128 = (long)((M + 127) / 128) * ((N + 127) / 128);
    const long full = t128 / (2 * C), rem = t128 % (2 * C);
    const double r128 = (double)full + (rem == 0 ? 0.0 : rem <= C ? 0.6 : 1.0);
    const double r256 = (double)((t256 + C - 1) / C);
    return r128 <= r256 - 0.3;
}
// in a forward planned on the device, for the host's estimate of the planned row count
static bool half_tiles(const GemmArgs &p) {
    const int est = p.rows ? device_rows().est : 0;
    return gemm_half_tiles(est > 0 && est < p.M ? est : p.M, p.N);
}

int launch_gemm_f32(hipStream_t s, GemmArgs p, bool dump, bool tok = false) {
    if (check_args(p, "i8_gemm", !dump && !tok)) return -1;
    if (!p.Y || p.ldy < p.N) {
        set_error("i8_gemm: null output or ldy < N");
        return -1;
    }
    if (dump) {
        if (!p.accd) {
            set_error("i8_gemm: null accumulator dump");
            return -1;
        }
        return launch_dump(s, p);
    }
    if (tok) return launch_t<EPI_F32>(s, p);
    if (half_tiles(p)) return launch_p<128, 128, 4, 1, EPI_F32>(s, p);
    return launch_p<256, 128, 8, 1, EPI_F32>(s, p);
}

int launch_gemm_i8q(hipStream_t s, GemmArgs p, bool tok = false) {
    if (check_args(p, "i8_gemm_q", !tok)) return -1;
    if (p.N % 128 || !p.Yq || !p.ys || p.ldyq < p.N || p.ldyq % 16 || !aligned16(p.Yq) ||
        p.ldys < p.N / 128) {
        set_error("i8_gemm_q: N must be a multiple of 128 with a 16-byte aligned int8 output");
        return -1;
    }
    if (tok) return launch_t<EPI_I8Q>(s, p);
    if (half_tiles(p)) return launch_p<128, 128, 4, 1, EPI_I8Q>(s, p);
    return launch_p<256, 128, 8, 1, EPI_I8Q>(s, p);
}

int launch_gemm_gelumul(hipStream_t s, GemmArgs p) {
    if (check_args(p, "i8_gemm_gelu_mul")) return -1;
    if (p.N % 128 || !p.Yq || !p.ys || p.ldyq < p.N || p.ldyq % 16 || !aligned16(p.Yq) ||
        p.ldys < p.N / 128 || !p.mul || p.ldmul < p.N || p.ldmul % 4 || !aligned16(p.mul) ||
        (p.Y && (p.ldy < p.N || p.ldy % 4 || !aligned16(p.Y)))) {
        set_error("i8_gemm_gelu_mul: N must be a multiple of 128; outputs and multiplier 16-byte aligned");
        return -1;
    }
    if (half_tiles(p)) return launch_p<128, 128, 4, 1, EPI_GELUMUL>(s, p);
    return launch_p<256, 128, 8, 1, EPI_GELUMUL>(s, p);
}

int launch_gemm_geglu(hipStream_t s, GemmArgs p) {
    if (check_args(p, "i8_gemm_geglu")) return -1;
    if (p.N % 256 || !p.Yq || !p.ys || p.ldyq < p.N / 2 || p.ldyq % 16 || !aligned16(p.Yq) ||
        p.ldys < p.N / 256 || (p.Y && (p.ldy < p.N / 2 || p.ldy % 4 || !aligned16(p.Y)))) {
        set_error("i8_gemm_geglu: N (gate|up interleaved) must be a multiple of 256, outputs aligned");
        return -1;
    }
    // 128 x 256 tiles: a tile holds the interleaved gate|up columns of one output block
    return launch_p<128, 256, 4, 2, EPI_GEGLU>(s, p);
}

int launch_gemm_qkv(hipStream_t s, GemmArgs p) {
    if (check_args(p, "i8_gemm_qkv")) return -1;
    const int heads = p.qH + 2 * p.qKV;
    if (p.qH <= 0 || p.qKV <= 0 || p.qH % p.qKV || p.N != heads * 256 || p.qS <= 0 ||
        (p.pos && p.qS != p.M) || (!p.pos && p.M % p.qS)) {
        set_error("i8_gemm_qkv: needs N = (H + 2 KV) * 256, H %% KV == 0 and M = B * S (packed: S = M) "
                  "(M=%d N=%d H=%d KV=%d S=%d)", p.M, p.N, p.qH, p.qKV, p.qS);
        return -1;
    }
    if (p.bias || p.lo > -1e30f || p.hi < 1e30f) {
        set_error("i8_gemm_qkv: the q|k|v weight takes no bias or clamp");
        return -1;
    }
    if (!p.q_gamma || !p.k_gamma || !p.cs || !p.sn || !p.q16 || !p.k16 || !p.vt16 || ((uintptr_t)p.vt16 & 7)) {
        set_error("i8_gemm_qkv: null gamma/table/output pointer or V^T not 8-byte aligned");
        return -1;
    }
    // the epilogue's buffer-store offsets are 32-bit byte offsets into each output
    const long widest = (long)p.M * (p.qH > p.qKV ? p.qH : p.qKV) * 256 * ((p.q32 || p.k32 || p.v32) ? 4 : 2);
    if (widest > 0x7fffffffL) {
        set_error("i8_gemm_qkv: %d rows of %d heads exceed 2^31 bytes of one output", p.M,
                  p.qH > p.qKV ? p.qH : p.qKV);
        return -1;
    }
    // 128 x 256 tiles: a tile is one head of 128 rows
    return launch_p<128, 256, 4, 2, EPI_QKV>(s, p);
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
    p.rows = device_rows().ptr;
    return p;
}

extern "C" int e2mi_gemm_set_fold(int mode) {
    if (mode != 0 && mode != 1) {
        set_error("gemm_set_fold: mode must be 0 (exact) or 1 (fast), got %d", mode);
        return -1;
    }
    const int prev = fold_fast() ? 1 : 0;
    g_fold = mode;
    return prev;
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

// per-token activation scales (a_scales [M], the reference's int8 path built with one block per
// row, int8.h:61-70 E2_I8_BLOCK = K)
extern "C" int e2mi_i8_gemm_tok(e2mi_stream stream, float *y, int ldy, const int8_t *qa,
                                const float *a_scales, const e2mi_q8w *w, int M, int n0, int n1) {
    if (!weight_ok(w, "i8_gemm_tok")) return -1;
    if (n0 < 0 || n1 > w->N || n0 >= n1 || !y) {
        set_error("i8_gemm_tok: bad column range [%d,%d) for N=%d", n0, n1, w ? w->N : 0);
        return -1;
    }
    GemmArgs p = make_args(qa, a_scales, w, M, n0, n1);
    p.Y = y + n0;
    p.ldy = ldy;
    return launch_gemm_f32((hipStream_t)stream, p, false, true);
}

extern "C" int e2mi_i8_gemm_tok_q(e2mi_stream stream, int8_t *yq, float *ys, const int8_t *qa,
                                  const float *a_scales, const e2mi_q8w *w, int M) {
    if (!weight_ok(w, "i8_gemm_tok_q")) return -1;
    GemmArgs p = make_args(qa, a_scales, w, M, 0, w->N);
    p.Yq = yq;
    p.ldyq = w->N;
    p.ys = ys;
    p.ldys = w->N / 128;
    return launch_gemm_i8q((hipStream_t)stream, p, true);
}

extern "C" int e2mi_i8_gemm_gelu_mul(e2mi_stream stream, int8_t *yq, float *ys, float *g, const int8_t *qa,
                                     const float *a_scales, const e2mi_q8w *w, int M, const float *mul,
                                     int ldmul) {
    if (!weight_ok(w, "i8_gemm_gelu_mul")) return -1;
    GemmArgs p = make_args(qa, a_scales, w, M, 0, w->N);
    p.Yq = yq;
    p.ldyq = w->N;
    p.ys = ys;
    p.ldys = w->N / 128;
    p.Y = g;
    p.ldy = w->N;
    p.mul = mul;
    p.ldmul = ldmul;
    return launch_gemm_gelumul((hipStream_t)stream, p);
}

extern "C" int e2mi_i8_gemm_qkv(e2mi_stream stream, const int8_t *qa, const float *a_scales,
                                const e2mi_q8w *w_qkv, int M, int S, const int32_t *pos, int H, int KV,
                                const float *q_gamma, const float *k_gamma, float eps, const float *cos_tab,
                                const float *sin_tab, uint16_t *q16, uint16_t *k16, uint16_t *vt16,
                                float *q32, float *k32, float *v32) {
    if (!weight_ok(w_qkv, "i8_gemm_qkv")) return -1;
    GemmArgs p = make_args(qa, a_scales, w_qkv, M, 0, w_qkv->N);
    p.q_gamma = q_gamma;
    p.k_gamma = k_gamma;
    p.cs = cos_tab;
    p.sn = sin_tab;
    p.pos = pos;
    p.q16 = q16;
    p.k16 = k16;
    p.vt16 = vt16;
    p.q32 = q32;
    p.k32 = k32;
    p.v32 = v32;
    p.qH = H;
    p.qKV = KV;
    p.qS = S;
    p.eps = eps;
    return launch_gemm_qkv((hipStream_t)stream, p);
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
