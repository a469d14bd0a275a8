// gemm_an.hip — a projection that feeds a sublayer's norm_add (the encoder's O and down
// projections, text.c:944-953) with the norm_add and the next GEMM's quantization in its epilogue
// (gfx950, wave64, v_mfma_i32_16x16x64_i8):
//
//   y = e2_i8_gemm(qa, W)                 the exact per-128 fold: y = sum_b fma((float)acc_b, RN(as*ws), .)
//   x = rmsnorm(y) * gamma_a + res        -> x_out (may alias res)          kernels.c:161-171
//   rmsnorm(x) * gamma_n                  -> q / qs per 128, and xn_out f32 when asked
//
// It gives the bits of e2mi_i8_gemm followed by e2mi_add_norm_quant without the GEMM's f32 output,
// which the row kernel read straight back (M x 768 x 4 bytes written, then read, per projection).
//
// The norm needs whole rows, so a 512-thread workgroup (one per CU) owns whole 768-wide rows: the
// (device) row count in 16-row units is cut evenly into ranges of at most UC units (80 rows), one
// per workgroup, UC chosen by the host so that the ranges fill the CUs in few rounds. Wave w holds
// columns 96 w .. 96 w + 95 (six 16-column units) of every row of its range as f32 running sums
// (UC x 24 registers). K is walked in 128-deep blocks, one quantization block each, as the fold
// needs:
//  - A (1-KB pieces of 16 rows x 64 bytes, one per (row unit, K half)) and the block's activation
//    scales go to LDS by direct-to-LDS loads one block ahead (two stages), two loads per wave per
//    block (a dummy where the pieces run out, so every wave issues the same count);
//  - each wave's 96 W rows go to a wave-private LDS ring of 12 pieces, one per (column unit, K
//    half), one block ahead; a piece is refilled as soon as the wave has read it;
//  - a piece holds lane l's 16 operand bytes at 16 l (row l % 16, K bytes 16 (l / 16) .. + 15 of
//    its half), so every fragment read is one contiguous ds_read_b128;
//  - per column unit, two MFMAs per row unit (the two K halves), then the fold of that 16 x 16
//    tile (lane l: column l % 16, rows 4 (l / 16) + i in register i).
// Every wave issues the same loads in the same order, so its waits are fixed counts: 12 loads are
// issued after any A group or W piece before the wave waits for it.
// Epilogue, per 16-row unit: the f32 tile goes through LDS (two staging buffers of [16][772] floats in
// the rings' and A stages' space, one barrier a unit) into the row kernel's layout (a row per wave, lane l holding chunks l, l + 64, l + 128)
// and the norm_add runs with the row kernel's arithmetic (rowmath.h), two rows per wave, their
// residual rows loaded before the tile is staged.
#include <algorithm>

#include "common.h"
#include "rowmath.h"

namespace e2mi {

struct AnArgs {
    const int8_t *A;       // activations [M][lda] (K bytes a row)
    const float *as;       // their per-128 scales [M][K/128]
    const int8_t *W;       // weight rows [768][ldw]
    const float *ws;       // weight scales [768]
    const float *res;      // residual x [M][768]
    const float *gamma_a;  // gamma of the norm of y
    const float *gamma_n;  // gamma of the norm of x (null: x only)
    float *x_out;          // new residual x [M][768] (may alias res), or null
    float *xn_out;         // rmsnorm(x) * gamma_n [M][768], or null
    int8_t *q;             // its quantized rows [M][768], or null
    float *qs;             // their per-128 scales [M][6]
    float *y;              // the projection itself [M][768] f32, or null (parity tests)
    int lda, ldw, M, K;
    float eps;
};

constexpr int kAnD = 768;                  // output width: the hidden size
constexpr int kAnPitch = kAnD + 4;         // staging pitch in floats: rows 4 apart 16 banks apart
constexpr int kAnPiece = 1024;
constexpr int kAnRing = 12 * kAnPiece;     // one wave's W ring
constexpr int kAnUCMax = 5;
constexpr int kAnAStage = 2 * kAnUCMax * kAnPiece;
constexpr int kAnSStage = 128 * 4;         // activation scales of up to 128 rows
constexpr int kAnOffA = 8 * kAnRing;
constexpr int kAnOffS = kAnOffA + 2 * kAnAStage;
constexpr int kAnOffDummy = kAnOffS + 2 * kAnSStage;
constexpr int kAnLds = kAnOffDummy + 256;
constexpr int kAnStage = 16 * kAnPitch;    // one staged 16-row unit, floats
static_assert(2 * kAnStage * 4 <= kAnOffS, "two staged units fit in the W rings and A stages");
static_assert(kAnLds <= 160 * 1024, "LDS budget");

// A workgroup barrier that orders LDS only: __syncthreads() also waits for every global load and
// store in flight (s_waitcnt vmcnt(0)), which in the epilogue would drain the residual rows loaded
// ahead and the stores of the rows already normed at every staged unit.
__device__ inline void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int UC, bool FAST>
__global__ __launch_bounds__(512, 1) void k_gemm_an(const int *rows, AnArgs a) {
    static_assert(UC >= 1 && UC <= kAnUCMax, "1-5 row units a chunk");
    extern __shared__ __align__(16) unsigned char smem[];
    // the row count in 16-row units, cut evenly into ceil(U / UC) ranges of at most UC units (the
    // grid was sized for the host's row count, which bounds the device's)
    const int Mr = rows ? min(a.M, *rows) : a.M;
    const int U = (Mr + 15) >> 4, Gd = (U + UC - 1) / UC;
    if ((int)blockIdx.x >= Gd) return;
    const int u0 = (int)((long)U * blockIdx.x / Gd), u1 = (int)((long)U * (blockIdx.x + 1) / Gd);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nb = a.K >> 7;

    const v4u rA = rsrc_words(a.A, (uint32_t)((size_t)a.M * a.lda));
    const v4u rW = rsrc_words(a.W, (uint32_t)((size_t)kAnD * a.ldw));
    const v4u rS = rsrc_words(a.as, (uint32_t)((size_t)a.M * nb * 4));
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const lds_void *)smem);
    const uint32_t ring = lds0 + wave * kAnRing;
    const unsigned char *ringp = smem + wave * kAnRing;
    // per-lane source offsets: row l % 16 of a 16-row piece, bytes 16 (l / 16) of its K half; the row
    // base goes into the per-lane offset, so rows past M fall outside the buffer and read as zero
    const uint32_t vw = (uint32_t)(wave * 96 + (lane & 15)) * (uint32_t)a.ldw + (uint32_t)((lane >> 4) << 4);
    const uint32_t va = (uint32_t)(lane & 15) * (uint32_t)a.lda + (uint32_t)((lane >> 4) << 4);
    const uint32_t vs = (uint32_t)lane * (uint32_t)nb * 4;
    float wsr[6];
#pragma unroll
    for (int c = 0; c < 6; c++) wsr[c] = a.ws[wave * 96 + 16 * c + (lane & 15)];
    // their wait here, before any direct-to-LDS load: at a first use inside the K loop it would
    // be a vmcnt(0) that every block executes, draining the prefetched loads
#pragma unroll
    for (int c = 0; c < 6; c++) asm volatile("" ::"v"(wsr[c]));

    // this wave's two A-group loads (pieces, then the scales of rows 0-63 and 64-127) of block b
    // of the chunk at row m0 into stage st, a dummy past the group. The loads after a chunk's last
    // block fetch that block again into the stage no longer read, so no load depends on a branch.
    auto issue_a = [&](int m0, int b, int st) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int item = wave + 8 * j;
            if (item < 2 * UC) {
                const int r = item >> 1, h = item & 1;
                dma16(rA, lds0 + kAnOffA + st * kAnAStage + item * kAnPiece,
                      va + (uint32_t)(m0 + 16 * r) * (uint32_t)a.lda, (uint32_t)(b * 128 + 64 * h));
            } else if (item < 2 * UC + 2) {
                const int jj = item - 2 * UC;
                dma4(rS, lds0 + kAnOffS + st * kAnSStage + jj * 256,
                     vs + (uint32_t)(m0 + 64 * jj) * (uint32_t)nb * 4, (uint32_t)(b * 4));
            } else {
                dma4(rS, lds0 + kAnOffDummy, vs, 0);
            }
        }
    };
    // W pieces (c, 0) and (c, 1) of block b into this wave's ring, after the wave's reads of the
    // pieces they replace have completed (after a chunk's last block: that block's pieces again,
    // the bytes the slots already hold)
    auto issue_w = [&](int b, int c) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const uint32_t v = vw + (uint32_t)(16 * c) * (uint32_t)a.ldw;
        dma16(rW, ring + (2 * c) * kAnPiece, v, (uint32_t)(b * 128));
        dma16(rW, ring + (2 * c + 1) * kAnPiece, v, (uint32_t)(b * 128 + 64));
    };

    const v4i zero = {};

    {
        const int m0 = u0 * 16, nu = u1 - u0;
        float f[UC][6][4];
#pragma unroll
        for (int r = 0; r < UC; r++)
#pragma unroll
            for (int c = 0; c < 6; c++)
#pragma unroll
                for (int i = 0; i < 4; i++) f[r][c][i] = 0.f;
        issue_a(m0, 0, 0);
#pragma unroll
        for (int c = 0; c < 6; c++) issue_w(0, c);

        for (int b = 0; b < nb; b++) {
            // this wave's A group of block b has landed (12 W loads were issued after it), and
            // every wave's after the barrier, which also frees the other stage
            asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
            __syncthreads();
            const int bn = min(b + 1, nb - 1);  // the block whose loads this block issues
            issue_a(m0, bn, (b + 1) & 1);
            const unsigned char *ast = smem + kAnOffA + (b & 1) * kAnAStage;
            const float *sst = (const float *)(smem + kAnOffS + (b & 1) * kAnSStage);
            // the block's A fragments and the activation scales of the lane's four rows of each
            // row unit, read once for all six column units
            v4i af[UC][2];
            float4 s4[UC];
#pragma unroll
            for (int r = 0; r < UC; r++) {
#pragma unroll
                for (int h = 0; h < 2; h++) af[r][h] = *(const v4i *)(ast + (2 * r + h) * kAnPiece + 16 * lane);
                s4[r] = *(const float4 *)(sst + 16 * r + 4 * (lane >> 4));
            }
#pragma unroll
            for (int c = 0; c < 6; c++) {
                // pieces (c, *) of block b: 12 loads issued after them (the rest of block b's
                // pieces, block b + 1's A group and its pieces (0 .. c-1, *))
                asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
                const v4i b0 = *(const v4i *)(ringp + (2 * c) * kAnPiece + 16 * lane);
                const v4i b1 = *(const v4i *)(ringp + (2 * c + 1) * kAnPiece + 16 * lane);
                // the MFMAs of row unit r and the fold of unit r - 1 are one scheduling region
                // (no wait or load issue between them), so the fold's VALU work runs under the
                // MFMAs; the refill of the slots just read comes after the last fold
                v4i acc[UC];
                auto fold = [&](int r) {
                    const float sv[4] = {s4[r].x, s4[r].y, s4[r].z, s4[r].w};
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        // the reference's order: f = fma((float)acc, RN(as * ws), f); FAST folds as
                        // only and multiplies by ws once at the end
                        f[r][c][i] = __builtin_fmaf((float)acc[r][i], FAST ? sv[i] : __fmul_rn(sv[i], wsr[c]), f[r][c][i]);
                    }
                };
#pragma unroll
                for (int r = 0; r < UC; r++) {
                    acc[r] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[r][0], b0, zero, 0, 0, 0);
                    acc[r] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[r][1], b1, acc[r], 0, 0, 0);
                    if (r > 0) fold(r - 1);
                }
                fold(UC - 1);
                issue_w(bn, c);
            }
        }

        // epilogue: every load of the chunk has landed and every wave is past its last fragment
        // read before the rings become the staging area
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        float *stg = (float *)smem;
        float4 ga[3], gn[3];
#pragma unroll
        for (int i = 0; i < 3; i++) {
            ga[i] = ld4(a.gamma_a + 4 * (lane + 64 * i));
            gn[i] = a.gamma_n ? ld4(a.gamma_n + 4 * (lane + 64 * i)) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        // this wave's two rows of unit u and their residual rows, loaded one unit ahead of their use
        // (the loads of unit u + 1 are in flight while unit u is staged and normed). The row index is
        // clamped into the rows rather than the load skipped: a conditional load would make the
        // compiler copy its result at once, waiting for it; the rows past the count are not used.
        float4 rr[2][2][3];
        auto load_res = [&](int u, float4 (&r)[2][3]) {
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int m = min(m0 + 16 * u + 2 * wave + j, Mr - 1);
#pragma unroll
                for (int i = 0; i < 3; i++) r[j][i] = ld4(a.res + (size_t)m * kAnD + 4 * (lane + 64 * i));
            }
        };
        load_res(0, rr[0]);
#pragma unroll
        for (int u = 0; u < UC; u++) {
            if (u >= nu) break;
            if (u + 1 < UC) load_res(u + 1, rr[(u + 1) & 1]);
            const int mu = m0 + 16 * u;
            int mm[2];
#pragma unroll
            for (int j = 0; j < 2; j++) mm[j] = mu + 2 * wave + j;
#pragma unroll
            for (int c = 0; c < 6; c++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    stg[(u & 1) * kAnStage + (4 * (lane >> 4) + i) * kAnPitch + wave * 96 + 16 * c + (lane & 15)] =
                        FAST ? __fmul_rn(f[u][c][i], wsr[c]) : f[u][c][i];
            lds_barrier();
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int m = mm[j];
                if (m >= Mr) continue;
                const float *srow = stg + (u & 1) * kAnStage + (2 * wave + j) * kAnPitch;
                // x = rmsnorm(y) * gamma_a + res, the row kernel's steps (rowops.hip, ROW_ADDNORM)
                float4 v[3];
                float ss = 0.f;
#pragma unroll
                for (int i = 0; i < 3; i++) {
                    v[i] = ld4(srow + 4 * (lane + 64 * i));
                    ss += sumsq4(v[i]);
                }
                if (a.y) {
#pragma unroll
                    for (int i = 0; i < 3; i++) st4(a.y + (size_t)m * kAnD + 4 * (lane + 64 * i), v[i]);
                }
                float inv = rms_inv(group_sum<64>(ss), kAnD, a.eps);
                ss = 0.f;
#pragma unroll
                for (int i = 0; i < 3; i++) {
                    const float4 t = scale4(v[i], inv, ga[i]), r = rr[u & 1][j][i];
                    v[i] = make_float4(t.x + r.x, t.y + r.y, t.z + r.z, t.w + r.w);
                    ss += sumsq4(v[i]);
                }
                if (a.x_out) {
#pragma unroll
                    for (int i = 0; i < 3; i++) st4(a.x_out + (size_t)m * kAnD + 4 * (lane + 64 * i), v[i]);
                }
                if (!a.gamma_n) continue;
                inv = rms_inv(group_sum<64>(ss), kAnD, a.eps);
#pragma unroll
                for (int i = 0; i < 3; i++) {
                    v[i] = scale4(v[i], inv, gn[i]);
                    if (a.xn_out) st4(a.xn_out + (size_t)m * kAnD + 4 * (lane + 64 * i), v[i]);
                }
                if (!a.q) continue;
#pragma unroll
                for (int i = 0; i < 3; i++) {
                    const int c = lane + 64 * i;
                    const QScale s = qscale(group_max<32>(amax4(v[i])));
                    *(uint32_t *)(a.q + (size_t)m * kAnD + 4 * c) =
                        pack4(qbyte(v[i].x, s.inv), qbyte(v[i].y, s.inv), qbyte(v[i].z, s.inv), qbyte(v[i].w, s.inv));
                    if ((lane & 31) == 0) a.qs[(size_t)m * (kAnD / kQBlock) + (4 * c) / kQBlock] = s.sc;
                }
            }
        }
    }
}

// Row units a workgroup (UC) at the expected row count: the fewest rounds of the CUs that ranges of
// at most five units need, then the smallest UC that covers the rows in that many rounds.
int gemm_an_units(int rows) {
    const long U = std::max(1L, ((long)rows + 15) / 16), C = num_cus();
    const long rounds = (U + kAnUCMax * C - 1) / (kAnUCMax * C);
    return (int)std::max(1L, (U + rounds * C - 1) / (rounds * C));
}

template <int UC, bool FAST>
static int launch_an1(hipStream_t s, const int *rows, const AnArgs &a, int grid) {
    auto kern = k_gemm_an<UC, FAST>;
    static bool attr = false;
    if (!attr) {
        if (check_hip(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, kAnLds),
                      "gemm_add_norm lds attribute"))
            return -1;
        attr = true;
    }
    hipLaunchKernelGGL(kern, dim3(grid), dim3(512), kAnLds, s, rows, a);
    return check_hip(hipGetLastError(), "gemm_add_norm launch");
}

template <bool FAST>
static int launch_an(hipStream_t s, const int *rows, const AnArgs &a, int grid, int uc) {
    switch (uc) {
    case 1: return launch_an1<1, FAST>(s, rows, a, grid);
    case 2: return launch_an1<2, FAST>(s, rows, a, grid);
    case 3: return launch_an1<3, FAST>(s, rows, a, grid);
    case 4: return launch_an1<4, FAST>(s, rows, a, grid);
    default: return launch_an1<5, FAST>(s, rows, a, grid);
    }
}

bool gemm_fold_fast();

}  // namespace e2mi

using namespace e2mi;

extern "C" int e2mi_i8_gemm_add_norm_quant(e2mi_stream stream, const int8_t *qa, const float *a_scales,
                                           const e2mi_q8w *w, int M, const float *res, const float *gamma_add,
                                           const float *gamma_next, float eps, float *x_out, float *xn_out,
                                           int8_t *q, float *qs, float *y) {
    if (!w || !w->w || !w->scale || w->N != kAnD || w->K <= 0 || w->K % kQBlock || w->ld < w->K || w->ld % 16) {
        set_error("i8_gemm_add_norm_quant: the weight must have N = %d rows of K = a multiple of 128", kAnD);
        return -1;
    }
    if (w->bias || w->out_min > -1e30f || w->out_max < 1e30f) {
        set_error("i8_gemm_add_norm_quant: no bias or output clamp (the norm_add takes the plain projection)");
        return -1;
    }
    auto al = [](const void *p) { return !p || aligned16(p); };
    if (M <= 0 || !qa || !a_scales || !res || !gamma_add || !aligned16(qa) || !al(res) || !al(gamma_add) ||
        !al(gamma_next) || !al(x_out) || !al(xn_out) || !al(q) || !al(y) || (!q) != (!qs) ||
        ((q || xn_out) && !gamma_next)) {
        set_error("i8_gemm_add_norm_quant: null/misaligned pointer, or normed output without gamma_next");
        return -1;
    }
    if ((long)M * w->K >= (1L << 32) || (long)M * kAnD * 4 >= (1L << 31)) {
        set_error("i8_gemm_add_norm_quant: problem too large (M=%d K=%d)", M, w->K);
        return -1;
    }
    const DeviceRows dr = device_rows();
    if (dr.ptr && dr.mul != 1) {
        set_error("i8_gemm_add_norm_quant: a device row count with a multiplier");
        return -1;
    }
    AnArgs a = {};
    a.A = qa; a.as = a_scales; a.W = w->w; a.ws = w->scale; a.res = res; a.gamma_a = gamma_add;
    a.gamma_n = gamma_next; a.x_out = x_out; a.xn_out = xn_out; a.q = q; a.qs = qs; a.y = y;
    a.lda = w->K; a.ldw = w->ld; a.M = M; a.K = w->K; a.eps = eps;
    const int est = dr.ptr && dr.est > 0 && dr.est < M ? dr.est : M;
    const int uc = gemm_an_units(est);
    const int grid = ((M + 15) / 16 + uc - 1) / uc;
    hipStream_t s = (hipStream_t)stream;
    return gemm_fold_fast() ? launch_an<true>(s, dr.ptr, a, grid, uc) : launch_an<false>(s, dr.ptr, a, grid, uc);
}
