// gemm_an.hip — a projection that feeds a sublayer's norm_add, with the norm_add and the next GEMM's
// quantization in its epilogue (gfx950, wave64, v_mfma_i32_16x16x64_i8): the text tower's O and
// down projections (text.c:944-953) and, at the reference checkpoint's geometry, its PLE projection
// (text.c:955-961), for rows of D = 768 or 512 columns:
//
//   y = e2_i8_gemm(qa, W)                 the exact per-128 fold: y = sum_b fma((float)acc_b, RN(as*ws), .)
//   x = rmsnorm(y) * gamma_a + res        -> x_out (may alias res)          kernels.c:161-171
//       (SCALE: then x * post_scale, the layer scalar, text.c:959)
//   rmsnorm(x) * gamma_n                  -> q / qs per 128, and xn_out f32 when asked
//       (SCALE without gamma_n: x itself quantized, for the PLE gate GEMM)
//
// It gives the bits of e2mi_i8_gemm followed by e2mi_add_norm_quant (e2mi_add_norm_scale_quant)
// without the GEMM's f32 output, which the row kernel read straight back (M x D x 4 bytes written,
// then read, per projection).
//
// The norm needs whole rows, so a 512-thread workgroup (one per CU) owns whole D-wide rows: the
// (device) row count in 16-row units is cut evenly into ranges of at most UC units (80 rows), one
// per workgroup, UC chosen by the host so that the ranges fill the CUs in few rounds. Wave w holds
// columns D/8 w .. + D/8 - 1 (NCU = D/128 16-column units) of every row of its range as f32 running
// sums (UC x 4 NCU registers). K is walked in 128-deep blocks, one quantization block each, as the
// fold needs:
//  - A (2-KB pieces of 16 rows x the block's 128 bytes, one per row unit, each filled by two 1-KB
//    loads of 8 whole rows) and the block's activation scales go to LDS by direct-to-LDS loads one
//    block ahead (two stages), two loads per wave per block (a dummy where the pieces run out, so
//    every wave issues the same count);
//  - each wave's W rows go to a wave-private LDS ring of NCU pieces, one per column unit, one block
//    ahead; a piece is refilled as soon as the wave has read it;
//  - a piece holds its 16 rows' 128-byte K slices with the 16-byte chunk c of row r at slot
//    c ^ ((r >> 1) & 7), so each load reads 8 whole 128-byte lines (the earlier half-line pieces,
//    16 rows x 64 bytes a load, made the W loads the loop's bound) and the ds_read_b128 of lane l's
//    operand (row l % 16, chunk 4 h + l / 16 for K half h) is free of bank conflicts (64 banks, 16
//    lanes at a time: rows of equal parity share a bank half and take distinct slots);
//  - per column unit, two MFMAs per row unit (the two K halves), then the fold of that 16 x 16
//    tile (lane l: column l % 16, rows 4 (l / 16) + i in register i).
// Every wave issues the same loads in the same order, so its waits are fixed counts: 2 NCU loads
// are issued after any A group or W piece before the wave waits for it.
// Epilogue, per 16-row unit: the f32 tile goes through LDS (two staging buffers of [16][D + 4] floats
// in the rings' and A stages' space, one barrier a unit) into the row kernel's layout (a row per
// wave, lane l holding chunks l, l + 64, ...) and the norm_add runs with the row kernel's arithmetic
// (rowmath.h), two rows per wave, their residual rows loaded one unit ahead.
#include <algorithm>

#include "common.h"
#include "rowmath.h"

namespace e2mi {

struct AnArgs {
    const int8_t *A;       // activations [M][lda] (K bytes a row)
    const float *as;       // their per-128 scales [M][K/128]
    const int8_t *W;       // weight rows [D][ldw]
    const float *ws;       // weight scales [D]
    const float *res;      // residual x [M][D]
    const float *gamma_a;  // gamma of the norm of y
    const float *gamma_n;  // gamma of the norm of x (null: x only, or x itself quantized with SCALE)
    float *x_out;          // new residual x [M][D] (may alias res), or null
    float *xn_out;         // rmsnorm(x) * gamma_n [M][D], or null
    int8_t *q;             // quantized rows [M][D], or null
    float *qs;             // their per-128 scales [M][D/128]
    float *y;              // the projection itself [M][D] f32, or null (parity tests)
    int lda, ldw, M, K;
    float eps;
    float post_scale;      // SCALE: x scaled after the add
};

constexpr int kAnPiece = 1024;
constexpr int kAnUCMax = 5;
constexpr int kAnAStage = 2 * kAnUCMax * kAnPiece;
constexpr int kAnSStage = 128 * 4;  // activation scales of up to 128 rows

// The LDS layout of a workgroup for rows of D columns.
template <int D>
struct AnShape {
    static constexpr int NCU = D / 128;                // 16-column units per wave (8 waves)
    static constexpr int CPW = 16 * NCU;               // columns per wave
    static constexpr int NC = D / 256;                 // float4 chunks per lane of a row
    static constexpr int PITCH = D + 4;                // staging pitch in floats: rows 4 apart 16 banks apart
    static constexpr int STAGE = 16 * PITCH;           // one staged 16-row unit, floats
    static constexpr int RING = 2 * NCU * kAnPiece;    // one wave's W ring: a block's 2-KB pieces
    static constexpr int OFF_A = 8 * RING;
    static constexpr int OFF_S = OFF_A + 2 * kAnAStage;
    static constexpr int OFF_D = OFF_S + 2 * kAnSStage;
    static constexpr int LDS = OFF_D + 256;
    static_assert(D == 512 || D == 768, "rows of 512 or 768");
    static_assert(2 * STAGE * 4 <= OFF_S, "two staged units fit in the W rings and A stages");
    static_assert(LDS <= 160 * 1024, "LDS budget");
};

// A workgroup barrier that orders LDS only: __syncthreads() also waits for every global load and
// store in flight (s_waitcnt vmcnt(0)), which in the epilogue would drain the residual rows loaded
// ahead and the stores of the rows already normed at every staged unit.
__device__ inline void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int N>
__device__ inline void vm_wait() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }

template <int D, bool SCALE, int UC, bool FAST>
__global__ __launch_bounds__(512, 1) void k_gemm_an(const int *rows, AnArgs a) {
    using S = AnShape<D>;
    constexpr int NCU = S::NCU, NC = S::NC, NQB = D / kQBlock;
    static_assert(UC >= 1 && UC <= kAnUCMax, "1-5 row units a workgroup");
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
    const v4u rW = rsrc_words(a.W, (uint32_t)((size_t)D * a.ldw));
    const v4u rS = rsrc_words(a.as, (uint32_t)((size_t)a.M * nb * 4));
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const lds_void *)smem);
    const uint32_t ring = lds0 + wave * S::RING;
    const unsigned char *ringp = smem + wave * S::RING;
    // per-lane source offsets: load j of a piece writes its rows 8 j + l / 8, lane l fetching the
    // chunk of slot l % 8 of its row, (l % 8) ^ ((row >> 1) & 7) = (l % 8) ^ (4 j + l / 16). The A
    // loads of a wave all have j = wave % 2 (its items are wave and wave + 8); the row base goes into
    // the per-lane offset, so rows past M fall outside the buffer and read as zero
    const uint32_t lrow = (uint32_t)(lane >> 3);
    auto chunk = [&](int j) { return (uint32_t)(((lane & 7) ^ (4 * j + (lane >> 4))) << 4); };
    const uint32_t vw0 = (uint32_t)(wave * S::CPW + lrow) * (uint32_t)a.ldw + chunk(0);
    const uint32_t vw1 = (uint32_t)(wave * S::CPW + 8 + lrow) * (uint32_t)a.ldw + chunk(1);
    const uint32_t va = (uint32_t)(8 * (wave & 1) + lrow) * (uint32_t)a.lda + chunk(wave & 1);
    // lane l's operand in a piece: row l % 16, chunk 4 h + l / 16, at its swizzled slot
    uint32_t fo[2];
#pragma unroll
    for (int h = 0; h < 2; h++)
        fo[h] = (uint32_t)((lane & 15) * 128 + (((4 * h + (lane >> 4)) ^ ((lane & 15) >> 1)) << 4));
    const uint32_t vs = (uint32_t)lane * (uint32_t)nb * 4;
    float wsr[NCU];
#pragma unroll
    for (int c = 0; c < NCU; c++) wsr[c] = a.ws[wave * S::CPW + 16 * c + (lane & 15)];
    // their wait here, before any direct-to-LDS load: at a first use inside the K loop it would
    // be a vmcnt(0) that every block executes, draining the prefetched loads
#pragma unroll
    for (int c = 0; c < NCU; c++) asm volatile("" ::"v"(wsr[c]));

    // this wave's two A-group loads (pieces, then the scales of rows 0-63 and 64-127) of block b
    // of the range at row m0 into stage st, a dummy past the group. The loads after the last block
    // fetch that block again into the stage no longer read, so no load depends on a branch.
    auto issue_a = [&](int m0, int b, int st) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int item = wave + 8 * j;
            if (item < 2 * UC) {
                const int r = item >> 1;
                dma16(rA, lds0 + S::OFF_A + st * kAnAStage + item * kAnPiece,
                      va + (uint32_t)(m0 + 16 * r) * (uint32_t)a.lda, (uint32_t)(b * 128));
            } else if (item < 2 * UC + 2) {
                const int jj = item - 2 * UC;
                dma4(rS, lds0 + S::OFF_S + st * kAnSStage + jj * 256,
                     vs + (uint32_t)(m0 + 64 * jj) * (uint32_t)nb * 4, (uint32_t)(b * 4));
            } else {
                dma4(rS, lds0 + S::OFF_D, vs, 0);
            }
        }
    };
    // W piece c of block b (rows 0-7, then 8-15) into this wave's ring, after the wave's reads of
    // the piece it replaces have completed (after the last block: that block's piece again, the
    // bytes the slots already hold)
    auto issue_w = [&](int b, int c) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const uint32_t so = (uint32_t)(16 * c) * (uint32_t)a.ldw + (uint32_t)(b * 128);
        dma16(rW, ring + (2 * c) * kAnPiece, vw0, so);
        dma16(rW, ring + (2 * c + 1) * kAnPiece, vw1, so);
    };

    const v4i zero = {};
    const int m0 = u0 * 16, nu = u1 - u0;
    float f[UC][NCU][4];
#pragma unroll
    for (int r = 0; r < UC; r++)
#pragma unroll
        for (int c = 0; c < NCU; c++)
#pragma unroll
            for (int i = 0; i < 4; i++) f[r][c][i] = 0.f;
    issue_a(m0, 0, 0);
#pragma unroll
    for (int c = 0; c < NCU; c++) issue_w(0, c);

    for (int b = 0; b < nb; b++) {
        // this wave's A group of block b has landed (2 NCU W loads were issued after it), and every
        // wave's after the barrier, which also frees the other stage
        vm_wait<2 * NCU>();
        __syncthreads();
        const int bn = min(b + 1, nb - 1);  // the block whose loads this block issues
        issue_a(m0, bn, (b + 1) & 1);
        const unsigned char *ast = smem + S::OFF_A + (b & 1) * kAnAStage;
        const float *sst = (const float *)(smem + S::OFF_S + (b & 1) * kAnSStage);
        // the block's A fragments and the activation scales of the lane's four rows of each row
        // unit, read once for all the column units
        v4i af[UC][2];
        float4 s4[UC];
#pragma unroll
        for (int r = 0; r < UC; r++) {
#pragma unroll
            for (int h = 0; h < 2; h++) af[r][h] = *(const v4i *)(ast + 2 * r * kAnPiece + fo[h]);
            s4[r] = *(const float4 *)(sst + 16 * r + 4 * (lane >> 4));
        }
        // W fragments one column unit ahead: piece c of block b has 2 NCU loads issued after it
        // when its unit starts (the rest of block b's pieces, block b + 1's A group and its pieces
        // 0 .. c-1), so piece c + 1, read during unit c, has 2 NCU - 2
        vm_wait<2 * NCU>();
        v4i nb0 = *(const v4i *)(ringp + fo[0]);
        v4i nb1 = *(const v4i *)(ringp + fo[1]);
#pragma unroll
        for (int c = 0; c < NCU; c++) {
            const v4i b0 = nb0, b1 = nb1;
            if (c + 1 < NCU) {
                vm_wait<2 * NCU - 2>();
                nb0 = *(const v4i *)(ringp + 2 * (c + 1) * kAnPiece + fo[0]);
                nb1 = *(const v4i *)(ringp + 2 * (c + 1) * kAnPiece + fo[1]);
            }
            // the MFMAs of row unit r and the fold of unit r - 1 are one scheduling region (no wait
            // or load issue between them), so the fold's VALU work runs under the MFMAs; the refill
            // of the slots just read comes after the last fold
            v4i acc[UC];
            auto fold = [&](int r) {
                const float sv[4] = {s4[r].x, s4[r].y, s4[r].z, s4[r].w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    // the reference's order: f = fma((float)acc, RN(as * ws), f); FAST folds as only
                    // and multiplies by ws once at the end
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

    // epilogue: every load has landed and every wave is past its last fragment read before the
    // rings become the staging area
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    float *stg = (float *)smem;
    float4 ga[NC], gn[NC];
#pragma unroll
    for (int i = 0; i < NC; i++) {
        ga[i] = ld4(a.gamma_a + 4 * (lane + 64 * i));
        gn[i] = a.gamma_n ? ld4(a.gamma_n + 4 * (lane + 64 * i)) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    // this wave's two rows of unit u and their residual rows, loaded one unit ahead of their use (the
    // loads of unit u + 1 are in flight while unit u is staged and normed). The row index is clamped
    // into the rows rather than the load skipped: a conditional load would make the compiler copy
    // its result at once, waiting for it; the rows past the count are not used.
    float4 rr[2][2][NC];
    auto load_res = [&](int u, float4 (&r)[2][NC]) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int m = min(m0 + 16 * u + 2 * wave + j, Mr - 1);
#pragma unroll
            for (int i = 0; i < NC; i++) r[j][i] = ld4(a.res + (size_t)m * D + 4 * (lane + 64 * i));
        }
    };
    load_res(0, rr[0]);
#pragma unroll
    for (int u = 0; u < UC; u++) {
        if (u >= nu) break;
        if (u + 1 < UC) load_res(u + 1, rr[(u + 1) & 1]);
        float *su = stg + (u & 1) * S::STAGE;
#pragma unroll
        for (int c = 0; c < NCU; c++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                su[(4 * (lane >> 4) + i) * S::PITCH + wave * S::CPW + 16 * c + (lane & 15)] =
                    FAST ? __fmul_rn(f[u][c][i], wsr[c]) : f[u][c][i];
        lds_barrier();
        // both rows' staged values read before either is used (the reads are in bounds for rows
        // past the count, whose results are not stored)
        float4 vv[2][NC];
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int i = 0; i < NC; i++) vv[j][i] = ld4(su + (2 * wave + j) * S::PITCH + 4 * (lane + 64 * i));
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int m = m0 + 16 * u + 2 * wave + j;
            if (m >= Mr) continue;
            // x = rmsnorm(y) * gamma_a + res (SCALE: then * post_scale), the row kernel's steps
            // (rowops.hip, ROW_ADDNORM / ROW_ADDSCALE)
            float4 v[NC];
            float ss = 0.f;
#pragma unroll
            for (int i = 0; i < NC; i++) {
                v[i] = vv[j][i];
                ss += sumsq4(v[i]);
            }
            if (a.y) {
#pragma unroll
                for (int i = 0; i < NC; i++) st4(a.y + (size_t)m * D + 4 * (lane + 64 * i), v[i]);
            }
            float inv = rms_inv(group_sum<64>(ss), D, a.eps);
            ss = 0.f;
#pragma unroll
            for (int i = 0; i < NC; i++) {
                const float4 t = scale4(v[i], inv, ga[i]), r = rr[u & 1][j][i];
                v[i] = make_float4(t.x + r.x, t.y + r.y, t.z + r.z, t.w + r.w);
                if constexpr (SCALE)
                    v[i] = make_float4(__fmul_rn(v[i].x, a.post_scale), __fmul_rn(v[i].y, a.post_scale),
                                       __fmul_rn(v[i].z, a.post_scale), __fmul_rn(v[i].w, a.post_scale));
                ss += sumsq4(v[i]);
            }
            if (a.x_out) {
#pragma unroll
                for (int i = 0; i < NC; i++) st4(a.x_out + (size_t)m * D + 4 * (lane + 64 * i), v[i]);
            }
            if (!SCALE && !a.gamma_n) continue;
            if (a.gamma_n) {
                inv = rms_inv(group_sum<64>(ss), D, a.eps);
#pragma unroll
                for (int i = 0; i < NC; i++) {
                    v[i] = scale4(v[i], inv, gn[i]);
                    if (a.xn_out) st4(a.xn_out + (size_t)m * D + 4 * (lane + 64 * i), v[i]);
                }
            }
            if (!a.q) continue;
#pragma unroll
            for (int i = 0; i < NC; i++) {
                const int c = lane + 64 * i;
                const QScale s = qscale(group_max<32>(amax4(v[i])));
                *(uint32_t *)(a.q + (size_t)m * D + 4 * c) =
                    pack4_magic(v[i].x, v[i].y, v[i].z, v[i].w, s.inv);
                if ((lane & 31) == 0) a.qs[(size_t)m * NQB + (4 * c) / kQBlock] = s.sc;
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

// One round of the CUs covers the rows (at most five units a workgroup): the engine's condition for
// these kernels. With more rows, every workgroup still fetches the whole weight for its few rows
// (1 MB at K = 2048 and 512-wide rows for 48 rows), which outweighs the f32 round trip saved: the
// reference geometry's batch of 16 x 2048 (about 24.5k rows, two rounds) ran 3 % slower fused.
bool gemm_an_fits(int rows) { return ((long)rows + 15) / 16 <= (long)kAnUCMax * num_cus(); }

template <int D, bool SCALE, int UC, bool FAST>
static int launch_an1(hipStream_t s, const int *rows, const AnArgs &a, int grid) {
    auto kern = k_gemm_an<D, SCALE, UC, FAST>;
    static bool attr = false;
    if (!attr) {
        if (check_hip(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                          AnShape<D>::LDS),
                      "gemm_add_norm lds attribute"))
            return -1;
        attr = true;
    }
    hipLaunchKernelGGL(kern, dim3(grid), dim3(512), AnShape<D>::LDS, s, rows, a);
    return check_hip(hipGetLastError(), "gemm_add_norm launch");
}

template <int D, bool SCALE, bool FAST>
static int launch_an(hipStream_t s, const int *rows, const AnArgs &a, int grid, int uc) {
    switch (uc) {
    case 1: return launch_an1<D, SCALE, 1, FAST>(s, rows, a, grid);
    case 2: return launch_an1<D, SCALE, 2, FAST>(s, rows, a, grid);
    case 3: return launch_an1<D, SCALE, 3, FAST>(s, rows, a, grid);
    case 4: return launch_an1<D, SCALE, 4, FAST>(s, rows, a, grid);
    default: return launch_an1<D, SCALE, 5, FAST>(s, rows, a, grid);
    }
}

bool gemm_fold_fast();

// The two entry points' checks and launch. SCALE: the norm_add of the reference checkpoint's PLE
// layers (x scaled after the add; without gamma_next, x itself quantized).
static int gemm_add_norm(hipStream_t s, const int8_t *qa, const float *a_scales, const e2mi_q8w *w, int M,
                         const float *res, const float *gamma_add, float post_scale, const float *gamma_next,
                         float eps, float *x_out, float *xn_out, int8_t *q, float *qs, float *y, bool scale,
                         const char *who) {
    if (!w || !w->w || !w->scale || (w->N != 512 && w->N != 768) || w->K <= 0 || w->K % kQBlock ||
        w->ld < w->K || w->ld % 16) {
        set_error("%s: the weight must have N = 512 or 768 rows of K = a multiple of 128", who);
        return -1;
    }
    if (w->bias || w->out_min > -1e30f || w->out_max < 1e30f) {
        set_error("%s: no bias or output clamp (the norm_add takes the plain projection)", who);
        return -1;
    }
    if (scale && w->N != 512) {
        set_error("%s: the scaled norm_add is built for 512-wide rows (the PLE geometry)", who);
        return -1;
    }
    auto al = [](const void *p) { return !p || aligned16(p); };
    if (M <= 0 || !qa || !a_scales || !res || !gamma_add || !aligned16(qa) || !al(res) || !al(gamma_add) ||
        !al(gamma_next) || !al(x_out) || !al(xn_out) || !al(q) || !al(y) || (!q) != (!qs) ||
        (xn_out && !gamma_next) || (q && !gamma_next && !scale)) {
        set_error("%s: null/misaligned pointer, or normed output without gamma_next", who);
        return -1;
    }
    const int D = w->N;
    if ((long)M * w->K >= (1L << 32) || (long)M * D * 4 >= (1L << 31)) {
        set_error("%s: problem too large (M=%d K=%d)", who, M, w->K);
        return -1;
    }
    const DeviceRows dr = device_rows();
    if (dr.ptr && dr.mul != 1) {
        set_error("%s: a device row count with a multiplier", who);
        return -1;
    }
    AnArgs a = {};
    a.A = qa; a.as = a_scales; a.W = w->w; a.ws = w->scale; a.res = res; a.gamma_a = gamma_add;
    a.gamma_n = gamma_next; a.x_out = x_out; a.xn_out = xn_out; a.q = q; a.qs = qs; a.y = y;
    a.lda = w->K; a.ldw = w->ld; a.M = M; a.K = w->K; a.eps = eps; a.post_scale = post_scale;
    const int est = dr.ptr && dr.est > 0 && dr.est < M ? dr.est : M;
    const int uc = gemm_an_units(est);
    const int grid = ((M + 15) / 16 + uc - 1) / uc;
    const bool fast = gemm_fold_fast();
    if (scale)
        return fast ? launch_an<512, true, true>(s, dr.ptr, a, grid, uc) : launch_an<512, true, false>(s, dr.ptr, a, grid, uc);
    if (D == 512)
        return fast ? launch_an<512, false, true>(s, dr.ptr, a, grid, uc) : launch_an<512, false, false>(s, dr.ptr, a, grid, uc);
    return fast ? launch_an<768, false, true>(s, dr.ptr, a, grid, uc) : launch_an<768, false, false>(s, dr.ptr, a, grid, uc);
}

}  // namespace e2mi

using namespace e2mi;

extern "C" int e2mi_i8_gemm_add_norm_quant(e2mi_stream stream, const int8_t *qa, const float *a_scales,
                                           const e2mi_q8w *w, int M, const float *res, const float *gamma_add,
                                           const float *gamma_next, float eps, float *x_out, float *xn_out,
                                           int8_t *q, float *qs, float *y) {
    return gemm_add_norm((hipStream_t)stream, qa, a_scales, w, M, res, gamma_add, 1.0f, gamma_next, eps, x_out,
                         xn_out, q, qs, y, false, "i8_gemm_add_norm_quant");
}

extern "C" int e2mi_i8_gemm_add_norm_scale_quant(e2mi_stream stream, const int8_t *qa, const float *a_scales,
                                                 const e2mi_q8w *w, int M, const float *res, const float *gamma_add,
                                                 float post_scale, const float *gamma_next, float eps, float *x_out,
                                                 float *xn_out, int8_t *q, float *qs, float *y) {
    return gemm_add_norm((hipStream_t)stream, qa, a_scales, w, M, res, gamma_add, post_scale, gamma_next, eps,
                         x_out, xn_out, q, qs, y, true, "i8_gemm_add_norm_scale_quant");
}
