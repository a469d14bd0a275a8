// attn_i8.hip — the int8 attention variant on gfx950 int8 MFMA (v_mfma_i32_32x32x32_i8), for
// packed batches of all-valid sequences.
//
// Reference semantics (text.c:638-700 attb_i8, selected by dispatch.c's attention rule for long
// sequences): per query head h (kv head h / (H / KV)) of a sequence of S rows,
//   Q rows quantized per 128 of D (the activation quantizer), K quantized per key row and V^T per
//   dim over the sequence's keys (the weight quantizer, e2_q8w_from_f32), both with scale
//   amax * RN(1/127) and bytes rne(x * RN(127 / amax));
//   scores[i][j] = fold over D's two 128-blocks b of fma((float)acc_b, RN(qs[i][b] * ks[j]), .);
//   p = softmax(scores[i]) (max, exp, sum, then p = e * RN(1 / sum));
//   P quantized per 128-key block of the row (the activation quantizer on p);
//   ctx[i][d] = fold over key blocks b of fma((float)acc_b, RN(ps[i][b] * vs[d]), .).
// The context is then quantized per (row, 128 dims) for the O-projection GEMM, as in attn.hip.
//
// Kernels:
//   k_i8_qk_prep   one wave per (row, q head | k head): Q per 128, K per row (float4 per lane)
//   k_i8_vmax      per (sequence, kv head, 64-row chunk): column maxima of V
//   k_i8_vquant    per (sequence, kv head, 32-row chunk): V^T bytes (thread d writes 32 bytes of
//                  row d of V^T [KV][D][M]) and the per-dim scales
//   k_attn_i8      a workgroup is (sequence, head, 128 queries), 4 waves of 32 queries, one wave
//                  per SIMD (the two f32 context sets need 256 registers). Pass 1 walks the key
//                  tiles for each query's softmax max and sum (online); pass 2 walks them again per
//                  128-key block: the block's probabilities (recomputed, bit-identical scores),
//                  their quantization with the block's scale (the largest probability is the one of
//                  the largest score: exp and the multiply by 1/sum are monotone), then
//                  O^T += V^T P^T on int8 MFMA with int32 accumulators folded into f32 once per
//                  block. S^T = K Q^T as in attn.hip: K tile rows are permuted so a lane's 16
//                  logits are 16 consecutive keys of its query, exactly its P^T operand bytes.
#include "common.h"

namespace e2mi {

constexpr int kI8D = 256;                           // head dim
constexpr int kI8Tile = 8192;                       // K [32 keys][256] or V^T [256 d][32 keys]
constexpr int kI8Buf = kI8Tile + 256;               // + the tile's key scales (64 loaded, 32 used)
constexpr int kI8Ring = 3;                          // tile buffers: loads two tiles ahead
constexpr int kAttnI8Lds = kI8Ring * kI8Buf + kI8D * 4;  // + the sequence's V scales

// ---------------------------------------------------------------- Q and K quantization
struct I8PrepArgs {
    const float *q32, *k32, *v32;  // [M][H*D], [M][KV*D], [M][KV*D]
    int8_t *q8;                    // [M][H*D]
    float *qs;                     // [M][H*2]
    int8_t *k8;                    // [M][KV*D]
    float *ks;                     // [M][KV]
    int8_t *vt8;                   // [KV][D][2 M]: sequence b's keys at columns 2 start[b] + j
    float *vpart;                  // [B][KV][nch][D] column maxima of 64-row chunks
    float *vs;                     // [B][KV][D]
    const int32_t *seq_start, *seq_len;
    int M, H, KV, nch;
};

__global__ __launch_bounds__(256) void k_i8_qk_prep(I8PrepArgs a) {
    const int lane = threadIdx.x & 63;
    const long item = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int per = a.H + a.KV;
    if (item >= (long)a.M * per) return;
    const int row = (int)(item / per), j = (int)(item % per);
    if (j < a.H) {
        // Q: lanes 0-31 hold block 0 (d < 128), lanes 32-63 block 1
        const float4 x = *(const float4 *)(a.q32 + (size_t)row * a.H * kI8D + j * kI8D + 4 * lane);
        const float am = group_max<32>(fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w))));
        const QScale s = qscale(am);
        *(uint32_t *)(a.q8 + (size_t)row * a.H * kI8D + j * kI8D + 4 * lane) = pack4_magic(x.x, x.y, x.z, x.w, s.inv);
        if ((lane & 31) == 0) a.qs[(size_t)row * a.H * 2 + j * 2 + (lane >> 5)] = s.sc;
    } else {
        // K: one scale per key row over all of D (the weight quantizer)
        const int kv = j - a.H;
        const float4 x = *(const float4 *)(a.k32 + (size_t)row * a.KV * kI8D + kv * kI8D + 4 * lane);
        const float am = group_max<64>(fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w))));
        const QScale s = qscale(am);
        *(uint32_t *)(a.k8 + (size_t)row * a.KV * kI8D + kv * kI8D + 4 * lane) = pack4_magic(x.x, x.y, x.z, x.w, s.inv);
        if (lane == 0) a.ks[(size_t)row * a.KV + kv] = s.sc;
    }
}

// ---------------------------------------------------------------- V^T quantization
// grid (B * KV, nch): column maxima of rows [64 c, 64 c + 64) of the sequence, thread = dim
__global__ __launch_bounds__(256) void k_i8_vmax(I8PrepArgs a) {
    const int b = blockIdx.x / a.KV, kv = blockIdx.x % a.KV, c = blockIdx.y, d = threadIdx.x;
    const int L = a.seq_len[b], r0 = 64 * c;
    if (r0 >= L) return;
    const int r1 = min(L, r0 + 64);
    const size_t st = (size_t)a.KV * kI8D;
    const float *src = a.v32 + ((size_t)a.seq_start[b] + r0) * st + kv * kI8D + d;
    float m8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int r = r0;
    for (; r + 8 <= r1; r += 8, src += 8 * st)
#pragma unroll
        for (int e = 0; e < 8; e++) m8[e] = fmaxf(m8[e], fabsf(src[e * st]));
    for (; r < r1; r++, src += st) m8[0] = fmaxf(m8[0], fabsf(*src));
    float am = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) am = fmaxf(am, m8[e]);
    a.vpart[((size_t)blockIdx.x * a.nch + c) * kI8D + d] = am;
}

// grid (B * KV, ceil(max_len / 32)): thread d reduces its column's chunk maxima, then quantizes rows
// [32 c, 32 c + 32) of the sequence into 32 bytes of V^T row d
__global__ __launch_bounds__(256) void k_i8_vquant(I8PrepArgs a) {
    const int b = blockIdx.x / a.KV, kv = blockIdx.x % a.KV, c = blockIdx.y, d = threadIdx.x;
    const int L = a.seq_len[b], r0 = 32 * c;
    if (r0 >= L) return;
    const int nc = (L + 63) / 64;
    const float *part = a.vpart + (size_t)blockIdx.x * a.nch * kI8D + d;
    float am = 0.f;
    for (int i = 0; i < nc; i++) am = fmaxf(am, part[(size_t)i * kI8D]);
    const QScale s = qscale(am);
    if (c == 0) a.vs[(size_t)blockIdx.x * kI8D + d] = s.sc;
    const int n = min(32, L - r0);
    const size_t row0 = (size_t)a.seq_start[b] + r0;
    const float *src = a.v32 + row0 * a.KV * kI8D + kv * kI8D + d;
    uint32_t w[8];
#pragma unroll
    for (int g = 0; g < 8; g++) {
        float x[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int r = 4 * g + e;
            x[e] = r < n ? src[(size_t)r * a.KV * kI8D] : 0.f;
        }
        w[g] = pack4_magic(x[0], x[1], x[2], x[3], s.inv);
    }
    // sequence b's keys start at column 2 start[b] (16-byte aligned; its columns end before the
    // next sequence's, which starts at least L rows later): whole 16-byte chunks are its own
    int8_t *dst = a.vt8 + ((size_t)kv * kI8D + d) * 2 * a.M + 2 * (size_t)a.seq_start[b] + r0;
#pragma unroll
    for (int g = 0; g < 2; g++)
        if (16 * g < n) *(uint4 *)(dst + 16 * g) = make_uint4(w[4 * g], w[4 * g + 1], w[4 * g + 2], w[4 * g + 3]);
}

// ---------------------------------------------------------------- attention
struct AttnI8Args {
    const int8_t *q8;
    const float *qs;
    const int8_t *k8;
    const float *ks;
    const int8_t *vt8;
    const float *vs;
    int8_t *cq;            // [M][H*D] int8 context
    float *cs;             // [M][H*D/128]
    float *c32;            // optional [M][H*D] f32 context
    const int32_t *seq_start, *seq_len;
    const int32_t *work;   // optional: b | h << 16 | query block << 24 per workgroup, negative idle
    int M, H, KV;
};

__global__ __launch_bounds__(256, 1) void k_attn_i8(AttnI8Args a) {
    extern __shared__ __align__(16) unsigned char smem[];
    int qb = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    if (a.work) {
        const int item = a.work[blockIdx.x];
        if (item < 0) return;
        b = item & 0xffff;
        h = (item >> 16) & 0xf;  // (one part: work_entry(b, h, 0, 1, qb))
        qb = item >> 24;
    }
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, half = lane >> 5;
    const int HD = a.H * kI8D, kvh = h / (a.H / a.KV);
    const size_t row0 = (size_t)a.seq_start[b];
    const int Sk = a.seq_len[b];
    if (qb * 128 >= Sk) return;

    const int qi = qb * 128 + w * 32 + (lane & 31);  // this lane's query
    const int qc = min(qi, Sk - 1);
    // Q^T operand (B of S^T = K Q^T): the query's d = 32 kk + 16 half .. + 16
    v4i qf[8];
    {
        const int8_t *qp = a.q8 + (row0 + qc) * HD + h * kI8D + 16 * half;
#pragma unroll
        for (int kk = 0; kk < 8; kk++) qf[kk] = *(const v4i *)(qp + 32 * kk);
    }
    const float qs0 = a.qs[(row0 + qc) * a.H * 2 + h * 2], qs1 = a.qs[(row0 + qc) * a.H * 2 + h * 2 + 1];
    float *vs_l = (float *)(smem + kI8Ring * kI8Buf);
    vs_l[tid] = a.vs[((size_t)b * a.KV + kvh) * kI8D + tid];
    // the loads above complete here, under a wait the compiler sees: otherwise its wait would sit
    // inside the tile loop and also cover the tile loads in flight
    __builtin_amdgcn_s_waitcnt(0x0F70);

    const int ntiles = (Sk + 31) / 32, nblk = (ntiles + 3) / 4;
    const uint32_t rowB = (uint32_t)a.KV * kI8D;
    const v4u rK = rsrc_words(a.k8 + row0 * rowB + kvh * kI8D, (uint32_t)Sk * rowB);
    const v4u rKS = rsrc_words(a.ks + row0 * a.KV + kvh, (uint32_t)Sk * a.KV * 4);
    const v4u rV = rsrc_words(a.vt8 + (size_t)kvh * kI8D * 2 * a.M, (uint32_t)((size_t)kI8D * 2 * a.M));
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const lds_void *)smem);
    const int wu = __builtin_amdgcn_readfirstlane(w);
    // K tile: load i (wave w issues 2 w, 2 w + 1) fills physical rows rho = 4 i + lane / 16, 16-byte
    // position lane % 16 holding chunk (lane % 16) ^ (rho % 16), of key kappa(rho) =
    // 16 ((rho / 4) % 2) + 4 (rho / 8) + rho % 4 = 16 (i % 2) + 4 (i / 2) + lane / 16
    uint32_t kvo[2];
#pragma unroll
    for (int e = 0; e < 2; e++) {
        const int i = 2 * wu + e;
        kvo[e] = (uint32_t)(lane >> 4) * rowB + (uint32_t)(((lane & 15) ^ ((4 * i + (lane >> 4)) & 15)) << 4);
    }
    // V^T tile: load i (wave w issues 2 w, 2 w + 1) fills rows d = 32 i + lane / 2, position lane % 2
    // holding chunk (lane % 2) ^ ((d / 8) % 2) = (lane % 2) ^ ((lane / 16) % 2)
    const uint32_t vpitch = 2u * (uint32_t)a.M;
    const uint32_t vvo = (uint32_t)(lane >> 1) * vpitch + (uint32_t)(((lane & 1) ^ ((lane >> 4) & 1)) << 4);
    // every tile costs each wave 3 loads (K: 2 row loads + the key scales, which all waves load
    // into the same place; V^T: 2 row loads + a spare scale load), so a wait for "all but the
    // next tile's loads" is vmcnt(3)
    auto issue = [&](bool isk, int kt, int buf) {
        const int k0 = kt * 32;
        const uint32_t base = lds0 + (uint32_t)(buf * kI8Buf);
        if (isk) {
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int i = 2 * wu + e;
                dma16(rK, base + i * 1024, kvo[e], (uint32_t)(k0 + 16 * (i & 1) + 4 * (i >> 1)) * rowB);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int i = 2 * wu + e;
                dma16(rV, base + i * 1024, vvo, (uint32_t)(32 * i) * vpitch + (uint32_t)(2 * row0 + k0));
            }
        }
        dma4(rKS, base + kI8Tile, (uint32_t)lane * a.KV * 4, (uint32_t)k0 * a.KV * 4);
    };
    // the tile stream: pass 1's K tiles, then per 128-key block its K tiles and its V^T tiles
    const int NS = 3 * ntiles;
    auto desc = [&](int n, bool &isk, int &kt) {
        if (n < ntiles) {
            isk = true;
            kt = n;
            return;
        }
        const int m = n - ntiles, full = 8 * (nblk - 1);
        if (m < full) {
            isk = (m & 7) < 4;
            kt = 4 * (m >> 3) + (m & 3);
            return;
        }
        const int ntl = ntiles - 4 * (nblk - 1), j = m - full;
        isk = j < ntl;
        kt = 4 * (nblk - 1) + (isk ? j : j - ntl);
    };
    int sn = 0;  // stream position of the step being computed
    // wait for step sn's tile (every wave's), release the buffer of step sn - 1 and refill it with
    // step sn + 2's tile; returns step sn's buffer
    auto begin_step = [&]() -> const unsigned char * {
        if (sn + 1 < NS) asm volatile("s_waitcnt vmcnt(3)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (sn + 2 < NS) {
            bool isk;
            int kt;
            desc(sn + 2, isk, kt);
            issue(isk, kt, (sn + 2) % kI8Ring);
        }
        const unsigned char *sb = smem + (sn % kI8Ring) * kI8Buf;
        ++sn;
        return sb;
    };
    // fragment offsets: K row rho = lane % 32, chunk 2 kk + half at position (2 kk + half) ^ (rho % 16);
    // V^T row d = 32 dt + lane % 32, chunk half at position half ^ ((d / 8) % 2)
    const int rho = lane & 31;
    const int vrd = rho * 32 + ((half ^ ((rho >> 3) & 1)) << 4);

    // one K tile: S^T (8 MFMAs, two 128-d blocks), folded like the reference's GEMM, keys past the
    // sequence at -inf. s[r] is key 16 half + r of the tile.
    auto scores = [&](const unsigned char *sb, int k0, float (&s)[16]) {
        v16i acc0 = (v16i){}, acc1 = (v16i){};
#pragma unroll
        for (int kk = 0; kk < 8; kk++) {
            const v4i kf = *(const v4i *)(sb + rho * 256 + (((2 * kk + half) ^ (rho & 15)) << 4));
            if (kk < 4) acc0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf, qf[kk], acc0, 0, 0, 0);
            else acc1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf, qf[kk], acc1, 0, 0, 0);
        }
        const float *ksl = (const float *)(sb + kI8Tile) + 16 * half;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const float4 k4 = *(const float4 *)(ksl + 4 * g);
            const float kv4[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int r = 4 * g + e;
                const float f = __builtin_fmaf((float)acc0[r], __fmul_rn(qs0, kv4[e]), 0.f);
                const float x = __builtin_fmaf((float)acc1[r], __fmul_rn(qs1, kv4[e]), f);
                s[r] = (k0 + 16 * half + r < Sk) ? x : -INFINITY;
            }
        }
    };

    for (int n = 0; n < 2 && n < NS; n++) {
        bool isk;
        int kt;
        desc(n, isk, kt);
        issue(isk, kt, n);
    }
    float mrun = -INFINITY, lrun = 0.f;
    for (int kt = 0; kt < ntiles; kt++) {
        const unsigned char *sb = begin_step();
        float s[16];
        scores(sb, kt * 32, s);
        float mloc = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; r++) mloc = fmaxf(mloc, s[r]);
        mloc = fmaxf(mloc, xor_lane<32>(mloc));
        const float mnew = fmaxf(mrun, mloc);
        if (mnew > -INFINITY) {
            float ps = 0.f;
#pragma unroll
            for (int r = 0; r < 16; r++) ps += s[r] == -INFINITY ? 0.f : __expf(s[r] - mnew);
            lrun = (mrun == -INFINITY ? 0.f : lrun * __expf(mrun - mnew)) + ps;
            mrun = mnew;
        }
    }
    const float ltot = lrun + xor_lane<32>(lrun);
    const float inv_l = ltot > 0.f ? __fdiv_rn(1.0f, ltot) : 0.f;

    v16i acco[8];
    float of[8][16];
#pragma unroll
    for (int dt = 0; dt < 8; dt++) {
        acco[dt] = (v16i){};
#pragma unroll
        for (int r = 0; r < 16; r++) of[dt][r] = 0.f;
    }
    for (int blk = 0; blk < nblk; blk++) {
        const int nt = min(4, ntiles - 4 * blk);
        float pv[4][16];
        float am = 0.f;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            if (t < nt) {
                const unsigned char *sb = begin_step();
                float s[16];
                scores(sb, (4 * blk + t) * 32, s);
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const float e = s[r] == -INFINITY ? 0.f : __expf(s[r] - mrun);
                    pv[t][r] = __fmul_rn(e, inv_l);
                    am = fmaxf(am, pv[t][r]);
                }
            } else {
#pragma unroll
                for (int r = 0; r < 16; r++) pv[t][r] = 0.f;
            }
        }
        am = fmaxf(am, xor_lane<32>(am));
        const QScale ps = qscale(am);
        v4i pq[4];
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int g = 0; g < 4; g++)
                pq[t][g] = (int)pack4_magic(pv[t][4 * g], pv[t][4 * g + 1], pv[t][4 * g + 2], pv[t][4 * g + 3], ps.inv);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            if (t < nt) {
                const unsigned char *sb = begin_step();
#pragma unroll
                for (int dt = 0; dt < 8; dt++) {
                    const v4i vf = *(const v4i *)(sb + dt * 32 * 32 + vrd);
                    acco[dt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(vf, pq[t], acco[dt], 0, 0, 0);
                }
            }
        }
        // fold the block: d = 32 dt + 8 (r / 4) + 4 half + r % 4
#pragma unroll
        for (int dt = 0; dt < 8; dt++) {
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const float4 v4 = *(const float4 *)(vs_l + 32 * dt + 8 * g + 4 * half);
                const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
                for (int e = 0; e < 4; e++)
                    of[dt][4 * g + e] = __builtin_fmaf((float)acco[dt][4 * g + e], __fmul_rn(ps.sc, vv[e]), of[dt][4 * g + e]);
            }
            acco[dt] = (v16i){};
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    if (qi >= Sk) return;  // rows past the sequence belong to the next one
    const size_t orow = row0 + qi;
#pragma unroll
    for (int blk = 0; blk < 2; blk++) {
        float am = 0.f;
#pragma unroll
        for (int dt = 4 * blk; dt < 4 * blk + 4; dt++)
#pragma unroll
            for (int r = 0; r < 16; r++) am = fmaxf(am, fabsf(of[dt][r]));
        am = fmaxf(am, xor_lane<32>(am));
        const QScale qs = qscale(am);
#pragma unroll
        for (int dt = 4 * blk; dt < 4 * blk + 4; dt++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int d = 32 * dt + 8 * g + 4 * half;
                *(uint32_t *)(a.cq + orow * HD + h * kI8D + d) =
                    pack4_magic(of[dt][4 * g], of[dt][4 * g + 1], of[dt][4 * g + 2], of[dt][4 * g + 3], qs.inv);
                if (a.c32)
                    *(float4 *)(a.c32 + orow * HD + h * kI8D + d) =
                        make_float4(of[dt][4 * g], of[dt][4 * g + 1], of[dt][4 * g + 2], of[dt][4 * g + 3]);
            }
        if (half == 0) a.cs[orow * (HD / kQBlock) + h * 2 + blk] = qs.sc;
    }
}

static size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

struct I8Ws {
    size_t q8, qs, k8, ks, vt8, vpart, vs, total;
};
static I8Ws i8_ws(int M, int B, int max_len, int H, int KV) {
    I8Ws w;
    const int nch = (max_len + 63) / 64;
    w.q8 = 0;
    w.qs = w.q8 + al256((size_t)M * H * kI8D);
    w.k8 = w.qs + al256((size_t)M * H * 2 * 4);
    w.ks = w.k8 + al256((size_t)M * KV * kI8D);
    w.vt8 = w.ks + al256((size_t)M * KV * 4);
    w.vpart = w.vt8 + al256((size_t)KV * kI8D * 2 * M);
    w.vs = w.vpart + al256((size_t)B * KV * nch * kI8D * 4);
    w.total = w.vs + al256((size_t)B * KV * kI8D * 4);
    return w;
}

}  // namespace e2mi

using namespace e2mi;

extern "C" size_t e2mi_attention_i8_workspace_bytes(int M, int B, int max_len, int H, int KV) {
    if (M <= 0 || B <= 0 || max_len <= 0 || H <= 0 || KV <= 0) return 0;
    return i8_ws(M, B, max_len, H, KV).total;
}

extern "C" int e2mi_attention_i8_packed(e2mi_stream stream, const float *q32, const float *k32,
                                        const float *v32, int M, const int32_t *seq_start,
                                        const int32_t *seq_len, int B, int max_len, int H, int KV,
                                        int D, void *workspace, int8_t *ctx_q, float *ctx_s,
                                        float *ctx32, const int32_t *work, int n_work) {
    if (D != kI8D || B <= 0 || M <= 0 || max_len <= 0 || H <= 0 || KV <= 0 || H % KV || M % 16) {
        set_error("attention_i8_packed: needs head_dim 256, H %% KV == 0 and M %% 16 == 0 "
                  "(B=%d M=%d H=%d KV=%d D=%d)", B, M, H, KV, D);
        return -1;
    }
    if (!q32 || !k32 || !v32 || !seq_start || !seq_len || !workspace || !ctx_q || !ctx_s ||
        !aligned16(q32) || !aligned16(k32) || !aligned16(v32) || ((uintptr_t)workspace & 255) ||
        ((uintptr_t)ctx_q & 3) || (ctx32 && !aligned16(ctx32))) {
        set_error("attention_i8_packed: null or misaligned pointer");
        return -1;
    }
    if ((size_t)kI8D * 2 * M >= 0x7fffffffu || (size_t)M * KV * kI8D >= 0x7fffffffu) {
        set_error("attention_i8_packed: too many rows");
        return -1;
    }
    // a work entry holds the head in 4 bits (b | h << 16 | part << 20 | parts - 1 << 22 | qb << 24,
    // the f16 kernels' encoding)
    if (work && (n_work <= 0 || B > 0xffff || H > 0xf || (max_len + 127) / 128 > 127)) {
        set_error("attention_i8_packed: work list needs n_work > 0, B < 65536, H < 16, max_len < 16257");
        return -1;
    }
    const I8Ws wo = i8_ws(M, B, max_len, H, KV);
    unsigned char *ws = (unsigned char *)workspace;
    I8PrepArgs p = {q32, k32, v32, (int8_t *)(ws + wo.q8), (float *)(ws + wo.qs), (int8_t *)(ws + wo.k8),
                    (float *)(ws + wo.ks), (int8_t *)(ws + wo.vt8), (float *)(ws + wo.vpart),
                    (float *)(ws + wo.vs), seq_start, seq_len, M, H, KV, (max_len + 63) / 64};
    hipStream_t s = (hipStream_t)stream;
    const long items = (long)M * (H + KV);
    hipLaunchKernelGGL(k_i8_qk_prep, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, s, p);
    hipLaunchKernelGGL(k_i8_vmax, dim3(B * KV, p.nch), dim3(256), 0, s, p);
    hipLaunchKernelGGL(k_i8_vquant, dim3(B * KV, (max_len + 31) / 32), dim3(256), 0, s, p);
    static bool attr = false;
    if (!attr) {
        if (check_hip(hipFuncSetAttribute((const void *)k_attn_i8, hipFuncAttributeMaxDynamicSharedMemorySize,
                                          kAttnI8Lds), "attention_i8 lds attribute"))
            return -1;
        attr = true;
    }
    AttnI8Args a = {p.q8, p.qs, p.k8, p.ks, p.vt8, p.vs, ctx_q, ctx_s, ctx32, seq_start, seq_len, work, M, H, KV};
    const dim3 grid = work ? dim3(n_work) : dim3((max_len + 127) / 128, H, B);
    hipLaunchKernelGGL(k_attn_i8, grid, dim3(256), kAttnI8Lds, s, a);
    return check_hip(hipGetLastError(), "attention_i8 launch");
}
