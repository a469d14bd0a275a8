// attn.hip — fused bidirectional GQA attention on gfx950 f16 MFMA with f32 softmax/accumulation,
// its context quantized per 128 dims for the O-projection GEMM.
//
// Reference semantics (text.c:534-572 attn_rows, 702-741 blocked, 817-891 attention):
//   logits = q . k_j * scale (scale 1.0 in the reference, text.c:8-9) over keys j with valid[j];
//   p = softmax(logits); ctx = sum_j p_j v_j; a query row with valid[i] == 0 gets ctx = 0; a row
//   with no valid key gets ctx = 0; GQA kv head = h / (H / KV). Then ctx is quantized per
//   (row, 128 block) like every GEMM input (text.c:890 -> gemm_quant_phase).
//
// Work decomposition: a workgroup is (sequence, head, 128 queries); its 4 waves own 32 queries each.
// Keys are walked in tiles of 32 staged in LDS (K as [key][d], V transposed as [d][key], both
// padded against bank conflicts). Per tile a wave computes S^T = K Q^T (16 v_mfma_f32_32x32x16_f16
// over d = 256) so that every lane holds 16 logits of ONE query: the running max/sum of the online
// softmax need only one exchange with the partner lane (lane ^ 32). P^T then feeds O^T += V^T P^T
// (16 more MFMAs) straight from registers: the 16 logits a lane holds are exactly the keys its
// B-operand slots must carry, once the A operand (V^T) is read in the same key order. K tile rows
// are stored with bits 2 and 3 of the key index exchanged, which makes those keys consecutive
// (16 j + 8 half + 0..7 for MFMA j), so a lane's V^T operand is 8 consecutive keys of one row.
#include "common.h"

namespace e2mi {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));

constexpr int kD = 256;          // head dim
constexpr int kKT = 32;          // keys per tile
constexpr int kKP = kD + 8;      // K row pitch in halves (528 B)
constexpr int kVP = kKT + 4;     // V^T row pitch in halves (72 B)

struct AttnArgs {
    const uint16_t *q;      // [M][H*D] f16
    const uint16_t *k;      // [M][KV*D] f16
    const uint16_t *vt;     // padded: [B][KV][D][S]; packed: [KV][D][S] with S = M
    const uint8_t *valid;   // padded: [M]
    int8_t *cq;             // [M][H*D] int8 context
    float *cs;              // [M][H*D/128] scales
    float *c32;             // optional [M][H*D] f32 context
    // packed batches: sequence b is rows [seq_start[b], seq_start[b] + seq_len[b]), all valid
    const int32_t *seq_start, *seq_len;
    // packed batches, optional: one work entry per workgroup of a 1-D grid, longest sequences
    // first; negative entries are no work. Entry = sequence | head << 16 | part << 20 |
    // (parts - 1) << 22 | query block << 24 (see work_entry): with parts > 1 the block's key tiles
    // are split into that many consecutive ranges, one workgroup each, which leave unnormalised
    // partial states in part_o / part_ml for k_attn_merge
    const int32_t *work;
    int B, S, H, KV;
    float scale;
    // packed batches, optional: keys with |pos_i - pos_j| > window are skipped (0: no window);
    // pos [M] is each row's position in its padded sequence (null: the packed index)
    int window;
    const int32_t *pos;
    // split key ranges (head_dim 256): part p of row r, head h holds the context sum o (before the
    // division by the softmax sum) at part_o[(p * part_rows + r) * H * D + h * D ..] and its row max
    // and sum at part_ml[((p * part_rows + r) * H + h) * 2 + 0 | 1]
    float *part_o, *part_ml;
    int part_rows;
};

// the packed work entry (AttnArgs::work); h < 16, parts <= 4, query block < 128
__host__ __device__ inline int work_entry(int b, int h, int part, int parts, int qb) {
    return b | (h << 16) | (part << 20) | ((parts - 1) << 22) | (qb << 24);
}
constexpr int kMaxParts = 4;

// One key tile of the online softmax for the 16 logits a lane holds (its partner lane ^ 32 holds
// the other 16 of the same query); every f16 attention kernel here calls it, so padded and packed
// batches stay bit-identical. Logits are kept in base-2 units, t = s * c with c = scale * log2(e)
// > 0 (the entry points refuse other scales), and p = 2^(t - m); masked keys arrive as s = -inf and
// give p = 0. The running max m only moves when the tile's max exceeds it by more than kTau, so
// p <= 2^kTau (f16 holds it, f32 sums too) and the context's rescale by alpha = 2^(m_old - m_new)
// is skipped on most tiles: the result is the same softmax, normalised at the end by the same sum l.
// Returns alpha (1 when m did not move).
constexpr float kTau = 8.f;
__device__ __forceinline__ float softmax_tile(const float (&s)[16], float c, float &mrun, float &lrun, h8 (&pb)[2]) {
    float mloc = s[0];
#pragma unroll
    for (int r = 1; r < 16; r++) mloc = fmaxf(mloc, s[r]);
    mloc = fmaxf(mloc, xor_lane<32>(mloc));
    const float mc = mloc * c;
    float alpha = 1.f;
    if (mc > mrun + kTau) {
        alpha = __builtin_amdgcn_exp2f(mrun - mc);
        mrun = mc;
    }
    const float ms = mrun == -INFINITY ? 0.f : mrun;  // no key yet: every p is 0
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const float pr = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], c, -ms));
        psum += pr;
        pb[r >> 3][r & 7] = (_Float16)pr;
    }
    lrun = lrun * alpha + psum;
    return alpha;
}

// Fragments read ahead of their MFMA in the attention loops: K (S^T A operand) PFK MFMAs ahead, V^T
// (PV A operand) PFV ahead (3 each: 4 reads in flight for most MFMAs; more spills registers)
constexpr int PFK = 3, PFV = 3;

__global__ __launch_bounds__(256, 2) void k_attn(AttnArgs a) {
    __shared__ __align__(16) _Float16 Ks[kKT * kKP];
    __shared__ __align__(16) _Float16 Vs[kD * kVP];
    __shared__ uint8_t vk[kKT];
    __shared__ int s_len;

    const int qb = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, half = lane >> 5;
    const int S = a.S, HD = a.H * kD, kvh = h / (a.H / a.KV);
    const bool packed = a.seq_start != nullptr;
    // padded: the sequence's rows b*S .. b*S+S-1 with a mask; packed: its own rows, all valid.
    // Sk: keys (and rows) of the sequence that can be read
    const size_t row0 = packed ? (size_t)a.seq_start[b] : (size_t)b * S;
    const int Sk = packed ? a.seq_len[b] : S;
    const uint8_t *valid = packed ? nullptr : a.valid + row0;

    // the sequence's last valid row + 1 (trailing padding is trimmed, text.c:849-852)
    if (packed) {
        if (tid == 0) s_len = Sk;
    } else {
        if (tid == 0) s_len = 0;
        __syncthreads();
        for (int i = tid; i < S; i += 256)
            if (valid[i]) atomicMax(&s_len, i + 1);
    }
    __syncthreads();
    const int Sb = s_len;
    if (packed && qb * 128 >= Sb) return;  // no rows of this sequence in the block

    const int qi = qb * 128 + w * 32 + (lane & 31);  // this lane's query
    const bool qvalid = qi < Sb && (packed || valid[qi]);
    const int qc = min(qi, Sk - 1);

    // Q fragments: B operand of S^T = K Q^T, lane holds Q[qi][16 s + 8 half .. +8]
    h8 qf[16];
    {
        const uint16_t *qp = a.q + (row0 + qc) * HD + h * kD + 8 * half;
#pragma unroll
        for (int s = 0; s < 16; s++) qf[s] = *(const h8 *)(qp + 16 * s);
    }
    f16v o[8];
#pragma unroll
    for (int t = 0; t < 8; t++) o[t] = (f16v){};
    float mrun = -INFINITY, lrun = 0.f;
    const float c2 = a.scale * 1.44269504088896341f;  // logits in base-2 units

    const bool block_live = qb * 128 < Sb;
    const int ntiles = block_live ? (Sb + kKT - 1) / kKT : 0;
    const uint16_t *kbase = a.k + row0 * a.KV * kD + kvh * kD;
    const uint16_t *vbase = packed ? a.vt + (size_t)kvh * kD * S + row0 : a.vt + ((size_t)(b * a.KV + kvh) * kD) * S;
    const bool vfast = (S % 8) == 0 && (row0 % 8) == 0;

    for (int kt = 0; kt < ntiles; kt++) {
        const int k0 = kt * kKT;
        __syncthreads();  // previous tile fully consumed
        // K tile: 32 keys x 256 dims, 16-byte chunks
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int key = tid / 32 + 8 * p, ch = tid % 32;
            uint4 val = make_uint4(0, 0, 0, 0);
            if (k0 + key < Sk) val = *(const uint4 *)(kbase + (size_t)(k0 + key) * a.KV * kD + ch * 8);
            // row swap23(key): see the S^T register layout below
            const int row = (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1);
            *(uint4 *)(Ks + row * kKP + ch * 8) = val;
        }
        // V^T tile: row d = tid, keys k0 .. k0+31
        {
            const uint16_t *vr = vbase + (size_t)tid * S + k0;
            _Float16 *dst = Vs + tid * kVP;
            if (vfast && k0 + kKT <= Sk) {
#pragma unroll
                for (int c = 0; c < 4; c++) *(uint2 *)(dst + 8 * c) = *(const uint2 *)(vr + 8 * c),
                                            *(uint2 *)(dst + 8 * c + 4) = *(const uint2 *)(vr + 8 * c + 4);
            } else {
                for (int j = 0; j < kKT; j++)
                    dst[j] = k0 + j < Sk ? __builtin_bit_cast(_Float16, vr[j]) : (_Float16)0.f;
            }
        }
        if (tid < kKT) vk[tid] = (k0 + tid < Sb) ? (packed ? 1 : valid[k0 + tid]) : 0;
        __syncthreads();

        // S^T tile (32 keys x 32 queries): A = K rows (lane%32 = key), B = Q
        f16v st = (f16v){};
        {
            const _Float16 *kp = Ks + (lane & 31) * kKP + 8 * half;
            h8 kr[PFK];
#pragma unroll
            for (int s = 0; s < PFK; s++) kr[s] = *(const h8 *)(kp + 16 * s);
#pragma unroll
            for (int s = 0; s < 16; s++) {
                st = __builtin_amdgcn_mfma_f32_32x32x16_f16(kr[s % PFK], qf[s], st, 0, 0, 0);
                if (s + PFK < 16) kr[s % PFK] = *(const h8 *)(kp + 16 * (s + PFK));
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // online softmax for this lane's query over the 16 keys it holds (+ the partner's 16).
        // K row i holds key swap23(i), so register r (row 8 (r / 4) + 4 half + r % 4) holds key
        // 16 (r / 8) + 8 half + 4 ((r / 4) % 2) + r % 4: registers 8 j .. 8 j + 7 hold the
        // consecutive keys 16 j + 8 half .. + 7, the PV MFMA's k order
        float tv[16];
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int key = 16 * (r >> 3) + 8 * half + 4 * ((r >> 2) & 1) + (r & 3);
            tv[r] = vk[key] ? st[r] : -INFINITY;
        }
        h8 pb[2];
        const float alpha = softmax_tile(tv, c2, mrun, lrun, pb);
        if (__any(alpha != 1.f)) {
#pragma unroll
            for (int t = 0; t < 8; t++) o[t] *= alpha;
        }
        // O^T += V^T P^T: MFMA #j covers the keys of registers 8j..8j+7, i.e. keys
        // 16 j + 8 half + 0..7; V^T is read in that order
        auto vfrag = [&](int i) {
            const _Float16 *vp = Vs + (32 * (i >> 1) + (lane & 31)) * kVP + 8 * half + 16 * (i & 1);
            h8 vf;
            *(uint2 *)&vf = *(const uint2 *)vp;
            *((uint2 *)&vf + 1) = *(const uint2 *)(vp + 4);
            return vf;
        };
        h8 vr[PFV];
#pragma unroll
        for (int i = 0; i < PFV; i++) vr[i] = vfrag(i);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            o[i >> 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vr[i % PFV], pb[i & 1], o[i >> 1], 0, 0, 0);
            if (i + PFV < 16) vr[i % PFV] = vfrag(i + PFV);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // normalise, quantise per 128 dims (tiles 0-3 and 4-7), store
    const float ltot = lrun + xor_lane<32>(lrun);
    const float inv = (qvalid && ltot > 0.f) ? __fdiv_rn(1.0f, ltot) : 0.f;
#pragma unroll
    for (int t = 0; t < 8; t++) o[t] *= inv;
    if (qi >= Sk) return;  // packed: rows past the sequence belong to the next one
    const size_t orow = (row0 + qi);
#pragma unroll
    for (int blk = 0; blk < 2; blk++) {
        float am = 0.f;
#pragma unroll
        for (int t = 4 * blk; t < 4 * blk + 4; t++)
#pragma unroll
            for (int r = 0; r < 16; r++) am = fmaxf(am, fabsf(o[t][r]));
        am = fmaxf(am, xor_lane<32>(am));
        const QScale qs = qscale(am);
#pragma unroll
        for (int t = 4 * blk; t < 4 * blk + 4; t++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int d = 32 * t + 8 * g + 4 * half;
                *(uint32_t *)(a.cq + orow * HD + h * kD + d) =
                    pack4_magic(o[t][4 * g], o[t][4 * g + 1], o[t][4 * g + 2], o[t][4 * g + 3], qs.inv);
                if (a.c32)
                    *(float4 *)(a.c32 + orow * HD + h * kD + d) =
                        make_float4(o[t][4 * g], o[t][4 * g + 1], o[t][4 * g + 2], o[t][4 * g + 3]);
            }
        if (half == 0) a.cs[orow * (HD / kQBlock) + h * 2 + blk] = qs.sc;
    }
}

// ---- packed batches: the same attention with K/V tiles fetched straight into LDS one tile ahead,
// with an optional sliding window (head_dim 256; k_attn_packed_d512 below takes 512). Every key of a packed sequence is valid, so no mask is read; the per-sequence
// work at D = 256 without a window is the arithmetic of k_attn bit for bit (same MFMA order, same
// softmax; masked keys read as zero here and contribute p = 0 in both).
//
// LDS per workgroup: 2 buffers of [K tile 32 keys x 2D B | V^T tile D rows x 64 B] (64 KB at
// D = 256, two workgroups per CU).
//   K tile row i holds key swap23(i) (bits 2 and 3 of the index exchanged). The S^T MFMA then
//     leaves in a lane's registers 8 j + e (e = 0..7) the keys 16 j + 8 half + e: consecutive keys,
//     so the PV MFMA's A operand is one 16-byte chunk of a V^T row in natural key order.
//   K rows are 2D bytes; 16-byte chunk x of row i sits at position x ^ (i & 7), so the eight lanes
//     of a read group (rows i..i+7, one chunk) hit eight bank groups.
//   V^T rows (one d, 32 keys) are 64 B; chunk c of row d sits at position c ^ ((d >> 2) & 3)
//     (conflict-free for rows d..d+7).
// The tile loads are 16-byte direct-to-LDS buffer loads: D/64 per wave for K (512/D rows each) and
// D/64 for V^T (16 rows each), whose lanes fetch the permuted, swizzled source chunks. Keys past
// the sequence read as zero (K: past the descriptor's range; V^T: 8-key chunks past the sequence
// get an offset past it, and the sequence's rows end on an 8-row boundary of the slab).
//
// Sliding window (text.c:542-546): query i reads key j when |pos_i - pos_j| <= window, pos being
// the token's position in its padded sequence (a.pos; the packed index when a.pos is null). The
// packed index never moves two tokens further apart than their positions, so the key tiles a query
// block reads are those within window of its rows by index; a tile whose every key is within window
// of every query of the block (checked on the positions of its first and last key and of the
// block's first and last query) needs no per-key test.
template <int D>
struct PackedTile {
    static constexpr int kK = kKT * 2 * D, kV = D * 64, kBuf = kK + kV;
    static constexpr size_t kLds = 2 * (size_t)kBuf;
};

// dma16 without a compiler memory clobber: the loads of tile kt + 1 fill the LDS buffer that no
// read of tile kt touches, so LDS reads and MFMAs may be scheduled across them; the loop-top wait
// and barrier order them with the reads of tile kt + 1
__device__ inline void dma16_nc(v4u r, uint32_t lds, uint32_t voff, uint32_t soff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 ::"s"(lds), "v"(voff), "s"(r), "s"(soff));
}

__device__ inline int swap23(int i) { return (i & ~12) | ((i & 4) << 1) | ((i & 8) >> 1); }

template <int D, bool WIN>
__global__ __launch_bounds__(256, D == 256 ? 2 : 1) void k_attn_packed(AttnArgs a) {
    using T = PackedTile<D>;
    // Q fragments, O tiles, K and V^T loads per wave and tile
    constexpr int NQ = D / 16, NO = D / 32, NLK = D / 64, NLV = D / 64;
    constexpr int RPI = 512 / D, LPR = D / 8;  // K rows per load, lanes per K row
    extern __shared__ __align__(16) unsigned char pk_smem[];
    int qb = blockIdx.x, h = blockIdx.y, b = blockIdx.z, part = 0, parts = 1;
    if (a.work) {
        const int item = a.work[blockIdx.x];
        if (item < 0) return;
        b = item & 0xffff;
        h = (item >> 16) & 0xf;
        part = (item >> 20) & 3;
        parts = ((item >> 22) & 3) + 1;
        qb = item >> 24;
    }
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, half = lane >> 5;
    const int S = a.S, HD = a.H * D, kvh = h / (a.H / a.KV);
    const size_t row0 = (size_t)a.seq_start[b];
    const int Sk = a.seq_len[b];
    if (qb * 128 >= Sk) return;  // no rows of this sequence in the block

    const int qi = qb * 128 + w * 32 + (lane & 31);  // this lane's query
    const bool qvalid = qi < Sk;
    const int qc = min(qi, Sk - 1);
    h8 qf[NQ];
    {
        const uint16_t *qp = a.q + (row0 + qc) * HD + h * D + 8 * half;
#pragma unroll
        for (int s = 0; s < NQ; s++) qf[s] = *(const h8 *)(qp + 16 * s);
    }
    // key tiles of this block: all, or those within window of its rows (by packed index)
    const int W = WIN ? a.window : 0;
    int kt0 = 0, kt1 = (Sk + kKT - 1) / kKT;
    int pq0 = 0, pq1 = 0, pqi = qc;
    if constexpr (WIN) {
        const int q0 = qb * 128, q1 = min(q0 + 127, Sk - 1);
        kt0 = max(q0 - W, 0) / kKT;
        kt1 = min((min(q1 + W, Sk - 1)) / kKT + 1, kt1);
        pq0 = a.pos ? a.pos[row0 + q0] : q0;
        pq1 = a.pos ? a.pos[row0 + q1] : q1;
        pqi = a.pos ? a.pos[row0 + qc] : qc;
    }
    if (parts > 1) {  // this workgroup's share of the block's key tiles
        const int n = kt1 - kt0, t0 = kt0;
        kt0 = t0 + n * part / parts;
        kt1 = t0 + n * (part + 1) / parts;
    }
    f16v o[NO];
#pragma unroll
    for (int t = 0; t < NO; t++) o[t] = (f16v){};
    float mrun = -INFINITY, lrun = 0.f;
    const float c2 = a.scale * 1.44269504088896341f;  // logits in base-2 units

    // sources: K rows of this kv head (row pitch KV*D halves), V^T slab [D][S] of this kv head
    const uint32_t rowB = (uint32_t)a.KV * D * 2;
    const v4u rK = rsrc_words(a.k + row0 * a.KV * D + kvh * D, (uint32_t)Sk * rowB);
    const uint16_t *vslab = a.vt + (size_t)kvh * D * S + row0;
    const v4u rV = rsrc_words(vslab, (uint32_t)((size_t)D * S * 2));
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const lds_void *)pk_smem);
    const int wu = __builtin_amdgcn_readfirstlane(w);
    const int lr = lane / LPR, lc = lane % LPR;
    // K: load i of wave w fills LDS rows 8 w + RPI i + lane / LPR, i.e. keys swap23 of those
    // (swap23 keeps bit 0, so the second row of a D = 256 load is the next key); lane's chunk
    // position lane % LPR holds source chunk (lane % LPR) ^ (row & 7).
    // V^T: load i of wave w fills rows d = (D/4) w + 16 i + lane / 4, chunk position lane % 4,
    // which holds source chunk (lane % 4) ^ ((d >> 2) & 3) = (lane % 4) ^ ((lane >> 4) & 3).
    const uint32_t vlane = (uint32_t)(lane >> 2) * (uint32_t)S * 2;
    const int vchunk = (lane & 3) ^ ((lane >> 4) & 3);
    // load j (0 .. NLK-1: K, NLK .. NLK+NLV-1: V^T) of tile kt; issued one per two S^T MFMAs of
    // the previous tile
    auto issue_load = [&](int kt, int j) {
        const int k0 = kt * kKT;
        const uint32_t base = lds0 + (uint32_t)((kt & 1) * T::kBuf);
        if (j < NLK) {
            // the first row's key goes to the scalar offset (range-checked with the lane offset:
            // keys past the sequence read as zero)
            const int i = j, r = 8 * wu + RPI * i;
            const uint32_t voff = (uint32_t)lr * rowB + (uint32_t)((lc ^ ((r + lr) & 7)) << 4);
            dma16_nc(rK, __builtin_amdgcn_readfirstlane(base + (uint32_t)r * (2 * D)), voff,
                     __builtin_amdgcn_readfirstlane((uint32_t)(swap23(r) + k0) * rowB));
        } else {
            const int i = j - NLK, d0 = (D / 4) * wu + 16 * i;
            const uint32_t vo = (k0 + 8 * vchunk < Sk) ? vlane + (uint32_t)vchunk * 16 : 0x80000000u;
            dma16_nc(rV, __builtin_amdgcn_readfirstlane(base + T::kK + d0 * 64), vo,
                     __builtin_amdgcn_readfirstlane((uint32_t)(d0 * S + k0) * 2));
        }
    };

    // per-lane LDS read offsets. K (S^T A operand): row lane % 32, chunk 2 s + half at position
    // (2 s + half) ^ (row & 7): for s = 4 t + u the position is 8 t + ((2 u + half) ^ (row & 7)).
    const int kkey = lane & 31;
    uint32_t krd[4];
#pragma unroll
    for (int u = 0; u < 4; u++) krd[u] = (uint32_t)(kkey * 2 * D + (((2 * u + half) ^ (kkey & 7)) << 4));
    // V^T (PV A operand): row d = 32 t + lane % 32, chunk 2 j + half at position ^ ((d >> 2) & 3)
    uint32_t vrd[2];
#pragma unroll
    for (int j = 0; j < 2; j++)
        vrd[j] = (uint32_t)(T::kK + (lane & 31) * 64 + (((2 * j + half) ^ (((lane & 31) >> 2) & 3)) << 4));

    if (kt0 < kt1)
#pragma unroll
        for (int j = 0; j < NLK + NLV; j++) issue_load(kt0, j);
    // wait for the Q loads here, after the first tile's loads are issued (the two latencies
    // overlap), with a wait the compiler's wait-count pass sees: otherwise it waits for them inside
    // the tile loop, where the count would also cover the tile loads in flight (s_waitcnt vmcnt(0)
    // expcnt(7) lgkmcnt(15))
    __builtin_amdgcn_s_waitcnt(0x0F70);
    for (int kt = kt0; kt < kt1; kt++) {
        const int k0 = kt * kKT;
        // this wave's loads of tile kt have landed; the barrier makes every wave's visible and
        // ends every wave's reads of tile kt - 1, whose buffer the next loads refill
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        const bool next = kt + 1 < kt1;
        const unsigned char *sb = pk_smem + (kt & 1) * T::kBuf;

        f16v st = (f16v){};
        // K fragments read PFK MFMAs ahead (a ring of fragment registers): each read is in flight
        // under the MFMAs before its own, where reading it just before its MFMA made every MFMA wait
        // for an LDS round trip
        h8 kr[PFK];
#pragma unroll
        for (int s = 0; s < PFK; s++) kr[s] = *(const h8 *)(sb + krd[s & 3] + (s >> 2) * 128);
#pragma unroll
        for (int s = 0; s < NQ; s++) {
            st = __builtin_amdgcn_mfma_f32_32x32x16_f16(kr[s % PFK], qf[s], st, 0, 0, 0);
            if (s + PFK < NQ) kr[s % PFK] = *(const h8 *)(sb + krd[(s + PFK) & 3] + ((s + PFK) >> 2) * 128);
            if ((s & 1) && (s >> 1) < NLK + NLV && next) issue_load(kt + 1, s >> 1);
        }
        // keys past the sequence, and with a window those out of range, get s = -inf; a tile inside
        // the sequence (and, with a window, inside the window of every query of the block) needs no
        // per-key test
        float tv[16];
#pragma unroll
        for (int r = 0; r < 16; r++) tv[r] = st[r];
        bool edge = k0 + kKT > Sk;
        if constexpr (WIN) {
            const int ka = k0, kb = min(k0 + kKT, Sk) - 1;
            const int pka = a.pos ? a.pos[row0 + ka] : ka, pkb = a.pos ? a.pos[row0 + kb] : kb;
            edge = edge || pkb - pq0 > W || pq1 - pka > W;
        }
        if (edge) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                // S^T row 8 (r / 4) + 4 half + r % 4 of this register holds key swap23(row)
                const int key = 16 * (r >> 3) + 8 * half + 4 * ((r >> 2) & 1) + (r & 3);
                bool keep = k0 + key < Sk;
                if constexpr (WIN) {
                    if (keep) {
                        const int pk = a.pos ? a.pos[row0 + k0 + key] : k0 + key;
                        keep = pk - pqi <= W && pqi - pk <= W;
                    }
                }
                if (!keep) tv[r] = -INFINITY;
            }
        }
        h8 pb[2];
        const float alpha = softmax_tile(tv, c2, mrun, lrun, pb);
        // V^T fragments (MFMA i = 2 t + j) read PFV ahead, as the K fragments above
        auto vfrag = [&](int i) { return *(const h8 *)(sb + vrd[i & 1] + (i >> 1) * 32 * 64); };
        h8 vr[PFV];
#pragma unroll
        for (int i = 0; i < PFV; i++) vr[i] = vfrag(i);
        // the running max moves on few tiles: skip the rescale when no lane's did
        if (__any(alpha != 1.f)) {
#pragma unroll
            for (int t = 0; t < NO; t++) o[t] *= alpha;
        }
#pragma unroll
        for (int i = 0; i < 2 * NO; i++) {
            o[i >> 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vr[i % PFV], pb[i & 1], o[i >> 1], 0, 0, 0);
            if (i + PFV < 2 * NO) vr[i % PFV] = vfrag(i + PFV);
            // (kept in this order: the scheduler would otherwise sink each read to its MFMA)
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    const float ltot = lrun + xor_lane<32>(lrun);
    if (parts > 1) {
        // a partial state: the context sum, the row max and the row sum (mrun is the pair's)
        if (qi >= Sk) return;
        const size_t prow = (size_t)part * a.part_rows + row0 + qi;
        float *po = a.part_o + prow * HD + h * D;
#pragma unroll
        for (int t = 0; t < NO; t++)
#pragma unroll
            for (int g = 0; g < 4; g++)
                *(float4 *)(po + 32 * t + 8 * g + 4 * half) =
                    make_float4(o[t][4 * g], o[t][4 * g + 1], o[t][4 * g + 2], o[t][4 * g + 3]);
        if (half == 0) *(float2 *)(a.part_ml + (prow * a.H + h) * 2) = make_float2(mrun, ltot);
        return;
    }
    const float inv = (qvalid && ltot > 0.f) ? __fdiv_rn(1.0f, ltot) : 0.f;
#pragma unroll
    for (int t = 0; t < NO; t++) o[t] *= inv;
    // The quantized context goes through LDS so that its global stores write whole rows: a lane
    // holds 4-byte pieces of one query's row, so storing them directly touched 32 rows (lines) per
    // instruction. The wave's 32 rows x D bytes go to its own part of the buffer the last tile did
    // not use (its last reads were before the last tile's barrier; no load was issued into it
    // since), dword dw of row r at dw ^ ((r & 15) << 2) (the 64 lanes of a write hit distinct bank
    // pairs, each 16-byte group stays whole); then 16-byte lane stores, D / 16 lanes a row. Lanes
    // past the sequence hold zeros and write nothing.
    unsigned char *stg = pk_smem + (kt1 & 1) * T::kBuf + w * 32 * D;
    const int qr = lane & 31;
    const size_t orow = (row0 + qi);
#pragma unroll
    for (int blk = 0; blk < D / 128; blk++) {
        float am = 0.f;
#pragma unroll
        for (int t = 4 * blk; t < 4 * blk + 4; t++)
#pragma unroll
            for (int r = 0; r < 16; r++) am = fmaxf(am, fabsf(o[t][r]));
        am = fmaxf(am, xor_lane<32>(am));
        const QScale qs = qscale(am);
#pragma unroll
        for (int t = 4 * blk; t < 4 * blk + 4; t++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int d = 32 * t + 8 * g + 4 * half;
                // (the quantizer's bytes by the 1.5 * 2^23 addition: |o * inv| <= 127, as in the GEMMs'
                // requantizing epilogues; the same bytes as rint and clamp)
                *(uint32_t *)(stg + qr * D + (((d >> 2) ^ ((qr & 15) << 2)) << 2)) =
                    pack4_magic(o[t][4 * g], o[t][4 * g + 1], o[t][4 * g + 2], o[t][4 * g + 3], qs.inv);
                if (a.c32 && qi < Sk)
                    *(float4 *)(a.c32 + orow * HD + h * D + d) =
                        make_float4(o[t][4 * g], o[t][4 * g + 1], o[t][4 * g + 2], o[t][4 * g + 3]);
            }
        if (half == 0 && qi < Sk) a.cs[orow * (HD / kQBlock) + h * (D / 128) + blk] = qs.sc;
    }
    // (one wave's LDS operations complete in order: the reads see its writes)
    constexpr int CPR = D / 16;  // 16-byte chunks a row
    if (((uintptr_t)a.cq & 15) == 0) {
#pragma unroll
        for (int k = 0; k < 32 * CPR / 64; k++) {
            const int r = (64 * k + lane) / CPR, ch = lane % CPR;
            const uint4 v = *(const uint4 *)(stg + r * D + ((ch ^ (r & 15)) << 4));
            const int q = qb * 128 + w * 32 + r;
            if (q < Sk) *(uint4 *)(a.cq + (row0 + q) * HD + h * D + 16 * ch) = v;
        }
    } else {
        // a context buffer aligned to 4 bytes only: the same rows by 4-byte lane stores
#pragma unroll 4
        for (int k = 0; k < 32 * D / 256; k++) {
            const int r = (256 * k + 4 * lane) / D, dw = ((256 * k + 4 * lane) % D) >> 2;
            const uint32_t v = *(const uint32_t *)(stg + r * D + ((dw ^ ((r & 15) << 2)) << 2));
            const int q = qb * 128 + w * 32 + r;
            if (q < Sk) *(uint32_t *)(a.cq + (row0 + q) * HD + h * D + 4 * dw) = v;
        }
    }
}

// ---- head_dim 512 (the reference checkpoint's full-attention layers): one 8-wave workgroup per
// (sequence, head, 128 queries). Waves w and w + 4 own the same 32 queries; wave w computes the
// logits over dims 0..255 and wave w + 4 over 256..511 (each holds only its half of the Q
// fragments), they add each other's partial logits through LDS, run the same softmax on the same
// sums, and each accumulates the context for its own 256 dims. The MFMA work is that of one pass
// (4 L^2 512 flops per head) and two waves share each SIMD.
//
// LDS: 2 buffers of [K tile 32 keys x 1024 B | V^T tile 512 rows x 64 B] (64 KB each), then the
// partial-logit exchange, 8 waves x 64 lanes x 16 floats (32 KB): 160 KB, one workgroup per CU.
// Tile layouts and swizzles are those of k_attn_packed (K row i holds key swap23(i), chunk x at
// x ^ (i & 7); V^T chunk c of row d at c ^ ((d >> 2) & 3)). Per tile: wait for its loads and a
// barrier; the partial S^T (16 MFMAs, the next tile's 8 loads per wave between them); write the
// partial logits; a barrier; read the partner's, softmax, PV (16 MFMAs). The exchange area is
// written after the first barrier of a tile and read before the first barrier of the next.
constexpr int kK512 = kKT * 1024, kV512 = 512 * 64, kBuf512 = kK512 + kV512;
constexpr int kXch512 = 8 * 64 * 16 * 4;
constexpr size_t kLds512 = 2 * (size_t)kBuf512 + kXch512;

__global__ __launch_bounds__(512, 1) void k_attn_packed_d512(AttnArgs a) {
    constexpr int D = 512, DH = 256;
    extern __shared__ __align__(16) unsigned char pk_smem[];
    int qb = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    if (a.work) {
        const int item = a.work[blockIdx.x];
        if (item < 0) return;
        b = item & 0xffff;
        h = (item >> 16) & 0xf;  // (one part: work_entry(b, h, 0, 1, qb))
        qb = item >> 24;
    }
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, half = lane >> 5;
    const int qw = w & 3, dh = w >> 2;  // query sub-block, dim half
    const int S = a.S, HD = a.H * D, kvh = h / (a.H / a.KV);
    const size_t row0 = (size_t)a.seq_start[b];
    const int Sk = a.seq_len[b];
    if (qb * 128 >= Sk) return;

    const int qi = qb * 128 + qw * 32 + (lane & 31);
    const bool qvalid = qi < Sk;
    const int qc = min(qi, Sk - 1);
    h8 qf[16];  // this wave's 256 dims of the query
    {
        const uint16_t *qp = a.q + (row0 + qc) * HD + h * D + dh * DH + 8 * half;
#pragma unroll
        for (int s = 0; s < 16; s++) qf[s] = *(const h8 *)(qp + 16 * s);
    }
    const int W = a.window;
    int kt0 = 0, kt1 = (Sk + kKT - 1) / kKT;
    int pq0 = 0, pq1 = 0, pqi = qc;
    if (W > 0) {
        const int q0 = qb * 128, q1 = min(q0 + 127, Sk - 1);
        kt0 = max(q0 - W, 0) / kKT;
        kt1 = min((min(q1 + W, Sk - 1)) / kKT + 1, kt1);
        pq0 = a.pos ? a.pos[row0 + q0] : q0;
        pq1 = a.pos ? a.pos[row0 + q1] : q1;
        pqi = a.pos ? a.pos[row0 + qc] : qc;
    }
    f16v o[8];
#pragma unroll
    for (int t = 0; t < 8; t++) o[t] = (f16v){};
    float mrun = -INFINITY, lrun = 0.f;
    const float c2 = a.scale * 1.44269504088896341f;  // logits in base-2 units

    const uint32_t rowB = (uint32_t)a.KV * D * 2;
    const v4u rK = rsrc_words(a.k + row0 * a.KV * D + kvh * D, (uint32_t)Sk * rowB);
    const uint16_t *vslab = a.vt + (size_t)kvh * D * S + row0;
    const v4u rV = rsrc_words(vslab, (uint32_t)((size_t)D * S * 2));
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const lds_void *)pk_smem);
    const int wu = __builtin_amdgcn_readfirstlane(w);
    // K: load i of wave w fills row r = 4 w + i (key swap23(r)), lane = chunk position holding
    // source chunk lane ^ (r & 7); V^T: load i of wave w fills rows d = 64 w + 16 i + lane / 4
    const uint32_t vlane = (uint32_t)(lane >> 2) * (uint32_t)S * 2;
    const int vchunk = (lane & 3) ^ ((lane >> 4) & 3);
    auto issue_load = [&](int kt, int j) {
        const int k0 = kt * kKT;
        const uint32_t base = lds0 + (uint32_t)((kt & 1) * kBuf512);
        if (j < 4) {
            const int r = 4 * wu + j;
            const uint32_t voff = (uint32_t)(swap23(r) + k0) * rowB + (uint32_t)((lane ^ (r & 7)) << 4);
            dma16_nc(rK, __builtin_amdgcn_readfirstlane(base + (uint32_t)r * 1024), voff, 0u);
        } else {
            const int d0 = 64 * wu + 16 * (j - 4);
            const uint32_t vo = (k0 + 8 * vchunk < Sk) ? vlane + (uint32_t)vchunk * 16 : 0x80000000u;
            dma16_nc(rV, __builtin_amdgcn_readfirstlane(base + kK512 + d0 * 64), vo,
                     __builtin_amdgcn_readfirstlane((uint32_t)(d0 * S + k0) * 2));
        }
    };
    const int kkey = lane & 31;
    uint32_t krd[4];
#pragma unroll
    for (int u = 0; u < 4; u++)
        krd[u] = (uint32_t)(kkey * 1024 + dh * 512 + (((2 * u + half) ^ (kkey & 7)) << 4));
    uint32_t vrd[2];
#pragma unroll
    for (int j = 0; j < 2; j++)
        vrd[j] = (uint32_t)(kK512 + (dh * DH + (lane & 31)) * 64 + (((2 * j + half) ^ (((lane & 31) >> 2) & 3)) << 4));
    float *xw = (float *)(pk_smem + 2 * kBuf512) + (w * 64 + lane) * 16;          // this wave's slot
    const float *xp = (const float *)(pk_smem + 2 * kBuf512) + ((w ^ 4) * 64 + lane) * 16;  // partner's

    if (kt0 < kt1)
#pragma unroll
        for (int j = 0; j < 8; j++) issue_load(kt0, j);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // the Q loads, after the first tile's (see k_attn_packed)
    for (int kt = kt0; kt < kt1; kt++) {
        const int k0 = kt * kKT;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        const bool next = kt + 1 < kt1;
        const unsigned char *sb = pk_smem + (kt & 1) * kBuf512;
        f16v st = (f16v){};
        h8 kr[PFK];
#pragma unroll
        for (int s = 0; s < PFK; s++) kr[s] = *(const h8 *)(sb + krd[s & 3] + (s >> 2) * 128);
#pragma unroll
        for (int s = 0; s < 16; s++) {
            st = __builtin_amdgcn_mfma_f32_32x32x16_f16(kr[s % PFK], qf[s], st, 0, 0, 0);
            if (s + PFK < 16) kr[s % PFK] = *(const h8 *)(sb + krd[(s + PFK) & 3] + ((s + PFK) >> 2) * 128);
            if ((s & 1) && next) issue_load(kt + 1, s >> 1);
        }
#pragma unroll
        for (int r = 0; r < 16; r += 4) *(float4 *)(xw + r) = make_float4(st[r], st[r + 1], st[r + 2], st[r + 3]);
        __syncthreads();
        float sfull[16];
#pragma unroll
        for (int r = 0; r < 16; r += 4) {
            const float4 x = *(const float4 *)(xp + r);
            // one rounded addition, commutative: both waves of the pair get the same sums
            sfull[r] = st[r] + x.x;
            sfull[r + 1] = st[r + 1] + x.y;
            sfull[r + 2] = st[r + 2] + x.z;
            sfull[r + 3] = st[r + 3] + x.w;
        }
        bool edge = k0 + kKT > Sk;
        if (W > 0) {
            const int ka = k0, kb = min(k0 + kKT, Sk) - 1;
            const int pka = a.pos ? a.pos[row0 + ka] : ka, pkb = a.pos ? a.pos[row0 + kb] : kb;
            edge = edge || pkb - pq0 > W || pq1 - pka > W;
        }
        if (edge) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int key = 16 * (r >> 3) + 8 * half + 4 * ((r >> 2) & 1) + (r & 3);
                bool keep = k0 + key < Sk;
                if (W > 0 && keep) {
                    const int pk = a.pos ? a.pos[row0 + k0 + key] : k0 + key;
                    keep = pk - pqi <= W && pqi - pk <= W;
                }
                if (!keep) sfull[r] = -INFINITY;
            }
        }
        // waves w and w + 4 hold the same sums and take the same steps
        h8 pb[2];
        const float alpha = softmax_tile(sfull, c2, mrun, lrun, pb);
        if (__any(alpha != 1.f)) {
#pragma unroll
            for (int t = 0; t < 8; t++) o[t] *= alpha;
        }
        h8 vr[PFV];
#pragma unroll
        for (int i = 0; i < PFV; i++) vr[i] = *(const h8 *)(sb + vrd[i & 1] + (i >> 1) * 32 * 64);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            o[i >> 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vr[i % PFV], pb[i & 1], o[i >> 1], 0, 0, 0);
            if (i + PFV < 16) vr[i % PFV] = *(const h8 *)(sb + vrd[(i + PFV) & 1] + ((i + PFV) >> 1) * 32 * 64);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    const float ltot = lrun + xor_lane<32>(lrun);
    const float inv = (qvalid && ltot > 0.f) ? __fdiv_rn(1.0f, ltot) : 0.f;
#pragma unroll
    for (int t = 0; t < 8; t++) o[t] *= inv;
    if (qi >= Sk) return;
    const size_t orow = (row0 + qi);
    const int dof = dh * DH;
#pragma unroll
    for (int blk = 0; blk < 2; blk++) {
        float am = 0.f;
#pragma unroll
        for (int t = 4 * blk; t < 4 * blk + 4; t++)
#pragma unroll
            for (int r = 0; r < 16; r++) am = fmaxf(am, fabsf(o[t][r]));
        am = fmaxf(am, xor_lane<32>(am));
        const QScale qs = qscale(am);
#pragma unroll
        for (int t = 4 * blk; t < 4 * blk + 4; t++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int d = dof + 32 * t + 8 * g + 4 * half;
                *(uint32_t *)(a.cq + orow * HD + h * D + d) =
                    pack4_magic(o[t][4 * g], o[t][4 * g + 1], o[t][4 * g + 2], o[t][4 * g + 3], qs.inv);
                if (a.c32)
                    *(float4 *)(a.c32 + orow * HD + h * D + d) =
                        make_float4(o[t][4 * g], o[t][4 * g + 1], o[t][4 * g + 2], o[t][4 * g + 3]);
            }
        if (half == 0) a.cs[orow * (HD / kQBlock) + h * 4 + dh * 2 + blk] = qs.sc;
    }
}

// Merge of split key ranges (k_attn_packed with parts > 1; head_dim 256), for the entries of the
// merge list (work_entry with part 0 and the block's part count): per query row, M = max_p m_p,
// w_p = 2^(m_p - M) (row maxima in base-2 units, see softmax_tile), ctx = (sum_p w_p o_p) * RN(1 / sum_p w_p l_p), parts in order, then the
// per-128 quantization of k_attn_packed's epilogue. Four workgroups per entry, 32 rows each, 8 rows
// per wave with all their loads issued before any is used; a lane holds 4 dims (lanes 0-31 the
// first 128-dim block, 32-63 the second).
__global__ __launch_bounds__(256) void k_attn_merge(AttnArgs a, const int32_t *merge) {
    constexpr int D = 256, RW = 8;  // rows per wave, their loads issued together
    const int item = merge[blockIdx.x >> 2];
    if (item < 0) return;
    const int b = item & 0xffff, h = (item >> 16) & 0xf, parts = ((item >> 22) & 3) + 1, qb = item >> 24;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, half = lane >> 5, d = 4 * lane;
    const int HD = a.H * D;
    const size_t row0 = (size_t)a.seq_start[b];
    const int Sk = a.seq_len[b];
    // workgroup blockIdx.x % 4 takes rows 32 (blockIdx.x % 4) .. + 31 of the block; wave w 8 of them
    const int q0 = qb * 128 + (blockIdx.x & 3) * 32 + w * RW;
    float mp[RW][kMaxParts], lp[RW][kMaxParts];
    float4 op[RW][kMaxParts];
#pragma unroll
    for (int r = 0; r < RW; r++) {
        const size_t row = row0 + min(q0 + r, Sk - 1);
#pragma unroll
        for (int p = 0; p < kMaxParts; p++) {
            if (p < parts) {
                const size_t prow = (size_t)p * a.part_rows + row;
                const float2 ml = *(const float2 *)(a.part_ml + (prow * a.H + h) * 2);
                mp[r][p] = ml.x;
                lp[r][p] = ml.y;
                op[r][p] = *(const float4 *)(a.part_o + prow * HD + h * D + d);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RW; r++) {
        const int qi = q0 + r;
        if (qi >= Sk) break;
        const size_t row = row0 + qi;
        float M = -INFINITY;
#pragma unroll
        for (int p = 0; p < kMaxParts; p++)
            if (p < parts) M = fmaxf(M, mp[r][p]);
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
        float L = 0.f;
        if (M != -INFINITY) {
#pragma unroll
            for (int p = 0; p < kMaxParts; p++) {
                if (p >= parts) break;
                const float wp = mp[r][p] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mp[r][p] - M);
                const float4 v = op[r][p];
                L += wp * lp[r][p];
                o = make_float4(o.x + wp * v.x, o.y + wp * v.y, o.z + wp * v.z, o.w + wp * v.w);
            }
        }
        const float inv = L > 0.f ? __fdiv_rn(1.0f, L) : 0.f;
        o = make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
        const float am = group_max<32>(fmaxf(fmaxf(fabsf(o.x), fabsf(o.y)), fmaxf(fabsf(o.z), fabsf(o.w))));
        const QScale qs = qscale(am);
        *(uint32_t *)(a.cq + row * HD + h * D + d) =
            pack4_magic(o.x, o.y, o.z, o.w, qs.inv);
        if (a.c32) *(float4 *)(a.c32 + row * HD + h * D + d) = o;
        if ((lane & 31) == 0) a.cs[row * (HD / kQBlock) + h * 2 + half] = qs.sc;
    }
}

template <int D, bool WIN>
static int attn_packed_attr() {
    static bool done = false;
    if (!done) {
        if (check_hip(hipFuncSetAttribute((const void *)k_attn_packed<D, WIN>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                          (int)PackedTile<D>::kLds), "attention lds attribute"))
            return -1;
        done = true;
    }
    return 0;
}

}  // namespace e2mi

using namespace e2mi;

extern "C" int e2mi_attention(e2mi_stream stream, const uint16_t *q16, const uint16_t *k16,
                              const uint16_t *vt16, const uint8_t *valid, int B, int S, int H,
                              int KV, int D, float scale, int8_t *ctx_q, float *ctx_s,
                              float *ctx32) {
    if (D != kD || B <= 0 || S <= 0 || H <= 0 || KV <= 0 || H % KV || !(scale > 0.f) || !(scale < INFINITY)) {
        set_error("attention: needs head_dim 256, H %% KV == 0 and a finite scale > 0 (B=%d S=%d H=%d KV=%d D=%d "
                  "scale=%g)", B, S, H, KV, D, (double)scale);
        return -1;
    }
    if (!q16 || !k16 || !vt16 || !valid || !ctx_q || !ctx_s || !aligned16(q16) || !aligned16(k16) ||
        ((uintptr_t)vt16 & 7) || ((uintptr_t)ctx_q & 3) || (ctx32 && !aligned16(ctx32))) {
        set_error("attention: null or misaligned pointer");
        return -1;
    }
    AttnArgs a = {q16, k16, vt16, valid, ctx_q, ctx_s, ctx32, nullptr, nullptr, nullptr, B, S, H, KV, scale};
    hipLaunchKernelGGL(k_attn, dim3((S + 127) / 128, H, B), dim3(256), 0, (hipStream_t)stream, a);
    return check_hip(hipGetLastError(), "attention launch");
}

static int attention_packed(const char *who, e2mi_stream stream, const uint16_t *q16,
                            const uint16_t *k16, const uint16_t *vt16, int M, const int32_t *seq_start,
                            const int32_t *seq_len, const int32_t *pos, int B, int max_len, int H,
                            int KV, int D, float scale, int window, int8_t *ctx_q, float *ctx_s,
                            float *ctx32, const int32_t *work, int n_work, const int32_t *merge = nullptr,
                            int n_merge = 0, float *part = nullptr, int part_rows = 0) {
    if ((D != 256 && D != 512) || B <= 0 || M <= 0 || max_len <= 0 || H <= 0 || KV <= 0 || H % KV ||
        window < 0 || !(scale > 0.f) || !(scale < INFINITY)) {
        set_error("%s: needs head_dim 256 or 512, H %% KV == 0, window >= 0 and a finite scale > 0 (B=%d M=%d "
                  "H=%d KV=%d D=%d scale=%g)", who, B, M, H, KV, D, (double)scale);
        return -1;
    }
    if (!q16 || !k16 || !vt16 || !seq_start || !seq_len || !ctx_q || !ctx_s || !aligned16(q16) ||
        !aligned16(k16) || ((uintptr_t)vt16 & 7) || ((uintptr_t)ctx_q & 3) ||
        (ctx32 && !aligned16(ctx32))) {
        set_error("%s: null or misaligned pointer", who);
        return -1;
    }
    if (work && (n_work <= 0 || B > 0xffff || H > 15 || (max_len + 127) / 128 > 127)) {
        set_error("%s: work list needs n_work > 0, B < 65536, H < 16, max_len < 16257", who);
        return -1;
    }
    if (merge && (D != 256 || !work || n_merge <= 0 || !part || part_rows < M || !aligned16(part))) {
        set_error("%s: split key ranges need head_dim 256, a work list, n_merge > 0 and a 16-byte aligned "
                  "partial workspace of at least M rows", who);
        return -1;
    }
    AttnArgs a = {q16, k16, vt16, nullptr, ctx_q, ctx_s, ctx32, seq_start, seq_len, work, B, M, H, KV, scale,
                  window, pos};
    if (merge) {
        a.part_o = part;
        a.part_ml = part + (size_t)kMaxParts * part_rows * H * D;
        a.part_rows = part_rows;
    }
    // the direct-to-LDS kernel needs 4-byte-aligned V^T rows and 32-bit offsets into the V^T slab
    // and the K rows; every sequence must start on an even row (the engine starts them on
    // multiples of 8)
    const bool direct = M % 2 == 0 && (size_t)KV * D * M * 2 < 0x7fffffffu &&
                        (size_t)M * KV * D * 2 < 0x7fffffffu && ((uintptr_t)vt16 & 3) == 0;
    const dim3 grid = work ? dim3(n_work) : dim3((max_len + 127) / 128, H, B);
    if (direct && D == 256 && window > 0) {
        if (attn_packed_attr<256, true>()) return -1;
        hipLaunchKernelGGL((k_attn_packed<256, true>), grid, dim3(256), PackedTile<256>::kLds, (hipStream_t)stream, a);
    } else if (direct && D == 256) {
        if (attn_packed_attr<256, false>()) return -1;
        hipLaunchKernelGGL((k_attn_packed<256, false>), grid, dim3(256), PackedTile<256>::kLds, (hipStream_t)stream, a);
    } else if (direct) {
        static bool attr512 = false;
        if (!attr512) {
            if (check_hip(hipFuncSetAttribute((const void *)k_attn_packed_d512,
                                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLds512),
                          "attention lds attribute"))
                return -1;
            attr512 = true;
        }
        hipLaunchKernelGGL(k_attn_packed_d512, grid, dim3(512), kLds512, (hipStream_t)stream, a);
    } else if (D == 256 && window == 0) {
        a.work = nullptr;
        hipLaunchKernelGGL(k_attn, dim3((max_len + 127) / 128, H, B), dim3(256), 0, (hipStream_t)stream, a);
    } else {
        set_error("%s: head_dim 512 or a window needs an even M, 4-byte-aligned V^T and slabs under 2 GiB", who);
        return -1;
    }
    if (merge) {
        if (!direct) {
            set_error("%s: split key ranges need the direct-to-LDS kernel (even M, aligned V^T)", who);
            return -1;
        }
        if (check_hip(hipGetLastError(), "attention launch")) return -1;
        hipLaunchKernelGGL(k_attn_merge, dim3(4 * n_merge), dim3(256), 0, (hipStream_t)stream, a, merge);
    }
    return check_hip(hipGetLastError(), "attention launch");
}

extern "C" int e2mi_attention_packed(e2mi_stream stream, const uint16_t *q16, const uint16_t *k16,
                                     const uint16_t *vt16, int M, const int32_t *seq_start,
                                     const int32_t *seq_len, int B, int max_len, int H, int KV, int D,
                                     float scale, int8_t *ctx_q, float *ctx_s, float *ctx32,
                                     const int32_t *work, int n_work) {
    if (D != 256) {
        set_error("attention_packed: needs head_dim 256 (D=%d; e2mi_attention_packed_window takes 512)", D);
        return -1;
    }
    return attention_packed("attention_packed", stream, q16, k16, vt16, M, seq_start, seq_len, nullptr, B,
                            max_len, H, KV, D, scale, 0, ctx_q, ctx_s, ctx32, work, n_work);
}

extern "C" size_t e2mi_attention_part_bytes(int part_rows, int H, int D) {
    if (part_rows <= 0 || H <= 0 || D != 256) return 0;
    return (size_t)kMaxParts * part_rows * H * ((size_t)D + 2) * 4;
}

extern "C" int e2mi_attention_packed_split(e2mi_stream stream, const uint16_t *q16, const uint16_t *k16,
                                           const uint16_t *vt16, int M, const int32_t *seq_start,
                                           const int32_t *seq_len, const int32_t *pos, int B, int max_len, int H,
                                           int KV, int D, float scale, int window, int8_t *ctx_q, float *ctx_s,
                                           float *ctx32, const int32_t *work, int n_work, const int32_t *merge,
                                           int n_merge, float *part, int part_rows) {
    if (!merge || !part) {
        set_error("attention_packed_split: null merge list or partial workspace");
        return -1;
    }
    return attention_packed("attention_packed_split", stream, q16, k16, vt16, M, seq_start, seq_len, pos, B,
                            max_len, H, KV, D, scale, window, ctx_q, ctx_s, ctx32, work, n_work, merge, n_merge,
                            part, part_rows);
}

extern "C" int e2mi_attention_packed_window(e2mi_stream stream, const uint16_t *q16, const uint16_t *k16,
                                            const uint16_t *vt16, int M, const int32_t *seq_start,
                                            const int32_t *seq_len, const int32_t *pos, int B, int max_len,
                                            int H, int KV, int D, float scale, int window, int8_t *ctx_q,
                                            float *ctx_s, float *ctx32, const int32_t *work, int n_work) {
    return attention_packed("attention_packed_window", stream, q16, k16, vt16, M, seq_start, seq_len, pos, B,
                            max_len, H, KV, D, scale, window, ctx_q, ctx_s, ctx32, work, n_work);
}
