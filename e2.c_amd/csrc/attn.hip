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
// B-operand slots must carry, once the A operand (V^T) is read in the same key order.
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
    int B, S, H, KV;
    float scale;
};

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
            *(uint4 *)(Ks + key * kKP + ch * 8) = val;
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
#pragma unroll
            for (int s = 0; s < 16; s++) {
                const h8 kf = *(const h8 *)(kp + 16 * s);
                st = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[s], st, 0, 0, 0);
            }
        }
        // online softmax for this lane's query over the 16 keys it holds (+ the partner's 16)
        float tv[16];
        float mloc = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int key = 8 * (r >> 2) + 4 * half + (r & 3);
            tv[r] = vk[key] ? st[r] * a.scale : -INFINITY;
            mloc = fmaxf(mloc, tv[r]);
        }
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
        const float mnew = fmaxf(mrun, mloc);
        float alpha = 1.f;
        float psum = 0.f;
        _Float16 ph[16];
        if (mnew == -INFINITY) {
#pragma unroll
            for (int r = 0; r < 16; r++) ph[r] = (_Float16)0.f;
        } else {
            alpha = __expf(mrun - mnew);
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const float pr = tv[r] == -INFINITY ? 0.f : __expf(tv[r] - mnew);
                psum += pr;
                ph[r] = (_Float16)pr;
            }
        }
        lrun = lrun * alpha + psum;
        mrun = mnew;
#pragma unroll
        for (int t = 0; t < 8; t++) o[t] *= alpha;
        // O^T += V^T P^T: MFMA #j covers the keys of registers 8j..8j+7, i.e. keys
        // 16j + {4 half + 0..3, 8 + 4 half + 0..3}; V^T is read in that order
        h8 pb[2];
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int e = 0; e < 8; e++) pb[j][e] = ph[8 * j + e];
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const _Float16 *vp = Vs + (32 * t + (lane & 31)) * kVP + 4 * half;
#pragma unroll
            for (int j = 0; j < 2; j++) {
                h8 vf;
                const uint2 lo = *(const uint2 *)(vp + 16 * j), hi = *(const uint2 *)(vp + 16 * j + 8);
                *(uint2 *)&vf = lo;
                *((uint2 *)&vf + 1) = hi;
                o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pb[j], o[t], 0, 0, 0);
            }
        }
    }

    // normalise, quantise per 128 dims (tiles 0-3 and 4-7), store
    const float ltot = lrun + __shfl_xor(lrun, 32);
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
        am = fmaxf(am, __shfl_xor(am, 32));
        const QScale qs = qscale(am);
#pragma unroll
        for (int t = 4 * blk; t < 4 * blk + 4; t++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int d = 32 * t + 8 * g + 4 * half;
                *(uint32_t *)(a.cq + orow * HD + h * kD + d) =
                    pack4(qbyte(o[t][4 * g], qs.inv), qbyte(o[t][4 * g + 1], qs.inv),
                          qbyte(o[t][4 * g + 2], qs.inv), qbyte(o[t][4 * g + 3], qs.inv));
                if (a.c32)
                    *(float4 *)(a.c32 + orow * HD + h * kD + d) =
                        make_float4(o[t][4 * g], o[t][4 * g + 1], o[t][4 * g + 2], o[t][4 * g + 3]);
            }
        if (half == 0) a.cs[orow * (HD / kQBlock) + h * 2 + blk] = qs.sc;
    }
}

}  // namespace e2mi

using namespace e2mi;

extern "C" int e2mi_attention(e2mi_stream stream, const uint16_t *q16, const uint16_t *k16,
                              const uint16_t *vt16, const uint8_t *valid, int B, int S, int H,
                              int KV, int D, float scale, int8_t *ctx_q, float *ctx_s,
                              float *ctx32) {
    if (D != kD || B <= 0 || S <= 0 || H <= 0 || KV <= 0 || H % KV) {
        set_error("attention: needs head_dim 256 and H %% KV == 0 (B=%d S=%d H=%d KV=%d D=%d)", B, S,
                  H, KV, D);
        return -1;
    }
    if (!q16 || !k16 || !vt16 || !valid || !ctx_q || !ctx_s || !aligned16(q16) || !aligned16(k16) ||
        ((uintptr_t)vt16 & 7) || ((uintptr_t)ctx_q & 3) || (ctx32 && !aligned16(ctx32))) {
        set_error("attention: null or misaligned pointer");
        return -1;
    }
    AttnArgs a = {q16, k16, vt16, valid, ctx_q, ctx_s, ctx32, nullptr, nullptr, B, S, H, KV, scale};
    hipLaunchKernelGGL(k_attn, dim3((S + 127) / 128, H, B), dim3(256), 0, (hipStream_t)stream, a);
    return check_hip(hipGetLastError(), "attention launch");
}

extern "C" int e2mi_attention_packed(e2mi_stream stream, const uint16_t *q16, const uint16_t *k16,
                                     const uint16_t *vt16, int M, const int32_t *seq_start,
                                     const int32_t *seq_len, int B, int max_len, int H, int KV, int D,
                                     float scale, int8_t *ctx_q, float *ctx_s, float *ctx32) {
    if (D != kD || B <= 0 || M <= 0 || max_len <= 0 || H <= 0 || KV <= 0 || H % KV) {
        set_error("attention_packed: needs head_dim 256 and H %% KV == 0 (B=%d M=%d H=%d KV=%d D=%d)", B,
                  M, H, KV, D);
        return -1;
    }
    if (!q16 || !k16 || !vt16 || !seq_start || !seq_len || !ctx_q || !ctx_s || !aligned16(q16) ||
        !aligned16(k16) || ((uintptr_t)vt16 & 7) || ((uintptr_t)ctx_q & 3) ||
        (ctx32 && !aligned16(ctx32))) {
        set_error("attention_packed: null or misaligned pointer");
        return -1;
    }
    AttnArgs a = {q16, k16, vt16, nullptr, ctx_q, ctx_s, ctx32, seq_start, seq_len, B, M, H, KV, scale};
    hipLaunchKernelGGL(k_attn, dim3((max_len + 127) / 128, H, B), dim3(256), 0, (hipStream_t)stream, a);
    return check_hip(hipGetLastError(), "attention launch");
}
