// rowops.hip — the memory-bound row kernels of the encoder layer (gfx950, wave64).
//
// Reference semantics (paths relative to the reference root):
//   RMSNorm        x * (1/sqrt(sum(x^2)/D + eps)) * gamma         kernels.c:76-87
//   norm_split     res := x, x := rmsnorm(x) * gamma              kernels.c:149-160, text.c:236-248
//   norm_add       out := rmsnorm(src) * gamma + res              kernels.c:161-171, text.c:250-264
//   embed          x := table[id] * embed_scale                   text.c:917-921
//   q/k/v norm     q,k rmsnorm*gamma, v rmsnorm without gamma     text.c:836-838
//   RoPE           rotate-half, pair (i, i+D/2), positions restart per sequence  kernels.c:112-126
//   GeGLU quant    g := gelu_tanh(gate) * up, quantized per 128   text.c:424-468
//   pooling        masked mean over valid rows, then L2           kernels.c:22-39, text.c:963-981
//
// Each row is held by one wave (D/256 float4 per lane): the sum of squares is a wave reduction,
// and a 128-element quantization block is exactly one half-wave's float4 slice, so the per-block
// amax is a 32-lane reduction. The fused variants read each row once and write the next GEMM's int8
// operand directly, instead of the reference's separate norm, copy and quantize passes.
#include <algorithm>
#include <mutex>

#include "common.h"
#include "rowmath.h"

namespace e2mi {

// ROW_ADDSCALE: ROW_ADDNORM with x scaled after the add and, without gamma_n, x itself quantized
enum { ROW_PLAIN = 0, ROW_EMBED = 1, ROW_ADDNORM = 2, ROW_ADDSCALE = 3 };

struct RowArgs {
    const float *src;      // PLAIN/ADDNORM input rows [M][D] (ld = D)
    const float *res;      // ADDNORM residual [M][D]
    const float *table;    // EMBED table [vocab][D]
    const int32_t *ids;    // EMBED token ids [M], clamped into [0, vocab)
    int vocab;
    int *bad_id;           // EMBED: set to 1 when an id was outside [0, vocab) (optional)
    float embed_scale;
    const float *gamma_a;  // ADDNORM: gamma of the norm applied to src
    const float *gamma_n;  // gamma of the norm producing the quantized operand (NULL: no norm)
    float eps;
    float *x_out;          // new residual stream x (may alias res), or NULL
    float *xn_out;         // normed rows (f32), or NULL
    int8_t *q;             // quantized rows [M][D] (normed; the rows themselves if gamma_n is NULL), or NULL
    float *qs;             // their per-128 scales [M][D/128]
    int M, D;
    float pre_scale = 1.f;   // PLAIN: rows scaled before the norm (the PLE inputs, text.c:930-931)
    float post_scale = 1.f;  // ADDNORM: x scaled after the add (layer_scalar, text.c:959)
    const int *rows = nullptr;  // device row count (times rows_mul, at most M), or null: M
    int rows_mul = 1;
};

// NC = float4 chunks per lane = D / 256 (rounded up); chunk i of lane l covers elements
// 4*(l + 64 i) .. +3, so quantization block (4*(l+64i))/128 = 2i + l/32.
template <int MODE, int NC>
__global__ __launch_bounds__(256) void k_rows(RowArgs a) {
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
    if (m >= a.M || (a.rows && m >= *a.rows * a.rows_mul)) return;
    const int D = a.D, nch = D / 4;
    float4 v[NC];
    const float *row;
    float escale = 1.f;
    if (MODE == ROW_EMBED) {
        const int id0 = a.ids[m];
        if ((id0 < 0 || id0 >= a.vocab) && a.bad_id && l == 0) *a.bad_id = 1;
        const int id = min(max(id0, 0), a.vocab - 1);
        row = a.table + (size_t)id * D;
        escale = a.embed_scale;
    } else {
        row = a.src + (size_t)m * D;
        if (MODE == ROW_PLAIN) escale = a.pre_scale;
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NC; i++) {
        const int c = l + 64 * i;
        v[i] = c < nch ? ld4(row + 4 * c) : make_float4(0.f, 0.f, 0.f, 0.f);
        if (MODE == ROW_EMBED || (MODE == ROW_PLAIN && escale != 1.f))
            v[i] = make_float4(__fmul_rn(v[i].x, escale), __fmul_rn(v[i].y, escale),
                               __fmul_rn(v[i].z, escale), __fmul_rn(v[i].w, escale));
        ss += sumsq4(v[i]);
    }
    if (MODE == ROW_ADDNORM || MODE == ROW_ADDSCALE) {
        // x = rmsnorm(src) * gamma_a + res (ROW_ADDSCALE: then * post_scale)
        const float inv = rms_inv(group_sum<64>(ss), D, a.eps);
        ss = 0.f;
#pragma unroll
        for (int i = 0; i < NC; i++) {
            const int c = l + 64 * i;
            if (c < nch) {
                const float4 g = ld4(a.gamma_a + 4 * c), r = ld4(a.res + (size_t)m * D + 4 * c);
                const float4 t = scale4(v[i], inv, g);
                v[i] = make_float4(t.x + r.x, t.y + r.y, t.z + r.z, t.w + r.w);
                if (MODE == ROW_ADDSCALE)
                    v[i] = make_float4(__fmul_rn(v[i].x, a.post_scale), __fmul_rn(v[i].y, a.post_scale),
                                       __fmul_rn(v[i].z, a.post_scale), __fmul_rn(v[i].w, a.post_scale));
            }
            ss += sumsq4(v[i]);
        }
    }
    if (a.x_out) {
#pragma unroll
        for (int i = 0; i < NC; i++)
            if (l + 64 * i < nch) st4(a.x_out + (size_t)m * D + 4 * (l + 64 * i), v[i]);
    }
    if (MODE != ROW_ADDSCALE && !a.gamma_n) return;
    if (a.gamma_n) {
        const float inv = rms_inv(group_sum<64>(ss), D, a.eps);
#pragma unroll
        for (int i = 0; i < NC; i++) {
            const int c = l + 64 * i;
            if (c < nch) v[i] = scale4(v[i], inv, ld4(a.gamma_n + 4 * c));
            if (a.xn_out && c < nch) st4(a.xn_out + (size_t)m * D + 4 * c, v[i]);
        }
    }
    if (!a.q) return;
    const int nb = D / kQBlock;
#pragma unroll
    for (int i = 0; i < NC; i++) {
        const int c = l + 64 * i;
        // both half-waves of chunk i are either fully inside D or fully outside (D % 128 == 0)
        if (64 * i >= nch) break;
        const float am = group_max<32>(c < nch ? amax4(v[i]) : 0.f);
        if (c < nch) {
            const QScale s = qscale(am);
            *(uint32_t *)(a.q + (size_t)m * D + 4 * c) =
                pack4(qbyte(v[i].x, s.inv), qbyte(v[i].y, s.inv), qbyte(v[i].z, s.inv),
                      qbyte(v[i].w, s.inv));
            if ((l & 31) == 0) a.qs[(size_t)m * nb + (4 * c) / kQBlock] = s.sc;
        }
    }
}

// ---- q/k/v RMSNorm + RoPE: one wave per (row, head) of 256 dims, outputs f16 for the attention.
struct QkvArgs {
    const float *qkv;          // [M][(H + 2 KV) * D]: q heads, k heads, v heads
    const float *q_gamma, *k_gamma;
    const float *cs, *sn;      // [S][D] RoPE tables (cos(f_i) at i and i + D/2)
    float eps;
    uint16_t *q16;             // [M][H*D] f16
    uint16_t *k16;             // [M][KV*D] f16
    uint16_t *vt16;            // [B][KV][D][S] f16 (V transposed per sequence)
    float *q32, *k32, *v32;    // optional f32 copies (parity tests), same layouts as q16/k16/[M][KV*D]
    const int32_t *pos;        // packed batches: RoPE position of each row (then S = M, B = 1)
    int M, S, H, KV;
    const int *rows;           // device row count (at most M), or null: M
};

// f16 of an f32 value that is already rounded: the register barrier keeps the compiler from folding
// the multiply that produced x into the conversion (v_fma_mix rounds the exact product to f16
// once, which differs from rounding it to f32 first)
__device__ inline uint16_t f2h(float x) {
    asm volatile("" : "+v"(x));
    return __builtin_bit_cast(uint16_t, (_Float16)x);
}

// a' = a c - y s and y' = y c + a s, each product rounded, then the sum (kernels.c:112-126)
__device__ inline float4 rot_lo(float4 a, float4 y, float4 c, float4 s) {
    return make_float4(__fmul_rn(a.x, c.x) - __fmul_rn(y.x, s.x), __fmul_rn(a.y, c.y) - __fmul_rn(y.y, s.y),
                       __fmul_rn(a.z, c.z) - __fmul_rn(y.z, s.z), __fmul_rn(a.w, c.w) - __fmul_rn(y.w, s.w));
}
__device__ inline float4 rot_hi(float4 y, float4 a, float4 c, float4 s) {
    return make_float4(__fmul_rn(y.x, c.x) + __fmul_rn(a.x, s.x), __fmul_rn(y.y, c.y) + __fmul_rn(a.y, s.y),
                       __fmul_rn(y.z, c.z) + __fmul_rn(a.z, s.z), __fmul_rn(y.w, c.w) + __fmul_rn(a.w, s.w));
}

// The first nv blocks take the v heads, 32 rows each (one block per kv head and row block), and
// write V^T through LDS so that each d row of V^T gets 64 contiguous bytes instead of one 2-byte
// store per (row, d); they come first so that their longer chains overlap the q/k blocks. The other
// blocks take the q and k heads, one wave per (row, head). D = 256 or 512 (the reference
// checkpoint's full-attention layers): a lane holds D/256 float4 of a row, chunk c covering
// elements 4 (l + 64 c) .. +3; the rotate-half partner of element e is e + D/2, in lane l ^ 32 at
// D = 256 and in the lane's other chunk at D = 512.
template <int D>
__global__ __launch_bounds__(256) void k_qkv_norm_rope(QkvArgs a, int nv) {
    constexpr int VR = 32, NCH = D / 256;
    const int heads = a.H + 2 * a.KV;
    const int l = threadIdx.x & 63;
    if ((int)blockIdx.x < nv) {
        __shared__ __align__(16) uint16_t vbuf[VR * D];
        const int vb = (int)blockIdx.x, nrb = (a.M + VR - 1) / VR;
        const int vh = vb / nrb, m0 = (vb % nrb) * VR, w = threadIdx.x >> 6;
        if (a.rows && m0 >= *a.rows) return;  // the whole block (a packed row count is a multiple of 256)
        const int h = a.H + a.KV + vh;
        // wave w: rows 8 w .. 8 w + 7, four at a time (independent loads in flight)
#pragma unroll
        for (int r0 = 8 * w; r0 < 8 * w + 8; r0 += 4) {
            float4 v[4][NCH];
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int c = 0; c < NCH; c++)
                    v[j][c] = m0 + r0 + j < a.M
                                  ? ld4(a.qkv + (size_t)(m0 + r0 + j) * heads * D + h * D + 4 * (l + 64 * c))
                                  : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                float ss = 0.f;
#pragma unroll
                for (int c = 0; c < NCH; c++) ss += sumsq4(v[j][c]);
                const float inv = rms_inv(group_sum<64>(ss), D, a.eps);
#pragma unroll
                for (int c = 0; c < NCH; c++) {
                    const int e = 4 * (l + 64 * c);
                    const float4 x = make_float4(__fmul_rn(v[j][c].x, inv), __fmul_rn(v[j][c].y, inv),
                                                 __fmul_rn(v[j][c].z, inv), __fmul_rn(v[j][c].w, inv));
                    const uint32_t lo = (uint32_t)f2h(x.x) | ((uint32_t)f2h(x.y) << 16);
                    const uint32_t hi = (uint32_t)f2h(x.z) | ((uint32_t)f2h(x.w) << 16);
                    *(uint2 *)(vbuf + (r0 + j) * D + e) = make_uint2(lo, hi);
                    if (a.v32 && m0 + r0 + j < a.M) st4(a.v32 + (size_t)(m0 + r0 + j) * a.KV * D + vh * D + e, x);
                }
            }
        }
        __syncthreads();
        // thread t writes V^T rows d = t + 256 c for the block's rows: [B][KV][D][S], row m at
        // (m / S, m % S)
        const int nr = min(VR, a.M - m0);
        const int b0 = m0 / a.S, p0 = m0 % a.S;
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            const int d = threadIdx.x + 256 * c;
            uint16_t *dst = a.vt16 + ((size_t)(b0 * a.KV + vh) * D + d) * a.S + p0;
            if (nr == VR && p0 + VR <= a.S && ((uintptr_t)dst & 15) == 0) {
#pragma unroll
                for (int k8 = 0; k8 < VR / 8; k8++) {
                    uint32_t wv[4];
#pragma unroll
                    for (int k = 0; k < 4; k++)
                        wv[k] = (uint32_t)vbuf[(8 * k8 + 2 * k) * D + d] |
                                ((uint32_t)vbuf[(8 * k8 + 2 * k + 1) * D + d] << 16);
                    *(uint4 *)(dst + 8 * k8) = make_uint4(wv[0], wv[1], wv[2], wv[3]);
                }
            } else {
                for (int r = 0; r < nr; r++) {
                    const int m = m0 + r, b = m / a.S, p = m % a.S;
                    a.vt16[((size_t)(b * a.KV + vh) * D + d) * a.S + p] = vbuf[r * D + d];
                }
            }
        }
        return;
    }
    const int qkh = a.H + a.KV;
    const long item = (long)(blockIdx.x - nv) * 4 + (threadIdx.x >> 6);
    if (item >= (long)a.M * qkh) return;
    const int m = (int)(item / qkh), h = (int)(item % qkh);
    if (a.rows && m >= *a.rows) return;
    const int kind = h < a.H ? 0 : 1;  // q, k
    const float *src = a.qkv + (size_t)m * heads * D + h * D;
    float4 v[NCH];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        v[c] = ld4(src + 4 * (l + 64 * c));
        ss += sumsq4(v[c]);
    }
    const float inv = rms_inv(group_sum<64>(ss), D, a.eps);
    const float *gam = kind == 0 ? a.q_gamma : a.k_gamma;
#pragma unroll
    for (int c = 0; c < NCH; c++) v[c] = scale4(v[c], inv, ld4(gam + 4 * (l + 64 * c)));
    // rotate-half (kernels.c:112-126): a' = a c - y s for the first half, y' = y c + a s for the
    // second, with a = x[i], y = x[i + D/2] and c, s the angle of i (duplicated at i + D/2)
    const int pos = a.pos ? a.pos[m] : m % a.S;
    const float *cp = a.cs + (size_t)pos * D, *sp = a.sn + (size_t)pos * D;
    if (NCH == 1) {
        const float4 c = ld4(cp + 4 * l), s = ld4(sp + 4 * l);
        const float4 o = make_float4(xor_lane<32>(v[0].x), xor_lane<32>(v[0].y), xor_lane<32>(v[0].z),
                                     xor_lane<32>(v[0].w));
        if (l < 32) v[0] = rot_lo(v[0], o, c, s);
        else v[0] = rot_hi(v[0], o, c, s);
    } else {
        const float4 c = ld4(cp + 4 * l), s = ld4(sp + 4 * l);
        const float4 x0 = v[0], x1 = v[NCH - 1];
        v[0] = rot_lo(x0, x1, c, s);
        v[NCH - 1] = rot_hi(x1, x0, c, s);
    }
#pragma unroll
    for (int c = 0; c < NCH; c++) {
        const int e = 4 * (l + 64 * c);
        const uint32_t lo = (uint32_t)f2h(v[c].x) | ((uint32_t)f2h(v[c].y) << 16);
        const uint32_t hi = (uint32_t)f2h(v[c].z) | ((uint32_t)f2h(v[c].w) << 16);
        if (kind == 0) {
            *(uint2 *)(a.q16 + (size_t)m * a.H * D + h * D + e) = make_uint2(lo, hi);
            if (a.q32) st4(a.q32 + (size_t)m * a.H * D + h * D + e, v[c]);
        } else {
            const int kh = h - a.H;
            *(uint2 *)(a.k16 + (size_t)m * a.KV * D + kh * D + e) = make_uint2(lo, hi);
            if (a.k32) st4(a.k32 + (size_t)m * a.KV * D + kh * D + e, v[c]);
        }
    }
}

// ---- standalone GeGLU * up + quantize (the unfused gate_quant of text.c:424-468)
__device__ inline float gelu_tanh_f(float v) {
    const float c = 0.7978845608028654f;
    return 0.5f * v * (1.f + tanhf(c * (v + 0.044715f * v * v * v)));
}

__global__ __launch_bounds__(256) void k_gelu_mul_quant(float *__restrict__ gate, int ldg,
                                                        const float *__restrict__ up, int ldu,
                                                        int M, int D, int8_t *__restrict__ q,
                                                        float *__restrict__ qs, int write_back) {
    const int nb = D / kQBlock;
    const long item = (long)blockIdx.x * 8 + (threadIdx.x >> 5);
    if (item >= (long)M * nb) return;
    const int m = (int)(item / nb), b = (int)(item % nb), l = threadIdx.x & 31;
    float4 g = ld4(gate + (size_t)m * ldg + b * kQBlock + 4 * l);
    const float4 u = ld4(up + (size_t)m * ldu + b * kQBlock + 4 * l);
    g = make_float4(gelu_tanh_f(g.x) * u.x, gelu_tanh_f(g.y) * u.y, gelu_tanh_f(g.z) * u.z,
                    gelu_tanh_f(g.w) * u.w);
    if (write_back) st4(gate + (size_t)m * ldg + b * kQBlock + 4 * l, g);
    const QScale s = qscale(group_max<32>(amax4(g)));
    *(uint32_t *)(q + (size_t)m * D + b * kQBlock + 4 * l) =
        pack4(qbyte(g.x, s.inv), qbyte(g.y, s.inv), qbyte(g.z, s.inv), qbyte(g.w, s.inv));
    if (l == 0) qs[(size_t)m * nb + b] = s.sc;
}

// ---- masked mean pool + L2: partial sums per (sequence, 64-row chunk), then a finishing pass
// rows are added in order, r0 .. r1 - 1, eight at a time: the eight loads are issued before the
// first addition, so a thread keeps eight 16-byte loads in flight instead of one
constexpr int kPoolBatch = 8;
__global__ __launch_bounds__(256) void k_pool_partial(const float *__restrict__ x,
                                                      const uint8_t *__restrict__ valid, int S,
                                                      int D, int chunks, float *__restrict__ part,
                                                      int *__restrict__ cnt) {
    const int b = blockIdx.x / chunks, ch = blockIdx.x % chunks;
    const int r0 = ch * 64, r1 = min(S, r0 + 64);
    for (int c = threadIdx.x; c < D / 4; c += blockDim.x) {
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int rb = r0; rb < r1; rb += kPoolBatch) {
            float4 v[kPoolBatch];
            bool keep[kPoolBatch];
#pragma unroll
            for (int i = 0; i < kPoolBatch; i++) {
                const int r = rb + i;
                keep[i] = r < r1 && valid[(size_t)b * S + r];
                v[i] = keep[i] ? ld4(x + ((size_t)b * S + r) * D + 4 * c) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int i = 0; i < kPoolBatch; i++)
                if (keep[i]) acc = make_float4(acc.x + v[i].x, acc.y + v[i].y, acc.z + v[i].z, acc.w + v[i].w);
        }
        st4(part + ((size_t)b * chunks + ch) * D + 4 * c, acc);
    }
    if (threadIdx.x == 0) {
        int n = 0;
        for (int r = r0; r < r1; r++) n += valid[(size_t)b * S + r] != 0;
        cnt[b * chunks + ch] = n;
    }
}

// packed batches: sequence b is rows [start[b], start[b] + len[b]), all valid; chunk ch covers its
// rows 64 ch .. 64 ch + 63, so a right-padded batch sums in the same order as the masked kernel
__global__ __launch_bounds__(256) void k_pool_partial_packed(const float *__restrict__ x,
                                                             const int32_t *__restrict__ start,
                                                             const int32_t *__restrict__ len, int D,
                                                             int chunks, float *__restrict__ part,
                                                             int *__restrict__ cnt) {
    const int b = blockIdx.x / chunks, ch = blockIdx.x % chunks;
    const int r0 = ch * 64, r1 = min(len[b], r0 + 64);
    const size_t base = (size_t)start[b];
    for (int c = threadIdx.x; c < D / 4; c += blockDim.x) {
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int rb = r0; rb < r1; rb += kPoolBatch) {
            float4 v[kPoolBatch];
#pragma unroll
            for (int i = 0; i < kPoolBatch; i++)
                v[i] = rb + i < r1 ? ld4(x + (base + rb + i) * D + 4 * c) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int i = 0; i < kPoolBatch; i++)
                if (rb + i < r1) acc = make_float4(acc.x + v[i].x, acc.y + v[i].y, acc.z + v[i].z, acc.w + v[i].w);
        }
        st4(part + ((size_t)b * chunks + ch) * D + 4 * c, acc);
    }
    if (threadIdx.x == 0) cnt[b * chunks + ch] = max(0, r1 - r0);
}

// the finishing kernel keeps up to kPoolPerThread means per thread: D <= 256 * kPoolPerThread
constexpr int kPoolPerThread = 5;
constexpr int kPoolMaxD = 256 * kPoolPerThread;

__global__ __launch_bounds__(256) void k_pool_finish(const float *__restrict__ part,
                                                     const int *__restrict__ cnt, int chunks,
                                                     int D, float *__restrict__ out) {
    const int b = blockIdx.x;
    __shared__ float red[256 / 64];
    int n = 0;
    for (int ch = 0; ch < chunks; ch++) n += cnt[b * chunks + ch];
    float ss = 0.f;
    float vals[kPoolPerThread];
    int k = 0;
    for (int d = threadIdx.x; d < D; d += blockDim.x, k++) {
        float s = 0.f;
        for (int ch = 0; ch < chunks; ch++) s += part[((size_t)b * chunks + ch) * D + d];
        const float mean = n > 0 ? __fdiv_rn(s, (float)n) : 0.f;
        if (k < kPoolPerThread) vals[k] = mean;
        ss += mean * mean;
    }
    ss = group_sum<64>(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
    for (int w = 0; w < (int)blockDim.x / 64; w++) tot += red[w];
    // all-invalid sequences stay an exact zero vector (text.c:968-980)
    const float inv = n > 0 ? __fdiv_rn(1.0f, __fsqrt_rn(tot)) : 1.0f;
    k = 0;
    for (int d = threadIdx.x; d < D && k < kPoolPerThread; d += blockDim.x, k++)
        out[(size_t)b * D + d] = n > 0 ? __fmul_rn(vals[k], inv) : 0.f;
}

// zero n floats (an all-padding chunk's embeddings): a kernel rather than a memset node, so a
// caller may capture it
__global__ __launch_bounds__(256) void k_zero_f32(float *__restrict__ p, long n) {
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) p[i] = 0.f;
}
// raise *flag when any of n ids lies outside [0, vocab) (masked positions included, e2.h:31-32)
__global__ __launch_bounds__(256) void k_check_ids(const int32_t *__restrict__ ids, long n, int vocab, int *flag) {
    bool bad = false;
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256)
        bad |= ids[i] < 0 || ids[i] >= vocab;
    if (bad) *flag = 1;
}

// ---- packed batches: token ids of the packed rows (filler rows, rowmap < 0, get token 0)
__global__ __launch_bounds__(256) void k_gather_ids(const int32_t *__restrict__ ids,
                                                    const int32_t *__restrict__ rowmap, int M,
                                                    int32_t *__restrict__ out) {
    const int r = blockIdx.x * 256 + threadIdx.x;
    if (r < M) {
        const int src = rowmap[r];
        out[r] = src >= 0 ? ids[src] : 0;
    }
}

// ------------------------------------------------------------------ launchers
static int row_launch(hipStream_t s, int mode, const RowArgs &a) {
    if (a.M <= 0 || a.D <= 0 || a.D % 128 || a.D > 1280) {
        set_error("row kernel: D must be a multiple of 128 up to 1280 (D=%d, M=%d)", a.D, a.M);
        return -1;
    }
    const int nc = (a.D / 4 + 63) / 64;
    dim3 grid((a.M + 3) / 4), block(256);
    RowArgs b = a;
    if (!b.rows) {
        b.rows = device_rows().ptr;
        b.rows_mul = device_rows().mul;
    }
#define ROWK(MODE)                                                                          \
    switch (nc) {                                                                           \
    case 1: hipLaunchKernelGGL((k_rows<MODE, 1>), grid, block, 0, s, b); break;             \
    case 2: hipLaunchKernelGGL((k_rows<MODE, 2>), grid, block, 0, s, b); break;             \
    case 3: hipLaunchKernelGGL((k_rows<MODE, 3>), grid, block, 0, s, b); break;             \
    case 4: hipLaunchKernelGGL((k_rows<MODE, 4>), grid, block, 0, s, b); break;             \
    default: hipLaunchKernelGGL((k_rows<MODE, 5>), grid, block, 0, s, b); break;            \
    }
    if (mode == ROW_EMBED) { ROWK(ROW_EMBED) }
    else if (mode == ROW_ADDNORM) { ROWK(ROW_ADDNORM) }
    else if (mode == ROW_ADDSCALE) { ROWK(ROW_ADDSCALE) }
    else { ROWK(ROW_PLAIN) }
#undef ROWK
    return check_hip(hipGetLastError(), "row kernel launch");
}

int launch_rows(hipStream_t s, int mode, const RowArgs &a) { return row_launch(s, mode, a); }

int launch_qkv_norm_rope(hipStream_t s, const QkvArgs &qa, int D) {
    QkvArgs a = qa;
    if (!a.rows) a.rows = device_rows().ptr;
    const long nqk = ((long)a.M * (a.H + a.KV) + 3) / 4;
    const long nv = (long)a.KV * ((a.M + 31) / 32);
    if (nqk + nv > 0x7fffffffL) {
        set_error("qkv_norm_rope: too many rows");
        return -1;
    }
    if (D == 512)
        hipLaunchKernelGGL(k_qkv_norm_rope<512>, dim3((unsigned)(nqk + nv)), dim3(256), 0, s, a, (int)nv);
    else
        hipLaunchKernelGGL(k_qkv_norm_rope<256>, dim3((unsigned)(nqk + nv)), dim3(256), 0, s, a, (int)nv);
    return check_hip(hipGetLastError(), "qkv_norm_rope launch");
}

int launch_pool_packed(hipStream_t s, const float *x, const int32_t *start, const int32_t *len,
                       int B, int max_len, int D, float *part, int *cnt, float *out) {
    const int chunks = (max_len + 63) / 64;
    hipLaunchKernelGGL(k_pool_partial_packed, dim3(B * chunks), dim3(256), 0, s, x, start, len, D,
                       chunks, part, cnt);
    hipLaunchKernelGGL(k_pool_finish, dim3(B), dim3(256), 0, s, part, cnt, chunks, D, out);
    return check_hip(hipGetLastError(), "pool launch");
}

int launch_pool(hipStream_t s, const float *x, const uint8_t *valid, int B, int S, int D,
                float *part, int *cnt, float *out) {
    const int chunks = (S + 63) / 64;
    hipLaunchKernelGGL(k_pool_partial, dim3(B * chunks), dim3(256), 0, s, x, valid, S, D, chunks,
                       part, cnt);
    hipLaunchKernelGGL(k_pool_finish, dim3(B), dim3(256), 0, s, part, cnt, chunks, D, out);
    return check_hip(hipGetLastError(), "pool launch");
}

}  // namespace e2mi

// ------------------------------------------------------------------ C ABI
using namespace e2mi;

static bool al16(const void *p) { return !p || aligned16(p); }

extern "C" int e2mi_norm_quant(e2mi_stream stream, const float *x, const float *gamma, float eps,
                               int M, int D, float *xn_out, int8_t *q, float *qs) {
    if (!x || !gamma || !al16(x) || !al16(xn_out) || !al16(gamma) || (!q) != (!qs)) {
        set_error("norm_quant: null/misaligned pointer");
        return -1;
    }
    RowArgs a = {};
    a.src = x; a.gamma_n = gamma; a.eps = eps; a.xn_out = xn_out; a.q = q; a.qs = qs; a.M = M; a.D = D;
    return launch_rows((hipStream_t)stream, ROW_PLAIN, a);
}

extern "C" int e2mi_add_norm_quant(e2mi_stream stream, const float *src, const float *res,
                                   const float *gamma_add, const float *gamma_next, float eps,
                                   int M, int D, float *x_out, float *xn_out, int8_t *q, float *qs) {
    if (!src || !res || !gamma_add || !al16(src) || !al16(res) || !al16(x_out) || !al16(xn_out) ||
        (q && !gamma_next) || (!q) != (!qs)) {
        set_error("add_norm_quant: null/misaligned pointer, or quantized output without gamma_next");
        return -1;
    }
    RowArgs a = {};
    a.src = src; a.res = res; a.gamma_a = gamma_add; a.gamma_n = gamma_next; a.eps = eps;
    a.x_out = x_out; a.xn_out = xn_out; a.q = q; a.qs = qs; a.M = M; a.D = D;
    return launch_rows((hipStream_t)stream, ROW_ADDNORM, a);
}

extern "C" int e2mi_add_norm_scale_quant(e2mi_stream stream, const float *src, const float *res,
                                         const float *gamma_add, float post_scale, const float *gamma_next,
                                         float eps, int M, int D, float *x_out, float *xn_out, int8_t *q,
                                         float *qs) {
    if (!src || !res || !gamma_add || !al16(src) || !al16(res) || !al16(x_out) || !al16(xn_out) ||
        (xn_out && !gamma_next) || (!q) != (!qs)) {
        set_error("add_norm_scale_quant: null/misaligned pointer, or normed output without gamma_next");
        return -1;
    }
    RowArgs a = {};
    a.src = src; a.res = res; a.gamma_a = gamma_add; a.gamma_n = gamma_next; a.eps = eps;
    a.x_out = x_out; a.xn_out = xn_out; a.q = q; a.qs = qs; a.M = M; a.D = D; a.post_scale = post_scale;
    return launch_rows((hipStream_t)stream, ROW_ADDSCALE, a);
}

extern "C" int e2mi_scale_norm(e2mi_stream stream, const float *x, int rows, int D, float pre_scale,
                               const float *gamma, float eps, float *out) {
    if (!x || !gamma || !out || !al16(x) || !al16(out) || !al16(gamma) || rows <= 0) {
        set_error("scale_norm: null/misaligned pointer or rows <= 0");
        return -1;
    }
    RowArgs a = {};
    a.src = x; a.gamma_n = gamma; a.eps = eps; a.xn_out = out; a.M = rows; a.D = D; a.pre_scale = pre_scale;
    return launch_rows((hipStream_t)stream, ROW_PLAIN, a);
}

namespace e2mi {
// the engine's embedding launch: e2mi_embed_norm_quant that also raises *bad_id for an id outside
// the vocabulary (the id itself is clamped, so the gather stays in the table)
int launch_embed_checked(hipStream_t s, const float *table, int vocab, const int32_t *ids, float embed_scale,
                         const float *gamma, float eps, int M, int D, float *x_out, int8_t *q, float *qs,
                         int *bad_id) {
    RowArgs a = {};
    a.table = table; a.vocab = vocab; a.ids = ids; a.embed_scale = embed_scale; a.gamma_n = gamma; a.eps = eps;
    a.x_out = x_out; a.q = q; a.qs = qs; a.M = M; a.D = D; a.bad_id = bad_id;
    return launch_rows(s, ROW_EMBED, a);
}
int launch_zero_f32(hipStream_t s, float *p, long n) {
    if (n <= 0) return 0;
    const long blocks = std::min((n + 255) / 256, 4096L);
    hipLaunchKernelGGL(k_zero_f32, dim3((unsigned)blocks), dim3(256), 0, s, p, n);
    return check_hip(hipGetLastError(), "zero fill launch");
}
int launch_check_ids(hipStream_t s, const int32_t *ids, long n, int vocab, int *flag) {
    if (n <= 0) return 0;
    const long blocks = std::min((n + 255) / 256, 1024L);
    hipLaunchKernelGGL(k_check_ids, dim3((unsigned)blocks), dim3(256), 0, s, ids, n, vocab, flag);
    return check_hip(hipGetLastError(), "id check launch");
}
}  // namespace e2mi

extern "C" int e2mi_embed_norm_quant(e2mi_stream stream, const float *table, int vocab,
                                     const int32_t *ids, float embed_scale, const float *gamma, float eps, int M, int D,
                                     float *x_out, int8_t *q, float *qs) {
    if (!table || vocab <= 0 || !ids || !gamma || !x_out || !al16(table) || !al16(x_out) ||
        (!q) != (!qs)) {
        set_error("embed_norm_quant: null/misaligned pointer");
        return -1;
    }
    RowArgs a = {};
    a.table = table; a.vocab = vocab; a.ids = ids; a.embed_scale = embed_scale; a.gamma_n = gamma; a.eps = eps;
    a.x_out = x_out; a.q = q; a.qs = qs; a.M = M; a.D = D;
    return launch_rows((hipStream_t)stream, ROW_EMBED, a);
}

extern "C" int e2mi_qkv_norm_rope(e2mi_stream stream, const float *qkv, int M, int S, int H, int KV,
                                  int D, const float *q_gamma, const float *k_gamma, float eps,
                                  const float *cos_tab, const float *sin_tab, uint16_t *q16,
                                  uint16_t *k16, uint16_t *vt16, float *q32, float *k32, float *v32) {
    if (D != 256 || H <= 0 || KV <= 0 || H % KV || M <= 0 || S <= 0 || M % S) {
        set_error("qkv_norm_rope: needs head_dim 256, H %% KV == 0 and M a multiple of S (M=%d S=%d H=%d KV=%d D=%d)",
                  M, S, H, KV, D);
        return -1;
    }
    if (!qkv || !q_gamma || !k_gamma || !cos_tab || !sin_tab || !q16 || !k16 || !vt16 ||
        !aligned16(qkv) || !al16(q32) || !al16(k32) || !al16(v32) || ((uintptr_t)q16 & 7) ||
        ((uintptr_t)k16 & 7)) {
        set_error("qkv_norm_rope: null/misaligned pointer");
        return -1;
    }
    QkvArgs a = {qkv, q_gamma, k_gamma, cos_tab, sin_tab, eps, q16, k16, vt16, q32, k32, v32, nullptr, M, S, H, KV};
    return launch_qkv_norm_rope((hipStream_t)stream, a, D);
}

extern "C" int e2mi_qkv_norm_rope_packed(e2mi_stream stream, const float *qkv, int M, const int32_t *pos,
                                         int H, int KV, int D, const float *q_gamma, const float *k_gamma,
                                         float eps, const float *cos_tab, const float *sin_tab,
                                         uint16_t *q16, uint16_t *k16, uint16_t *vt16, float *q32,
                                         float *k32, float *v32) {
    if ((D != 256 && D != 512) || H <= 0 || KV <= 0 || H % KV || M <= 0) {
        set_error("qkv_norm_rope_packed: needs head_dim 256 or 512 and H %% KV == 0 (M=%d H=%d KV=%d D=%d)", M,
                  H, KV, D);
        return -1;
    }
    if (!qkv || !pos || !q_gamma || !k_gamma || !cos_tab || !sin_tab || !q16 || !k16 || !vt16 ||
        !aligned16(qkv) || !al16(q32) || !al16(k32) || !al16(v32) || ((uintptr_t)q16 & 7) ||
        ((uintptr_t)k16 & 7)) {
        set_error("qkv_norm_rope_packed: null/misaligned pointer");
        return -1;
    }
    QkvArgs a = {qkv, q_gamma, k_gamma, cos_tab, sin_tab, eps, q16, k16, vt16, q32, k32, v32, pos, M, M, H, KV};
    return launch_qkv_norm_rope((hipStream_t)stream, a, D);
}

extern "C" int e2mi_gelu_mul_quant(e2mi_stream stream, float *gate, int ldg, const float *up,
                                   int ldu, int M, int D, int8_t *q, float *qs, int write_back) {
    if (!gate || !up || !q || !qs || M <= 0 || D <= 0 || D % 128 || ldg < D || ldu < D ||
        ldg % 4 || ldu % 4 || !aligned16(gate) || !aligned16(up)) {
        set_error("gelu_mul_quant: bad geometry or pointers (D %% 128 == 0)");
        return -1;
    }
    const long items = (long)M * (D / 128);
    hipLaunchKernelGGL(k_gelu_mul_quant, dim3((unsigned)((items + 7) / 8)), dim3(256), 0,
                       (hipStream_t)stream, gate, ldg, up, ldu, M, D, q, qs, write_back);
    return check_hip(hipGetLastError(), "gelu_mul_quant launch");
}

extern "C" int e2mi_pool_l2(e2mi_stream stream, const float *x, const uint8_t *valid, int B, int S,
                            int D, float *workspace, float *out) {
    if (!x || !valid || !workspace || !out || B <= 0 || S <= 0 || D <= 0 || D % 4 || D > kPoolMaxD ||
        !aligned16(x) || !aligned16(workspace)) {
        set_error("pool_l2: bad geometry or pointers (D a multiple of 4 up to %d)", kPoolMaxD);
        return -1;
    }
    const int chunks = (S + 63) / 64;
    float *part = workspace;
    int *cnt = (int *)(workspace + (size_t)B * chunks * D);
    return launch_pool((hipStream_t)stream, x, valid, B, S, D, part, cnt, out);
}

extern "C" int e2mi_pool_l2_packed(e2mi_stream stream, const float *x, const int32_t *seq_start,
                                   const int32_t *seq_len, int B, int max_len, int D, float *workspace,
                                   float *out) {
    if (!x || !seq_start || !seq_len || !workspace || !out || B <= 0 || max_len <= 0 || D <= 0 ||
        D % 4 || D > kPoolMaxD || !aligned16(x) || !aligned16(workspace)) {
        set_error("pool_l2_packed: bad geometry or pointers (D a multiple of 4 up to %d)", kPoolMaxD);
        return -1;
    }
    const int chunks = (max_len + 63) / 64;
    float *part = workspace;
    int *cnt = (int *)(workspace + (size_t)B * chunks * D);
    return launch_pool_packed((hipStream_t)stream, x, seq_start, seq_len, B, max_len, D, part, cnt, out);
}

extern "C" size_t e2mi_pool_workspace_bytes(int B, int S, int D) {
    const size_t chunks = (size_t)(S + 63) / 64;
    return (size_t)B * chunks * (D + 1) * sizeof(float);
}

extern "C" int e2mi_gather_ids(e2mi_stream stream, const int32_t *ids, const int32_t *rowmap, int M,
                               int32_t *out) {
    if (!ids || !rowmap || !out || M <= 0) {
        set_error("gather_ids: null pointer or M <= 0");
        return -1;
    }
    hipLaunchKernelGGL(k_gather_ids, dim3((unsigned)((M + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       ids, rowmap, M, out);
    return check_hip(hipGetLastError(), "gather_ids launch");
}

// ------------------------------------------------------------------ allocation-free pooling
// e2mi_pool_l2 with its partial sums in a file-scope device array instead of a caller workspace,
// for callers that cannot allocate (graph capture, serving loops). The array's address on each
// device is looked up once, with that device current, and kept; host code passes that address to
// the kernels, never the array's name.
namespace {
constexpr size_t kPoolScratchFloats = (size_t)2 << 20;  // 8 MiB per device
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float *g_scratch_ptr[kMaxDevices] = {};
}  // namespace
static __device__ __align__(256) float scratch[kPoolScratchFloats];

static float *pool_scratch(int dev) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        float *p = nullptr;
        if (check_hip(hipGetSymbolAddress((void **)&p, HIP_SYMBOL(scratch)), "pool scratch address")) return nullptr;
        g_scratch_ptr[dev] = p;
    }
    return g_scratch_ptr[dev];
}

extern "C" int e2mi_pool_l2_noalloc(e2mi_stream stream, const float *x, const uint8_t *valid, int B, int S,
                                    int D, float *out) {
    if (!x || !valid || !out || B <= 0 || S <= 0 || D <= 0 || D % 4 || D > kPoolMaxD || !aligned16(x)) {
        set_error("pool_l2_noalloc: bad geometry or pointers (D a multiple of 4 up to %d)", kPoolMaxD);
        return -1;
    }
    const size_t need = e2mi_pool_workspace_bytes(B, S, D) / sizeof(float);
    if (need > kPoolScratchFloats) {
        set_error("pool_l2_noalloc: %d sequences of %d rows x %d need %zu bytes of scratch, the limit is %zu",
                  B, S, D, need * sizeof(float), kPoolScratchFloats * sizeof(float));
        return -1;
    }
    int dev = 0;
    if (check_hip(hipGetDevice(&dev), "get device")) return -1;
    if (dev < 0 || dev >= kMaxDevices) {
        set_error("pool_l2_noalloc: device %d beyond the %d this library tracks", dev, kMaxDevices);
        return -1;
    }
    float *ws = pool_scratch(dev);
    if (!ws) return -1;
    // every partial sum and count slot is written by the first kernel: nothing to clear
    const int chunks = (S + 63) / 64;
    return launch_pool((hipStream_t)stream, x, valid, B, S, D, ws, (int *)(ws + (size_t)B * chunks * D), out);
}
