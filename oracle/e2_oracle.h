/* e2_oracle.h — CPU restatement of the reference's int8 encoder hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load liboracle.so, and only as the checker or the timed CPU baseline; the product library never
 * links it and must fail loudly if its HIP code is missing.
 *
 * Conventions follow the reference (Damix48/e2.c, paths relative to its root):
 *   - activations are quantized per (row, 128-element block): src/int8.h:61-70;
 *   - the quantizer arithmetic is the one GCC emits for src/kernels_i8_avx512_vnni.c:321-363 under
 *     the reference's flags (-O3 -ffast-math, CMakeLists.txt:110): sc = amax * RN(1/127) and
 *     inv = 127 / amax (a true division), q = round-to-nearest-even(x * inv), saturated to int8;
 *   - the GEMM accumulates exact int32 per block and folds each block into the f32 output with
 *     f = fma((float)acc, RN(as * ws), f) in block order: kernels_i8_avx512_vnni.c:100-122;
 *   - activation bytes are stored SIGNED here (the HIP convention, include/e2hip.h:19-21); the CPU
 *     reference stores q+128, so cpu_byte == (uint8_t)(signed_byte ^ 0x80).
 *
 * Parity status of every function is listed in the header comment of e2_oracle.c.
 */
#ifndef E2_ORACLE_H
#define E2_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- a1/a2: weight container (int8.h:14-36,79-92; int8.c:19-66) */
int or_q8w_from_f32(const float *w, int N, int K, int8_t *wq, float *scale, int32_t *bsq);
void or_q8w_unpack(const int8_t *wq, int N, int K, int8_t *rowmajor);
void or_q8w_pack(const int8_t *rowmajor, int N, int K, int8_t *wq, int32_t *bsq);

/* ---- a3/a4: activation quantizer (int8.c:178-209; kernels_i8_avx512_vnni.c:312-366) */
void or_quantize(const float *x, int M, int K, int ldx, int block, int8_t *q, float *scales);

/* ---- a5/a6: int8 GEMM, AVX-512 fold order (kernels_i8_avx512_vnni.c:84-307) */
void or_i8_gemm(const int8_t *qa, const float *as, const int8_t *w, const float *ws,
                const float *bias, int M, int N, int K, int block, float lo, float hi, float *y);
void or_i8_gemm_acc(const int8_t *qa, const int8_t *w, int M, int N, int K, int block,
                    int32_t *acc);
/* the scalar reference's fold, y += (float)acc * (as * ws) without fma (int8.c:113-171) */
void or_i8_gemm_scalar(const int8_t *qa, const float *as, const int8_t *w, const float *ws, int M,
                       int N, int K, float *y);

/* ---- a8: GELU-tanh * up, then the quantizer (text.c:424-468; kernels.c:89-95) */
float or_gelu_tanh(float v);
void or_gelu_mul_quant(float *gate, int ldg, const float *up, int ldu, int rows, int D, int block,
                       int8_t *q, float *scales);

/* ---- a10: RMSNorm family (kernels.c:76-87,144-171) */
void or_rmsnorm(float *x, int rows, int D, const float *gamma, float eps);
void or_norm_split(float *x, float *res, int rows, int D, const float *gamma, float eps);
void or_norm_add(float *out, const float *src, const float *res, int rows, int D,
                 const float *gamma, float eps);

/* ---- a11: RoPE (text.c:483-506; kernels.c:112-126) */
void or_rope_table(int max_pos, int head_dim, float theta, float *cs, float *sn);
void or_rope_rows(float *x, int rows, int ngroups, int head_dim, const float *cs, const float *sn);

/* ---- a13/a14: attention core, row-wise oracle (text.c:534-572), softmax (kernels.c:97-104) */
void or_softmax(float *x, int n);
void or_attention(const float *q, int ldq, const float *k, int ldk, const float *v, int ldv,
                  const uint8_t *valid, int S, int H, int KV, int D, float scale, float *ctx,
                  int ldc, int nthreads);
/* the same with the sliding window of text.c:542-546: query i reads keys j with |i-j| <= window
 * (window <= 0: all keys) */
void or_attention_win(const float *q, int ldq, const float *k, int ldk, const float *v, int ldv,
                      const uint8_t *valid, int S, int H, int KV, int D, float scale, int window,
                      float *ctx, int ldc, int nthreads);
int or_attention_i8(const float *q, int ldq, const float *k, int ldk, const float *v, int ldv,
                    int S, int H, int KV, int D, float *ctx, int ldc);
int or_attention_i8_win(const float *q, int ldq, const float *k, int ldk, const float *v, int ldv,
                        int S, int H, int KV, int D, int window, float *ctx, int ldc);

/* ---- a15/a16: pooling + L2 (kernels.c:22-39), embedding (text.c:917-921) */
void or_meanpool(const float *x, int M, int D, const uint8_t *valid, float *out);
void or_l2norm(float *x, int n);
void or_embed(const float *table, const int32_t *ids, int n, int D, float scale, float *x);

/* ---- a6 at scale: threaded GEMM driver (text.c:275-421) for the CPU baseline */
void or_i8_gemm_mt(const int8_t *qa, const float *as, const int8_t *w, const float *ws,
                   const float *bias, int M, int N, int K, float *y, int nthreads);
/* the same with one activation scale per `block` columns (K % block == 0, block % 4 == 0): block = K
 * is the per-token fold (int8.h:61-70, E2_I8_BLOCK = K) */
void or_i8_gemm_mt_block(const int8_t *qa, const float *as, const int8_t *w, const float *ws,
                         const float *bias, int M, int N, int K, int block, float *y, int nthreads);
void or_quantize_mt(const float *x, int M, int K, int8_t *q, float *scales, int nthreads);

/* ---- a9/a12 + text_forward (text.c:817-984): the BASELINE geometry, or the reference
 *      checkpoint's (PLE, sliding window, per-layer head_dim, embed_proj) */
typedef struct {
    const int8_t *wqkv;  /* [(H+2KV)*D][hidden] row-major: q rows, then k, then v */
    const float *sqkv;
    const int8_t *wo;    /* [hidden][H*D] */
    const float *so;
    const int8_t *wgate; /* [ffn][hidden] */
    const float *sgate;
    const int8_t *wup;   /* [ffn][hidden] */
    const float *sup;
    const int8_t *wdown; /* [hidden][ffn] */
    const float *sdown;
    const float *input_ln, *post_attn_ln, *pre_ffn_ln, *post_ffn_ln; /* [hidden] */
    const float *q_norm, *k_norm;                                    /* [head_dim] */
    /* the reference checkpoint's PLE block (text.c:906-915) and layer scale (text.c:959-961);
     * unused when the model has no PLE (ple_dim 0) */
    const int8_t *wple_gate; /* [ple_dim][hidden] */
    const float *sple_gate;
    const int8_t *wple_proj; /* [hidden][ple_dim] */
    const float *sple_proj;
    const float *ple_norm;   /* [hidden] */
    float layer_scalar;      /* 1.0 where the model has none */
} or_layer;

typedef struct {
    int n_layers, hidden, ffn, n_heads, n_kv, head_dim, vocab;
    float eps, rope_theta, embed_scale, attn_scale;
    const float *embed;      /* [vocab][hidden] */
    const float *final_norm; /* [hidden] */
    const or_layer *layers;
    /* 1: the int8 attention (text.c:638-700, with the layer's window) for sequences of >= 32 rows
     * with no padding inside (the reference's blocked path, text.c:873-875, selected as dispatch.c
     * picks i8); 0: f32 */
    int attn_i8;
    /* the reference checkpoint's geometry (e2.c:294-301, text.c:467-478); zeros give the BASELINE
     * geometry (every layer alike, no window, no PLE, embeddings are hidden rows) */
    int ple_dim;           /* per-layer embedding width (512); 0 = no PLE */
    int out_dim;           /* embed_proj output width (768); 0 = no embed_proj */
    int window;            /* sliding layers keep keys with |i-j| <= window (512); 0 = no window */
    int full_period;       /* layer l is a full-attention layer when l % full_period == full_period-1
                            * (6: layers 5, 11, 17, 23, text.c:267); 0 = none */
    int full_head_dim, full_kv; /* head_dim and kv heads of the full layers (512, 1) */
    float rope_theta_full; /* RoPE theta of the full layers (1e6); the others use rope_theta */
    float ple_scale;       /* 1/sqrt(hidden) */
    const int8_t *wple_model;   /* [n_layers*ple_dim][hidden] */
    const float *sple_model;
    const float *ple_proj_norm; /* [ple_dim] */
    const int8_t *wembed_proj;  /* [out_dim][hidden] */
    const float *sembed_proj;
    /* with attn_i8: the fewest keys that take the int8 attention (dispatch.c:46-52 rule's gate:
     * 128 on the reference's CPU backends); 0 = only the blocked path's own 32 (an override) */
    int i8_min_keys;
} or_model;

/* Geometry of layer l: head_dim, kv heads, RoPE theta and window (0 = none) (text.c:467-478). */
void or_layer_geom(const or_model *m, int l, int *head_dim, int *kv, float *theta, int *window);

/* One layer over B x S rows, x updated in place (text.c:939-961): attention and FFN sublayers,
 * then, with PLE, the PLE block on this layer's slice of `ple` ([B*S][n_layers*ple_dim], from
 * or_ple_inputs; NULL without PLE) and the layer scale. */
int or_layer_forward(const or_model *m, int l, float *x, int B, int S, const uint8_t *valid,
                     int nthreads);
int or_layer_forward_ple(const or_model *m, int l, float *x, const float *ple, int B, int S,
                         const uint8_t *valid, int nthreads);
/* The per-layer inputs (text.c:929-932): ple = rms(int8 GEMM(quant(x), ple_model) * ple_scale)
 * * ple_proj_norm per ple_dim slice; x = the scaled embeddings [rows][hidden]. */
int or_ple_inputs(const or_model *m, const float *x, int rows, float *ple, int nthreads);
/* Attention sublayer only: x [B*S][hidden] -> out = O-proj of the context. */
int or_attention_sublayer(const or_model *m, int l, const float *x, int B, int S,
                          const uint8_t *valid, float *out, int nthreads);
/* FFN sublayer: x -> norm_split -> gate|up -> GeGLU -> down -> norm_add. */
int or_ffn_sublayer(const or_model *m, int l, float *x, int rows, int nthreads);
/* The whole encoder: ids [B][S] -> out [B][out_dim or hidden] (text.c:924-984). */
int or_encode(const or_model *m, const int32_t *ids, const uint8_t *valid, int B, int S,
              float *out, int nthreads);

#ifdef __cplusplus
}
#endif
#endif /* E2_ORACLE_H */
