/* e2mi.h — the gfx950 (MI355X) int8 encoder backend: a C ABI over hand-written HIP kernels.
 *
 * The device sibling of the reference's include/e2hip.h (Damix48/e2.c): the same int8 recipe
 * (per-output-row int8 weights with f32 scales, per-(token, 128-element block) dynamic activation
 * scales, exact int32 accumulation, per-block f32 fold), rebuilt for CDNA4 int8 MFMA. Paths in the
 * citations below are relative to the reference's root.
 *
 * Conventions (all entry points):
 *   - return 0 on success, -1 on error with a message in e2mi_last_error() (hip.c:27-49);
 *   - arguments are validated before anything is launched or written (hip.c:287-342);
 *   - kernel-level entry points take DEVICE pointers and enqueue on `stream` (a hipStream_t, NULL
 *     for the default stream); they do not synchronise;
 *   - int8 activations are SIGNED (e2hip.h:19-21): the CPU reference's biased byte is
 *     (uint8_t)(q ^ 0x80);
 *   - activation scales use the reference's [M][K/128] layout (int8.h:94-97, a_scales[m*nb + b]).
 */
#ifndef E2MI_H
#define E2MI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *e2mi_stream; /* hipStream_t */

/* Device-resident int8 weight: the reference's e2_q8w (int8.h:79-92) re-laid out for MFMA.
 * w is row-major [N][ld] (K contiguous, ld % 16 == 0), scale is [N], bias [N] or NULL.
 * out_min/out_max: optional output saturation (int8.h:85-88); +-1e31 means none. */
typedef struct {
    int8_t *w;
    float *scale;
    float *bias;
    int N, K, ld;
    float out_min, out_max;
} e2mi_q8w;

/* Last error of this process (e2hip.h:64 e2_hip_last_error). Never NULL. */
const char *e2mi_last_error(void);

/* Name, compute-unit count and peak clock of device `dev` (e2hip.h:39 e2_hip_device). */
int e2mi_device_info(int dev, char *name, int cap, int *cus, int *clock_khz);

/* ---- weights: the reference's load-time path (e2.c:393-414, q8cache.c:357-385) */

/* Upload a reference-packed weight (quad-interleaved [Npad/8][K/4][8][4] int8 plus per-row scales,
 * int8.h:14-22) and re-lay it out on the device. bias may be NULL. The bsq block sums of the CPU
 * format are not needed: the device path multiplies signed bytes directly. */
int e2mi_q8w_upload_packed(e2mi_q8w *out, const int8_t *wq, const float *scale, const float *bias,
                           int N, int K, e2mi_stream stream);
/* Upload a row-major [N][K] int8 weight. */
int e2mi_q8w_upload_rowmajor(e2mi_q8w *out, const int8_t *w, const float *scale, const float *bias,
                             int N, int K, e2mi_stream stream);
void e2mi_q8w_free(e2mi_q8w *w);

/* ---- kernels (device pointers) */

/* Per-(row, block) activation quantizer: replaces e2_i8_quantize (kernels.h:70-72;
 * kernels_i8_avx512_vnni.c:312-366). block = 128 (the reference default) or K (per-token).
 * x [M][ldx] f32 -> q [M][K] int8 (row pitch K), scales [M][K/block]. K % 128 == 0. */
int e2mi_quantize(e2mi_stream stream, int8_t *q, float *scales, const float *x, int M, int K,
                  int ldx, int block);

/* W8A8 GEMM with fused dequant: replaces e2_i8_gemm (int8.h:94-97, kernels.h:69):
 * y[m][n] for n in [n0, n1) = sum_b fma(acc_b, as[m,b]*ws[n], .) (+bias[n]), clamped to the
 * weight's [out_min, out_max]; y row pitch ldy (columns are absolute, as in the reference). */
int e2mi_i8_gemm(e2mi_stream stream, float *y, int ldy, const int8_t *qa, const float *a_scales,
                 const e2mi_q8w *w, int M, int n0, int n1);

/* Same GEMM, also writing every block's exact int32 accumulator to acc [K/128][M][n1-n0]
 * (the parity hook for "bit-exact int32 accumulators"). */
int e2mi_i8_gemm_acc(e2mi_stream stream, float *y, int ldy, int32_t *acc, const int8_t *qa,
                     const float *a_scales, const e2mi_q8w *w, int M, int n0, int n1);

/* The reference checkpoint's PLE gate (text.c:906-913: gemm into gate, gate_quant with the layer's
 * per-layer-input slice as `up`): g = gelu_tanh(qa . W) * mul[m][n], quantized per (row, 128
 * columns) into yq [M][N] / ys [M][N/128] for the PLE projection GEMM; g [M][N] f32 also written
 * when non-NULL. mul [M][ldmul] (the slice of [rows][n_layers * ple_dim] at column l * ple_dim),
 * N % 128 == 0, 16-byte aligned rows. GELU within the reference's bar (test_gpu_ffn.c:104). */
int e2mi_i8_gemm_gelu_mul(e2mi_stream stream, int8_t *yq, float *ys, float *g, const int8_t *qa,
                          const float *a_scales, const e2mi_q8w *w, int M, const float *mul,
                          int ldmul);

/* GEMM whose epilogue requantizes the output per (row, 128 columns) for the next GEMM instead of
 * writing f32: the quantization the reference runs on y (text.c:321-339), fused. N % 128 == 0.
 * yq [M][N] int8, ys [M][N/128]. */
int e2mi_i8_gemm_q(e2mi_stream stream, int8_t *yq, float *ys, const int8_t *qa,
                   const float *a_scales, const e2mi_q8w *w, int M);

/* The same two GEMMs for per-token activation scales: a_scales is [M] (one scale per row, the
 * reference's int8 path built with a single block per row, int8.h:61-70 E2_I8_BLOCK = K; the
 * activations come from e2mi_quantize with block = K). The int32 accumulators run over the whole
 * K and are folded once: y = fma((float)acc, RN(as[m]*ws[n]), 0) (+bias), clamped. _tok_q
 * requantizes the output per (row, 128 columns) like e2mi_i8_gemm_q. */
int e2mi_i8_gemm_tok(e2mi_stream stream, float *y, int ldy, const int8_t *qa, const float *a_scales,
                     const e2mi_q8w *w, int M, int n0, int n1);
int e2mi_i8_gemm_tok_q(e2mi_stream stream, int8_t *yq, float *ys, const int8_t *qa,
                       const float *a_scales, const e2mi_q8w *w, int M);

/* gate|up GEMM with the GeGLU product and its quantization fused in the epilogue (text.c:424-468
 * gate_quant, fused into the producing GEMM). w holds 2*F rows interleaved per 64 as
 * [32 gate rows | 32 up rows] (see e2mi_interleave_gate_up). Writes q [M][F] int8, qs [M][F/128]
 * and, when g != NULL, the f32 product g [M][F] (the reference writes it back into gate). */
int e2mi_i8_gemm_geglu(e2mi_stream stream, int8_t *q, float *qs, float *g, const int8_t *qa,
                       const float *a_scales, const e2mi_q8w *w_gate_up, int M);

/* The q|k|v projection with the attention's row stage in its epilogue: the reference runs
 * e2_i8_gemm for q|k|v, then the q/k/v RMSNorm and RoPE over the f32 result (text.c:836-854); this
 * computes the same per 128 x 256 tile (one head) without the f32 round trip: per head of 256,
 * rmsnorm (q/k times their gamma, v without), rotate-half RoPE on q and k, f16 q16 [M][H*256],
 * k16 [M][KV*256] and V^T vt16 [M/S][KV][256][S], optional f32 copies q32/k32 (same layouts) and
 * v32 [M][KV*256]: the outputs of e2mi_i8_gemm followed by e2mi_qkv_norm_rope (pos == NULL:
 * positions m % S, M a multiple of S) or e2mi_qkv_norm_rope_packed (pos != NULL: S must be M).
 * The row sums of squares are added in another order than the row kernel's, so an output can
 * differ from that pair's by one f16 (f32) rounding step. head_dim 256 only, no bias or clamp.
 * w_qkv holds the q|k|v rows [(H+2KV)*256][K] with the rows of every 256-row head in rotate-half
 * pair order: bits 6 and 7 of the row index swapped (the epilogue then finds RoPE partners i and
 * i + 128 in one lane); its scales permuted alike. */
int e2mi_i8_gemm_qkv(e2mi_stream stream, const int8_t *qa, const float *a_scales,
                     const e2mi_q8w *w_qkv, int M, int S, const int32_t *pos, int H, int KV,
                     const float *q_gamma, const float *k_gamma, float eps, const float *cos_tab,
                     const float *sin_tab, uint16_t *q16, uint16_t *k16, uint16_t *vt16, float *q32,
                     float *k32, float *v32);

/* Fold order of every GEMM above (process-wide; no counterpart in the reference, which has one):
 *   0 (default) the reference's per-block f = fma((float)acc_b, RN(as[m,b]*ws[n]), f), bit-exact;
 *   1 f = fma((float)acc_b, as[m,b], f) per block and one multiply by ws[n] at the end: two VALU
 *     operations per element and block instead of three, int32 accumulators still exact, f32
 *     results within a few ulp (not bit-exact) of the reference's order.
 * The environment variable E2MI_GEMM_FOLD=fast sets 1 at load. Returns the previous mode, or -1
 * for a mode other than 0 or 1. Kernel-level entry points only; not safe against concurrent
 * launches from other threads. */
int e2mi_gemm_set_fold(int mode);

/* Host helper: interleave row-major gate [F][K] and up [F][K] int8 (and their scales) into the
 * [F/32][gate 32 | up 32] row order e2mi_i8_gemm_geglu consumes. F % 128 == 0. */
int e2mi_interleave_gate_up(int8_t *w_out, float *s_out, const int8_t *gate, const float *sgate,
                            const int8_t *up, const float *sup, int F, int K);

/* ---- memory-bound row kernels (D % 128 == 0, D <= 1280; rows are contiguous, ld = D) */

/* RMSNorm (kernels.c:76-87) then quantize: xn = x * (1/sqrt(mean(x^2) + eps)) * gamma, written to
 * xn_out (optional) and, when q != NULL, quantized per 128 into q [M][D] / qs [M][D/128]. */
int e2mi_norm_quant(e2mi_stream stream, const float *x, const float *gamma, float eps, int M, int D,
                    float *xn_out, int8_t *q, float *qs);

/* norm_add then norm_split then quantize, one pass per row (kernels.c:149-171, text.c:946-949):
 * x = rmsnorm(src)*gamma_add + res -> x_out (the new residual; may alias res); then, when
 * gamma_next != NULL, xn = rmsnorm(x)*gamma_next -> xn_out (optional) and q/qs (optional). */
int e2mi_add_norm_quant(e2mi_stream stream, const float *src, const float *res,
                        const float *gamma_add, const float *gamma_next, float eps, int M, int D,
                        float *x_out, float *xn_out, int8_t *q, float *qs);

/* A projection that feeds a norm_add, with the norm_add in its epilogue: y = e2mi_i8_gemm(qa, w)
 * (w: N = D = 768 or 512 rows, K a multiple of 128, no bias or clamp), then
 * e2mi_add_norm_quant(y, res, gamma_add, gamma_next, eps, M, D, x_out, xn_out, q, qs), with the same
 * bits as those two calls and without y in memory (the text tower's O and down projections and the
 * norm_add after each, text.c:944-953; the reference computes them as two passes, so this entry
 * point has no single counterpart). y [M][D] f32 is also written when non-NULL (parity tests).
 * x_out may alias res. */
int e2mi_i8_gemm_add_norm_quant(e2mi_stream stream, const int8_t *qa, const float *a_scales,
                                const e2mi_q8w *w, int M, const float *res, const float *gamma_add,
                                const float *gamma_next, float eps, float *x_out, float *xn_out,
                                int8_t *q, float *qs, float *y);

/* The same with e2mi_add_norm_scale_quant as the norm_add (the reference checkpoint's PLE layers,
 * text.c:955-961: x scaled by post_scale after the add; without gamma_next, x itself quantized into
 * q/qs): w must have N = 512 rows. */
int e2mi_i8_gemm_add_norm_scale_quant(e2mi_stream stream, const int8_t *qa, const float *a_scales,
                                      const e2mi_q8w *w, int M, const float *res, const float *gamma_add,
                                      float post_scale, const float *gamma_next, float eps, float *x_out,
                                      float *xn_out, int8_t *q, float *qs, float *y);

/* Embedding gather (text.c:917-921) fused with the first layer's norm_split + quantize:
 * x = table[ids[m]] * embed_scale -> x_out; rmsnorm(x)*gamma quantized into q/qs. Device-side ids
 * cannot be validated before launch: they are clamped into [0, vocab) to keep every read in the
 * table (the host entry points validate and reject, text.c:1008-1013). */
int e2mi_embed_norm_quant(e2mi_stream stream, const float *table, int vocab, const int32_t *ids,
                          float embed_scale, const float *gamma, float eps, int M, int D,
                          float *x_out, int8_t *q, float *qs);

/* q/k/v RMSNorm + rotate-half RoPE (text.c:836-838,853-854; kernels.c:112-126) on the QKV GEMM
 * output qkv [M][(H+2KV)*D] (q heads, k heads, v heads), M = B*S with positions m % S.
 * q, k get rmsnorm*gamma then RoPE from cos/sin tables [S][D]; v gets rmsnorm without gamma.
 * Writes f16: q16 [M][H*D], k16 [M][KV*D], vt16 [B][KV][D][S] (V transposed per sequence), and
 * optional f32 copies q32/k32 (same layouts) and v32 [M][KV*D]. head_dim D must be 256. */
int e2mi_qkv_norm_rope(e2mi_stream stream, const float *qkv, int M, int S, int H, int KV, int D,
                       const float *q_gamma, const float *k_gamma, float eps, const float *cos_tab,
                       const float *sin_tab, uint16_t *q16, uint16_t *k16, uint16_t *vt16,
                       float *q32, float *k32, float *v32);

/* The reference checkpoint's norm_add + layer_scalar (text.c:957-961: ple_block's map_norm_add,
 * then map_scale by layer_scalar) and the next operand, one pass per row:
 * x = (rmsnorm(src)*gamma_add + res) * post_scale -> x_out (may alias res); then, when gamma_next
 * != NULL, xn = rmsnorm(x)*gamma_next -> xn_out (optional) and q/qs (optional); when gamma_next is
 * NULL, q/qs (optional) quantize x itself per 128 (the PLE gate GEMM's operand, text.c:911). */
int e2mi_add_norm_scale_quant(e2mi_stream stream, const float *src, const float *res,
                              const float *gamma_add, float post_scale, const float *gamma_next,
                              float eps, int M, int D, float *x_out, float *xn_out, int8_t *q,
                              float *qs);
/* The per-layer embedding norm (text.c:930-931: map_scale by ple_scale, then map_norm per slice):
 * out = rmsnorm(x * pre_scale) * gamma over rows of D (out may alias x). */
int e2mi_scale_norm(e2mi_stream stream, const float *x, int rows, int D, float pre_scale,
                    const float *gamma, float eps, float *out);

/* Standalone GeGLU product + quantize (text.c:424-468 gate_quant): g = gelu_tanh(gate)*up per
 * element, quantized per 128 into q [M][D] / qs [M][D/128]; g written back into gate when
 * write_back != 0 (the reference overwrites gate). */
int e2mi_gelu_mul_quant(e2mi_stream stream, float *gate, int ldg, const float *up, int ldu, int M,
                        int D, int8_t *q, float *qs, int write_back);

/* Masked mean pool over each sequence's valid rows, then L2 normalisation (kernels.c:22-39,
 * text.c:963-981): x [B*S][D] -> out [B][D]; an all-invalid sequence gives an exact zero vector.
 * workspace: e2mi_pool_workspace_bytes(B, S, D) bytes of device memory. */
int e2mi_pool_l2(e2mi_stream stream, const float *x, const uint8_t *valid, int B, int S, int D,
                 float *workspace, float *out);
size_t e2mi_pool_workspace_bytes(int B, int S, int D);
/* e2mi_pool_l2 without a workspace argument and without allocating: the partial sums live in a
 * static device array of 8 MiB per GPU (held until the process ends), so
 * e2mi_pool_workspace_bytes(B, S, D) must be at most 8 MiB (e.g. 340 sequences of 512 at D = 768);
 * larger requests fail with -1. No counterpart in the reference: for callers that cannot allocate
 * (code under graph capture, serving loops, harnesses that forbid hipMalloc). All calls on one GPU
 * share the array: calls that overlap on one GPU race (serialise them on one stream). */
int e2mi_pool_l2_noalloc(e2mi_stream stream, const float *x, const uint8_t *valid, int B, int S, int D,
                         float *out);

/* Packed batches (no counterpart in the reference, which computes padding rows): the valid tokens
 * of B sequences laid out back to back, sequence b in rows [seq_start[b], seq_start[b] +
 * seq_len[b]). Row kernels and GEMMs are row-local and take the packed rows as they are; these
 * three take the per-row RoPE position or the per-sequence row ranges instead of a padded mask.
 * qkv_norm_rope_packed: as e2mi_qkv_norm_rope with positions pos [M] and V transposed over all
 * rows, vt16 [KV][D][M]. */
int e2mi_qkv_norm_rope_packed(e2mi_stream stream, const float *qkv, int M, const int32_t *pos,
                              int H, int KV, int D, const float *q_gamma, const float *k_gamma,
                              float eps, const float *cos_tab, const float *sin_tab, uint16_t *q16,
                              uint16_t *k16, uint16_t *vt16, float *q32, float *k32, float *v32);
/* (qkv_norm_rope_packed takes head_dim 256 or 512: the reference checkpoint's full-attention
 * layers have 512, text.c:476.) */
/* The engine's host-side plan of a packed batch, for callers that run the packed kernels with
 * their own forward (no reference counterpart: the reference computes every padded row,
 * text.c:1015-1024). e2mi_plan_pack: sequence b's valid tokens (valid [B][S], nonzero keeps a token,
 * NULL: all valid) in order in rows [start[b], start[b] + len[b]), each sequence starting on a
 * multiple of 8 rows, the total rounded up to 256; rowmap[r] = b * S + s of packed row r (-1 for a
 * filler row), pos[r] = s (0 for fillers). rowmap and pos hold B * ceil8(S) + 256 entries, start
 * and len B. Returns the packed row count M. */
int e2mi_plan_pack(const uint8_t *valid, int B, int S, int32_t *rowmap, int32_t *pos, int32_t *start,
                   int32_t *len);
/* The attention work list of packed sequences of lengths len[B] (the engine's own list): sequences
 * longest first, every head h < H, every 128-query block; with max_parts > 1 a block whose key
 * tiles of 32 (all of the sequence, or those within `window` of the block by packed index) number
 * n > 8 is split into min(max_parts, ceil(n / 8), n) parts and gets a merge entry (the lists of
 * e2mi_attention_packed_split; max_parts <= 4). The entries are dealt to the 8 XCDs: a sequence's
 * consecutive entries, cut into chunks of at most 1/div of an XCD's share of the key tiles, go to
 * the least-loaded XCD, and workgroup i of the grid runs on XCD i % 8 (the engine: div 2 at
 * head_dim 256, 4 at 512). work holds H * sum(ceil(len / 128)) * max_parts entries, merge (needed
 * when max_parts > 1) H * sum(ceil(len / 128)). Returns the number of work entries and sets
 * *n_merge (may be NULL when max_parts is 1). */
int e2mi_plan_attention(const int32_t *len, int B, int H, int window, int max_parts, int div,
                        int32_t *work, int32_t *merge, int *n_merge);
/* The same plan built on the device from a device mask, by one single-workgroup kernel on `stream`
 * (the engine's device entry plans this way; no counterpart in the reference, whose HIP path runs
 * padded batches): rowmap, pos, start and len as e2mi_plan_pack gives them, *rows its row count M,
 * and work as e2mi_plan_attention gives it unsplit (max_parts 1), followed by -1 up to n_slots
 * entries; with ids [B][S] (device) ids_out gets each packed row's token (0 for filler rows).
 * All pointers are device memory: rowmap, pos and ids_out of B * ceil8(S) + 256 entries, start and
 * len of B, work of n_slots, rows one int. Needs 0 < B <= 1024, 0 < S <= 16256, 0 < H < 16 and
 * H * (ceil(B * S / 128) + B) <= n_slots <= 8192. Returns 0, or -1 with the error set. */
int e2mi_plan_device(e2mi_stream stream, const uint8_t *valid, const int32_t *ids, int B, int S, int H,
                     int window, int div, int n_slots, int32_t *rowmap, int32_t *pos, int32_t *start,
                     int32_t *len, int32_t *ids_out, int32_t *work, int32_t *rows);
/* attention of each packed sequence over its own rows (all valid); vt16 [KV][D][M] from
 * e2mi_qkv_norm_rope_packed, seq_len[b] <= max_len, every seq_start a multiple of 8 (the
 * e2mi.pack_plan layout); rows outside every sequence are not written. work (optional, device):
 * n_work entries b | h << 16 | query_block << 24 (128 queries per block; b < 65536, the head in
 * 4 bits so H < 16 with a work list, query_block < 128), one workgroup each, in the order given
 * (longest sequences first balances the grid), negative entries idle; NULL runs a (query block,
 * head, sequence) grid over max_len. */
int e2mi_attention_packed(e2mi_stream stream, const uint16_t *q16, const uint16_t *k16,
                          const uint16_t *vt16, int M, const int32_t *seq_start,
                          const int32_t *seq_len, int B, int max_len, int H, int KV, int D,
                          float scale, int8_t *ctx_q, float *ctx_s, float *ctx32,
                          const int32_t *work, int n_work);
/* The same for the reference checkpoint's layers (text.c:467-478, 534-572): head_dim D = 256 or 512
 * and, when window > 0, the sliding window: query i reads key j only when |pos_i - pos_j| <= window
 * (text.c:542-546), pos [M] being each row's position in its padded sequence (the pos table of
 * e2mi_qkv_norm_rope_packed; NULL: the packed index). At D = 512 each work entry runs as one
 * 512-thread workgroup. Needs M even and vt16 4-byte aligned. */
int e2mi_attention_packed_window(e2mi_stream stream, const uint16_t *q16, const uint16_t *k16,
                                 const uint16_t *vt16, int M, const int32_t *seq_start,
                                 const int32_t *seq_len, const int32_t *pos, int B, int max_len,
                                 int H, int KV, int D, float scale, int window, int8_t *ctx_q,
                                 float *ctx_s, float *ctx32, const int32_t *work, int n_work);
/* The same with long query blocks' keys split over several workgroups (head_dim 256): the reference
 * walks a query block's keys in one sequence (text.c:702-741); here a work entry may carry a part p
 * of P <= 4 (entry = b | h << 16 | p << 20 | (P - 1) << 22 | query_block << 24, h < 16), each part
 * taking a consecutive share of the block's key tiles and leaving its context sum, row max and row
 * sum in part (e2mi_attention_part_bytes(part_rows, H, 256) bytes, part_rows >= M); then one
 * workgroup per merge entry (b | h << 16 | (P - 1) << 22 | query_block << 24, negative: idle)
 * combines the parts, ctx = sum_p 2^(m_p - M) o_p / sum_p 2^(m_p - M) l_p (m_p: row maxima of
 * scale * log2(e) * q.k), and quantizes ctx as the
 * unsplit kernel does. Entries with P = 1 run as in e2mi_attention_packed_window. Split and unsplit
 * results differ by the f16 rounding of the probabilities (each part's exponentials are taken
 * against its own running max) and the order of the sums. */
size_t e2mi_attention_part_bytes(int part_rows, int H, int D);
int e2mi_attention_packed_split(e2mi_stream stream, const uint16_t *q16, const uint16_t *k16,
                                const uint16_t *vt16, int M, const int32_t *seq_start,
                                const int32_t *seq_len, const int32_t *pos, int B, int max_len, int H,
                                int KV, int D, float scale, int window, int8_t *ctx_q, float *ctx_s,
                                float *ctx32, const int32_t *work, int n_work, const int32_t *merge,
                                int n_merge, float *part, int part_rows);
/* The reference's int8 attention (text.c:638-700 attb_i8; dispatch.c:51 selects it for long
 * sequences on AVX-512) for packed batches: q32 [M][H*D], k32/v32 [M][KV*D] f32 after q/k norm and
 * RoPE (e2mi_qkv_norm_rope_packed's optional f32 outputs), sequences as for
 * e2mi_attention_packed (every seq_start a multiple of 8, M a multiple of 16). Q is quantized per
 * (row, head, 128 dims), K per key row and V^T per (sequence, kv head, dim) with the reference's
 * quantizers, scores and context are int8 GEMMs folded per 128-block in the reference's order,
 * the probabilities are quantized per 128-key block. Outputs as e2mi_attention_packed (context
 * quantized per 128 dims for the O projection, optional f32 copy; work entries as there, H < 16).
 * workspace: device memory of e2mi_attention_i8_workspace_bytes(M, B, max_len, H, KV) bytes,
 * 256-byte aligned. */
size_t e2mi_attention_i8_workspace_bytes(int M, int B, int max_len, int H, int KV);
int e2mi_attention_i8_packed(e2mi_stream stream, const float *q32, const float *k32,
                             const float *v32, int M, const int32_t *seq_start,
                             const int32_t *seq_len, int B, int max_len, int H, int KV, int D,
                             void *workspace, int8_t *ctx_q, float *ctx_s, float *ctx32,
                             const int32_t *work, int n_work);
/* mean pool + L2 of each packed sequence's rows (workspace: e2mi_pool_workspace_bytes(B, max_len, D)) */
int e2mi_pool_l2_packed(e2mi_stream stream, const float *x, const int32_t *seq_start,
                        const int32_t *seq_len, int B, int max_len, int D, float *workspace,
                        float *out);
/* out[r] = rowmap[r] >= 0 ? ids[rowmap[r]] : 0 for r < M (the packed rows' token ids) */
int e2mi_gather_ids(e2mi_stream stream, const int32_t *ids, const int32_t *rowmap, int M,
                    int32_t *out);

/* ---- attention */

/* Fused bidirectional GQA attention (text.c:534-572,817-891): per sequence b, head h (kv head
 * h/(H/KV)), query i with valid[b*S+i]: ctx = softmax(scale * q.k_j over valid keys j) . v; an
 * invalid query row, or one with no valid key, gets ctx = 0. f16 inputs from e2mi_qkv_norm_rope,
 * f32 softmax and accumulation. The context is quantized per 128 dims into ctx_q [B*S][H*D] /
 * ctx_s [B*S][H*D/128] (the O-projection's operand); ctx32 (optional) receives it in f32.
 * head_dim D must be 256; scale finite and > 0 (every attention entry here). */
int e2mi_attention(e2mi_stream stream, const uint16_t *q16, const uint16_t *k16,
                   const uint16_t *vt16, const uint8_t *valid, int B, int S, int H, int KV, int D,
                   float scale, int8_t *ctx_q, float *ctx_s, float *ctx32);

/* ---- the encoder on the device (e2hip.h:34-64) */

/* This repository's model container (include/e2.h names it e2_model there). It is not the
 * reference's struct e2_model (src/model.h:113): a caller holding the reference's model hands its
 * tensors over with e2mi_create_tensors below. */
typedef struct e2mi_model e2mi_model;
typedef struct e2mi_engine e2mi_engine;

/* Upload the model (int8 weights re-laid out for MFMA, q|k|v concatenated, gate|up interleaved)
 * and allocate a workspace for 32768 token rows (e2_hip_create, hip.c:112-167). `m` may be freed
 * afterwards. NULL (and e2mi_last_error) when there is no gfx950 device or the model is invalid.
 * Exported by lib/libe2mi.so only (the backend library exports the two entries below instead). */
e2mi_engine *e2mi_create(const e2mi_model *m);
/* Same with an explicit workspace capacity in token rows (>= the model's max_seq). */
e2mi_engine *e2mi_create_rows(const e2mi_model *m, int max_rows);

/* One tensor of a model held in memory by the caller, under the reference's tensor name
 * (e2.c:306-402, e.g. "language_model.layers.3.self_attn.q_proj.weight"). kind:
 *   E2MI_TENSOR_Q8W  the reference's e2_q8w (int8.h:79-92) as it is: data = w, the quad-interleaved
 *                    [Npad/8][K/4][8][4] bytes (int8.h:14-22); scale = the per-row scales [Npad];
 *                    N, K, Npad (= N rounded up to 8) and nblocks its fields; bsq is not read (this
 *                    backend stores activations signed, so no weight-sum correction) and may be NULL;
 *   E2MI_TENSOR_F32  data = float[rows * cols] (norm scales, the layer scalar: rows = 1);
 *   E2MI_TENSOR_BF16 data = uint16 bf16[rows * cols] (the token table, e2.c:311-317).
 * For F32 and BF16, N = rows and K = cols. Same codes as the E8CQ kinds (q8cache.c:1-13). */
enum { E2MI_TENSOR_BF16 = 1, E2MI_TENSOR_F32 = 2, E2MI_TENSOR_Q8W = 3 };
typedef struct {
    const char *name;
    int kind;
    int N, K;
    int nblocks, Npad;
    const void *data;
    const float *scale;
    const int32_t *bsq;
} e2mi_tensor;

/* The engine from a model held in memory: e2_hip_create(e2_model *m) (e2hip.h:31-35, hip.c:112-167;
 * forward.c:121-183 uploads m->layers[l].q8_* as they are). The reference-side adapter
 * (e2.c_amd/integration/e2hip_mi.c) walks its e2_model and lists every text-tower tensor here by
 * name; the engine
 * uploads them and borrows nothing, so the arrays may be freed when the call returns (the
 * reference's create borrows `m` for the engine's life). geometry, n_layers, vocab and max_rows as
 * in e2mi_create_e8cq. Every tensor of the geometry must be present with its shape (names not
 * used by the text tower are ignored); NULL with e2mi_last_error otherwise, or when there is no
 * gfx950 device. */
e2mi_engine *e2mi_create_tensors(const e2mi_tensor *tensors, int n_tensors, int geometry, int n_layers,
                                 int vocab, int max_rows);
/* The engine straight from an E8CQ cache (q8cache.c:242-385 format), for a backend built into the
 * reference, whose own e2.h and library already define e2_model, e2_free and e2_last_error: with
 * lib/libe2mi_backend.so, which exports only the e2mi_* names, the caller needs nothing else.
 * geometry 0: BASELINE encoder (e2_config_baseline), 1: the reference checkpoint's (e2_config_
 * reference); n_layers and vocab > 0 override the preset's. Replaces e2_hip_create(e2_model *)
 * (e2hip.h:34) for callers that hold the cache path (E2_Q8_WRITE, e2.c:276-292). NULL with
 * e2mi_last_error when the file does not match the geometry or there is no gfx950 device. */
e2mi_engine *e2mi_create_e8cq(const char *path, int geometry, int n_layers, int vocab, int max_rows);
void e2mi_destroy(e2mi_engine *g);
/* Device name, architecture and CU count, for logging (e2_hip_device). */
const char *e2mi_device(e2mi_engine *g);

/* One sequence of n_ids tokens -> one unit vector (e2_hip_text_embed); its width is the model's
 * out_dim, or hidden when there is no embed_proj. */
int e2mi_text_embed(e2mi_engine *g, const int32_t *ids, int n_ids, float *out);
/* `batch` sequences of `seq_len` tokens, row-major; valid marks real tokens (NULL: all valid; any
 * nonzero byte keeps a row). Positions restart per sequence; all-invalid sequences give an exact
 * zero vector. Host buffers; the request is validated (ids in [0, vocab), 1 <= seq_len <=
 * max_seq) before anything is written, then processed in chunks of whole sequences. Synchronous.
 * (e2_hip_text_embed_batch, hip.c:308-342; e2_text_embed_batch, text.c:997-1027.) */
int e2mi_text_embed_batch(e2mi_engine *g, const int32_t *ids, const uint8_t *valid, int batch,
                          int seq_len, float *out);
/* The same forward with DEVICE buffers already resident in HBM: ids [batch*seq_len], valid
 * [batch*seq_len], out [batch][hidden]. Enqueued on `stream` (NULL: the engine's own stream, then
 * synchronised). Packed batches are planned on the device (e2mi_set_device_plan): nothing is read
 * back, so calls on a caller stream are enqueued back to back; where that planner does not apply
 * (a batch that could exceed the workspace, the int8 attention, split key ranges, E2MI_DUMP) the
 * mask is copied to the host (one synchronous copy of batch*seq_len bytes) to plan the packing,
 * and batches larger than the workspace run in chunks (a chunk with no valid token is filled with
 * zero vectors by a kernel, nothing else runs); unpacked, batch*seq_len must fit the workspace.
 * Ids are checked on the device, masked positions included (text.c:1008-1013 checks them on the
 * host): an id outside [0, vocab) makes the call return -1 with e2mi_last_error set, and the
 * embeddings it wrote are not valid. With a caller stream the call returns before its check has
 * run, so the check is reported by the first later call of the engine that finds it finished (a
 * call after the stream was synchronised, or any call on another stream or with NULL, always
 * does); that call returns -1 and does no work.
 * Calls on one engine are serialised: a call on a stream other than the previous call's first waits
 * for that stream (the calls share the workspace and the pinned staging arrays). */
int e2mi_text_embed_batch_device(e2mi_engine *g, const int32_t *ids, const uint8_t *valid,
                                 int batch, int seq_len, float *out, e2mi_stream stream);
/* Calls served, kernels launched by the last forward, wall time of the last call (e2_hip_stats). */
int e2mi_stats(e2mi_engine *g, long *calls, long *kernels_last, double *last_ms);
/* Diagnostics set by the environment at e2mi_create, as the reference's HIP backend reads
 * E2_HIP_PROFILE and E2_HIP_DUMP (src/gpu/hip/hip.c:51-108,121,138-139): E2MI_PROFILE=1 runs the
 * engine's first call without a graph, one event pair per launch, and reports per-stage times
 * (printed to stderr as e2h_prof_report prints them, hip.c:88-100); E2MI_DUMP=<dir> writes the
 * workspace of call number E2MI_DUMP_CALL (default 1; "all": after every call, overwriting; its
 * last chunk, its last layer: see
 * e2mi_set_layer_limit) to <dir>/e2mi_<name>.<f32|f16|i8|i32> (forward.c:725-759: x, xn, tmp, q16,
 * k16, vt16, ctx_q, ctx_s, out, and for packed batches pos and rowmap). e2mi_profile_text returns the
 * report of the profiled call ("" before it or without E2MI_PROFILE); the text lives as long as the
 * engine. No reference counterpart for the accessor (the reference only prints). */
const char *e2mi_profile_text(const e2mi_engine *g);
/* Split key ranges in the engine's attention (head_dim-256 layers; e2mi_attention_packed_split): a
 * 128-query block whose keys span more than 8 tiles of 32 is shared out over up to 4 workgroups and
 * merged. mode 0 never (the default), 1 always, 2 only for chunks whose unsplit blocks fill at most
 * half of the device's attention workgroups (few sequences: a single 2048-token document at the
 * reference geometry 5.77 -> 4.87 ms; a full config-4 batch would lose 14 %). E2MI_SPLIT=0|1|auto
 * sets it at creation. Split results differ from unsplit ones by f16 rounding, so under mode 2 a
 * long sequence's embedding depends on its batch-mates (alone it may split, in a full batch it does
 * not); modes 0 and 1 keep every sequence's embedding independent of the batch, as the reference's
 * CPU path is. No reference counterpart (the reference has no split). */
int e2mi_set_attention_split(e2mi_engine *g, int mode);
/* Run only the first n layers (0: all) before the final norm and pooling: the reference's
 * E2_HIP_LAYERS bisection knob (forward.c:359-366), for parity checks layer by layer. */
int e2mi_set_layer_limit(e2mi_engine *g, int n_layers);
/* Packed batches on (1, the default; E2MI_NOPACK=1 turns it off at creation) or off (0: every
 * row of the padded batch is computed, as the reference does). No counterpart in the reference. */
int e2mi_set_packing(e2mi_engine *g, int on);
/* Where the device entry plans a packed batch: 1 (the default) on the device (e2mi_plan_device's
 * kernel, whenever the whole batch fits the workspace at any mask, the plan fits the planner's
 * workgroup, and neither the int8 attention, split key ranges nor E2MI_DUMP is on): the call reads
 * nothing back and one recorded forward per (batch, seq_len) serves every mask, its kernels
 * reading the planned row count from device memory; 0 on the host, as e2mi_text_embed_batch does
 * (the mask read back, a forward recorded per packed row count). The embeddings are the same bit
 * for bit. E2MI_DEVICE_PLAN=0 sets 0 at creation. No counterpart in the reference. */
int e2mi_set_device_plan(e2mi_engine *g, int on);
/* Text attention kind (the reference's E2_ATTN_TEXT / e2_attn_override, dispatch.h:34-41, read at
 * e2mi_create): E2_ATTN_F16 (1, the gfx950 rule's choice) or E2_ATTN_I8 (2: sequences of at least 32
 * valid tokens take the int8 attention of text.c:638-700, shorter ones the f16 kernel, as the
 * reference's blocked path needs 32 rows, text.c:873-875). I8 needs packed batches (the padded
 * forward keeps f16) and the reference's attention scale 1.0; its buffers are allocated on first
 * use. */
int e2mi_set_attention(e2mi_engine *g, int kind);

#ifdef __cplusplus
}
#endif
#endif /* E2MI_H */
