/* e2.h — the model container of the int8 encoder (host side).
 *
 * Mirrors the reference's include/e2.h handle (e2_model, e2_free, e2_last_error; e2.h:21-22,159)
 * for two geometries: the BASELINE one (hidden 768, every layer alike) and the reference
 * checkpoint's own (hidden 512, PLE, sliding window, per-layer head_dim, embed_proj; e2.c:254-434,
 * e2_config_reference below). A model here comes from
 *   - e2_model_synthetic: seeded random-init int8 weights at a given geometry,
 *   - e2_load_e8cq: an E8CQ packed int8 cache, the reference's q8cache.c v1 format (q8cache.c:1-13):
 *     header "E8CQ" v1, 16-byte aligned blobs, 152-byte index entries; int8 weights as kind 3
 *     (quad-interleaved w | per-row scale | per-block sums bsq), f32 tensors as kind 2.
 * Tensor names follow the reference's safetensors names (e2.c:306-402), e.g.
 * "language_model.layers.3.self_attn.q_proj.weight", "language_model.embed_tokens.weight".
 *
 * Weights are held in the reference's e2_q8w layout (int8.h:14-36): [Npad/8][K/4][8][4] int8,
 * per-row f32 scale, bsq[nb][Npad]. The GPU engine (e2mi.h) re-lays them out on upload.
 */
#ifndef E2_H
#define E2_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The reference's handle name over this repository's own model struct (tag e2mi_model, the one
 * include/e2mi.h names): the reference's struct e2_model (src/model.h:113) is a different layout,
 * and the engine's entry points take e2mi_model, so a reference model cannot be handed to them by
 * mistake. A caller holding the reference's model uses e2mi_create_tensors (e2mi.h). */
typedef struct e2mi_model e2_model;

typedef struct {
    int n_layers;      /* 24 */
    int hidden;        /* 768 */
    int ffn;           /* 1152 */
    int n_heads;       /* 3 query heads */
    int n_kv_heads;    /* 1 kv head (GQA 3:1) */
    int head_dim;      /* 256 */
    int vocab;         /* 262144 */
    int max_seq;       /* 2048 (model.h:16) */
    float rms_eps;     /* 1e-6 (e2.c:297) */
    float rope_theta;  /* 10000 */
    float embed_scale; /* sqrt(hidden) (e2.c:298) */
    float attn_scale;  /* 1.0: the reference does not scale the logits (text.c:8-9) */
    /* The reference checkpoint's extras (e2.c:294-301, text.c:467-478). Zeros give the BASELINE
     * geometry: every layer alike (head_dim, n_kv_heads, rope_theta), no window, no PLE, the
     * embeddings are the final-normed hidden rows. */
    int ple_dim;           /* per-layer embedding width: 512 (0 = no PLE) */
    int out_dim;           /* embed_proj output width: 768 (0 = no embed_proj) */
    int window;            /* sliding layers keep keys with |i-j| <= window: 512 (0 = no window) */
    int full_period;       /* layer l is a full-attention layer when l % full_period ==
                            * full_period - 1: 6, i.e. layers 5, 11, 17, 23 (text.c:267); 0 = none */
    int full_head_dim;     /* head_dim of the full-attention layers: 512 */
    int full_kv_heads;     /* kv heads of the full-attention layers: 1 */
    float rope_theta_full; /* RoPE theta of the full-attention layers: 1e6 */
    float ple_scale;       /* 1/sqrt(hidden) */
} e2_config;

/* The BASELINE config-4 geometry (values in the comments above, extras zero). */
void e2_config_baseline(e2_config *c);
/* The reference checkpoint's text-tower geometry (e2.c:294-301, model.h:12-16, text.c:467-478):
 * 24 layers, hidden 512, ffn 2048, 4 query heads; sliding layers head_dim 256 with 2 kv heads,
 * RoPE theta 1e4 and window 512; full layers (5, 11, 17, 23) head_dim 512 with 1 kv head, theta
 * 1e6; PLE 24 x 512 with ple_scale 1/sqrt(512); embed_scale sqrt(512); embed_proj 512 -> 768;
 * vocab 262144, max_seq 2048. Tensors beyond the BASELINE set (reference names, e2.c:316-381):
 *   language_model.ple.per_layer_model_projection.weight    int8 [n_layers*ple_dim][hidden]
 *   language_model.ple.per_layer_projection_norm.weight     f32 [ple_dim]
 *   language_model.embedding_projection.weight              int8 [out_dim][hidden]
 *   language_model.layers.L.ple_block.per_layer_input_gate.weight       int8 [ple_dim][hidden]
 *   language_model.layers.L.ple_block.per_layer_projection.weight       int8 [hidden][ple_dim]
 *   language_model.layers.L.ple_block.post_per_layer_input_norm.weight  f32 [hidden]
 *   language_model.layers.L.layer_scalar                                 f32 [1] */
void e2_config_reference(e2_config *c);

/* Random-init model: int8 weights uniform in [-127,127] with per-row scales U(0.001, 0.02), norm
 * gammas ~N(1, 0.05), embedding table ~N(0, 0.02). Deterministic in `seed` (the reference tests'
 * LCG s = s*1664525 + 1013904223, one stream per tensor row). NULL on error. */
e2_model *e2_model_synthetic(const e2_config *c, uint64_t seed);

/* Load an E8CQ cache written by e2_save_e8cq or by the reference's q8c writer (q8cache.c:61-222).
 * The file is validated before any pointer into it is used (q8cache.c:242-280) and memory-mapped;
 * int8 blobs are borrowed from the mapping, which lives until e2_free. NULL on error. */
e2_model *e2_load_e8cq(const char *path, const e2_config *c);
/* Write the model as an E8CQ cache (atomic: temp file + rename, q8cache.c:183-222). */
int e2_save_e8cq(const e2_model *m, const char *path);

/* Releases the model and the GPU engine e2_text_embed* created for it. */
void e2_free(e2_model *m);

/* Text: token ids -> embedding unit vector (include/e2.h:25); e2_text_embed_batch with one
 * all-valid sequence. */
int e2_text_embed(e2_model *m, const int32_t *ids, int n_ids, float *out768);
/* Batch (include/e2.h:35-36): ids/valid row-major [batch, seq_len], out [batch, 768]; valid may be
 * NULL (all valid), any nonzero byte keeps the token; seq_len 1..max_seq, batch > 0; every id,
 * masked or not, inside the vocabulary; all-invalid sequences give an exact zero vector. Returns 0,
 * or -1 without writing out when the input is invalid (e2_last_error). The reference runs this on
 * its CPU backends; here the first call creates the model's gfx950 engine (e2mi.h, e2mi_create),
 * which the model owns until e2_free. Not reentrant, like the reference. */
int e2_text_embed_batch(e2_model *m, const int32_t *ids, const uint8_t *valid, int batch, int seq_len,
                        float *out);

/* Last error of this process (e2.h:159). Never NULL. */
const char *e2_last_error(void);

int e2_model_config(const e2_model *m, e2_config *out);

/* A read-only view of one tensor. kind: 2 = f32 (data), 3 = int8 weight (data = packed w,
 * scale, bsq; dims = {N, K, nblocks, Npad}). */
typedef struct {
    int kind, ndim;
    int64_t dims[4];
    const void *data;
    const float *scale;
    const int32_t *bsq;
    size_t nbytes;
} e2_tensor_view;
int e2_model_tensor(const e2_model *m, const char *name, e2_tensor_view *out);

#ifdef __cplusplus
}
#endif
#endif /* E2_H */
