/* ref_text.c — TEST INFRASTRUCTURE: drives the reference's own text tower (text.c, compiled from
 * /root/reference/src by oracle/Makefile into _ref/libreftext.so) on a model built in memory from
 * an E8CQ cache, so that the reference's CPU path can be timed and compared without its bf16
 * safetensors checkpoint.
 *
 * The reference builds its model in e2_load (e2.c:254-434): text tower, then the vision and audio
 * towers, all from one checkpoint. This harness does the text part of that, with the reference's
 * own pieces: the int8 weights come from the cache through the reference's reader (q8c_get_q8w,
 * q8cache.c:357-385, the same borrowed e2_q8w the loader assigns), layer types and RoPE tables
 * from e2_text_init (text.c:1033-1036), the workspace from e2_ws_alloc (e2.c:188-203), the worker
 * pool from e2_pool_global_init (threads.c:261). The token table and the norm scales are kept in
 * bf16 and f32 by the reference (e2.c:311-323, 356-375); the cache written by this repository's
 * e2_save_e8cq holds them in f32, so the table is rounded to bf16 here (round to nearest even)
 * and the norms are copied. The geometry is the reference checkpoint's (hidden 512, PLE, windowed
 * layers, head_dim 512 on layers 5/11/17/23): text.c hard-wires it, so only a model of that
 * geometry can run here; n_layers may be below 24 (text_forward walks m->n_layers).
 *
 * Not part of the product: only tests/ and bench.py's CPU-baseline leg load it. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "dispatch.h"
#include "model.h"
#include "q8cache.h"
#include "threads.h"

int e2_text_init(e2_model *m);
int e2_ws_alloc(e2_model *m, int max_seq, int max_patches);

static e2_model *g_m;
static uint16_t *g_table;
static char g_err[512];

const char *rt_error(void) { return g_err[0] ? g_err : e2_last_error(); }

static int fail(const char *what) {
    snprintf(g_err, sizeof g_err, "%s: %s", what, q8c_error());
    return -1;
}

/* f32 [n] from the cache (kind F32) into a fresh allocation */
static float *get_f32(const char *name, int64_t n) {
    size_t nb = 0;
    const int64_t d[1] = { n };
    const float *p = q8c_get(name, Q8C_F32, 1, d, &nb);
    if (!p || nb != (size_t)n * 4) return NULL;
    float *o = malloc((size_t)n * 4);
    if (o) memcpy(o, p, (size_t)n * 4);
    return o;
}

static uint16_t bf16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t)(u >> 16);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

void rt_close(void) {
    if (!g_m) return;
    e2_model *m = g_m;
    for (int l = 0; l < m->n_layers; l++) {
        e2_layer *L = &m->layers[l];
        free(L->q_norm); free(L->k_norm); free(L->input_ln); free(L->post_attn_ln);
        free(L->pre_ffn_ln); free(L->post_ffn_ln); free(L->ple_norm);
    }
    free(m->ple_proj_norm);
    free(m->final_norm);
    for (int t = 0; t < 2; t++) { free(m->rope_cos[t]); free(m->rope_sin[t]); }
    free(m->ws.x);
    free(m);
    free(g_table);
    g_m = NULL;
    g_table = NULL;
    q8c_read_close();
    e2_pool_global_free();
}

/* Build the text tower from `path` (an E8CQ cache of the reference geometry, `vocab` rows of the
 * token table, `n_layers` layers) with `nthreads` workers (0: the reference's default). */
int rt_open(const char *path, int n_layers, int vocab, int nthreads) {
    g_err[0] = 0;
    rt_close();
    if (n_layers <= 0 || n_layers > E2_MAX_LAYERS || vocab <= 0 || vocab > E2_VOCAB) {
        snprintf(g_err, sizeof g_err, "rt_open: bad n_layers %d or vocab %d", n_layers, vocab);
        return -1;
    }
    e2_cpu_init();
    if (q8c_read_open(path)) return fail("open cache");
    e2_model *m = calloc(1, sizeof *m);
    if (!m) return fail("oom");
    g_m = m;
    m->st.fd = -1;
    m->wdtype = E2_DT_BF16;
    m->use_int8 = 1;
    /* e2.c:303-310 */
    m->hidden = 512;
    m->intermediate = 2048;
    m->ple_dim = 512;
    m->rms_eps = 1e-6f;
    m->embed_scale = sqrtf((float)m->hidden);
    m->ple_scale = 1.0f / sqrtf((float)m->hidden);
    m->rope_theta_full = 1000000.0f;
    m->rope_theta_sliding = 10000.0f;
    m->n_layers = n_layers;
    if (e2_text_init(m)) { snprintf(g_err, sizeof g_err, "e2_text_init: %s", e2_last_error()); return -1; }

    /* the token table: the reference's loader checks E2_VOCAB rows (e2.c:317); rows past the
     * cache's vocabulary are zero (the caller keeps its ids below `vocab`) */
    size_t nb = 0;
    const int64_t dv[2] = { vocab, m->hidden };
    const float *tab = q8c_get("language_model.embed_tokens.weight", Q8C_F32, 2, dv, &nb);
    if (!tab || nb != (size_t)vocab * m->hidden * 4) return fail("token table");
    g_table = calloc((size_t)E2_VOCAB * m->hidden, 2);
    if (!g_table) return fail("oom table");
    for (size_t i = 0; i < (size_t)vocab * m->hidden; i++) g_table[i] = bf16_rne(tab[i]);
    m->embed_tokens = g_table;

    if (q8c_get_q8w("language_model.ple.per_layer_model_projection.weight", &m->q8_ple_model) ||
        q8c_get_q8w("language_model.embedding_projection.weight", &m->q8_embed_proj))
        return fail("ple/embed_proj weights");
    m->ple_proj_norm = get_f32("language_model.ple.per_layer_projection_norm.weight", m->ple_dim);
    m->final_norm = get_f32("language_model.norm.weight", m->hidden);
    if (!m->ple_proj_norm || !m->final_norm) return fail("norms");

    static const char *q8s[9] = { "self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
                                  "self_attn.o_proj.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight",
                                  "mlp.down_proj.weight", "ple_block.per_layer_input_gate.weight",
                                  "ple_block.per_layer_projection.weight" };
    static const char *ns[5] = { "input_layernorm.weight", "post_attention_layernorm.weight",
                                 "pre_feedforward_layernorm.weight", "post_feedforward_layernorm.weight",
                                 "ple_block.post_per_layer_input_norm.weight" };
    char name[192];
    for (int l = 0; l < n_layers; l++) {
        e2_layer *L = &m->layers[l];
        e2_q8w *dst[9] = { &L->q8_q, &L->q8_k, &L->q8_v, &L->q8_o, &L->q8_gate, &L->q8_up,
                           &L->q8_down, &L->q8_ple_gate, &L->q8_ple_proj };
        for (int s = 0; s < 9; s++) {
            snprintf(name, sizeof name, "language_model.layers.%d.%s", l, q8s[s]);
            if (q8c_get_q8w(name, dst[s])) return fail(name);
        }
        float **nd[5] = { &L->input_ln, &L->post_attn_ln, &L->pre_ffn_ln, &L->post_ffn_ln, &L->ple_norm };
        for (int s = 0; s < 5; s++) {
            snprintf(name, sizeof name, "language_model.layers.%d.%s", l, ns[s]);
            if (!(*nd[s] = get_f32(name, m->hidden))) return fail(name);
        }
        snprintf(name, sizeof name, "language_model.layers.%d.self_attn.q_norm.weight", l);
        L->q_norm = get_f32(name, L->head_dim);
        snprintf(name, sizeof name, "language_model.layers.%d.self_attn.k_norm.weight", l);
        L->k_norm = get_f32(name, L->head_dim);
        if (!L->q_norm || !L->k_norm) return fail("q/k norms");
        snprintf(name, sizeof name, "language_model.layers.%d.layer_scalar", l);
        const int64_t d1[1] = { 1 };
        const float *ls = q8c_get(name, Q8C_F32, 1, d1, NULL);
        if (!ls) return fail(name);
        L->layer_scalar = ls[0];
    }
    if (e2_pool_global_init(nthreads) <= 0) { snprintf(g_err, sizeof g_err, "worker pool: %s", e2_last_error()); return -1; }
    if (e2_ws_alloc(m, E2_MAX_SEQ, 0)) { snprintf(g_err, sizeof g_err, "workspace: %s", e2_last_error()); return -1; }
    return 0;
}

/* the reference's batch entry (text.c:997-1027) */
int rt_embed_batch(const int32_t *ids, const uint8_t *valid, int batch, int seq_len, float *out) {
    if (!g_m) { snprintf(g_err, sizeof g_err, "rt_embed_batch: no model"); return -1; }
    return e2_text_embed_batch(g_m, ids, valid, batch, seq_len, out);
}

/* Make layer l an identity: its O, down and PLE-projection outputs become zero (their per-row
 * weight scales are replaced by zeros), so the sublayers add rmsnorm(0) * gamma = 0, and the layer
 * scalar is 1. Lets a test reach one layer of the reference's recipe (e.g. the head_dim-512 layer 5)
 * without the layers before it. */
static float *g_zero;
int rt_identity_layer(int l) {
    if (!g_m || l < 0 || l >= g_m->n_layers) return -1;
    if (!g_zero && !(g_zero = calloc(4096, sizeof(float)))) return -1;
    e2_layer *L = &g_m->layers[l];
    L->q8_o.scale = L->q8_down.scale = L->q8_ple_proj.scale = g_zero;
    L->layer_scalar = 1.0f;
    return 0;
}

/* The reference's choice of text attention for S keys on this CPU (dispatch.c:180, its rule table
 * at dispatch.c:47-57): 1 = int8, 0 = f32. The blocked path also needs S >= 32 and every position
 * valid (text.c:873-876). */
int rt_attn_i8(int S) { return e2_attn_pick(e2_cpu_backend(), E2_TOWER_TEXT, S) == E2_ATTN_I8; }

/* Force the reference's text attention kind (e2_attn_override, dispatch.c:139-142): 0 f32, 2 int8,
 * -1 back to the rule table. */
void rt_attn_text(int kind) { e2_attn_override(E2_TOWER_TEXT, kind); }

/* The reference's model built by rt_open, for the reference-side adapter (e2hip_mi.c), which walks
 * it as e2_hip_create does. NULL before rt_open. */
e2_model *rt_model(void) { return g_m; }

int rt_threads(void) { return e2_nthreads(); }
const char *rt_cpu(void) { return e2_cpu_name(); }
