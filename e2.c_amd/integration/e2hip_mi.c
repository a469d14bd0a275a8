/* e2hip_mi.c — the reference-side adapter that binds Damix48/e2.c's loaded model to the gfx950
 * engine, in place of e2_hip_create(e2_model *m) (include/e2hip.h:31-35, src/gpu/hip/hip.c:112-167).
 *
 * This file is compiled INSIDE the reference's source tree (it includes the reference's internal
 * model.h, src/model.h:60-126, like src/gpu/hip/forward.c does) and links lib/libe2mi_backend.so,
 * which exports only e2mi_* names, so nothing clashes with the reference's own e2_* symbols. It does
 * what the reference's HIP create does with the model (forward.c:121-183: every m->layers[l].q8_*
 * uploaded as it is): it lists the text tower's tensors under their checkpoint names
 * (e2.c:306-402) with pointers into the live model, and e2mi_create_tensors uploads them. The engine
 * copies everything it needs, so unlike e2_hip_create the model need not outlive the engine.
 *
 * Build (from the reference's root; what a CMake option would add):
 *   cc -O2 -std=gnu11 -Isrc -Iinclude -I<this repository>/include -c e2hip_mi.c
 *   ... -L<this repository>/e2.c_amd/lib -le2mi_backend
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "model.h" /* the reference's e2_model, e2_layer, e2_q8w, E2_VOCAB */
#include "e2mi.h"  /* the engine's C ABI (this repository's include/e2mi.h) */

e2mi_engine *e2_hip_mi_create(e2_model *m);

/* The adapter's own last message (the engine's messages come from e2mi_last_error). */
static char g_adapter_err[256];
const char *e2_hip_mi_last_error(void) { return g_adapter_err[0] ? g_adapter_err : e2mi_last_error(); }

#define NAME_CAP 112 /* "language_model.layers.23.ple_block.post_per_layer_input_norm.weight" fits */

typedef struct {
    e2mi_tensor *t;
    char *names;
    int n, cap;
} tensor_list;

static e2mi_tensor *push(tensor_list *L, int kind, const char *fmt, int layer) {
    if (L->n == L->cap) return NULL;
    char *name = L->names + (size_t)L->n * NAME_CAP;
    if (layer >= 0) snprintf(name, NAME_CAP, "language_model.layers.%d.%s", layer, fmt);
    else snprintf(name, NAME_CAP, "%s", fmt);
    e2mi_tensor *t = &L->t[L->n++];
    memset(t, 0, sizeof *t);
    t->name = name;
    t->kind = kind;
    return t;
}

/* an e2_q8w exactly as the reference holds it: quad-interleaved bytes, per-row scales */
static int add_q8(tensor_list *L, const e2_q8w *q, const char *suffix, int layer) {
    e2mi_tensor *t = push(L, E2MI_TENSOR_Q8W, suffix, layer);
    if (!t || !q->w || !q->scale) return -1;
    t->N = q->N;
    t->K = q->K;
    t->nblocks = q->nblocks;
    t->Npad = q->Npad;
    t->data = q->w;
    t->scale = q->scale;
    t->bsq = q->bsq;
    return 0;
}

/* an f32 vector: a norm's scales (e2.c:356-375 converts them once to f32) or the layer scalar */
static int add_f32(tensor_list *L, const float *p, int n, const char *suffix, int layer) {
    e2mi_tensor *t = push(L, E2MI_TENSOR_F32, suffix, layer);
    if (!t || !p) return -1;
    t->N = 1;
    t->K = n;
    t->data = p;
    return 0;
}

e2mi_engine *e2_hip_mi_create(e2_model *m) {
    g_adapter_err[0] = 0;
    if (!m) {
        snprintf(g_adapter_err, sizeof g_adapter_err, "model is NULL");
        return NULL;
    }
    /* the same refusal as e2_hip_create (hip.c:150-153): the engine runs the int8 recipe */
    if (!m->use_int8) {
        snprintf(g_adapter_err, sizeof g_adapter_err,
                 "the gfx950 backend needs the int8 weights (E2_INT8=0 disables them)");
        return NULL;
    }
    tensor_list L = {0};
    L.cap = m->n_layers * 17 + 5;
    L.t = calloc((size_t)L.cap, sizeof *L.t);
    L.names = calloc((size_t)L.cap, NAME_CAP);
    if (!L.t || !L.names) {
        free(L.t);
        free(L.names);
        snprintf(g_adapter_err, sizeof g_adapter_err, "oom for the tensor list");
        return NULL;
    }
    int bad = 0;
    /* the token table stays bf16 [E2_VOCAB][hidden] (e2.c:311-317); the engine widens it */
    e2mi_tensor *tab = push(&L, E2MI_TENSOR_BF16, "language_model.embed_tokens.weight", -1);
    if (tab && m->embed_tokens) {
        tab->N = E2_VOCAB;
        tab->K = m->hidden;
        tab->data = m->embed_tokens;
    } else {
        bad = 1;
    }
    bad |= add_f32(&L, m->final_norm, m->hidden, "language_model.norm.weight", -1);
    bad |= add_q8(&L, &m->q8_ple_model, "language_model.ple.per_layer_model_projection.weight", -1);
    bad |= add_f32(&L, m->ple_proj_norm, m->ple_dim, "language_model.ple.per_layer_projection_norm.weight", -1);
    bad |= add_q8(&L, &m->q8_embed_proj, "language_model.embedding_projection.weight", -1);
    for (int l = 0; l < m->n_layers && !bad; l++) {
        const e2_layer *ly = &m->layers[l];
        bad |= add_q8(&L, &ly->q8_q, "self_attn.q_proj.weight", l);
        bad |= add_q8(&L, &ly->q8_k, "self_attn.k_proj.weight", l);
        bad |= add_q8(&L, &ly->q8_v, "self_attn.v_proj.weight", l);
        bad |= add_q8(&L, &ly->q8_o, "self_attn.o_proj.weight", l);
        bad |= add_q8(&L, &ly->q8_gate, "mlp.gate_proj.weight", l);
        bad |= add_q8(&L, &ly->q8_up, "mlp.up_proj.weight", l);
        bad |= add_q8(&L, &ly->q8_down, "mlp.down_proj.weight", l);
        bad |= add_q8(&L, &ly->q8_ple_gate, "ple_block.per_layer_input_gate.weight", l);
        bad |= add_q8(&L, &ly->q8_ple_proj, "ple_block.per_layer_projection.weight", l);
        bad |= add_f32(&L, ly->input_ln, m->hidden, "input_layernorm.weight", l);
        bad |= add_f32(&L, ly->post_attn_ln, m->hidden, "post_attention_layernorm.weight", l);
        bad |= add_f32(&L, ly->pre_ffn_ln, m->hidden, "pre_feedforward_layernorm.weight", l);
        bad |= add_f32(&L, ly->post_ffn_ln, m->hidden, "post_feedforward_layernorm.weight", l);
        bad |= add_f32(&L, ly->q_norm, ly->head_dim, "self_attn.q_norm.weight", l);
        bad |= add_f32(&L, ly->k_norm, ly->head_dim, "self_attn.k_norm.weight", l);
        bad |= add_f32(&L, ly->ple_norm, m->hidden, "ple_block.post_per_layer_input_norm.weight", l);
        bad |= add_f32(&L, &ly->layer_scalar, 1, "layer_scalar", l);
    }
    e2mi_engine *g = NULL;
    if (bad) {
        snprintf(g_adapter_err, sizeof g_adapter_err, "the model lacks a text-tower tensor (tensor %d)", L.n);
    } else {
        /* geometry 1: the reference checkpoint's text tower (text.c hard-wires it: hidden 512,
         * PLE, window 512, head_dim 512 on layers 5/11/17/23, embed_proj to 768) */
        g = e2mi_create_tensors(L.t, L.n, 1, m->n_layers, E2_VOCAB, 0);
    }
    free(L.t);
    free(L.names);
    return g;
}
