/* e2_oracle_model.c — the text tower's layer recipe (test infrastructure).
 *
 * Restates text.c:924-984 (text_forward), text.c:817-891 (attention), text.c:893-903 (mlp) and
 * text.c:906-915 (ple_block). Per layer:
 *
 *   res = x; x = rms(x)*input_ln                       norm_split   text.c:942
 *   q|k|v = int8 GEMM(quant(x))                        gemm_segs    text.c:826-833
 *   q,k rms*gamma, v rms (no gamma)                    map_norm     text.c:836-838
 *   per sequence: trim trailing pad, RoPE, attention   text.c:840-887
 *     (sliding layers: keys with |i-j| <= window)      text.c:542-546
 *   tmp = int8 GEMM(quant(ctx), O)                     text.c:890
 *   x = rms(tmp)*post_attn_ln + res                    norm_add     text.c:946
 *   res = x; x = rms(x)*pre_ffn_ln                     norm_split   text.c:949
 *   g|u = int8 GEMM(quant(x)); quant(gelu(g)*u); down  mlp          text.c:893-903
 *   x = rms(tmp)*post_ffn_ln + res                     norm_add     text.c:953
 *   with PLE: g = int8 GEMM(quant(x), ple_gate); quant(gelu(g)*ple_l);
 *             tmp = int8 GEMM(., ple_proj); x = rms(tmp)*ple_norm + x       text.c:906-915,957
 *   x *= layer_scalar                                  map_scale    text.c:959
 *
 * with, before the layers, the PLE inputs ple = rms(GEMM(quant(x0), ple_model) * ple_scale) *
 * ple_proj_norm per slice (text.c:929-932), and after them rms(x)*final_norm, the embed_proj GEMM
 * (text.c:964-965), masked mean pool, L2 (text.c:966-981). Layer geometry (head_dim, kv heads,
 * RoPE theta, window) per layer type as text.c:467-478. Every GEMM runs on the threaded VNNI
 * kernel, which tests/test_oracle_ref.py pins bit-exact to the single-threaded restatement.
 */
#include "e2_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define OR_CHECK(p) do { if (!(p)) goto fail; } while (0)

void or_layer_geom(const or_model *m, int l, int *head_dim, int *kv, float *theta, int *window) {
    const int full = m->full_period > 0 && l % m->full_period == m->full_period - 1;
    *head_dim = full ? m->full_head_dim : m->head_dim;
    *kv = full ? m->full_kv : m->n_kv;
    *theta = full ? m->rope_theta_full : m->rope_theta;
    *window = full ? 0 : m->window;
}

int or_attention_sublayer(const or_model *m, int l, const float *x, int B, int S,
                          const uint8_t *valid, float *out, int nthreads) {
    const or_layer *L = &m->layers[l];
    int D, KV, window;
    float theta;
    or_layer_geom(m, l, &D, &KV, &theta, &window);
    const int M = B * S, Dm = m->hidden, H = m->n_heads;
    const int GD = H * D, NQKV = (H + 2 * KV) * D, nb = Dm / 128, nbg = GD / 128;
    int rc = -1;
    int8_t *qa = malloc((size_t)M * (Dm > GD ? Dm : GD));
    float *as = malloc(sizeof(float) * (size_t)M * (nb > nbg ? nb : nbg));
    float *qkv = malloc(sizeof(float) * (size_t)M * NQKV);
    float *q = malloc(sizeof(float) * (size_t)M * GD);
    float *k = malloc(sizeof(float) * (size_t)M * KV * D);
    float *v = malloc(sizeof(float) * (size_t)M * KV * D);
    float *ctx = calloc((size_t)M * GD, sizeof(float));
    float *cs = malloc(sizeof(float) * (size_t)S * D), *sn = malloc(sizeof(float) * (size_t)S * D);
    OR_CHECK(qa && as && qkv && q && k && v && ctx && cs && sn);

    or_quantize_mt(x, M, Dm, qa, as, nthreads);
    or_i8_gemm_mt(qa, as, L->wqkv, L->sqkv, NULL, M, NQKV, Dm, qkv, nthreads);
    for (int r = 0; r < M; r++) {
        memcpy(q + (size_t)r * GD, qkv + (size_t)r * NQKV, sizeof(float) * GD);
        memcpy(k + (size_t)r * KV * D, qkv + (size_t)r * NQKV + GD, sizeof(float) * KV * D);
        memcpy(v + (size_t)r * KV * D, qkv + (size_t)r * NQKV + GD + KV * D, sizeof(float) * KV * D);
    }
    or_rmsnorm(q, M * H, D, L->q_norm, m->eps);
    or_rmsnorm(k, M * KV, D, L->k_norm, m->eps);
    or_rmsnorm(v, M * KV, D, NULL, m->eps);
    or_rope_table(S, D, theta, cs, sn);
    for (int b = 0; b < B; b++) {
        const uint8_t *vb = valid + (size_t)b * S;
        int Sb = S;
        while (Sb && !vb[Sb - 1]) Sb--; /* trailing padding is trimmed: text.c:849-852 */
        if (!Sb) continue;
        or_rope_rows(q + (size_t)b * S * GD, Sb * H, H, D, cs, sn);
        or_rope_rows(k + (size_t)b * S * KV * D, Sb * KV, KV, D, cs, sn);
        int all = 1;
        for (int i = 0; i < Sb; i++) all &= vb[i] != 0;
        if (m->attn_i8 && all && Sb >= 32 && Sb >= m->i8_min_keys && m->attn_scale == 1.0f) {
            if (or_attention_i8_win(q + (size_t)b * S * GD, GD, k + (size_t)b * S * KV * D, KV * D,
                                    v + (size_t)b * S * KV * D, KV * D, Sb, H, KV, D, window,
                                    ctx + (size_t)b * S * GD, GD))
                goto fail;
        } else {
            or_attention_win(q + (size_t)b * S * GD, GD, k + (size_t)b * S * KV * D, KV * D,
                             v + (size_t)b * S * KV * D, KV * D, vb, Sb, H, KV, D, m->attn_scale,
                             window, ctx + (size_t)b * S * GD, GD, nthreads);
        }
    }
    or_quantize_mt(ctx, M, GD, qa, as, nthreads);
    or_i8_gemm_mt(qa, as, L->wo, L->so, NULL, M, Dm, GD, out, nthreads);
    rc = 0;
fail:
    free(qa); free(as); free(qkv); free(q); free(k); free(v); free(ctx); free(cs); free(sn);
    return rc;
}

static int ffn_core(const or_model *m, const or_layer *L, const float *xin, int rows, float *tmp,
                    int nthreads) {
    const int Dm = m->hidden, F = m->ffn;
    int rc = -1;
    int8_t *qa = malloc((size_t)rows * (F > Dm ? F : Dm));
    float *as = malloc(sizeof(float) * (size_t)rows * ((F > Dm ? F : Dm) / 128));
    float *g = malloc(sizeof(float) * (size_t)rows * F), *u = malloc(sizeof(float) * (size_t)rows * F);
    OR_CHECK(qa && as && g && u);
    or_quantize_mt(xin, rows, Dm, qa, as, nthreads);
    or_i8_gemm_mt(qa, as, L->wgate, L->sgate, NULL, rows, F, Dm, g, nthreads);
    or_i8_gemm_mt(qa, as, L->wup, L->sup, NULL, rows, F, Dm, u, nthreads);
    or_gelu_mul_quant(g, F, u, F, rows, F, 128, qa, as);
    or_i8_gemm_mt(qa, as, L->wdown, L->sdown, NULL, rows, Dm, F, tmp, nthreads);
    rc = 0;
fail:
    free(qa); free(as); free(g); free(u);
    return rc;
}

int or_ffn_sublayer(const or_model *m, int l, float *x, int rows, int nthreads) {
    const or_layer *L = &m->layers[l];
    const int Dm = m->hidden;
    float *res = malloc(sizeof(float) * (size_t)rows * Dm);
    float *tmp = malloc(sizeof(float) * (size_t)rows * Dm);
    int rc = -1;
    OR_CHECK(res && tmp);
    or_norm_split(x, res, rows, Dm, L->pre_ffn_ln, m->eps);
    OR_CHECK(ffn_core(m, L, x, rows, tmp, nthreads) == 0);
    or_norm_add(x, tmp, res, rows, Dm, L->post_ffn_ln, m->eps);
    rc = 0;
fail:
    free(res); free(tmp);
    return rc;
}

/* text.c:906-915: x = rms(GEMM(quant(gelu(GEMM(quant(x), ple_gate)) * ple_l), ple_proj)) *
 * ple_norm + x, ple_l = this layer's slice of the per-layer inputs (row stride ldp) */
static int ple_block(const or_model *m, const or_layer *L, float *x, int rows, const float *ple_l,
                     int ldp, int nthreads) {
    const int Dm = m->hidden, P = m->ple_dim, W = Dm > P ? Dm : P;
    int rc = -1;
    int8_t *qa = malloc((size_t)rows * W);
    float *as = malloc(sizeof(float) * (size_t)rows * (W / 128));
    float *g = malloc(sizeof(float) * (size_t)rows * P), *tmp = malloc(sizeof(float) * (size_t)rows * Dm);
    OR_CHECK(qa && as && g && tmp);
    or_quantize_mt(x, rows, Dm, qa, as, nthreads);
    or_i8_gemm_mt(qa, as, L->wple_gate, L->sple_gate, NULL, rows, P, Dm, g, nthreads);
    or_gelu_mul_quant(g, P, ple_l, ldp, rows, P, 128, qa, as);
    or_i8_gemm_mt(qa, as, L->wple_proj, L->sple_proj, NULL, rows, Dm, P, tmp, nthreads);
    or_norm_add(x, tmp, x, rows, Dm, L->ple_norm, m->eps);
    rc = 0;
fail:
    free(qa); free(as); free(g); free(tmp);
    return rc;
}

int or_layer_forward(const or_model *m, int l, float *x, int B, int S, const uint8_t *valid,
                     int nthreads) {
    return or_layer_forward_ple(m, l, x, NULL, B, S, valid, nthreads);
}

int or_layer_forward_ple(const or_model *m, int l, float *x, const float *ple, int B, int S,
                         const uint8_t *valid, int nthreads) {
    const or_layer *L = &m->layers[l];
    const int M = B * S, Dm = m->hidden;
    if (m->ple_dim > 0 && !ple) return -1;
    float *res = malloc(sizeof(float) * (size_t)M * Dm);
    float *tmp = malloc(sizeof(float) * (size_t)M * Dm);
    int rc = -1;
    OR_CHECK(res && tmp);
    or_norm_split(x, res, M, Dm, L->input_ln, m->eps);
    OR_CHECK(or_attention_sublayer(m, l, x, B, S, valid, tmp, nthreads) == 0);
    or_norm_add(x, tmp, res, M, Dm, L->post_attn_ln, m->eps);
    or_norm_split(x, res, M, Dm, L->pre_ffn_ln, m->eps);
    OR_CHECK(ffn_core(m, L, x, M, tmp, nthreads) == 0);
    or_norm_add(x, tmp, res, M, Dm, L->post_ffn_ln, m->eps);
    if (m->ple_dim > 0) {
        const int ldp = m->n_layers * m->ple_dim;
        OR_CHECK(ple_block(m, L, x, M, ple + (size_t)l * m->ple_dim, ldp, nthreads) == 0);
        if (L->layer_scalar != 1.0f)
            for (size_t i = 0; i < (size_t)M * Dm; i++) x[i] *= L->layer_scalar;
    }
    rc = 0;
fail:
    free(res); free(tmp);
    return rc;
}

int or_ple_inputs(const or_model *m, const float *x, int rows, float *ple, int nthreads) {
    const int Dm = m->hidden, NP = m->n_layers * m->ple_dim;
    int8_t *qa = malloc((size_t)rows * Dm);
    float *as = malloc(sizeof(float) * (size_t)rows * (Dm / 128));
    if (!qa || !as) {
        free(qa); free(as);
        return -1;
    }
    or_quantize_mt(x, rows, Dm, qa, as, nthreads);
    or_i8_gemm_mt(qa, as, m->wple_model, m->sple_model, NULL, rows, NP, Dm, ple, nthreads);
    for (size_t i = 0; i < (size_t)rows * NP; i++) ple[i] *= m->ple_scale;
    or_rmsnorm(ple, rows * m->n_layers, m->ple_dim, m->ple_proj_norm, m->eps);
    free(qa); free(as);
    return 0;
}

int or_encode(const or_model *m, const int32_t *ids, const uint8_t *valid, int B, int S,
              float *out, int nthreads) {
    const int M = B * S, Dm = m->hidden, Do = m->out_dim > 0 ? m->out_dim : Dm;
    for (int i = 0; i < M; i++)
        if (ids[i] < 0 || ids[i] >= m->vocab) return -1;
    int rc = -1;
    float *x = malloc(sizeof(float) * (size_t)M * Dm), *ple = NULL, *emb = NULL;
    int8_t *qa = NULL;
    float *as = NULL;
    OR_CHECK(x);
    or_embed(m->embed, ids, M, Dm, m->embed_scale, x);
    if (m->ple_dim > 0 && m->n_layers > 0) {
        ple = malloc(sizeof(float) * (size_t)M * m->n_layers * m->ple_dim);
        OR_CHECK(ple && or_ple_inputs(m, x, M, ple, nthreads) == 0);
    }
    for (int l = 0; l < m->n_layers; l++)
        OR_CHECK(or_layer_forward_ple(m, l, x, ple, B, S, valid, nthreads) == 0);
    or_rmsnorm(x, M, Dm, m->final_norm, m->eps);
    const float *rows = x;
    if (m->out_dim > 0) {
        emb = malloc(sizeof(float) * (size_t)M * Do);
        qa = malloc((size_t)M * Dm);
        as = malloc(sizeof(float) * (size_t)M * (Dm / 128));
        OR_CHECK(emb && qa && as);
        or_quantize_mt(x, M, Dm, qa, as, nthreads);
        or_i8_gemm_mt(qa, as, m->wembed_proj, m->sembed_proj, NULL, M, Do, Dm, emb, nthreads);
        rows = emb;
    }
    for (int b = 0; b < B; b++) {
        float *o = out + (size_t)b * Do;
        const uint8_t *vb = valid + (size_t)b * S;
        or_meanpool(rows + (size_t)b * S * Do, S, Do, vb, o);
        int any = 0;
        for (int i = 0; i < S; i++) any |= vb[i];
        if (any) or_l2norm(o, Do); /* all-invalid stays an exact zero vector: text.c:968-980 */
    }
    rc = 0;
fail:
    free(x); free(ple); free(emb); free(qa); free(as);
    return rc;
}
