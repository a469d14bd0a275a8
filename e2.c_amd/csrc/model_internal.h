// model_internal.h — the host model's tensor records, shared by model.cpp and forward.cpp.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "../../include/e2.h"
#include "../../include/e2mi.h"

namespace e2mi {

struct HostQ8W {  // the reference's e2_q8w (int8.h:79-92), owned or borrowed from a mapping
    const int8_t *w = nullptr;
    const float *scale = nullptr;
    const int32_t *bsq = nullptr;
    int N = 0, K = 0, nb = 0, Npad = 0;
    std::vector<int8_t> ow;
    std::vector<float> os;
    std::vector<int32_t> ob;
    size_t bytes() const { return (size_t)Npad * ((K + 3) / 4) * 4; }
};

struct F32T {
    const float *p = nullptr;
    std::vector<float> own;
    int ndim = 1;
    int64_t dims[4] = {0, 0, 0, 0};
    size_t count() const {
        size_t n = 1;
        for (int i = 0; i < ndim; i++) n *= (size_t)dims[i];
        return n;
    }
};

// geometry of layer l (text.c:467-478): head_dim, kv heads, RoPE theta, window (0 = none), and
// whether it is a full-attention layer (layers l % full_period == full_period - 1)
struct LayerGeom {
    int D, KV, window;
    float theta;
    bool full;
};
inline LayerGeom layer_geom(const e2_config &c, int l) {
    const bool full = c.full_period > 0 && l % c.full_period == c.full_period - 1;
    LayerGeom g;
    g.full = full;
    g.D = full ? c.full_head_dim : c.head_dim;
    g.KV = full ? c.full_kv_heads : c.n_kv_heads;
    g.theta = full ? c.rope_theta_full : c.rope_theta;
    g.window = full ? 0 : c.window;
    return g;
}

std::string layer_name(int l, const char *suffix);
const HostQ8W *model_q8(const e2_model *m, const std::string &name);
const float *model_f32(const e2_model *m, const std::string &name, size_t count);
const char *q8_suffix(int s);    // 0 q, 1 k, 2 v, 3 o, 4 gate, 5 up, 6 down, 7 ple gate, 8 ple proj
const char *norm_suffix(int s);  // 0 input, 1 post_attn, 2 pre_ffn, 3 post_ffn, 4 q_norm, 5 k_norm,
                                 // 6 ple norm
const char *embed_name();
const char *final_norm_name();
const char *ple_model_name();
const char *ple_norm_name();
const char *embed_proj_name();
const char *layer_scalar_suffix();

// a model over caller-held tensors (e2mi_create_tensors); NULL with the error set
e2_model *model_from_tensors(const e2mi_tensor *t, int n, const e2_config &c);

// the engine e2_text_embed* created for a model, owned by it: e2_free calls the destructor
void **model_engine_slot(e2_model *m);
void model_set_engine_free(e2_model *m, void (*destroy)(void *));

// weights.hip: unpack a packed [Npad/8][K/4][8][4] blob into dst rows (n / grp) * gstride + goff +
// n % grp of a row-major [*][ld] device matrix; pair_order swaps bits 6 and 7 of that row index
// (the rotate-half pair order of the fused q|k|v GEMM, e2mi_i8_gemm_qkv)
int upload_packed_rows(int8_t *dst, int ld, const int8_t *wq, int N, int K, int grp, int gstride,
                       int goff, hipStream_t s, bool pair_order = false);

}  // namespace e2mi
