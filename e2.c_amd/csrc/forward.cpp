// forward.cpp — the encoder on the device: weight upload, workspace, the per-layer kernel sequence,
// hipGraph capture per (batch, seq_len) shape, and the e2hip-style entry points.
//
// Layer recipe (text.c:939-961), as fused launches:
//   [embed | add_norm] + norm + quant -> int8 x     (e2mi_embed_norm_quant / e2mi_add_norm_quant)
//   q|k|v int8 GEMM -> f32                          (one GEMM over the concatenated N = (H+2KV)*D)
//   q/k/v RMSNorm + RoPE -> f16 q, k, V^T           (e2mi_qkv_norm_rope)
//   attention -> int8 context + scales              (e2mi_attention)
//   O int8 GEMM -> f32
//   norm_add(post_attn) + norm_split(pre_ffn) + quant
//   gate|up int8 GEMM + GeGLU + quant -> int8       (e2mi_i8_gemm_geglu)
//   down int8 GEMM -> f32
// and after the last layer norm_add(post_ffn) + final RMSNorm, masked mean pool, L2
// (text.c:963-981). The reference checkpoint's geometry (e2_config_reference) adds:
//   before the layers: quant(x0), the PLE model GEMM -> f32 [rows][L*P], scale + norm per slice
//     (text.c:929-932: e2mi_quantize, e2mi_i8_gemm, e2mi_scale_norm);
//   per layer its own head_dim / kv heads / RoPE table / window (text.c:467-478), and after the FFN
//     norm_add(post_ffn) + quant of x itself, the PLE gate GEMM with gelu(gate) * ple slice + quant
//     in its epilogue, the PLE projection GEMM, norm_add(ple_norm) * layer_scalar + the next norm +
//     quant (text.c:906-915, 955-961: e2mi_add_norm_scale_quant, e2mi_i8_gemm_gelu_mul);
//   after the final norm: quant + the embed_proj GEMM to out_dim, pooled (text.c:964-965).
// The recorded graph is replayed for every later call of the same shape, like the reference's HIP
// backend (forward.c:553-579).
//
// Packed batches (the default): only valid tokens are computed. Each sequence's valid tokens are
// laid out in order from a row that is a multiple of 8, the total rounded up to a multiple of 256
// (filler rows carry token 0 and belong to no sequence). Every row kernel and GEMM is row-local,
// attention and pooling take each sequence's row range, and RoPE positions come from a per-row
// table, so the embeddings are those of the padded batch (bit-identical for right-padded masks,
// where the attention key tiles and the pooling chunks fall the same way).
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include <algorithm>
#include <deque>
#include <map>
#include <string>
#include <tuple>
#include <utility>
#include <vector>

#include "../../include/e2.h"
#include "../../include/e2_dispatch.h"
#include "common.h"
#include "model_internal.h"
#include "plan.h"
#include "plan_dev.h"

namespace e2mi {

struct LayerDev {
    LayerGeom geo{};
    e2mi_q8w qkv{}, o{}, gu{}, down{}, ple_gate{}, ple_proj{};
    float *ln_in = nullptr, *ln_attn = nullptr, *ln_pre = nullptr, *ln_ffn = nullptr;
    float *q_norm = nullptr, *k_norm = nullptr, *ple_norm = nullptr;
    float layer_scalar = 1.f;
    // the q|k|v weight is stored in the fused GEMM's rotate-half pair order (head_dim 256 layers):
    // e2mi_i8_gemm_qkv runs the q/k/v norms and RoPE in its epilogue
    bool qkv_fused = false;
    // the O and down projections (and the PLE projection) run the norm_add after them in their
    // epilogue (hidden size 768 or 512): e2mi_i8_gemm_add_norm_quant, and at the PLE geometry
    // e2mi_i8_gemm_add_norm_scale_quant for the norm_adds that scale or quantize x itself
    bool o_an = false, down_an = false;
};

static double now_ms() {
    timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return t.tv_sec * 1e3 + t.tv_nsec * 1e-6;
}

}  // namespace e2mi

using namespace e2mi;

// one launch's event pair of the per-kernel profile
struct ProfEv {
    const char *name;
    hipEvent_t a, b;
};

struct e2mi_engine {
    e2_config cfg{};
    int dev = 0;
    hipStream_t stream = nullptr;
    char devname[256] = "";
    std::vector<LayerDev> layers;
    float *embed = nullptr, *final_norm = nullptr, *cos_tab = nullptr, *sin_tab = nullptr;
    // the reference checkpoint's extras: full-layer RoPE tables, PLE model projection and norm,
    // embed_proj; ple32 holds the per-layer inputs [R][n_layers * ple_dim]
    float *cos_full = nullptr, *sin_full = nullptr, *ple_proj_norm = nullptr, *ple32 = nullptr;
    e2mi_q8w ple_model{}, embed_proj{};
    int dout = 0;  // embedding width: out_dim, or hidden
    int R = 0;  // workspace capacity in rows (tokens)
    // activations
    float *x = nullptr, *tmp = nullptr, *qkv = nullptr, *xn = nullptr, *pool_ws = nullptr;
    int8_t *qa = nullptr, *qg = nullptr, *cq = nullptr;
    float *as = nullptr, *gs = nullptr, *cs = nullptr;
    uint16_t *q16 = nullptr, *k16 = nullptr, *vt16 = nullptr;
    int32_t *ids = nullptr;
    uint8_t *valid = nullptr;
    float *out = nullptr;
    int bmax = 0;  // sequences per chunk (pinned output staging)
    int32_t *h_ids = nullptr;
    uint8_t *h_valid = nullptr;
    float *h_out = nullptr;
    // packed batches: per packed row its source index in the chunk (-1 filler) and RoPE position,
    // per sequence its first row and length, and the attention work lists: regions of one device
    // buffer (d_plan) and of its pinned staging twin (h_plan), laid out per (sequences, rows) by
    // plan_layout, so one copy uploads a chunk's plan and every graph of a shape reads it at the
    // same addresses
    int32_t *d_plan = nullptr, *h_plan = nullptr;
    // the device entry plans on the device when the whole batch fits one chunk (device_plan_fits):
    // the planner writes the packed row count here, and the forward's kernels read it
    int32_t *d_rows = nullptr;
    bool device_plan = true;  // E2MI_DEVICE_PLAN=0 / e2mi_set_device_plan(0): plan on the host
    int32_t *rowmap = nullptr, *pos = nullptr, *seq_start = nullptr, *seq_len = nullptr;
    int32_t *h_rowmap = nullptr, *h_pos = nullptr, *h_start = nullptr, *h_len = nullptr;
    // attention work list (longest sequences first), a fixed number of slots per (sequences, rows):
    // with split key ranges (head_dim-256 layers) split_factor times the unsplit slots, the merge
    // list, the partial states, and an unsplit list for the head_dim-512 layers
    int32_t *work = nullptr, *h_work = nullptr;
    int split_factor = 1;  // the most parts a block of this geometry can take (1: never split)
    // 0 never (the default: a sequence's embedding does not depend on its batch-mates, as on the
    // reference's CPU path), 1 always, 2 when a chunk's blocks fill less than half the device
    int split_mode = 0;
    bool split_now = false;  // the planned chunk splits (part of the graph key)
    int slots_device = 512;  // attention workgroups the device runs at once (2 per CU)
    int32_t *mwork = nullptr, *h_mwork = nullptr, *work_full = nullptr, *h_work_full = nullptr;
    float *part = nullptr;
    // the int8 attention (text.c:638-700) when the selection surface picks it: sequences of at
    // least kI8MinKeys keys go to its own work list, f32 q/k/v feed it (packed batches only)
    bool attn_i8 = false;
    float *q32 = nullptr, *k32 = nullptr, *v32 = nullptr;
    unsigned char *i8ws = nullptr;
    int32_t *work8 = nullptr, *h_work8 = nullptr;
    uint8_t *h_mask = nullptr;  // device-entry mask copy
    size_t mask_cap = 0;
    // the stream of the previous call: a call on another stream first waits for it (the calls share
    // the workspace and the pinned staging arrays)
    hipStream_t last_stream = nullptr;
    // device-side id check of the device entry: each call's check kernel raises its own flag for an
    // id outside the vocabulary, one of kFlagSlots ints of mapped pinned host memory (h_flags;
    // d_flags is its device address), used in turn; the slots of calls whose flags are still unread
    // wait in `unread`, in call order, each with an event recorded after the call's check kernel. A
    // call reads the flags of the earlier checks that have finished without waiting for the others,
    // so calls on a caller stream are enqueued back to back.
    static constexpr int kFlagSlots = 64;
    int *d_flags = nullptr, *h_flags = nullptr;
    hipEvent_t flag_ev[kFlagSlots] = {};
    std::deque<int> unread;
    int next_slot = 0;
    // a device-planned call's planner also writes its row count into its slot of h_rows (mapped
    // pinned memory; 0 until written); when the host reads the slot of a finished call it keeps the
    // count per (sequences, seq_len) in rows_seen, the estimate from which the next calls of that
    // shape choose their GEMM tile shapes
    int *d_rows_seen = nullptr, *h_rows = nullptr;
    std::pair<int, int> slot_shape[kFlagSlots];
    std::map<std::pair<int, int>, int> rows_seen;
    bool packed = true;
    // (sequences, seq_len, rows, bits: packed 1, split 2, planned on the device 4)
    std::map<std::tuple<int, int, int, int>, hipGraphExec_t> graphs;
    bool use_graph = true;
    bool fuse_qkv = true;  // E2MI_NOFUSE=1: the q|k|v GEMM and the norm/RoPE kernel run separately
    bool fuse_an = true;   // E2MI_NOFUSE_AN=1: the O and down GEMMs and their norm_add run separately
    int layer_limit = 0;
    long calls = 0, kernels_last = 0;
    double last_ms = 0.0;
    std::vector<void *> allocs;
    // diagnostics (the reference's E2_HIP_PROFILE and E2_HIP_DUMP, hip.c:51-108,138-139,279,
    // forward.c:715-759). E2MI_PROFILE: the first call runs without a graph with an event pair per
    // launch, totalled per stage into prof_text (printed to stderr). E2MI_DUMP=dir: after call
    // number E2MI_DUMP_CALL (default 1) the workspace of its last chunk is written to dir.
    bool prof_on = false, prof_rec = false;
    std::vector<ProfEv> pev;
    std::string prof_text;
    std::string dump_dir;
    long dump_call = 1;
    int last_M = 0, last_B = 0, last_S = 0, last_layer = 0;
    bool last_pk = false;
};

namespace e2mi {

// rowops.hip
int launch_embed_checked(hipStream_t s, const float *table, int vocab, const int32_t *ids, float embed_scale,
                         const float *gamma, float eps, int M, int D, float *x_out, int8_t *q, float *qs,
                         int *bad_id);
int launch_zero_f32(hipStream_t s, float *p, long n);
int launch_check_ids(hipStream_t s, const int32_t *ids, long n, int vocab, int *flag);
// gemm.hip: whether a per-128 GEMM of M x N rows takes 128 x 128 tiles (else 256 x 128)
bool gemm_half_tiles(int M, int N);
// gemm_an.hip: the 16-row units per workgroup of e2mi_i8_gemm_add_norm_quant at a row count, and
// whether one round of the CUs covers that count
int gemm_an_units(int rows);
bool gemm_an_fits(int rows);

template <class T>
static int dalloc(e2mi_engine *g, T **p, size_t count) {
    *p = nullptr;
    void *v = nullptr;
    if (check_hip(hipMalloc(&v, count * sizeof(T) + 256), "hipMalloc workspace")) return -1;
    g->allocs.push_back(v);
    *p = (T *)v;
    return 0;
}

static int upload_f32(e2mi_engine *g, float **dst, const float *src, size_t n) {
    if (!src) {
        set_error("create: missing f32 tensor");
        return -1;
    }
    if (dalloc(g, dst, n)) return -1;
    return check_hip(hipMemcpyAsync(*dst, src, n * 4, hipMemcpyHostToDevice, g->stream), "upload f32");
}

// one weight as it is (row-major device copy of its packed blob, per-row scales)
static int upload_q8(e2mi_engine *g, e2mi_q8w &d, const HostQ8W *w) {
    if (!w) {
        set_error("create: missing int8 weight");
        return -1;
    }
    memset(&d, 0, sizeof d);
    d.N = w->N;
    d.K = w->K;
    d.ld = (w->K + 15) & ~15;
    d.out_min = -1e31f;
    d.out_max = 1e31f;
    if (dalloc(g, &d.w, (size_t)w->N * d.ld) || dalloc(g, &d.scale, (size_t)w->N) ||
        upload_packed_rows(d.w, d.ld, w->w, w->N, w->K, w->N, 0, 0, g->stream) ||
        check_hip(hipMemcpyAsync(d.scale, w->scale, (size_t)w->N * 4, hipMemcpyHostToDevice, g->stream), "q8 scale"))
        return -1;
    return check_hip(hipStreamSynchronize(g->stream), "q8 upload sync");
}

// concatenate / interleave the reference's separate weights into the fused device operands
static int upload_layer(e2mi_engine *g, const e2_model *m, int l, LayerDev &L) {
    const e2_config &c = g->cfg;
    const int nq8 = c.ple_dim > 0 ? 9 : 7;
    const HostQ8W *w[9] = {};
    for (int s = 0; s < nq8; s++) {
        w[s] = model_q8(m, layer_name(l, q8_suffix(s)));
        if (!w[s]) {
            set_error("create: layer %d: %s missing", l, q8_suffix(s));
            return -1;
        }
    }
    L.geo = layer_geom(c, l);
    const int K = c.hidden, qd = c.n_heads * L.geo.D, kvd = L.geo.KV * L.geo.D;
    auto make = [&](e2mi_q8w &d, int N, int Kd) {
        memset(&d, 0, sizeof d);
        d.N = N;
        d.K = Kd;
        d.ld = (Kd + 15) & ~15;
        d.out_min = -1e31f;
        d.out_max = 1e31f;
        if (dalloc(g, &d.w, (size_t)N * d.ld) || dalloc(g, &d.scale, (size_t)N)) return -1;
        return 0;
    };
    // q|k|v rows (head_dim 256: in the fused GEMM's pair order, bits 6 and 7 of the row swapped)
    if (make(L.qkv, qd + 2 * kvd, K)) return -1;
    L.qkv_fused = g->fuse_qkv && L.geo.D == 256;
    const int off[3] = {0, qd, qd + kvd}, nrows[3] = {qd, kvd, kvd};
    std::vector<float> sc(qd + 2 * kvd);
    for (int s = 0; s < 3; s++) {
        if (upload_packed_rows(L.qkv.w, L.qkv.ld, w[s]->w, nrows[s], K, nrows[s], 0, off[s], g->stream,
                               L.qkv_fused))
            return -1;
        for (int n = 0; n < nrows[s]; n++) {
            const int r = off[s] + n;
            sc[L.qkv_fused ? (r & ~0xC0) | ((r & 0x40) << 1) | ((r & 0x80) >> 1) : r] = w[s]->scale[n];
        }
    }
    if (check_hip(hipMemcpyAsync(L.qkv.scale, sc.data(), sc.size() * 4, hipMemcpyHostToDevice, g->stream),
                  "upload qkv scale") ||
        hipStreamSynchronize(g->stream) != hipSuccess)
        return -1;
    // o, down
    if (make(L.o, c.hidden, qd) || upload_packed_rows(L.o.w, L.o.ld, w[3]->w, c.hidden, qd, c.hidden, 0, 0, g->stream) ||
        check_hip(hipMemcpyAsync(L.o.scale, w[3]->scale, (size_t)c.hidden * 4, hipMemcpyHostToDevice, g->stream), "o scale"))
        return -1;
    if (make(L.down, c.hidden, c.ffn) ||
        upload_packed_rows(L.down.w, L.down.ld, w[6]->w, c.hidden, c.ffn, c.hidden, 0, 0, g->stream) ||
        check_hip(hipMemcpyAsync(L.down.scale, w[6]->scale, (size_t)c.hidden * 4, hipMemcpyHostToDevice, g->stream), "down scale"))
        return -1;
    // gate|up interleaved per 32 rows: [gate 32 | up 32] blocks (the GeGLU epilogue's layout)
    if (make(L.gu, 2 * c.ffn, K) ||
        upload_packed_rows(L.gu.w, L.gu.ld, w[4]->w, c.ffn, K, 32, 64, 0, g->stream) ||
        upload_packed_rows(L.gu.w, L.gu.ld, w[5]->w, c.ffn, K, 32, 64, 32, g->stream))
        return -1;
    std::vector<float> gus(2 * c.ffn);
    for (int n = 0; n < c.ffn; n++) {
        gus[(n / 32) * 64 + n % 32] = w[4]->scale[n];
        gus[(n / 32) * 64 + 32 + n % 32] = w[5]->scale[n];
    }
    if (check_hip(hipMemcpyAsync(L.gu.scale, gus.data(), gus.size() * 4, hipMemcpyHostToDevice, g->stream), "gu scale"))
        return -1;
    L.o_an = g->fuse_an && (c.hidden == 768 || c.hidden == 512);
    L.down_an = L.o_an;
    float **norms[7] = {&L.ln_in, &L.ln_attn, &L.ln_pre, &L.ln_ffn, &L.q_norm, &L.k_norm, &L.ple_norm};
    for (int s = 0; s < (c.ple_dim > 0 ? 7 : 6); s++) {
        const size_t n = (s == 4 || s == 5) ? (size_t)L.geo.D : (size_t)c.hidden;
        if (upload_f32(g, norms[s], model_f32(m, layer_name(l, norm_suffix(s)), n), n)) return -1;
    }
    if (c.ple_dim > 0) {  // the PLE block's two GEMMs and the layer scale (text.c:906-915, 959)
        if (upload_q8(g, L.ple_gate, w[7]) || upload_q8(g, L.ple_proj, w[8])) return -1;
        const float *ls = model_f32(m, layer_name(l, layer_scalar_suffix()), 1);
        if (!ls) {
            set_error("create: layer %d: layer_scalar missing", l);
            return -1;
        }
        L.layer_scalar = ls[0];
    }
    return check_hip(hipStreamSynchronize(g->stream), "layer upload sync");
}

// RoPE tables, text.c:483-506: inv = 1/theta^(2i/D), f = p * inv, duplicated over both halves
static void rope_tables(int D, float theta, int S, std::vector<float> &cs, std::vector<float> &sn) {
    cs.resize((size_t)S * D);
    sn.resize((size_t)S * D);
    for (int p = 0; p < S; p++)
        for (int i = 0; i < D / 2; i++) {
            const float inv = 1.0f / powf(theta, (float)(2 * i) / (float)D);
            const float f = (float)p * inv;
            cs[(size_t)p * D + i] = cs[(size_t)p * D + i + D / 2] = cosf(f);
            sn[(size_t)p * D + i] = sn[(size_t)p * D + i + D / 2] = sinf(f);
        }
}

// a geometry beyond the BASELINE one: only the packed forward implements it (window by position,
// head_dim 512, PLE)
static bool reference_geometry(const e2_config &c) {
    return c.window > 0 || c.full_period > 0 || c.ple_dim > 0 || c.out_dim > 0;
}

// the shortest sequence the int8 attention takes (text.c:873-875: its blocked kernels need 32 rows)
constexpr int kI8MinKeys = 32;

// attention workgroups of a packed chunk of n sequences in M rows: at most H (M / 128 + n)
static int work_slots(const e2mi_engine *g, int n, int M) { return g->cfg.n_heads * (M / 128 + n); }

// split key ranges: a 128-query block whose keys span more than 8 tiles of 32 is split into
// ceil(tiles / 8) parts (at most kMaxAttnParts), so the longest blocks no longer set the
// attention's time alone; the parts depend only on the sequence's own length and the window
// (block_parts, plan.cpp). The attention work lists are dealt to the XCDs (xcd_deal, plan.cpp).
constexpr int kAttnPartTiles = 8, kMaxAttnParts = 4;

// every kernel of one forward over B sequences of S tokens (M rows: B * S padded, or the packed
// row count), on stream s; returns the launch count or -1
static int enqueue(e2mi_engine *g, int B, int S, int Mp, bool pk, hipStream_t s, bool dev = false, int est = 0) {
    // dev: planned on the device, Mp rows of capacity; the kernels read the planned count, the GEMMs
    // choose their tiles for about `est` rows
    const DeviceRowsScope dev_rows(dev ? g->d_rows : nullptr, 1, est);
    const e2_config &c = g->cfg;
    const int M = pk ? Mp : B * S, Dm = c.hidden, H = c.n_heads, P = c.ple_dim;
    // the projections with their norm_add in the epilogue when one round of the CUs covers the
    // (expected) rows; past that each workgroup's weight fetch costs more than the f32 round trip
    const bool an = gemm_an_fits(dev && est > 0 ? est : M);
    if (M <= 0 || M > g->R) {
        set_error("forward: %d rows for a %d-row workspace", M, g->R);
        return -1;
    }
    const int nl = g->layer_limit > 0 && g->layer_limit < c.n_layers ? g->layer_limit : c.n_layers;
    const float eps = c.rms_eps;
    int k = 0;
    g->last_M = M;
    g->last_B = B;
    g->last_S = S;
    g->last_pk = pk;
    g->last_layer = nl - 1;
    // with the per-kernel profile on (E2MI_PROFILE, first call only), each launch is bracketed by
    // an event pair on its stream; the times are read after the call has synchronized
#define RUN(name, call)                                                                            \
    do {                                                                                           \
        hipEvent_t ea_ = nullptr, eb_ = nullptr;                                                   \
        if (g->prof_rec && (hipEventCreate(&ea_) != hipSuccess || hipEventCreate(&eb_) != hipSuccess || \
                            hipEventRecord(ea_, s) != hipSuccess)) {                               \
            if (ea_) (void)hipEventDestroy(ea_);                                                   \
            if (eb_) (void)hipEventDestroy(eb_);                                                   \
            ea_ = eb_ = nullptr;                                                                   \
        }                                                                                          \
        if ((call) != 0) {                                                                         \
            if (ea_) (void)hipEventDestroy(ea_), (void)hipEventDestroy(eb_);                       \
            return -1;                                                                             \
        }                                                                                          \
        k++;                                                                                       \
        if (ea_) {                                                                                 \
            if (hipEventRecord(eb_, s) == hipSuccess) g->pev.push_back({name, ea_, eb_});          \
            else (void)hipEventDestroy(ea_), (void)hipEventDestroy(eb_);                           \
        }                                                                                          \
    } while (0)
    RUN("embed", launch_embed_checked(s, g->embed, c.vocab, g->ids, c.embed_scale, g->layers[0].ln_in, eps, M, Dm,
                             g->x, g->qa, g->as, nullptr));
    if (P > 0) {  // the per-layer inputs from the scaled embeddings (text.c:929-932)
        const int NP = c.n_layers * P;
        RUN("ple_quant", e2mi_quantize(s, g->qg, g->gs, g->x, M, Dm, Dm, 128));
        RUN("ple_model", e2mi_i8_gemm(s, g->ple32, NP, g->qg, g->gs, &g->ple_model, M, 0, NP));
        const DeviceRowsScope ple_rows(dev ? g->d_rows : nullptr, c.n_layers, est);  // n_layers slices per row
        RUN("ple_norm", e2mi_scale_norm(s, g->ple32, M * c.n_layers, P, c.ple_scale, g->ple_proj_norm, eps, g->ple32));
    }
    for (int l = 0; l < nl; l++) {
        const LayerDev &L = g->layers[l];
        const int D = L.geo.D, KV = L.geo.KV, qd = H * D;
        const float *cs = L.geo.full ? g->cos_full : g->cos_tab, *sn = L.geo.full ? g->sin_full : g->sin_tab;
        if (L.qkv_fused)
            RUN("qkv_norm_rope_gemm", e2mi_i8_gemm_qkv(s, g->qa, g->as, &L.qkv, M, pk ? M : S, pk ? g->pos : nullptr, H, KV, L.q_norm,
                                 L.k_norm, eps, cs, sn, g->q16, g->k16, g->vt16, g->attn_i8 ? g->q32 : nullptr,
                                 g->attn_i8 ? g->k32 : nullptr, g->attn_i8 ? g->v32 : nullptr));
        else
            RUN("qkv", e2mi_i8_gemm(s, g->qkv, qd + 2 * KV * D, g->qa, g->as, &L.qkv, M, 0, L.qkv.N));
        if (pk) {
            if (!L.qkv_fused)
                RUN("qkv_norm_rope", e2mi_qkv_norm_rope_packed(s, g->qkv, M, g->pos, H, KV, D, L.q_norm, L.k_norm, eps, cs, sn,
                                              g->q16, g->k16, g->vt16, g->q32, g->k32, g->v32));
            if (D == 256 && g->split_now) {
                RUN("attention", e2mi_attention_packed_split(s, g->q16, g->k16, g->vt16, M, g->seq_start, g->seq_len,
                                                             g->pos, B, S, H, KV, D, c.attn_scale, L.geo.window,
                                                             g->cq, g->cs, nullptr, g->work,
                                                             work_slots(g, B, M) * g->split_factor, g->mwork,
                                                             work_slots(g, B, M), g->part, g->R));
                k++;  // the merge
            } else {
                RUN("attention", e2mi_attention_packed_window(s, g->q16, g->k16, g->vt16, M, g->seq_start, g->seq_len,
                                                              g->pos, B, S, H, KV, D, c.attn_scale, L.geo.window,
                                                              g->cq, g->cs, nullptr,
                                                              D == 512 && g->work_full ? g->work_full : g->work,
                                                              work_slots(g, B, M)));
            }
            if (g->attn_i8)
                RUN("attention_i8", e2mi_attention_i8_packed(s, g->q32, g->k32, g->v32, M, g->seq_start, g->seq_len, B, S,
                                             H, KV, D, g->i8ws, g->cq, g->cs, nullptr, g->work8,
                                             work_slots(g, B, M)));
        } else {
            if (!L.qkv_fused)
                RUN("qkv_norm_rope", e2mi_qkv_norm_rope(s, g->qkv, M, S, H, KV, D, L.q_norm, L.k_norm, eps, cs, sn, g->q16,
                                       g->k16, g->vt16, nullptr, nullptr, nullptr));
            RUN("attention", e2mi_attention(s, g->q16, g->k16, g->vt16, g->valid, B, S, H, KV, D, c.attn_scale,
                               g->cq, g->cs, nullptr));
        }
        if (L.o_an && an) {
            RUN("o_proj+add_norm", e2mi_i8_gemm_add_norm_quant(s, g->cq, g->cs, &L.o, M, g->x, L.ln_attn, L.ln_pre, eps,
                                                               g->x, nullptr, g->qa, g->as, nullptr));
        } else {
            RUN("o_proj", e2mi_i8_gemm(s, g->tmp, Dm, g->cq, g->cs, &L.o, M, 0, Dm));
            RUN("add_norm", e2mi_add_norm_quant(s, g->tmp, g->x, L.ln_attn, L.ln_pre, eps, M, Dm, g->x, nullptr,
                                                g->qa, g->as));
        }
        RUN("gate_up_geglu", e2mi_i8_gemm_geglu(s, g->qg, g->gs, nullptr, g->qa, g->as, &L.gu, M));
        const bool last = l + 1 == nl;
        const float *gnext = last ? g->final_norm : g->layers[l + 1].ln_in;
        if (L.down_an && an && P > 0) {
            // post_ffn norm_add in the down projection, x itself quantized for the PLE gate; the PLE
            // block, its norm_add and the layer scale in the PLE projection
            RUN("down+add_norm", e2mi_i8_gemm_add_norm_scale_quant(s, g->qg, g->gs, &L.down, M, g->x, L.ln_ffn, 1.0f,
                                                                   nullptr, eps, g->x, nullptr, g->qa, g->as, nullptr));
            RUN("ple_gate", e2mi_i8_gemm_gelu_mul(s, g->qg, g->gs, nullptr, g->qa, g->as, &L.ple_gate, M,
                                                  g->ple32 + (size_t)l * P, c.n_layers * P));
            RUN("ple_proj+add_norm", e2mi_i8_gemm_add_norm_scale_quant(s, g->qg, g->gs, &L.ple_proj, M, g->x, L.ple_norm,
                                                                       L.layer_scalar, gnext, eps, g->x,
                                                                       last ? g->xn : nullptr, g->qa, g->as, nullptr));
            continue;
        }
        if (L.down_an && an) {
            RUN("down+add_norm", e2mi_i8_gemm_add_norm_quant(s, g->qg, g->gs, &L.down, M, g->x, L.ln_ffn, gnext, eps, g->x,
                                                             last ? g->xn : nullptr,
                                                             !last || c.out_dim > 0 ? g->qa : nullptr,
                                                             !last || c.out_dim > 0 ? g->as : nullptr, nullptr));
            continue;
        }
        RUN("down", e2mi_i8_gemm(s, g->tmp, Dm, g->qg, g->gs, &L.down, M, 0, Dm));
        if (P > 0) {
            // post_ffn norm_add, x itself quantized for the PLE gate; the PLE block; layer scale
            RUN("add_norm", e2mi_add_norm_scale_quant(s, g->tmp, g->x, L.ln_ffn, 1.0f, nullptr, eps, M, Dm, g->x, nullptr,
                                          g->qa, g->as));
            RUN("ple_gate", e2mi_i8_gemm_gelu_mul(s, g->qg, g->gs, nullptr, g->qa, g->as, &L.ple_gate, M,
                                      g->ple32 + (size_t)l * P, c.n_layers * P));
            RUN("ple_proj", e2mi_i8_gemm(s, g->tmp, Dm, g->qg, g->gs, &L.ple_proj, M, 0, Dm));
            RUN("add_norm", e2mi_add_norm_scale_quant(s, g->tmp, g->x, L.ple_norm, L.layer_scalar, gnext, eps, M, Dm, g->x,
                                          last ? g->xn : nullptr, g->qa, g->as));
        } else if (!last) {
            RUN("add_norm", e2mi_add_norm_quant(s, g->tmp, g->x, L.ln_ffn, gnext, eps, M, Dm, g->x, nullptr, g->qa, g->as));
        } else {
            RUN("add_norm", e2mi_add_norm_quant(s, g->tmp, g->x, L.ln_ffn, gnext, eps, M, Dm, g->x, g->xn,
                                    c.out_dim > 0 ? g->qa : nullptr, c.out_dim > 0 ? g->as : nullptr));
        }
    }
    const float *rows = g->xn;
    if (c.out_dim > 0) {  // embed_proj of the final-normed rows (text.c:964-965)
        RUN("embed_proj", e2mi_i8_gemm(s, g->qkv, c.out_dim, g->qa, g->as, &g->embed_proj, M, 0, c.out_dim));
        rows = g->qkv;
    }
    if (pk)
        RUN("pool", e2mi_pool_l2_packed(s, rows, g->seq_start, g->seq_len, B, S, g->dout, g->pool_ws, g->out));
    else
        RUN("pool", e2mi_pool_l2(s, rows, g->valid, B, S, g->dout, g->pool_ws, g->out));
#undef RUN
    return k + 1;  // the pool is two launches
}

// dev: planned on the device (est: the expected row count, sig: the GEMM tile shapes it gives)
static int run_shape(e2mi_engine *g, int B, int S, int Mp, bool pk, hipStream_t s, bool dev = false, int est = 0,
                     int sig = 0) {
    if (!g->use_graph || g->prof_rec) {
        const int k = enqueue(g, B, S, Mp, pk, s, dev, est);
        if (k < 0) return -1;
        g->kernels_last = k;
        return 0;
    }
    auto key = std::make_tuple(B, S, Mp, (pk ? 1 : 0) | (pk && g->split_now ? 2 : 0) | (dev ? 4 : 0) | sig << 3);
    auto it = g->graphs.find(key);
    if (it == g->graphs.end()) {
        // the first call of a shape runs eagerly (kernel attributes get set outside any capture),
        // then the sequence is recorded for every later call
        const int k = enqueue(g, B, S, Mp, pk, s, dev, est);
        if (k < 0) return -1;
        g->kernels_last = k;
        hipGraph_t graph = nullptr;
        if (check_hip(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "begin capture"))
            return -1;
        const int k2 = enqueue(g, B, S, Mp, pk, s, dev, est);
        const hipError_t e = hipStreamEndCapture(s, &graph);
        if (k2 < 0 || check_hip(e, "end capture")) {
            if (graph) (void)hipGraphDestroy(graph);
            return -1;
        }
        hipGraphExec_t exec = nullptr;
        const hipError_t ei = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        if (check_hip(ei, "graph instantiate")) return -1;
        g->graphs[key] = exec;
        return 0;
    }
    return check_hip(hipGraphLaunch(it->second, s), "graph launch");
}

static int validate_batch(const e2mi_engine *g, const int32_t *ids, int batch, int seq_len, bool host_ids) {
    if (batch <= 0 || seq_len <= 0 || seq_len > g->cfg.max_seq) {
        set_error("bad batch geometry (batch=%d, seq_len=%d, max %d)", batch, seq_len, g->cfg.max_seq);
        return -1;
    }
    if (!ids) {
        set_error("token ids pointer is NULL");
        return -1;
    }
    if (host_ids) {  // the whole request is validated before any output is written (text.c:1008-1013)
        const size_t n = (size_t)batch * seq_len;
        for (size_t i = 0; i < n; i++)
            if (ids[i] < 0 || ids[i] >= g->cfg.vocab) {
                set_error("token id %d at position %zu is out of range [0,%d)", ids[i], i, g->cfg.vocab);
                return -1;
            }
    }
    return 0;
}

// The plan's regions for n sequences in Mp packed rows, in int32 units from the start of d_plan /
// h_plan (each region 256-byte aligned): positions, sequence starts and lengths, the f16 work list
// (split_factor times the slots), the merge list, the head_dim-512 list, the int8 list, and last the
// row map (uploaded only by the device entry).
struct PlanLayout {
    size_t pos, start, len, work, mwork, work_full, work8, rowmap, end;
};
static bool has_full_list(const e2mi_engine *g) { return g->split_factor > 1 && g->cfg.full_period > 0; }
static PlanLayout plan_layout(const e2mi_engine *g, int n, int Mp) {
    auto up = [](size_t x) { return (x + 63) & ~(size_t)63; };
    const size_t slots = (size_t)work_slots(g, n, Mp);
    PlanLayout L;
    size_t o = 0;
    L.pos = o, o = up(o + (size_t)Mp);
    L.start = o, o = up(o + (size_t)n);
    L.len = o, o = up(o + (size_t)n);
    L.work = o, o = up(o + slots * (size_t)g->split_factor);
    L.mwork = o, o = up(o + (g->split_factor > 1 ? slots : 0));
    L.work_full = o, o = up(o + (has_full_list(g) ? slots : 0));
    L.work8 = o, o = up(o + slots);
    L.rowmap = o, o = up(o + (size_t)Mp);
    L.end = o;
    return L;
}
static void plan_bind(e2mi_engine *g, const PlanLayout &L) {
    int32_t *d = g->d_plan, *h = g->h_plan;
    g->pos = d + L.pos, g->h_pos = h + L.pos;
    g->seq_start = d + L.start, g->h_start = h + L.start;
    g->seq_len = d + L.len, g->h_len = h + L.len;
    g->work = d + L.work, g->h_work = h + L.work;
    g->mwork = g->split_factor > 1 ? d + L.mwork : nullptr, g->h_mwork = g->split_factor > 1 ? h + L.mwork : nullptr;
    g->work_full = has_full_list(g) ? d + L.work_full : nullptr;
    g->h_work_full = has_full_list(g) ? h + L.work_full : nullptr;
    g->work8 = d + L.work8, g->h_work8 = h + L.work8;
    g->rowmap = d + L.rowmap, g->h_rowmap = h + L.rowmap;
}

// the packed layout of n sequences of S tokens (valid: host mask, null = all valid) into the
// engine's host staging arrays, and the attention work lists; returns the row count
static int plan_pack(e2mi_engine *g, const uint8_t *valid, int n, int S) {
    long rows = 0;
    for (int b = 0; b < n; b++) rows += seq_rows(valid ? valid + (size_t)b * S : nullptr, S);
    plan_bind(g, plan_layout(g, n, (int)((rows + 255) & ~255L)));
    const int Mp = pack_rows(valid, n, S, g->h_rowmap, g->h_pos, g->h_start, g->h_len);
    const int H = g->cfg.n_heads, slots = work_slots(g, n, Mp);
    // split long blocks' keys only where the unsplit blocks leave most of the device idle (few
    // sequences; mode 2): a full batch's blocks already fill it, and the parts' partial states then
    // cost more than they balance (config 4: 9460 -> 8115 embeddings/s split; one 2048-token
    // sequence at the reference geometry: 5.77 -> 4.87 ms)
    long blocks = 0;
    for (int b = 0; b < n; b++) blocks += (long)H * ((g->h_len[b] + 127) / 128);
    const bool split = g->split_factor > 1 &&
                       (g->split_mode == 1 || (g->split_mode == 2 && 2 * blocks <= g->slots_device));
    AttnParams p{H, g->cfg.window, split ? g->split_factor : 1, g->attn_i8, kI8MinKeys, 2};
    AttnLists o;
    o.work = g->h_work;
    o.merge = g->h_mwork;
    o.work_full = g->h_work_full;
    o.work8 = g->attn_i8 ? g->h_work8 : nullptr;
    attention_lists(p, g->h_len, g->h_start, g->h_pos, n, o);
    g->split_now = o.n_merge > 0;  // no block long enough: the unsplit kernel, no merge launch
    int k = o.n_work, km = o.n_merge, kf = o.n_full, k8 = o.n_work8;
    while (k < slots * g->split_factor) g->h_work[k++] = -1;
    if (g->h_mwork)
        while (km < slots) g->h_mwork[km++] = -1;
    if (g->h_work_full)
        while (kf < slots) g->h_work_full[kf++] = -1;
    if (g->attn_i8)
        while (k8 < slots) g->h_work8[k8++] = -1;
    return Mp;
}

// The GEMM tile shapes of a device-planned forward of about `est` rows: one bit per distinct output
// width of the forward's GEMMs whose tile shape follows the row count (gemm_half_tiles)
static int tile_signature(const e2mi_engine *g, int est) {
    std::vector<int> ns;
    const bool an = gemm_an_fits(est);
    for (const LayerDev &L : g->layers) {
        if (!(L.o_an && an)) ns.push_back(L.o.N);
        if (!(L.down_an && an)) ns.push_back(L.down.N);
        if (!L.qkv_fused) ns.push_back(L.qkv.N);
        if (g->cfg.ple_dim > 0) {
            ns.push_back(L.ple_gate.N);
            if (!(L.down_an && an)) ns.push_back(L.ple_proj.N);
        }
    }
    if (g->cfg.ple_dim > 0) ns.push_back(g->ple_model.N);
    if (g->cfg.out_dim > 0) ns.push_back(g->embed_proj.N);
    std::sort(ns.begin(), ns.end());
    ns.erase(std::unique(ns.begin(), ns.end()), ns.end());
    int sig = 0;
    for (size_t i = 0; i < ns.size(); i++)
        if (gemm_half_tiles(est, ns[i])) sig |= 1 << i;
    // whether the GEMMs with the norm_add run, and their row units per workgroup (1-5), in the bits above
    if (!g->layers.empty() && g->layers[0].o_an && an) sig |= 1 << 15 | gemm_an_units(est) << 16;
    return sig;
}

// The device entry plans on the device (plan_dev.hip) when the whole batch is one chunk whatever its
// mask (every token valid: n ceil8(S) rows, rounded up to 256, within the workspace) and its lists fit
// the planner's workgroup, with the unsplit f16 lists (no int8 attention, no split mode) and no
// workspace dump (which writes the host plan). Returns the rows the forward is sized for, or 0.
static int device_plan_rows(const e2mi_engine *g, int n, int S) {
    if (!g->device_plan || !g->packed || g->attn_i8 || g->split_mode != 0 || !g->dump_dir.empty() || n > g->bmax)
        return 0;
    const long cap = ((long)n * ((S + 7) & ~7) + 255) & ~255L;
    if (cap > g->R || !plan_device_fits(n, S, g->cfg.n_heads, work_slots(g, n, (int)cap))) return 0;
    return (int)cap;
}

// sequences of the next chunk starting at b0: as many as fit the workspace rows (packed: rounded
// up to 256), the staging arrays and the pooling workspace; at least one
static int chunk_size(const e2mi_engine *g, const uint8_t *valid, int b0, int batch, int S) {
    if (!g->packed) {
        int per = g->R / S;
        if (per > g->bmax) per = g->bmax;
        return batch - b0 < per ? batch - b0 : per;
    }
    const long pool_cap = (long)g->R / 64 + g->R + 64, chunks = (S + 63) / 64;
    int n = 0;
    long rows = 0;
    while (b0 + n < batch && n < g->bmax && (long)(n + 1) * chunks <= pool_cap) {
        const long r = seq_rows(valid ? valid + (size_t)n * S : nullptr, S);
        if (n > 0 && ((rows + r + 255) & ~255L) > g->R) break;
        rows += r;
        n++;
    }
    return n;
}

// upload the chunk's plan on stream s in one copy (and, from host ids, its packed ids in a second):
// every region but the row map for host ids, the whole plan for device ids
static int upload_pack(e2mi_engine *g, int n, int Mp, const int32_t *host_ids, hipStream_t s) {
    const PlanLayout L = plan_layout(g, n, Mp);
    if (host_ids) {
        for (int r = 0; r < Mp; r++) g->h_ids[r] = g->h_rowmap[r] >= 0 ? host_ids[g->h_rowmap[r]] : 0;
        if (check_hip(hipMemcpyAsync(g->ids, g->h_ids, (size_t)Mp * 4, hipMemcpyHostToDevice, s), "ids H2D"))
            return -1;
    }
    const size_t count = host_ids ? L.rowmap : L.end;
    return check_hip(hipMemcpyAsync(g->d_plan, g->h_plan, count * 4, hipMemcpyHostToDevice, s), "plan H2D");
}

// switch the int8 attention on or off; its buffers (f32 q/k/v, the quantized operands, a second
// work list) are allocated the first time it is switched on
static int set_attention_i8(e2mi_engine *g, bool on) {
    const e2_config &c = g->cfg;
    if (on && (c.window > 0 || c.full_period > 0)) {
        set_error("int8 attention: built for head_dim 256 without a sliding window; this model has "
                  "windowed or head_dim-%d layers", c.full_head_dim);
        return -1;
    }
    if (on && c.attn_scale != 1.0f) {
        set_error("int8 attention implements the reference's attention scale 1.0 (text.c:8-9), the model has %g",
                  (double)c.attn_scale);
        return -1;
    }
    if (on && !g->q32) {
        const size_t R = (size_t)g->R;
        const int qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim;
        const size_t wsb = e2mi_attention_i8_workspace_bytes(g->R, g->bmax, c.max_seq, c.n_heads, c.n_kv_heads);
        if (dalloc(g, &g->q32, R * qd) || dalloc(g, &g->k32, R * kvd) || dalloc(g, &g->v32, R * kvd) ||
            dalloc(g, &g->i8ws, wsb))
            return -1;
    }
    g->attn_i8 = on;
    for (auto &kv : g->graphs) (void)hipGraphExecDestroy(kv.second);
    g->graphs.clear();
    return 0;
}

}  // namespace e2mi

// ------------------------------------------------------------------ C ABI (e2hip.h:34-64)
extern "C" void e2mi_destroy(e2mi_engine *g) {
    if (!g) return;
    if (g->stream) (void)hipStreamSynchronize(g->stream);
    for (const ProfEv &e : g->pev) (void)hipEventDestroy(e.a), (void)hipEventDestroy(e.b);
    for (auto &kv : g->graphs) (void)hipGraphExecDestroy(kv.second);
    for (void *p : g->allocs) (void)hipFree(p);
    if (g->h_ids) (void)hipHostFree(g->h_ids);
    if (g->h_valid) (void)hipHostFree(g->h_valid);
    if (g->h_out) (void)hipHostFree(g->h_out);
    if (g->h_plan) (void)hipHostFree(g->h_plan);
    if (g->h_mask) (void)hipHostFree(g->h_mask);
    if (g->h_flags) (void)hipHostFree(g->h_flags);
    if (g->h_rows) (void)hipHostFree(g->h_rows);
    for (hipEvent_t e : g->flag_ev)
        if (e) (void)hipEventDestroy(e);
    if (g->last_stream) (void)hipStreamSynchronize(g->last_stream);
    if (g->stream) (void)hipStreamDestroy(g->stream);
    delete g;
}

extern "C" e2mi_engine *e2mi_create_rows(const e2_model *m, int max_rows) {
    if (!m) {
        set_error("create: null model");
        return nullptr;
    }
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0) {
        set_error("create: no HIP device");
        return nullptr;
    }
    e2mi_engine *g = new (std::nothrow) e2mi_engine();
    if (!g) {
        set_error("oom: engine");
        return nullptr;
    }
    e2_model_config(m, &g->cfg);
    const e2_config &c = g->cfg;
    g->R = max_rows > 0 ? max_rows : 32768;
    if (g->R < c.max_seq) g->R = c.max_seq;
    g->R = (g->R + 255) & ~255;  // a packed chunk of one full sequence fits
    const char *ng = getenv("E2MI_NOGRAPH");
    g->use_graph = !(ng && ng[0] && ng[0] != '0');
    const char *nf = getenv("E2MI_NOFUSE");
    g->fuse_qkv = !(nf && nf[0] && nf[0] != '0');
    const char *na = getenv("E2MI_NOFUSE_AN");
    g->fuse_an = !(na && na[0] && na[0] != '0');
    const char *dp = getenv("E2MI_DEVICE_PLAN");  // 1 (default) | 0
    g->device_plan = !(dp && dp[0] == '0');
    const char *ns = getenv("E2MI_SPLIT");  // 0 (default) | 1 | auto
    if (ns && ns[0]) g->split_mode = ns[0] == '0' ? 0 : ns[0] == '1' ? 1 : 2;
    {
        // the most key tiles a query block can span: the sequence, or the window around the block
        int tiles = (c.max_seq + 31) / 32;
        if (c.window > 0) tiles = std::min(tiles, (128 + 2 * c.window) / 32 + 2);
        g->split_factor = std::max(1, std::min(kMaxAttnParts, (tiles + kAttnPartTiles - 1) / kAttnPartTiles));
    }
    const char *pf = getenv("E2MI_PROFILE");
    g->prof_on = pf && pf[0] && pf[0] != '0';
    const char *dd = getenv("E2MI_DUMP");
    if (dd && dd[0]) {
        g->dump_dir = dd;
        const char *dc = getenv("E2MI_DUMP_CALL");  // a call number (default 1), or "all"
        g->dump_call = dc && !strcmp(dc, "all") ? -1 : dc && atol(dc) > 0 ? atol(dc) : 1;
    }
    auto fail = [&]() -> e2mi_engine * {
        e2mi_destroy(g);
        return nullptr;
    };
    if (check_hip(hipGetDevice(&g->dev), "get device")) return fail();
    hipDeviceProp_t prop;
    if (check_hip(hipGetDeviceProperties(&prop, g->dev), "device properties")) return fail();
    g->slots_device = 2 * prop.multiProcessorCount;  // k_attn_packed<256>: two workgroups per CU
    snprintf(g->devname, sizeof g->devname, "%s (%s, %d CUs)", prop.name, prop.gcnArchName,
             prop.multiProcessorCount);
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        set_error("create: this backend is built for gfx950, the device is %s", prop.gcnArchName);
        return fail();
    }
    // the attention precision comes from the selection surface (dispatch.c:180-197)
    e2_attn_env_reload();
    const e2_attn_kind ak = e2_attn_pick(E2_BK_HIP_GFX950, E2_TOWER_TEXT, E2_ATTN_ANY_KEYS);
    if (ak == E2_ATTN_F32) {
        set_error("create: attention kind f32 requested; this backend implements f16 and i8");
        return fail();
    }
    if (check_hip(hipStreamCreateWithFlags(&g->stream, hipStreamNonBlocking), "stream")) return fail();
    // weights
    g->layers.resize(c.n_layers);
    for (int l = 0; l < c.n_layers; l++)
        if (upload_layer(g, m, l, g->layers[l])) return fail();
    if (upload_f32(g, &g->embed, model_f32(m, embed_name(), (size_t)c.vocab * c.hidden),
                   (size_t)c.vocab * c.hidden) ||
        upload_f32(g, &g->final_norm, model_f32(m, final_norm_name(), (size_t)c.hidden), (size_t)c.hidden))
        return fail();
    std::vector<float> cs, sn;
    rope_tables(c.head_dim, c.rope_theta, c.max_seq, cs, sn);
    if (upload_f32(g, &g->cos_tab, cs.data(), cs.size()) || upload_f32(g, &g->sin_tab, sn.data(), sn.size()))
        return fail();
    if (c.full_period > 0) {
        rope_tables(c.full_head_dim, c.rope_theta_full, c.max_seq, cs, sn);
        if (upload_f32(g, &g->cos_full, cs.data(), cs.size()) || upload_f32(g, &g->sin_full, sn.data(), sn.size()))
            return fail();
    }
    if (c.ple_dim > 0 && (upload_q8(g, g->ple_model, model_q8(m, ple_model_name())) ||
                          upload_f32(g, &g->ple_proj_norm, model_f32(m, ple_norm_name(), (size_t)c.ple_dim),
                                     (size_t)c.ple_dim)))
        return fail();
    if (c.out_dim > 0 && upload_q8(g, g->embed_proj, model_q8(m, embed_proj_name()))) return fail();
    g->dout = c.out_dim > 0 ? c.out_dim : c.hidden;
    // workspace for R rows, sized for the widest layer
    const size_t R = (size_t)g->R;
    int qd = 0, kvd = 0, nqkv = 0;
    for (const LayerDev &L : g->layers) {
        qd = std::max(qd, c.n_heads * L.geo.D);
        kvd = std::max(kvd, L.geo.KV * L.geo.D);
        nqkv = std::max(nqkv, (c.n_heads + 2 * L.geo.KV) * L.geo.D);
    }
    nqkv = std::max(nqkv, std::max(c.out_dim, c.ple_dim));  // also the PLE gate and embed_proj rows
    const int kmax = std::max(c.hidden, c.ffn), gmax = std::max(kmax, c.ple_dim);
    g->bmax = g->R < 4096 ? g->R : 4096;
    if (dalloc(g, &g->x, R * c.hidden) || dalloc(g, &g->tmp, R * c.hidden) ||
        dalloc(g, &g->xn, R * c.hidden) || dalloc(g, &g->qkv, R * nqkv) ||
        dalloc(g, &g->qa, R * kmax) || dalloc(g, &g->as, R * (kmax / 128)) ||
        dalloc(g, &g->qg, R * gmax) || dalloc(g, &g->gs, R * (gmax / 128)) ||
        dalloc(g, &g->cq, R * qd) || dalloc(g, &g->cs, R * (qd / 128)) ||
        dalloc(g, &g->q16, R * qd) || dalloc(g, &g->k16, R * kvd) || dalloc(g, &g->vt16, R * kvd) ||
        dalloc(g, &g->ids, R) || dalloc(g, &g->valid, R) || dalloc(g, &g->out, R * g->dout) ||
        dalloc(g, &g->pool_ws, (R / 64 + R + 64) * (size_t)(g->dout + 1)) ||
        (c.ple_dim > 0 && dalloc(g, &g->ple32, R * c.n_layers * c.ple_dim)) ||
        dalloc(g, &g->d_plan, plan_layout(g, g->bmax, (int)R).end) || dalloc(g, &g->d_rows, 1) ||
        (g->split_factor > 1 && dalloc(g, &g->part, e2mi_attention_part_bytes(R, c.n_heads, 256) / 4 + 64)))
        return fail();
    if (check_hip(hipHostMalloc((void **)&g->h_ids, R * 4), "pinned ids") ||
        check_hip(hipHostMalloc((void **)&g->h_valid, R), "pinned valid") ||
        check_hip(hipHostMalloc((void **)&g->h_out, (size_t)g->bmax * g->dout * 4), "pinned out") ||
        check_hip(hipHostMalloc((void **)&g->h_plan, plan_layout(g, g->bmax, (int)R).end * 4), "pinned plan") ||
        check_hip(hipHostMalloc((void **)&g->h_flags, e2mi_engine::kFlagSlots * 4,
                                hipHostMallocMapped | hipHostMallocCoherent), "pinned flags") ||
        check_hip(hipHostGetDevicePointer((void **)&g->d_flags, g->h_flags, 0), "flag device address") ||
        check_hip(hipHostMalloc((void **)&g->h_rows, e2mi_engine::kFlagSlots * 4,
                                hipHostMallocMapped | hipHostMallocCoherent), "pinned row counts") ||
        check_hip(hipHostGetDevicePointer((void **)&g->d_rows_seen, g->h_rows, 0), "row count device address"))
        return fail();
    for (int k = 0; k < e2mi_engine::kFlagSlots; k++) {
        g->h_flags[k] = 0;
        g->h_rows[k] = 0;
        if (check_hip(hipEventCreateWithFlags(&g->flag_ev[k], hipEventDisableTiming), "flag event")) return fail();
    }
    plan_bind(g, plan_layout(g, g->bmax, (int)R));
    // filler rows of packed batches read contexts that no attention writes: start them at zero; a
    // device-planned forward writes its plan's rows only up to its row count, so the plan's rows
    // past it hold earlier calls' entries or these zeros (valid positions and tokens)
    if (check_hip(hipMemsetAsync(g->d_plan, 0, plan_layout(g, g->bmax, (int)R).end * 4, g->stream), "clear plan") ||
        check_hip(hipMemsetAsync(g->ids, 0, R * 4, g->stream), "clear ids") ||
        check_hip(hipMemsetAsync(g->cq, 0, R * qd, g->stream), "clear ctx") ||
        check_hip(hipMemsetAsync(g->cs, 0, R * (qd / 128) * 4, g->stream), "clear ctx scales"))
        return fail();
    const char *np = getenv("E2MI_NOPACK");
    g->packed = !(np && np[0] && np[0] != '0');
    if (!g->packed && reference_geometry(c)) {
        set_error("create: the padded-rows forward takes the BASELINE geometry; this model (window, "
                  "head_dim %d layers or PLE) runs packed batches only (unset E2MI_NOPACK)", c.full_head_dim);
        return fail();
    }
    if (ak == E2_ATTN_I8 && set_attention_i8(g, true)) return fail();
    if (check_hip(hipStreamSynchronize(g->stream), "create sync")) return fail();
    return g;
}

extern "C" e2mi_engine *e2mi_create(const e2_model *m) { return e2mi_create_rows(m, 0); }

// the geometry presets of the entries that take no e2_config (callers inside the reference, whose
// own e2.h defines e2_model and e2_config differently): 0 the BASELINE encoder, 1 the reference
// checkpoint's; n_layers and vocab > 0 override the preset's
static int preset_config(const char *who, int geometry, int n_layers, int vocab, e2_config *c) {
    if ((geometry != 0 && geometry != 1) || n_layers < 0 || vocab < 0) {
        set_error("%s: geometry %d (0 baseline, 1 reference) or negative override", who, geometry);
        return -1;
    }
    if (geometry == 0) e2_config_baseline(c);
    else e2_config_reference(c);
    if (n_layers > 0) c->n_layers = n_layers;
    if (vocab > 0) c->vocab = vocab;
    return 0;
}

// the engine straight from an E8CQ cache, for a caller that links only the e2mi_* names (a backend
// inside the reference, whose own e2.h and library define e2_model, e2_free and e2_last_error)
extern "C" e2mi_engine *e2mi_create_e8cq(const char *path, int geometry, int n_layers, int vocab,
                                         int max_rows) {
    e2_config c;
    if (!path) {
        set_error("create_e8cq: null path");
        return nullptr;
    }
    if (preset_config("create_e8cq", geometry, n_layers, vocab, &c)) return nullptr;
    e2_model *m = e2_load_e8cq(path, &c);
    if (!m) return nullptr;
    e2mi_engine *g = e2mi_create_rows(m, max_rows);
    e2_free(m);  // the engine holds its own device copy
    return g;
}

// the engine from tensors the caller holds in memory (the reference's e2_model walked by its
// adapter, e2_hip_create's upload of m->layers[l].q8_* as they are, forward.c:121-183)
extern "C" e2mi_engine *e2mi_create_tensors(const e2mi_tensor *tensors, int n_tensors, int geometry,
                                            int n_layers, int vocab, int max_rows) {
    e2_config c;
    if (preset_config("create_tensors", geometry, n_layers, vocab, &c)) return nullptr;
    e2_model *m = model_from_tensors(tensors, n_tensors, c);
    if (!m) return nullptr;
    e2mi_engine *g = e2mi_create_rows(m, max_rows);
    e2_free(m);  // borrowed views only: the engine holds its own device copy
    return g;
}

extern "C" const char *e2mi_device(e2mi_engine *g) { return g ? g->devname : ""; }

namespace e2mi {
// a call on stream s first drains the previous call's stream when it is another one (the calls
// share the workspace and the pinned staging arrays), and reads the id flag an asynchronous device
// call left behind
// the profiled call's event pairs, after its stream has synchronized: per-stage totals into the
// report (stages in order of first launch)
static void prof_flush(e2mi_engine *g) {
    if (g->pev.empty()) return;
    std::vector<std::string> names;
    std::vector<double> ms;
    std::vector<long> n;
    for (const ProfEv &e : g->pev) {
        float t = 0.f;
        if (hipEventElapsedTime(&t, e.a, e.b) != hipSuccess) t = 0.f;
        (void)hipEventDestroy(e.a);
        (void)hipEventDestroy(e.b);
        size_t i = 0;
        while (i < names.size() && names[i] != e.name) i++;
        if (i == names.size()) {
            names.push_back(e.name);
            ms.push_back(0.0);
            n.push_back(0);
        }
        ms[i] += t;
        n[i]++;
    }
    g->pev.clear();
    double total = 0.0;
    for (double t : ms) total += t;
    char line[256];
    snprintf(line, sizeof line, "[e2mi] kernel profile, one call (ms, total %.3f):\n", total);
    std::string text = line;
    for (size_t i = 0; i < names.size(); i++) {
        snprintf(line, sizeof line, "[e2mi]   %-20s %9.3f ms %6ld calls %8.4f ms/call %5.1f%%\n", names[i].c_str(),
                 ms[i], n[i], ms[i] / n[i], total > 0 ? 100.0 * ms[i] / total : 0.0);
        text += line;
    }
    g->prof_text += text;
    fputs(text.c_str(), stderr);
}

static int dump_file(const std::string &dir, const char *name, const void *dptr, size_t bytes) {
    if (!dptr || !bytes) return 0;
    std::vector<unsigned char> h(bytes);
    if (check_hip(hipMemcpy(h.data(), dptr, bytes, hipMemcpyDeviceToHost), "dump copy")) return -1;
    const std::string path = dir + "/" + name;
    FILE *f = fopen(path.c_str(), "wb");
    if (!f) {
        set_error("dump: cannot write %s", path.c_str());
        return -1;
    }
    const size_t w = fwrite(h.data(), 1, bytes, f);
    fclose(f);
    if (w != bytes) {
        set_error("dump: short write to %s", path.c_str());
        return -1;
    }
    return 0;
}

// the workspace of the last chunk after a call (its last layer's values; e2mi_set_layer_limit
// picks the layer): residual x, final-normed rows xn, the attention's f16 inputs, the quantized
// context and its scales, the last GEMM output tmp, the embeddings, and for packed batches each
// row's position and source index. File names carry the element type.
static int dump_workspace(e2mi_engine *g, hipStream_t s) {
    if (check_hip(hipStreamSynchronize(s), "dump sync")) return -1;
    const e2_config &c = g->cfg;
    const LayerGeom &L = g->layers[g->last_layer].geo;
    const size_t M = (size_t)g->last_M, qd = (size_t)c.n_heads * L.D, kvd = (size_t)L.KV * L.D;
    const std::string &d = g->dump_dir;
    int rc = dump_file(d, "e2mi_x.f32", g->x, M * c.hidden * 4) || dump_file(d, "e2mi_xn.f32", g->xn, M * c.hidden * 4) ||
             dump_file(d, "e2mi_tmp.f32", g->tmp, M * c.hidden * 4) || dump_file(d, "e2mi_q16.f16", g->q16, M * qd * 2) ||
             dump_file(d, "e2mi_k16.f16", g->k16, M * kvd * 2) || dump_file(d, "e2mi_vt16.f16", g->vt16, M * kvd * 2) ||
             dump_file(d, "e2mi_ctx_q.i8", g->cq, M * qd) || dump_file(d, "e2mi_ctx_s.f32", g->cs, M * (qd / 128) * 4) ||
             dump_file(d, "e2mi_out.f32", g->out, (size_t)g->last_B * g->dout * 4);
    if (!rc && g->last_pk) {
        // positions as the kernels read them; the row map of the last chunk's plan (host staging)
        rc = dump_file(d, "e2mi_pos.i32", g->pos, M * 4);
        FILE *f = rc ? nullptr : fopen((d + "/e2mi_rowmap.i32").c_str(), "wb");
        if (!rc && (!f || fwrite(g->h_rowmap, 4, M, f) != M)) {
            set_error("dump: cannot write %s/e2mi_rowmap.i32", d.c_str());
            rc = -1;
        }
        if (f) fclose(f);
    }
    return rc ? -1 : 0;
}

// after a call's last chunk: the profile (first call) and the dump (call E2MI_DUMP_CALL)
static int end_call(e2mi_engine *g, hipStream_t s) {
    if (g->prof_rec) {
        if (check_hip(hipStreamSynchronize(s), "profile sync")) return -1;
        prof_flush(g);
        g->prof_rec = false;
    }
    if (!g->dump_dir.empty() && (g->dump_call < 0 || g->calls == g->dump_call)) return dump_workspace(g, s);
    return 0;
}

// Read the flags of earlier device-entry calls in call order: those whose work has finished, or,
// with `wait` > 0, also waiting for the oldest `wait` calls. Stops at the first raised flag: returns
// its slot (cleared) and leaves the later calls unread; -1 when none was raised, -2 on a HIP error.
static int read_flags(e2mi_engine *g, int wait) {
    while (!g->unread.empty()) {
        const int k = g->unread.front();
        if (wait > 0) {
            if (check_hip(hipEventSynchronize(g->flag_ev[k]), "flag event")) return -2;
            wait--;
        } else {
            const hipError_t e = hipEventQuery(g->flag_ev[k]);
            if (e == hipErrorNotReady) break;
            if (check_hip(e, "flag event")) return -2;
        }
        g->unread.pop_front();
        if (g->h_rows[k] > 0) g->rows_seen[g->slot_shape[k]] = g->h_rows[k];
        if (g->h_flags[k]) {
            g->h_flags[k] = 0;
            return k;
        }
    }
    return -1;
}

static int flag_error(e2mi_engine *g, int slot, int own) {
    if (slot == -2) return -1;
    if (slot == own)
        set_error("text_embed_batch_device: a token id is outside [0,%d); the embeddings are not valid", g->cfg.vocab);
    else
        set_error("text_embed_batch_device: a previous asynchronous call had a token id outside [0,%d); its "
                  "embeddings are not valid", g->cfg.vocab);
    return -1;
}

static int begin_call(e2mi_engine *g, hipStream_t s) {
    if (g->last_stream && g->last_stream != s && check_hip(hipStreamSynchronize(g->last_stream), "previous call sync"))
        return -1;
    g->last_stream = s;
    const int k = read_flags(g, 0);
    if (k != -1) return flag_error(g, k, -1);
    for (const ProfEv &e : g->pev) (void)hipEventDestroy(e.a), (void)hipEventDestroy(e.b);  // a failed call's
    g->pev.clear();
    g->prof_rec = g->prof_on && g->calls == 0;
    return 0;
}
}  // namespace e2mi

extern "C" int e2mi_text_embed_batch(e2mi_engine *g, const int32_t *ids, const uint8_t *valid, int batch,
                                     int seq_len, float *out) {
    if (!g || !out) {
        set_error("text_embed_batch: null engine or output");
        return -1;
    }
    if (validate_batch(g, ids, batch, seq_len, true) || begin_call(g, g->stream)) return -1;
    const double t0 = now_ms();
    const int D = g->dout;
    for (int b0 = 0; b0 < batch;) {
        const size_t off = (size_t)b0 * seq_len;
        const uint8_t *vchunk = valid ? valid + off : nullptr;
        const int n = chunk_size(g, vchunk, b0, batch, seq_len);
        const size_t rows = (size_t)n * seq_len;
        int Mp = 0;
        if (g->packed) {
            Mp = plan_pack(g, vchunk, n, seq_len);
            if (Mp == 0) {
                // no valid token in the chunk: every sequence's embedding is the zero vector
                // (text.c:968-980), nothing to run
                memset(out + (size_t)b0 * D, 0, (size_t)n * D * 4);
                b0 += n;
                continue;
            }
            if (upload_pack(g, n, Mp, ids + off, g->stream)) return -1;
        } else {
            memcpy(g->h_ids, ids + off, rows * 4);
            for (size_t i = 0; i < rows; i++) g->h_valid[i] = valid ? (valid[off + i] != 0) : 1;
            if (check_hip(hipMemcpyAsync(g->ids, g->h_ids, rows * 4, hipMemcpyHostToDevice, g->stream), "ids H2D") ||
                check_hip(hipMemcpyAsync(g->valid, g->h_valid, rows, hipMemcpyHostToDevice, g->stream), "valid H2D"))
                return -1;
        }
        if (run_shape(g, n, seq_len, Mp, g->packed, g->stream) ||
            check_hip(hipMemcpyAsync(g->h_out, g->out, (size_t)n * D * 4, hipMemcpyDeviceToHost, g->stream), "out D2H") ||
            check_hip(hipStreamSynchronize(g->stream), "forward sync"))
            return -1;
        memcpy(out + (size_t)b0 * D, g->h_out, (size_t)n * D * 4);
        b0 += n;
    }
    g->calls++;
    g->last_ms = now_ms() - t0;
    return end_call(g, g->stream);
}

extern "C" int e2mi_text_embed(e2mi_engine *g, const int32_t *ids, int n_ids, float *out) {
    return e2mi_text_embed_batch(g, ids, nullptr, 1, n_ids, out);
}

extern "C" int e2mi_text_embed_batch_device(e2mi_engine *g, const int32_t *ids, const uint8_t *valid,
                                            int batch, int seq_len, float *out, e2mi_stream stream) {
    if (!g || !out || !valid) {
        set_error("text_embed_batch_device: null engine, mask or output");
        return -1;
    }
    if (validate_batch(g, ids, batch, seq_len, false)) return -1;
    hipStream_t s = stream ? (hipStream_t)stream : g->stream;
    if (begin_call(g, s)) return -1;
    const size_t rows = (size_t)batch * seq_len;
    const double t0 = now_ms();
    // ids are checked on the device, masked positions included, into this call's flag slot (only the
    // check kernel writes it; an event after it marks the flag final); the flag is read at the end
    // of this call, or, with a caller stream, by the first later call that finds the check finished
    // (a full ring waits for its oldest call)
    if ((int)g->unread.size() == e2mi_engine::kFlagSlots) {
        const int k = read_flags(g, 1);
        if (k != -1) return flag_error(g, k, -1);
    }
    const int slot = g->next_slot;
    g->next_slot = (slot + 1) % e2mi_engine::kFlagSlots;
    g->h_flags[slot] = 0;
    g->h_rows[slot] = 0;
    g->slot_shape[slot] = std::make_pair(batch, seq_len);
    if (launch_check_ids(s, ids, (long)rows, g->cfg.vocab, g->d_flags + slot) ||
        check_hip(hipEventRecord(g->flag_ev[slot], s), "flag event record"))
        return -1;
    g->unread.push_back(slot);
    if (!g->packed) {
        if ((long)batch * seq_len > g->R) {
            set_error("text_embed_batch_device: %d x %d rows exceed the engine's %d-row workspace",
                      batch, seq_len, g->R);
            return -1;
        }
        if (check_hip(hipMemcpyAsync(g->ids, ids, rows * 4, hipMemcpyDeviceToDevice, s), "ids D2D") ||
            check_hip(hipMemcpyAsync(g->valid, valid, rows, hipMemcpyDeviceToDevice, s), "valid D2D") ||
            run_shape(g, batch, seq_len, 0, false, s) ||
            check_hip(hipMemcpyAsync(out, g->out, (size_t)batch * g->dout * 4, hipMemcpyDeviceToDevice, s),
                      "out D2D"))
            return -1;
    } else if (const int cap = device_plan_rows(g, batch, seq_len)) {
        // planned on the device: the call reads nothing back, and one recorded forward serves every
        // mask of this batch shape (its kernels read the planned row count)
        plan_bind(g, plan_layout(g, batch, cap));
        g->split_now = false;
        PlanDevArgs pa{};
        pa.valid = valid;
        pa.ids = ids;
        pa.n = batch;
        pa.S = seq_len;
        pa.H = g->cfg.n_heads;
        pa.window = g->cfg.window;
        pa.div = 2;
        pa.full_div = 4;
        pa.slots = work_slots(g, batch, cap);
        pa.rowmap = g->rowmap;
        pa.pos = g->pos;
        pa.start = g->seq_start;
        pa.len = g->seq_len;
        pa.ids_out = g->ids;
        pa.work = g->work;
        pa.work_full = g->work_full;
        pa.rows = g->d_rows;
        pa.rows_host = g->d_rows_seen + slot;
        // the GEMM tiles follow the row count of this shape's latest finished call (the capacity
        // before one has finished): the same embeddings either way, one recorded forward per choice
        const auto seen = g->rows_seen.find(std::make_pair(batch, seq_len));
        const int est = seen != g->rows_seen.end() ? seen->second : cap;
        if (launch_plan_packed(s, pa) ||
            run_shape(g, batch, seq_len, cap, true, s, true, est, tile_signature(g, est)) ||
            check_hip(hipMemcpyAsync(out, g->out, (size_t)batch * g->dout * 4, hipMemcpyDeviceToDevice, s),
                      "out D2D"))
            return -1;
    } else {
        // the packing is planned on the host from the mask: one synchronous copy of B*S bytes
        // (which also drains earlier work on the stream that used the staging arrays)
        if (rows > g->mask_cap) {
            uint8_t *m = nullptr;
            if (check_hip(hipHostMalloc((void **)&m, rows), "pinned mask")) return -1;
            if (g->h_mask) (void)hipHostFree(g->h_mask);
            g->h_mask = m;
            g->mask_cap = rows;
        }
        if (check_hip(hipMemcpyAsync(g->h_mask, valid, rows, hipMemcpyDeviceToHost, s), "mask D2H") ||
            check_hip(hipStreamSynchronize(s), "mask sync"))
            return -1;
        for (int b0 = 0; b0 < batch;) {
            const size_t off = (size_t)b0 * seq_len;
            const int n = chunk_size(g, g->h_mask + off, b0, batch, seq_len);
            const int Mp = plan_pack(g, g->h_mask + off, n, seq_len);
            if (Mp == 0) {
                // no valid token in the chunk: zero embeddings (a fill kernel, capturable)
                if (launch_zero_f32(s, out + (size_t)b0 * g->dout, (long)n * g->dout)) return -1;
            } else if (upload_pack(g, n, Mp, nullptr, s) ||
                       e2mi_gather_ids(s, ids + off, g->rowmap, Mp, g->ids) ||
                       run_shape(g, n, seq_len, Mp, true, s) ||
                       check_hip(hipMemcpyAsync(out + (size_t)b0 * g->dout, g->out, (size_t)n * g->dout * 4,
                                                hipMemcpyDeviceToDevice, s), "out D2D")) {
                return -1;
            }
            b0 += n;
            // the staging arrays are reused by the next chunk
            if (b0 < batch && check_hip(hipStreamSynchronize(s), "chunk sync")) return -1;
        }
    }
    if (!stream) {
        if (check_hip(hipStreamSynchronize(s), "forward sync")) return -1;
        const int k = read_flags(g, (int)g->unread.size());
        if (k != -1) return flag_error(g, k, slot);
    }
    g->calls++;
    g->last_ms = now_ms() - t0;
    return end_call(g, s);
}

// ------------------------------------------------------------------ e2.h text entries
// (include/e2.h:25,35-36): the model's engine, created at the first call and owned by the model
static e2mi_engine *model_engine(e2_model *m) {
    if (!m) {
        set_error("text_embed: null model");
        return nullptr;
    }
    void **slot = e2mi::model_engine_slot(m);
    if (!*slot) {
        e2mi_engine *g = e2mi_create(m);
        if (!g) return nullptr;
        *slot = g;
        e2mi::model_set_engine_free(m, [](void *p) { e2mi_destroy((e2mi_engine *)p); });
    }
    return (e2mi_engine *)*slot;
}

extern "C" int e2_text_embed_batch(e2_model *m, const int32_t *ids, const uint8_t *valid, int batch,
                                   int seq_len, float *out) {
    e2mi_engine *g = model_engine(m);
    return g ? e2mi_text_embed_batch(g, ids, valid, batch, seq_len, out) : -1;
}

extern "C" int e2_text_embed(e2_model *m, const int32_t *ids, int n_ids, float *out768) {
    return e2_text_embed_batch(m, ids, nullptr, 1, n_ids, out768);
}

extern "C" int e2mi_set_packing(e2mi_engine *g, int on) {
    if (!g) {
        set_error("set_packing: null engine");
        return -1;
    }
    if (!on && reference_geometry(g->cfg)) {
        set_error("set_packing: this model (window, per-layer head_dim or PLE) runs packed batches only");
        return -1;
    }
    if (g->stream) (void)hipStreamSynchronize(g->stream);
    if (g->last_stream) (void)hipStreamSynchronize(g->last_stream);
    g->packed = on != 0;
    return 0;
}

extern "C" int e2mi_set_device_plan(e2mi_engine *g, int on) {
    if (!g) {
        set_error("set_device_plan: null engine");
        return -1;
    }
    if (g->stream) (void)hipStreamSynchronize(g->stream);
    if (g->last_stream) (void)hipStreamSynchronize(g->last_stream);
    g->device_plan = on != 0;
    return 0;
}

extern "C" int e2mi_set_attention(e2mi_engine *g, int kind) {
    if (!g || (kind != E2_ATTN_F16 && kind != E2_ATTN_I8)) {
        set_error("set_attention: null engine or kind %d (f16 = %d, i8 = %d)", kind, (int)E2_ATTN_F16,
                  (int)E2_ATTN_I8);
        return -1;
    }
    if (g->stream) (void)hipStreamSynchronize(g->stream);
    if (g->last_stream) (void)hipStreamSynchronize(g->last_stream);
    return set_attention_i8(g, kind == E2_ATTN_I8);
}

extern "C" const char *e2mi_profile_text(const e2mi_engine *g) { return g ? g->prof_text.c_str() : ""; }

extern "C" int e2mi_set_attention_split(e2mi_engine *g, int mode) {
    if (!g || mode < 0 || mode > 2) {
        set_error("set_attention_split: null engine or mode %d (0 never, 1 always, 2 auto)", mode);
        return -1;
    }
    if (g->stream) (void)hipStreamSynchronize(g->stream);
    if (g->last_stream) (void)hipStreamSynchronize(g->last_stream);
    g->split_mode = mode;
    return 0;
}

extern "C" int e2mi_stats(e2mi_engine *g, long *calls, long *kernels_last, double *last_ms) {
    if (!g) {
        set_error("stats: null engine");
        return -1;
    }
    if (calls) *calls = g->calls;
    if (kernels_last) *kernels_last = g->kernels_last;
    if (last_ms) *last_ms = g->last_ms;
    return 0;
}

extern "C" int e2mi_set_layer_limit(e2mi_engine *g, int n_layers) {
    if (!g || n_layers < 0) {
        set_error("set_layer_limit: null engine or negative limit");
        return -1;
    }
    g->layer_limit = n_layers;
    for (auto &kv : g->graphs) (void)hipGraphExecDestroy(kv.second);
    g->graphs.clear();
    return 0;
}
