// model.cpp — host-side model container: BASELINE geometry, seeded synthetic int8 weights, and
// the E8CQ packed int8 cache (the reference's q8cache.c v1 on-disk format, restated).
#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <map>
#include <string>
#include <thread>
#include <vector>

#include "../../include/e2.h"
#include "../../include/e2mi.h"
#include "common.h"
#include "model_internal.h"

struct e2mi_model {
    e2_config cfg;
    std::map<std::string, e2mi::HostQ8W> q8;
    std::map<std::string, e2mi::F32T> f32;
    void *map = nullptr;
    size_t map_size = 0;
    void *engine = nullptr;                    // created by e2_text_embed*, destroyed by e2_free
    void (*engine_free)(void *) = nullptr;
};

namespace e2mi {

// ------------------------------------------------------------------ names (e2.c:306-402)
std::string layer_name(int l, const char *suffix) {
    char b[128];
    snprintf(b, sizeof b, "language_model.layers.%d.%s", l, suffix);
    return b;
}
static const char *kEmbed = "language_model.embed_tokens.weight";
static const char *kFinalNorm = "language_model.norm.weight";
// the reference checkpoint's extra tensors (e2.c:316-381)
static const char *kPleModel = "language_model.ple.per_layer_model_projection.weight";
static const char *kPleNorm = "language_model.ple.per_layer_projection_norm.weight";
static const char *kEmbedProj = "language_model.embedding_projection.weight";
static const char *kLayerScalar = "layer_scalar";
static const char *kQ8Suffix[9] = {"self_attn.q_proj.weight", "self_attn.k_proj.weight",
                                   "self_attn.v_proj.weight", "self_attn.o_proj.weight",
                                   "mlp.gate_proj.weight", "mlp.up_proj.weight",
                                   "mlp.down_proj.weight", "ple_block.per_layer_input_gate.weight",
                                   "ple_block.per_layer_projection.weight"};
static const char *kNormSuffix[7] = {"input_layernorm.weight", "post_attention_layernorm.weight",
                                     "pre_feedforward_layernorm.weight",
                                     "post_feedforward_layernorm.weight", "self_attn.q_norm.weight",
                                     "self_attn.k_norm.weight",
                                     "ple_block.post_per_layer_input_norm.weight"};

// int8 weights and norms of layer l: 7 without PLE, 9 with; 6 norms without, 7 with
static int n_q8(const e2_config &c) { return c.ple_dim > 0 ? 9 : 7; }
static int n_norm(const e2_config &c) { return c.ple_dim > 0 ? 7 : 6; }

// (N, K) of weight s of layer l; norm s length
static void q8_shape(const e2_config &c, int l, int s, int *N, int *K) {
    const LayerGeom g = layer_geom(c, l);
    const int qd = c.n_heads * g.D, kvd = g.KV * g.D;
    const int Ns[9] = {qd, kvd, kvd, c.hidden, c.ffn, c.ffn, c.hidden, c.ple_dim, c.hidden};
    const int Ks[9] = {c.hidden, c.hidden, c.hidden, qd, c.hidden, c.hidden, c.ffn, c.hidden, c.ple_dim};
    *N = Ns[s];
    *K = Ks[s];
}
static int norm_len(const e2_config &c, int l, int s) {
    return (s == 4 || s == 5) ? layer_geom(c, l).D : c.hidden;
}

// ------------------------------------------------------------------ packing (int8.h:14-22)
static void pack_rows(const int8_t *rm, int N, int K, HostQ8W &q) {
    q.N = N;
    q.K = K;
    q.nb = (K + kQBlock - 1) / kQBlock;
    q.Npad = (N + 7) & ~7;
    const int kq = (K + 3) / 4;
    q.ow.assign((size_t)q.Npad * kq * 4, 0);
    q.ob.assign((size_t)q.nb * q.Npad, 0);
    for (int n = 0; n < N; n++)
        for (int k = 0; k < K; k++) {
            const int8_t v = rm[(size_t)n * K + k];
            q.ow[(size_t)(n >> 3) * kq * 32 + (size_t)(k >> 2) * 32 + (n & 7) * 4 + (k & 3)] = v;
            q.ob[(size_t)(k / kQBlock) * q.Npad + n] += v;
        }
    q.w = q.ow.data();
    q.bsq = q.ob.data();
}

// ------------------------------------------------------------------ synthetic weights
// The reference tests' LCG (test_scalar_kernels.c:26-28), one stream per (tensor, row).
struct Lcg {
    uint32_t s;
    uint32_t next() { return s = s * 1664525u + 1013904223u; }
    double unit() { return ((next() >> 8) + 0.5) * (1.0 / 16777216.0); }  // (0, 1)
    int i8() { return (int)((next() >> 8) % 255u) - 127; }
    float normal(double sd) {  // Box-Muller
        const double u1 = unit(), u2 = unit();
        return (float)(sd * sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
    }
};
static uint32_t row_seed(uint64_t seed, int tensor, long row) {
    uint64_t z = seed ^ ((uint64_t)(tensor + 1) << 40) ^ (uint64_t)row * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;  // splitmix64 finaliser
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return (uint32_t)(z ^ (z >> 31));
}

template <class F>
static void parallel_rows(long n, F f) {
    int nt = (int)std::thread::hardware_concurrency();
    nt = nt < 1 ? 1 : (nt > 16 ? 16 : nt);
    if (n < 4096) nt = 1;
    std::vector<std::thread> th;
    for (int t = 0; t < nt; t++)
        th.emplace_back([=] {
            for (long r = t; r < n; r += nt) f(r);
        });
    for (auto &x : th) x.join();
}

static void synth_q8(HostQ8W &q, int N, int K, uint64_t seed, int tensor) {
    std::vector<int8_t> rm((size_t)N * K);
    q.os.assign((size_t)((N + 7) & ~7), 0.f);
    parallel_rows(N, [&](long n) {
        Lcg g{row_seed(seed, tensor, n)};
        for (int k = 0; k < K; k++) rm[(size_t)n * K + k] = (int8_t)g.i8();
        q.os[n] = (float)(0.001 + 0.019 * g.unit());
    });
    pack_rows(rm.data(), N, K, q);
    q.scale = q.os.data();
}

static void synth_f32(F32T &t, long rows, int cols, double mean, double sd, uint64_t seed,
                      int tensor) {
    t.own.resize((size_t)rows * cols);
    t.ndim = rows > 1 ? 2 : 1;
    t.dims[0] = rows > 1 ? rows : cols;
    t.dims[1] = rows > 1 ? cols : 0;
    float *p = t.own.data();
    parallel_rows(rows, [&](long r) {
        Lcg g{row_seed(seed, tensor, r)};
        for (int c = 0; c < cols; c++) p[(size_t)r * cols + c] = (float)mean + g.normal(sd);
    });
    t.p = t.own.data();
}

static bool config_ok(const e2_config &c) {
    if (c.n_layers < 1 || c.hidden <= 0 || c.hidden % 128 || c.ffn <= 0 || c.ffn % 128 ||
        c.n_heads <= 0 || c.n_kv_heads <= 0 || c.n_heads % c.n_kv_heads || c.head_dim != 256 ||
        c.vocab <= 0 || c.max_seq <= 0 || c.max_seq > 2048 || c.hidden > 1280 ||
        (c.n_heads * c.head_dim) % 128) {
        set_error("config: unsupported geometry (hidden/ffn multiples of 128, hidden <= 1280, "
                  "head_dim 256, H %% KV == 0, 1 <= max_seq <= 2048)");
        return false;
    }
    // the attention work lists carry the head in 4 bits (b | h << 16 | part << 20 | ... | qb << 24)
    if (c.n_heads > 15) {
        set_error("config: at most 15 query heads (the attention work entries hold the head in 4 bits)");
        return false;
    }
    if (c.ple_dim < 0 || c.ple_dim % 128 || c.ple_dim > 1280 || c.out_dim < 0 || c.out_dim % 128 ||
        c.out_dim > 1280 || c.window < 0 || c.full_period < 0 || (long)c.n_layers * c.ple_dim > (1 << 20) ||
        (c.full_period > 0 && (c.full_kv_heads <= 0 || c.n_heads % c.full_kv_heads ||
                               (c.full_head_dim != 256 && c.full_head_dim != 512) ||
                               !(c.rope_theta_full > 0.f))) ||
        (c.ple_dim > 0 && !(c.ple_scale > 0.f)) || !(c.attn_scale > 0.f) || !(c.attn_scale < INFINITY)) {
        set_error("config: unsupported extras (ple_dim/out_dim multiples of 128 up to 1280, "
                  "window >= 0, full layers with head_dim 256 or 512 and H %% kv == 0, attn_scale > 0)");
        return false;
    }
    return true;
}

// ------------------------------------------------------------------ E8CQ (q8cache.c:1-13)
constexpr uint32_t kMagic = 0x51433845u;  // "E8CQ"
constexpr uint32_t kVersion = 1u;
enum { KIND_BF16 = 1, KIND_F32 = 2, KIND_Q8W = 3 };
struct Entry {  // 152 bytes, the reference's q8c_entry
    char name[96];
    uint32_t kind, ndim;
    int64_t dims[4];
    uint64_t nbytes, off;
};
static_assert(sizeof(Entry) == 152, "E8CQ index entry is 152 bytes");

// The payload an index entry's kind and dims imply, in bytes (the format: kinds 1 and 2 are dense
// bf16 / f32 arrays of the product of their dims; kind 3 is a packed int8 weight whose dims are
// {N, K, blocks of 128 along K, N rounded up to 8} and whose payload is the interleaved bytes
// [Npad][ceil(K/4) * 4], then Npad f32 scales, then blocks x Npad int32 sums). 0 with a reason when
// the dims are not those of any valid tensor of that kind.
static uint64_t implied_bytes(const Entry &e, const char **why) {
    if (e.kind == KIND_Q8W) {
        const int64_t N = e.dims[0], K = e.dims[1];
        const bool shape = N > 0 && K > 0 && N <= (1 << 30) && K <= (1 << 30) &&
                           e.dims[2] == (K + kQBlock - 1) / kQBlock && e.dims[3] == ((N + 7) & ~7ll);
        if (!shape) {
            *why = "packed int8 dims are not {N, K, ceil(K/128), ceil8(N)} with 0 < N, K <= 2^30";
            return 0;
        }
        const uint64_t rows = (uint64_t)e.dims[3], quads = (uint64_t)(K + 3) / 4;
        return rows * quads * 4 + rows * 4 + (uint64_t)e.dims[2] * rows * 4;
    }
    uint64_t n = e.kind == KIND_BF16 ? 2 : 4;
    for (uint32_t d = 0; d < e.ndim; d++) {
        if (e.dims[d] < 0) {
            *why = "a dimension is negative";
            return 0;
        }
        if (__builtin_mul_overflow(n, (uint64_t)e.dims[d], &n)) {
            *why = "the dims multiply past 64 bits";
            return 0;
        }
    }
    return n;
}

// One index entry, checked before anything reads through it: a usable name, a known kind and rank,
// a payload placed inside the data area (16-byte aligned, after the header, before the index) and
// sized exactly as its kind and dims imply.
static bool entry_ok(const Entry &e, uint64_t idx_off, const char *path) {
    const void *nul = memchr(e.name, 0, sizeof e.name);
    if (!nul || nul == e.name) {
        set_error("%s: index entry without a NUL-terminated name", path);
        return false;
    }
    const bool rank_ok = e.kind == KIND_Q8W ? e.ndim == 4 : e.ndim <= 4;
    if (e.kind < KIND_BF16 || e.kind > KIND_Q8W || !rank_ok) {
        set_error("%s: %.64s: kind %u with %u dims is not a tensor this format stores", path, e.name, e.kind, e.ndim);
        return false;
    }
    const uint64_t end = e.off + e.nbytes;
    if (e.off % 16 || e.off < 16 || end < e.off || end > idx_off) {
        set_error("%s: %.64s: payload [%llu, +%llu) is not a 16-byte aligned range of the data area", path,
                  e.name, (unsigned long long)e.off, (unsigned long long)e.nbytes);
        return false;
    }
    const char *why = nullptr;
    const uint64_t want = implied_bytes(e, &why);
    if (why) {
        set_error("%s: %.64s: %s", path, e.name, why);
        return false;
    }
    if (e.nbytes != want) {
        set_error("%s: %.64s: %llu payload bytes where the dims call for %llu", path, e.name,
                  (unsigned long long)e.nbytes, (unsigned long long)want);
        return false;
    }
    return true;
}

static bool write_all(int fd, const void *p, size_t n) {
    const char *c = (const char *)p;
    while (n) {
        const ssize_t w = write(fd, c, n);
        if (w <= 0) return false;
        c += w;
        n -= (size_t)w;
    }
    return true;
}

}  // namespace e2mi

using namespace e2mi;

extern "C" const char *e2_last_error(void) { return e2mi_last_error(); }

extern "C" void e2_config_baseline(e2_config *c) {
    if (!c) return;
    memset(c, 0, sizeof *c);
    c->n_layers = 24;
    c->hidden = 768;
    c->ffn = 1152;
    c->n_heads = 3;
    c->n_kv_heads = 1;
    c->head_dim = 256;
    c->vocab = 262144;
    c->max_seq = 2048;
    c->rms_eps = 1e-6f;
    c->rope_theta = 10000.0f;
    c->embed_scale = sqrtf(768.0f);
    c->attn_scale = 1.0f;
}

extern "C" void e2_config_reference(e2_config *c) {
    if (!c) return;
    memset(c, 0, sizeof *c);
    c->n_layers = 24;
    c->hidden = 512;
    c->ffn = 2048;
    c->n_heads = 4;
    c->n_kv_heads = 2;
    c->head_dim = 256;
    c->vocab = 262144;
    c->max_seq = 2048;
    c->rms_eps = 1e-6f;
    c->rope_theta = 10000.0f;
    c->embed_scale = sqrtf(512.0f);
    c->attn_scale = 1.0f;
    c->ple_dim = 512;
    c->out_dim = 768;
    c->window = 512;
    c->full_period = 6;
    c->full_head_dim = 512;
    c->full_kv_heads = 1;
    c->rope_theta_full = 1000000.0f;
    c->ple_scale = 1.0f / sqrtf(512.0f);
}

extern "C" e2_model *e2_model_synthetic(const e2_config *c, uint64_t seed) {
    if (!c || !config_ok(*c)) {
        if (!c) set_error("model_synthetic: null config");
        return nullptr;
    }
    e2_model *m = new (std::nothrow) e2_model();
    if (!m) {
        set_error("oom: model");
        return nullptr;
    }
    m->cfg = *c;
    try {
        int t = 0;
        synth_f32(m->f32[kEmbed], c->vocab, c->hidden, 0.0, 0.02, seed, t++);
        synth_f32(m->f32[kFinalNorm], 1, c->hidden, 1.0, 0.05, seed, t++);
        for (int l = 0; l < c->n_layers; l++) {
            for (int s = 0; s < 7; s++) {
                int N, K;
                q8_shape(*c, l, s, &N, &K);
                synth_q8(m->q8[layer_name(l, kQ8Suffix[s])], N, K, seed, t++);
            }
            for (int s = 0; s < 6; s++)
                synth_f32(m->f32[layer_name(l, kNormSuffix[s])], 1, norm_len(*c, l, s), 1.0, 0.05, seed, t++);
        }
        // the reference geometry's extras draw from their own streams, so the BASELINE tensors
        // are the same whichever geometry fields are set
        int te = 1 << 20;
        if (c->ple_dim > 0) {
            synth_q8(m->q8[kPleModel], c->n_layers * c->ple_dim, c->hidden, seed, te++);
            synth_f32(m->f32[kPleNorm], 1, c->ple_dim, 1.0, 0.05, seed, te++);
            for (int l = 0; l < c->n_layers; l++) {
                for (int s = 7; s < 9; s++) {
                    int N, K;
                    q8_shape(*c, l, s, &N, &K);
                    synth_q8(m->q8[layer_name(l, kQ8Suffix[s])], N, K, seed, te++);
                }
                synth_f32(m->f32[layer_name(l, kNormSuffix[6])], 1, c->hidden, 1.0, 0.05, seed, te++);
                synth_f32(m->f32[layer_name(l, kLayerScalar)], 1, 1, 1.0, 0.05, seed, te++);
            }
        }
        if (c->out_dim > 0) synth_q8(m->q8[kEmbedProj], c->out_dim, c->hidden, seed, te++);
    } catch (...) {
        delete m;
        set_error("oom: synthetic weights");
        return nullptr;
    }
    return m;
}

namespace e2mi {
void **model_engine_slot(e2_model *m) { return &m->engine; }
void model_set_engine_free(e2_model *m, void (*destroy)(void *)) { m->engine_free = destroy; }
}  // namespace e2mi

extern "C" void e2_free(e2_model *m) {
    if (!m) return;
    if (m->engine && m->engine_free) m->engine_free(m->engine);
    if (m->map) munmap(m->map, m->map_size);
    delete m;
}

extern "C" int e2_model_config(const e2_model *m, e2_config *out) {
    if (!m || !out) {
        set_error("model_config: null argument");
        return -1;
    }
    *out = m->cfg;
    return 0;
}

extern "C" int e2_model_tensor(const e2_model *m, const char *name, e2_tensor_view *v) {
    if (!m || !name || !v) {
        set_error("model_tensor: null argument");
        return -1;
    }
    memset(v, 0, sizeof *v);
    auto q = m->q8.find(name);
    if (q != m->q8.end()) {
        const HostQ8W &w = q->second;
        v->kind = KIND_Q8W;
        v->ndim = 4;
        v->dims[0] = w.N;
        v->dims[1] = w.K;
        v->dims[2] = w.nb;
        v->dims[3] = w.Npad;
        v->data = w.w;
        v->scale = w.scale;
        v->bsq = w.bsq;
        v->nbytes = w.bytes();
        return 0;
    }
    auto f = m->f32.find(name);
    if (f != m->f32.end()) {
        v->kind = KIND_F32;
        v->ndim = f->second.ndim;
        memcpy(v->dims, f->second.dims, sizeof v->dims);
        v->data = f->second.p;
        v->nbytes = f->second.count() * sizeof(float);
        return 0;
    }
    set_error("model_tensor: %s: not in the model", name);
    return -1;
}

extern "C" int e2_save_e8cq(const e2_model *m, const char *path) {
    if (!m || !path) {
        set_error("save_e8cq: null argument");
        return -1;
    }
    std::string tmp = std::string(path) + ".tmp.XXXXXX";
    std::vector<char> tb(tmp.begin(), tmp.end());
    tb.push_back(0);
    const int fd = mkstemp(tb.data());
    if (fd < 0) {
        set_error("save_e8cq: cannot create %s", tb.data());
        return -1;
    }
    std::vector<Entry> idx;
    uint64_t off = 16;
    const uint32_t hdr0[4] = {kMagic, kVersion, 0, 0};
    bool ok = write_all(fd, hdr0, sizeof hdr0);
    auto pad = [&]() {
        static const char z[16] = {0};
        const size_t p = (16 - (off & 15)) & 15;
        if (p) ok = ok && write_all(fd, z, p);
        off += p;
    };
    auto begin = [&](const std::string &name, uint32_t kind, uint32_t ndim, const int64_t *dims) {
        Entry e;
        memset(&e, 0, sizeof e);
        if (name.size() >= sizeof e.name) {
            set_error("save_e8cq: tensor name too long: %s", name.c_str());
            ok = false;
        }
        snprintf(e.name, sizeof e.name, "%s", name.c_str());
        e.kind = kind;
        e.ndim = ndim;
        for (uint32_t i = 0; i < ndim; i++) e.dims[i] = dims[i];
        e.off = off;
        idx.push_back(e);
    };
    auto bytes = [&](const void *p, size_t n) {
        ok = ok && write_all(fd, p, n);
        off += n;
        idx.back().nbytes += n;
    };
    for (auto &kv : m->q8) {  // q8c_put_q8w (q8cache.c:163-181): w | scale | bsq
        const HostQ8W &w = kv.second;
        const int64_t dims[4] = {w.N, w.K, w.nb, w.Npad};
        begin(kv.first, KIND_Q8W, 4, dims);
        bytes(w.w, w.bytes());
        bytes(w.scale, (size_t)w.Npad * 4);
        bytes(w.bsq, (size_t)w.nb * w.Npad * 4);
        pad();
    }
    for (auto &kv : m->f32) {
        begin(kv.first, KIND_F32, (uint32_t)kv.second.ndim, kv.second.dims);
        bytes(kv.second.p, kv.second.count() * 4);
        pad();
    }
    if (off > UINT32_MAX || idx.size() > UINT32_MAX) {
        set_error("save_e8cq: the model exceeds the v1 32-bit index format");
        ok = false;
    }
    const uint32_t hdr[4] = {kMagic, kVersion, (uint32_t)idx.size(), (uint32_t)off};
    ok = ok && write_all(fd, idx.data(), idx.size() * sizeof(Entry));
    ok = ok && lseek(fd, 0, SEEK_SET) == 0 && write_all(fd, hdr, sizeof hdr);
    ok = ok && fsync(fd) == 0;
    ok = (close(fd) == 0) && ok;
    if (ok && rename(tb.data(), path) != 0) ok = false;
    if (!ok) {
        unlink(tb.data());
        if (!strstr(e2mi_last_error(), "save_e8cq")) set_error("save_e8cq: write/commit of %s failed", path);
        return -1;
    }
    return 0;
}

static float bf16f(uint16_t v) {
    const uint32_t u = (uint32_t)v << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

// Every tensor the text tower of geometry `cf` reads is present with its shape (e2.c:306-402 names,
// q8_shape / norm_len sizes); `who` prefixes the message.
static bool geometry_ok(const e2_model *m, const e2_config &cf, const char *who) {
    auto need_f32 = [&](const std::string &name, size_t count) {
        auto it = m->f32.find(name);
        if (it == m->f32.end() || it->second.count() != count) {
            set_error("%s: %s missing or mis-shaped", who, name.c_str());
            return false;
        }
        return true;
    };
    auto need_q8 = [&](const std::string &name, int N, int K) {
        auto it = m->q8.find(name);
        if (it == m->q8.end() || it->second.N != N || it->second.K != K) {
            set_error("%s: %s missing or mis-shaped", who, name.c_str());
            return false;
        }
        return true;
    };
    if (!need_f32(kEmbed, (size_t)cf.vocab * cf.hidden) || !need_f32(kFinalNorm, (size_t)cf.hidden))
        return false;
    // the PLE projection holds ple_dim rows per layer of the checkpoint; a model run on its first
    // n_layers layers (the reference's n_layers below 24) reads the first n_layers slices
    if (cf.ple_dim > 0) {
        auto it = m->q8.find(kPleModel);
        if (it == m->q8.end() || it->second.K != cf.hidden || it->second.N % cf.ple_dim ||
            it->second.N < cf.n_layers * cf.ple_dim) {
            set_error("%s: %s missing or mis-shaped", who, kPleModel);
            return false;
        }
        if (!need_f32(kPleNorm, (size_t)cf.ple_dim)) return false;
    }
    if (cf.out_dim > 0 && !need_q8(kEmbedProj, cf.out_dim, cf.hidden)) return false;
    for (int l = 0; l < cf.n_layers; l++) {
        for (int s = 0; s < n_q8(cf); s++) {
            int N, K;
            q8_shape(cf, l, s, &N, &K);
            if (!need_q8(layer_name(l, kQ8Suffix[s]), N, K)) return false;
        }
        for (int s = 0; s < n_norm(cf); s++)
            if (!need_f32(layer_name(l, kNormSuffix[s]), (size_t)norm_len(cf, l, s))) return false;
        if (cf.ple_dim > 0 && !need_f32(layer_name(l, kLayerScalar), 1)) return false;
    }
    return true;
}

extern "C" e2_model *e2_load_e8cq(const char *path, const e2_config *c) {
    if (!path || !c || !config_ok(*c)) {
        if (!path || !c) set_error("load_e8cq: null argument");
        return nullptr;
    }
    const int fd = open(path, O_RDONLY);
    if (fd < 0) {
        set_error("%s: cannot open", path);
        return nullptr;
    }
    struct stat st;
    if (fstat(fd, &st) || st.st_size < 16) {
        close(fd);
        set_error("%s: too small", path);
        return nullptr;
    }
    const size_t size = (size_t)st.st_size;
    void *map = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) {
        set_error("%s: mmap failed", path);
        return nullptr;
    }
    e2_model *m = new (std::nothrow) e2_model();
    if (!m) {
        munmap(map, size);
        set_error("oom: model");
        return nullptr;
    }
    m->cfg = *c;
    m->map = map;
    m->map_size = size;
    const uint8_t *base = (const uint8_t *)map;
    const uint32_t *h = (const uint32_t *)base;
    const uint64_t io = h[3];
    const uint32_t n = h[2];
    auto fail = [&](void) -> e2_model * {
        e2_free(m);
        return nullptr;
    };
    if (h[0] != kMagic || h[1] != kVersion) {
        set_error("%s: bad magic/version", path);
        return fail();
    }
    if (io < 16 || (io & 15) || io > size || (uint64_t)n > (size - io) / sizeof(Entry)) {
        set_error("%s: truncated or misaligned index", path);
        return fail();
    }
    const Entry *idx = (const Entry *)(base + io);
    for (uint32_t i = 0; i < n; i++)
        if (!entry_ok(idx[i], io, path)) return fail();
    for (uint32_t i = 0; i < n; i++) {
        const Entry &e = idx[i];
        const uint8_t *p = base + e.off;
        if (e.kind == KIND_Q8W) {
            HostQ8W &w = m->q8[e.name];
            w.N = (int)e.dims[0];
            w.K = (int)e.dims[1];
            w.nb = (int)e.dims[2];
            w.Npad = (int)e.dims[3];
            w.w = (const int8_t *)p;
            w.scale = (const float *)(p + w.bytes());
            w.bsq = (const int32_t *)(p + w.bytes() + (size_t)w.Npad * 4);
        } else {
            F32T &t = m->f32[e.name];
            t.ndim = (int)e.ndim;
            for (uint32_t d = 0; d < e.ndim; d++) t.dims[d] = e.dims[d];
            if (e.kind == KIND_F32) {
                t.p = (const float *)p;
            } else {  // bf16 tensors (the reference keeps norm scales in bf16)
                t.own.resize(e.nbytes / 2);
                for (size_t j = 0; j < t.own.size(); j++) t.own[j] = bf16f(((const uint16_t *)p)[j]);
                t.p = t.own.data();
            }
        }
    }
    if (!geometry_ok(m, *c, path)) return fail();
    return m;
}

namespace e2mi {
// A model over tensors the caller holds in memory (e2mi_create_tensors): int8 weights and f32
// tensors are borrowed for the engine's upload, bf16 ones widened to f32 (exact: a bf16 value is the
// high half of its f32). Checked like a cache: every tensor of the geometry present with its shape.
e2_model *model_from_tensors(const e2mi_tensor *t, int n, const e2_config &c) {
    if (!config_ok(c)) return nullptr;
    if (!t || n <= 0) {
        set_error("create_tensors: no tensors");
        return nullptr;
    }
    e2_model *m = new (std::nothrow) e2_model();
    if (!m) {
        set_error("oom: model");
        return nullptr;
    }
    m->cfg = c;
    // bf16 tensors are widened only once every shape has been checked: nothing past a shape the
    // geometry does not expect is ever read
    std::vector<std::pair<F32T *, const uint16_t *>> widen;
    try {
        for (int i = 0; i < n; i++) {
            const e2mi_tensor &x = t[i];
            if (!x.name || !x.name[0] || !x.data) {
                set_error("create_tensors: tensor %d has no name or no data", i);
                e2_free(m);
                return nullptr;
            }
            if (m->q8.count(x.name) || m->f32.count(x.name)) {
                set_error("create_tensors: %s given twice", x.name);
                e2_free(m);
                return nullptr;
            }
            if (x.kind == E2MI_TENSOR_Q8W) {
                if (x.N <= 0 || x.K <= 0 || x.Npad != ((x.N + 7) & ~7) || !x.scale) {
                    set_error("create_tensors: %s: int8 weight with N %d, K %d, Npad %d or no scales", x.name,
                              x.N, x.K, x.Npad);
                    e2_free(m);
                    return nullptr;
                }
                HostQ8W &w = m->q8[x.name];
                w.N = x.N;
                w.K = x.K;
                w.nb = x.nblocks;
                w.Npad = x.Npad;
                w.w = (const int8_t *)x.data;
                w.scale = x.scale;
                w.bsq = x.bsq;
            } else if (x.kind == E2MI_TENSOR_F32 || x.kind == E2MI_TENSOR_BF16) {
                if (x.N <= 0 || x.K <= 0) {
                    set_error("create_tensors: %s: %d x %d", x.name, x.N, x.K);
                    e2_free(m);
                    return nullptr;
                }
                F32T &f = m->f32[x.name];
                f.ndim = 2;
                f.dims[0] = x.N;
                f.dims[1] = x.K;
                if (x.kind == E2MI_TENSOR_F32) f.p = (const float *)x.data;
                else widen.push_back({&f, (const uint16_t *)x.data});
            } else {
                set_error("create_tensors: %s: kind %d (bf16 1, f32 2, q8w 3)", x.name, x.kind);
                e2_free(m);
                return nullptr;
            }
        }
    } catch (...) {
        e2_free(m);
        set_error("oom: create_tensors");
        return nullptr;
    }
    if (!geometry_ok(m, c, "create_tensors")) {
        e2_free(m);
        return nullptr;
    }
    try {
        for (auto &w : widen) {
            F32T &f = *w.first;
            f.own.resize(f.count());
            const uint16_t *src = w.second;
            float *dst = f.own.data();
            const long cols = (long)f.dims[1];
            parallel_rows((long)f.dims[0], [=](long r) {
                for (long j = 0; j < cols; j++) dst[r * cols + j] = bf16f(src[r * cols + j]);
            });
            f.p = dst;
        }
    } catch (...) {
        e2_free(m);
        set_error("oom: create_tensors");
        return nullptr;
    }
    return m;
}
}  // namespace e2mi

// ------------------------------------------------------------------ accessors for the engine
namespace e2mi {
const HostQ8W *model_q8(const e2_model *m, const std::string &name) {
    auto it = m->q8.find(name);
    return it == m->q8.end() ? nullptr : &it->second;
}
const float *model_f32(const e2_model *m, const std::string &name, size_t count) {
    auto it = m->f32.find(name);
    return (it == m->f32.end() || it->second.count() != count) ? nullptr : it->second.p;
}
const char *q8_suffix(int s) { return kQ8Suffix[s]; }
const char *norm_suffix(int s) { return kNormSuffix[s]; }
const char *embed_name() { return kEmbed; }
const char *final_norm_name() { return kFinalNorm; }
const char *ple_model_name() { return kPleModel; }
const char *ple_norm_name() { return kPleNorm; }
const char *embed_proj_name() { return kEmbedProj; }
const char *layer_scalar_suffix() { return kLayerScalar; }
}  // namespace e2mi
