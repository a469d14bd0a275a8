// host_checks.cpp — TEST SUPPORT: the library's host code built with g++ -fsanitize=address,undefined
// and driven over good and corrupt inputs, as the reference's CI runs its CPU code under ASan/UBSan
// (.github/workflows/cpu.yml:19-23). Sources linked: model.cpp (the E8CQ reader and writer, the
// synthetic model, the caller-held tensor list), plan.cpp (packed rows and attention work lists)
// and dispatch.cpp (backend tables). tests/test_host_sanitize.py builds and runs it; a sanitizer
// report or a failed check fails that test. No HIP call is made: the two error-reporting functions
// the sources use from api.cpp are defined here.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <fcntl.h>
#include <unistd.h>

#include <algorithm>
#include <random>
#include <string>
#include <vector>

#include "../../include/e2.h"
#include "../../include/e2_dispatch.h"
#include "../../include/e2mi.h"
#include "../../e2.c_amd/csrc/model_internal.h"
#include "../../e2.c_amd/csrc/plan.h"

static char g_err[512];
namespace e2mi {
void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}
}  // namespace e2mi
extern "C" const char *e2mi_last_error(void) { return g_err; }

static int g_fail = 0;
#define CHECK(c)                                                                  \
    do {                                                                          \
        if (!(c)) {                                                               \
            fprintf(stderr, "check failed at line %d: %s (%s)\n", __LINE__, #c, g_err); \
            g_fail = 1;                                                           \
        }                                                                         \
    } while (0)

static std::vector<unsigned char> slurp(const std::string &p) {
    std::vector<unsigned char> b;
    FILE *f = fopen(p.c_str(), "rb");
    if (!f) return b;
    fseek(f, 0, SEEK_END);
    b.resize((size_t)ftell(f));
    fseek(f, 0, SEEK_SET);
    if (fread(b.data(), 1, b.size(), f) != b.size()) b.clear();
    fclose(f);
    return b;
}
static void spit(const std::string &p, const std::vector<unsigned char> &b) {
    FILE *f = fopen(p.c_str(), "wb");
    if (!b.empty()) fwrite(b.data(), 1, b.size(), f);
    fclose(f);
}

// E8CQ: round trip, the index and header corrupted byte by byte, truncations
static void e8cq_checks(const e2_config &c, const std::string &dir, std::mt19937 &rng, int entries) {
    e2_model *m = e2_model_synthetic(&c, 7);
    CHECK(m);
    const std::string good = dir + "/good.e8cq", bad = dir + "/bad.e8cq";
    CHECK(e2_save_e8cq(m, good.c_str()) == 0);
    e2_model *r = e2_load_e8cq(good.c_str(), &c);
    CHECK(r);
    if (r) {
        e2_tensor_view a, b;
        const std::string n = e2mi::layer_name(0, "self_attn.q_proj.weight");
        CHECK(e2_model_tensor(m, n.c_str(), &a) == 0 && e2_model_tensor(r, n.c_str(), &b) == 0);
        CHECK(a.nbytes == b.nbytes && memcmp(a.data, b.data, a.nbytes) == 0);
        e2_free(r);
    }
    const std::vector<unsigned char> raw = slurp(good);
    CHECK(raw.size() > 64);
    uint32_t hdr[4];
    memcpy(hdr, raw.data(), 16);
    const size_t io = hdr[3];
    int loaded = 0, refused = 0;
    // every byte of the header and of the first index entries, set to values that hit the checks'
    // edges (0, 0xff, +-1, random)
    const size_t idx_bytes = std::min(raw.size() - io, (size_t)152 * entries);
    std::vector<size_t> spots;
    for (size_t i = 0; i < 16; i++) spots.push_back(i);
    for (size_t i = 0; i < idx_bytes; i++) spots.push_back(io + i);
    // one copy of the cache, patched in place and restored around each load
    spit(bad, raw);
    const int fd = open(bad.c_str(), O_WRONLY);
    CHECK(fd >= 0);
    auto try_patch = [&](size_t at, const void *bytes, size_t n) {
        CHECK(pwrite(fd, bytes, n, (off_t)at) == (ssize_t)n);
        e2_model *x = e2_load_e8cq(bad.c_str(), &c);
        (x ? loaded : refused)++;
        e2_free(x);
        CHECK(pwrite(fd, raw.data() + at, n, (off_t)at) == (ssize_t)n);
    };
    for (size_t s : spots)
        for (int v : {0x00, 0xff, (raw[s] + 1) & 0xff, (raw[s] + 255) & 0xff, (int)(rng() & 0xff)}) {
            const unsigned char b = (unsigned char)v;
            try_patch(s, &b, 1);
        }
    // 64-bit fields of the index (dims, nbytes, offset) set to large values
    for (int e = 0; e < 4; e++)
        for (size_t f : {(size_t)104, (size_t)112, (size_t)136, (size_t)144})
            for (uint64_t v : {(uint64_t)~0ull, (uint64_t)1 << 63, (uint64_t)raw.size(), (uint64_t)io - 8})
                try_patch(io + 152 * e + f, &v, 8);
    close(fd);
    for (size_t n : {(size_t)0, (size_t)15, (size_t)16, io / 2, io, raw.size() - 1}) {
        std::vector<unsigned char> b(raw.begin(), raw.begin() + (long)n);
        spit(bad, b);
        e2_model *x = e2_load_e8cq(bad.c_str(), &c);
        CHECK(!x);
        e2_free(x);
    }
    CHECK(refused > 0);
    printf("e8cq: %d corrupt variants refused, %d still valid\n", refused, loaded);
    e2_free(m);
    unlink(good.c_str());
    unlink(bad.c_str());
}

// the caller-held tensor list (e2mi_create_tensors' model): a good list, then each field broken
static void tensor_checks(const e2_config &c) {
    e2_model *m = e2_model_synthetic(&c, 11);
    CHECK(m);
    std::vector<std::string> names;
    names.push_back("language_model.embed_tokens.weight");
    names.push_back("language_model.norm.weight");
    if (c.ple_dim > 0) {
        names.push_back("language_model.ple.per_layer_model_projection.weight");
        names.push_back("language_model.ple.per_layer_projection_norm.weight");
    }
    if (c.out_dim > 0) names.push_back("language_model.embedding_projection.weight");
    for (int l = 0; l < c.n_layers; l++) {
        for (int s = 0; s < (c.ple_dim > 0 ? 9 : 7); s++) names.push_back(e2mi::layer_name(l, e2mi::q8_suffix(s)));
        for (int s = 0; s < (c.ple_dim > 0 ? 7 : 6); s++) names.push_back(e2mi::layer_name(l, e2mi::norm_suffix(s)));
        if (c.ple_dim > 0) names.push_back(e2mi::layer_name(l, "layer_scalar"));
    }
    std::vector<e2mi_tensor> t(names.size());
    std::vector<uint16_t> table;
    for (size_t i = 0; i < names.size(); i++) {
        e2_tensor_view v;
        CHECK(e2_model_tensor(m, names[i].c_str(), &v) == 0);
        e2mi_tensor &x = t[i];
        memset(&x, 0, sizeof x);
        x.name = names[i].c_str();
        if (v.kind == 3) {
            x.kind = E2MI_TENSOR_Q8W;
            x.N = (int)v.dims[0];
            x.K = (int)v.dims[1];
            x.nblocks = (int)v.dims[2];
            x.Npad = (int)v.dims[3];
            x.data = v.data;
            x.scale = v.scale;
            x.bsq = v.bsq;
        } else if (i == 0) {  // the table handed over in bf16, as the reference holds it
            const size_t n = v.nbytes / 4;
            table.resize(n);
            for (size_t j = 0; j < n; j++) {
                uint32_t u;
                memcpy(&u, (const float *)v.data + j, 4);
                table[j] = (uint16_t)(u >> 16);
            }
            x.kind = E2MI_TENSOR_BF16;
            x.N = c.vocab;
            x.K = c.hidden;
            x.data = table.data();
        } else {
            x.kind = E2MI_TENSOR_F32;
            x.N = 1;
            x.K = (int)(v.nbytes / 4);
            x.data = v.data;
        }
    }
    e2_model *g = e2mi::model_from_tensors(t.data(), (int)t.size(), c);
    CHECK(g);
    e2_free(g);
    int refused = 0;
    for (size_t i = 0; i < t.size(); i++) {
        std::vector<e2mi_tensor> b = t;
        switch (i % 6) {
        case 0: b[i].N += 8; b[i].Npad += 8; break;
        case 1: b[i].data = nullptr; break;
        case 2: b[i].kind = 9; break;
        case 3: b[i].name = names[(i + 1) % names.size()].c_str(); break;
        case 4: b[i].K = -b[i].K; break;
        default:
            if (b[i].kind == E2MI_TENSOR_Q8W) b[i].Npad = b[i].N + 9;
            else b[i].N = 0;
            break;
        }
        e2_model *x = e2mi::model_from_tensors(b.data(), (int)b.size(), c);
        refused += x == nullptr;
        e2_free(x);
    }
    CHECK(refused == (int)t.size());
    CHECK(!e2mi::model_from_tensors(t.data(), (int)t.size() - 1, c));
    CHECK(!e2mi::model_from_tensors(nullptr, 0, c));
    printf("tensors: %zu valid, every broken list refused\n", t.size());
    e2_free(m);
}

// packed rows and attention lists on random masks, into arrays of exactly the documented sizes
static void plan_checks(std::mt19937 &rng) {
    for (int it = 0; it < 300; it++) {
        const int B = 1 + (int)(rng() % 64), S = 1 + (int)(rng() % 2048);
        const double keep = (rng() % 100) / 100.0;
        std::vector<uint8_t> valid((size_t)B * S);
        const bool right = rng() & 1;
        for (int b = 0; b < B; b++) {
            const int L = (int)(rng() % (S + 1));
            for (int s = 0; s < S; s++)
                valid[(size_t)b * S + s] = right ? (s < L) : ((rng() % 1000) < keep * 1000);
        }
        const long cap = e2mi::pack_rows_cap(B, S);
        std::vector<int32_t> rowmap(cap), pos(cap), start(B), len(B);
        const int M = e2mi::pack_rows(valid.data(), B, S, rowmap.data(), pos.data(), start.data(), len.data());
        CHECK(M % 256 == 0 && M <= cap);
        long blocks = 0;
        for (int b = 0; b < B; b++) blocks += (len[b] + 127) / 128;
        const int H = 1 + (int)(rng() % 15), parts = 1 + (int)(rng() % 4);
        const int window = (rng() & 1) ? 0 : 64 * (1 + (int)(rng() % 16));
        e2mi::AttnParams p{H, window, parts, (rng() & 1) != 0, 32, 2};
        // exactly the documented capacities: an overflow is an ASan report
        std::vector<int32_t> work((size_t)(H * blocks * parts) + 1), merge((size_t)(H * blocks) + 1),
            full((size_t)(H * blocks) + 1), work8((size_t)(H * blocks) + 1);
        work.resize(work.size() - 1);
        merge.resize(merge.size() - 1);
        full.resize(full.size() - 1);
        work8.resize(work8.size() - 1);
        work.shrink_to_fit();
        merge.shrink_to_fit();
        full.shrink_to_fit();
        work8.shrink_to_fit();
        e2mi::AttnLists o;
        o.work = work.data();
        o.merge = merge.data();
        o.work_full = full.data();
        o.work8 = work8.data();
        e2mi::attention_lists(p, len.data(), start.data(), pos.data(), B, o);
        CHECK(o.n_work <= (long)work.size() && o.n_merge <= (long)merge.size());
        CHECK((long)o.n_full + o.n_work8 == H * blocks);
        // the dealt list is a permutation of the plain one
        std::vector<int32_t> got(work.begin(), work.begin() + o.n_work);
        std::sort(got.begin(), got.end());
        CHECK(std::adjacent_find(got.begin(), got.end()) == got.end());
    }
    printf("plans: 300 random masks\n");
}

static void dispatch_checks() {
    for (int bk = -1; bk <= (int)E2_BK_COUNT; bk++)
        for (int tw = -1; tw <= (int)E2_TOWER_COUNT; tw++)
            for (int n : {-1, 0, 1, 31, 32, 63, 64, 127, 128, 4096}) {
                const e2_attn_kind k = e2_attn_pick((e2_backend)bk, (e2_tower)tw, n);
                CHECK(k == E2_ATTN_F32 || k == E2_ATTN_F16 || k == E2_ATTN_I8);
                CHECK(e2_attn_kind_name(k) != nullptr);
                (void)e2_attn_min_keys((e2_backend)bk, (e2_tower)tw);
                (void)e2_backend_caps((e2_backend)bk);
            }
    for (int k : {-5, -1, 0, 1, 2, 3, 99}) e2_attn_override(E2_TOWER_TEXT, k);
    e2_attn_override((e2_tower)77, 1);
    setenv("E2_ATTN_TEXT", "nonsense", 1);
    e2_attn_env_reload();
    unsetenv("E2_ATTN_TEXT");
    e2_attn_env_reload();
    printf("dispatch: tables queried over every backend, tower and edge length\n");
}

int main(int argc, char **argv) {
    const std::string dir = argc > 1 ? argv[1] : "/tmp";
    std::mt19937 rng(12345);
    e2_config c;
    e2_config_baseline(&c);
    c.n_layers = 2;
    c.vocab = 64;
    c.max_seq = 512;
    e8cq_checks(c, dir, rng, 6);
    tensor_checks(c);
    e2_config r;
    e2_config_reference(&r);
    r.n_layers = 6;
    r.vocab = 64;
    e8cq_checks(r, dir, rng, 2);
    tensor_checks(r);
    plan_checks(rng);
    dispatch_checks();
    printf(g_fail ? "host checks: FAILED\n" : "host checks: ok\n");
    return g_fail;
}
