// dispatch.cpp — capability and attention-precision tables (the reference's dispatch.c surface,
// src/dispatch.c:13-197) with the gfx950 row added. Pure data plus one lookup; no kernel is ever
// called to discover a capability (dispatch.h:1-11).
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/e2_dispatch.h"

namespace {

constexpr unsigned kCpuI8 = E2_CAP_GEMM_I8 | E2_CAP_QUANT_I8 | E2_CAP_SOFTMAX_Q_I8;

// caps per backend (dispatch.c:15-31); the gfx950 row has the int8 MFMA GEMM, the quantizer, the
// f16-MFMA fused attention and the int8 attention kernel (attn_i8.hip, text only)
unsigned caps_of(e2_backend bk) {
    switch (bk) {
    case E2_BK_CPU_SCALAR: return E2_CAP_GEMM_I8 | E2_CAP_QUANT_I8;
    case E2_BK_CPU_AVX2: return kCpuI8;
    case E2_BK_CPU_VNNI:
    case E2_BK_CPU_AVX512:
    case E2_BK_CPU_NEON: return kCpuI8 | E2_CAP_ATTN_I8_FUSED;
    case E2_BK_INTEL_GPU: return kCpuI8 | E2_CAP_ATTN_I8_FUSED | E2_CAP_ATTN_F16;
    case E2_BK_HIP: return kCpuI8 | E2_CAP_ATTN_I8_FUSED;
    case E2_BK_HIP_GFX950: return E2_CAP_GEMM_I8 | E2_CAP_QUANT_I8 | E2_CAP_ATTN_I8_FUSED | E2_CAP_ATTN_F16;
    default: return 0;
    }
}

struct Rule {
    e2_attn_kind at_or_above, below;
    int min_keys;  // 0: no length gate
};

// preference rules (dispatch.c:47-72); unlisted pairs are fp32 at any length
Rule rule_of(e2_backend bk, e2_tower t) {
    const Rule f32 = {E2_ATTN_F32, E2_ATTN_F32, 0};
    if (t == E2_TOWER_AUDIO) return f32;
    if (t == E2_TOWER_TEXT) {
        switch (bk) {
        case E2_BK_CPU_AVX2:
        case E2_BK_CPU_VNNI:
        case E2_BK_CPU_AVX512:
        case E2_BK_CPU_NEON: return {E2_ATTN_I8, E2_ATTN_F32, 128};
        case E2_BK_INTEL_GPU: return {E2_ATTN_I8, E2_ATTN_F16, 512};
        case E2_BK_HIP: return {E2_ATTN_I8, E2_ATTN_F32, 64};
        // f16 MFMA attention at every length: measured faster than the int8 kernel at every
        // length of the config-4 batch (the int8 one quantizes K and V^T per sequence first and
        // walks the keys twice); E2_ATTN_TEXT=i8 selects the int8 kernel
        case E2_BK_HIP_GFX950: return {E2_ATTN_F16, E2_ATTN_F16, 0};
        default: return f32;
        }
    }
    switch (bk) {  // image: no length gate; capability decides
    case E2_BK_CPU_AVX2:
    case E2_BK_CPU_VNNI:
    case E2_BK_CPU_AVX512:
    case E2_BK_CPU_NEON:
    case E2_BK_INTEL_GPU:
    case E2_BK_HIP: return {E2_ATTN_I8, E2_ATTN_F32, 0};
    // no vision tower on this backend: the table keeps the f16 kernel's row
    case E2_BK_HIP_GFX950: return {E2_ATTN_F16, E2_ATTN_F16, 0};
    default: return f32;
    }
}

e2_backend g_cpu = E2_BK_CPU_SCALAR;
int g_override[E2_TOWER_COUNT] = {-1, -1, -1};
e2_attn_stage g_stage = E2_ATTN_STAGE_AUTO;

bool valid_bk(e2_backend bk) { return (unsigned)bk < (unsigned)E2_BK_COUNT; }
bool valid_tower(e2_tower t) { return (unsigned)t < (unsigned)E2_TOWER_COUNT; }

int parse_kind(const char *v, const char *var) {
    if (!v || !*v || !strcmp(v, "auto")) return -1;
    if (!strcmp(v, "f32")) return E2_ATTN_F32;
    if (!strcmp(v, "f16")) return E2_ATTN_F16;
    if (!strcmp(v, "i8")) return E2_ATTN_I8;
    fprintf(stderr, "e2: ignoring %s=%s (expected auto|f32|f16|i8)\n", var, v);
    return -1;
}

e2_attn_stage parse_stage(const char *v, const char *var) {
    if (!v || !*v || !strcmp(v, "auto")) return E2_ATTN_STAGE_AUTO;
    if (!strcmp(v, "direct")) return E2_ATTN_STAGE_DIRECT;
    if (!strcmp(v, "lds")) return E2_ATTN_STAGE_LDS;
    if (!strcmp(v, "legacy") || !strcmp(v, "old")) return E2_ATTN_STAGE_LEGACY;
    fprintf(stderr, "e2: ignoring %s=%s (expected auto|direct|lds|legacy)\n", var, v);
    return E2_ATTN_STAGE_AUTO;
}

bool executable(e2_backend bk, e2_tower t, e2_attn_kind k) {
    const unsigned c = caps_of(bk);
    if (k == E2_ATTN_F32) return true;
    if (k == E2_ATTN_F16) return (c & E2_CAP_ATTN_F16) != 0;
    if (t == E2_TOWER_TEXT) {
        // text int8 attention is the weight GEMM on quantized Q and P on the reference's
        // backends; the gfx950 row runs its own int8 attention kernel
        if (bk == E2_BK_HIP_GFX950) return (c & E2_CAP_ATTN_I8_FUSED) != 0;
        return (c & (E2_CAP_GEMM_I8 | E2_CAP_QUANT_I8)) == (E2_CAP_GEMM_I8 | E2_CAP_QUANT_I8);
    }
    return t == E2_TOWER_IMAGE && (c & E2_CAP_ATTN_I8_FUSED);
}

}  // namespace

extern "C" void e2_dispatch_set_cpu_backend(e2_backend bk) {
    g_cpu = valid_bk(bk) ? bk : E2_BK_CPU_SCALAR;
}
extern "C" e2_backend e2_cpu_backend(void) { return g_cpu; }
extern "C" unsigned e2_backend_caps(e2_backend bk) { return valid_bk(bk) ? caps_of(bk) : 0; }

extern "C" void e2_attn_env_reload(void) {
    g_override[E2_TOWER_TEXT] = parse_kind(getenv("E2_ATTN_TEXT"), "E2_ATTN_TEXT");
    g_override[E2_TOWER_IMAGE] = parse_kind(getenv("E2_ATTN_IMAGE"), "E2_ATTN_IMAGE");
    g_override[E2_TOWER_AUDIO] = -1;
    g_stage = parse_stage(getenv("E2_ATTN_STAGE"), "E2_ATTN_STAGE");
    if (g_override[E2_TOWER_TEXT] < 0) {  // deprecated alias, lowest precedence
        const char *e = getenv("E2_ATTN_I8");
        if (e && e[0] == '0') g_override[E2_TOWER_TEXT] = E2_ATTN_F32;
        else if (e && e[0] == '1') g_override[E2_TOWER_TEXT] = E2_ATTN_I8;
    }
    if (g_override[E2_TOWER_IMAGE] < 0 && getenv("E2_VATTN_OFF")) g_override[E2_TOWER_IMAGE] = E2_ATTN_F32;
    if (g_stage == E2_ATTN_STAGE_AUTO) {
        const char *ae = getenv("E2_HIP_ATTN"), *ai = getenv("E2_HIP_ATTN_I8");
        if (ae && !strcmp(ae, "old")) g_stage = E2_ATTN_STAGE_LEGACY;
        else if (ai && !strcmp(ai, "direct")) g_stage = E2_ATTN_STAGE_DIRECT;
        if (g_override[E2_TOWER_TEXT] < 0 && ae && (!strcmp(ae, "old") || !strcmp(ae, "lds")))
            g_override[E2_TOWER_TEXT] = E2_ATTN_F32;
    }
}

extern "C" void e2_attn_override(e2_tower tower, int kind) {
    if (!valid_tower(tower)) return;
    g_override[tower] = (kind < 0 || kind > E2_ATTN_I8) ? -1 : kind;
}

extern "C" e2_attn_stage e2_attn_stage_override(void) { return g_stage; }

extern "C" const char *e2_attn_kind_name(e2_attn_kind kind) {
    switch (kind) {
    case E2_ATTN_F32: return "f32";
    case E2_ATTN_F16: return "f16";
    case E2_ATTN_I8: return "i8";
    }
    return "?";
}

extern "C" int e2_attn_min_keys(e2_backend bk, e2_tower tower) {
    if (!valid_bk(bk) || !valid_tower(tower) || g_override[tower] >= 0) return 0;
    return rule_of(bk, tower).min_keys;
}

extern "C" e2_attn_kind e2_attn_pick(e2_backend bk, e2_tower tower, int n_keys) {
    if (!valid_bk(bk) || !valid_tower(tower)) return E2_ATTN_F32;
    e2_attn_kind k;
    if (g_override[tower] >= 0) {
        k = (e2_attn_kind)g_override[tower];
    } else {
        const Rule r = rule_of(bk, tower);
        k = (r.min_keys > 0 && n_keys < r.min_keys) ? r.below : r.at_or_above;
    }
    while (!executable(bk, tower, k)) k = (k == E2_ATTN_I8) ? E2_ATTN_F16 : E2_ATTN_F32;
    return k;
}
