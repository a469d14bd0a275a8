/* e2_dispatch.h — the backend-selection surface of the reference (src/dispatch.h:15-90), kept as a
 * drop-in, with one new backend row: E2_BK_HIP_GFX950, this library's MI355X backend.
 *
 * Everything here is inert data (dispatch.h:1-11): capabilities say what a backend has, rules say
 * which attention precision it prefers per tower, and e2_attn_pick() combines the two, degrading
 * I8 -> F16 -> F32 by capability (dispatch.c:180-197). Enum values of the reference's rows are
 * unchanged; the new row is appended before E2_BK_COUNT.
 */
#ifndef E2_DISPATCH_H
#define E2_DISPATCH_H

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    E2_BK_CPU_SCALAR = 0,
    E2_BK_CPU_AVX2,
    E2_BK_CPU_VNNI,
    E2_BK_CPU_AVX512,
    E2_BK_CPU_NEON,
    E2_BK_INTEL_GPU,
    E2_BK_HIP,          /* the reference's RDNA v_dot4 backend */
    E2_BK_HIP_GFX950,   /* this backend: CDNA4 int8/f16 MFMA (new row) */
    E2_BK_COUNT
} e2_backend;

typedef enum { E2_TOWER_TEXT = 0, E2_TOWER_IMAGE, E2_TOWER_AUDIO, E2_TOWER_COUNT } e2_tower;
typedef enum { E2_ATTN_F32 = 0, E2_ATTN_F16, E2_ATTN_I8 } e2_attn_kind;
typedef enum {
    E2_ATTN_STAGE_AUTO = 0,
    E2_ATTN_STAGE_DIRECT,
    E2_ATTN_STAGE_LDS,
    E2_ATTN_STAGE_LEGACY
} e2_attn_stage;

enum {
    E2_CAP_GEMM_I8 = 1u << 0,
    E2_CAP_QUANT_I8 = 1u << 1,
    E2_CAP_SOFTMAX_Q_I8 = 1u << 2,
    E2_CAP_ATTN_I8_FUSED = 1u << 3,
    E2_CAP_ATTN_F16 = 1u << 4
};

#define E2_ATTN_ANY_KEYS (1 << 30)

/* dispatch.h:62-63 */
void e2_dispatch_set_cpu_backend(e2_backend bk);
e2_backend e2_cpu_backend(void);
/* dispatch.h:67 */
unsigned e2_backend_caps(e2_backend bk);
/* dispatch.h:78-80: E2_ATTN_TEXT / E2_ATTN_IMAGE (auto|f32|f16|i8), deprecated E2_ATTN_I8,
 * E2_VATTN_OFF, E2_ATTN_STAGE (+ E2_HIP_ATTN, E2_HIP_ATTN_I8 aliases) */
void e2_attn_env_reload(void);
void e2_attn_override(e2_tower tower, int kind);
e2_attn_stage e2_attn_stage_override(void);
const char *e2_attn_kind_name(e2_attn_kind kind);
/* dispatch.h:86 */
int e2_attn_min_keys(e2_backend bk, e2_tower tower);
/* dispatch.h:91 */
e2_attn_kind e2_attn_pick(e2_backend bk, e2_tower tower, int n_keys);

#ifdef __cplusplus
}
#endif
#endif /* E2_DISPATCH_H */
