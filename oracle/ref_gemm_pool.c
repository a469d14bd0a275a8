/* ref_gemm_pool.c — TEST INFRASTRUCTURE: the CPU baseline of the int8 GEMM sweep on the reference's
 * own machinery. Built by oracle/Makefile with the reference's sources (one build per activation
 * block size, E2_I8_BLOCK = K, int8.h:61-70), it runs the reference's e2_i8_gemm_avx512 (or
 * e2_i8_gemm_vnni on hosts without AVX-512 VNNI) on the reference's persistent worker pool
 * (e2_pool_global_init / e2_parallel, threads.c:143-160,261-282), with the columns claimed in tiles
 * from a shared counter as text.c's GEMM regions claim them (gemm_worker / gemm_claim,
 * text.c:297-318,341-356; tile = total / (8 * threads), between 8 and 64, rounded up to 16,
 * text.c:395-406). The activations are already quantized (the text tower's reuse = 1 regions).
 * Only bench.py's CPU-baseline leg and tests load it; nothing in the product does. */
#include <stdatomic.h>
#include <stdint.h>
#include <string.h>
#include <time.h>

#include "int8.h"
#include "kernels.h"
#include "model.h"
#include "threads.h"

typedef void (*gemm_fn)(float *y, const int8_t *qa, const float *a_scales, const e2_q8w *w, int M, int N,
                        int n0, int n1);
/* the two kernels, defined in kernels_i8_avx512_vnni.c:276 and kernels_i8_vnni.c:181 */
void e2_i8_gemm_avx512(float *y, const int8_t *qa, const float *a_scales, const e2_q8w *w, int M, int N,
                       int n0, int n1);
void e2_i8_gemm_vnni(float *y, const int8_t *qa, const float *a_scales, const e2_q8w *w, int M, int N,
                     int n0, int n1);

struct claim_region {
    gemm_fn fn;
    float *y;
    const int8_t *qa;
    const float *as;
    const e2_q8w *w;
    int M, N, tile;
    _Atomic int next;
};

static void claim_worker(void *arg, int tid, int nthreads) {
    struct claim_region *r = arg;
    (void)tid;
    (void)nthreads;
    for (int a; (a = atomic_fetch_add_explicit(&r->next, r->tile, memory_order_relaxed)) < r->N;) {
        const int b = a + r->tile < r->N ? a + r->tile : r->N;
        r->fn(r->y, r->qa, r->as, r->w, r->M, r->N, a, b);
    }
}

static int g_threads;

/* The reference's pool with `nthreads` workers (0: its own policy, physical cores within the
 * affinity / cgroup budget, threads.c:177-261). Returns the worker count. */
int rg_init(int nthreads) {
    e2_cpu_init();
    g_threads = e2_pool_global_init(nthreads);
    return g_threads;
}

void rg_close(void) {
    e2_pool_global_free();
    g_threads = 0;
}

static int region_tile(int N) {
    int tile = N / (E2_TILE_PER_THREAD * (g_threads > 0 ? g_threads : 1));
    if (tile < E2_I8_MR) tile = E2_I8_MR;
    if (tile > 64) tile = 64;
    tile = (tile + 15) & ~15;
    return tile < 16 ? 16 : tile;
}

/* One GEMM y [M][N] (M a multiple of 8, the reference's padded token count) as one parallel region.
 * kind 0: e2_i8_gemm_avx512, 1: e2_i8_gemm_vnni. qa holds the biased bytes (q + 128). */
int rg_gemm(int kind, float *y, const int8_t *qa, const float *as, const e2_q8w *w, int M, int N) {
    if (!g_threads || M % 8 || N <= 0) return -1;
    struct claim_region r;
    memset(&r, 0, sizeof r);
    r.fn = kind ? e2_i8_gemm_vnni : e2_i8_gemm_avx512;
    r.y = y;
    r.qa = qa;
    r.as = as;
    r.w = w;
    r.M = M;
    r.N = N;
    r.tile = region_tile(N);
    atomic_init(&r.next, 0);
    e2_parallel(claim_worker, &r);
    return 0;
}

/* Seconds for one pass over n GEMMs (one region each), monotonic clock. */
double rg_pass(int kind, int n, float *const *y, const int8_t *const *qa, const float *const *as,
               const e2_q8w *const *w, const int *M, const int *N) {
    struct timespec t0, t1;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    for (int i = 0; i < n; i++)
        if (rg_gemm(kind, y[i], qa[i], as[i], w[i], M[i], N[i])) return -1.0;
    clock_gettime(CLOCK_MONOTONIC, &t1);
    return (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
}
