// fault_shim.cpp — test support only, not part of the product library. Linked with the library's own
// objects into lib/libe2mi_fault.so with -Wl,--wrap=<call> for the HIP runtime calls below (the way
// the reference's tests/test_oom.c wraps malloc, CMakeLists.txt:370-374), so that a test can make
// the n-th call of a kind fail and check that the library reports it, releases what it holds and
// keeps working once the failure is cleared. Every forced failure happens on the host, before the
// runtime is asked to do anything: no kernel is affected.
#include <hip/hip_runtime_api.h>

extern "C" {
hipError_t __real_hipMalloc(void **p, size_t n);
hipError_t __real_hipHostMalloc(void **p, size_t n, unsigned int flags);
hipError_t __real_hipStreamCreateWithFlags(hipStream_t *s, unsigned int flags);
hipError_t __real_hipGraphInstantiate(hipGraphExec_t *e, hipGraph_t g, hipGraphNode_t *node, char *log,
                                      size_t len);
hipError_t __real_hipGraphLaunch(hipGraphExec_t e, hipStream_t s);

// countdown per kind: -1 never fails; n >= 0 lets n calls through, fails the next one, then stops
enum { F_ALLOC = 0, F_STREAM = 1, F_INSTANTIATE = 2, F_LAUNCH = 3, F_KINDS = 4 };
static int g_left[F_KINDS] = {-1, -1, -1, -1};
static long g_calls[F_KINDS];

static bool trip(int kind) {
    g_calls[kind]++;
    if (g_left[kind] < 0) return false;
    if (g_left[kind] == 0) {
        g_left[kind] = -1;
        return true;
    }
    g_left[kind]--;
    return false;
}

// kind: 0 device and pinned allocations, 1 stream creation, 2 graph instantiation, 3 graph launch
int e2mi_fault_arm(int kind, int countdown) {
    if (kind < 0 || kind >= F_KINDS) return -1;
    g_left[kind] = countdown;
    return 0;
}
long e2mi_fault_calls(int kind) { return kind >= 0 && kind < F_KINDS ? g_calls[kind] : -1; }

hipError_t __wrap_hipMalloc(void **p, size_t n) {
    if (trip(F_ALLOC)) {
        if (p) *p = nullptr;
        return hipErrorOutOfMemory;
    }
    return __real_hipMalloc(p, n);
}
hipError_t __wrap_hipHostMalloc(void **p, size_t n, unsigned int flags) {
    if (trip(F_ALLOC)) {
        if (p) *p = nullptr;
        return hipErrorOutOfMemory;
    }
    return __real_hipHostMalloc(p, n, flags);
}
hipError_t __wrap_hipStreamCreateWithFlags(hipStream_t *s, unsigned int flags) {
    if (trip(F_STREAM)) return hipErrorOutOfMemory;
    return __real_hipStreamCreateWithFlags(s, flags);
}
hipError_t __wrap_hipGraphInstantiate(hipGraphExec_t *e, hipGraph_t g, hipGraphNode_t *node, char *log,
                                      size_t len) {
    if (trip(F_INSTANTIATE)) return hipErrorOutOfMemory;
    return __real_hipGraphInstantiate(e, g, node, log, len);
}
hipError_t __wrap_hipGraphLaunch(hipGraphExec_t e, hipStream_t s) {
    if (trip(F_LAUNCH)) return hipErrorLaunchFailure;
    return __real_hipGraphLaunch(e, s);
}
}
