// api.cpp — C-ABI entry points of the kernel layer: error state, device info, argument checks,
// and the launches of quant.hip / gemm.hip.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "common.h"

namespace e2mi {

// One process-global message, like the reference's g_err (src/gpu/hip/hip.c:27-49); the backend
// is not reentrant (e2.h:8-10), so no per-thread state is needed.
static char g_err[512] = "";

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}

int check_hip(hipError_t e, const char *what) {
    if (e == hipSuccess) return 0;
    set_error("%s: %s", what, hipGetErrorString(e));
    return -1;
}

static thread_local DeviceRows t_rows;
DeviceRows device_rows() { return t_rows; }
DeviceRowsScope::DeviceRowsScope(const int *ptr, int mul, int est) : prev_(t_rows) { t_rows = DeviceRows{ptr, mul, est}; }
DeviceRowsScope::~DeviceRowsScope() { t_rows = prev_; }

struct GemmArgs;
int launch_quantize(hipStream_t s, int8_t *q, int ldq, float *scales, const float *x, int M,
                    int K, int ldx, int block);

}  // namespace e2mi

using namespace e2mi;

extern "C" const char *e2mi_last_error(void) { return g_err; }

extern "C" int e2mi_device_info(int dev, char *name, int cap, int *cus, int *clock_khz) {
    hipDeviceProp_t p;
    E2MI_HIP(hipGetDeviceProperties(&p, dev));
    if (name && cap > 0) snprintf(name, (size_t)cap, "%s (%s)", p.name, p.gcnArchName);
    if (cus) *cus = p.multiProcessorCount;
    if (clock_khz) *clock_khz = p.clockRate;
    return 0;
}

extern "C" int e2mi_quantize(e2mi_stream stream, int8_t *q, float *scales, const float *x, int M,
                             int K, int ldx, int block) {
    return launch_quantize((hipStream_t)stream, q, K, scales, x, M, K, ldx, block);
}
