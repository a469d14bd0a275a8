// plan_dev.h — the device-side planner of packed batches (plan_dev.hip), used by the engine's device
// entry and by e2mi_plan_device.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace e2mi {

// one workgroup holds the whole plan: at most this many sequences and work entries per list
constexpr int kPlanMaxSeqs = 1024, kPlanMaxItems = 8192;

struct PlanDevArgs {
    const uint8_t *valid;   // [n][S] device mask, nonzero keeps a token
    const int32_t *ids;     // [n][S] device token ids (read when ids_out is set)
    int n, S, H;
    int window, div;        // the work list's window (0: none) and chunking (xcd_deal)
    int full_div;           // work_full's chunking (no window), when work_full is set
    int slots;              // entries of work and work_full: each list, then -1
    int32_t *rowmap, *pos;  // per packed row (n * round8(S) + 256 entries)
    int32_t *start, *len;   // per sequence
    int32_t *ids_out;       // per packed row its token (0 for fillers), or null
    int32_t *work, *work_full;
    int32_t *rows;          // the packed row count
    int32_t *rows_host;     // ... also written here (mapped host memory), or null
};

// the plan of n sequences of S tokens with H heads fits one planner workgroup in `slots` entries
// per list (at least the longest list, H (ceil(n S / 128) + n)); a work entry holds 127 query blocks
// of a sequence at most (S <= 16256)
inline bool plan_device_fits(int n, int S, int H, int slots) {
    if (n <= 0 || n > kPlanMaxSeqs || S <= 0 || S > 16256 || H <= 0 || H > 15 || slots > kPlanMaxItems)
        return false;
    const long need = (long)H * (((long)n * S + 127) / 128 + n);
    return slots >= need && (long)n * ((S + 7) & ~7) + 256 <= 0x7fffffffL;
}

int launch_plan_packed(hipStream_t s, const PlanDevArgs &a);

}  // namespace e2mi
