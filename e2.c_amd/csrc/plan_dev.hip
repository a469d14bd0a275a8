// plan_dev.hip — the packed batch's plan built on the device from the mask, for the device entry
// (e2mi_text_embed_batch_device): the same rows, positions, sequence ranges and attention work
// lists as the host planner (plan.cpp: pack_rows, attention_lists without split parts, xcd_deal),
// entry for entry, plus each packed row's token id, from one single-workgroup kernel. The call then
// reads nothing back to the host, and one recorded forward per batch shape serves every mask: its
// kernels read the row count the planner writes.
#include <limits.h>

#include "common.h"
#include "plan_dev.h"

namespace e2mi {

constexpr int kPlanThreads = 1024, kPlanWaves = kPlanThreads / 64;

// shared-memory layout, in int32 units: per sequence (kPlanMaxSeqs each) its valid count, first
// row, the sequence at each place of the longest-first order and its first entry; per entry
// (kPlanMaxItems each) the longest-first list, the XCD queues, and per chunk its first entry and its
// load (later its queue and offset); 32 words of reduction scratch
constexpr int kLdsLen = 0, kLdsStart = kPlanMaxSeqs, kLdsOrder = 2 * kPlanMaxSeqs, kLdsIBase = 3 * kPlanMaxSeqs,
              kLdsItems = 4 * kPlanMaxSeqs, kLdsQueue = kLdsItems + kPlanMaxItems,
              kLdsCStart = kLdsQueue + kPlanMaxItems, kLdsCLoad = kLdsCStart + kPlanMaxItems,
              kLdsMisc = kLdsCLoad + kPlanMaxItems, kLdsWords = kLdsMisc + 32;
constexpr size_t kPlanLds = (size_t)kLdsWords * 4;
static_assert(kPlanLds <= 160 * 1024, "LDS budget");

// key tiles of 32 that an unsplit entry for query block q of a sequence of L tokens walks
// (plan.cpp block_tiles / item_tiles with one part)
__device__ inline int entry_tiles(int L, int q, int window) {
    int t0 = 0, t1 = (L + 31) / 32;
    if (window > 0) {
        const int q0 = q * 128, q1 = min(q0 + 127, L - 1);
        t0 = max(q0 - window, 0) / 32;
        t1 = min(min(q1 + window, L - 1) / 32 + 1, t1);
    }
    return max(1, t1 - t0);
}

__device__ inline int wave_sum(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// exclusive prefix sum of one value per thread over the workgroup; *total gets the sum
__device__ inline int block_scan(int v, int *wsum, int *total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    if (lane == 63) wsum[w] = x;
    __syncthreads();
    int base = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < kPlanWaves; i++) {
        const int s = wsum[i];
        base += i < w ? s : 0;
        tot += s;
    }
    __syncthreads();
    *total = tot;
    return base + x - v;
}

__device__ inline int block_sum(int v, int *wsum) {
    int t;
    (void)block_scan(v, wsum, &t);
    return t;
}

// The longest-first list items[0, K) (sequence order `order`, item bases ibase) dealt to the XCDs
// into out[0, slots) as xcd_deal does (plan.cpp), then -1 up to slots: each sequence's entries cut
// into chunks of at most lim key tiles, each chunk to the least-loaded XCD queue in list order, the
// queues interleaved (a dry queue refilled from the fullest).
__device__ void deal(int *lds, int n, int K, int window, int div, int32_t *out, int slots) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int *len = lds + kLdsLen, *order = lds + kLdsOrder, *ibase = lds + kLdsIBase, *items = lds + kLdsItems;
    int *queue = lds + kLdsQueue, *cstart = lds + kLdsCStart, *cload = lds + kLdsCLoad;
    int *misc = lds + kLdsMisc;
    if (K <= 8) {
        for (int i = tid; i < slots; i += kPlanThreads) out[i] = i < K ? items[i] : -1;
        return;
    }
    // the chunk limit: a 1/div share of an XCD's key tiles
    int part = 0;
    for (int i = tid; i < K; i += kPlanThreads) {
        const int it = items[i];
        part += entry_tiles(len[it & 0xffff], it >> 24, window);
    }
    const int total = block_sum(part, misc);
    const int lim = max(1, (total + 8 * div - 1) / (8 * div));
    // chunks of each sequence (one thread per sequence of the order): counted, placed, recorded
    int nck = 0, r = tid, i0 = 0, i1 = 0, L = 0;
    if (r < n) {
        L = len[order[r]];
        i0 = ibase[r];
        i1 = r + 1 < n ? ibase[r + 1] : K;
        for (int i = i0, c = 0; i < i1; i++) {
            const int t = entry_tiles(L, items[i] >> 24, window);
            if (i == i0 || c + t > lim) {
                nck++;
                c = 0;
            }
            c += t;
        }
    }
    int NC;
    const int cb = block_scan(nck, misc, &NC);
    if (r < n && i1 > i0) {
        int k = cb, c = 0;
        for (int i = i0; i < i1; i++) {
            const int t = entry_tiles(L, items[i] >> 24, window);
            if (i > i0 && c + t > lim) {  // chunk k ends before item i
                cload[k++] = c;
                c = 0;
            }
            if (c == 0) cstart[k] = i;
            c += t;
        }
        cload[k] = c;
    }
    __syncthreads();
    // each chunk in list order to the least-loaded queue (lowest index on ties): wave 0, lanes 0..7
    // hold the queues' loads and sizes; a chunk's load word becomes its queue << 24 | offset
    if (wave == 0) {
        int ld = 0, qs = 0;
        for (int c = 0; c < NC; c++) {
            const int cl = cload[c], cn = (c + 1 < NC ? cstart[c + 1] : K) - cstart[c];
            int key = lane < 8 ? ld * 8 + lane : INT_MAX;
            key = min(key, __shfl_xor(key, 1, 64));
            key = min(key, __shfl_xor(key, 2, 64));
            key = min(key, __shfl_xor(key, 4, 64));
            const int x = __shfl(key, 0, 64) & 7;
            if (lane == x) {
                cload[c] = (x << 24) | qs;
                qs += cn;
                ld += cl;
            }
        }
        if (lane < 8) misc[16 + lane] = qs;
    }
    __syncthreads();
    int qsize[8], qbase[8], m = INT_MAX;
#pragma unroll
    for (int x = 0, b = 0; x < 8; x++) {
        qsize[x] = misc[16 + x];
        qbase[x] = b;
        b += qsize[x];
        m = min(m, qsize[x]);
    }
    for (int c = tid; c < NC; c += kPlanThreads) {
        const int w = cload[c], x = w >> 24, off = w & 0xffffff;
        const int s0 = cstart[c], s1 = c + 1 < NC ? cstart[c + 1] : K;
        int base = 0;
#pragma unroll
        for (int y = 0; y < 8; y++) base = y == x ? qbase[y] : base;
        for (int i = s0; i < s1; i++) queue[base + off + i - s0] = items[i];
    }
    __syncthreads();
    // rounds in which every queue still has entries: output k = 8 j + x takes entry j of queue x
    for (int k = tid; k < 8 * m; k += kPlanThreads) {
        const int x = k & 7;
        int base = 0;
#pragma unroll
        for (int y = 0; y < 8; y++) base = y == x ? qbase[y] : base;
        out[k] = queue[base + (k >> 3)];
    }
    // the rest in order by wave 0 (lanes 0..7: each queue's next entry and size); a dry queue's
    // turn goes to the queue with the most entries left (lowest index on ties)
    if (wave == 0) {
        int at = m, sz = 0, qb = 0;
#pragma unroll
        for (int y = 0; y < 8; y++) {
            sz = lane == y ? qsize[y] : sz;
            qb = lane == y ? qbase[y] : qb;
        }
        for (int k = 8 * m; k < K;) {
            for (int x = 0; x < 8 && k < K; x++, k++) {
                int y = x;
                if (__shfl(at, x, 64) == __shfl(sz, x, 64)) {
                    int key = lane < 8 ? (sz - at) * 8 + (7 - lane) : -1;
                    key = max(key, __shfl_xor(key, 1, 64));
                    key = max(key, __shfl_xor(key, 2, 64));
                    key = max(key, __shfl_xor(key, 4, 64));
                    y = 7 - (__shfl(key, 0, 64) & 7);
                }
                const int idx = __shfl(qb + at, y, 64);
                if (lane == 0) out[k] = queue[idx];
                if (lane == y) at++;
            }
        }
    }
    for (int k = K + tid; k < slots; k += kPlanThreads) out[k] = -1;
    __syncthreads();
}

__global__ __launch_bounds__(kPlanThreads) void k_plan_packed(PlanDevArgs a) {
    extern __shared__ __align__(16) int lds[];
    int *len = lds + kLdsLen, *start = lds + kLdsStart, *order = lds + kLdsOrder, *ibase = lds + kLdsIBase;
    int *items = lds + kLdsItems, *misc = lds + kLdsMisc;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, n = a.n, S = a.S;
    // 1. valid tokens per sequence (one wave per sequence)
    for (int b = wave; b < n; b += kPlanWaves) {
        const uint8_t *v = a.valid + (size_t)b * S;
        int c = 0;
        for (int i = lane; i < S; i += 64) c += v[i] != 0;
        c = wave_sum(c);
        if (lane == 0) len[b] = c;
    }
    __syncthreads();
    // 2. first rows: each sequence on a multiple of 8, the total rounded up to 256
    int rows8;
    const int st = block_scan(tid < n ? (len[tid] + 7) & ~7 : 0, misc, &rows8);
    const int M = (rows8 + 255) & ~255;
    if (tid < n) {
        start[tid] = st;
        a.start[tid] = st;
        a.len[tid] = len[tid];
    }
    if (tid == 0) *a.rows = M;
    __syncthreads();
    // 3. the rows of each sequence in token order (ballot compaction), its filler rows after them
    for (int b = wave; b < n; b += kPlanWaves) {
        const uint8_t *v = a.valid + (size_t)b * S;
        const int r0 = start[b];
        int c = 0;
        for (int i0 = 0; i0 < S; i0 += 64) {
            const int i = i0 + lane;
            const bool keep = i < S && v[i] != 0;
            const uint64_t bal = __ballot(keep);
            if (keep) {
                const int r = r0 + c + __popcll(bal & ((1ull << lane) - 1));
                a.rowmap[r] = b * S + i;
                a.pos[r] = i;
                if (a.ids_out) a.ids_out[r] = a.ids[(size_t)b * S + i];
            }
            c += __popcll(bal);
        }
        for (int r = r0 + c + lane; r < r0 + ((c + 7) & ~7); r += 64) {
            a.rowmap[r] = -1;
            a.pos[r] = 0;
            if (a.ids_out) a.ids_out[r] = 0;
        }
    }
    for (int r = rows8 + tid; r < M; r += kPlanThreads) {
        a.rowmap[r] = -1;
        a.pos[r] = 0;
        if (a.ids_out) a.ids_out[r] = 0;
    }
    // 4. sequences longest first, ties in index order (a stable sort by length)
    if (tid < n) {
        const int Lb = len[tid];
        int rk = 0;
        for (int j = 0; j < n; j++) {
            const int Lj = len[j];
            rk += (Lj > Lb) | ((Lj == Lb) & (j < tid));
        }
        order[rk] = tid;
    }
    __syncthreads();
    // 5. the longest-first list: per sequence every head, every 128-query block
    int K;
    const int nq = tid < n ? (len[order[tid]] + 127) / 128 : 0;
    const int ib = block_scan(a.H * nq, misc, &K);
    if (tid < n) {
        ibase[tid] = ib;
        const int b = order[tid];
        for (int h = 0, i = ib; h < a.H; h++)
            for (int q = 0; q < nq; q++, i++) items[i] = b | (h << 16) | (q << 24);
    }
    __syncthreads();
    // 6. the lists dealt to the XCDs (the head_dim-512 list without a window)
    deal(lds, n, K, a.window, a.div, a.work, a.slots);
    if (a.work_full) deal(lds, n, K, 0, a.full_div, a.work_full, a.slots);
}

int launch_plan_packed(hipStream_t s, const PlanDevArgs &a) {
    if (!plan_device_fits(a.n, a.S, a.H, a.slots) || !a.valid || !a.rowmap || !a.pos || !a.start || !a.len ||
        !a.work || !a.rows || (a.ids_out && !a.ids) || a.window < 0 || a.div < 1 || (a.work_full && a.full_div < 1)) {
        set_error("plan_device: needs 0 < B <= %d, 0 < H < 16, slots <= %d covering H (ceil(B S / 128) + B), "
                  "non-null outputs, window >= 0, div >= 1 (B=%d S=%d H=%d slots=%d)",
                  kPlanMaxSeqs, kPlanMaxItems, a.n, a.S, a.H, a.slots);
        return -1;
    }
    static bool attr = false;
    if (!attr) {
        if (check_hip(hipFuncSetAttribute((const void *)k_plan_packed, hipFuncAttributeMaxDynamicSharedMemorySize,
                                          (int)kPlanLds),
                      "plan lds attribute"))
            return -1;
        attr = true;
    }
    hipLaunchKernelGGL(k_plan_packed, dim3(1), dim3(kPlanThreads), kPlanLds, s, a);
    return check_hip(hipGetLastError(), "plan launch");
}

}  // namespace e2mi

using namespace e2mi;

extern "C" int e2mi_plan_device(e2mi_stream stream, const uint8_t *valid, const int32_t *ids, int B, int S, int H,
                                int window, int div, int n_slots, int32_t *rowmap, int32_t *pos, int32_t *start,
                                int32_t *len, int32_t *ids_out, int32_t *work, int32_t *rows) {
    PlanDevArgs a{};
    a.valid = valid;
    a.ids = ids;
    a.n = B;
    a.S = S;
    a.H = H;
    a.window = window;
    a.div = div;
    a.slots = n_slots;
    a.rowmap = rowmap;
    a.pos = pos;
    a.start = start;
    a.len = len;
    a.ids_out = ids_out;
    a.work = work;
    a.rows = rows;
    return launch_plan_packed((hipStream_t)stream, a);
}
