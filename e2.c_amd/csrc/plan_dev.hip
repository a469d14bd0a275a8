// plan_dev.hip — the packed batch's plan built on the device from the mask, for the device entry
// (e2mi_text_embed_batch_device): the same rows, positions, sequence ranges and attention work
// lists as the host planner (plan.cpp: pack_rows, attention_lists without split parts, xcd_deal),
// entry for entry, plus each packed row's token id. The call then reads nothing back to the host,
// and one recorded forward per batch shape serves every mask: its kernels read the row count the
// planner writes.
//
// Two launches: k_plan_count counts each sequence's valid tokens (one workgroup per sequence);
// k_plan_packed then builds the attention lists in its workgroup 0 (sequences longest first, the
// entries cut into chunks, the chunks dealt to the XCD queues, the queues interleaved: sequential
// steps, done by one wave with the queue state in eight lanes and 8-lane DPP reductions) while its
// other workgroups write the rows of the sequences, each by a workgroup-wide scan of its mask.
#include <limits.h>

#include "common.h"
#include "plan_dev.h"

namespace e2mi {

constexpr int kPlanThreads = 1024;
constexpr int kPlanRowGroups = 255;  // workgroups writing rows (k_plan_packed's others)

// shared-memory layout of the lists workgroup, in int32 units: per sequence (kPlanMaxSeqs each) its
// valid count (padded with -1 to a multiple of 4), the sequence at each place of the longest-first
// order and its first entry; per entry (kPlanMaxItems each) the longest-first list, the XCD queues
// (first the entries' key tiles), per chunk its first entry (once the queues are filled: the queue
// positions of the interleave's last rounds) and its load (later its queue and offset); 32 words of
// reduction scratch
constexpr int kLdsLen = 0, kLdsOrder = kPlanMaxSeqs, kLdsIBase = 2 * kPlanMaxSeqs, kLdsItems = 3 * kPlanMaxSeqs,
              kLdsQueue = kLdsItems + kPlanMaxItems, kLdsCStart = kLdsQueue + kPlanMaxItems,
              kLdsCLoad = kLdsCStart + kPlanMaxItems, kLdsTail = kLdsCStart, kLdsMisc = kLdsCLoad + kPlanMaxItems,
              kLdsWords = kLdsMisc + 32;
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

// exclusive prefix sum of one value per thread over the workgroup; *total gets the sum
__device__ inline int block_scan(int v, int *wsum, int *total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    if (lane == 63) wsum[w] = x;
    __syncthreads();
    int base = 0, tot = 0;
    for (int i = 0; i < nw; i++) {
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

// min / max over each group of 8 lanes, every lane of the group gets it (DPP: swap neighbours, swap
// pairs, mirror within 8)
__device__ inline int min8(int v) {
    v = min(v, __builtin_amdgcn_mov_dpp(v, 0xb1, 0xf, 0xf, false));
    v = min(v, __builtin_amdgcn_mov_dpp(v, 0x4e, 0xf, 0xf, false));
    return min(v, __builtin_amdgcn_mov_dpp(v, 0x141, 0xf, 0xf, false));
}
__device__ inline int max8(int v) {
    v = max(v, __builtin_amdgcn_mov_dpp(v, 0xb1, 0xf, 0xf, false));
    v = max(v, __builtin_amdgcn_mov_dpp(v, 0x4e, 0xf, 0xf, false));
    return max(v, __builtin_amdgcn_mov_dpp(v, 0x141, 0xf, 0xf, false));
}

// valid tokens of each sequence: one workgroup per sequence
__global__ __launch_bounds__(256) void k_plan_count(const uint8_t *__restrict__ valid, int S, int32_t *__restrict__ len) {
    __shared__ int wsum[4];
    const uint8_t *v = valid + (size_t)blockIdx.x * S;
    int c = 0;
#pragma unroll 4
    for (int i = threadIdx.x; i < S; i += 256) c += v[i] != 0;
    const int t = block_sum(c, wsum);
    if (threadIdx.x == 0) len[blockIdx.x] = t;
}

// The longest-first list items[0, K) (sequence order `order`, item bases ibase) dealt to the XCDs
// into out[0, slots) as xcd_deal does (plan.cpp), then -1 up to slots: each sequence's entries cut
// into chunks of at most lim key tiles, each chunk to the least-loaded XCD queue in list order, the
// queues interleaved (a dry queue refilled from the fullest).
__device__ void deal(int *lds, int n, int K, int window, int div, int32_t *out, int slots) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int *len = lds + kLdsLen, *ibase = lds + kLdsIBase, *items = lds + kLdsItems;
    int *queue = lds + kLdsQueue, *cstart = lds + kLdsCStart, *cload = lds + kLdsCLoad, *tail = lds + kLdsTail;
    int *misc = lds + kLdsMisc;
    if (K <= 8) {
        for (int i = tid; i < slots; i += kPlanThreads) out[i] = i < K ? items[i] : -1;
        return;
    }
    // the chunk limit: a 1/div share of an XCD's key tiles; each entry's tiles kept (in the queue
    // area, which the queues fill later)
    int *tiles = queue;
    int part = 0;
    for (int i = tid; i < K; i += kPlanThreads) {
        const int it = items[i];
        tiles[i] = entry_tiles(len[it & 0xffff], it >> 24, window);
        part += tiles[i];
    }
    const int total = block_sum(part, misc);
    const int lim = max(1, (total + 8 * div - 1) / (8 * div));
    // chunks of each sequence (one thread per sequence of the order): counted, placed, recorded
    int nck = 0, i0 = 0, i1 = 0;
    if (tid < n) {
        i0 = ibase[tid];
        i1 = tid + 1 < n ? ibase[tid + 1] : K;
        for (int i = i0, c = 0; i < i1; i++) {
            const int t = tiles[i];
            if (i == i0 || c + t > lim) {
                nck++;
                c = 0;
            }
            c += t;
        }
    }
    int NC;
    const int cb = block_scan(nck, misc, &NC);
    if (tid < n && i1 > i0) {
        int k = cb, c = 0;
        for (int i = i0; i < i1; i++) {
            const int t = tiles[i];
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
    // each chunk in list order to the least-loaded queue (lowest index on ties), by wave 0: lane y < 8
    // holds queue y's load, and 64 chunks at a time sit in the lanes. The loop carries only the loads
    // (the lane whose key is its group's minimum adds the chunk); each chunk's offset in its queue
    // follows per batch from prefix sums of the batch's entry counts per queue. A chunk's load word
    // becomes its queue << 24 | offset in the queue.
    if (wave == 0) {
        int ld = 0, qs = 0;
        for (int c0 = 0; c0 < NC; c0 += 64) {
            const int c = c0 + lane;
            const int cl = c < NC ? cload[c] : 0;
            const int cn = c < NC ? (c + 1 < NC ? cstart[c + 1] : K) - cstart[c] : 0;
            int xw = 0;
            const int nb = __builtin_amdgcn_readfirstlane(min(64, NC - c0));
            const int in8 = lane < 8 ? -1 : 0;
            for (int j = 0; j < nb; j++) {
                // no branch in the chain: the least-loaded lane adds the chunk's load by a mask, and
                // lane 0's group minimum is read with readlane (readfirstlane in a lane == j branch
                // would read lane j)
                const int key = ld * 8 + (lane & 7), mk = min8(key);
                ld += __builtin_amdgcn_readlane(cl, j) & (in8 & -(int)(key == mk));
                const int x = __builtin_amdgcn_readlane(mk, 0) & 7;
                xw = lane == j ? x : xw;
            }
            int off = 0;
#pragma unroll
            for (int y = 0; y < 8; y++) {
                const bool mine = c < NC && xw == y;
                const int sel = mine ? cn : 0;
                int incl = sel;
#pragma unroll
                for (int o = 1; o < 64; o <<= 1) {
                    const int t = __shfl_up(incl, o, 64);
                    if (lane >= o) incl += t;
                }
                if (mine) off = __builtin_amdgcn_readlane(qs, y) + incl - sel;
                const int tot = __builtin_amdgcn_readlane(incl, 63);
                if (lane == y) qs += tot;
            }
            if (c < NC) cload[c] = (xw << 24) | off;
        }
        // queue sizes and first positions
        int qb = qs;
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) {
            const int y = __shfl_up(qb, o, 64);
            if (lane >= o) qb += y;
        }
        if (lane < 8) {
            misc[16 + lane] = qs;
            misc[24 + lane] = qb - qs;
        }
    }
    __syncthreads();
    const int *qsize = misc + 16, *qbase = misc + 24;
    int m = qsize[0];
#pragma unroll
    for (int x = 1; x < 8; x++) m = min(m, qsize[x]);
    for (int c = tid; c < NC; c += kPlanThreads) {
        const int w = cload[c], x = w >> 24, off = w & 0xffffff;
        const int s0 = cstart[c], s1 = c + 1 < NC ? cstart[c + 1] : K;
        const int base = qbase[x];
        for (int i = s0; i < s1; i++) queue[base + off + i - s0] = items[i];
    }
    __syncthreads();  // the chunk starts are read; their words take the tail positions
    // the rest of the interleave (after the m rounds in which every queue has an entry) in order by
    // wave 0, lane y < 8 holding queue y's entries left and next position: turn x takes queue x's next
    // entry, or, once queue x is dry, the next entry of the queue with the most left (lowest index on
    // ties); the queue positions go to tail[]
    if (wave == 0) {
        int rem = lane < 8 ? qsize[lane] - m : 0, qp = lane < 8 ? qbase[lane] + m : 0, pos = 0;
        const int T = K - 8 * m;
        for (int t = 0; t < T; t++) {
            int y = t & 7;
            if (__builtin_amdgcn_readlane(rem, y) == 0)
                y = 7 - (__builtin_amdgcn_readlane(max8(rem * 8 + 7 - (lane & 7)), 0) & 7);
            const int at = __builtin_amdgcn_readlane(qp, y), me = lane == y ? 1 : 0;
            pos = lane == (t & 63) ? at : pos;
            rem -= me;
            qp += me;
            if ((t & 63) == 63 || t + 1 == T) {
                const int i = (t & ~63) + lane;
                if (i < T) tail[i] = pos;
            }
        }
    }
    __syncthreads();
    // rounds in which every queue still has entries: output k = 8 j + x takes entry j of queue x;
    // then the recorded positions; then -1
    for (int k = tid; k < slots; k += kPlanThreads) {
        int v = -1;
        if (k < 8 * m) v = queue[qbase[k & 7] + (k >> 3)];
        else if (k < K) v = queue[tail[k - 8 * m]];
        out[k] = v;
    }
    __syncthreads();
}

// workgroup 0 of k_plan_packed: sequence starts, the row count, the total's filler rows, and the
// attention lists
__device__ void plan_lists(const PlanDevArgs &a, int *lds) {
    int *len = lds + kLdsLen, *order = lds + kLdsOrder, *ibase = lds + kLdsIBase, *items = lds + kLdsItems;
    int *misc = lds + kLdsMisc;
    const int tid = threadIdx.x, n = a.n, n4 = (n + 3) & ~3;
    const int L = tid < n ? a.len[tid] : 0;
    if (tid < n4) len[tid] = tid < n ? L : -1;  // -1: no sequence (the rank loop reads 4 at a time)
    int rows8;
    const int st = block_scan((L + 7) & ~7, misc, &rows8);
    const int M = (rows8 + 255) & ~255;
    if (tid < n) a.start[tid] = st;
    if (tid == 0) {
        *a.rows = M;
        if (a.rows_host) *a.rows_host = M;
    }
    for (int r = rows8 + tid; r < M; r += kPlanThreads) {
        a.rowmap[r] = -1;
        a.pos[r] = 0;
        if (a.ids_out) a.ids_out[r] = 0;
    }
    // sequences longest first, ties in index order (a stable sort by length)
    if (tid < n) {
        int rk = 0;
#pragma unroll 2
        for (int j = 0; j < n4; j += 4) {
            const int4 q = *(const int4 *)(len + j);
            rk += (q.x > L) | ((q.x == L) & (j < tid));
            rk += (q.y > L) | ((q.y == L) & (j + 1 < tid));
            rk += (q.z > L) | ((q.z == L) & (j + 2 < tid));
            rk += (q.w > L) | ((q.w == L) & (j + 3 < tid));
        }
        order[rk] = tid;
    }
    __syncthreads();
    // the longest-first list: per sequence every head, every 128-query block
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
    // dealt to the XCDs (the head_dim-512 list without a window)
    deal(lds, n, K, a.window, a.div, a.work, a.slots);
    if (a.work_full) deal(lds, n, K, 0, a.full_div, a.work_full, a.slots);
}

// the other workgroups: the rows of sequences g, g + groups, ...: each valid token's row is its
// sequence's first row plus the valid tokens before it (a workgroup scan over 1024 tokens a step),
// so consecutive tokens write consecutive rows; then the sequence's filler rows
__device__ void plan_rows(const PlanDevArgs &a, int *lds, int g, int groups) {
    int *misc = lds + kLdsMisc;
    const int tid = threadIdx.x, n = a.n, S = a.S;
    for (int b = g; b < n; b += groups) {
        int part = 0;
        for (int j = tid; j < b; j += kPlanThreads) part += (a.len[j] + 7) & ~7;
        const int st = block_sum(part, misc), L = a.len[b];
        const uint8_t *v = a.valid + (size_t)b * S;
        int cnt = 0;
        for (int s0 = 0; s0 < S; s0 += kPlanThreads) {
            const int s = s0 + tid;
            const bool keep = s < S && v[s] != 0;
            const int id = keep && a.ids_out ? a.ids[(size_t)b * S + s] : 0;
            int step;
            const int r = st + cnt + block_scan(keep ? 1 : 0, misc, &step);
            if (keep) {
                a.rowmap[r] = b * S + s;
                a.pos[r] = s;
                if (a.ids_out) a.ids_out[r] = id;
            }
            cnt += step;
        }
        if (tid < ((L + 7) & ~7) - L) {
            const int r = st + L + tid;
            a.rowmap[r] = -1;
            a.pos[r] = 0;
            if (a.ids_out) a.ids_out[r] = 0;
        }
    }
}

__global__ __launch_bounds__(kPlanThreads) void k_plan_packed(PlanDevArgs a) {
    extern __shared__ __align__(16) int lds[];
    if (blockIdx.x == 0) plan_lists(a, lds);
    else plan_rows(a, lds, blockIdx.x - 1, gridDim.x - 1);
}

int launch_plan_packed(hipStream_t s, const PlanDevArgs &a) {
    if (!plan_device_fits(a.n, a.S, a.H, a.slots) || !a.valid || !a.rowmap || !a.pos || !a.start || !a.len ||
        !a.work || !a.rows || (a.ids_out && !a.ids) || a.window < 0 || a.div < 1 || (a.work_full && a.full_div < 1)) {
        set_error("plan_device: needs 0 < B <= %d, 0 < S <= 16256, 0 < H < 16, slots <= %d covering H (ceil(B S / 128) "
                  "+ B), non-null outputs, window >= 0, div >= 1 (B=%d S=%d H=%d slots=%d)",
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
    hipLaunchKernelGGL(k_plan_count, dim3(a.n), dim3(256), 0, s, a.valid, a.S, a.len);
    hipLaunchKernelGGL(k_plan_packed, dim3(1 + min(a.n, kPlanRowGroups)), dim3(kPlanThreads), kPlanLds, s, a);
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
