// plan.cpp — the host-side plan of a packed batch (rows and attention work lists), and the public
// planner entries for callers that run the packed kernels with their own forward.
#include "plan.h"

#include <algorithm>
#include <vector>

#include "../../include/e2mi.h"

namespace e2mi {

void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));

constexpr int kXcds = 8;
constexpr int kPartTiles = 8;  // a split part walks about this many 32-key tiles

long pack_rows_cap(int n, int S) { return (long)n * ((S + 7) & ~7) + 256; }

int seq_rows(const uint8_t *valid, int S) {
    int len = 0;
    for (int i = 0; i < S; i++) len += valid ? (valid[i] != 0) : 1;
    return (len + 7) & ~7;
}

int pack_rows(const uint8_t *valid, int n, int S, int32_t *rowmap, int32_t *pos, int32_t *start, int32_t *len) {
    int r = 0;
    for (int b = 0; b < n; b++) {
        start[b] = r;
        int L = 0;
        for (int i = 0; i < S; i++)
            if (!valid || valid[(size_t)b * S + i]) {
                rowmap[r + L] = b * S + i;
                pos[r + L] = i;
                L++;
            }
        len[b] = L;
        const int end = (r + L + 7) & ~7;
        for (int i = r + L; i < end; i++) rowmap[i] = -1, pos[i] = 0;
        r = end;
    }
    const int M = (r + 255) & ~255;
    for (int i = r; i < M; i++) rowmap[i] = -1, pos[i] = 0;
    return M;
}

// first and one-past-last key tile of query block q of a sequence of L tokens
static void block_tiles(int L, int q, int window, int *t0, int *t1) {
    *t0 = 0;
    *t1 = (L + 31) / 32;
    if (window > 0) {
        const int q0 = q * 128, q1 = std::min(q0 + 127, L - 1);
        *t0 = std::max(q0 - window, 0) / 32;
        *t1 = std::min(std::min(q1 + window, L - 1) / 32 + 1, *t1);
    }
}

int item_tiles(int32_t it, const int32_t *len, int window) {
    const int b = it & 0xffff, part = (it >> 20) & 3, parts = ((it >> 22) & 3) + 1, q = it >> 24;
    int t0, t1;
    block_tiles(len[b], q, window, &t0, &t1);
    const int n = t1 - t0;
    return std::max(1, n * (part + 1) / parts - n * part / parts);
}

int block_parts(int L, int q, int window, int max_parts) {
    if (max_parts <= 1) return 1;
    int t0, t1;
    block_tiles(L, q, window, &t0, &t1);
    const int n = t1 - t0;
    return std::max(1, std::min({max_parts, (n + kPartTiles - 1) / kPartTiles, n}));
}

void xcd_deal(int32_t *w, int n, const int32_t *len, int window, int div) {
    if (n <= kXcds) return;
    long total = 0;
    for (int i = 0; i < n; i++) total += item_tiles(w[i], len, window);
    const long lim = std::max(1L, (total + (long)kXcds * div - 1) / ((long)kXcds * div));
    std::vector<int32_t> q[kXcds];
    long load[kXcds] = {};
    for (int i = 0; i < n;) {
        const int b = w[i] & 0xffff;
        long c = 0;
        int j = i;
        for (; j < n && (w[j] & 0xffff) == b; j++) {
            const int t = item_tiles(w[j], len, window);
            if (j > i && c + t > lim) break;
            c += t;
        }
        const int x = (int)(std::min_element(load, load + kXcds) - load);
        q[x].insert(q[x].end(), w + i, w + j);
        load[x] += c;
        i = j;
    }
    size_t at[kXcds] = {};
    for (int k = 0; k < n;) {
        for (int x = 0; x < kXcds && k < n; x++) {
            int y = x;
            if (at[y] == q[y].size()) {
                y = 0;
                for (int z = 1; z < kXcds; z++)
                    if (q[z].size() - at[z] > q[y].size() - at[y]) y = z;
            }
            w[k++] = q[y][at[y]++];
        }
    }
}

void attention_lists(const AttnParams &p, const int32_t *len, const int32_t *start, const int32_t *pos, int n,
                     AttnLists &o) {
    // longest sequences first: the grid holds more workgroups than the CUs run at once, and the last
    // to start should be the short ones
    std::vector<int> order(n);
    for (int b = 0; b < n; b++) order[b] = b;
    std::stable_sort(order.begin(), order.end(), [&](int x, int y) { return len[x] > len[y]; });
    int k = 0, k8 = 0, km = 0, kf = 0;
    for (int b : order) {
        const int L = len[b], r0 = start[b];
        // the int8 path needs the trimmed sequence all valid: its tokens are positions 0 .. L - 1
        const bool i8 = p.attn_i8 && L >= p.i8_min && L > 0 && pos[r0] == 0 && pos[r0 + L - 1] == L - 1;
        for (int h = 0; h < p.H; h++)
            for (int q = 0; q < (L + 127) / 128; q++) {
                if (i8) {
                    o.work8[k8++] = work_item(b, h, 0, 1, q);
                    continue;
                }
                const int P = block_parts(L, q, p.window, p.max_parts);
                for (int part = 0; part < P; part++) o.work[k++] = work_item(b, h, part, P, q);
                if (P > 1) o.merge[km++] = work_item(b, h, 0, P, q);
                if (o.work_full) o.work_full[kf++] = work_item(b, h, 0, 1, q);
            }
    }
    // head_dim 256 lists take chunks of half an XCD's share (one per sequence at config 4); the
    // head_dim-512 list a quarter (one workgroup per CU there, fewer slots to balance)
    xcd_deal(o.work, k, len, p.window, p.div);
    if (o.work_full) xcd_deal(o.work_full, kf, len, 0, 4);
    if (o.work8) xcd_deal(o.work8, k8, len, 0, 2);
    o.n_work = k;
    o.n_merge = km;
    o.n_full = kf;
    o.n_work8 = k8;
}

}  // namespace e2mi

using namespace e2mi;

extern "C" int e2mi_plan_pack(const uint8_t *valid, int B, int S, int32_t *rowmap, int32_t *pos,
                              int32_t *start, int32_t *len) {
    if (B <= 0 || S <= 0 || (long)B * ((S + 7) & ~7) + 256 > 0x7fffffffL || !rowmap || !pos || !start || !len) {
        set_error("plan_pack: B %d, S %d or a null output", B, S);
        return -1;
    }
    return pack_rows(valid, B, S, rowmap, pos, start, len);
}

extern "C" int e2mi_plan_attention(const int32_t *len, int B, int H, int window, int max_parts, int div,
                                   int32_t *work, int32_t *merge, int *n_merge) {
    if (!len || !work || B <= 0 || B > 0xffff || H <= 0 || H > 15 || window < 0 || max_parts < 1 ||
        max_parts > 4 || div < 1 || (max_parts > 1 && (!merge || !n_merge))) {
        set_error("plan_attention: needs 0 < B < 65536, 0 < H < 16, window >= 0, 1 <= max_parts <= 4, div >= 1, "
                  "and merge outputs when splitting");
        return -1;
    }
    std::vector<int32_t> start(B), pos;
    long rows = 0;
    for (int b = 0; b < B; b++) {
        if (len[b] < 0 || (len[b] + 127) / 128 > 127) {
            set_error("plan_attention: sequence %d has length %d (0 .. 16256)", b, len[b]);
            return -1;
        }
        start[b] = (int32_t)rows;
        rows += (len[b] + 7) & ~7;
    }
    AttnParams p{H, window, max_parts, false, 0, div};
    AttnLists o;
    o.work = work;
    o.merge = max_parts > 1 ? merge : nullptr;
    attention_lists(p, len, start.data(), pos.data(), B, o);
    if (n_merge) *n_merge = o.n_merge;
    return o.n_work;
}
