// plan.h — the host-side plan of a packed batch: which token rows the forward computes, and the
// attention's work lists. Plain C++ (no HIP), shared by the engine (forward.cpp), the public
// planner entries (e2mi_plan_pack, e2mi_plan_attention) and the CPU sanitizer build.
#pragma once

#include <stdint.h>

namespace e2mi {

// Packed layout of n sequences of S tokens (valid: [n][S] host mask, nonzero keeps a token; null:
// all valid): sequence b's valid tokens in order in rows [start[b], start[b] + len[b]), each
// sequence starting on a multiple of 8 rows, the total rounded up to 256. rowmap[r] = b * S + s of
// packed row r (-1: a filler row), pos[r] = s (0 for fillers). Capacities: rowmap and pos hold
// pack_rows_cap(n, S) entries, start and len n. Returns the row count.
long pack_rows_cap(int n, int S);
int pack_rows(const uint8_t *valid, int n, int S, int32_t *rowmap, int32_t *pos, int32_t *start, int32_t *len);
// the rows sequence b takes: its valid tokens rounded up to 8
int seq_rows(const uint8_t *valid, int S);

// One attention work entry: sequence b, head h, key part p of P, 128-query block qb.
inline int32_t work_item(int b, int h, int part, int parts, int qb) {
    return b | (h << 16) | (part << 20) | ((parts - 1) << 22) | (qb << 24);
}
// Key tiles of 32 an entry walks: its share of its block's range (all keys of the sequence, or those
// within `window` of the block's queries by packed index).
int item_tiles(int32_t it, const int32_t *len, int window);
// Parts of a block whose range spans n tiles: ceil(n / 8), at most max_parts and n (1: unsplit).
int block_parts(int L, int q, int window, int max_parts);
// Workgroup i of a 1-D grid runs on XCD i % 8, each XCD with its own L2: a sequence's consecutive
// entries (which read the same K and V^T) are cut into chunks of at most 1/div of an XCD's share of
// the key tiles, each chunk goes to the least-loaded XCD in list order, and the XCD queues are
// interleaved into the grid (a dry queue is refilled from the fullest). A permutation of w.
void xcd_deal(int32_t *w, int n, const int32_t *len, int window, int div);

struct AttnParams {
    int H;           // query heads (H < 16: the entry's head field is 4 bits)
    int window;      // sliding window of the split list's layers (0: none)
    int max_parts;   // split key ranges into at most this many parts (1: never)
    bool attn_i8;    // long unpadded sequences go to the int8 list instead (work8)
    int i8_min;      // ... when they have at least this many tokens
    int div = 2;     // xcd_deal chunking of the split list (the engine: 2 at head_dim 256)
};
struct AttnLists {
    int32_t *work = nullptr;       // f16 entries (split parts), dealt with AttnParams::div
    int32_t *merge = nullptr;      // one entry per split block (null when max_parts == 1)
    int32_t *work_full = nullptr;  // unsplit entries for the head_dim-512 layers, div 4 (optional)
    int32_t *work8 = nullptr;      // int8 entries, div 2 (needed when attn_i8)
    int n_work = 0, n_merge = 0, n_full = 0, n_work8 = 0;
};
// The lists of a packed batch (start/len/pos from pack_rows): sequences longest first, every head,
// every 128-query block; int8 entries for sequences of at least i8_min tokens with no padding inside
// (the reference's blocked-path rule, text.c:873-875), f16 entries (split into parts) for the rest.
// Capacities: work H * sum(ceil(len / 128)) * max_parts, the others H * sum(ceil(len / 128)).
void attention_lists(const AttnParams &p, const int32_t *len, const int32_t *start, const int32_t *pos, int n,
                     AttnLists &o);

}  // namespace e2mi
