"""The engine's host-side plan of a packed batch, through the library's own planner (plan.cpp:
e2mi_plan_pack and e2mi_plan_attention are the functions the engine's forward calls, no mirror).

Rows: every valid token once, in order, each sequence on a multiple of 8 rows, M a multiple of 256.
Attention work: every (sequence, head, 128-query block) present once per part; the order deals
each sequence's entries (which read the same K and V^T) to one XCD where its share allows, since
workgroup i of the 1-D grid runs on XCD i % 8. Order only: each entry computes the same rows
wherever it sits (the GPU tests run the kernels on these lists)."""
import collections

import numpy as np
import pytest


@pytest.fixture(scope="module")
def e2mi_mod():
    import e2mi
    return e2mi


def _plain(e2mi_mod, lens, H):
    order = sorted(range(len(lens)), key=lambda b: -int(lens[b]))
    return [e2mi_mod.work_entry(b, h, 0, 1, q) for b in order for h in range(H)
            for q in range((int(lens[b]) + 127) // 128)]


def _xcds_of(work):
    seqs = collections.defaultdict(set)
    for i, it in enumerate(work):
        seqs[int(it) & 0xffff].add(i % 8)
    return seqs


def _tiles(it, lens, window):
    """Key tiles of 32 an entry walks, from the definition: the block's queries q0..q1 see keys j
    with |i - j| <= window (all keys without a window), split evenly over its parts."""
    b, part, parts, q = it & 0xffff, (it >> 20) & 3, ((it >> 22) & 3) + 1, it >> 24
    L = int(lens[b])
    q0, q1 = 128 * q, min(128 * q + 127, L - 1)
    lo, hi = (max(q0 - window, 0), min(q1 + window, L - 1)) if window else (0, L - 1)
    n = hi // 32 - lo // 32 + 1
    return max(1, n * (part + 1) // parts - n * part // parts)


def test_pack_rows(e2mi_mod):
    rng = np.random.default_rng(3)
    valid = (rng.random((7, 300)) < 0.6).astype(np.uint8)
    valid[2] = 0                                   # an all-invalid sequence takes no rows
    valid[3] = 1
    rowmap, pos, start, lens, M = e2mi_mod.pack_plan(valid)
    assert M % 256 == 0 and M == len(rowmap)
    assert np.array_equal(lens, valid.sum(1))
    assert np.all(start % 8 == 0) and np.all(np.diff(start) == (lens[:-1] + 7) // 8 * 8)
    live = rowmap >= 0
    assert live.sum() == valid.sum()
    for b in range(7):
        r = slice(start[b], start[b] + lens[b])
        idx = np.flatnonzero(valid[b])
        assert np.array_equal(rowmap[r], b * 300 + idx) and np.array_equal(pos[r], idx)
    assert np.all(pos[~live] == 0)
    # no mask: every token
    rm, ps, st, ln, M2 = e2mi_mod.pack_plan(np.ones((2, 5), np.uint8))
    assert M2 == 256 and st.tolist() == [0, 8] and ln.tolist() == [5, 5]


def test_config4_lengths_one_xcd_per_sequence(e2mi_mod):
    rng = np.random.default_rng(5)
    lens = rng.integers(64, 513, 64)
    plain = _plain(e2mi_mod, lens, 3)
    work = e2mi_mod.attention_work(lens, 3)
    assert sorted(work.tolist()) == sorted(plain)
    seqs = _xcds_of(work)
    # every sequence costs less than half an XCD's share: one chunk each; only the tail's refills
    # (a queue that ran dry) put items elsewhere
    one = sum(len(x) == 1 for x in seqs.values())
    assert one >= 0.85 * len(seqs), one
    # the plain longest-first list spreads nearly every sequence over several XCDs
    assert sum(len(x) == 1 for x in _xcds_of(plain).values()) < 0.2 * len(seqs)
    # key tiles per XCD balanced
    load = np.zeros(8)
    for i, it in enumerate(work):
        load[i % 8] += (int(lens[int(it) & 0xffff]) + 31) // 32
    assert load.max() <= 1.1 * load.mean(), load


def test_long_sequences_split_into_chunks(e2mi_mod):
    """16 sequences of 1024-2048 tokens at head_dim 512 (div 4): a sequence larger than a quarter of
    an XCD's share is cut, so the XCDs stay balanced."""
    rng = np.random.default_rng(5)
    lens = rng.integers(1024, 2049, 16)
    work = e2mi_mod.attention_work(lens, 4, div=4)
    assert sorted(work.tolist()) == sorted(_plain(e2mi_mod, lens, 4))
    load = np.zeros(8)
    for i, it in enumerate(work):
        load[i % 8] += (int(lens[int(it) & 0xffff]) + 31) // 32
    assert load.max() <= 1.15 * load.mean(), load
    # each sequence on a few XCDs (the plain list puts every one on all 8)
    spread = [len(x) for x in _xcds_of(work).values()]
    assert np.mean(spread) <= 3.5 and max(spread) <= 6, spread


def test_window_and_split_costs(e2mi_mod):
    """Split blocks: parts 0..P-1 of P = min(4, ceil(tiles / 8), tiles) for each block, a merge entry
    for exactly the split blocks; the window caps a block's tiles."""
    lens = np.array([2048, 700, 300, 40])
    work, merge = e2mi_mod.attention_split_work(lens, 4, 4, window=512)
    items = work.tolist()
    assert len(items) == len(set(items))
    blocks = collections.defaultdict(list)
    for it in items:
        blocks[(it & 0xffff, (it >> 16) & 0xf, it >> 24)].append(it)
    for (b, h, q), its in blocks.items():
        full = _tiles(e2mi_mod.work_entry(b, h, 0, 1, q), lens, 512)
        P = max(1, min(4, -(-full // 8), full))
        assert sorted((it >> 20) & 3 for it in its) == list(range(P)), (b, q)
        assert all(((it >> 22) & 3) + 1 == P for it in its)
        # the parts cover the block's tiles exactly
        assert sum(_tiles(it, lens, 512) for it in its) == max(full, P)
    split = {(it & 0xffff, (it >> 16) & 0xf, it >> 24) for it in merge.tolist() if it >= 0}
    assert {k for k, v in blocks.items() if len(v) > 1} == split
    # 128 queries and +-512 keys are at most 37 tiles; without a window a block sees the sequence
    assert max(_tiles(e2mi_mod.work_entry(b, h, 0, 1, q), lens, 512) for b, h, q in blocks) <= 37
    assert _tiles(e2mi_mod.work_entry(0, 0, 0, 1, 8), lens, 0) == 64
    # every sequence, head and block present
    want = {(b, h, q) for b in range(4) for h in range(4) for q in range((int(lens[b]) + 127) // 128)}
    assert set(blocks) == want


def test_short_lists_unchanged(e2mi_mod):
    lens = np.array([100, 50])
    assert e2mi_mod.attention_work(lens, 3).tolist() == _plain(e2mi_mod, lens, 3)


def test_planner_refusals(e2mi_mod):
    lib = e2mi_mod.load()
    lens = np.array([100, 50], np.int32)
    w = np.empty(64, np.int32)
    assert lib.e2mi_plan_attention(lens.ctypes.data, 2, 16, 0, 1, 2, w.ctypes.data, None, None) == -1
    assert "H < 16" in e2mi_mod.last_error()
    assert lib.e2mi_plan_attention(lens.ctypes.data, 2, 3, 0, 4, 2, w.ctypes.data, None, None) == -1
    assert lib.e2mi_plan_pack(None, 0, 8, w.ctypes.data, w.ctypes.data, w.ctypes.data, w.ctypes.data) == -1
