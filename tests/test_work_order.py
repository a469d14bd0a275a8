"""The attention work list's order (e2mi.xcd_deal, the engine's forward.cpp xcd_deal): workgroup i of
the 1-D grid runs on XCD i % 8, so the items of one sequence, which read the same K and V^T, are
dealt to one XCD where its share allows. Order only: every item stays in the list once, and each
item computes the same rows whatever its position (the GPU tests run the kernels on these lists)."""
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
    """Windowed sequences cost the key tiles inside the window; split parts their own share."""
    lens = np.array([2048, 700, 300, 40])
    work, merge = e2mi_mod.attention_split_work(lens, 4, lambda n: -(-n // 8), window=512)
    items = work.tolist()
    assert len(items) == len(set(items))
    # part p of P for every split block, merge entries for exactly the split blocks
    blocks = collections.Counter((it & 0xffff, (it >> 16) & 0xf, it >> 24) for it in items)
    split = {(it & 0xffff, (it >> 16) & 0xf, it >> 24) for it in merge.tolist() if it >= 0}
    assert {k for k, v in blocks.items() if v > 1} == split
    # the window caps a block's tiles: 128 queries and +-512 keys are at most 37 tiles
    assert max(e2mi_mod._item_tiles(it, lens, 512) for it in items) <= 37
    assert e2mi_mod._item_tiles(e2mi_mod.work_entry(0, 0, 0, 1, 8), lens, 0) == 64


def test_short_lists_unchanged(e2mi_mod):
    lens = np.array([100, 50])
    assert e2mi_mod.attention_work(lens, 3).tolist() == _plain(e2mi_mod, lens, 3)
