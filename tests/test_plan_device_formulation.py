"""The device planner's formulation of xcd_deal (plan_dev.hip) against the host planner itself
(e2mi_plan_attention, plan.cpp), on the CPU.

The device kernel restructures the host's sequential deal for a workgroup: the entries' key tiles
computed once, each sequence's chunks cut by one thread, the chunks assigned to the least-loaded
XCD queue 64 at a time with each chunk's offset in its queue taken afterwards from per-queue prefix
sums over the batch, and the queues interleaved in two phases (every round in which all eight
queues still hold an entry written at once, the rest turn by turn). This restates those steps in
numpy-free Python and requires the host planner's exact list on random batches: lengths 1-16256,
windows, div 2 and 4, 1-15 heads, up to 1024 sequences. test_gpu_plan_device.py checks the kernel
itself against the host planner on the GPU."""
import numpy as np
import pytest


def _tiles(L, q, window):
    t0, t1 = 0, (L + 31) // 32
    if window > 0:
        q0 = q * 128
        q1 = min(q0 + 127, L - 1)
        t0 = max(q0 - window, 0) // 32
        t1 = min(min(q1 + window, L - 1) // 32 + 1, t1)
    return max(1, t1 - t0)


def _device_deal(lens, H, window, div):
    n = len(lens)
    order = sorted(range(n), key=lambda b: (-lens[b], b))
    items = [b | (h << 16) | (q << 24) for b in order for h in range(H) for q in range((lens[b] + 127) // 128)]
    K = len(items)
    if K <= 8:
        return items
    tiles = [_tiles(lens[it & 0xFFFF], it >> 24, window) for it in items]
    lim = max(1, (sum(tiles) + 8 * div - 1) // (8 * div))
    # chunks: one thread per sequence of the order
    cstart, cload, ib = [], [], 0
    for b in order:
        i0, i1 = ib, ib + H * ((lens[b] + 127) // 128)
        ib = i1
        c = 0
        for i in range(i0, i1):
            if i > i0 and c + tiles[i] > lim:
                cload.append(c)
                c = 0
            if c == 0:
                cstart.append(i)
            c += tiles[i]
        if i1 > i0:
            cload.append(c)
    NC = len(cstart)
    cn = [(cstart[c + 1] if c + 1 < NC else K) - cstart[c] for c in range(NC)]
    # assignment, 64 chunks a batch: the loads alone in the loop, offsets from per-queue prefix sums
    ld, qs, word = [0] * 8, [0] * 8, [None] * NC
    for c0 in range(0, NC, 64):
        xs = []
        for c in range(c0, min(NC, c0 + 64)):
            x = min(range(8), key=lambda y: ld[y] * 8 + y)
            ld[x] += cload[c]
            xs.append(x)
        for y in range(8):
            run = 0
            for j, x in enumerate(xs):
                if x == y:
                    word[c0 + j] = (x, qs[y] + run)
                    run += cn[c0 + j]
            qs[y] += run
    qbase = [sum(qs[:y]) for y in range(8)]
    queue = [None] * K
    for c in range(NC):
        x, off = word[c]
        for i in range(cn[c]):
            queue[qbase[x] + off + i] = items[cstart[c] + i]
    # interleave: the full rounds at once, then turn by turn
    m = min(qs)
    out = [queue[qbase[k & 7] + (k >> 3)] for k in range(8 * m)]
    rem = [qs[y] - m for y in range(8)]
    qp = [qbase[y] + m for y in range(8)]
    for t in range(K - 8 * m):
        y = t & 7
        if rem[y] == 0:
            y = 7 - (max(rem[z] * 8 + 7 - z for z in range(8)) & 7)
        out.append(queue[qp[y]])
        rem[y] -= 1
        qp[y] += 1
    return out


def _cases():
    rng = np.random.default_rng(2026)
    yield "config4", [int(x) for x in rng.integers(64, 513, 64)], 3, 0, 2
    yield "window", [int(x) for x in rng.integers(100, 2049, 12)], 4, 512, 2
    yield "d512", [int(x) for x in rng.integers(100, 2049, 12)], 4, 0, 4
    yield "heads15", [int(x) for x in rng.integers(1, 1025, 8)], 15, 0, 2
    yield "b1024", [int(x) for x in rng.integers(0, 25, 1024)], 3, 0, 2
    yield "long", [16256, 1, 300, 16000], 2, 0, 2
    yield "few", [100, 40], 3, 0, 2
    for k in range(12):
        n = int(rng.integers(1, 200))
        S = int(rng.choice([64, 512, 2048, 4096]))
        lens = [int(x) for x in rng.integers(0, S + 1, n)]
        yield f"random{k}", lens, int(rng.integers(1, 16)), int(rng.choice([0, 128, 512])), int(rng.choice([2, 4]))


@pytest.mark.parametrize("case", list(_cases()), ids=lambda c: c[0])
def test_device_formulation_equals_host_deal(case):
    import e2mi
    name, lens, H, window, div = case
    want = e2mi.attention_work(np.asarray(lens, np.int32), H, window, div) if sum(lens) else []
    got = _device_deal(lens, H, window, div)
    assert list(map(int, want)) == got, name
