"""Split key ranges (e2mi_attention_packed_split): a 128-query block's key tiles shared out over up to
four workgroups, each leaving its context sum, row max and row sum, then merged (the reference walks
a block's keys in one pass, text.c:702-741). Against the oracle's attention on the same f16 inputs
(every row-head at cosine >= 0.9999 and within 2e-3 of max|v|, the f16 attention's bars), against
the unsplit kernel (blocks with one part bit for bit, split blocks within the same 2e-3), and the
quantized context equal to the quantizer applied to the f32 context. Cases: the BASELINE heads at
logit scale 1.0 with the engine's split rule and with 2, 3 and 4 parts forced on every block; the
reference checkpoint's sliding layers (4 heads on 2 kv heads, window 512 by position, with and
without holes) with the engine's rule."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _np(t):
    return t.cpu().numpy()


def _split_work(e2mi, lens, H, parts, window):
    """The engine's lists (e2mi_plan_attention: ceil(tiles / 8) parts, at most 4), or every block in
    min(parts, tiles) parts (window 0; the order of the entries changes no result)."""
    if parts == "engine":
        return e2mi.attention_split_work(lens, H, 4, window=window)
    assert window == 0
    work, merge = [], []
    for b, L in enumerate(int(x) for x in lens):
        for h in range(H):
            for q in range((L + 127) // 128):
                P = max(1, min(parts, (L + 31) // 32))
                work += [e2mi.work_entry(b, h, p, P, q) for p in range(P)]
                if P > 1:
                    merge.append(e2mi.work_entry(b, h, 0, P, q))
    return np.asarray(work, np.int32), np.asarray(merge or [-1], np.int32)


def _case(gpu, oracle, rng, valid, H, KV, window, scale, parts):
    import e2mi
    D = 256
    B, S = valid.shape
    rowmap, pos, start, lens, M = e2mi.pack_plan(valid)
    q = rng.standard_normal((M, H * D)).astype(np.float32)
    k = rng.standard_normal((M, KV * D)).astype(np.float32)
    v = rng.standard_normal((M, KV * D)).astype(np.float32)
    q16, k16, v16 = (_t(a, gpu).half() for a in (q, k, v))
    vt16 = v16.reshape(M, KV, D).permute(1, 2, 0).contiguous()
    sd, ld, pd = _t(start, gpu), _t(lens, gpu), _t(pos, gpu)
    work, merge = _split_work(e2mi, lens, H, parts, window)
    assert len(merge) > 0 and merge[0] >= 0, "the case must split some block"
    work = np.concatenate([work, np.full(5, -1, np.int32)])
    merge = np.concatenate([merge, np.full(3, -1, np.int32)])
    cq, cs, c32 = e2mi.attention_packed_split(q16, k16, vt16, sd, ld, S, H, KV, work, merge, window=window,
                                              pos=pd, scale=scale)
    uq, us, u32 = e2mi.attention_packed_window(q16, k16, vt16, sd, ld, S, H, KV, D, window=window, pos=pd,
                                               scale=scale, work=_t(e2mi.attention_work(lens, H), gpu))
    got, unsplit = _np(c32), _np(u32)
    qf, kf, vf = (_np(t.float()) for t in (q16, k16, v16))
    split_rows = np.zeros(M, bool)
    for e in merge[merge >= 0]:
        b, qb = e & 0xffff, e >> 24
        split_rows[start[b] + qb * 128:start[b] + min(lens[b], qb * 128 + 128)] = True
    for b in range(B):
        if lens[b] == 0:
            continue
        r = slice(start[b], start[b] + lens[b])
        p = pos[r]
        n = int(p.max()) + 1
        vb = np.zeros(n, np.uint8)
        vb[p] = 1
        qs_, ks_, vs_ = (np.zeros((n, x.shape[1]), np.float32) for x in (qf, kf, vf))
        qs_[p], ks_[p], vs_[p] = qf[r], kf[r], vf[r]
        want = oracle.attention(qs_, ks_, vs_, vb, H, KV, D, scale=scale, window=window)[p]
        gv, wv = got[r].reshape(-1, D).astype(np.float64), want.reshape(-1, D).astype(np.float64)
        cos = (gv * wv).sum(1) / (np.linalg.norm(gv, axis=1) * np.linalg.norm(wv, axis=1))
        assert cos.min() >= 0.9999, f"seq {b}: min row cosine {cos.min()}"
        assert np.abs(gv - wv).max() <= 2e-3 * np.abs(wv).max(), b
        assert np.abs(got[r] - unsplit[r]).max() <= 2e-3 * np.abs(wv).max(), b
    live = rowmap >= 0
    one = live & ~split_rows
    assert np.array_equal(got[one], unsplit[one]) and np.array_equal(_np(cq)[one], _np(uq)[one])
    qo, so = oracle.quantize(got)
    assert np.array_equal(_np(cq)[live], qo[live]) and np.array_equal(_np(cs)[live], so[live])
    assert np.all(_np(cq)[~live] == 0)  # filler rows are not written
    return split_rows[live].mean()


@pytest.mark.parametrize("parts", ["engine", 2, 3, 4])
def test_split_baseline_heads(gpu, oracle, rng, parts):
    valid = np.zeros((6, 512), np.uint8)
    for b, L in enumerate((512, 300, 257, 129, 33, 1)):
        valid[b, :L] = 1
    frac = _case(gpu, oracle, rng, valid, 3, 1, 0, 1.0, parts)
    assert frac > 0.3


@pytest.mark.parametrize("holes", [False, True])
def test_split_sliding_window(gpu, oracle, rng, holes):
    S = 1100
    valid = np.zeros((4, S), np.uint8)
    for b, L in enumerate((1100, 700, 513, 60)):
        valid[b, :L] = 1
    if holes:
        valid[0, 200:260] = 0
        valid[1, rng.random(S) < 0.2] = 0
    _case(gpu, oracle, rng, valid, 4, 2, 512, 1.0 / 16, "engine")
