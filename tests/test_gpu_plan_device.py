"""The device planner (e2mi_plan_device, the engine's device entry) against the host planner
(e2mi_plan_pack, e2mi_plan_attention with one part, which test_work_order.py checks from the
definition): every array equal entry for entry, the work list followed by -1, each packed row's
token gathered.

Masks: right-padded and with holes, all-invalid sequences, a single short sequence (a list of at
most 8 entries, which is not dealt), odd S, the reference geometry's window and head_dim-512 chunking
(window 512, div 4), 15 heads, and the planner's largest batch (1024 sequences)."""
import zlib

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _mask(rng, B, S, lo=1, holes=0.0):
    lens = rng.integers(lo, S + 1, B)
    valid = (np.arange(S)[None, :] < lens[:, None]).astype(np.uint8)
    if holes:
        valid[rng.random((B, S)) < holes] = 0
    return valid


CASES = [
    # name, B, S, H, window, div, mask builder
    ("config4", 64, 512, 3, 0, 2, lambda r: _mask(r, 64, 512, lo=64)),
    ("holes", 48, 300, 3, 0, 2, lambda r: _mask(r, 48, 300, holes=0.3)),
    ("empty_rows", 16, 200, 3, 0, 2, lambda r: np.where(np.arange(16)[:, None] % 3 == 0, 0,
                                                          _mask(r, 16, 200)).astype(np.uint8)),
    ("all_empty", 5, 64, 3, 0, 2, lambda r: np.zeros((5, 64), np.uint8)),
    ("short_list", 1, 100, 3, 0, 2, lambda r: np.ones((1, 100), np.uint8)),
    ("odd_S", 33, 77, 8, 0, 2, lambda r: _mask(r, 33, 77, holes=0.05)),
    ("window", 12, 2048, 4, 512, 2, lambda r: _mask(r, 12, 2048, lo=100)),
    ("window_d512", 12, 2048, 4, 0, 4, lambda r: _mask(r, 12, 2048, lo=100)),
    ("heads15", 8, 1024, 15, 0, 2, lambda r: _mask(r, 8, 1024)),
    ("b1024", 1024, 24, 3, 0, 2, lambda r: _mask(r, 1024, 24, holes=0.2)),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_device_plan_equals_host_plan(gpu, case):
    import torch
    import e2mi
    name, B, S, H, window, div, build = case
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    valid = build(rng)
    ids = rng.integers(0, 1000, (B, S)).astype(np.int32)
    dvalid = torch.from_numpy(valid).to(gpu)
    dids = torch.from_numpy(ids).to(gpu)
    rowmap, pos, start, lens, M, work, ids_out = e2mi.plan_device(dvalid, H, window, div, ids=dids)
    torch.cuda.synchronize()
    lib = e2mi.load()
    cap = B * ((S + 7) & ~7) + 256
    h_rowmap, h_pos = np.empty(cap, np.int32), np.empty(cap, np.int32)
    h_start, h_len = np.empty(B, np.int32), np.empty(B, np.int32)
    hM = lib.e2mi_plan_pack(valid.ctypes.data, B, S, h_rowmap.ctypes.data, h_pos.ctypes.data,
                            h_start.ctypes.data, h_len.ctypes.data)
    assert M == hM, (M, hM)
    assert np.array_equal(rowmap.cpu().numpy(), h_rowmap[:M])
    assert np.array_equal(pos.cpu().numpy(), h_pos[:M])
    assert np.array_equal(start.cpu().numpy(), h_start)
    assert np.array_equal(lens.cpu().numpy(), h_len)
    src = h_rowmap[:M]
    want_ids = np.where(src >= 0, ids.reshape(-1)[np.maximum(src, 0)], 0)
    assert np.array_equal(ids_out.cpu().numpy(), want_ids)
    h_work = e2mi.attention_work(h_len, H, window, div) if h_len.sum() else np.empty(0, np.int32)
    w = work.cpu().numpy()
    n = len(h_work)
    assert np.array_equal(w[:n], h_work), (name, np.flatnonzero(w[:n] != h_work)[:8])
    assert np.all(w[n:] == -1)


def test_device_plan_refusals(gpu):
    import torch
    import e2mi
    lib = e2mi.load()
    v = torch.ones((4, 64), dtype=torch.uint8, device=gpu)
    buf = torch.empty(4096, dtype=torch.int32, device=gpu)
    p = buf.data_ptr()
    # too few slots for the list's bound H (ceil(B S / 128) + B) = 3 * (2 + 4)
    assert lib.e2mi_plan_device(None, v.data_ptr(), None, 4, 64, 3, 0, 2, 17, p, p, p, p, None, p, p) == -1
    assert "slots" in e2mi.last_error()
    # 16 heads do not fit an entry's head field
    assert lib.e2mi_plan_device(None, v.data_ptr(), None, 4, 64, 16, 0, 2, 4000, p, p, p, p, None, p, p) == -1
    # ids_out without ids
    assert lib.e2mi_plan_device(None, v.data_ptr(), None, 4, 64, 3, 0, 2, 18, p, p, p, p, p, p, p) == -1


def _embed_both(eng, ids, valid, dev):
    """The device entry's embeddings (device plan) and the host entry's (host plan)."""
    import torch
    out = torch.full((ids.shape[0], eng.dim), 7.0, device=dev)
    eng.embed_batch_device(torch.from_numpy(ids).to(dev), torch.from_numpy(valid).to(dev), out)
    torch.cuda.synchronize()
    return out.cpu().numpy(), eng.embed_batch(ids, valid)


def test_engine_device_plan_equals_host_plan(gpu):
    """Masks of one shape whose packed row counts differ (so one recorded forward serves them all
    and its kernels take the planned count): the device entry's embeddings equal the host entry's
    bit for bit, an all-invalid batch (no rows) gives zero vectors, and two calls enqueued on a
    stream without a wait in between (the second planner run follows the first forward) give each
    call's own result."""
    import torch
    import e2mi
    from model_util import random_batch, small_config
    rng = np.random.default_rng(77)
    cfg = small_config(e2mi, n_layers=3)
    m = e2mi.Model.synthetic(cfg, 5)
    eng = e2mi.Engine(m, max_rows=16 * 200)
    B, S = 16, 200
    masks = []
    for k in range(4):
        ids, valid = random_batch(rng, B, S, cfg.vocab, min_len=1, holes=k % 2 == 1)
        if k == 2:
            valid[3] = 0
        masks.append((ids, valid))
    masks.append((masks[0][0], np.zeros((B, S), np.uint8)))
    for ids, valid in masks:
        d, h = _embed_both(eng, ids, valid, gpu)
        assert np.array_equal(d, h)
        if not valid.any():
            assert np.all(d == 0)
    s = torch.cuda.Stream()
    outs = [torch.empty((B, eng.dim), device=gpu) for _ in range(2)]
    dev_in = [(torch.from_numpy(i).to(gpu), torch.from_numpy(v).to(gpu)) for i, v in masks[:2]]
    torch.cuda.synchronize()
    for (it, vt), o in zip(dev_in, outs):
        eng.embed_batch_device(it, vt, o, stream=s)
    s.synchronize()
    for (ids, valid), o in zip(masks[:2], outs):
        assert np.array_equal(o.cpu().numpy(), eng.embed_batch(ids, valid))
    eng.set_device_plan(False)
    d, h = _embed_both(eng, *masks[1], gpu)
    assert np.array_equal(d, h)
    eng.set_device_plan(True)


def test_reference_geometry_device_plan(gpu):
    """The reference checkpoint's geometry (windowed layers dealt with the window, the head_dim-512
    layer's own list, the PLE norm over n_layers slices of each row): device plan == host plan."""
    import e2mi
    from model_util import random_batch, reference_small_config
    rng = np.random.default_rng(78)
    cfg = reference_small_config(e2mi, n_layers=6)
    m = e2mi.Model.synthetic(cfg, 6)
    B, S = 6, 1500
    eng = e2mi.Engine(m, max_rows=B * 1504)
    for k in range(2):
        ids, valid = random_batch(rng, B, S, cfg.vocab, min_len=100, holes=k == 1)
        d, h = _embed_both(eng, ids, valid, gpu)
        assert np.array_equal(d, h)
