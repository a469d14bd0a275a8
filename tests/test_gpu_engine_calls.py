"""The engine's call-level contracts (e2hip.h:31-64, e2.h:25-36 semantics on the device engine):

- a chunk with no valid token at all gives exact zero embeddings without running a forward, also
  when the batch is far larger than the workspace and at the reference geometry (whose
  padded-rows forward does not exist);
- ids handed over on the device are checked on the device: an out-of-range id fails the call (or,
  with a caller stream, the next call) instead of being silently clamped;
- a host call made right after an asynchronous device call on another stream waits for it;
- the e2.h-level e2_text_embed / e2_text_embed_batch route to the model's engine.
"""
import numpy as np
import pytest

from model_util import random_batch, reference_small_config, small_config

pytestmark = pytest.mark.gpu


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.fixture(scope="module", params=["baseline", "reference"])
def small_engine(request, gpu):
    """An engine with a 1024-row workspace, so that a few sequences of 512 already exceed it."""
    import e2mi
    if request.param == "baseline":
        m = e2mi.Model.synthetic(small_config(e2mi, n_layers=1), 71)
    else:
        m = e2mi.Model.synthetic(reference_small_config(e2mi, n_layers=6), 72)
    return e2mi, m, e2mi.Engine(m, max_rows=1024)


def test_all_padding_batches_give_zero_vectors(small_engine, rng):
    import torch
    e2mi, m, eng = small_engine
    B, S = 12, 512                                     # 6144 rows against a 1024-row workspace
    ids = rng.integers(0, 1000, (B, S)).astype(np.int32)
    valid = np.zeros((B, S), np.uint8)
    out = eng.embed_batch(ids, valid)
    assert out.shape == (B, eng.dim) and np.all(out == 0.0)
    dev = torch.device("cuda:0")
    dout = torch.full((B, eng.dim), 7.0, device=dev)
    eng.embed_batch_device(_t(ids, dev), _t(valid, dev), dout)
    torch.cuda.synchronize()
    assert np.all(dout.cpu().numpy() == 0.0)
    # mixed: the all-padding sequences stay zero, the others equal their single-sequence embedding
    valid[3, :40] = 1
    valid[9, :300] = 1
    out = eng.embed_batch(ids, valid)
    dout.fill_(7.0)
    eng.embed_batch_device(_t(ids, dev), _t(valid, dev), dout)
    torch.cuda.synchronize()
    assert np.array_equal(dout.cpu().numpy(), out)
    for b in range(B):
        if b in (3, 9):
            single = eng.embed_batch(ids[b:b + 1, :int(valid[b].sum())], None)
            assert np.array_equal(out[b], single[0])
            assert abs(np.linalg.norm(out[b]) - 1.0) < 1e-5
        else:
            assert np.all(out[b] == 0.0)


def test_device_entry_reports_out_of_range_ids(small_engine, rng):
    import torch
    e2mi, m, eng = small_engine
    lib = e2mi.load()
    dev = torch.device("cuda:0")
    ids, valid = random_batch(rng, 3, 64, 1000)
    good = eng.embed_batch(ids, valid)
    bad = ids.copy()
    bad[1, 2] = 1000                                   # one past the vocabulary, a valid token
    idt, vt = _t(bad, dev), _t(valid, dev)
    out = torch.empty((3, eng.dim), device=dev)
    rc = lib.e2mi_text_embed_batch_device(eng.h, e2mi.ptr(idt), e2mi.ptr(vt), 3, 64, e2mi.ptr(out), None)
    assert rc == -1 and "outside" in e2mi.last_error()
    bad[1, 2] = -5                                     # negative, on a masked position
    valid2 = valid.copy()
    valid2[1, 2] = 0
    rc = lib.e2mi_text_embed_batch_device(eng.h, e2mi.ptr(_t(bad, dev)), e2mi.ptr(_t(valid2, dev)), 3, 64,
                                          e2mi.ptr(out), None)
    assert rc == -1
    # with a caller stream the call returns at once; the next call reports it
    s = torch.cuda.Stream()
    rc = lib.e2mi_text_embed_batch_device(eng.h, e2mi.ptr(idt), e2mi.ptr(vt), 3, 64, e2mi.ptr(out),
                                          e2mi.stream_ptr(s))
    assert rc == 0
    rc = lib.e2mi_text_embed_batch_device(eng.h, e2mi.ptr(_t(ids, dev)), e2mi.ptr(vt), 3, 64,
                                          e2mi.ptr(out), None)
    assert rc == -1 and "previous" in e2mi.last_error()
    # on one caller stream: calls are enqueued back to back; once the stream is synchronised the next
    # call reports the flagged one
    rc = lib.e2mi_text_embed_batch_device(eng.h, e2mi.ptr(idt), e2mi.ptr(vt), 3, 64, e2mi.ptr(out),
                                          e2mi.stream_ptr(s))
    assert rc == 0
    s.synchronize()
    gd = _t(ids, dev)
    rc = lib.e2mi_text_embed_batch_device(eng.h, e2mi.ptr(gd), e2mi.ptr(vt), 3, 64, e2mi.ptr(out),
                                          e2mi.stream_ptr(s))
    assert rc == -1 and "previous" in e2mi.last_error()
    rc = lib.e2mi_text_embed_batch_device(eng.h, e2mi.ptr(gd), e2mi.ptr(vt), 3, 64, e2mi.ptr(out),
                                          e2mi.stream_ptr(s))
    assert rc == 0
    s.synchronize()
    assert np.array_equal(out.cpu().numpy(), good)
    # more calls than the engine's 64 flag slots in flight on one stream, all good
    for _ in range(70):
        assert lib.e2mi_text_embed_batch_device(eng.h, e2mi.ptr(gd), e2mi.ptr(vt), 3, 64, e2mi.ptr(out),
                                                e2mi.stream_ptr(s)) == 0
    s.synchronize()
    assert np.array_equal(out.cpu().numpy(), good)
    # the engine is usable again, with the right results
    eng.embed_batch_device(_t(ids, dev), vt, out)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), good)


def test_host_call_after_async_device_call(small_engine, rng):
    """A host call right after an asynchronous device call on another stream: the host call waits
    for it (shared workspace and staging arrays), both results are the sequences' own."""
    import torch
    e2mi, m, eng = small_engine
    dev = torch.device("cuda:0")
    ids_a, valid_a = random_batch(rng, 6, 512, 1000, min_len=300)
    ids_b, valid_b = random_batch(rng, 5, 200, 1000)
    want_a = eng.embed_batch(ids_a, valid_a)
    want_b = eng.embed_batch(ids_b, valid_b)
    s = torch.cuda.Stream()
    ia, va = _t(ids_a, dev), _t(valid_a, dev)
    torch.cuda.synchronize()
    out = torch.empty((6, eng.dim), device=dev)
    for _ in range(3):
        eng.embed_batch_device(ia, va, out, stream=s)  # returns before the forward ends
        got_b = eng.embed_batch(ids_b, valid_b)        # host entry on the engine's own stream
        s.synchronize()
        assert np.array_equal(got_b, want_b)
        assert np.array_equal(out.cpu().numpy(), want_a)


def test_model_level_text_entries(small_engine, rng):
    """e2_text_embed_batch / e2_text_embed (include/e2.h:25,35-36) on the model handle: the same
    embeddings as the engine, validation before any output is written."""
    e2mi, m, eng = small_engine
    lib = e2mi.load()
    ids, valid = random_batch(rng, 4, 96, 1000)
    want = eng.embed_batch(ids, valid)
    out = np.full((4, eng.dim), 7.0, np.float32)
    assert lib.e2_text_embed_batch(m.h, e2mi.ptr(ids), e2mi.ptr(valid), 4, 96, e2mi.ptr(out)) == 0
    assert np.array_equal(out, want)
    one = np.empty(eng.dim, np.float32)
    L = int(valid[2].sum())
    assert lib.e2_text_embed(m.h, e2mi.ptr(np.ascontiguousarray(ids[2, :L])), L, e2mi.ptr(one)) == 0
    assert np.array_equal(one, eng.embed_batch(ids[2:3, :L], None)[0])
    bad = ids.copy()
    bad[0, 0] = 1 << 20
    out[:] = 7.0
    assert lib.e2_text_embed_batch(m.h, e2mi.ptr(bad), e2mi.ptr(valid), 4, 96, e2mi.ptr(out)) == -1
    assert "out of range" in e2mi.last_error() and np.all(out == 7.0)
    assert lib.e2_text_embed_batch(None, e2mi.ptr(ids), None, 1, 4, e2mi.ptr(out)) == -1
