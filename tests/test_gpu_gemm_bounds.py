"""Every GEMM entry point writes exactly its output rows [0, M) and columns [n0, n1), nothing else.

The outputs are views into larger buffers whose guard rows (past M) and guard columns (a leading
dimension wider than N) hold a sentinel pattern; after the call the guard must be untouched. The
shapes leave a partial last row tile, so the stores of rows past M inside a tile are exercised (the
kernels drop them through the buffer descriptor's range or an explicit row test). All accesses
stay inside the allocations: a kernel that wrote past M would overwrite the guard, not fault.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GUARD_ROWS = 64
SENT_F32 = np.float32(-12345.5)
SENT_I8 = -77


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _case(rng, M, N, K, block=128):
    qa = rng.integers(-127, 128, (M, K), dtype=np.int8)
    as_ = rng.uniform(0.001, 0.05, (M, K // block)).astype(np.float32)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    ws = rng.uniform(0.001, 0.02, N).astype(np.float32)
    return qa, as_, w, ws


def _guarded(torch, dev, M, ld, dtype, sent):
    buf = torch.full((M + GUARD_ROWS, ld), sent, dtype=dtype, device=dev)
    return buf


def _check_guard(buf, M, c0, c1, sent):
    b = buf.cpu().numpy()
    assert (b[M:] == sent).all(), "rows past M written"
    assert (b[:M, :c0] == sent).all(), "columns before n0 written"
    assert (b[:M, c1:] == sent).all(), "columns past n1 written"
    assert not (b[:M, c0:c1] == sent).all(), "output not written"


@pytest.mark.parametrize("M", [300, 257, 33, 1000])
@pytest.mark.parametrize("n0,n1", [(0, 384), (128, 320), (3, 250)])
@pytest.mark.parametrize("K", [256, 768])
def test_f32_gemm_bounds(gpu, oracle, rng, M, n0, n1, K):
    """(K = 768 with whole 128-column blocks also takes the per-token kernel with the overlapped
    epilogue.)"""
    import torch
    import e2mi
    N = 384
    qa, as_, w, ws = _case(rng, M, N, K)
    W = e2mi.DeviceWeight.from_rowmajor(w, ws)
    ld = N + 96
    for tok in (False, True):
        if tok:
            qa_, as_d = _t(qa, gpu), _t(as_[:, :1].copy(), gpu)
            fn = e2mi.load().e2mi_i8_gemm_tok
        else:
            qa_, as_d = _t(qa, gpu), _t(as_, gpu)
            fn = e2mi.load().e2mi_i8_gemm
        buf = _guarded(torch, gpu, M, ld, torch.float32, float(SENT_F32))
        e2mi.check(fn(e2mi.stream_ptr(None), e2mi.ptr(buf), ld, e2mi.ptr(qa_), e2mi.ptr(as_d), W.ref,
                      M, n0, n1), "gemm")
        torch.cuda.synchronize()
        _check_guard(buf, M, n0, n1, SENT_F32)
        yo = oracle.i8_gemm(qa, as_[:, :1].copy() if tok else as_, w, ws, block=K if tok else 128)
        got = buf.cpu().numpy()[:M, n0:n1]
        assert np.array_equal(got.view(np.uint32), yo[:, n0:n1].view(np.uint32))


@pytest.mark.parametrize("M", [300, 33])
def test_acc_dump_bounds(gpu, rng, M):
    import torch
    import e2mi
    N, K, n0, n1 = 256, 256, 64, 224
    qa, as_, w, ws = _case(rng, M, N, K)
    W = e2mi.DeviceWeight.from_rowmajor(w, ws)
    ld = N + 32
    y = _guarded(torch, gpu, M, ld, torch.float32, float(SENT_F32))
    nacc = (K // 128) * M * (n1 - n0)
    acc = torch.full((nacc + 4096,), -5, dtype=torch.int32, device=gpu)
    qd, sd = _t(qa, gpu), _t(as_, gpu)  # held: a freed temporary's memory would be reused
    e2mi.check(e2mi.load().e2mi_i8_gemm_acc(e2mi.stream_ptr(None), e2mi.ptr(y), ld, e2mi.ptr(acc),
                                           e2mi.ptr(qd), e2mi.ptr(sd), W.ref, M, n0, n1), "gemm_acc")
    torch.cuda.synchronize()
    _check_guard(y, M, n0, n1, SENT_F32)
    a = acc.cpu().numpy()
    assert (a[nacc:] == -5).all(), "accumulator dump past its extent"
    ref = qa.astype(np.int64).reshape(M, K // 128, 128)
    want = np.einsum("mbk,nbk->bmn", ref, w.astype(np.int64).reshape(N, K // 128, 128))[:, :, n0:n1]
    assert np.array_equal(a[:nacc].reshape(K // 128, M, n1 - n0), want)


@pytest.mark.parametrize("M", [300, 33])
def test_requant_gemm_bounds(gpu, oracle, rng, M):
    import torch
    import e2mi
    N, K = 384, 256
    L = e2mi.load()
    for tok in (False, True):
        qa, as_, w, ws = _case(rng, M, N, K, block=K if tok else 128)
        W = e2mi.DeviceWeight.from_rowmajor(w, ws)
        yq = torch.full((M + GUARD_ROWS, N), SENT_I8, dtype=torch.int8, device=gpu)
        ys = torch.full((M + GUARD_ROWS, N // 128), float(SENT_F32), dtype=torch.float32, device=gpu)
        fn = L.e2mi_i8_gemm_tok_q if tok else L.e2mi_i8_gemm_q
        qd, sd = _t(qa, gpu), _t(as_, gpu)
        e2mi.check(fn(e2mi.stream_ptr(None), e2mi.ptr(yq), e2mi.ptr(ys), e2mi.ptr(qd), e2mi.ptr(sd),
                      W.ref, M), "gemm_q")
        torch.cuda.synchronize()
        assert (yq.cpu().numpy()[M:] == SENT_I8).all()
        assert (ys.cpu().numpy()[M:] == SENT_F32).all()
        assert not (ys.cpu().numpy()[:M] == SENT_F32).any()
        qo, so = oracle.quantize(oracle.i8_gemm(qa, as_, w, ws, block=K if tok else 128))
        assert np.array_equal(yq.cpu().numpy()[:M], qo)
        assert np.array_equal(ys.cpu().numpy()[:M].view(np.uint32), so.view(np.uint32))


@pytest.mark.parametrize("M", [300, 33])
def test_geglu_gemm_bounds(gpu, rng, M):
    import torch
    import e2mi
    F, K = 256, 256
    qa, as_, _, _ = _case(rng, M, 2 * F, K)
    wg = rng.integers(-127, 128, (F, K), dtype=np.int8)
    wu = rng.integers(-127, 128, (F, K), dtype=np.int8)
    sg = rng.uniform(0.001, 0.02, F).astype(np.float32)
    su = rng.uniform(0.001, 0.02, F).astype(np.float32)
    wi, si = e2mi.interleave_gate_up(wg, sg, wu, su)
    W = e2mi.DeviceWeight.from_rowmajor(wi, si)
    q = torch.full((M + GUARD_ROWS, F), SENT_I8, dtype=torch.int8, device=gpu)
    qs = torch.full((M + GUARD_ROWS, F // 128), float(SENT_F32), dtype=torch.float32, device=gpu)
    g = torch.full((M + GUARD_ROWS, F), float(SENT_F32), dtype=torch.float32, device=gpu)
    qd, sd = _t(qa, gpu), _t(as_, gpu)
    e2mi.check(e2mi.load().e2mi_i8_gemm_geglu(e2mi.stream_ptr(None), e2mi.ptr(q), e2mi.ptr(qs), e2mi.ptr(g),
                                             e2mi.ptr(qd), e2mi.ptr(sd), W.ref, M), "gemm_geglu")
    torch.cuda.synchronize()
    assert (q.cpu().numpy()[M:] == SENT_I8).all()
    assert (qs.cpu().numpy()[M:] == SENT_F32).all()
    assert (g.cpu().numpy()[M:] == SENT_F32).all()
    assert not (g.cpu().numpy()[:M] == SENT_F32).any()
