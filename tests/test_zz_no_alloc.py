"""e2mi_pool_l2_noalloc (the allocation-free variant of e2mi_pool_l2, partial sums in a static
device array) against e2mi_pool_l2 with its caller workspace, through the C ABI: bit-identical
embeddings on two calls in a row, the second smaller than the first (the array keeps the first
call's partial sums, which the second must not read), and a request beyond the array's size is
refused without touching the output."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _pool_ref(e2mi, x, valid, B, S):
    return e2mi.pool_l2(x, valid, B, S).cpu().numpy()


def _pool_noalloc(e2mi, x, valid, B, S, D):
    import torch
    out = torch.full((B, D), 7.0, device=x.device)
    rc = e2mi.load().e2mi_pool_l2_noalloc(None, e2mi.ptr(x), e2mi.ptr(valid), B, S, D, e2mi.ptr(out))
    assert rc == 0, e2mi.last_error()
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_pool_noalloc_matches_workspace_entry(gpu, rng):
    import torch
    import e2mi
    for B, S, D in [(64, 512, 768), (7, 130, 768), (3, 1000, 1280)]:
        x = _t(rng.standard_normal((B * S, D)).astype(np.float32), gpu)
        valid = (rng.random(B * S) > 0.25).astype(np.uint8)
        valid[:S] = 0                                   # an all-invalid sequence: exact zeros
        vd = _t(valid, gpu)
        want = _pool_ref(e2mi, x, vd, B, S)
        got = _pool_noalloc(e2mi, x, vd, B, S, D)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (B, S, D)
        assert np.all(got[0] == 0.0)
    # beyond the static array (8 MiB): refused, output untouched
    B, S, D = 400, 512, 768
    x = torch.zeros((B * S, D), device=gpu)
    vd = torch.ones(B * S, dtype=torch.uint8, device=gpu)
    out = torch.full((B, D), 7.0, device=gpu)
    rc = e2mi.load().e2mi_pool_l2_noalloc(None, e2mi.ptr(x), e2mi.ptr(vd), B, S, D, e2mi.ptr(out))
    assert rc == -1 and "limit" in e2mi.last_error()
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
