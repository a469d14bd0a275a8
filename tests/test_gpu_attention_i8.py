"""The int8 attention variant (the reference's text.c:638-700 path) on packed batches.

Q, K and V^T bytes and scales are bit-exact with the oracle's quantizers (the reference's, pinned
in test_oracle_ref.py). The context is compared with the oracle's int8 attention: both quantize the
same values the same way and fold the int8 GEMMs in the same order, but the softmax's exponentials
and sums are computed differently (the GPU's exp, an online sum), so a probability can land on the
other side of a quantization step; the bar is a per-(row, head) cosine >= 0.9999 and an absolute
error <= 2e-3 of max|v|. On the reference's own attention-test inputs the result is within its
int8 bar of a float64 attention (2e-2, test_text_attention.c:69-71).
"""
import numpy as np
import pytest

from test_oracle_math import _attention_f64, _ref_test_inputs

pytestmark = pytest.mark.gpu

D = 256


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _np(t):
    return t.cpu().numpy()


def _packed(rng, e2mi, lens, S):
    B = len(lens)
    valid = np.zeros((B, S), np.uint8)
    for b, L in enumerate(lens):
        valid[b, :L] = 1
    return e2mi.pack_plan(valid)


def _ws_layout(M, B, max_len, H, KV):
    """The workspace layout of attn_i8.hip (i8_ws): q8, qs, k8, ks, vt8 ([KV][D][2 M]), vpart, vs."""
    al = lambda x: (x + 255) & ~255
    nch = (max_len + 63) // 64
    q8 = 0
    qs = q8 + al(M * H * D)
    k8 = qs + al(M * H * 2 * 4)
    ks = k8 + al(M * KV * D)
    vt8 = ks + al(M * KV * 4)
    vpart = vt8 + al(KV * D * 2 * M)
    vs = vpart + al(B * KV * nch * D * 4)
    return dict(q8=q8, qs=qs, k8=k8, ks=ks, vt8=vt8, vs=vs)


def _inputs(rng, M, H, KV, scale_qk=0.3):
    q = (rng.standard_normal((M, H * D)) * scale_qk).astype(np.float32)
    k = (rng.standard_normal((M, KV * D)) * scale_qk).astype(np.float32)
    v = rng.standard_normal((M, KV * D)).astype(np.float32)
    return q, k, v


def _cos_rows(a, b):
    a, b = a.reshape(-1, D).astype(np.float64), b.reshape(-1, D).astype(np.float64)
    return (a * b).sum(1) / (np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1))


@pytest.mark.parametrize("H,KV,lens", [(3, 1, [512, 300, 130]), (4, 2, [197, 64, 1, 256])])
def test_i8_quantized_operands_bit_exact(gpu, oracle, rng, H, KV, lens):
    import torch
    import e2mi
    S = max(lens)
    rowmap, pos, start, plen, M = _packed(rng, e2mi, lens, S)
    q, k, v = _inputs(rng, M, H, KV)
    B = len(lens)
    nbytes = e2mi.load().e2mi_attention_i8_workspace_bytes(M, B, S, H, KV)
    ws = torch.zeros(nbytes + 256, dtype=torch.uint8, device=gpu)
    e2mi.attention_i8_packed(_t(q, gpu), _t(k, gpu), _t(v, gpu), _t(start, gpu), _t(plen, gpu), S, H, KV,
                             workspace=ws)
    torch.cuda.synchronize()
    base = (ws.data_ptr() + 255) & ~255
    raw = _np(ws)[base - ws.data_ptr():]
    lay = _ws_layout(M, B, S, H, KV)
    q8 = raw[lay["q8"]:lay["q8"] + M * H * D].view(np.int8).reshape(M, H, D)
    qs = raw[lay["qs"]:lay["qs"] + M * H * 8].view(np.float32).reshape(M, H, 2)
    k8 = raw[lay["k8"]:lay["k8"] + M * KV * D].view(np.int8).reshape(M, KV, D)
    ks = raw[lay["ks"]:lay["ks"] + M * KV * 4].view(np.float32).reshape(M, KV)
    vt8 = raw[lay["vt8"]:lay["vt8"] + KV * D * 2 * M].view(np.int8).reshape(KV, D, 2 * M)
    vs = raw[lay["vs"]:lay["vs"] + B * KV * D * 4].view(np.float32).reshape(B, KV, D)
    live = rowmap >= 0
    # Q per (row, head, 128 dims): the activation quantizer
    qo, qso = oracle.quantize(q.reshape(M * H, D))
    assert np.array_equal(q8.reshape(M * H, D)[np.repeat(live, H)], qo[np.repeat(live, H)])
    assert np.array_equal(qs.reshape(M * H, 2)[np.repeat(live, H)].view(np.uint32), qso[np.repeat(live, H)].view(np.uint32))
    # K per key row, V^T per (sequence, dim): the weight quantizer (e2_q8w_from_f32)
    for kv in range(KV):
        wq, sc, _ = oracle.q8w_from_f32(k[live][:, kv * D:(kv + 1) * D])
        n = int(live.sum())
        assert np.array_equal(k8[live][:, kv], oracle.q8w_unpack(wq, n, D))
        assert np.array_equal(ks[live][:, kv].view(np.uint32), sc[:n].view(np.uint32))
        for b, L in enumerate(lens):
            if L == 0:
                continue
            r = slice(start[b], start[b] + L)
            wq, sc, _ = oracle.q8w_from_f32(np.ascontiguousarray(v[r][:, kv * D:(kv + 1) * D].T))
            # sequence b's keys sit at V^T columns 2 start[b] + j (16-byte aligned tiles)
            assert np.array_equal(vt8[kv][:, 2 * start[b]:2 * start[b] + L], oracle.q8w_unpack(wq, D, L))
            assert np.array_equal(vs[b, kv].view(np.uint32), sc[:D].view(np.uint32))


@pytest.mark.parametrize("H,KV,lens", [(3, 1, [512, 300, 130]), (4, 2, [197, 64, 1, 256, 33])])
def test_attention_i8_vs_oracle(gpu, oracle, rng, H, KV, lens):
    import torch
    import e2mi
    S = max(lens)
    rowmap, pos, start, plen, M = _packed(rng, e2mi, lens, S)
    q, k, v = _inputs(rng, M, H, KV)
    qd, kd, vd, sd, ld = _t(q, gpu), _t(k, gpu), _t(v, gpu), _t(start, gpu), _t(plen, gpu)
    cq, cs, c32 = e2mi.attention_i8_packed(qd, kd, vd, sd, ld, S, H, KV)
    # the same through a longest-first work list (with idle slots), bit for bit
    work = _t(np.concatenate([e2mi.attention_work(plen, H), np.full(3, -1, np.int32)]), gpu)
    wq, ws_, w32 = e2mi.attention_i8_packed(qd, kd, vd, sd, ld, S, H, KV, work=work)
    torch.cuda.synchronize()
    assert torch.equal(wq, cq) and torch.equal(ws_, cs) and torch.equal(w32, c32)
    got = _np(c32)
    live = rowmap >= 0
    assert np.all(_np(cq)[~live] == 0) and np.all(_np(cs)[~live] == 0)
    for b, L in enumerate(lens):
        r = slice(start[b], start[b] + L)
        want = oracle.attention_i8(q[r], k[r], v[r], H, KV, D)
        g = got[r]
        assert np.abs(g - want).max() <= 2e-3 * np.abs(v[r]).max()
        assert _cos_rows(g, want).min() >= 0.9999
    # the quantized context is the reference quantizer applied to the f32 context
    qo, so = oracle.quantize(got[live])
    assert np.array_equal(_np(cq)[live], qo) and np.array_equal(_np(cs)[live].view(np.uint32), so.view(np.uint32))


def test_attention_i8_reference_inputs_within_bar(gpu, rng):
    """The reference attention test's inputs (test_text_attention.c:47-53) at its lengths, against a
    float64 attention: within the reference's int8 bar."""
    import e2mi
    H, KV = 3, 1
    lens = [512, 300]
    S = max(lens)
    rowmap, pos, start, plen, M = _packed(rng, e2mi, lens, S)
    q = np.zeros((M, H * D), np.float32)
    k = np.zeros((M, KV * D), np.float32)
    v = np.zeros((M, KV * D), np.float32)
    for b, L in enumerate(lens):
        qq, kk, vv = _ref_test_inputs(L, H, KV, D)
        q[start[b]:start[b] + L], k[start[b]:start[b] + L], v[start[b]:start[b] + L] = qq, kk, vv
    _, _, c32 = e2mi.attention_i8_packed(_t(q, gpu), _t(k, gpu), _t(v, gpu), _t(start, gpu), _t(plen, gpu), S, H, KV)
    got = _np(c32)
    for b, L in enumerate(lens):
        r = slice(start[b], start[b] + L)
        assert np.abs(got[r] - _attention_f64(q[r], k[r], v[r], H, KV, D)).max() < 2e-2


def test_attention_i8_close_to_f16_path(gpu, oracle, rng):
    """Both attention paths approximate the same softmax attention: per-(row, head) cosine >= 0.999."""
    import e2mi
    H, KV = 3, 1
    lens = [400, 160]
    S = max(lens)
    rowmap, pos, start, plen, M = _packed(rng, e2mi, lens, S)
    q, k, v = _inputs(rng, M, H, KV)
    sd, ld = _t(start, gpu), _t(plen, gpu)
    _, _, c8 = e2mi.attention_i8_packed(_t(q, gpu), _t(k, gpu), _t(v, gpu), sd, ld, S, H, KV)
    vt = np.ascontiguousarray(v.reshape(M, KV, D).transpose(1, 2, 0))  # [KV][D][M]
    _, _, c16 = e2mi.attention_packed(_t(q.astype(np.float16), gpu), _t(k.astype(np.float16), gpu),
                                      _t(vt.astype(np.float16), gpu), sd, ld, S, H, KV)
    live = rowmap >= 0
    assert _cos_rows(_np(c8)[live], _np(c16)[live]).min() >= 0.999


def test_attention_i8_rejects_bad_geometry(gpu):
    import e2mi
    lib = e2mi.load()
    assert lib.e2mi_attention_i8_packed(None, None, None, None, 17, None, None, 1, 8, 3, 1, 256, None,
                                        None, None, None, None, 0) == -1
    assert b"M % 16" in lib.e2mi_last_error() or b"head_dim" in lib.e2mi_last_error()


def test_engine_int8_attention_vs_oracle(gpu, rng):
    """The engine with the int8 attention selected (E2_ATTN_TEXT=i8's setter) against the oracle's
    text recipe with the same selection: one layer at the reference's scale 1.0, right-padded
    sequences of 1 to 300 tokens (those under 32 tokens take the f16 / f32 path in both); embeddings
    within the north star's cosine bar. The f16 engine on the same batch is farther from it."""
    import e2mi
    from model_util import oracle_model, random_batch, small_config
    from oracle.binding import Oracle
    o = Oracle()
    m = e2mi.Model.synthetic(small_config(e2mi, n_layers=1), 4242)
    eng = e2mi.Engine(m, max_rows=2048)
    ids, valid = random_batch(rng, 6, 300, 1000, min_len=1)
    valid[0, :] = 1                                    # a full-length sequence
    valid[1, 20:] = 0                                  # a short one (f16 / f32 path)
    want = oracle_model(o, m, attn_i8=True).encode(ids, valid)
    f16 = eng.embed_batch(ids, valid)
    eng.set_attention("i8")
    try:
        got = eng.embed_batch(ids, valid)
        again = eng.embed_batch(ids, valid)            # graph replay
    finally:
        eng.set_attention("f16")
    assert np.array_equal(got, again)
    cos = (got * want).sum(1) / (np.linalg.norm(got, axis=1) * np.linalg.norm(want, axis=1))
    cos16 = (f16 * want).sum(1) / (np.linalg.norm(f16, axis=1) * np.linalg.norm(want, axis=1))
    print("engine int8 attention cos", cos, "f16 engine vs int8 oracle", cos16)
    assert cos.min() >= 0.9999
    assert np.array_equal(f16, eng.embed_batch(ids, valid))  # switched back
    with pytest.raises(Exception):
        e2mi.Engine(e2mi.Model.synthetic(small_config(e2mi, n_layers=1), 1), max_rows=512).set_attention("f32")
