"""The reference checkpoint's text geometry on the device (text.c:467-478, 906-984): head_dim 512
q/k/v norm + RoPE and attention (the full-attention layers), the sliding window by position, the
PLE row kernels, and the whole engine at that geometry vs the oracle's recipe.

Bars as for the BASELINE path: f32 row outputs within 1e-5 relative of the oracle; attention per
row within cosine >= 0.9999 and max |err| <= 2e-3 * max |ctx| of the oracle's fp32 attention on the
same f16-rounded inputs, the quantized context bit-exact for the kernel's own f32 context;
embeddings within cosine >= 0.9999."""
import numpy as np
import pytest

from conftest import assert_f32_close
from model_util import oracle_model, random_batch, reference_small_config

pytestmark = pytest.mark.gpu
EPS = 1e-6


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _np(t):
    return t.cpu().numpy()


def _rowcos(a, b):
    a, b = a.astype(np.float64), b.astype(np.float64)
    return (a * b).sum(1) / (np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1) + 1e-300)


def test_qkv_norm_rope_packed_head_dim_512(gpu, oracle, rng):
    """Full-attention layer stage: H = 4, 1 kv head of 512, RoPE theta 1e6 at per-row positions."""
    import e2mi
    import torch
    H, KV, D = 4, 1, 512
    lens = [200, 56]
    M = 256
    pos = np.concatenate([np.arange(200), np.arange(56)]).astype(np.int32)
    qkv = (rng.standard_normal((M, (H + 2 * KV) * D)) * 15).astype(np.float32)
    gq = (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)
    gk = (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)
    cs, sn = oracle.rope_table(256, D, 1e6)
    q16, k16, vt16, q32, k32, v32 = e2mi.qkv_norm_rope_packed(
        _t(qkv, gpu), _t(pos, gpu), H, KV, _t(gq, gpu), _t(gk, gpu), _t(cs, gpu), _t(sn, gpu), EPS, D=D)
    r0 = 0
    for L in lens:
        rows = slice(r0, r0 + L)
        qo = oracle.rmsnorm(qkv[rows, :H * D].reshape(-1, D), gq, EPS)
        qo = oracle.rope_rows(qo, H, cs, sn).reshape(L, H * D)
        ko = oracle.rmsnorm(qkv[rows, H * D:(H + KV) * D].reshape(-1, D), gk, EPS)
        ko = oracle.rope_rows(ko, KV, cs, sn).reshape(L, KV * D)
        vo = oracle.rmsnorm(qkv[rows, (H + KV) * D:].reshape(-1, D), None, EPS).reshape(L, KV * D)
        assert_f32_close(_np(q32)[rows], qo, rtol=1e-5, atol=2e-6, what="q")
        assert_f32_close(_np(k32)[rows], ko, rtol=1e-5, atol=2e-6, what="k")
        assert_f32_close(_np(v32)[rows], vo, rtol=1e-5, atol=2e-6, what="v")
        r0 += L
    assert torch.equal(q16, q32.half()) and torch.equal(k16, k32.half())
    vt = _np(vt16.float())                              # [KV][D][M]
    assert np.array_equal(vt, _np(v32.half().float()).reshape(M, KV, D).transpose(1, 2, 0))


def _packed_attention_case(gpu, oracle, rng, valid, H, KV, D, window, scale, use_work):
    import e2mi
    import torch
    B, S = valid.shape
    rowmap, pos, start, lens, M = e2mi.pack_plan(valid)
    q = rng.standard_normal((M, H * D)).astype(np.float32)
    k = rng.standard_normal((M, KV * D)).astype(np.float32)
    v = rng.standard_normal((M, KV * D)).astype(np.float32)
    q16, k16, v16 = (_t(a, gpu).half() for a in (q, k, v))
    vt16 = v16.reshape(M, KV, D).permute(1, 2, 0).contiguous()
    work = None
    if use_work:
        work = _t(np.concatenate([e2mi.attention_work(lens, H), np.full(3, -1, np.int32)]), gpu)
    cq, cs, c32 = e2mi.attention_packed_window(q16, k16, vt16, _t(start, gpu), _t(lens, gpu), S, H, KV, D,
                                               window=window, pos=_t(pos, gpu), scale=scale, work=work)
    got = _np(c32)
    qf, kf, vf = (_np(t.float()) for t in (q16, k16, v16))
    for b in range(B):
        if lens[b] == 0:
            continue
        # the oracle runs on the padded sequence: packed rows scattered back to their positions
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
    qo, so = oracle.quantize(got)
    live = rowmap >= 0
    assert np.array_equal(_np(cq)[live], qo[live]) and np.array_equal(_np(cs)[live], so[live])
    return got


@pytest.mark.parametrize("use_work", [False, True])
def test_attention_head_dim_512(gpu, oracle, rng, use_work):
    """Full-attention layers: 4 query heads on 1 kv head of 512, no window, sequences of 1..600."""
    valid = np.zeros((4, 600), np.uint8)
    for b, L in enumerate((600, 333, 1, 129)):
        valid[b, :L] = 1
    _packed_attention_case(gpu, oracle, rng, valid, 4, 1, 512, 0, 1.0 / 16, use_work)


@pytest.mark.parametrize("holes", [False, True])
def test_attention_sliding_window(gpu, oracle, rng, holes):
    """Sliding layers: 4 heads on 2 kv heads of 256, |i-j| <= 512 by position; sequences longer
    than the window (1100, 700), at its edge (513) and short (60); with holes the packed index and
    the position differ and the window follows the position (text.c:542-546)."""
    S = 1100
    valid = np.zeros((4, S), np.uint8)
    for b, L in enumerate((1100, 700, 513, 60)):
        valid[b, :L] = 1
    if holes:
        valid[0, 200:260] = 0
        valid[1, rng.random(S) < 0.2] = 0
    got = _packed_attention_case(gpu, oracle, rng, valid, 4, 2, 256, 512, 1.0 / 16, True)
    assert np.isfinite(got).all()


def test_add_norm_scale_quant_and_scale_norm(gpu, oracle, rng):
    import e2mi
    M, D = 300, 512
    src = (rng.standard_normal((M, D)) * 20).astype(np.float32)
    res = rng.standard_normal((M, D)).astype(np.float32)
    ga = (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)
    gn = (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)
    ls = np.float32(0.8125)
    # x = (norm_add) * layer_scalar, then the next norm + quant
    x, xn, q, qs = e2mi.add_norm_scale_quant(_t(src, gpu), _t(res, gpu), _t(ga, gpu), float(ls), _t(gn, gpu), EPS)
    xo = oracle.norm_add(src, res, ga, EPS) * ls
    assert_f32_close(_np(x), xo, rtol=1e-5, atol=1e-5, what="norm_add * scale")
    xno, _ = oracle.norm_split(_np(x), gn, EPS)
    assert_f32_close(_np(xn), xno, rtol=1e-5, atol=1e-6, what="next norm")
    qg, sg = oracle.quantize(_np(xn))
    assert np.array_equal(_np(q), qg) and np.array_equal(_np(qs), sg)
    # no next norm: x itself quantized (the PLE gate's operand)
    x2, xn2, q2, qs2 = e2mi.add_norm_scale_quant(_t(src, gpu), _t(res, gpu), _t(ga, gpu), 1.0, None, EPS)
    assert xn2 is None
    assert_f32_close(_np(x2), oracle.norm_add(src, res, ga, EPS), rtol=1e-5, atol=1e-5, what="norm_add")
    qg2, sg2 = oracle.quantize(_np(x2))
    assert np.array_equal(_np(q2), qg2) and np.array_equal(_np(qs2), sg2)
    # the per-layer input norm: rms(x * ple_scale) * gamma per 512-slice, in place
    rows = (rng.standard_normal((M * 3, D)) * 1e-3).astype(np.float32)
    s = float(np.float32(1 / np.sqrt(512.0)))
    t = _t(rows, gpu)
    e2mi.scale_norm(t, s, _t(gn, gpu), EPS, out=t)
    want = oracle.rmsnorm((rows * np.float32(s)).astype(np.float32), gn, EPS)
    assert_f32_close(_np(t), want, rtol=1e-5, atol=1e-6, what="scale_norm")


@pytest.mark.parametrize("M", [4096, 1000])
def test_ple_gate_gemm_gelu_mul(gpu, oracle, rng, M):
    """The PLE gate GEMM with gelu(gate) * ple slice quantized in its epilogue (text.c:906-913),
    the slice a column range of the [rows][layers * 512] per-layer inputs."""
    import e2mi
    K = N = 512
    qa = rng.integers(-127, 128, (M, K), dtype=np.int8)
    as_ = rng.uniform(0.001, 0.01, (M, K // 128)).astype(np.float32)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    ws = rng.uniform(0.001, 0.02, N).astype(np.float32)
    ple = rng.standard_normal((M, 3 * N)).astype(np.float32)
    W = e2mi.DeviceWeight.from_rowmajor(w, ws)
    pt = _t(ple, gpu)
    q, qs, g = e2mi.i8_gemm_gelu_mul(_t(qa, gpu), _t(as_, gpu), W, pt[:, N:2 * N])
    gate = oracle.i8_gemm(qa, as_, w, ws)
    go, _, _ = oracle.gelu_mul_quant(gate, np.ascontiguousarray(ple[:, N:2 * N]))
    gk = _np(g)
    assert_f32_close(gk, go, rtol=1e-4, atol=1e-4, what="gelu(gate) * ple")
    qo, so = oracle.quantize(gk)
    assert np.array_equal(_np(q), qo) and np.array_equal(_np(qs).view(np.uint32), so.view(np.uint32))
    # the slice of another layer gives other bytes: the multiplier is read at its own columns
    q2, _, _ = e2mi.i8_gemm_gelu_mul(_t(qa, gpu), _t(as_, gpu), W, pt[:, 2 * N:], want_g=False)
    assert not np.array_equal(_np(q2), _np(q))


@pytest.fixture(scope="module")
def ref_setup(gpu):
    import e2mi
    from oracle.binding import Oracle
    o = Oracle()
    m = e2mi.Model.synthetic(reference_small_config(e2mi, n_layers=6, attn_scale=1 / 16), 77)
    eng = e2mi.Engine(m, max_rows=4096)
    return e2mi, o, m, eng


def test_engine_reference_geometry_vs_oracle(ref_setup, rng):
    """Six layers of the reference geometry (sliding layers 0-4, full layer 5, PLE, embed_proj to
    768) with tempered logits (see test_gpu_encoder: deeper stacks at scale 1.0 are chaotic)."""
    e2mi, o, m, eng = ref_setup
    om = oracle_model(o, m)
    S = 1100
    ids = rng.integers(0, 1000, (4, S)).astype(np.int32)
    valid = np.zeros((4, S), np.uint8)
    for b, L in enumerate((1100, 640, 90, 0)):
        valid[b, :L] = 1
    valid[1, 100:130] = 0                              # a hole: positions and packed index differ
    got = eng.embed_batch(ids, valid)
    want = om.encode(ids, valid)
    assert got.shape == (4, 768)
    cos = _rowcos(got[:3], want[:3])
    print("reference-geometry 6-layer cos", cos)
    assert cos.min() >= 0.9999, cos
    assert np.all(got[3] == 0) and np.all(want[3] == 0)
    # the graph replay gives the same embeddings, bit for bit
    assert np.array_equal(eng.embed_batch(ids, valid), got)


def test_engine_reference_geometry_scale_one(gpu, rng):
    """One layer at the reference's unscaled logits, a sequence past the window."""
    import e2mi
    from oracle.binding import Oracle
    o = Oracle()
    m = e2mi.Model.synthetic(reference_small_config(e2mi, n_layers=1), 5)
    eng = e2mi.Engine(m, max_rows=4096)
    om = oracle_model(o, m)
    ids, valid = random_batch(rng, 3, 800, 1000, min_len=500)
    got = eng.embed_batch(ids, valid)
    cos = _rowcos(got, om.encode(ids, valid))
    print("reference-geometry 1-layer cos", cos)
    assert cos.min() >= 0.9999, cos


def test_engine_reference_geometry_refusals(ref_setup):
    """Paths built for the BASELINE geometry only fail loudly here."""
    e2mi, o, m, eng = ref_setup
    with pytest.raises(e2mi.E2MIError, match="packed"):
        eng.set_packing(False)
    with pytest.raises(e2mi.E2MIError, match="int8 attention"):
        eng.set_attention("i8")


def test_engine_reference_geometry_from_e8cq(ref_setup, rng, tmp_path):
    """The production weight path at this geometry (an E8CQ cache with the PLE / embed_proj tensors,
    q8cache.c:242-385, re-laid out on the device) gives the in-memory model's embeddings, bit for bit."""
    e2mi, o, m, eng = ref_setup
    p = str(tmp_path / "ref.e8cq")
    m.save_e8cq(p)
    m2 = e2mi.Model.load_e8cq(p, m.config)
    eng2 = e2mi.Engine(m2, max_rows=4096)
    ids, valid = random_batch(rng, 3, 700, 1000, min_len=100)
    assert np.array_equal(eng2.embed_batch(ids, valid), eng.embed_batch(ids, valid))
