"""The encoder on the device (e2mi_engine) vs the oracle's text recipe at the BASELINE geometry
(hidden 768, FFN 1152, 3q/1kv heads of 256), random-init int8 weights.

Bars: embeddings within cosine >= 0.9999 of the oracle; sublayer outputs
(configs 2 and 3) within cosine >= 0.9999 and 1e-4 relative where no f16 stage intervenes."""
import numpy as np
import pytest

from conftest import cosine
from model_util import NORMS, Q8, lname, oracle_model, random_batch, small_config

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def setup(gpu):
    import e2mi
    from oracle.binding import Oracle
    o = Oracle()
    m = e2mi.Model.synthetic(small_config(e2mi, n_layers=2), 2026)
    eng = e2mi.Engine(m, max_rows=4096)
    om = oracle_model(o, m)
    return e2mi, o, m, eng, om


def _rowcos(a, b):
    a, b = a.astype(np.float64), b.astype(np.float64)
    return (a * b).sum(1) / (np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1) + 1e-300)


def test_device_name(setup):
    e2mi, o, m, eng, om = setup
    assert "gfx950" in eng.device


def test_encoder_vs_oracle_reference_scale(setup, rng):
    """One layer with the reference's unscaled logits (text.c:8-9). Deeper random-init stacks at
    scale 1.0 are chaotic: a 1-ulp change of the embedding table alone moves the oracle's own
    embeddings to cosine 0.9998 after 2 layers and 0.965 after 8, so depth is tested below with
    tempered logits, where the f32 reproducibility floor stays above 0.99998 at 24 layers."""
    e2mi, o, m, eng, om = setup
    om1 = oracle_model(o, m, n_layers=1)
    ids, valid = random_batch(rng, 4, 128, 1000, min_len=1)
    valid[3] = 0                                       # an all-padding sequence
    eng.set_layer_limit(1)
    try:
        got = eng.embed_batch(ids, valid)
        calls, kern, ms = eng.stats()
    finally:
        eng.set_layer_limit(0)
    want = om1.encode(ids, valid)
    cos = _rowcos(got[:3], want[:3])
    print("1-layer cos", cos)
    assert cos.min() >= 0.9999, cos
    assert np.all(got[3] == 0) and np.all(want[3] == 0)
    assert np.allclose(np.linalg.norm(got[:3], axis=1), 1, atol=1e-5)
    # embedding; per layer the fused q|k|v GEMM (norms and RoPE in its epilogue), attention, O with
    # the add-norm in its epilogue, GeGLU, down with the add-norm; pooling (two kernels)
    assert calls >= 1 and kern == 1 + 5 + 2


def test_encoder_24_layers_vs_oracle(gpu, rng):
    """The full 24-layer stack (BASELINE config 4 geometry, reduced vocab and batch) with logits
    scaled by 1/sqrt(head_dim)."""
    import e2mi
    from oracle.binding import Oracle
    o = Oracle()
    cfg = small_config(e2mi, n_layers=24)
    cfg.attn_scale = 1.0 / 16
    m = e2mi.Model.synthetic(cfg, 4004)
    eng = e2mi.Engine(m, max_rows=2048)
    om = oracle_model(o, m)
    ids, valid = random_batch(rng, 4, 128, 1000, min_len=30)
    got = eng.embed_batch(ids, valid)
    want = om.encode(ids, valid, nthreads=16)
    cos = _rowcos(got, want)
    print("24-layer cos", cos)
    assert cos.min() >= 0.9999, cos


def test_batch_equals_single(setup, rng):
    """test_text_batch.c: a padded batch row == the same sequence alone (bit-exact here: every
    kernel's arithmetic for a row is independent of the other rows)."""
    e2mi, o, m, eng, om = setup
    ids, valid = random_batch(rng, 3, 64, 1000, min_len=5)
    batch = eng.embed_batch(ids, valid)
    for b in range(3):
        L = int(valid[b].sum())
        single = eng.embed_batch(ids[b:b + 1, :L], None)
        assert np.array_equal(single[0], batch[b])


def test_replay_and_device_path(setup, rng):
    import torch
    e2mi, o, m, eng, om = setup
    ids, valid = random_batch(rng, 2, 100, 1000)
    a = eng.embed_batch(ids, valid)                    # first call of the shape: eager + record
    b = eng.embed_batch(ids, valid)                    # graph replay
    c = eng.embed_batch(ids, valid)
    assert np.array_equal(a, b) and np.array_equal(a, c)
    dev = torch.device("cuda:0")
    idt, vt = torch.from_numpy(ids).to(dev), torch.from_numpy(valid).to(dev)
    out = torch.empty((2, 768), device=dev)
    for _ in range(3):                                  # eager, record, replay
        eng.embed_batch_device(idt, vt, out)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), a)


def test_validation_leaves_output_untouched(setup, rng):
    e2mi, o, m, eng, om = setup
    ids, valid = random_batch(rng, 2, 16, 1000)
    out = np.full((2, 768), 7.0, np.float32)
    bad = ids.copy()
    bad[1, 3] = 1000                                    # out of vocabulary
    lib = e2mi.load()
    rc = lib.e2mi_text_embed_batch(eng.h, e2mi.ptr(bad), e2mi.ptr(valid), 2, 16, e2mi.ptr(out))
    assert rc == -1 and "out of range" in e2mi.last_error() and np.all(out == 7.0)
    too_long = np.zeros((1, 513), np.int32)
    rc = lib.e2mi_text_embed_batch(eng.h, e2mi.ptr(too_long), None, 1, 513, e2mi.ptr(out))
    assert rc == -1 and np.all(out == 7.0)


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("B", [4, 32])
def test_config3_attention_sublayer(setup, rng, B):
    """BASELINE config 3 (B x S with padding, QKV 768->1280, q/k norm, RoPE, GQA 3:1, O 768->768),
    composed from the kernel entry points, vs the oracle's attention sublayer; B = 32 x S = 512 with
    lengths U[64, 512] is the configuration as stated."""
    import torch
    e2mi, o, m, eng, om = setup
    dev = torch.device("cuda:0")
    S = 512
    x = rng.standard_normal((B * S, 768)).astype(np.float32)
    ids, valid = random_batch(rng, B, S, 1000, min_len=64)
    valid = valid.reshape(-1)
    want = om.attention_sublayer(0, x, valid, B, S, nthreads=16)
    L = om._keep[0][0]
    Wqkv = e2mi.DeviceWeight.from_rowmajor(L["wqkv"], L["sqkv"])
    Wo = e2mi.DeviceWeight.from_rowmajor(L["wo"], L["so"])
    cs, sn = o.rope_table(S, 256, 10000.0)
    q, s = e2mi.quantize(_t(x, dev))
    qkv = e2mi.i8_gemm(q, s, Wqkv)
    q16, k16, vt16, *_ = e2mi.qkv_norm_rope(qkv, S, 3, 1, _t(L["q_norm"], dev), _t(L["k_norm"], dev),
                                            _t(cs, dev), _t(sn, dev), want_f32=False)
    cq, csc, _ = e2mi.attention(q16, k16, vt16, _t(valid, dev), B, S, 3, 1, want_f32=False)
    got = e2mi.i8_gemm(cq, csc, Wo).cpu().numpy()
    v = valid.astype(bool)
    rc = _rowcos(got[v], want[v])
    q = np.quantile(1 - rc, [0.5, 0.9, 0.99, 0.999, 1.0])
    print("attn sublayer cos", cosine(got[v], want[v]), "1-cos quantiles 50/90/99/99.9/100 %", q,
          "rows below 0.9999:", int((rc < 0.9999).sum()), "of", int(v.sum()))
    # The f16 attention of config 3 rounds q and k to f16 (relative 2^-11) before QK^T; at the
    # reference's logit scale 1.0 (logit std ~16) that moves a logit by ~0.01, which is what
    # separates the rows from the f32 oracle (measured on this seed: 1 - cos median 5e-6, max
    # 7e-5). Every row holds the north star's 0.9999.
    assert cosine(got[v], want[v]) >= 0.9999
    assert rc.min() >= 0.9999


def test_config2_ffn_sublayer(setup, rng):
    """x [2048 x 768] -> RMSNorm -> gate|up int8 GEMMs -> GELU-tanh * up ->
    requantize -> down GEMM -> norm_add residual (text.c:893-903,949-953)."""
    import torch
    e2mi, o, m, eng, om = setup
    dev = torch.device("cuda:0")
    x = rng.standard_normal((2048, 768)).astype(np.float32)
    want = om.ffn_sublayer(0, x)
    L = om._keep[0][0]
    wi, si = e2mi.interleave_gate_up(L["wgate"], L["sgate"], L["wup"], L["sup"])
    Wgu = e2mi.DeviceWeight.from_rowmajor(wi, si)
    Wd = e2mi.DeviceWeight.from_rowmajor(L["wdown"], L["sdown"])
    xt = _t(x, dev)
    xn, q, qs = e2mi.norm_quant(xt, _t(L["pre_ffn_ln"], dev), 1e-6, want_xn=False)
    gq, gs, _ = e2mi.i8_gemm_geglu(q, qs, Wgu, want_g=False)
    tmp = e2mi.i8_gemm(gq, gs, Wd)
    out, *_ = e2mi.add_norm_quant(tmp, xt, _t(L["post_ffn_ln"], dev), None, 1e-6)
    got = out.cpu().numpy()
    rc = _rowcos(got, want)
    print("ffn sublayer row-cos min", rc.min())
    # elementwise differences come from +-1 requantization steps at rounding boundaries (the
    # reference's own byte rule); the bar is the BASELINE one, cosine >= 0.9999 per row
    assert rc.min() >= 0.9999


def test_config4_full_size_properties(gpu, rng):
    """BASELINE config 4 at its stated size: 24 layers at the reference recipe's attention scale
    1.0, vocabulary 262144, B = 64 x S = 512 with lengths U[64, 512]. No oracle comparison at this
    depth (random-init stacks at scale 1.0 are chaotic, see above); size-independent properties
    instead: every embedding finite and unit-norm, packed and padded-rows forwards bit-identical,
    graph replays bit-identical to the eager first call, and a sample of sequences embedded alone
    bit-identical to their batch rows (the default: split key ranges off, so no embedding depends on
    its batch-mates). Split and unsplit attention agree to cosine 0.9999 after one layer, and the
    opt-in "auto" rule splits a lone long sequence."""
    import torch
    import e2mi
    cfg = small_config(e2mi, n_layers=24, vocab=262144)
    m = e2mi.Model.synthetic(cfg, 4044)
    eng = e2mi.Engine(m, max_rows=64 * 512)
    B, S = 64, 512
    ids = rng.integers(0, cfg.vocab, (B, S)).astype(np.int32)
    lens = rng.integers(64, S + 1, B)
    valid = (np.arange(S)[None, :] < lens[:, None]).astype(np.uint8)
    first = eng.embed_batch(ids, valid)                 # eager + graph record (blocks fill the device)
    assert np.all(np.isfinite(first))
    assert np.abs(np.linalg.norm(first.astype(np.float64), axis=1) - 1).max() < 1e-5
    dev = torch.device("cuda:0")
    out = torch.empty((B, cfg.hidden), device=dev)
    for _ in range(2):                                  # replays, device entry
        eng.embed_batch_device(_t(ids, dev), _t(valid, dev), out)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), first)
    eng.set_packing(False)
    try:
        padded = eng.embed_batch(ids, valid)
    finally:
        eng.set_packing(True)
    assert np.array_equal(padded, first)
    for b in rng.choice(B, 4, replace=False):
        L = int(lens[b])
        single = eng.embed_batch(ids[b:b + 1, :L], None)
        assert np.array_equal(single[0], first[b]), b
    # one layer: split against unsplit over the whole batch; the default rule on a lone sequence
    eng.set_layer_limit(1)
    one_unsplit = eng.embed_batch(ids, valid)
    eng.set_split("on")
    one_split = eng.embed_batch(ids, valid)
    cos = (one_split * one_unsplit).sum(1) / (np.linalg.norm(one_split, axis=1) * np.linalg.norm(one_unsplit, axis=1))
    assert cos.min() >= 0.9999, cos.min()
    assert not np.array_equal(one_split, one_unsplit)  # sequences over 256 tokens did split
    b = int(np.argmax(lens))
    lone_on = eng.embed_batch(ids[b:b + 1, :int(lens[b])], None)
    eng.set_split("auto")
    assert np.array_equal(eng.embed_batch(ids[b:b + 1, :int(lens[b])], None), lone_on)
    eng.set_layer_limit(0)
