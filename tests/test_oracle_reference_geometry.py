"""The oracle's recipe for the reference checkpoint's geometry (text.c:467-478, 906-984: sliding
window, per-layer head_dim / kv heads / RoPE theta, PLE, layer_scalar, embed_proj), pinned by what
the mathematics fixes and by composition of the stage functions that tests/test_oracle_ref.py and
tests/test_oracle_math.py pin against the reference:

- the window restricts the keys to |i-j| <= window (W_q = W_k = 0 makes attention the mean of the
  valid V rows of the window: an off-by-one or an exclusive bound changes the key set);
- a layer whose attention, FFN and PLE projection weights are zero maps x to layer_scalar * x
  exactly (the PLE block's placement and the scale's order are visible);
- the PLE block reads its own layer's slice of the per-layer inputs, at their row stride;
- the per-layer inputs are rms(GEMM(quant(x)) * ple_scale) * gamma per ple_dim slice;
- a full-attention layer runs at head_dim 512 with 1 kv head and RoPE theta 1e6, a sliding layer
  at 256 / 2 / 1e4 with the window;
- with no layers the embedding is l2(meanpool(embed_proj(quant(rms(table[id] * scale) * final)))).
"""
import sys

import numpy as np
import pytest

from conftest import assert_f32_close
from model_util import oracle_model, reference_small_config


@pytest.fixture(scope="module")
def e2mi_mod():
    import e2mi
    return e2mi


def _model(e2mi, oracle, n_layers=6, seed=3, **over):
    cfg = reference_small_config(e2mi, n_layers=n_layers, **over)
    m = e2mi.Model.synthetic(cfg, seed)
    return m, oracle_model(oracle, m)


def _zero(om, l, names):
    L = om._keep[0][l]
    for n in names:
        L[n][...] = 0


def test_window_closed_form(oracle, rng):
    """W_q = W_k = 0: every score is 0, so query i's context is the mean of the valid V rows j with
    |i-j| <= window (text.c:542-546)."""
    S, H, KV, D, W = 40, 4, 2, 256, 3
    q = np.zeros((S, H * D), np.float32)
    k = np.zeros((S, KV * D), np.float32)
    v = rng.standard_normal((S, KV * D)).astype(np.float32)
    valid = np.ones(S, np.uint8)
    valid[[5, 6, 20]] = 0
    got = oracle.attention(q, k, v, valid, H, KV, D, window=W)
    for i in range(S):
        if not valid[i]:
            assert not got[i].any()
            continue
        keys = [j for j in range(max(0, i - W), min(S, i + W + 1)) if valid[j]]
        for h in range(H):
            kv = h // (H // KV)
            want = v[keys, kv * D:(kv + 1) * D].astype(np.float64).mean(0)
            assert np.abs(got[i, h * D:(h + 1) * D] - want).max() < 1e-5, (i, h)
    # a window covering the sequence is no window, bit for bit
    full = oracle.attention(q, k, v, valid, H, KV, D)
    assert np.array_equal(oracle.attention(q, k, v, valid, H, KV, D, window=S), full)
    # and the window matters where it cuts
    assert np.abs(got - full).max() > 0.1


def test_zero_layer_is_layer_scale(e2mi_mod, oracle, rng):
    m, om = _model(e2mi_mod, oracle, n_layers=2)
    for l in range(2):
        _zero(om, l, ("wqkv", "wo", "wgate", "wup", "wdown", "wple_proj"))
    B, S = 2, 24
    x = (2 * rng.standard_normal((B * S, 512))).astype(np.float32)
    valid = np.ones((B, S), np.uint8)
    valid[1, 15:] = 0
    ple = om.ple_inputs(x)
    for l in range(2):
        ls = np.float32(om._keep[0][l]["layer_scalar"])
        assert ls != 1
        got = om.layer_ple(l, x, ple, valid, B, S)
        assert np.array_equal(got, x * ls), l


def test_ple_block_slice_and_stride(e2mi_mod, oracle, rng):
    """Attention and FFN zero, PLE weights live: layer l's block reads slice l of every row."""
    m, om = _model(e2mi_mod, oracle, n_layers=3)
    for l in range(3):
        _zero(om, l, ("wqkv", "wo", "wgate", "wup", "wdown"))
    B, S, P, NL = 2, 16, 512, 3
    x = (2 * rng.standard_normal((B * S, 512))).astype(np.float32)
    valid = np.ones((B, S), np.uint8)
    ple = np.zeros((B * S, NL * P), np.float32)
    ple[:, P:2 * P] = rng.standard_normal((B * S, P)).astype(np.float32)  # only layer 1's slice
    L0, L1 = om._keep[0][0], om._keep[0][1]
    assert np.array_equal(om.layer_ple(0, x, ple, valid, B, S), x * np.float32(L0["layer_scalar"]))
    got = om.layer_ple(1, x, ple, valid, B, S)
    eps = 1e-6
    qa, as_ = oracle.quantize(x)
    gate = oracle.i8_gemm(qa, as_, L1["wple_gate"], L1["sple_gate"])
    _, qg, gs = oracle.gelu_mul_quant(gate, np.ascontiguousarray(ple[:, P:2 * P]))
    tmp = oracle.i8_gemm(qg, gs, L1["wple_proj"], L1["sple_proj"])
    want = oracle.norm_add(tmp, x, L1["ple_norm"], eps) * np.float32(L1["layer_scalar"])
    assert np.array_equal(got, want)
    # the slice of the wrong layer (or a contiguous stride) would give the identity branch
    assert np.abs(got - x * np.float32(L1["layer_scalar"])).max() > 0.1


def test_ple_inputs_closed_form(e2mi_mod, oracle, rng):
    m, om = _model(e2mi_mod, oracle, n_layers=2)
    ex = om._keep[3]
    x = (rng.standard_normal((6, 512)) * 3).astype(np.float32)
    got = om.ple_inputs(x)
    qa, as_ = oracle.quantize(x)
    y = oracle.i8_gemm(qa, as_, ex["wple_model"], ex["sple_model"]).astype(np.float64)
    scale = float(np.float32(1 / np.sqrt(512.0)))
    g = ex["ple_proj_norm"].astype(np.float64)

    def form(y, s):
        z = (y * s).reshape(6, 2, 512)
        return (z / np.sqrt((z * z).mean(-1, keepdims=True) + 1e-6) * g).reshape(6, 1024)
    want = form(y, scale)
    assert np.abs(got - want).max() < 2e-5
    # the norm runs per 512-slice, after the scale: normalising the whole row differs by the
    # slices' rms ratio; with outputs this small (ple_scale^2 * y^2 ~ eps) dropping the scale
    # moves the result by the eps term
    whole = y * scale / np.sqrt(((y * scale) ** 2).mean(-1, keepdims=True) + 1e-6)
    assert np.abs(got - np.tile(g, 2) * whole).max() > 1e-3
    small = (x * 1e-4).astype(np.float32)
    got_s = om.ple_inputs(small)
    qs_, ss_ = oracle.quantize(small)
    ys = oracle.i8_gemm(qs_, ss_, ex["wple_model"], ex["sple_model"]).astype(np.float64)
    assert np.abs(got_s - form(ys, scale)).max() < 2e-4
    assert np.abs(got_s - form(ys, 1.0)).max() > 1e-2


@pytest.mark.parametrize("layer", [0, 5])
def test_layer_geometry_by_composition(e2mi_mod, oracle, rng, layer):
    """Layer 5 of the reference geometry is a full-attention layer (head_dim 512, 1 kv head, theta
    1e6, no window); layer 0 a sliding one (256, 2, 1e4, window 512). The attention sublayer equals
    the composition of the pinned stages at that geometry, and not at the other layer type's."""
    m, om = _model(e2mi_mod, oracle, n_layers=6, attn_scale=1 / 16)
    L = om._keep[0][layer]
    full = layer == 5
    D, KV, theta, W = (512, 1, 1e6, 0) if full else (256, 2, 1e4, 512)
    H, S, eps = 4, 600, 1e-6
    x = (rng.standard_normal((S, 512))).astype(np.float32)
    valid = np.ones((1, S), np.uint8)
    valid[0, 590:] = 0
    got = om.attention_sublayer(layer, x, valid, 1, S)

    def compose(theta, W):
        qa, as_ = oracle.quantize(x)
        qkv = oracle.i8_gemm(qa, as_, L["wqkv"], L["sqkv"])
        q = oracle.rmsnorm(np.ascontiguousarray(qkv[:, :H * D]).reshape(S * H, D), L["q_norm"], eps)
        k = oracle.rmsnorm(np.ascontiguousarray(qkv[:, H * D:(H + KV) * D]).reshape(S * KV, D), L["k_norm"], eps)
        v = oracle.rmsnorm(np.ascontiguousarray(qkv[:, (H + KV) * D:]).reshape(S * KV, D), np.ones(D, np.float32), eps)
        cs, sn = oracle.rope_table(S, D, theta)
        Sb = 590
        q = q.reshape(S, H * D)
        k = k.reshape(S, KV * D)
        # rows of one head each, position = row / heads (or_rope_rows)
        q[:Sb] = oracle.rope_rows(q[:Sb].reshape(Sb * H, D), H, cs, sn).reshape(Sb, H * D)
        k[:Sb] = oracle.rope_rows(k[:Sb].reshape(Sb * KV, D), KV, cs, sn).reshape(Sb, KV * D)
        ctx = np.zeros((S, H * D), np.float32)
        ctx[:Sb] = oracle.attention(np.ascontiguousarray(q[:Sb]), np.ascontiguousarray(k[:Sb]),
                                    np.ascontiguousarray(v.reshape(S, KV * D)[:Sb]), valid[0, :Sb].copy(),
                                    H, KV, D, scale=np.float32(1 / 16), window=W)
        cq, cs_ = oracle.quantize(ctx)
        return oracle.i8_gemm(cq, cs_, L["wo"], L["so"])
    want = compose(theta, W)
    assert_f32_close(got, want, rtol=1e-5, atol=1e-5, what=f"layer {layer} attention")
    other = compose(1e4 if full else 1e6, 512 if full else 0)
    assert np.abs(other - got).max() > 100 * max(np.abs(want - got).max(), 1e-6)


def test_no_layers_embed_proj_closed_form(e2mi_mod, oracle, rng):
    m, om = _model(e2mi_mod, oracle, n_layers=1)
    om.m.n_layers = 0
    S = 20
    ids = rng.integers(0, 1000, (2, S)).astype(np.int32)
    valid = np.ones((2, S), np.uint8)
    valid[1, 11:] = 0
    valid[1, 2] = 0
    got = om.encode(ids, valid)
    assert got.shape == (2, 768)
    table, fn, ex = om._keep[1], om._keep[2], om._keep[3]
    for b in range(2):
        x = (table[ids[b]] * np.float32(np.sqrt(512.0))).astype(np.float32)
        xn = oracle.rmsnorm(x, fn, 1e-6)
        qa, as_ = oracle.quantize(xn)
        e = oracle.i8_gemm(qa, as_, ex["wembed_proj"], ex["sembed_proj"])
        assert np.array_equal(got[b], oracle.meanpool_l2(e, valid[b].copy())), b
