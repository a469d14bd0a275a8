"""The oracle's whole recipe at the reference checkpoint's geometry against the reference's own text
tower: e2_text_embed_batch (text.c:997-1027) from the reference sources, compiled by
oracle/Makefile into oracle/_ref/libreftext.so and run on the same weights (an E8CQ cache written by
the product's e2_save_e8cq, read back by the reference's q8c reader; oracle/ref_text.c).

This pins what the stage-by-stage tests cannot: the order and placement of every norm and residual
(a gamma folded as 1 + w, a norm before instead of after a sublayer), the PLE block, the per-layer
geometry (window, head_dim 512 and RoPE theta 1e6 on layer 5) and the attention rule the reference
applies (int8 attention for sequences with no padding inside and at least the rule table's key count,
dispatch.c:47-52, text.c:873-876; f32 attention otherwise).

The reference holds its token table in bf16 (e2.c:316-317), so the oracle's table is rounded the
same way here. Bars are on 1 - cosine of the L2-normalised embeddings: one layer agrees to about
1e-5 (f32 softmax / norm arithmetic in a different order, then requantised), two layers to a few
1e-4 (attention at scale 1.0 on random weights amplifies the differences layer by layer). The
planted mistakes below land 10x or more beyond the bars.
"""
import os

import numpy as np
import pytest

from model_util import oracle_model, random_batch, reference_small_config

BAR_ONE = 4e-5
BAR_TWO = 1e-3
VOCAB = 1000


@pytest.fixture(scope="module")
def setup(oracle, tmp_path_factory):
    from oracle.binding import RefText
    if not RefText.available():
        pytest.skip("oracle/_ref/libreftext.so not built (the reference tree is absent on this host)")
    import e2mi
    m = e2mi.Model.synthetic(reference_small_config(e2mi, n_layers=6, vocab=VOCAB), 1234)
    path = str(tmp_path_factory.mktemp("reftext") / "model.e8cq")
    m.save_e8cq(path)
    return m, path


def _open(path, n_layers, identity=()):
    from oracle.binding import RefText
    rt = RefText(path, n_layers, VOCAB, nthreads=4)
    for l in identity:
        rt.identity_layer(l)
    return rt


def _oracle(oracle, m, n_layers, i8_min_keys, attn_i8=True, identity=()):
    om = oracle_model(oracle, m, n_layers=n_layers, attn_i8=attn_i8, embed_bf16=True,
                      i8_min_keys=i8_min_keys)
    for l in identity:  # the same edit as rt_identity_layer: O, down, PLE projection scaled to 0
        for n in ("so", "sdown", "sple_proj"):
            om._keep[0][l][n][...] = 0
        om._arr[l].layer_scalar = 1.0
    return om


def _dist(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    c = (a * b).sum(1) / (np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1))
    return float(1 - c.min())


def _threshold(rt):
    return next(s for s in range(32, 2049) if rt.attn_i8(s))


def _takes_i8(valid, thr):
    """text.c:849-852 trims trailing padding; the blocked path needs every remaining row valid."""
    for v in valid:
        n = int(np.flatnonzero(v)[-1]) + 1 if v.any() else 0
        if n >= max(32, thr) and v[:n].all():
            return True
    return False


def _batch(kind, rng):
    if kind == "padded64":
        return random_batch(rng, 3, 64, VOCAB, min_len=20)
    S = {"full200": 200, "window700": 700, "window700_tail": 700, "full300": 300}[kind]
    B = 1 if S == 700 else 2
    ids = rng.integers(0, VOCAB, (B, S)).astype(np.int32)
    valid = np.ones((B, S), np.uint8)
    if kind == "window700_tail":
        valid[0, 650:] = 0
    return ids, valid


@pytest.mark.parametrize("kind", ["padded64", "full200", "window700", "window700_tail"])
def test_one_sliding_layer(setup, oracle, rng, kind):
    """Layer 0 (sliding, head_dim 256, window 512): f32 attention with padding, int8 attention with
    none, the window cutting in at 700 tokens."""
    m, path = setup
    ids, valid = _batch(kind, rng)
    rt = _open(path, 1)
    thr = _threshold(rt)
    got = rt.embed_batch(ids, valid)
    rt.close()
    d = _dist(got, _oracle(oracle, m, 1, thr).encode(ids, valid))
    assert d < BAR_ONE, (kind, d)
    if _takes_i8(valid, thr):
        # the attention rule matters: the f32 attention lands far from the reference here
        d32 = _dist(got, _oracle(oracle, m, 1, thr, attn_i8=False).encode(ids, valid))
        assert d32 > 10 * BAR_ONE, (kind, d32)


@pytest.mark.parametrize("tail", [False, True])
def test_full_attention_layer(setup, oracle, rng, tail):
    """Layer 5 alone (layers 0-4 made identities on both sides): head_dim 512, one kv head, RoPE
    theta 1e6, no window."""
    m, path = setup
    ids, valid = _batch("full300", rng)
    if tail:
        valid[1, 250:] = 0
    ident = range(5)
    rt = _open(path, 6, ident)
    thr = _threshold(rt)
    got = rt.embed_batch(ids, valid)
    rt.close()
    d = _dist(got, _oracle(oracle, m, 6, thr, identity=ident).encode(ids, valid))
    assert d < BAR_ONE, d
    # a sliding layer's geometry on layer 5 (theta 1e4) is far off
    om = _oracle(oracle, m, 6, thr, identity=ident)
    om.m.rope_theta_full = 1e4
    assert _dist(got, om.encode(ids, valid)) > 10 * BAR_ONE


@pytest.mark.parametrize("kind", ["padded64", "full200"])
def test_two_layers(setup, oracle, rng, kind):
    m, path = setup
    ids, valid = _batch(kind, rng)
    rt = _open(path, 2)
    thr = _threshold(rt)
    got = rt.embed_batch(ids, valid)
    rt.close()
    d = _dist(got, _oracle(oracle, m, 2, thr).encode(ids, valid))
    assert d < BAR_TWO, (kind, d)


def test_planted_mistakes_fail(setup, oracle, rng):
    """Mistakes planted in the oracle (on the CPU) land beyond the one-layer bar: each norm's gamma
    read as 1 + w, the embedding scale dropped, the sliding layers' RoPE theta taken from the full
    layers, the token table kept in f32."""
    m, path = setup
    ids, valid = _batch("padded64", rng)
    rt = _open(path, 1)
    thr = _threshold(rt)
    got = rt.embed_batch(ids, valid)
    rt.close()

    def gamma(n):
        def f(om):
            om._keep[0][0][n][...] += 1
        return f

    def no_embed_scale(om):
        om.m.embed_scale = 1.0

    def theta(om):
        om.m.rope_theta = om.m.rope_theta_full

    def f32_table(om):
        om._keep[1][...] = m.tensor("language_model.embed_tokens.weight")

    plants = {n: gamma(n) for n in ("input_ln", "post_attn_ln", "pre_ffn_ln", "post_ffn_ln", "q_norm",
                                     "k_norm", "ple_norm")}
    plants.update(no_embed_scale=no_embed_scale, theta=theta, f32_table=f32_table)
    for name, plant in plants.items():
        om = _oracle(oracle, m, 1, thr)
        plant(om)
        assert _dist(got, om.encode(ids, valid)) > 5 * BAR_ONE, name
