"""The oracle's text-layer recipe (oracle/e2_oracle_model.c, restating text.c:817-984) pinned by
special cases the mathematics fixes, independently of the stage functions it composes:

- a layer whose int8 weights are all zero is the identity on the residual stream (a dropped or
  misplaced residual, or a norm applied to the stream instead of the branch, fails);
- with W_q = W_k = 0 every score is 0, so attention is the mean of the normalised V rows over the
  valid keys of the sequence: the O-branch is then a closed form of the stage functions
  (masking, per-sequence segmentation, the gamma-free V norm, the GQA head mapping and the
  post-attention norm placement are all visible);
- trailing padding and the other sequences of a batch do not change an embedding (bit-exact);
- with no layers the embedding is l2(meanpool(rms(table[id] * scale) * final_norm)).
"""
import numpy as np

from conftest import assert_f32_close
from oracle.binding import OracleModel

H, KV, D, DM, F, VOCAB = 3, 1, 256, 768, 1152, 500
CFG = {"hidden": DM, "ffn": F, "n_heads": H, "n_kv_heads": KV, "head_dim": D, "vocab": VOCAB,
       "rms_eps": 1e-6, "rope_theta": 10000.0, "embed_scale": float(np.float32(np.sqrt(768.0)))}


def _layer(rng, zero=()):
    def q8(N, K, name):
        w = np.zeros((N, K), np.int8) if name in zero else \
            rng.integers(-127, 128, (N, K), dtype=np.int8)
        return w, rng.uniform(0.001, 0.02, N).astype(np.float32)

    nq = (H + 2 * KV) * D
    L = {}
    L["wqkv"], L["sqkv"] = q8(nq, DM, "qkv")
    if "qk" in zero:
        L["wqkv"][: (H + KV) * D] = 0
    L["wo"], L["so"] = q8(DM, H * D, "o")
    L["wgate"], L["sgate"] = q8(F, DM, "ffn")
    L["wup"], L["sup"] = q8(F, DM, "ffn")
    L["wdown"], L["sdown"] = q8(DM, F, "ffn")
    for k in ("input_ln", "post_attn_ln", "pre_ffn_ln", "post_ffn_ln"):
        L[k] = (1 + 0.05 * rng.standard_normal(DM)).astype(np.float32)
    for k in ("q_norm", "k_norm"):
        L[k] = (1 + 0.05 * rng.standard_normal(D)).astype(np.float32)
    return {k: np.ascontiguousarray(v) for k, v in L.items()}


def _model(oracle, rng, layers):
    embed = (0.02 * rng.standard_normal((VOCAB, DM))).astype(np.float32)
    fnorm = (1 + 0.05 * rng.standard_normal(DM)).astype(np.float32)
    return OracleModel(oracle, CFG, layers, embed, fnorm)


def test_zero_weight_layer_is_identity(oracle, rng):
    m = _model(oracle, rng, [_layer(rng, zero=("qkv", "o", "ffn"))])
    B, S = 2, 32
    x = (3 * rng.standard_normal((B * S, DM))).astype(np.float32)
    valid = np.ones((B, S), np.uint8)
    valid[1, 20:] = 0
    assert np.array_equal(m.layer(0, x, valid, B, S), x)


def test_uniform_attention_closed_form(oracle, rng):
    """W_q = W_k = 0: ctx of every query of a sequence (every head: KV = 1) is the mean of the
    gamma-free RMS-normalised V rows over its valid keys."""
    L = _layer(rng, zero=("qk", "ffn"))
    m = _model(oracle, rng, [L])
    B, S = 3, 32
    x = (2 * rng.standard_normal((B * S, DM))).astype(np.float32)
    valid = np.ones((B, S), np.uint8)
    valid[0, 25:] = 0                      # trailing padding (trimmed)
    valid[1, [3, 7, 8]] = 0                 # holes: masked keys
    valid[2, :] = 1
    got = m.layer(0, x, valid, B, S)

    eps = CFG["rms_eps"]
    xn, res = oracle.norm_split(x, L["input_ln"], eps)
    qa, as_ = oracle.quantize(xn)
    qkv = oracle.i8_gemm(qa, as_, L["wqkv"], L["sqkv"])
    v = oracle.rmsnorm(np.ascontiguousarray(qkv[:, (H + KV) * D:]), np.ones(D, np.float32), eps)
    ctx = np.zeros((B * S, H * D), np.float32)
    for b in range(B):
        keys = np.flatnonzero(valid[b])
        mean = v[b * S + keys].astype(np.float64).mean(0).astype(np.float32)
        ctx[b * S + keys] = np.tile(mean, H)    # invalid query rows keep a zero context
    # the closed form holds up to the float summation order of the mean: compare the O-branch
    # through the same quantizer with a tolerance on ctx, then the full layer output
    cq, cs = oracle.quantize(ctx)
    o = oracle.i8_gemm(cq, cs, L["wo"], L["so"])
    want = oracle.norm_add(o, res, L["post_attn_ln"], eps)
    # W_ffn = 0: the FFN sub-layer is the identity
    assert_f32_close(got, want, rtol=2e-3, atol=1e-2, what="uniform attention layer")
    # and a misplaced mask (holes ignored) would be far off
    ctx_bad = ctx.copy()
    ctx_bad[S + np.flatnonzero(valid[1])] = np.tile(
        v[S: 2 * S].astype(np.float64).mean(0).astype(np.float32), H)
    cq, cs = oracle.quantize(ctx_bad)
    bad = oracle.norm_add(oracle.i8_gemm(cq, cs, L["wo"], L["so"]), res, L["post_attn_ln"], eps)
    assert np.abs(bad[S: 2 * S] - got[S: 2 * S]).max() > 50 * np.abs(want - got).max()


def test_padding_and_batch_independence(oracle, rng):
    m = _model(oracle, rng, [_layer(rng), _layer(rng)])
    S = 48
    ids = rng.integers(0, VOCAB, (3, S)).astype(np.int32)
    valid = np.zeros((3, S), np.uint8)
    for b, n in enumerate((48, 30, 17)):
        valid[b, :n] = 1
    valid[0, [5, 9]] = 0
    full = m.encode(ids, valid)
    for b in range(3):
        n = int(np.flatnonzero(valid[b]).max()) + 1
        one = m.encode(np.ascontiguousarray(ids[b: b + 1, :n]), np.ascontiguousarray(valid[b: b + 1, :n]))
        assert np.array_equal(one[0], full[b]), b
    # the ids under padding do not matter
    ids2 = ids.copy()
    ids2[valid == 0] = (ids2[valid == 0] + 1) % VOCAB
    assert np.array_equal(m.encode(ids2, valid), full)


def test_no_layers_closed_form(oracle, rng):
    m = _model(oracle, rng, [_layer(rng)])
    m.m.n_layers = 0
    S = 20
    ids = rng.integers(0, VOCAB, (2, S)).astype(np.int32)
    valid = np.ones((2, S), np.uint8)
    valid[1, 11:] = 0
    valid[1, 2] = 0
    got = m.encode(ids, valid)
    table, fn = m._keep[1], m._keep[2]
    for b in range(2):
        x = table[ids[b]].astype(np.float64) * CFG["embed_scale"]
        x = x / np.sqrt((x * x).mean(1, keepdims=True) + CFG["rms_eps"]) * fn
        p = x[valid[b] == 1].mean(0)
        want = p / np.linalg.norm(p)
        assert np.abs(got[b] - want).max() < 2e-6
    # an all-invalid sequence embeds as an exact zero vector (text.c:968-980)
    z = m.encode(ids[:1], np.zeros((1, S), np.uint8))
    assert not z.any()
