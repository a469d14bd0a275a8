"""Test helpers: small model geometries and the oracle view of a product model's weights."""
import numpy as np

Q8 = ("self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
      "self_attn.o_proj.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight")
NORMS = ("input_layernorm.weight", "post_attention_layernorm.weight",
         "pre_feedforward_layernorm.weight", "post_feedforward_layernorm.weight",
         "self_attn.q_norm.weight", "self_attn.k_norm.weight")


PLE_Q8 = ("ple_block.per_layer_input_gate.weight", "ple_block.per_layer_projection.weight")
PLE_NORM = "ple_block.post_per_layer_input_norm.weight"


def small_config(e2mi, n_layers=2, vocab=1000, max_seq=512):
    return e2mi.baseline_config(n_layers=n_layers, vocab=vocab, max_seq=max_seq)


def reference_small_config(e2mi, n_layers=6, vocab=1000, max_seq=2048, **over):
    """The reference checkpoint's geometry (hidden 512, PLE, window 512, full layer 5 with
    head_dim 512) with a small vocabulary and n_layers layers."""
    return e2mi.reference_config(n_layers=n_layers, vocab=vocab, max_seq=max_seq, **over)


def lname(l, s):
    return f"language_model.layers.{l}.{s}"


def bf16_round(a):
    """Round f32 values to bf16 (nearest even), kept in f32: the precision the reference holds its
    token table in (e2.c:316-317)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def oracle_model(oracle, model, n_layers=None, attn_i8=False, embed_bf16=False, i8_min_keys=0):
    """Build the oracle's or_model from the product model's host tensors (packed weights unpacked
    with the oracle's own layout code). embed_bf16: the token table rounded to bf16, as the
    reference's own text tower holds it."""
    from oracle.binding import OracleModel
    cfg = model.config
    L = cfg.n_layers if n_layers is None else n_layers
    ple = cfg.ple_dim > 0

    def q8(name):
        wq, sc, _, N, K = model.tensor(name)
        return oracle.q8w_unpack(wq, N, K), np.ascontiguousarray(sc[:N], np.float32)

    layers = []
    for l in range(L):
        w = {}
        for s in Q8:
            w[s] = q8(lname(l, s))
        d = {
            "wqkv": np.ascontiguousarray(np.concatenate([w[Q8[i]][0] for i in range(3)])),
            "sqkv": np.ascontiguousarray(np.concatenate([w[Q8[i]][1] for i in range(3)])),
            "wo": w[Q8[3]][0], "so": w[Q8[3]][1],
            "wgate": w[Q8[4]][0], "sgate": w[Q8[4]][1],
            "wup": w[Q8[5]][0], "sup": w[Q8[5]][1],
            "wdown": w[Q8[6]][0], "sdown": w[Q8[6]][1],
        }
        for s, key in zip(NORMS, ("input_ln", "post_attn_ln", "pre_ffn_ln", "post_ffn_ln",
                                  "q_norm", "k_norm")):
            d[key] = np.ascontiguousarray(model.tensor(lname(l, s)), np.float32)
        if ple:
            d["wple_gate"], d["sple_gate"] = q8(lname(l, PLE_Q8[0]))
            d["wple_proj"], d["sple_proj"] = q8(lname(l, PLE_Q8[1]))
            d["ple_norm"] = np.ascontiguousarray(model.tensor(lname(l, PLE_NORM)), np.float32)
            d["layer_scalar"] = float(np.asarray(model.tensor(lname(l, "layer_scalar"))).reshape(-1)[0])
        layers.append(d)
    c = {"hidden": cfg.hidden, "ffn": cfg.ffn, "n_heads": cfg.n_heads, "n_kv_heads": cfg.n_kv_heads,
         "head_dim": cfg.head_dim, "vocab": cfg.vocab, "rms_eps": cfg.rms_eps,
         "rope_theta": cfg.rope_theta, "embed_scale": cfg.embed_scale,
         "ple_dim": cfg.ple_dim, "out_dim": cfg.out_dim, "window": cfg.window,
         "full_period": cfg.full_period, "full_head_dim": cfg.full_head_dim,
         "full_kv_heads": cfg.full_kv_heads, "rope_theta_full": cfg.rope_theta_full,
         "ple_scale": cfg.ple_scale}
    extra = {}
    if ple:
        extra["wple_model"], extra["sple_model"] = q8("language_model.ple.per_layer_model_projection.weight")
        extra["ple_proj_norm"] = np.ascontiguousarray(
            model.tensor("language_model.ple.per_layer_projection_norm.weight"), np.float32)
    if cfg.out_dim > 0:
        extra["wembed_proj"], extra["sembed_proj"] = q8("language_model.embedding_projection.weight")
    embed = np.ascontiguousarray(model.tensor("language_model.embed_tokens.weight"), np.float32)
    if embed_bf16:
        embed = bf16_round(embed)
    fnorm = np.ascontiguousarray(model.tensor("language_model.norm.weight"), np.float32)
    return OracleModel(oracle, c, layers, embed, fnorm, attn_scale=cfg.attn_scale, attn_i8=attn_i8,
                       extra=extra, i8_min_keys=i8_min_keys)


def random_batch(rng, B, S, vocab, min_len=1, holes=False):
    ids = rng.integers(0, vocab, (B, S)).astype(np.int32)
    valid = np.zeros((B, S), np.uint8)
    for b in range(B):
        L = int(rng.integers(min_len, S + 1))
        valid[b, :L] = 1
    if holes:
        valid[rng.random((B, S)) < 0.05] = 0
    return ids, valid
