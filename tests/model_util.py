"""Test helpers: small model geometries and the oracle view of a product model's weights."""
import numpy as np

Q8 = ("self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
      "self_attn.o_proj.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight")
NORMS = ("input_layernorm.weight", "post_attention_layernorm.weight",
         "pre_feedforward_layernorm.weight", "post_feedforward_layernorm.weight",
         "self_attn.q_norm.weight", "self_attn.k_norm.weight")


def small_config(e2mi, n_layers=2, vocab=1000, max_seq=512):
    return e2mi.baseline_config(n_layers=n_layers, vocab=vocab, max_seq=max_seq)


def lname(l, s):
    return f"language_model.layers.{l}.{s}"


def oracle_model(oracle, model, n_layers=None, attn_i8=False):
    """Build the oracle's or_model from the product model's host tensors (packed weights unpacked
    with the oracle's own layout code)."""
    from oracle.binding import OracleModel
    cfg = model.config
    L = cfg.n_layers if n_layers is None else n_layers
    layers = []
    for l in range(L):
        w = {}
        for s in Q8:
            wq, sc, _, N, K = model.tensor(lname(l, s))
            w[s] = (oracle.q8w_unpack(wq, N, K), sc)
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
        layers.append(d)
    c = {"hidden": cfg.hidden, "ffn": cfg.ffn, "n_heads": cfg.n_heads, "n_kv_heads": cfg.n_kv_heads,
         "head_dim": cfg.head_dim, "vocab": cfg.vocab, "rms_eps": cfg.rms_eps,
         "rope_theta": cfg.rope_theta, "embed_scale": cfg.embed_scale}
    embed = np.ascontiguousarray(model.tensor("language_model.embed_tokens.weight"), np.float32)
    fnorm = np.ascontiguousarray(model.tensor("language_model.norm.weight"), np.float32)
    return OracleModel(oracle, c, layers, embed, fnorm, attn_scale=cfg.attn_scale, attn_i8=attn_i8)


def random_batch(rng, B, S, vocab, min_len=1, holes=False):
    ids = rng.integers(0, vocab, (B, S)).astype(np.int32)
    valid = np.zeros((B, S), np.uint8)
    for b in range(B):
        L = int(rng.integers(min_len, S + 1))
        valid[b, :L] = 1
    if holes:
        valid[rng.random((B, S)) < 0.05] = 0
    return ids, valid
