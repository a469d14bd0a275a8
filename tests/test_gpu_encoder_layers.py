"""BASELINE config 4 as stated (24 layers at the reference's attention scale 1.0, vocabulary 262144,
64 x 512 with lengths U[64, 512]), pinned layer by layer against the oracle.

A whole 24-layer random-init stack at scale 1.0 is chaotic (a 1-ulp change of the embedding table
moves the oracle's own embedding to cosine 0.965 after 8 layers), so the end-to-end embeddings are
checked by properties (test_gpu_encoder.py). Here every checked layer starts from the DEVICE's own
input to it: the engine runs l layers (e2mi_set_layer_limit) and dumps its residual rows
(E2MI_DUMP, the reference HIP backend's E2_HIP_DUMP), the oracle runs layer l alone on those rows
(text.c:924-961 recipe), and the device's own output of layer l (l + 1 layers, dumped again) must
match: no amplification across layers, so the bar is one layer's.

Bars: per sequence, the layer's output through the final RMSNorm, mean pool and L2 (the embedding
the engine would return after that layer) at cosine >= 0.9999 of the oracle's; per row of the
residual stream, cosine >= 0.9999 at the median and >= 0.999 for every row: the f16 q and k of the
attention move a logit at scale 1.0 (std ~16) by ~0.01, which leaves a few rows near 0.9998
(test_gpu_diagnostics.py)."""
import numpy as np
import pytest

from model_util import oracle_model, small_config

pytestmark = pytest.mark.gpu

B, S = 64, 512
LAYERS = (0, 5, 11, 23)


def _rowcos(a, b):
    a, b = a.astype(np.float64), b.astype(np.float64)
    return (a * b).sum(1) / (np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1) + 1e-300)


def _embed(x, gamma, eps, valid):
    """final RMSNorm, masked mean over the valid rows, L2 (text.c:963-981), in float64"""
    x = x.astype(np.float64)
    xn = x / np.sqrt((x * x).mean(1, keepdims=True) + eps) * gamma.astype(np.float64)
    v = valid.reshape(B, S).astype(bool)
    out = np.stack([xn.reshape(B, S, -1)[b][v[b]].mean(0) for b in range(B)])
    return out / np.linalg.norm(out, axis=1, keepdims=True)


def test_config4_layer_by_layer(gpu, oracle, tmp_path, monkeypatch):
    import e2mi
    rng = np.random.default_rng(2024)
    cfg = small_config(e2mi, n_layers=24, vocab=262144)
    assert cfg.attn_scale == 1.0
    m = e2mi.Model.synthetic(cfg, 4044)
    ids = rng.integers(0, cfg.vocab, (B, S)).astype(np.int32)
    lens = rng.integers(64, S + 1, B)
    valid = (np.arange(S)[None, :] < lens[:, None]).astype(np.uint8)
    vflat = valid.reshape(-1)
    monkeypatch.setenv("E2MI_DUMP", str(tmp_path))
    monkeypatch.setenv("E2MI_DUMP_CALL", "all")
    eng = e2mi.Engine(m, max_rows=B * S)
    monkeypatch.delenv("E2MI_DUMP")
    monkeypatch.delenv("E2MI_DUMP_CALL")
    om = oracle_model(oracle, m)
    gamma = m.tensor("language_model.norm.weight")

    def run(n_layers):
        eng.set_layer_limit(n_layers)
        out = eng.embed_batch(ids, valid)
        rowmap = np.fromfile(tmp_path / "e2mi_rowmap.i32", np.int32)
        x = np.fromfile(tmp_path / "e2mi_x.f32", np.float32).reshape(len(rowmap), cfg.hidden)
        assert np.array_equal(np.fromfile(tmp_path / "e2mi_out.f32", np.float32).reshape(B, -1), out)
        return rowmap, x, out

    table = m.tensor("language_model.embed_tokens.weight")
    x0 = table[ids.reshape(-1)] * np.float32(cfg.embed_scale)
    del table
    for l in LAYERS:
        if l == 0:
            x_in = x0
        else:
            rowmap, x, _ = run(l)
            live = rowmap >= 0
            x_in = np.zeros((B * S, cfg.hidden), np.float32)
            x_in[rowmap[live]] = x[live]
        rowmap, x_out, emb = run(l + 1)
        live = rowmap >= 0
        assert live.sum() == vflat.sum()
        want = om.layer(l, x_in, vflat, B, S, nthreads=16)
        rc = _rowcos(x_out[live], want[rowmap[live]])
        want_emb = _embed(want, gamma, cfg.rms_eps, vflat)
        ec = _rowcos(emb, want_emb)
        print(f"layer {l}: rows 1-cos median {1 - np.median(rc):.2e} max {1 - rc.min():.2e} "
              f"(below 0.9999: {(rc < 0.9999).sum()} of {rc.size}); embeddings 1-cos max {1 - ec.min():.2e}",
              flush=True)
        assert ec.min() >= 0.9999, (l, ec.min())
        assert np.median(rc) >= 0.9999 and rc.min() >= 0.999, (l, np.median(rc), rc.min())
    eng.set_layer_limit(0)
