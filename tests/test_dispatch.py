"""The backend-selection surface asserted as data (mirrors the reference's tests/test_dispatch.c
matrix, plus the gfx950 row). Runs on any host: nothing here calls a kernel."""
import ctypes as C
import os

import pytest

BK = dict(CPU_SCALAR=0, CPU_AVX2=1, CPU_VNNI=2, CPU_AVX512=3, CPU_NEON=4, INTEL_GPU=5, HIP=6,
          HIP_GFX950=7, COUNT=8)
TEXT, IMAGE, AUDIO = 0, 1, 2
F32, F16, I8 = 0, 1, 2
CAP_GEMM_I8, CAP_QUANT_I8, CAP_SOFTMAX_Q_I8, CAP_ATTN_I8_FUSED, CAP_ATTN_F16 = 1, 2, 4, 8, 16
ANY = 1 << 30
ENV = ("E2_ATTN_TEXT", "E2_ATTN_IMAGE", "E2_ATTN_I8", "E2_VATTN_OFF", "E2_ATTN_AUDIO",
       "E2_ATTN_STAGE", "E2_HIP_ATTN", "E2_HIP_ATTN_I8")


@pytest.fixture
def d(monkeypatch):
    import e2mi
    lib = C.CDLL(e2mi.LIB_PATH)
    for n in ("e2_attn_pick", "e2_attn_min_keys", "e2_backend_caps", "e2_cpu_backend",
              "e2_attn_stage_override"):
        getattr(lib, n).restype = C.c_int if n != "e2_backend_caps" else C.c_uint
    lib.e2_attn_kind_name.restype = C.c_char_p
    for v in ENV:
        monkeypatch.delenv(v, raising=False)
    lib.e2_attn_env_reload()
    yield lib
    for v in ENV:
        os.environ.pop(v, None)
    lib.e2_attn_env_reload()


def pick(d, bk, tower, keys):
    return d.e2_attn_pick(BK[bk], tower, keys)


SIMD = ("CPU_AVX2", "CPU_VNNI", "CPU_AVX512", "CPU_NEON")


def test_text_rules(d):
    assert pick(d, "CPU_SCALAR", TEXT, 0) == F32 and pick(d, "CPU_SCALAR", TEXT, 2048) == F32
    for bk in SIMD:
        for keys, want in ((0, F32), (63, F32), (127, F32), (128, I8), (512, I8), (ANY, I8)):
            assert pick(d, bk, TEXT, keys) == want, (bk, keys)
    for keys, want in ((0, F16), (511, F16), (512, I8), (2048, I8)):
        assert pick(d, "INTEL_GPU", TEXT, keys) == want
    for keys, want in ((0, F32), (63, F32), (64, I8), (2048, I8)):
        assert pick(d, "HIP", TEXT, keys) == want
    # the gfx950 row: f16 MFMA attention at every length
    for keys in (0, 1, 64, 512, 2048, ANY):
        assert pick(d, "HIP_GFX950", TEXT, keys) == F16


def test_image_and_audio_rules(d):
    for bk in SIMD:
        want = F32 if bk == "CPU_AVX2" else I8
        assert pick(d, bk, IMAGE, 0) == want and pick(d, bk, IMAGE, 2520) == want
    assert pick(d, "CPU_SCALAR", IMAGE, 2520) == F32
    assert pick(d, "INTEL_GPU", IMAGE, 2520) == I8 and pick(d, "HIP", IMAGE, 2520) == I8
    assert pick(d, "HIP_GFX950", IMAGE, 2520) == F16   # no vision tower: the f16 row
    for bk in range(BK["COUNT"]):
        for keys in (0, 750, 2048):
            assert d.e2_attn_pick(bk, AUDIO, keys) == F32


def test_thresholds_and_caps(d):
    mk = lambda bk, t: d.e2_attn_min_keys(BK[bk], t)
    assert mk("CPU_VNNI", TEXT) == 128 and mk("CPU_AVX2", TEXT) == 128 and mk("CPU_NEON", TEXT) == 128
    assert mk("INTEL_GPU", TEXT) == 512 and mk("HIP", TEXT) == 64 and mk("CPU_SCALAR", TEXT) == 0
    assert mk("HIP_GFX950", TEXT) == 0
    for bk in range(BK["COUNT"]):
        assert d.e2_attn_min_keys(bk, IMAGE) == 0 and d.e2_attn_min_keys(bk, AUDIO) == 0
    caps = lambda bk: d.e2_backend_caps(BK[bk])
    assert caps("CPU_SCALAR") & 3 == 3 and not caps("CPU_SCALAR") & (CAP_ATTN_I8_FUSED | CAP_SOFTMAX_Q_I8)
    for bk in SIMD:
        c = caps(bk)
        assert c & (CAP_GEMM_I8 | CAP_QUANT_I8 | CAP_SOFTMAX_Q_I8)
        assert bool(c & CAP_ATTN_I8_FUSED) == (bk != "CPU_AVX2") and not c & CAP_ATTN_F16
    assert caps("INTEL_GPU") & CAP_ATTN_I8_FUSED and caps("INTEL_GPU") & CAP_ATTN_F16
    assert caps("HIP") & CAP_ATTN_I8_FUSED and not caps("HIP") & CAP_ATTN_F16
    g = caps("HIP_GFX950")
    assert g & CAP_GEMM_I8 and g & CAP_QUANT_I8 and g & CAP_ATTN_F16 and g & CAP_ATTN_I8_FUSED
    assert d.e2_backend_caps(99) == 0 and ANY >= 2048


def test_cpu_backend_roundtrip(d):
    saved = d.e2_cpu_backend()
    d.e2_dispatch_set_cpu_backend(BK["CPU_NEON"])
    assert d.e2_cpu_backend() == BK["CPU_NEON"]
    d.e2_dispatch_set_cpu_backend(99)
    assert d.e2_cpu_backend() == BK["CPU_SCALAR"]
    d.e2_dispatch_set_cpu_backend(saved)


def test_overrides(d, monkeypatch):
    def env(**kv):
        for k, v in kv.items():
            if v is None:
                monkeypatch.delenv(k, raising=False)
            else:
                monkeypatch.setenv(k, v)
        d.e2_attn_env_reload()

    assert pick(d, "CPU_VNNI", TEXT, 2048) == I8
    env(E2_ATTN_TEXT="i8")
    assert pick(d, "CPU_VNNI", TEXT, 0) == I8 and pick(d, "CPU_SCALAR", TEXT, 0) == I8
    assert pick(d, "HIP_GFX950", TEXT, 0) == I8        # forced i8: the int8 attention kernel
    env(E2_ATTN_TEXT="f32")
    assert pick(d, "CPU_VNNI", TEXT, 2048) == F32 and pick(d, "HIP_GFX950", TEXT, 512) == F32
    env(E2_ATTN_TEXT="auto")
    assert pick(d, "CPU_VNNI", TEXT, 2048) == I8 and pick(d, "CPU_VNNI", TEXT, 0) == F32
    env(E2_ATTN_I8="0", E2_ATTN_TEXT="i8")
    assert pick(d, "CPU_VNNI", TEXT, 0) == I8           # the new name wins
    env(E2_ATTN_TEXT=None)
    assert pick(d, "CPU_VNNI", TEXT, 2048) == F32       # E2_ATTN_I8=0
    env(E2_ATTN_I8="1")
    assert pick(d, "CPU_VNNI", TEXT, 0) == I8
    env(E2_VATTN_OFF="1")
    assert pick(d, "CPU_VNNI", IMAGE, 2520) == F32
    env(E2_ATTN_AUDIO="i8")
    assert pick(d, "CPU_VNNI", AUDIO, 2048) == F32
    env(E2_ATTN_IMAGE="i8")
    assert pick(d, "CPU_VNNI", IMAGE, 2520) == I8
    d.e2_attn_override(IMAGE, F32)
    assert pick(d, "CPU_VNNI", IMAGE, 2520) == F32
    d.e2_attn_override(IMAGE, -1)
    assert pick(d, "CPU_VNNI", IMAGE, 2520) == I8
    env(E2_ATTN_TEXT="i8x", E2_ATTN_I8=None)            # a typo is ignored
    assert pick(d, "CPU_VNNI", TEXT, 2048) == I8 and pick(d, "CPU_VNNI", TEXT, 0) == F32
    assert d.e2_attn_kind_name(F16) == b"f16"


def test_stage_switch(d, monkeypatch):
    assert d.e2_attn_stage_override() == 0
    for v, want in (("direct", 1), ("lds", 2), ("legacy", 3), ("old", 3), ("bogus", 0)):
        monkeypatch.setenv("E2_ATTN_STAGE", v)
        d.e2_attn_env_reload()
        assert d.e2_attn_stage_override() == want
    monkeypatch.delenv("E2_ATTN_STAGE")
    monkeypatch.setenv("E2_HIP_ATTN", "lds")
    d.e2_attn_env_reload()
    assert pick(d, "HIP", TEXT, 2048) == F32            # old "lds" meant "not int8"
