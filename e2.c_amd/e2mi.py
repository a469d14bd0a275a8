"""Python mirror of include/e2mi.h over ctypes.

The product is the C-ABI library lib/libe2mi.so (hand-written HIP for gfx950). This module only
binds it for tests and bench.py: device buffers are torch tensors (plumbing for HBM allocation and
streams), passed to the library as raw pointers. There is no fallback: if the library is missing,
`load()` raises.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libe2mi.so")

_P, _I, _F = C.c_void_p, C.c_int, C.c_float


class Q8W(C.Structure):
    """e2mi_q8w (include/e2mi.h)."""
    _fields_ = [("w", _P), ("scale", _P), ("bias", _P), ("N", _I), ("K", _I), ("ld", _I),
                ("out_min", _F), ("out_max", _F)]


class E2Config(C.Structure):
    """e2_config (include/e2.h)."""
    _fields_ = [("n_layers", _I), ("hidden", _I), ("ffn", _I), ("n_heads", _I),
                ("n_kv_heads", _I), ("head_dim", _I), ("vocab", _I), ("max_seq", _I),
                ("rms_eps", _F), ("rope_theta", _F), ("embed_scale", _F), ("attn_scale", _F),
                ("ple_dim", _I), ("out_dim", _I), ("window", _I), ("full_period", _I),
                ("full_head_dim", _I), ("full_kv_heads", _I), ("rope_theta_full", _F), ("ple_scale", _F)]

    def layer_geom(self, l):
        """(head_dim, kv heads, RoPE theta, window) of layer l (text.c:467-478)."""
        full = self.full_period > 0 and l % self.full_period == self.full_period - 1
        if full:
            return self.full_head_dim, self.full_kv_heads, self.rope_theta_full, 0
        return self.head_dim, self.n_kv_heads, self.rope_theta, self.window


class TensorView(C.Structure):
    """e2_tensor_view (include/e2.h)."""
    _fields_ = [("kind", _I), ("ndim", _I), ("dims", C.c_int64 * 4), ("data", _P), ("scale", _P),
                ("bsq", _P), ("nbytes", C.c_size_t)]


class E2MITensor(C.Structure):
    """e2mi_tensor (include/e2mi.h): one caller-held tensor under the reference's name."""
    _fields_ = [("name", C.c_char_p), ("kind", _I), ("N", _I), ("K", _I), ("nblocks", _I), ("Npad", _I),
                ("data", _P), ("scale", _P), ("bsq", _P)]


# name -> (restype, argtypes); every symbol include/*.h declares appears here
SIGNATURES = {
    "e2mi_last_error": (C.c_char_p, []),
    "e2mi_device_info": (_I, [_I, C.c_char_p, _I, C.POINTER(_I), C.POINTER(_I)]),
    "e2mi_q8w_upload_packed": (_I, [C.POINTER(Q8W), _P, _P, _P, _I, _I, _P]),
    "e2mi_q8w_upload_rowmajor": (_I, [C.POINTER(Q8W), _P, _P, _P, _I, _I, _P]),
    "e2mi_q8w_free": (None, [C.POINTER(Q8W)]),
    "e2mi_quantize": (_I, [_P, _P, _P, _P, _I, _I, _I, _I]),
    "e2mi_i8_gemm": (_I, [_P, _P, _I, _P, _P, C.POINTER(Q8W), _I, _I, _I]),
    "e2mi_i8_gemm_acc": (_I, [_P, _P, _I, _P, _P, _P, C.POINTER(Q8W), _I, _I, _I]),
    "e2mi_i8_gemm_q": (_I, [_P, _P, _P, _P, _P, C.POINTER(Q8W), _I]),
    "e2mi_i8_gemm_tok": (_I, [_P, _P, _I, _P, _P, C.POINTER(Q8W), _I, _I, _I]),
    "e2mi_i8_gemm_tok_q": (_I, [_P, _P, _P, _P, _P, C.POINTER(Q8W), _I]),
    "e2mi_i8_gemm_geglu": (_I, [_P, _P, _P, _P, _P, _P, C.POINTER(Q8W), _I]),
    "e2mi_i8_gemm_qkv": (_I, [_P, _P, _P, C.POINTER(Q8W), _I, _I, _P, _I, _I, _P, _P, _F, _P, _P, _P, _P, _P, _P,
                              _P, _P]),
    "e2mi_gemm_set_fold": (_I, [_I]),
    "e2mi_interleave_gate_up": (_I, [_P, _P, _P, _P, _P, _P, _I, _I]),
    "e2mi_norm_quant": (_I, [_P, _P, _P, _F, _I, _I, _P, _P, _P]),
    "e2mi_add_norm_quant": (_I, [_P, _P, _P, _P, _P, _F, _I, _I, _P, _P, _P, _P]),
    "e2mi_i8_gemm_add_norm_quant": (_I, [_P, _P, _P, C.POINTER(Q8W), _I, _P, _P, _P, _F, _P, _P, _P, _P,
                                         _P]),
    "e2mi_i8_gemm_add_norm_scale_quant": (_I, [_P, _P, _P, C.POINTER(Q8W), _I, _P, _P, _F, _P, _F, _P, _P, _P,
                                               _P, _P]),
    "e2mi_embed_norm_quant": (_I, [_P, _P, _I, _P, _F, _P, _F, _I, _I, _P, _P, _P]),
    "e2mi_qkv_norm_rope": (_I, [_P, _P, _I, _I, _I, _I, _I, _P, _P, _F, _P, _P, _P, _P, _P, _P, _P, _P]),
    "e2mi_gelu_mul_quant": (_I, [_P, _P, _I, _P, _I, _I, _I, _P, _P, _I]),
    "e2mi_pool_l2": (_I, [_P, _P, _P, _I, _I, _I, _P, _P]),
    "e2mi_pool_l2_noalloc": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "e2mi_pool_workspace_bytes": (C.c_size_t, [_I, _I, _I]),
    "e2mi_attention": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _P, _P, _P]),
    "e2mi_qkv_norm_rope_packed": (_I, [_P, _P, _I, _P, _I, _I, _I, _P, _P, _F, _P, _P, _P, _P, _P, _P, _P, _P]),
    "e2mi_attention_packed": (_I, [_P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _F, _P, _P, _P, _P, _I]),
    "e2mi_attention_packed_window": (_I, [_P, _P, _P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I, _P, _P, _P,
                                          _P, _I]),
    "e2mi_attention_part_bytes": (C.c_size_t, [_I, _I, _I]),
    "e2mi_attention_packed_split": (_I, [_P, _P, _P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I, _P, _P, _P,
                                         _P, _I, _P, _I, _P, _I]),
    "e2mi_add_norm_scale_quant": (_I, [_P, _P, _P, _P, _F, _P, _F, _I, _I, _P, _P, _P, _P]),
    "e2mi_scale_norm": (_I, [_P, _P, _I, _I, _F, _P, _F, _P]),
    "e2mi_i8_gemm_gelu_mul": (_I, [_P, _P, _P, _P, _P, _P, C.POINTER(Q8W), _I, _P, _I]),
    "e2mi_attention_i8_workspace_bytes": (C.c_size_t, [_I, _I, _I, _I, _I]),
    "e2mi_attention_i8_packed": (_I, [_P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _I]),
    "e2mi_pool_l2_packed": (_I, [_P, _P, _P, _P, _I, _I, _I, _P, _P]),
    "e2mi_gather_ids": (_I, [_P, _P, _P, _I, _P]),
    # backend-selection surface (include/e2_dispatch.h)
    "e2_dispatch_set_cpu_backend": (None, [_I]),
    "e2_cpu_backend": (_I, []),
    "e2_backend_caps": (C.c_uint, [_I]),
    "e2_attn_env_reload": (None, []),
    "e2_attn_override": (None, [_I, _I]),
    "e2_attn_stage_override": (_I, []),
    "e2_attn_kind_name": (C.c_char_p, [_I]),
    "e2_attn_min_keys": (_I, [_I, _I]),
    "e2_attn_pick": (_I, [_I, _I, _I]),
    # model container (include/e2.h)
    "e2_config_baseline": (None, [C.POINTER(E2Config)]),
    "e2_config_reference": (None, [C.POINTER(E2Config)]),
    "e2_model_synthetic": (_P, [C.POINTER(E2Config), C.c_uint64]),
    "e2_load_e8cq": (_P, [C.c_char_p, C.POINTER(E2Config)]),
    "e2_save_e8cq": (_I, [_P, C.c_char_p]),
    "e2_free": (None, [_P]),
    "e2_text_embed": (_I, [_P, _P, _I, _P]),
    "e2_text_embed_batch": (_I, [_P, _P, _P, _I, _I, _P]),
    "e2_last_error": (C.c_char_p, []),
    "e2_model_config": (_I, [_P, C.POINTER(E2Config)]),
    "e2_model_tensor": (_I, [_P, C.c_char_p, C.POINTER(TensorView)]),
    # the encoder engine (include/e2mi.h)
    "e2mi_create": (_P, [_P]),
    "e2mi_create_rows": (_P, [_P, _I]),
    "e2mi_create_e8cq": (_P, [C.c_char_p, _I, _I, _I, _I]),
    "e2mi_create_tensors": (_P, [C.POINTER(E2MITensor), _I, _I, _I, _I, _I]),
    "e2mi_plan_pack": (_I, [_P, _I, _I, _P, _P, _P, _P]),
    "e2mi_plan_attention": (_I, [_P, _I, _I, _I, _I, _I, _P, _P, C.POINTER(_I)]),
    "e2mi_plan_device": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P]),
    "e2mi_destroy": (None, [_P]),
    "e2mi_device": (C.c_char_p, [_P]),
    "e2mi_text_embed": (_I, [_P, _P, _I, _P]),
    "e2mi_text_embed_batch": (_I, [_P, _P, _P, _I, _I, _P]),
    "e2mi_text_embed_batch_device": (_I, [_P, _P, _P, _I, _I, _P, _P]),
    "e2mi_stats": (_I, [_P, C.POINTER(C.c_long), C.POINTER(C.c_long), C.POINTER(C.c_double)]),
    "e2mi_profile_text": (C.c_char_p, [_P]),
    "e2mi_set_attention_split": (_I, [_P, _I]),
    "e2mi_set_layer_limit": (_I, [_P, _I]),
    "e2mi_set_device_plan": (_I, [_P, _I]),
    "e2mi_set_packing": (_I, [_P, _I]),
    "e2mi_set_attention": (_I, [_P, _I]),
}

_lib = None


class E2MIError(RuntimeError):
    pass


def load(path: str = LIB_PATH):
    """Load lib/libe2mi.so and declare every entry point. Raises if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise E2MIError(f"{path} is missing: the HIP backend was not built (run __graft_entry__.build())")
    # torch (ROCm wheels) ships its own HIP runtime under the same soname as the system one this
    # library links; loaded first, the library would pull in the system runtime and torch would
    # then run against a second one. Import torch first so the process holds one runtime (torch's,
    # to which the library's dependency then resolves).
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = C.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    return load().e2mi_last_error().decode(errors="replace")


def check(rc: int, what: str = "e2mi"):
    if rc != 0:
        raise E2MIError(f"{what}: {last_error()}")


def ptr(t):
    """Raw device (or host numpy) pointer of a tensor/array, None for None."""
    if t is None:
        return None
    if hasattr(t, "data_ptr"):
        return C.c_void_p(t.data_ptr())
    return t.ctypes.data_as(C.c_void_p)


def stream_ptr(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


class DeviceWeight:
    """An uploaded e2mi_q8w; freed with the object."""

    def __init__(self, q8w: Q8W):
        self.q = q8w

    @classmethod
    def from_rowmajor(cls, w, scale, bias=None, stream=None):
        import numpy as np
        w = np.ascontiguousarray(w, np.int8)
        scale = np.ascontiguousarray(scale, np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        q = Q8W()
        check(load().e2mi_q8w_upload_rowmajor(C.byref(q), ptr(w), ptr(scale), ptr(b), w.shape[0],
                                              w.shape[1], stream_ptr(stream)), "q8w_upload_rowmajor")
        return cls(q)

    @classmethod
    def from_packed(cls, wq, scale, N, K, bias=None, stream=None):
        import numpy as np
        wq = np.ascontiguousarray(wq, np.int8)
        scale = np.ascontiguousarray(scale, np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        q = Q8W()
        check(load().e2mi_q8w_upload_packed(C.byref(q), ptr(wq), ptr(scale), ptr(b), N, K,
                                            stream_ptr(stream)), "q8w_upload_packed")
        return cls(q)

    def set_clamp(self, lo, hi):
        self.q.out_min, self.q.out_max = lo, hi

    def __del__(self):
        if _lib is not None and self.q.w:
            _lib.e2mi_q8w_free(C.byref(self.q))

    @property
    def ref(self):
        return C.byref(self.q)


def interleave_gate_up(gate, sgate, up, sup):
    import numpy as np
    F, K = gate.shape
    w = np.empty((2 * F, K), np.int8)
    s = np.empty(2 * F, np.float32)
    args = [np.ascontiguousarray(a) for a in (gate, sgate, up, sup)]
    check(load().e2mi_interleave_gate_up(ptr(w), ptr(s), ptr(args[0]), ptr(args[1]), ptr(args[2]),
                                         ptr(args[3]), F, K), "interleave_gate_up")
    return w, s


def set_gemm_fold(mode: str) -> str:
    """Select the GEMM fold order ("exact": the reference's, bit-exact; "fast": as-only fold and
    one ws multiply per output). Returns the previous mode."""
    prev = load().e2mi_gemm_set_fold({"exact": 0, "fast": 1}[mode])
    if prev < 0:
        raise RuntimeError(last_error())
    return "fast" if prev == 1 else "exact"


# ---- kernel wrappers over torch device tensors
def quantize(x, block=128, q=None, scales=None, stream=None):
    import torch
    M, K = x.shape
    q = torch.empty((M, K), dtype=torch.int8, device=x.device) if q is None else q
    nb = K // block
    scales = torch.empty((M, nb), dtype=torch.float32, device=x.device) if scales is None else scales
    check(load().e2mi_quantize(stream_ptr(stream), ptr(q), ptr(scales), ptr(x), M, K, x.stride(0),
                               block), "quantize")
    return q, scales


def i8_gemm(qa, as_, w: DeviceWeight, n0=0, n1=None, y=None, stream=None):
    import torch
    M = qa.shape[0]
    n1 = w.q.N if n1 is None else n1
    y = torch.zeros((M, w.q.N), dtype=torch.float32, device=qa.device) if y is None else y
    check(load().e2mi_i8_gemm(stream_ptr(stream), ptr(y), y.stride(0), ptr(qa), ptr(as_), w.ref, M,
                              n0, n1), "i8_gemm")
    return y


def i8_gemm_acc(qa, as_, w: DeviceWeight, n0=0, n1=None, stream=None):
    import torch
    M = qa.shape[0]
    n1 = w.q.N if n1 is None else n1
    y = torch.zeros((M, w.q.N), dtype=torch.float32, device=qa.device)
    acc = torch.zeros((w.q.K // 128, M, n1 - n0), dtype=torch.int32, device=qa.device)
    check(load().e2mi_i8_gemm_acc(stream_ptr(stream), ptr(y), y.stride(0), ptr(acc), ptr(qa),
                                  ptr(as_), w.ref, M, n0, n1), "i8_gemm_acc")
    return y, acc


def i8_gemm_q(qa, as_, w: DeviceWeight, stream=None):
    import torch
    M = qa.shape[0]
    yq = torch.empty((M, w.q.N), dtype=torch.int8, device=qa.device)
    ys = torch.empty((M, w.q.N // 128), dtype=torch.float32, device=qa.device)
    check(load().e2mi_i8_gemm_q(stream_ptr(stream), ptr(yq), ptr(ys), ptr(qa), ptr(as_), w.ref, M),
          "i8_gemm_q")
    return yq, ys


def i8_gemm_tok(qa, as_, w: DeviceWeight, n0=0, n1=None, y=None, stream=None):
    """GEMM over per-token activation scales as_ [M] (or [M, 1])."""
    import torch
    M = qa.shape[0]
    n1 = w.q.N if n1 is None else n1
    y = torch.zeros((M, w.q.N), dtype=torch.float32, device=qa.device) if y is None else y
    check(load().e2mi_i8_gemm_tok(stream_ptr(stream), ptr(y), y.stride(0), ptr(qa), ptr(as_), w.ref,
                                  M, n0, n1), "i8_gemm_tok")
    return y


def i8_gemm_tok_q(qa, as_, w: DeviceWeight, stream=None):
    import torch
    M = qa.shape[0]
    yq = torch.empty((M, w.q.N), dtype=torch.int8, device=qa.device)
    ys = torch.empty((M, w.q.N // 128), dtype=torch.float32, device=qa.device)
    check(load().e2mi_i8_gemm_tok_q(stream_ptr(stream), ptr(yq), ptr(ys), ptr(qa), ptr(as_), w.ref, M),
          "i8_gemm_tok_q")
    return yq, ys


def i8_gemm_gelu_mul(qa, as_, w: DeviceWeight, mul, want_g=True, stream=None):
    """q, qs = quantize(gelu_tanh(qa . W) * mul) per 128 (the PLE gate, text.c:906-913); mul may be a
    column slice of a wider row-major f32 tensor. Returns (q, qs, g)."""
    import torch
    M = qa.shape[0]
    N = w.q.N
    q = torch.empty((M, N), dtype=torch.int8, device=qa.device)
    qs = torch.empty((M, N // 128), dtype=torch.float32, device=qa.device)
    g = torch.empty((M, N), dtype=torch.float32, device=qa.device) if want_g else None
    check(load().e2mi_i8_gemm_gelu_mul(stream_ptr(stream), ptr(q), ptr(qs), ptr(g), ptr(qa), ptr(as_),
                                       w.ref, M, ptr(mul), mul.stride(0)), "i8_gemm_gelu_mul")
    return q, qs, g


def i8_gemm_geglu(qa, as_, w: DeviceWeight, want_g=True, stream=None):
    import torch
    M = qa.shape[0]
    F = w.q.N // 2
    q = torch.empty((M, F), dtype=torch.int8, device=qa.device)
    qs = torch.empty((M, F // 128), dtype=torch.float32, device=qa.device)
    g = torch.empty((M, F), dtype=torch.float32, device=qa.device) if want_g else None
    check(load().e2mi_i8_gemm_geglu(stream_ptr(stream), ptr(q), ptr(qs), ptr(g), ptr(qa), ptr(as_),
                                    w.ref, M), "i8_gemm_geglu")
    return q, qs, g


# ---- row kernels
def norm_quant(x, gamma, eps=1e-6, want_xn=True, quant=True, stream=None):
    import torch
    M, D = x.shape
    xn = torch.empty_like(x) if want_xn else None
    q = torch.empty((M, D), dtype=torch.int8, device=x.device) if quant else None
    qs = torch.empty((M, D // 128), dtype=torch.float32, device=x.device) if quant else None
    check(load().e2mi_norm_quant(stream_ptr(stream), ptr(x), ptr(gamma), eps, M, D, ptr(xn), ptr(q),
                                 ptr(qs)), "norm_quant")
    return xn, q, qs


def add_norm_quant(src, res, gamma_add, gamma_next=None, eps=1e-6, x_out=None, want_xn=True,
                   quant=True, stream=None):
    import torch
    M, D = src.shape
    x_out = torch.empty_like(src) if x_out is None else x_out
    has_next = gamma_next is not None
    xn = torch.empty_like(src) if (want_xn and has_next) else None
    q = torch.empty((M, D), dtype=torch.int8, device=src.device) if (quant and has_next) else None
    qs = torch.empty((M, D // 128), dtype=torch.float32, device=src.device) if q is not None else None
    check(load().e2mi_add_norm_quant(stream_ptr(stream), ptr(src), ptr(res), ptr(gamma_add),
                                     ptr(gamma_next), eps, M, D, ptr(x_out), ptr(xn), ptr(q),
                                     ptr(qs)), "add_norm_quant")
    return x_out, xn, q, qs


def i8_gemm_add_norm_quant(qa, as_, w: DeviceWeight, res, gamma_add, gamma_next=None, eps=1e-6,
                           x_out=None, want_xn=True, quant=True, want_y=False, stream=None):
    """e2mi_i8_gemm_add_norm_quant: i8_gemm then add_norm_quant in one kernel; returns
    (x, xn, q, qs, y) like add_norm_quant, plus the projection y when want_y."""
    import torch
    M, D = res.shape
    x_out = torch.empty_like(res) if x_out is None else x_out
    has_next = gamma_next is not None
    xn = torch.empty_like(res) if (want_xn and has_next) else None
    q = torch.empty((M, D), dtype=torch.int8, device=res.device) if (quant and has_next) else None
    qs = torch.empty((M, D // 128), dtype=torch.float32, device=res.device) if q is not None else None
    y = torch.empty_like(res) if want_y else None
    check(load().e2mi_i8_gemm_add_norm_quant(stream_ptr(stream), ptr(qa), ptr(as_), w.ref, M, ptr(res),
                                             ptr(gamma_add), ptr(gamma_next), eps, ptr(x_out), ptr(xn),
                                             ptr(q), ptr(qs), ptr(y)), "i8_gemm_add_norm_quant")
    return x_out, xn, q, qs, y


def i8_gemm_add_norm_scale_quant(qa, as_, w: DeviceWeight, res, gamma_add, post_scale, gamma_next=None,
                                 eps=1e-6, x_out=None, want_xn=True, quant=True, want_y=False, stream=None):
    """e2mi_i8_gemm_add_norm_scale_quant: i8_gemm then add_norm_scale_quant in one kernel (512-wide
    rows); returns (x, xn, q, qs, y); without gamma_next, q/qs quantize x itself."""
    import torch
    M, D = res.shape
    x_out = torch.empty_like(res) if x_out is None else x_out
    has_next = gamma_next is not None
    xn = torch.empty_like(res) if (want_xn and has_next) else None
    q = torch.empty((M, D), dtype=torch.int8, device=res.device) if quant else None
    qs = torch.empty((M, D // 128), dtype=torch.float32, device=res.device) if quant else None
    y = torch.empty_like(res) if want_y else None
    check(load().e2mi_i8_gemm_add_norm_scale_quant(stream_ptr(stream), ptr(qa), ptr(as_), w.ref, M, ptr(res),
                                                   ptr(gamma_add), post_scale, ptr(gamma_next), eps, ptr(x_out),
                                                   ptr(xn), ptr(q), ptr(qs), ptr(y)),
          "i8_gemm_add_norm_scale_quant")
    return x_out, xn, q, qs, y


def embed_norm_quant(table, ids, embed_scale, gamma, eps=1e-6, stream=None):
    import torch
    M = ids.shape[0]
    V, D = table.shape
    x = torch.empty((M, D), dtype=torch.float32, device=table.device)
    q = torch.empty((M, D), dtype=torch.int8, device=table.device)
    qs = torch.empty((M, D // 128), dtype=torch.float32, device=table.device)
    check(load().e2mi_embed_norm_quant(stream_ptr(stream), ptr(table), V, ptr(ids), embed_scale,
                                       ptr(gamma), eps, M, D, ptr(x), ptr(q), ptr(qs)),
          "embed_norm_quant")
    return x, q, qs


def qkv_norm_rope(qkv, S, H, KV, q_gamma, k_gamma, cos_tab, sin_tab, eps=1e-6, want_f32=True,
                  stream=None):
    import torch
    M = qkv.shape[0]
    D = 256
    B = M // S
    dev = qkv.device
    q16 = torch.empty((M, H * D), dtype=torch.float16, device=dev)
    k16 = torch.empty((M, KV * D), dtype=torch.float16, device=dev)
    vt16 = torch.empty((B, KV, D, S), dtype=torch.float16, device=dev)
    f = (lambda *s: torch.empty(s, dtype=torch.float32, device=dev)) if want_f32 else (lambda *s: None)
    q32, k32, v32 = f(M, H * D), f(M, KV * D), f(M, KV * D)
    check(load().e2mi_qkv_norm_rope(stream_ptr(stream), ptr(qkv), M, S, H, KV, D, ptr(q_gamma),
                                    ptr(k_gamma), eps, ptr(cos_tab), ptr(sin_tab), ptr(q16),
                                    ptr(k16), ptr(vt16), ptr(q32), ptr(k32), ptr(v32)),
          "qkv_norm_rope")
    return q16, k16, vt16, q32, k32, v32


def qkv_pair_order(n):
    """Row order of the fused q|k|v weight (e2mi_i8_gemm_qkv): device row r holds logical row
    pair_order(r), bits 6 and 7 of the index swapped (its own inverse)."""
    import numpy as np
    n = np.asarray(n)
    return (n & ~0xC0) | ((n & 0x40) << 1) | ((n & 0x80) >> 1)


def i8_gemm_qkv(qa, as_, w: DeviceWeight, H, KV, q_gamma, k_gamma, cos_tab, sin_tab, S=None, pos=None,
                eps=1e-6, want_f32=False, stream=None):
    """The fused q|k|v GEMM + norms + RoPE (w uploaded in qkv_pair_order). pos given: packed rows
    (V^T [KV][256][M]); else positions m % S (V^T [M/S][KV][256][S])."""
    import torch
    M = qa.shape[0]
    D = 256
    dev = qa.device
    S = M if pos is not None else S
    q16 = torch.empty((M, H * D), dtype=torch.float16, device=dev)
    k16 = torch.empty((M, KV * D), dtype=torch.float16, device=dev)
    vt16 = torch.empty((M // S, KV, D, S), dtype=torch.float16, device=dev)
    f = (lambda *s: torch.empty(s, dtype=torch.float32, device=dev)) if want_f32 else (lambda *s: None)
    q32, k32, v32 = f(M, H * D), f(M, KV * D), f(M, KV * D)
    check(load().e2mi_i8_gemm_qkv(stream_ptr(stream), ptr(qa), ptr(as_), w.ref, M, S, ptr(pos), H, KV,
                                  ptr(q_gamma), ptr(k_gamma), eps, ptr(cos_tab), ptr(sin_tab), ptr(q16),
                                  ptr(k16), ptr(vt16), ptr(q32), ptr(k32), ptr(v32)), "i8_gemm_qkv")
    return q16, k16, vt16, q32, k32, v32


def gelu_mul_quant(gate, up, write_back=True, stream=None):
    import torch
    M, D = gate.shape
    q = torch.empty((M, D), dtype=torch.int8, device=gate.device)
    qs = torch.empty((M, D // 128), dtype=torch.float32, device=gate.device)
    check(load().e2mi_gelu_mul_quant(stream_ptr(stream), ptr(gate), gate.stride(0), ptr(up),
                                     up.stride(0), M, D, ptr(q), ptr(qs), int(write_back)),
          "gelu_mul_quant")
    return q, qs


def pool_l2(x, valid, B, S, stream=None):
    import torch
    D = x.shape[1]
    lib = load()
    ws = torch.empty(lib.e2mi_pool_workspace_bytes(B, S, D) // 4 + 64, dtype=torch.float32,
                     device=x.device)
    out = torch.empty((B, D), dtype=torch.float32, device=x.device)
    check(lib.e2mi_pool_l2(stream_ptr(stream), ptr(x), ptr(valid), B, S, D, ptr(ws), ptr(out)),
          "pool_l2")
    return out


def attention(q16, k16, vt16, valid, B, S, H, KV, scale=1.0, want_f32=True, stream=None):
    import torch
    M = B * S
    D = 256
    dev = q16.device
    cq = torch.empty((M, H * D), dtype=torch.int8, device=dev)
    cs = torch.empty((M, H * D // 128), dtype=torch.float32, device=dev)
    c32 = torch.empty((M, H * D), dtype=torch.float32, device=dev) if want_f32 else None
    check(load().e2mi_attention(stream_ptr(stream), ptr(q16), ptr(k16), ptr(vt16), ptr(valid), B, S,
                                H, KV, D, scale, ptr(cq), ptr(cs), ptr(c32)), "attention")
    return cq, cs, c32


# ---- packed batches (valid tokens only, sequence b in rows [start[b], start[b] + len[b]))
def pack_plan(valid):
    """The engine's packed layout of a [B, S] mask (e2mi_plan_pack): each sequence's valid tokens in
    order from a row that is a multiple of 8, the total rounded up to 256. Returns (rowmap, pos,
    start, len, M): rowmap[r] = b * S + s of packed row r (-1 for filler rows), pos[r] = s."""
    import numpy as np
    valid = np.ascontiguousarray(np.asarray(valid) != 0, np.uint8)
    B, S = valid.shape
    cap = B * ((S + 7) & ~7) + 256
    rowmap, pos = np.empty(cap, np.int32), np.empty(cap, np.int32)
    start, lens = np.empty(B, np.int32), np.empty(B, np.int32)
    M = load().e2mi_plan_pack(ptr(valid), B, S, ptr(rowmap), ptr(pos), ptr(start), ptr(lens))
    check(0 if M > 0 else -1, "plan_pack")
    return rowmap[:M].copy(), pos[:M].copy(), start, lens, M


def qkv_norm_rope_packed(qkv, pos, H, KV, q_gamma, k_gamma, cos_tab, sin_tab, eps=1e-6,
                         want_f32=True, stream=None, D=256):
    import torch
    M = qkv.shape[0]
    dev = qkv.device
    q16 = torch.empty((M, H * D), dtype=torch.float16, device=dev)
    k16 = torch.empty((M, KV * D), dtype=torch.float16, device=dev)
    vt16 = torch.empty((KV, D, M), dtype=torch.float16, device=dev)
    f = (lambda *s: torch.empty(s, dtype=torch.float32, device=dev)) if want_f32 else (lambda *s: None)
    q32, k32, v32 = f(M, H * D), f(M, KV * D), f(M, KV * D)
    check(load().e2mi_qkv_norm_rope_packed(stream_ptr(stream), ptr(qkv), M, ptr(pos), H, KV, D,
                                           ptr(q_gamma), ptr(k_gamma), eps, ptr(cos_tab),
                                           ptr(sin_tab), ptr(q16), ptr(k16), ptr(vt16), ptr(q32),
                                           ptr(k32), ptr(v32)), "qkv_norm_rope_packed")
    return q16, k16, vt16, q32, k32, v32


def work_entry(b, h, part, parts, qb):
    """An attention work entry (include/e2mi.h, e2mi_attention_packed_split)."""
    return b | (h << 16) | (part << 20) | ((parts - 1) << 22) | (qb << 24)


def plan_attention(lens, H, window=0, max_parts=1, div=2):
    """The engine's attention work list (e2mi_plan_attention): returns (work, merge) as int32 arrays
    (merge empty when nothing is split)."""
    import numpy as np
    lens = np.ascontiguousarray(lens, np.int32)
    blocks = int(sum((int(L) + 127) // 128 for L in lens))
    work = np.empty(max(1, H * blocks * max_parts), np.int32)
    merge = np.empty(max(1, H * blocks), np.int32)
    nm = C.c_int(0)
    n = load().e2mi_plan_attention(ptr(lens), len(lens), H, window, max_parts, div, ptr(work), ptr(merge),
                                   C.byref(nm))
    check(0 if n >= 0 else -1, "plan_attention")
    return work[:n].copy(), merge[:nm.value].copy()


def attention_work(lens, H, window=0, div=2):
    """The engine's unsplit attention work list for packed sequences of these lengths (one entry per
    128-query block, longest sequences first, dealt to the XCDs; div 4 at head_dim 512)."""
    return plan_attention(lens, H, window, 1, div)[0]


def plan_device(valid, H, window=0, div=2, ids=None, n_slots=None, stream=None):
    """The device planner (e2mi_plan_device) on a [B, S] device mask (uint8 tensor): returns
    (rowmap, pos, start, len, M, work, ids_out) as device tensors, rowmap, pos and ids_out cut to M
    rows, work to n_slots entries (default H (ceil(B S / 128) + B)); ids_out is None without ids."""
    import torch
    B, S = valid.shape
    dev = valid.device
    cap = B * ((S + 7) & ~7) + 256
    n_slots = n_slots or H * ((B * S + 127) // 128 + B)
    i32 = lambda n: torch.full((n,), -7, dtype=torch.int32, device=dev)
    rowmap, pos, start, lens, work, rows = i32(cap), i32(cap), i32(B), i32(B), i32(n_slots), i32(1)
    ids_out = i32(cap) if ids is not None else None
    check(load().e2mi_plan_device(stream_ptr(stream), ptr(valid), ptr(ids), B, S, H, window, div, n_slots,
                                  ptr(rowmap), ptr(pos), ptr(start), ptr(lens), ptr(ids_out), ptr(work),
                                  ptr(rows)), "plan_device")
    M = int(rows.item())
    return (rowmap[:M], pos[:M], start, lens, M, work, None if ids_out is None else ids_out[:M])


def attention_split_work(lens, H, max_parts=4, window=0):
    """Work and merge lists with split key ranges (e2mi_attention_packed_split): merge is [-1] when
    no block is split."""
    import numpy as np
    work, merge = plan_attention(lens, H, window, max_parts)
    return work, (merge if len(merge) else np.asarray([-1], np.int32))


def attention_packed_split(q16, k16, vt16, start, lens, max_len, H, KV, work, merge, window=0, pos=None,
                           scale=1.0, want_f32=True, stream=None):
    """e2mi_attention_packed_split (head_dim 256) with work/merge lists from attention_split_work."""
    import torch
    M = q16.shape[0]
    dev = q16.device
    D = 256
    cq = torch.zeros((M, H * D), dtype=torch.int8, device=dev)
    cs = torch.zeros((M, H * D // 128), dtype=torch.float32, device=dev)
    c32 = torch.zeros((M, H * D), dtype=torch.float32, device=dev) if want_f32 else None
    nb = load().e2mi_attention_part_bytes(M, H, D)
    part = torch.empty(nb // 4, dtype=torch.float32, device=dev)
    wt = torch.from_numpy(work).to(dev)
    mt = torch.from_numpy(merge).to(dev)
    check(load().e2mi_attention_packed_split(stream_ptr(stream), ptr(q16), ptr(k16), ptr(vt16), M, ptr(start),
                                             ptr(lens), ptr(pos), start.shape[0], max_len, H, KV, D, scale,
                                             window, ptr(cq), ptr(cs), ptr(c32), ptr(wt), wt.shape[0], ptr(mt),
                                             mt.shape[0], ptr(part), M), "attention_packed_split")
    return cq, cs, c32


def attention_packed(q16, k16, vt16, start, lens, max_len, H, KV, scale=1.0, want_f32=True,
                     cq=None, cs=None, c32=None, work=None, stream=None):
    import torch
    M = q16.shape[0]
    D = 256
    dev = q16.device
    cq = torch.zeros((M, H * D), dtype=torch.int8, device=dev) if cq is None else cq
    cs = torch.zeros((M, H * D // 128), dtype=torch.float32, device=dev) if cs is None else cs
    if want_f32 and c32 is None:
        c32 = torch.zeros((M, H * D), dtype=torch.float32, device=dev)
    check(load().e2mi_attention_packed(stream_ptr(stream), ptr(q16), ptr(k16), ptr(vt16), M,
                                       ptr(start), ptr(lens), start.shape[0], max_len, H, KV, D,
                                       scale, ptr(cq), ptr(cs), ptr(c32), ptr(work),
                                       0 if work is None else work.shape[0]), "attention_packed")
    return cq, cs, c32


def attention_packed_window(q16, k16, vt16, start, lens, max_len, H, KV, D, window=0, pos=None,
                            scale=1.0, want_f32=True, cq=None, cs=None, c32=None, work=None, stream=None):
    """Packed attention at head_dim 256 or 512 with the sliding window of text.c:542-546 (keys with
    |pos_i - pos_j| <= window; pos None: the packed index); returns (cq, cs, c32)."""
    import torch
    M = q16.shape[0]
    dev = q16.device
    cq = torch.zeros((M, H * D), dtype=torch.int8, device=dev) if cq is None else cq
    cs = torch.zeros((M, H * D // 128), dtype=torch.float32, device=dev) if cs is None else cs
    if want_f32 and c32 is None:
        c32 = torch.zeros((M, H * D), dtype=torch.float32, device=dev)
    check(load().e2mi_attention_packed_window(stream_ptr(stream), ptr(q16), ptr(k16), ptr(vt16), M,
                                              ptr(start), ptr(lens), ptr(pos), start.shape[0], max_len,
                                              H, KV, D, scale, window, ptr(cq), ptr(cs), ptr(c32), ptr(work),
                                              0 if work is None else work.shape[0]), "attention_packed_window")
    return cq, cs, c32


def add_norm_scale_quant(src, res, gamma_add, post_scale, gamma_next=None, eps=1e-6, x_out=None,
                         want_xn=True, quant=True, stream=None):
    """x = (rms(src)*gamma_add + res) * post_scale; with gamma_next its norm (+ quant), without it
    x itself quantized (text.c:957-961, 911). Returns (x, xn, q, qs)."""
    import torch
    M, D = src.shape
    x_out = torch.empty_like(src) if x_out is None else x_out
    has_next = gamma_next is not None
    xn = torch.empty_like(src) if (want_xn and has_next) else None
    q = torch.empty((M, D), dtype=torch.int8, device=src.device) if quant else None
    qs = torch.empty((M, D // 128), dtype=torch.float32, device=src.device) if quant else None
    check(load().e2mi_add_norm_scale_quant(stream_ptr(stream), ptr(src), ptr(res), ptr(gamma_add), post_scale,
                                           ptr(gamma_next), eps, M, D, ptr(x_out), ptr(xn), ptr(q), ptr(qs)),
          "add_norm_scale_quant")
    return x_out, xn, q, qs


def scale_norm(x, pre_scale, gamma, eps=1e-6, out=None, stream=None):
    """rms(x * pre_scale) * gamma per row of x [rows][D] (text.c:930-931)."""
    import torch
    rows, D = x.shape
    out = torch.empty_like(x) if out is None else out
    check(load().e2mi_scale_norm(stream_ptr(stream), ptr(x), rows, D, pre_scale, ptr(gamma), eps, ptr(out)),
          "scale_norm")
    return out


def attention_i8_packed(q32, k32, v32, start, lens, max_len, H, KV, want_f32=True, cq=None, cs=None,
                        c32=None, work=None, workspace=None, stream=None):
    """The int8 attention variant (text.c:638-700) of each packed sequence; returns (cq, cs, c32)."""
    import torch
    M = q32.shape[0]
    D = 256
    dev = q32.device
    B = start.shape[0]
    lib = load()
    if workspace is None:
        nbytes = lib.e2mi_attention_i8_workspace_bytes(M, B, max_len, H, KV)
        workspace = torch.empty(nbytes + 256, dtype=torch.uint8, device=dev)
    cq = torch.zeros((M, H * D), dtype=torch.int8, device=dev) if cq is None else cq
    cs = torch.zeros((M, H * D // 128), dtype=torch.float32, device=dev) if cs is None else cs
    if want_f32 and c32 is None:
        c32 = torch.zeros((M, H * D), dtype=torch.float32, device=dev)
    wp = C.c_void_p((workspace.data_ptr() + 255) & ~255)
    check(lib.e2mi_attention_i8_packed(stream_ptr(stream), ptr(q32), ptr(k32), ptr(v32), M, ptr(start),
                                       ptr(lens), B, max_len, H, KV, D, wp, ptr(cq), ptr(cs), ptr(c32),
                                       ptr(work), 0 if work is None else work.shape[0]),
          "attention_i8_packed")
    return cq, cs, c32


def pool_l2_packed(x, start, lens, max_len, stream=None):
    import torch
    D = x.shape[1]
    B = start.shape[0]
    lib = load()
    ws = torch.empty(lib.e2mi_pool_workspace_bytes(B, max_len, D) // 4 + 64, dtype=torch.float32,
                     device=x.device)
    out = torch.empty((B, D), dtype=torch.float32, device=x.device)
    check(lib.e2mi_pool_l2_packed(stream_ptr(stream), ptr(x), ptr(start), ptr(lens), B, max_len, D,
                                  ptr(ws), ptr(out)), "pool_l2_packed")
    return out


def gather_ids(ids, rowmap, stream=None):
    import torch
    M = rowmap.shape[0]
    out = torch.empty(M, dtype=torch.int32, device=rowmap.device)
    check(load().e2mi_gather_ids(stream_ptr(stream), ptr(ids), ptr(rowmap), M, ptr(out)), "gather_ids")
    return out


# ---- model container and encoder engine
Q8_SUFFIXES = ("self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
               "self_attn.o_proj.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight",
               "ple_block.per_layer_input_gate.weight", "ple_block.per_layer_projection.weight")
NORM_SUFFIXES = ("input_layernorm.weight", "post_attention_layernorm.weight", "pre_feedforward_layernorm.weight",
                 "post_feedforward_layernorm.weight", "self_attn.q_norm.weight", "self_attn.k_norm.weight",
                 "ple_block.post_per_layer_input_norm.weight")


def tensor_names(cfg):
    """The reference's names (e2.c:306-402) of every tensor the text tower of `cfg` reads."""
    ple = cfg.ple_dim > 0
    names = ["language_model.embed_tokens.weight", "language_model.norm.weight"]
    if ple:
        names += ["language_model.ple.per_layer_model_projection.weight",
                  "language_model.ple.per_layer_projection_norm.weight"]
    if cfg.out_dim > 0:
        names.append("language_model.embedding_projection.weight")
    for l in range(cfg.n_layers):
        pre = f"language_model.layers.{l}."
        names += [pre + s for s in Q8_SUFFIXES[:9 if ple else 7]]
        names += [pre + s for s in NORM_SUFFIXES[:7 if ple else 6]]
        if ple:
            names.append(pre + "layer_scalar")
    return names


def model_tensors(model, table=None):
    """e2mi_tensor records viewing `model`'s own buffers (no copies; keep the model alive while they
    are used). `table`, a uint16 bf16 array [vocab][hidden], replaces the f32 token table (the
    reference holds it in bf16)."""
    cfg = model.config
    recs, keep = [], []
    for name in tensor_names(cfg):
        v = TensorView()
        check(load().e2_model_tensor(model.h, name.encode(), C.byref(v)), "model_tensor")
        bname = name.encode()
        keep.append(bname)
        if v.kind == 3:
            N, K, nb, Npad = (int(d) for d in v.dims)
            recs.append(E2MITensor(bname, 3, N, K, nb, Npad, v.data, v.scale, v.bsq))
        elif name == "language_model.embed_tokens.weight" and table is not None:
            keep.append(table)
            recs.append(E2MITensor(bname, 1, table.shape[0], table.shape[1], 0, 0, table.ctypes.data, None, None))
        else:
            n = v.nbytes // 4
            rows = int(v.dims[0]) if v.ndim == 2 else 1
            recs.append(E2MITensor(bname, 2, rows, n // rows, 0, 0, v.data, None, None))
    arr = (E2MITensor * len(recs))(*recs)
    arr._keep = keep
    return arr


def baseline_config(**over):
    c = E2Config()
    load().e2_config_baseline(C.byref(c))
    for k, v in over.items():
        setattr(c, k, v)
    return c


def reference_config(**over):
    """The reference checkpoint's text geometry (include/e2.h e2_config_reference)."""
    c = E2Config()
    load().e2_config_reference(C.byref(c))
    for k, v in over.items():
        setattr(c, k, v)
    return c


class Model:
    """An e2_model (include/e2.h): synthetic or loaded from an E8CQ cache; freed with the object."""

    def __init__(self, handle):
        if not handle:
            raise E2MIError(f"model: {last_error()}")
        self.h = C.c_void_p(handle)

    @classmethod
    def synthetic(cls, cfg: E2Config, seed: int):
        return cls(load().e2_model_synthetic(C.byref(cfg), seed))

    @classmethod
    def load_e8cq(cls, path: str, cfg: E2Config):
        return cls(load().e2_load_e8cq(path.encode(), C.byref(cfg)))

    def save_e8cq(self, path: str):
        check(load().e2_save_e8cq(self.h, path.encode()), "save_e8cq")

    @property
    def config(self) -> E2Config:
        c = E2Config()
        check(load().e2_model_config(self.h, C.byref(c)), "model_config")
        return c

    def tensor(self, name: str):
        """numpy copies: f32 tensors -> array; int8 weights -> (packed w, scale[N], bsq, N, K)."""
        import numpy as np
        v = TensorView()
        check(load().e2_model_tensor(self.h, name.encode(), C.byref(v)), "model_tensor")
        if v.kind == 2:
            n = v.nbytes // 4
            a = np.ctypeslib.as_array(C.cast(v.data, C.POINTER(C.c_float)), (n,)).copy()
            return a.reshape([int(d) for d in v.dims[:v.ndim]])
        N, K, nb, Npad = (int(d) for d in v.dims)
        w = np.ctypeslib.as_array(C.cast(v.data, C.POINTER(C.c_int8)), (v.nbytes,)).copy()
        sc = np.ctypeslib.as_array(C.cast(v.scale, C.POINTER(C.c_float)), (N,)).copy()
        bsq = np.ctypeslib.as_array(C.cast(v.bsq, C.POINTER(C.c_int32)), (nb * Npad,)).copy()
        return w, sc, bsq.reshape(nb, Npad), N, K

    def __del__(self):
        if _lib is not None and getattr(self, "h", None):
            _lib.e2_free(self.h)
            self.h = None


class Engine:
    """An e2mi_engine (include/e2mi.h) on the current device; destroyed with the object."""

    def __init__(self, model: Model, max_rows: int = 0, _handle=None, _cfg=None):
        h = _handle if _handle is not None else load().e2mi_create_rows(model.h, max_rows)
        if not h:
            raise E2MIError(f"create: {last_error()}")
        self.h = C.c_void_p(h)
        cfg = _cfg if _cfg is not None else model.config
        self.hidden = cfg.hidden
        self.dim = cfg.out_dim if cfg.out_dim > 0 else cfg.hidden  # embedding width

    @classmethod
    def from_tensors(cls, tensors, cfg, geometry: int, max_rows: int = 0):
        """e2mi_create_tensors over e2mi_tensor records (model_tensors); cfg gives n_layers, vocab
        and the embedding width."""
        h = load().e2mi_create_tensors(tensors, len(tensors), geometry, cfg.n_layers, cfg.vocab, max_rows)
        if not h:
            raise E2MIError(f"create_tensors: {last_error()}")
        return cls(None, _handle=h, _cfg=cfg)

    @property
    def device(self) -> str:
        return load().e2mi_device(self.h).decode()

    def embed_batch(self, ids, valid=None):
        import numpy as np
        ids = np.ascontiguousarray(ids, np.int32)
        B, S = ids.shape
        v = None if valid is None else np.ascontiguousarray(valid, np.uint8)
        out = np.empty((B, self.dim), np.float32)
        check(load().e2mi_text_embed_batch(self.h, ptr(ids), ptr(v), B, S, ptr(out)),
              "text_embed_batch")
        return out

    def embed_batch_device(self, ids, valid, out, stream=None):
        B, S = ids.shape
        check(load().e2mi_text_embed_batch_device(self.h, ptr(ids), ptr(valid), B, S, ptr(out),
                                                  stream_ptr(stream)), "text_embed_batch_device")
        return out

    def stats(self):
        calls, kern, ms = C.c_long(), C.c_long(), C.c_double()
        check(load().e2mi_stats(self.h, C.byref(calls), C.byref(kern), C.byref(ms)), "stats")
        return calls.value, kern.value, ms.value

    def set_layer_limit(self, n: int):
        check(load().e2mi_set_layer_limit(self.h, n), "set_layer_limit")

    def set_packing(self, on: bool):
        """Packed batches (valid tokens only) on or off; off computes every padded row."""
        check(load().e2mi_set_packing(self.h, 1 if on else 0), "set_packing")

    def set_device_plan(self, on: bool):
        """The device entry's packed plan built on the device (default) or on the host."""
        check(load().e2mi_set_device_plan(self.h, 1 if on else 0), "set_device_plan")

    def set_split(self, mode: str):
        """Split key ranges: "off", "on" or "auto" (e2mi_set_attention_split)."""
        check(load().e2mi_set_attention_split(self.h, {"off": 0, "on": 1, "auto": 2}[mode]), "set_attention_split")

    def set_attention(self, kind: str):
        """Text attention kind: "f16" (default) or "i8" (the reference's int8 attention for
        sequences of at least 32 tokens)."""
        check(load().e2mi_set_attention(self.h, {"f16": 1, "i8": 2}[kind]), "set_attention")

    def __del__(self):
        if _lib is not None and getattr(self, "h", None):
            _lib.e2mi_destroy(self.h)
            self.h = None
