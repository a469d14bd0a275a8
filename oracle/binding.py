"""ctypes bindings for the CPU oracle (liboracle.so) and the reference build (oracle/_ref).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, never by the product package. Arrays are numpy; every function checks dtype/contiguity and
shapes before handing raw pointers to C.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libe2ref.so")
REFTEXT_SO = os.path.join(HERE, "_ref", "libreftext.so")

_P = C.c_void_p
_I = C.c_int
_F = C.c_float


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _need(a, dtype, shape=None):
    if not isinstance(a, np.ndarray) or a.dtype != np.dtype(dtype) or not a.flags.c_contiguous:
        raise TypeError(f"expected C-contiguous {dtype} array, got {type(a)} {getattr(a, 'dtype', None)}")
    if shape is not None and tuple(a.shape) != tuple(shape):
        raise ValueError(f"expected shape {shape}, got {a.shape}")
    return a


_LAYER_PTRS = ("wqkv", "sqkv", "wo", "so", "wgate", "sgate", "wup", "sup", "wdown", "sdown",
               "input_ln", "post_attn_ln", "pre_ffn_ln", "post_ffn_ln", "q_norm", "k_norm")
_LAYER_PLE = ("wple_gate", "sple_gate", "wple_proj", "sple_proj", "ple_norm")


class OrLayer(C.Structure):
    _fields_ = [(n, _P) for n in _LAYER_PTRS + _LAYER_PLE] + [("layer_scalar", _F)]


class OrModel(C.Structure):
    _fields_ = [("n_layers", _I), ("hidden", _I), ("ffn", _I), ("n_heads", _I), ("n_kv", _I),
                ("head_dim", _I), ("vocab", _I), ("eps", _F), ("rope_theta", _F),
                ("embed_scale", _F), ("attn_scale", _F), ("embed", _P), ("final_norm", _P),
                ("layers", C.POINTER(OrLayer)), ("attn_i8", _I),
                ("ple_dim", _I), ("out_dim", _I), ("window", _I), ("full_period", _I),
                ("full_head_dim", _I), ("full_kv", _I), ("rope_theta_full", _F), ("ple_scale", _F),
                ("wple_model", _P), ("sple_model", _P), ("ple_proj_norm", _P),
                ("wembed_proj", _P), ("sembed_proj", _P), ("i8_min_keys", _I)]


class Oracle:
    """The C restatement; see oracle/e2_oracle.c for what pins each function."""

    def __init__(self, path=ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not built (run __graft_entry__.build())")
        L = self.lib = C.CDLL(path)
        sig = {
            "or_q8w_from_f32": (_I, [_P, _I, _I, _P, _P, _P]),
            "or_q8w_unpack": (None, [_P, _I, _I, _P]),
            "or_q8w_pack": (None, [_P, _I, _I, _P, _P]),
            "or_quantize": (None, [_P, _I, _I, _I, _I, _P, _P]),
            "or_quantize_mt": (None, [_P, _I, _I, _P, _P, _I]),
            "or_i8_gemm": (None, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _F, _P]),
            "or_i8_gemm_acc": (None, [_P, _P, _I, _I, _I, _I, _P]),
            "or_i8_gemm_scalar": (None, [_P, _P, _P, _P, _I, _I, _I, _P]),
            "or_i8_gemm_mt": (None, [_P, _P, _P, _P, _P, _I, _I, _I, _P, _I]),
            "or_i8_gemm_mt_block": (None, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _I]),
            "or_gelu_tanh": (_F, [_F]),
            "or_gelu_mul_quant": (None, [_P, _I, _P, _I, _I, _I, _I, _P, _P]),
            "or_rmsnorm": (None, [_P, _I, _I, _P, _F]),
            "or_norm_split": (None, [_P, _P, _I, _I, _P, _F]),
            "or_norm_add": (None, [_P, _P, _P, _I, _I, _P, _F]),
            "or_rope_table": (None, [_I, _I, _F, _P, _P]),
            "or_rope_rows": (None, [_P, _I, _I, _I, _P, _P]),
            "or_softmax": (None, [_P, _I]),
            "or_attention": (None, [_P, _I, _P, _I, _P, _I, _P, _I, _I, _I, _I, _F, _P, _I, _I]),
            "or_attention_win": (None, [_P, _I, _P, _I, _P, _I, _P, _I, _I, _I, _I, _F, _I, _P, _I, _I]),
            "or_attention_i8": (_I, [_P, _I, _P, _I, _P, _I, _I, _I, _I, _I, _P, _I]),
            "or_meanpool": (None, [_P, _I, _I, _P, _P]),
            "or_l2norm": (None, [_P, _I]),
            "or_embed": (None, [_P, _P, _I, _I, _F, _P]),
            "or_layer_forward": (_I, [C.POINTER(OrModel), _I, _P, _I, _I, _P, _I]),
            "or_attention_sublayer": (_I, [C.POINTER(OrModel), _I, _P, _I, _I, _P, _P, _I]),
            "or_ffn_sublayer": (_I, [C.POINTER(OrModel), _I, _P, _I, _I]),
            "or_encode": (_I, [C.POINTER(OrModel), _P, _P, _I, _I, _P, _I]),
            "or_layer_forward_ple": (_I, [C.POINTER(OrModel), _I, _P, _P, _I, _I, _P, _I]),
            "or_ple_inputs": (_I, [C.POINTER(OrModel), _P, _I, _P, _I]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args

    # ---- weights
    def q8w_from_f32(self, w):
        w = _need(np.ascontiguousarray(w, np.float32), np.float32)
        N, K = w.shape
        Npad, kq, nb = (N + 7) & ~7, (K + 3) // 4, (K + 127) // 128
        wq = np.zeros(Npad // 8 * kq * 32, np.int8)
        sc = np.zeros(Npad, np.float32)
        bsq = np.zeros((nb, Npad), np.int32)
        self.lib.or_q8w_from_f32(_ptr(w), N, K, _ptr(wq), _ptr(sc), _ptr(bsq))
        return wq, sc, bsq

    def q8w_unpack(self, wq, N, K):
        out = np.empty((N, K), np.int8)
        self.lib.or_q8w_unpack(_ptr(_need(wq, np.int8)), N, K, _ptr(out))
        return out

    def q8w_pack(self, w):
        w = _need(w, np.int8)
        N, K = w.shape
        Npad, kq, nb = (N + 7) & ~7, (K + 3) // 4, (K + 127) // 128
        wq = np.zeros(Npad // 8 * kq * 32, np.int8)
        bsq = np.zeros((nb, Npad), np.int32)
        self.lib.or_q8w_pack(_ptr(w), N, K, _ptr(wq), _ptr(bsq))
        return wq, bsq

    # ---- activations
    def quantize(self, x, block=128):
        x = _need(x, np.float32)
        M, K = x.shape
        nb = (K + block - 1) // block
        q = np.empty((M, K), np.int8)
        s = np.empty((M, nb), np.float32)
        self.lib.or_quantize(_ptr(x), M, K, K, block, _ptr(q), _ptr(s))
        return q, s

    def i8_gemm(self, qa, as_, w, ws, bias=None, block=128, lo=-1e31, hi=1e31):
        M, K = qa.shape
        N = w.shape[0]
        _need(qa, np.int8), _need(as_, np.float32), _need(w, np.int8, (N, K)), _need(ws, np.float32)
        if bias is not None:
            _need(bias, np.float32, (N,))
        y = np.empty((M, N), np.float32)
        self.lib.or_i8_gemm(_ptr(qa), _ptr(as_), _ptr(w), _ptr(ws), _ptr(bias), M, N, K, block,
                            lo, hi, _ptr(y))
        return y

    def i8_gemm_acc(self, qa, w, block=128):
        M, K = qa.shape
        N = w.shape[0]
        nb = (K + block - 1) // block
        acc = np.empty((nb, M, N), np.int32)
        self.lib.or_i8_gemm_acc(_ptr(_need(qa, np.int8)), _ptr(_need(w, np.int8)), M, N, K, block,
                                _ptr(acc))
        return acc

    def i8_gemm_scalar(self, qa, as_, w, ws):
        M, K = qa.shape
        N = w.shape[0]
        y = np.empty((M, N), np.float32)
        self.lib.or_i8_gemm_scalar(_ptr(qa), _ptr(as_), _ptr(w), _ptr(ws), M, N, K, _ptr(y))
        return y

    def i8_gemm_mt(self, qa, as_, w, ws, bias=None, nthreads=8, block=128):
        """The threaded VNNI form of i8_gemm (same fold): blocks of 128, or block = K (per token)."""
        M, K = qa.shape
        N = w.shape[0]
        if K % block or block % 4:
            raise ValueError("K must be a multiple of the block, the block of 4")
        y = np.empty((M, N), np.float32)
        self.lib.or_i8_gemm_mt_block(_ptr(_need(qa, np.int8)), _ptr(_need(as_, np.float32)),
                                     _ptr(_need(w, np.int8)), _ptr(_need(ws, np.float32)), _ptr(bias),
                                     M, N, K, block, _ptr(y), nthreads)
        return y

    def quantize_mt(self, x, nthreads=8):
        x = _need(x, np.float32)
        M, K = x.shape
        q = np.empty((M, K), np.int8)
        s = np.empty((M, K // 128), np.float32)
        self.lib.or_quantize_mt(_ptr(x), M, K, _ptr(q), _ptr(s), nthreads)
        return q, s

    # ---- fp32 ops (copies in, results out)
    def gelu_mul_quant(self, gate, up, block=128):
        g = np.array(gate, np.float32, copy=True, order="C")
        up = _need(np.ascontiguousarray(up, np.float32), np.float32)
        R, D = g.shape
        nb = (D + block - 1) // block
        q = np.empty((R, D), np.int8)
        s = np.empty((R, nb), np.float32)
        self.lib.or_gelu_mul_quant(_ptr(g), D, _ptr(up), D, R, D, block, _ptr(q), _ptr(s))
        return g, q, s

    def rmsnorm(self, x, gamma, eps):
        x = np.array(x, np.float32, copy=True, order="C")
        R, D = x.shape
        self.lib.or_rmsnorm(_ptr(x), R, D, _ptr(gamma), eps)
        return x

    def norm_split(self, x, gamma, eps):
        x = np.array(x, np.float32, copy=True, order="C")
        res = np.empty_like(x)
        self.lib.or_norm_split(_ptr(x), _ptr(res), x.shape[0], x.shape[1], _ptr(gamma), eps)
        return x, res

    def norm_add(self, src, res, gamma, eps):
        src = _need(np.ascontiguousarray(src, np.float32), np.float32)
        res = _need(np.ascontiguousarray(res, np.float32), np.float32)
        out = np.empty_like(src)
        self.lib.or_norm_add(_ptr(out), _ptr(src), _ptr(res), src.shape[0], src.shape[1],
                             _ptr(gamma), eps)
        return out

    def rope_table(self, max_pos, head_dim, theta):
        cs = np.empty((max_pos, head_dim), np.float32)
        sn = np.empty((max_pos, head_dim), np.float32)
        self.lib.or_rope_table(max_pos, head_dim, theta, _ptr(cs), _ptr(sn))
        return cs, sn

    def rope_rows(self, x, ngroups, cs, sn):
        x = np.array(x, np.float32, copy=True, order="C")
        R, D = x.shape
        self.lib.or_rope_rows(_ptr(x), R, ngroups, D, _ptr(cs), _ptr(sn))
        return x

    def softmax(self, x):
        x = np.array(x, np.float32, copy=True, order="C")
        self.lib.or_softmax(_ptr(x), x.size)
        return x

    def attention(self, q, k, v, valid, H, KV, D, scale=1.0, nthreads=8, window=0):
        """q [S][H*D], k/v [S][KV*D] (contiguous), valid [S] u8 -> ctx [S][H*D]; window > 0 keeps
        the keys with |i-j| <= window (text.c:542-546)."""
        S = q.shape[0]
        ctx = np.zeros((S, H * D), np.float32)
        self.lib.or_attention_win(_ptr(_need(q, np.float32)), H * D, _ptr(_need(k, np.float32)), KV * D,
                                  _ptr(_need(v, np.float32)), KV * D, _ptr(_need(valid, np.uint8)), S,
                                  H, KV, D, scale, window, _ptr(ctx), H * D, nthreads)
        return ctx

    def attention_i8(self, q, k, v, H, KV, D):
        """The reference's int8 attention (text.c:638-700) of one all-valid sequence:
        q [S][H*D], k/v [S][KV*D] -> ctx [S][H*D]."""
        S = q.shape[0]
        ctx = np.zeros((S, H * D), np.float32)
        if self.lib.or_attention_i8(_ptr(_need(q, np.float32)), H * D, _ptr(_need(k, np.float32)), KV * D,
                                    _ptr(_need(v, np.float32)), KV * D, S, H, KV, D, _ptr(ctx), H * D):
            raise MemoryError
        return ctx

    def meanpool_l2(self, x, valid):
        M, D = x.shape
        out = np.empty(D, np.float32)
        self.lib.or_meanpool(_ptr(_need(x, np.float32)), M, D, _ptr(valid), _ptr(out))
        if valid is None or valid.any():
            self.lib.or_l2norm(_ptr(out), D)
        return out


class OracleModel:
    """Holds numpy weight arrays alive and exposes them as an or_model for the recipe functions.

    cfg keys: hidden, ffn, n_heads, n_kv_heads, head_dim, vocab, rms_eps, rope_theta, embed_scale;
    for the reference checkpoint's geometry also ple_dim, out_dim, window, full_period,
    full_head_dim, full_kv_heads, rope_theta_full, ple_scale, with `extra` holding ple_model (w, s),
    ple_proj_norm and embed_proj (w, s), and each layer dict wple_gate/sple_gate, wple_proj/sple_proj,
    ple_norm and layer_scalar."""

    def __init__(self, oracle, cfg, layers, embed, final_norm, attn_scale=1.0, attn_i8=False, extra=None,
                 i8_min_keys=0):
        self.o = oracle
        extra = extra or {}
        self._keep = [layers, embed, final_norm, extra]
        ple = cfg.get("ple_dim", 0) > 0
        arr = (OrLayer * len(layers))()
        for i, Lw in enumerate(layers):
            for name in _LAYER_PTRS + (_LAYER_PLE if ple else ()):
                a = Lw[name]
                if not a.flags.c_contiguous:
                    raise ValueError(name)
                setattr(arr[i], name, a.ctypes.data)
            arr[i].layer_scalar = float(Lw.get("layer_scalar", 1.0))
        self._arr = arr

        def p(name):
            return extra[name].ctypes.data if name in extra else None
        self.m = OrModel(len(layers), cfg["hidden"], cfg["ffn"], cfg["n_heads"], cfg["n_kv_heads"],
                         cfg["head_dim"], cfg["vocab"], cfg["rms_eps"], cfg["rope_theta"],
                         cfg["embed_scale"], attn_scale, embed.ctypes.data, final_norm.ctypes.data,
                         C.cast(arr, C.POINTER(OrLayer)), 1 if attn_i8 else 0,
                         cfg.get("ple_dim", 0), cfg.get("out_dim", 0), cfg.get("window", 0),
                         cfg.get("full_period", 0), cfg.get("full_head_dim", 0), cfg.get("full_kv_heads", 0),
                         cfg.get("rope_theta_full", 0.0), cfg.get("ple_scale", 0.0),
                         p("wple_model"), p("sple_model"), p("ple_proj_norm"), p("wembed_proj"),
                         p("sembed_proj"), i8_min_keys)
        self.out_dim = cfg.get("out_dim", 0) or cfg["hidden"]

    def encode(self, ids, valid, nthreads=8):
        B, S = ids.shape
        out = np.empty((B, self.out_dim), np.float32)
        rc = self.o.lib.or_encode(C.byref(self.m), _ptr(_need(ids, np.int32)),
                                  _ptr(_need(valid, np.uint8)), B, S, _ptr(out), nthreads)
        if rc:
            raise RuntimeError("or_encode failed")
        return out

    def ple_inputs(self, x, nthreads=8):
        """x [rows][hidden] (the scaled embeddings) -> ple [rows][n_layers*ple_dim]."""
        x = _need(np.ascontiguousarray(x, np.float32), np.float32)
        ple = np.empty((x.shape[0], self.m.n_layers * self.m.ple_dim), np.float32)
        if self.o.lib.or_ple_inputs(C.byref(self.m), _ptr(x), x.shape[0], _ptr(ple), nthreads):
            raise RuntimeError("or_ple_inputs failed")
        return ple

    def layer_ple(self, l, x, ple, valid, B, S, nthreads=8):
        x = np.array(x, np.float32, copy=True, order="C")
        if self.o.lib.or_layer_forward_ple(C.byref(self.m), l, _ptr(x), _ptr(ple), B, S, _ptr(valid), nthreads):
            raise RuntimeError("or_layer_forward_ple failed")
        return x

    def layer(self, l, x, valid, B, S, nthreads=8):
        x = np.array(x, np.float32, copy=True, order="C")
        if self.o.lib.or_layer_forward(C.byref(self.m), l, _ptr(x), B, S, _ptr(valid), nthreads):
            raise RuntimeError("or_layer_forward failed")
        return x

    def attention_sublayer(self, l, x, valid, B, S, nthreads=8):
        x = _need(np.ascontiguousarray(x, np.float32), np.float32)
        out = np.empty((B * S, self.m.hidden), np.float32)
        if self.o.lib.or_attention_sublayer(C.byref(self.m), l, _ptr(x), B, S, _ptr(valid),
                                            _ptr(out), nthreads):
            raise RuntimeError("or_attention_sublayer failed")
        return out

    def ffn_sublayer(self, l, x, nthreads=8):
        x = np.array(x, np.float32, copy=True, order="C")
        if self.o.lib.or_ffn_sublayer(C.byref(self.m), l, _ptr(x), x.shape[0], nthreads):
            raise RuntimeError("or_ffn_sublayer failed")
        return x


# ------------------------------------------------------------------ the reference build
class Q8W(C.Structure):
    """e2_q8w (reference src/int8.h:79-92)."""
    _fields_ = [("w", _P), ("bsq", _P), ("scale", _P), ("N", _I), ("K", _I), ("nblocks", _I),
                ("Npad", _I), ("out_min", _F), ("out_max", _F), ("borrowed", _I)]


class Ref:
    """The reference's own kernels, compiled from /root/reference/src by oracle/Makefile."""

    def __init__(self, path=REF_SO, block=128):
        """block: the build's E2_I8_BLOCK (int8.h:61-70); the per-row builds under _ref/b<K>/ set
        it to K, so activation scales are one per row and weight block sums one per row."""
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        self.block = block
        L = self.lib = C.CDLL(path)
        L.e2_cpu_init.restype = None
        L.e2_cpu_init()
        for n in ("e2_quantize_blocks_avx512", "e2_quantize_blocks_scalar", "e2_quantize_blocks_vnni"):
            getattr(L, n).argtypes = [_P, _P, _P, _I, _I, _F, _F]
            getattr(L, n).restype = None
        for n in ("e2_i8_gemm_avx512", "e2_i8_gemm_scalar", "e2_i8_gemm_vnni_range"):
            getattr(L, n).argtypes = [_P, _P, _P, C.POINTER(Q8W), _I, _I, _I, _I]
            getattr(L, n).restype = None
        L.e2_q8w_from_f32.argtypes = [C.POINTER(Q8W), _P, _I, _I]
        L.e2_q8w_from_f32.restype = _I
        L.e2_q8w_free.argtypes = [C.POINTER(Q8W)]
        L.e2_q8w_free.restype = None
        L.e2_meanpool_f32.argtypes = [_P, _P, _I, _I, _P]
        L.e2_l2norm_f32.argtypes = [_P, _I]
        L.e2_k.restype = C.POINTER(_Kernels)

    @staticmethod
    def available(path=REF_SO):
        return os.path.exists(path)

    @staticmethod
    def per_row_path(K):
        """The reference built with E2_I8_BLOCK = K (oracle/Makefile ROWK)."""
        return os.path.join(HERE, "_ref", f"b{K}", "libe2ref.so")

    @classmethod
    def per_row(cls, K):
        return cls(cls.per_row_path(K), block=K)

    def quantize(self, x, which="avx512"):
        x = _need(np.ascontiguousarray(x, np.float32), np.float32)
        M, K = x.shape
        nb = (K + self.block - 1) // self.block
        q = np.empty((M, K), np.int8)
        s = np.empty((M, nb), np.float32)
        getattr(self.lib, f"e2_quantize_blocks_{which}")(_ptr(q), _ptr(s), _ptr(x), M, K,
                                                          -np.inf, np.inf)
        return (q.view(np.uint8) ^ 0x80).view(np.int8), s  # signed, like the HIP path

    def q8w_from_f32(self, w):
        q = Q8W()
        w = _need(np.ascontiguousarray(w, np.float32), np.float32)
        if self.lib.e2_q8w_from_f32(C.byref(q), _ptr(w), w.shape[0], w.shape[1]):
            raise MemoryError
        N, K = w.shape
        Npad, kq = q.Npad, (K + 3) // 4
        wq = np.ctypeslib.as_array(C.cast(q.w, C.POINTER(C.c_int8)), (Npad // 8 * kq * 32,)).copy()
        sc = np.ctypeslib.as_array(C.cast(q.scale, C.POINTER(C.c_float)), (Npad,)).copy()
        bsq = np.ctypeslib.as_array(C.cast(q.bsq, C.POINTER(C.c_int32)), (q.nblocks * Npad,)).copy()
        self.lib.e2_q8w_free(C.byref(q))
        return wq, sc, bsq.reshape(-1, Npad)

    def gemm(self, qa_signed, as_, wq, ws, bsq, N, K, which="avx512", n0=0, n1=None):
        """y = e2_i8_gemm_<which>(biased(qa), as, q8w{wq, ws, bsq}) over columns [n0, n1)."""
        M = qa_signed.shape[0]
        n1 = N if n1 is None else n1
        qb = (qa_signed.view(np.uint8) ^ 0x80).view(np.int8)
        qb = np.ascontiguousarray(qb)
        Npad = (N + 7) & ~7
        kq = (K + 3) // 4
        # the kernels read 16/32-wide scale and bsq vectors and 8-row weight groups; give them
        # zero-padded copies with the leading dimension Npad they index with
        wsp = np.zeros(Npad + 32, np.float32)
        wsp[:N] = ws[:N]
        nbq = bsq.shape[0]
        bs_pad = np.zeros((nbq, Npad), np.int32)
        bs_pad[:, : min(Npad, bsq.shape[1])] = bsq[:, :Npad]
        bs_flat = np.zeros(nbq * Npad + 32, np.int32)
        bs_flat[: nbq * Npad] = bs_pad.reshape(-1)
        wq_pad = np.zeros(wq.size + 4 * kq * 32, np.int8)
        wq_pad[: wq.size] = wq
        q = Q8W(wq_pad.ctypes.data, bs_flat.ctypes.data, wsp.ctypes.data, N, K,
                (K + self.block - 1) // self.block, Npad, -1e31, 1e31, 1)
        y = np.zeros((M, N), np.float32)
        getattr(self.lib, f"e2_i8_gemm_{which}")(_ptr(y), _ptr(qb), _ptr(as_), C.byref(q), M, N,
                                                 n0, n1)
        return y

    def kernels(self):
        return self.lib.e2_k().contents

    def meanpool_l2(self, x, valid):
        M, D = x.shape
        out = np.empty(D, np.float32)
        self.lib.e2_meanpool_f32(_ptr(out), _ptr(x), M, D, _ptr(valid))
        self.lib.e2_l2norm_f32(_ptr(out), D)
        return out


class RefGemmPool:
    """The reference's int8 GEMM (e2_i8_gemm_avx512, or e2_i8_gemm_vnni without AVX-512 VNNI) on the
    reference's own worker pool, columns claimed in tiles as text.c's GEMM regions claim them
    (oracle/ref_gemm_pool.c, built with E2_I8_BLOCK = K: one activation scale per row). One pool
    per block size; nthreads 0 takes the reference's thread policy (threads.c:177-261)."""

    def __init__(self, K, nthreads=0):
        path = os.path.join(HERE, "_ref", f"b{K}", "libgemmpool.so")
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        L = self.lib = C.CDLL(path)
        L.rg_init.argtypes = [_I]
        L.rg_init.restype = _I
        L.rg_close.restype = None
        L.rg_gemm.argtypes = [_I, _P, _P, _P, C.POINTER(Q8W), _I, _I]
        L.rg_gemm.restype = _I
        L.rg_pass.argtypes = [_I, _I, _P, _P, _P, _P, _P, _P]
        L.rg_pass.restype = C.c_double
        self.K = K
        self.threads = L.rg_init(nthreads)

    @staticmethod
    def available(K):
        return os.path.exists(os.path.join(HERE, "_ref", f"b{K}", "libgemmpool.so"))

    def gemm(self, kind, y, qa_biased, as_, q8w):
        M, N = y.shape
        if self.lib.rg_gemm(kind, _ptr(y), _ptr(qa_biased), _ptr(as_), C.byref(q8w), M, N):
            raise RuntimeError("rg_gemm")

    def timed(self, kind, y, qa_biased, as_, q8w):
        """Seconds of one GEMM region, timed inside the library."""
        M, N = y.shape
        ys, qs, ss = (C.c_void_p * 1)(y.ctypes.data), (C.c_void_p * 1)(qa_biased.ctypes.data), \
            (C.c_void_p * 1)(as_.ctypes.data)
        ws = (C.POINTER(Q8W) * 1)(C.pointer(q8w))
        Ms, Ns = (C.c_int * 1)(M), (C.c_int * 1)(N)
        t = self.lib.rg_pass(kind, 1, ys, qs, ss, ws, Ms, Ns)
        if t < 0:
            raise RuntimeError("rg_pass")
        return t

    def close(self):
        self.lib.rg_close()


class RefText:
    """The reference's own text tower (text.c, with the rest of the reference library) driven by
    oracle/ref_text.c on a model read from an E8CQ cache of the reference geometry. One model per
    process: the reference keeps its worker pool and cache reader global."""

    def __init__(self, cache, n_layers, vocab, nthreads=0, path=REFTEXT_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        L = self.lib = C.CDLL(path)
        L.rt_open.argtypes = [C.c_char_p, _I, _I, _I]
        L.rt_embed_batch.argtypes = [_P, _P, _I, _I, _P]
        L.rt_identity_layer.argtypes = [_I]
        L.rt_error.restype = C.c_char_p
        L.rt_cpu.restype = C.c_char_p
        L.rt_close.restype = None
        if L.rt_open(os.fsencode(cache), n_layers, vocab, nthreads):
            raise RuntimeError("rt_open: " + L.rt_error().decode())
        self.vocab = vocab
        self.dim = 768

    @staticmethod
    def available(path=REFTEXT_SO):
        return os.path.exists(path)

    @property
    def threads(self):
        return self.lib.rt_threads()

    @property
    def cpu(self):
        return self.lib.rt_cpu().decode()

    def attn_i8(self, S):
        """Whether the reference takes int8 attention for S keys on this CPU."""
        return bool(self.lib.rt_attn_i8(S))

    def identity_layer(self, l):
        if self.lib.rt_identity_layer(l):
            raise ValueError(l)

    def embed_batch(self, ids, valid=None):
        ids = _need(np.ascontiguousarray(ids, np.int32), np.int32)
        B, S = ids.shape
        v = None if valid is None else _need(np.ascontiguousarray(valid, np.uint8), np.uint8)
        out = np.zeros((B, self.dim), np.float32)
        if self.lib.rt_embed_batch(_ptr(ids), _ptr(v), B, S, _ptr(out)):
            raise RuntimeError("e2_text_embed_batch: " + self.lib.rt_error().decode())
        return out

    def close(self):
        self.lib.rt_close()


_FN = C.CFUNCTYPE
class _Kernels(C.Structure):
    """e2_kernels vtable (reference src/kernels.h:22-66)."""
    _fields_ = [
        ("name", C.c_char_p),
        ("gemm_nt", _P), ("gemv", _P),
        ("rmsnorm", _FN(None, _P, _I, _I, _P, _F)),
        ("gelu_tanh", _FN(None, _P, C.c_size_t)),
        ("softmax", _FN(None, _P, _I)),
        ("dot_f32", _P), ("axpy", _P), ("mul", _P), ("add", _P), ("scale", _P), ("mul_rows", _P),
        ("silu", _P), ("glu", _P), ("clamp", _P),
        ("norm_split", _FN(None, _P, _P, _I, _I, _P, _F)),
        ("norm_add", _FN(None, _P, _P, _P, _I, _I, _P, _F)),
        ("rope_rows", _FN(None, _P, _I, _I, _I, _I, _I, _P, _P)),
    ]
