"""ctypes wrapper of oracle/liboracle.so -- TEST INFRASTRUCTURE ONLY.

The CPU restatement of the reference algorithms (kquant_oracle.c).  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use it,
and only as the checker / reported CPU baseline, never as a product path.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE, "-B", "liboracle.so"], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        P, I, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        sig = {
            "orc_set_threads": (None, [I]),
            "orc_f16_to_f32": (F, [ctypes.c_uint16]),
            "orc_f32_to_f16": (ctypes.c_uint16, [F]),
            "orc_dequant_q4k": (None, [P, P, ctypes.c_int64]),
            "orc_dequant_q6k": (None, [P, P, ctypes.c_int64]),
            "orc_dequant_q5k": (None, [P, P, ctypes.c_int64]),
            "orc_gemv_quant_cpu": (I, [P, P, I, P, I, I]),
            "orc_gemv_quant_cpu_mt": (I, [P, P, I, P, I, I, I]),
            "orc_quantize_q8_1": (None, [P, P, I]),
            "orc_quantize_mmq": (None, [P, P, I, I, I, I]),
            "orc_mmvq": (None, [P, P, I, P, I, I]),
            "orc_mmq_subdots": (None, [P, P, I, P, I, I, I, I]),
            "orc_mmq_q4k": (None, [P, P, P, I, I, I, I]),
            "orc_mmq_q6k": (None, [P, P, P, I, I, I, I]),
            "orc_fp16_to_int8": (None, [P, P, P, I, I]),
            "orc_decode_attn_splits": (I, [I]),
            "orc_attn_decode_int8": (None, [P, P, P, P, I, I, I, I, I, F, P, P, I, I]),
            "orc_rmsnorm": (None, [P, P, P, P, I, I, F, I]),
            "orc_swiglu": (None, [P, P, P, ctypes.c_int64]),
            "orc_vec_add": (None, [P, P, P, ctypes.c_int64]),
            "orc_rope": (None, [P, P, I, I, I, I, I, I, I, F, I]),
            "orc_qk_post": (None, [P, P, P, P, P, I, F, P, P, P, P, I, I, I, I, I, I, F, I, I]),
            "orc_embed_row": (None, [P, P, I, I, I]),
            "orc_argmax": (I, [P, I]),
            "orc_attn_prefill_int8": (None, [P, P, P, P, I, I, I, I, I, I, F, P, P, I]),
            "orc_geglu": (None, [P, P, P, ctypes.c_int64]),
            "orc_vec_scale": (None, [P, ctypes.c_int64, F]),
            "orc_logit_softcap": (None, [P, ctypes.c_int64, F]),
            "orc_softmax": (None, [P, I]),
            "orc_dense": (None, [P, P, I, P, I, I, I]),
        }
        for n, (r, a) in sig.items():
            f = getattr(_lib, n)
            f.restype, f.argtypes = r, a
    return _lib


_threads = 1


def set_threads(n):
    """Thread count of the oracle's row/token-parallel loops (MMVQ, MMQ,
    prefill attention, and gemv_quant_cpu when called with threads=None).
    Results are independent of it."""
    global _threads
    _threads = max(1, int(n))
    lib().orc_set_threads(_threads)


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def _c(a, dtype):
    a = np.ascontiguousarray(a, dtype=dtype)
    return a


def f32_to_f16_bits(f):
    return lib().orc_f32_to_f16(float(f))


def f16_bits_to_f32(h):
    return lib().orc_f16_to_f32(int(h))


def dequant(W, ggml_type, rows, K):
    W = _c(W, np.uint8)
    out = np.empty((rows, K), dtype=np.float32)
    fn = {12: lib().orc_dequant_q4k, 13: lib().orc_dequant_q5k, 14: lib().orc_dequant_q6k}[ggml_type]
    fn(_p(out), _p(W), rows * (K // 256))
    return out


def gemv_quant_cpu(W, ggml_type, x, M, K, threads=1):
    W, x = _c(W, np.uint8), _c(x, np.uint16)
    if threads is None:
        threads = _threads
    y = np.empty(M, dtype=np.float32)
    if threads == 1:
        st = lib().orc_gemv_quant_cpu(_p(y), _p(W), ggml_type, _p(x), M, K)
    else:
        st = lib().orc_gemv_quant_cpu_mt(_p(y), _p(W), ggml_type, _p(x), M, K, threads)
    if st != 0:
        raise ValueError(f"unsupported ggml type {ggml_type}")
    return y


def quantize_q8_1(x, K):
    x = _c(x, np.uint16)
    y = np.zeros(K // 32 * 36, dtype=np.uint8)
    lib().orc_quantize_q8_1(_p(x), _p(y), K)
    return y


def quantize_mmq(x, N, K, Npad, ds4):
    x = _c(x, np.uint16)
    y = np.zeros((K // 128) * Npad * 144, dtype=np.uint8)
    lib().orc_quantize_mmq(_p(x), _p(y), N, K, Npad, 1 if ds4 else 0)
    return y


def mmvq(W, ggml_type, xq, M, K):
    W, xq = _c(W, np.uint8), _c(xq, np.uint8)
    y = np.empty(M, dtype=np.float32)
    lib().orc_mmvq(_p(y), _p(W), ggml_type, _p(xq), M, K)
    return y


def mmq_subdots(W, ggml_type, q8, M, N, K, Npad):
    W, q8 = _c(W, np.uint8), _c(q8, np.uint8)
    G = 32 if ggml_type == 12 else 16
    out = np.empty((N, M, K // G), dtype=np.int32)
    lib().orc_mmq_subdots(_p(out), _p(W), ggml_type, _p(q8), M, N, K, Npad)
    return out


def mmq(W, ggml_type, q8, M, N, K, Npad):
    W, q8 = _c(W, np.uint8), _c(q8, np.uint8)
    y = np.empty((N, M), dtype=np.float32)
    fn = lib().orc_mmq_q4k if ggml_type == 12 else lib().orc_mmq_q6k
    fn(_p(y), _p(W), _p(q8), M, N, K, Npad)
    return y


def fp16_to_int8(src, rows, cols):
    src = _c(src, np.uint16)
    dst = np.empty((rows, cols), dtype=np.int8)
    sc = np.empty(rows, dtype=np.float32)
    lib().orc_fp16_to_int8(_p(dst), _p(sc), _p(src), rows, cols)
    return dst, sc


def decode_attn_splits(seq):
    return lib().orc_decode_attn_splits(seq)


def attn_decode_int8(q, k, v, n_heads, n_kv, hd, chd, seq, scale, ks, vs, window, n_splits):
    q, k, v = _c(q, np.uint16), _c(k, np.int8), _c(v, np.int8)
    ks = _c(ks, np.float32) if ks is not None else None
    vs = _c(vs, np.float32) if vs is not None else None
    out = np.empty(n_heads * hd, dtype=np.uint16)
    lib().orc_attn_decode_int8(_p(out), _p(q), _p(k), _p(v), n_heads, n_kv, hd, chd, seq, float(scale),
                               _p(ks), _p(vs), window, n_splits)
    return out


# ---- decoder-layer operations (layer_oracle.c) ----

def rmsnorm(x, res, w, rows, dim, eps, w_fp32):
    x = _c(x, np.uint16)
    res = _c(res, np.uint16) if res is not None else None
    w = _c(w, np.float32 if w_fp32 else np.uint16)
    out = np.empty(rows * dim, dtype=np.uint16)
    lib().orc_rmsnorm(_p(out), _p(x), _p(res), _p(w), rows, dim, float(eps), 1 if w_fp32 else 0)
    return out


def swiglu(g, u):
    g, u = _c(g, np.uint16).ravel(), _c(u, np.uint16).ravel()
    out = np.empty(g.size, dtype=np.uint16)
    lib().orc_swiglu(_p(out), _p(g), _p(u), g.size)
    return out


def vec_add(a, b):
    a, b = _c(a, np.uint16).ravel(), _c(b, np.uint16).ravel()
    out = np.empty(a.size, dtype=np.uint16)
    lib().orc_vec_add(_p(out), _p(a), _p(b), a.size)
    return out


def rope(q, k, n_heads, n_kv, hd, start_pos, N, theta, neox, q_stride=None, k_stride=None):
    """Returns rotated copies (q, k); k may be None."""
    q = np.array(q, dtype=np.uint16, copy=True).ravel()
    k = np.array(k, dtype=np.uint16, copy=True).ravel() if k is not None else None
    lib().orc_rope(_p(q), _p(k), n_heads, n_kv if k is not None else 0, hd, start_pos, N,
                   q_stride or n_heads * hd, k_stride or n_kv * hd, float(theta), 1 if neox else 0)
    return q, k


def qk_post(q, k, v, q_norm, k_norm, norm_fp32, eps, k_cache, v_cache, k_scales, v_scales,
            n_heads, n_kv, hd, chd, start_pos, N, theta, neox, kv_int8):
    """q, k rotated in place (copies returned); caches/scales updated in place."""
    q = np.array(q, dtype=np.uint16, copy=True).ravel()
    k = np.array(k, dtype=np.uint16, copy=True).ravel()
    v = _c(v, np.uint16)
    wt = np.float32 if norm_fp32 else np.uint16
    qn = _c(q_norm, wt) if q_norm is not None else None
    kn = _c(k_norm, wt) if k_norm is not None else None
    lib().orc_qk_post(_p(q), _p(k), _p(v), _p(qn), _p(kn), 1 if norm_fp32 else 0, float(eps),
                      _p(k_cache), _p(v_cache), _p(k_scales), _p(v_scales),
                      n_heads, n_kv, hd, chd, start_pos, N, float(theta), 1 if neox else 0, 1 if kv_int8 else 0)
    return q, k


def embed_row(W, ggml_type, token, hidden):
    W = _c(W, np.uint8)
    out = np.empty(hidden, dtype=np.uint16)
    lib().orc_embed_row(_p(out), _p(W), ggml_type, int(token), hidden)
    return out


def argmax(x):
    x = _c(x, np.float32).ravel()
    return lib().orc_argmax(_p(x), x.size)


def attn_prefill_int8(q, k, v, n_heads, n_kv, hd, chd, N, start_pos, scale, ks, vs, window):
    q, k, v = _c(q, np.uint16), _c(k, np.int8), _c(v, np.int8)
    ks = _c(ks, np.float32) if ks is not None else None
    vs = _c(vs, np.float32) if vs is not None else None
    out = np.empty(N * n_heads * hd, dtype=np.uint16)
    lib().orc_attn_prefill_int8(_p(out), _p(q), _p(k), _p(v), n_heads, n_kv, hd, chd, N, start_pos, float(scale),
                                _p(ks), _p(vs), window)
    return out


# ---- kernels outside the Llama/Qwen decode path (layer_oracle.c) ----

def geglu(g, u):
    g, u = _c(g, np.uint16).ravel(), _c(u, np.uint16).ravel()
    out = np.empty(g.size, dtype=np.uint16)
    lib().orc_geglu(_p(out), _p(g), _p(u), g.size)
    return out


def vec_scale(x, s):
    x = np.array(x, dtype=np.uint16, copy=True).ravel()
    lib().orc_vec_scale(_p(x), x.size, float(s))
    return x


def logit_softcap(x, cap):
    x = np.array(x, dtype=np.float32, copy=True).ravel()
    lib().orc_logit_softcap(_p(x), x.size, float(cap))
    return x


def softmax(x):
    x = np.array(x, dtype=np.float32, copy=True).ravel()
    lib().orc_softmax(_p(x), x.size)
    return x


def dense(W, wtype, x, M, N, K):
    """W raw bytes/values [M][K] (float32 for wtype 0, uint16 bits for 1 / 30)."""
    W = _c(W, np.float32 if wtype == 0 else np.uint16)
    x = _c(x, np.uint16)
    out = np.empty(N * M, dtype=np.uint16)
    lib().orc_dense(_p(out), _p(W), wtype, _p(x), M, N, K)
    return out
