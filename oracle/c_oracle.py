"""ctypes binding of the plain-C oracle (oracle/q4k_oracle.c) -- test infrastructure only."""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle_q4k.so")
_lib = None


def build():
    """Compile the C oracle in place (gcc via oracle/Makefile)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle_q4k.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        L.oq_dequant.argtypes = [ctypes.c_int, P, I64, P]
        L.oq_dequant.restype = ctypes.c_int
        L.oq_gemv_ref.argtypes = [ctypes.c_int, P, I64, I64, P, I64, I64, I64, P, P, P]
        L.oq_gemv_ref.restype = ctypes.c_int
        L.oq_bf16_round.argtypes = [ctypes.c_float]
        L.oq_bf16_round.restype = ctypes.c_uint16
        L.oq_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.oq_f16_to_f32.restype = ctypes.c_float
        L.oq_rsqrt.argtypes = [ctypes.c_float]
        L.oq_rsqrt.restype = ctypes.c_float
        L.oq_bf16_round_bits.argtypes = [ctypes.c_uint32]
        L.oq_bf16_round_bits.restype = ctypes.c_uint16
        L.oq_rsqrt_bits.argtypes = [ctypes.c_uint32]
        L.oq_rsqrt_bits.restype = ctypes.c_uint32
        L.oq_f16_to_f32_bits.argtypes = [ctypes.c_uint16]
        L.oq_f16_to_f32_bits.restype = ctypes.c_uint32
        L.oq_glm_silu.argtypes = [ctypes.c_uint16]
        L.oq_glm_silu.restype = ctypes.c_uint16
        L.oq_glm_sigmoid.argtypes = [ctypes.c_uint16]
        L.oq_glm_sigmoid.restype = ctypes.c_uint16
        L.oq_bf16_dot7.argtypes = [P, P, I64, P]
        L.oq_bf16_dot7.restype = ctypes.c_uint16
        L.oq_bf16_gt.argtypes = [ctypes.c_uint16, ctypes.c_uint16]
        L.oq_bf16_gt.restype = ctypes.c_int
        L.oq_lm_head.argtypes = [P, I64, I64, P, I64, I64, P, P]
        L.oq_lm_head.restype = ctypes.c_int
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def dequant(ggml_type, raw, n_weights):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty(n_weights, np.float32)
    if lib().oq_dequant(int(ggml_type), _p(raw), int(n_weights), _p(out)) != 0:
        raise ValueError("oq_dequant rejected its arguments")
    return out


def gemv_ref(ggml_type, raw, N, K, x_bf16, n0=0, n1=None):
    """Reference-order GEMV on rows [n0, n1).  Returns (acc f32[M,N], y bf16[M,N])."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    x = np.ascontiguousarray(np.atleast_2d(x_bf16), dtype=np.uint16)
    M = x.shape[0]
    n1 = N if n1 is None else n1
    acc = np.zeros((M, N), np.float32)
    y = np.zeros((M, N), np.uint16)
    scratch = np.empty(K, np.float32)
    rc = lib().oq_gemv_ref(int(ggml_type), _p(raw), int(N), int(K), _p(x), int(M), int(n0), int(n1),
                           _p(scratch), _p(acc), _p(y))
    if rc != 0:
        raise ValueError("oq_gemv_ref rejected its arguments")
    return acc, y


def bf16_dot7(a_bits, w_bits):
    """matmul_bf16_dot of one bf16 row pair: (bf16 bits, fp32 sum before rounding)."""
    a = np.ascontiguousarray(a_bits, dtype=np.uint16)
    w = np.ascontiguousarray(w_bits, dtype=np.uint16)
    s = np.zeros(1, np.float32)
    b = lib().oq_bf16_dot7(_p(a), _p(w), int(a.size), _p(s))
    return int(b), s[0]


def lm_head(w_bits, x_bits, v0=0, v1=None):
    """LM-head logits (bf16 bits, rows [v0, v1); other rows 0) and, for the full range, argmax."""
    w = np.ascontiguousarray(w_bits, dtype=np.uint16)
    x = np.ascontiguousarray(x_bits, dtype=np.uint16).reshape(-1)
    V, K = w.shape
    v1 = V if v1 is None else v1
    logits = np.zeros(V, np.uint16)
    am = np.zeros(1, np.int32)
    if lib().oq_lm_head(_p(w), int(V), int(K), _p(x), int(v0), int(v1), _p(logits), _p(am)) != 0:
        raise ValueError("oq_lm_head rejected its arguments")
    return logits, int(am[0])


def bf16_gt(a, b):
    return bool(lib().oq_bf16_gt(int(a) & 0xFFFF, int(b) & 0xFFFF))
