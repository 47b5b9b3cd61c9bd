"""ctypes binding of ``libaipu_q4k.so`` (the C ABI declared in ``include/aipu_q4k.h``).

The library is loaded from this package directory only.  There is no CPU fallback: if the
shared library is missing, every entry point raises ``AipuLibraryMissing``.
"""
from __future__ import annotations

import ctypes
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libaipu_q4k.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "aipu_q4k.h")

# ggml type ids and modes (mirrors include/aipu_q4k.h)
TYPE_F16 = 1
TYPE_Q8_0 = 8
TYPE_Q4_K = 12
TYPE_Q6_K = 14
TYPE_BF16 = 30
MODE_FAST = 0
MODE_REF = 1
MODE_FAST_DENSE = 2
PREFILL_CODES = 0
MAX_TILES = 64

STATUS = {
    0: "AIPU_OK",
    -1: "AIPU_ERR_ARG",
    -2: "AIPU_ERR_TYPE",
    -3: "AIPU_ERR_SHAPE",
    -4: "AIPU_ERR_ALIGN",
    -5: "AIPU_ERR_HIP",
    -6: "AIPU_ERR_WORKSPACE",
}


class AipuError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, code, message):
        super().__init__(f"{STATUS.get(code, code)}: {message}")
        self.code = code


class AipuLibraryMissing(ImportError):
    """libaipu_q4k.so has not been built (run ``python -m aipu_amd.build``)."""


class TileDesc(ctypes.Structure):
    _fields_ = [
        ("ggml_type", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("w", ctypes.c_void_p),
        ("row0", ctypes.c_int64),
        ("nrows", ctypes.c_int64),
    ]


_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_U32 = ctypes.c_uint32

# name -> (restype, argtypes)
SIGNATURES = {
    "aipu_version": (_I, []),
    "aipu_last_error": (ctypes.c_char_p, []),
    "aipu_dequant": (_I, [_I, _P, _I64, _P, _P]),
    "aipu_q4k_scale_min": (_I, [_P, _I64, _P, _P]),
    "aipu_bf16_round": (_I, [_P, _I64, _P, _P]),
    "aipu_gemv_f32": (_I, [_P, _I64, _I64, _P, _I64, _P, _P, _P]),
    "aipu_gemv": (_I, [_I, _P, _I64, _I64, _P, _I64, _P, _P, _I, _P]),
    "aipu_gemv_tiles": (_I, [ctypes.POINTER(TileDesc), _I, _I64, _I64, _P, _I64, _P, _P, _I, _P]),
    "aipu_glm_silu": (_I, [_P, _I64, _P, _P]),
    "aipu_glm_sigmoid": (_I, [_P, _I64, _P, _P]),
    "aipu_fp32_rsqrt": (_I, [_P, _I64, _P, _P]),
    "aipu_router_topk": (_I, [_P, _I64, _I, _U32, _P, _P, _P, _P]),
    "aipu_moe_workspace_bytes": (_I64, [_I64, _I64, _I64, _I]),
    "aipu_swiglu_expert": (_I, [_I, _P, _P, _P, _I64, _I64, _P, _P, _P, _I, _P, _I64, _P]),
    "aipu_moe_swiglu_decode": (_I, [_I, _P, _I, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _U32, _P, _P, _P,
                                    _P, _I, _P, _I64, _P]),
    "aipu_moe_swiglu_decode_noalloc": (_I, [_I, _P, _I, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _U32, _P, _P,
                                            _P, _P, _I, _P]),
    "aipu_moe_batched_workspace_bytes": (_I64, [_I64, _I64, _I64, _I]),
    "aipu_moe_swiglu_decode_batched": (_I, [_I, _P, _I, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _U32, _P,
                                            _I64, _P, _P, _P, _I, _P, _I64, _P]),
    "aipu_rmsnorm": (_I, [_P, _P, _I64, _P, _I, _P]),
    "aipu_moe_layer_workspace_bytes": (_I64, [_I64, _I64, _I64, _I]),
    "aipu_moe_layer_decode": (_I, [_I, _P, _I, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _U32, _P, _P, _P, _P,
                                   _P, _I, _P, _I64, _P]),
    "aipu_gemm_prefill_workspace_bytes": (_I64, [_I64, _I64]),
    "aipu_gemm_prefill": (_I, [_I, _P, _I64, _I64, _P, _I64, _P, _P, _I, _P, _I64, _P]),
    "aipu_lm_head_workspace_bytes": (_I64, [_I64]),
    "aipu_lm_head": (_I, [_P, _I64, _I64, _P, _P, _P, _P, _I64, _P]),
    "aipu_stream_read": (_I, [_P, _I64, _P, _P]),
    "aipu_wait_timeouts": (_I, [_P]),
    "aipu_measure_gemv": (_I, [_I, _P, _I64, _I64, _P, _P]),
}

_lib = None


def lib():
    """Load (once) and return the ctypes handle; raise if the library is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise AipuLibraryMissing(f"{LIB_PATH} is missing; build it with `python -m aipu_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc, what):
    if rc != 0:
        msg = lib().aipu_last_error()
        raise AipuError(rc, f"{what}: {msg.decode() if msg else ''}")


def call(name, *args):
    """Call a status-returning entry point; raise AipuError on a non-zero status."""
    rc = getattr(lib(), name)(*args)
    check(rc, name)
    return rc


def header_functions(path=HEADER_PATH):
    """Names of every function declared in include/aipu_q4k.h."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(aipu_[a-z0-9_]+)\s*\(", text)))
