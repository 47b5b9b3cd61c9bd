"""The C-ABI boundary, checked without a GPU: the library loads, exports exactly what
include/aipu_q4k.h declares, and rejects bad arguments with the documented status codes
before it touches the GPU (fake device pointers below are never dereferenced)."""
import ctypes
import os
import subprocess
import sys

import pytest

from aipu_amd import _lib
from aipu_amd._lib import TileDesc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

FAKE = ctypes.c_void_p(0x100000)       # 16-B aligned, never dereferenced
FAKE_ODD = ctypes.c_void_p(0x100001)
NULL = None
S = None

ARG, TYPE, SHAPE, ALIGN, WS = -1, -2, -3, -4, -6


def L():
    return _lib.lib()


def test_library_loads():
    assert L().aipu_version() >= 100


def test_every_declared_symbol_is_exported_and_bound():
    declared = _lib.header_functions()
    assert len(declared) >= 16
    for name in declared:
        assert hasattr(L(), name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(declared)


def test_header_constants_match_python():
    text = open(_lib.HEADER_PATH).read()
    for name, val in [("AIPU_TYPE_Q4_K", 12), ("AIPU_TYPE_Q6_K", 14), ("AIPU_TYPE_Q8_0", 8), ("AIPU_TYPE_F16", 1),
                      ("AIPU_TYPE_BF16", 30), ("AIPU_MODE_FAST", 0), ("AIPU_MODE_REF", 1), ("AIPU_MAX_TILES", 64)]:
        assert f"#define {name}" in text
        assert int(text.split(f"#define {name}")[1].split()[0]) == val
    assert ctypes.sizeof(TileDesc) == 32


def last():
    return L().aipu_last_error().decode()


def test_gemv_validation():
    f = L().aipu_gemv
    assert f(99, FAKE, 64, 256, FAKE, 1, FAKE, NULL, 0, S) == TYPE
    assert "unsupported" in last()
    assert f(12, NULL, 64, 256, FAKE, 1, FAKE, NULL, 0, S) == ARG
    assert f(12, FAKE, 64, 100, FAKE, 1, FAKE, NULL, 0, S) == SHAPE
    assert "multiple" in last()
    assert f(12, FAKE, 0, 256, FAKE, 1, FAKE, NULL, 0, S) == SHAPE
    assert f(12, FAKE, 64, 256, FAKE, 0, FAKE, NULL, 0, S) == SHAPE
    assert f(12, FAKE_ODD, 64, 256, FAKE, 1, FAKE, NULL, 0, S) == ALIGN
    assert f(12, FAKE, 64, 256, ctypes.c_void_p(0x100008), 1, FAKE, NULL, 0, S) == ALIGN  # fast mode wants 16 B
    assert f(12, FAKE, 64, 256, FAKE, 1, FAKE, NULL, 7, S) == ARG
    # AIPU_MODE_FAST_DENSE: the fast mode's checks (16-B activations); other entry points refuse it
    assert f(12, FAKE, 64, 256, ctypes.c_void_p(0x100008), 1, FAKE, NULL, 2, S) == ALIGN
    assert f(12, FAKE, 64, 100, FAKE, 1, FAKE, NULL, 2, S) == SHAPE
    assert L().aipu_swiglu_expert(12, FAKE, FAKE, FAKE, 256, 256, FAKE, FAKE, NULL, 2, FAKE, 1 << 20, S) == ARG
    assert f(8, FAKE, 64, 48, FAKE, 1, FAKE, NULL, 1, S) == SHAPE     # Q8_0: K = 48 is not a whole number of blocks


def test_dequant_and_elementwise_validation():
    assert L().aipu_dequant(12, FAKE, 100, FAKE, S) == SHAPE
    assert L().aipu_dequant(13, FAKE, 256, FAKE, S) == TYPE
    assert L().aipu_dequant(12, NULL, 256, FAKE, S) == ARG
    assert L().aipu_dequant(12, FAKE, 0, FAKE, S) == 0                # empty input is a no-op
    assert L().aipu_q4k_scale_min(FAKE, -1, FAKE, S) == SHAPE
    assert L().aipu_bf16_round(FAKE_ODD, 4, FAKE, S) == ALIGN
    assert L().aipu_glm_silu(NULL, 4, FAKE, S) == ARG
    assert L().aipu_glm_sigmoid(FAKE, -3, FAKE, S) == SHAPE
    assert L().aipu_fp32_rsqrt(FAKE, 0, FAKE, S) == 0
    assert L().aipu_gemv_f32(FAKE, 0, 4, FAKE, 1, FAKE, NULL, S) == SHAPE


def test_router_validation():
    f = L().aipu_router_topk
    assert f(FAKE, 0, 1, 0x40200000, FAKE, FAKE, NULL, S) == SHAPE
    assert f(FAKE, 16, 17, 0x40200000, FAKE, FAKE, NULL, S) == SHAPE
    assert f(FAKE, 8192, 8, 0x40200000, FAKE, FAKE, NULL, S) == SHAPE
    assert f(FAKE, 16, 0, 0x40200000, FAKE, FAKE, NULL, S) == SHAPE
    assert f(NULL, 16, 2, 0x40200000, FAKE, FAKE, NULL, S) == ARG


def test_tiles_validation():
    f = L().aipu_gemv_tiles
    t = (TileDesc * 2)(TileDesc(12, 0, 0x100000, 0, 64), TileDesc(14, 0, 0x200000, 32, 64))
    assert f(t, 2, 128, 256, FAKE, 1, FAKE, NULL, 0, S) == SHAPE      # overlap
    assert "overlap" in last()
    t = (TileDesc * 1)(TileDesc(12, 1, 0x100000, 0, 64))
    assert f(t, 1, 128, 256, FAKE, 1, FAKE, NULL, 0, S) == ARG        # reserved != 0
    t = (TileDesc * 1)(TileDesc(12, 0, 0x100000, 100, 64))
    assert f(t, 1, 128, 256, FAKE, 1, FAKE, NULL, 0, S) == SHAPE      # outside N
    assert f(t, 0, 128, 256, FAKE, 1, FAKE, NULL, 0, S) == ARG
    assert f(t, 65, 128, 256, FAKE, 1, FAKE, NULL, 0, S) == ARG


def test_moe_validation():
    assert L().aipu_moe_workspace_bytes(256, 6144, 2048, 8) > 9 * 2048 * 2
    assert L().aipu_moe_workspace_bytes(0, 6144, 2048, 8) == -1
    f = L().aipu_moe_swiglu_decode
    ws = L().aipu_moe_workspace_bytes(16, 512, 256, 4)
    args = dict(rt=30, rw=FAKE, t=12, g=FAKE, u=FAKE, d=FAKE, sg=NULL, su=NULL, sd=NULL, E=16, H=512, I=256, k=4,
                sc=0x40200000, x=FAKE, y=FAKE, si=NULL, sw=NULL, mode=1, ws=FAKE, wsb=ws)

    def call(**kw):
        a = dict(args, **kw)
        return f(a["rt"], a["rw"], a["t"], a["g"], a["u"], a["d"], a["sg"], a["su"], a["sd"], a["E"], a["H"],
                 a["I"], a["k"], a["sc"], a["x"], a["y"], a["si"], a["sw"], a["mode"], a["ws"], a["wsb"], S)

    assert call(wsb=ws - 1) == WS
    assert call(ws=NULL) == WS
    assert call(sg=FAKE) == ARG                 # partial shared expert
    assert call(k=17) == SHAPE
    assert call(I=300) == SHAPE
    assert call(rt=5) == TYPE
    assert call(g=NULL) == ARG
    # the allocation-free step checks every argument before it looks up its scratch on the GPU
    # (this container has none: any HIP call would fail with AIPU_ERR_HIP)
    f3 = L().aipu_moe_swiglu_decode_noalloc

    def call3(**kw):
        a = dict(args, **kw)
        return f3(a["rt"], a["rw"], a["t"], a["g"], a["u"], a["d"], a["sg"], a["su"], a["sd"], a["E"], a["H"],
                  a["I"], a["k"], a["sc"], a["x"], a["y"], a["si"], a["sw"], a["mode"], S)

    assert call3(g=NULL) == ARG
    assert call3(sg=FAKE) == ARG
    assert call3(rt=5) == TYPE
    assert call3(k=17) == SHAPE
    assert call3(x=ctypes.c_void_p(0x100008), mode=0) == ALIGN
    assert call3(mode=2) == ARG
    assert call3(E=256, H=6144, I=2048 * 128) == WS    # beyond the per-GPU scratch array
    f2 = L().aipu_swiglu_expert
    assert f2(12, FAKE, FAKE, FAKE, 512, 256, FAKE, FAKE, NULL, 1, FAKE, 10, S) == WS
    assert f2(12, FAKE, FAKE, FAKE, 500, 256, FAKE, FAKE, NULL, 1, FAKE, 10, S) == SHAPE


def test_prefill_validation():
    f = L().aipu_gemm_prefill
    wsb = L().aipu_gemm_prefill_workspace_bytes
    need = wsb(512, 256)
    assert need == 4 * 1 * 73728 + 512 * 4          # one 72 KB chunk per 128-row tile and super-block
    assert wsb(513, 6144) == 5 * 24 * 73728 + 640 * 4
    assert wsb(0, 256) < 0 and wsb(4, 100) < 0
    assert f(14, FAKE, 64, 256, FAKE, 512, FAKE, NULL, 0, FAKE, need, S) == TYPE
    assert f(12, FAKE, 64, 256, FAKE, 512, FAKE, NULL, 9, FAKE, need, S) == ARG
    assert f(12, FAKE, 64, 300, FAKE, 512, FAKE, NULL, 0, FAKE, need, S) == SHAPE
    assert f(12, FAKE, 64, 256, FAKE, 512, FAKE, NULL, 0, FAKE, need - 1, S) == WS
    assert f(12, FAKE, 64, 256, FAKE, 512, FAKE, NULL, 0, NULL, need, S) == WS
    assert f(12, FAKE, 64, 256, ctypes.c_void_p(0x100002), 512, FAKE, NULL, 0, FAKE, need, S) == ALIGN
    assert f(12, FAKE, 64, 256, FAKE, 512, FAKE, NULL, 0, ctypes.c_void_p(0x100010), need, S) == ALIGN


def test_python_api_rejects_host_tensors():
    import torch

    from aipu_amd import device as dev
    with pytest.raises(ValueError):
        dev.gemv(12, torch.zeros(144, dtype=torch.uint8), 1, 256, torch.zeros(1, 256, dtype=torch.bfloat16))
    with pytest.raises(TypeError):
        dev._bf16(torch.zeros(4, dtype=torch.float32))
    with pytest.raises(ValueError):
        dev._mode("fastest")


def test_error_raises_with_message():
    with pytest.raises(_lib.AipuError) as ei:
        _lib.call("aipu_gemv", 12, FAKE, 64, 100, FAKE, 1, FAKE, NULL, 0, S)
    assert ei.value.code == SHAPE and "multiple" in str(ei.value)


def test_lm_head_validation():
    f = L().aipu_lm_head
    wsb = L().aipu_lm_head_workspace_bytes
    assert wsb(154880) == 4303 * 8                  # one 8-byte (key, index) pair per 36-row workgroup
    assert wsb(65) == 16 and wsb(0) < 0
    need = wsb(1000)
    assert f(NULL, 1000, 64, FAKE, FAKE, FAKE, FAKE, need, S) == ARG
    assert f(FAKE, 1000, 64, FAKE, NULL, NULL, FAKE, need, S) == ARG
    assert f(FAKE, 1000, 60, FAKE, FAKE, FAKE, FAKE, need, S) == SHAPE
    assert f(FAKE, 0, 64, FAKE, FAKE, FAKE, FAKE, need, S) == SHAPE
    assert f(FAKE, 1000, 64, ctypes.c_void_p(0x100008), FAKE, FAKE, FAKE, need, S) == ALIGN
    assert f(FAKE, 1000, 64, FAKE, FAKE, FAKE, FAKE, need - 1, S) == WS
    assert f(FAKE, 1000, 64, FAKE, FAKE, FAKE, NULL, need, S) == WS
    assert f(FAKE, 1000, 64, FAKE, FAKE, FAKE, ctypes.c_void_p(0x100010), need, S) == ALIGN


def test_missing_library_fails_loudly():
    """Without the built HIP library every call raises AipuLibraryMissing: there is no CPU
    fallback to run instead (checked in a child process, with the loader pointed at a path
    that does not exist)."""
    code = ("import aipu_amd._lib as L, aipu_amd.device as dev, torch\n"
            "L.LIB_PATH = '/nonexistent/libaipu_q4k.so'; L._lib = None\n"
            "try:\n"
            "    L.call('aipu_last_error')\n"
            "except L.AipuLibraryMissing as e:\n"
            "    print('missing:', e)\n"
            "else:\n"
            "    raise SystemExit('no error')\n")
    r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "missing:" in r.stdout
