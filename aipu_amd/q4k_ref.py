"""GPU-backed drop-in for the entry points of the reference's ``tools/q4k_ref.py``.

Same names, arguments and return types as the reference (numpy in, numpy out), so a
harness written against the numpy golden runs unchanged; the arithmetic runs on the GPU
through the C ABI (``include/aipu_q4k.h``) and is bit-identical to the reference:

=============================  =================================  ==========================
reference (tools/q4k_ref.py)   here                               C ABI
=============================  =================================  ==========================
get_scale_min_k4   :27-37      get_scale_min_k4                   aipu_q4k_scale_min
dequantize_block_q4_K :39-61   dequantize_block_q4_K              aipu_dequant (Q4_K)
dequantize_row_q4_K :63-65     dequantize_row_q4_K                aipu_dequant (Q4_K)
bf16_round :76-84              bf16_round                         aipu_bf16_round
matmul_q4k_col :86-92          matmul_q4k_col                     aipu_gemv_f32
dequantize_block_q6_K :105-124 dequantize_block_q6_K              aipu_dequant (Q6_K)
dequantize_block_q8_0 :126-129 dequantize_block_q8_0              aipu_dequant (Q8_0)
_s8 / _pack_6bit_scales /      same names (host-side encoders; no arithmetic on the path)
_f32_to_f16bits
=============================  =================================  ==========================

Per call the data makes a round trip to the device; batch work belongs in
``aipu_amd.device`` (tensor API) or the batched helpers at the bottom of this module.
Errors follow the reference: bad scale packs raise (the reference asserts), bad shapes
raise ``ValueError``; a missing GPU library raises ``AipuLibraryMissing``.
"""
from __future__ import annotations

import numpy as np
import torch

from . import device as dev
from ._lib import MODE_FAST, MODE_REF, TYPE_F16, TYPE_Q4_K, TYPE_Q6_K, TYPE_Q8_0

QK_K = 256


def _device():
    if not torch.cuda.is_available():
        raise RuntimeError("aipu_amd.q4k_ref needs a GPU (no CPU fallback)")
    return torch.device("cuda", torch.cuda.current_device())


def _to_dev(a, dtype=np.uint8):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=dtype)).to(_device())


def _u8(seq, n):
    """Bytes / list of ints (raw 0..255 or signed int8) -> uint8[n]."""
    a = np.asarray(list(seq) if not isinstance(seq, (bytes, bytearray, np.ndarray)) else
                   (np.frombuffer(bytes(seq), np.uint8) if isinstance(seq, (bytes, bytearray)) else seq))
    a = (a.astype(np.int64) & 0xFF).astype(np.uint8)
    if a.size != n:
        raise ValueError(f"expected {n} bytes, got {a.size}")
    return a


# ------------------------------------------------------------- host encoders
def _s8(b):
    """Raw byte (0..255) -> signed int8 value; idempotent on signed input."""
    return b - 256 if b > 127 else b


def _pack_6bit_scales(scs, mns):
    """8 six-bit scales + 8 six-bit mins -> 12 packed bytes (inverse of get_scale_min_k4)."""
    assert len(scs) == 8 and len(mns) == 8 and all(0 <= v < 64 for v in list(scs) + list(mns))
    q = [0] * 12
    for j in range(4):
        q[j] = int(scs[j])
        q[j + 4] = int(mns[j])
    for j in range(4, 8):
        q[j + 4] = (int(scs[j]) & 0xF) | ((int(mns[j]) & 0xF) << 4)
        q[j - 4] |= ((int(scs[j]) >> 4) & 0x3) << 6
        q[j] |= ((int(mns[j]) >> 4) & 0x3) << 6
    return q


def _f32_to_f16bits(x):
    return int(np.frombuffer(np.float16(x).tobytes(), dtype=np.uint16)[0])


# ------------------------------------------------------------ block builders
def q4k_block_bytes(d_h, dmin_h, scales, qs):
    """One 144-byte ggml Q4_K block from its fields."""
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([int(d_h) & 0xFFFF], np.uint16).view(np.uint8)
    b[2:4] = np.array([int(dmin_h) & 0xFFFF], np.uint16).view(np.uint8)
    b[4:16] = _u8(scales, 12)
    b[16:144] = _u8(qs, 128)
    return b


def q6k_block_bytes(d_h, ql, qh, sc):
    """One 210-byte ggml Q6_K block (ql | qh | int8 sc | fp16 d)."""
    b = np.zeros(210, np.uint8)
    b[0:128] = _u8(ql, 128)
    b[128:192] = _u8(qh, 64)
    b[192:208] = _u8(sc, 16)
    b[208:210] = np.array([int(d_h) & 0xFFFF], np.uint16).view(np.uint8)
    return b


def q8_0_block_bytes(d_h, qs):
    """One 34-byte ggml Q8_0 block (fp16 d | int8 qs[32])."""
    b = np.zeros(34, np.uint8)
    b[0:2] = np.array([int(d_h) & 0xFFFF], np.uint16).view(np.uint8)
    b[2:34] = _u8(qs, 32)
    return b


# --------------------------------------------------------------- entry points
def get_scale_min_k4(j, scales):
    """Unpack the j-th 6-bit (scale, min) pair of a Q4_K super-block on the GPU."""
    if not 0 <= int(j) < 8:
        raise IndexError("sub-block index must be 0..7")
    blk = q4k_block_bytes(0, 0, scales, np.zeros(128, np.uint8))
    sm = dev.q4k_scale_min(_to_dev(blk)).cpu().numpy().view(np.uint16)[0]
    v = int(sm[int(j)])
    return v & 0xFF, v >> 8


def dequantize_blocks(ggml_type, raw):
    """Batched exact dequant: flat ggml image (bytes / uint8 array) -> float32 array."""
    t = _to_dev(np.frombuffer(bytes(raw), np.uint8) if isinstance(raw, (bytes, bytearray)) else raw)
    return dev.dequantize(int(ggml_type), t).cpu().numpy()


def dequantize_block_q4_K(d_h, dmin_h, scales, qs):
    """ONE Q4_K super-block -> 256 fp32 values, bit-exact (GPU)."""
    return dequantize_blocks(TYPE_Q4_K, q4k_block_bytes(d_h, dmin_h, scales, qs))


def dequantize_row_q4_K(blocks):
    """blocks: iterable of (d_h, dmin_h, scales, qs) -> concatenated fp32 row (one GPU call)."""
    img = np.concatenate([q4k_block_bytes(*b) for b in blocks])
    return dequantize_blocks(TYPE_Q4_K, img)


def dequantize_block_q6_K(d_h, ql, qh, sc):
    """ONE Q6_K super-block -> 256 fp32 values, bit-exact (GPU)."""
    return dequantize_blocks(TYPE_Q6_K, q6k_block_bytes(d_h, ql, qh, sc))


def dequantize_block_q8_0(d_h, qs):
    """ONE Q8_0 block -> 32 fp32 values, bit-exact (GPU)."""
    return dequantize_blocks(TYPE_Q8_0, q8_0_block_bytes(d_h, qs))


def dequantize_f16(raw16):
    """fp16 bit patterns -> fp32 (GPU passthrough decoder)."""
    h = np.ascontiguousarray(raw16, dtype=np.uint16)
    return dequantize_blocks(TYPE_F16, h.view(np.uint8))


def bf16_round(x):
    """fp32 -> bf16 value kept in fp32 (RNE; inf/nan truncated), on the GPU."""
    a = np.asarray(x, dtype=np.float32)
    out = dev.bf16_round(torch.from_numpy(np.ascontiguousarray(a.reshape(-1))).to(_device()))
    r = out.view(torch.int16).cpu().numpy().view(np.uint16).astype(np.uint32) << 16
    r = r.view(np.float32)
    return np.float32(r[0]) if a.ndim == 0 else r.reshape(a.shape)


def matmul_q4k_col(a_row_f32, wdeq_col_f32):
    """One output: sequential fp32 dot in K order, rounded to bf16 (GPU, bit-exact)."""
    a = np.asarray(a_row_f32, dtype=np.float32).reshape(1, -1)
    w = np.asarray(wdeq_col_f32, dtype=np.float32).reshape(1, -1)
    if a.shape[1] != w.shape[1]:
        raise ValueError("activation and weight lengths differ")
    y = dev.gemv_f32(torch.from_numpy(w).to(_device()), torch.from_numpy(a).to(_device()))
    return np.float32(bf16_bits_to_f32(y.view(torch.int16).cpu().numpy().view(np.uint16))[0, 0])


# ------------------------------------------------------------ batched helpers
def bf16_bits_to_f32(b):
    return (np.asarray(b, np.uint32) << 16).astype(np.uint32).view(np.float32)


def gemv(ggml_type, raw, N, K, x_bf16_bits, mode="ref"):
    """Batched GEMV on a ggml image: returns (acc float32[M,N], y bf16 bits uint16[M,N])."""
    w = _to_dev(np.frombuffer(bytes(raw), np.uint8) if isinstance(raw, (bytes, bytearray)) else raw)
    x = torch.from_numpy(np.ascontiguousarray(np.atleast_2d(x_bf16_bits), np.uint16).view(np.int16)).to(_device())
    y, yf = dev.gemv(int(ggml_type), w, N, K, x, mode=mode, out_f32=True)
    return yf.cpu().numpy(), y.view(torch.int16).cpu().numpy().view(np.uint16)


__all__ = [
    "QK_K", "get_scale_min_k4", "dequantize_block_q4_K", "dequantize_row_q4_K", "bf16_round",
    "matmul_q4k_col", "_s8", "dequantize_block_q6_K", "dequantize_block_q8_0", "_pack_6bit_scales",
    "_f32_to_f16bits", "dequantize_blocks", "dequantize_f16", "gemv", "MODE_FAST", "MODE_REF",
]
