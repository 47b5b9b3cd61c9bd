"""Torch-tensor API over the C ABI: device tensors in, device tensors out, no host sync.

Every function launches on ``torch.cuda.current_stream()`` of the tensors' device, so the
calls compose with torch work and can be captured in a CUDA/HIP graph.  Weights are
uint8 tensors holding ggml row blocks ``[N][K/QK][bytes]``; activations and outputs are
``torch.bfloat16`` tensors (or int16/uint16 tensors holding bf16 bit patterns).
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import (MODE_FAST, MODE_FAST_DENSE, MODE_REF, TYPE_BF16, TYPE_F16, TYPE_Q4_K, TYPE_Q6_K, TYPE_Q8_0, TileDesc, call)

QK = {TYPE_Q4_K: 256, TYPE_Q6_K: 256, TYPE_Q8_0: 32, TYPE_F16: 1, TYPE_BF16: 1}
BLOCK_BYTES = {TYPE_Q4_K: 144, TYPE_Q6_K: 210, TYPE_Q8_0: 34, TYPE_F16: 2, TYPE_BF16: 2}
RSCALE_BITS = 0x40200000   # 2.5, the routed scaling of tools/glm_model_q4k_ref.py:581


def row_bytes(ggml_type, K):
    return K // QK[ggml_type] * BLOCK_BYTES[ggml_type]


def _mode(mode):
    if mode in (MODE_FAST, "fast"):
        return MODE_FAST
    if mode in (MODE_REF, "ref"):
        return MODE_REF
    raise ValueError(f"mode must be 'fast' or 'ref', got {mode!r}")


def _gemv_mode(mode):
    """aipu_gemv also takes 'fast_dense' (dense multi-row Q4_K batches, rows within tolerance)."""
    if mode in (MODE_FAST_DENSE, "fast_dense"):
        return MODE_FAST_DENSE
    return _mode(mode)


def _stream(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _need_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("aipu_amd device API needs tensors on a GPU device")


def _bf16(t):
    if t.dtype in (torch.bfloat16, torch.int16, torch.uint16):
        return t.contiguous()
    raise TypeError(f"activations must be bfloat16 (or 16-bit bf16 patterns), got {t.dtype}")


def dequantize(ggml_type, blocks, n_weights=None):
    """Exact dequantisation of whole ggml blocks -> float32 tensor."""
    _need_cuda(blocks)
    blocks = blocks.contiguous()
    if n_weights is None:
        n_weights = blocks.numel() // BLOCK_BYTES[ggml_type] * QK[ggml_type]
    out = torch.empty(n_weights, dtype=torch.float32, device=blocks.device)
    call("aipu_dequant", ggml_type, _ptr(blocks), n_weights, _ptr(out), _stream(blocks))
    return out


def q4k_scale_min(blocks):
    """[nb, 8] int32 tensor of sc | m << 8 for every Q4_K sub-block."""
    _need_cuda(blocks)
    nb = blocks.numel() // 144
    out = torch.empty(nb * 8, dtype=torch.int16, device=blocks.device)
    call("aipu_q4k_scale_min", _ptr(blocks.contiguous()), nb, _ptr(out), _stream(blocks))
    return out.view(nb, 8)


def bf16_round(x):
    """float32 tensor -> bfloat16 tensor (RNE, inf/nan truncated as the reference does)."""
    _need_cuda(x)
    x = x.contiguous().float()
    out = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
    call("aipu_bf16_round", _ptr(x), x.numel(), _ptr(out), _stream(x))
    return out


def gemv_f32(w, x, out_f32=False):
    """Reference-order GEMV on fp32 weights w[N,K] and fp32 activations x[M,K]."""
    _need_cuda(w, x)
    w = w.contiguous().float()
    x = x.contiguous().float()
    if x.dim() == 1:
        x = x[None]
    N, K = w.shape
    M = x.shape[0]
    y = torch.empty((M, N), dtype=torch.bfloat16, device=w.device)
    yf = torch.empty((M, N), dtype=torch.float32, device=w.device) if out_f32 else None
    call("aipu_gemv_f32", _ptr(w), N, K, _ptr(x), M, _ptr(y), _ptr(yf), _stream(w))
    return (y, yf) if out_f32 else y


def gemv(ggml_type, w, N, K, x, mode="fast", out=None, out_f32=False):
    """y[M,N] = bf16(x[M,K] . dequant(w)^T).  Returns y (and the fp32 accumulators).

    mode: "fast", "ref" or "fast_dense" (Q4_K batches of 2..8 rows on the dense multi-row
    kernel, rows within the tolerance of their one-row results)."""
    _need_cuda(w, x)
    x = _bf16(x)
    if x.dim() == 1:
        x = x[None]
    M = x.shape[0]
    y = out if out is not None else torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    yf = torch.empty((M, N), dtype=torch.float32, device=x.device) if out_f32 else None
    call("aipu_gemv", ggml_type, _ptr(w), N, K, _ptr(x), M, _ptr(y), _ptr(yf), _gemv_mode(mode), _stream(x))
    return (y, yf) if out_f32 else y


def gemv_tiles(tiles, N, K, x, mode="fast", out=None, out_f32=False):
    """Mixed-type GEMV.  ``tiles`` = [(ggml_type, w_tensor, row0, nrows), ...]."""
    x = _bf16(x)
    if x.dim() == 1:
        x = x[None]
    M = x.shape[0]
    arr = (TileDesc * len(tiles))()
    for i, (t, w, r0, nr) in enumerate(tiles):
        _need_cuda(w)
        arr[i] = TileDesc(int(t), 0, w.data_ptr(), int(r0), int(nr))
    y = out if out is not None else torch.zeros((M, N), dtype=torch.bfloat16, device=x.device)
    if isinstance(out_f32, torch.Tensor):   # caller-provided fp32 output (rows outside tiles kept)
        yf = out_f32
    else:
        yf = torch.zeros((M, N), dtype=torch.float32, device=x.device) if out_f32 else None
    call("aipu_gemv_tiles", arr, len(tiles), N, K, _ptr(x), M, _ptr(y), _ptr(yf), _mode(mode), _stream(x))
    return (y, yf) if yf is not None else y


def glm_silu(x):
    x = _bf16(x)
    y = torch.empty_like(x)
    call("aipu_glm_silu", _ptr(x), x.numel(), _ptr(y), _stream(x))
    return y


def glm_sigmoid(x):
    x = _bf16(x)
    y = torch.empty_like(x)
    call("aipu_glm_sigmoid", _ptr(x), x.numel(), _ptr(y), _stream(x))
    return y


def fp32_rsqrt(x):
    _need_cuda(x)
    x = x.contiguous().float()
    y = torch.empty_like(x)
    call("aipu_fp32_rsqrt", _ptr(x), x.numel(), _ptr(y), _stream(x))
    return y


def router_topk(logits, topk, scale_bits=RSCALE_BITS, return_gates=False):
    """bf16 logits[E] -> (sel_idx int32[topk], sel_w bf16[topk][, gates bf16[E]])."""
    logits = _bf16(logits)
    E = logits.numel()
    sel = torch.empty(topk, dtype=torch.int32, device=logits.device)
    sw = torch.empty(topk, dtype=torch.bfloat16, device=logits.device)
    gates = torch.empty(E, dtype=torch.bfloat16, device=logits.device) if return_gates else None
    call("aipu_router_topk", _ptr(logits), E, topk, scale_bits, _ptr(sel), _ptr(sw), _ptr(gates), _stream(logits))
    return (sel, sw, gates) if return_gates else (sel, sw)


def moe_workspace(E, H, I, topk, device):
    """Workspace of aipu_moe_workspace_bytes() (logits, routing, h, per-slot scratch; every
    call writes what it reads, so the initial contents do not matter)."""
    n = _lib.lib().aipu_moe_workspace_bytes(E, H, I, topk)
    if n < 0:
        raise ValueError("bad MoE shape")
    return torch.zeros(n, dtype=torch.uint8, device=device)


def moe_workspace_views(ws, E, I, nslots):
    """The step's router logits (E bf16) and per-slot h (nslots x I bf16) inside a MoE
    workspace after aipu_moe_swiglu_decode / aipu_moe_layer_decode (include/aipu_q4k.h
    documents the offsets)."""
    h0 = 256 * ((E + 127) // 128) + 512
    logits = ws[:2 * E].view(torch.bfloat16)
    h = ws[h0:h0 + 2 * nslots * I].view(torch.bfloat16).view(nslots, I)
    return logits, h


def swiglu_expert(ggml_type, wg, wu, wd, H, I, x, mode="fast", workspace=None, return_h=False):
    """One SwiGLU expert (tools/glm_model_q4k_ref.py:702-708) on device tensors."""
    _need_cuda(wg, wu, wd, x)
    x = _bf16(x).reshape(-1)
    ws = workspace if workspace is not None else moe_workspace(1, H, I, 1, x.device)
    y = torch.empty(H, dtype=torch.bfloat16, device=x.device)
    h = torch.empty(I, dtype=torch.bfloat16, device=x.device) if return_h else None
    call("aipu_swiglu_expert", ggml_type, _ptr(wg), _ptr(wu), _ptr(wd), H, I, _ptr(x), _ptr(y), _ptr(h),
         _mode(mode), _ptr(ws), ws.numel(), _stream(x))
    return (y, h) if return_h else y


def moe_swiglu_decode(router_type, router_w, ggml_type, gate_exps, up_exps, down_exps, E, H, I, topk, x,
                      mode="fast", shared=None, scale_bits=RSCALE_BITS, workspace=None, out=None, sel_out=None):
    """One MoE FFN decode step.  Returns (y bf16[H], sel_idx int32[topk], sel_w bf16[topk])."""
    _need_cuda(router_w, gate_exps, up_exps, down_exps, x)
    x = _bf16(x).reshape(-1)
    ws = workspace if workspace is not None else moe_workspace(E, H, I, topk, x.device)
    y = out if out is not None else torch.empty(H, dtype=torch.bfloat16, device=x.device)
    if sel_out is None:
        sel = torch.empty(topk, dtype=torch.int32, device=x.device)
        sw = torch.empty(topk, dtype=torch.bfloat16, device=x.device)
    else:
        sel, sw = sel_out
    sg, su, sd = shared if shared is not None else (None, None, None)
    call("aipu_moe_swiglu_decode", router_type, _ptr(router_w), ggml_type, _ptr(gate_exps), _ptr(up_exps),
         _ptr(down_exps), _ptr(sg), _ptr(su), _ptr(sd), E, H, I, topk, scale_bits, _ptr(x), _ptr(y), _ptr(sel),
         _ptr(sw), _mode(mode), _ptr(ws), ws.numel(), _stream(x))
    return y, sel, sw


def moe_swiglu_decode_noalloc(router_type, router_w, ggml_type, gate_exps, up_exps, down_exps, E, H, I, topk, x,
                              mode="fast", shared=None, scale_bits=RSCALE_BITS, out=None, sel_out=None):
    """moe_swiglu_decode through aipu_moe_swiglu_decode_noalloc: no workspace, the library's
    per-GPU scratch array instead (calls that overlap on one GPU must be serialised).  With
    `out` and `sel_out` given, the call allocates nothing at all."""
    _need_cuda(router_w, gate_exps, up_exps, down_exps, x)
    x = _bf16(x).reshape(-1)
    y = out if out is not None else torch.empty(H, dtype=torch.bfloat16, device=x.device)
    if sel_out is None:
        sel = torch.empty(topk, dtype=torch.int32, device=x.device)
        sw = torch.empty(topk, dtype=torch.bfloat16, device=x.device)
    else:
        sel, sw = sel_out
    sg, su, sd = shared if shared is not None else (None, None, None)
    call("aipu_moe_swiglu_decode_noalloc", router_type, _ptr(router_w), ggml_type, _ptr(gate_exps), _ptr(up_exps),
         _ptr(down_exps), _ptr(sg), _ptr(su), _ptr(sd), E, H, I, topk, scale_bits, _ptr(x), _ptr(y), _ptr(sel),
         _ptr(sw), _mode(mode), _stream(x))
    return y, sel, sw


def moe_batched_workspace(E, H, I, topk, device):
    """Workspace for moe_swiglu_decode_batched (any initial contents)."""
    n = _lib.lib().aipu_moe_batched_workspace_bytes(E, H, I, topk)
    if n < 0:
        raise ValueError("bad MoE shape")
    return torch.zeros(n, dtype=torch.uint8, device=device)


def moe_swiglu_decode_batched(router_type, router_w, ggml_type, gate_exps, up_exps, down_exps, E, H, I, topk, x,
                              mode="fast", shared=None, scale_bits=RSCALE_BITS, workspace=None, out=None):
    """MoE decode step for x[M, H]: per-row routing, union of experts evaluated once, each row
    combining its experts in ascending index (M > 1).  Returns (y [M, H], sel [M, topk],
    sel_w [M, topk])."""
    _need_cuda(router_w, gate_exps, up_exps, down_exps, x)
    x = _bf16(x)
    if x.dim() == 1:
        x = x[None]
    M = x.shape[0]
    ws = workspace if workspace is not None else moe_batched_workspace(E, H, I, topk, x.device)
    y = out if out is not None else torch.empty((M, H), dtype=torch.bfloat16, device=x.device)
    sel = torch.empty((M, topk), dtype=torch.int32, device=x.device)
    sw = torch.empty((M, topk), dtype=torch.bfloat16, device=x.device)
    sg, su, sd = shared if shared is not None else (None, None, None)
    call("aipu_moe_swiglu_decode_batched", router_type, _ptr(router_w), ggml_type, _ptr(gate_exps), _ptr(up_exps),
         _ptr(down_exps), _ptr(sg), _ptr(su), _ptr(sd), E, H, I, topk, scale_bits, _ptr(x), M, _ptr(y), _ptr(sel),
         _ptr(sw), _mode(mode), _ptr(ws), ws.numel(), _stream(x))
    return y, sel, sw


def rmsnorm(x, gamma, mode="fast", out=None):
    """y = bf16((x * inv) * gamma), inv = fp32_rsqrt(mean(x^2) + 1e-5) (ref: element-order sum)."""
    _need_cuda(x, gamma)
    x = _bf16(x).reshape(-1)
    gamma = _bf16(gamma).reshape(-1)
    if gamma.numel() != x.numel():
        raise ValueError("gamma and x differ in length")
    y = out if out is not None else torch.empty(x.numel(), dtype=torch.bfloat16, device=x.device)
    call("aipu_rmsnorm", _ptr(x), _ptr(gamma), x.numel(), _ptr(y), _mode(mode), _stream(x))
    return y


def moe_layer_workspace(E, H, I, topk, device):
    """Zero-filled workspace for moe_layer_decode."""
    n = _lib.lib().aipu_moe_layer_workspace_bytes(E, H, I, topk)
    if n < 0:
        raise ValueError("bad MoE layer shape")
    return torch.zeros(n, dtype=torch.uint8, device=device)


def moe_layer_decode(router_type, router_w, ggml_type, gate_exps, up_exps, down_exps, E, H, I, topk, h, gamma,
                     mode="fast", shared=None, scale_bits=RSCALE_BITS, workspace=None, out=None, sel_out=None):
    """FFN half of a MoE decoder block: y = bf16(h + moe(rmsnorm(h, gamma))).
    Returns (y bf16[H], sel_idx int32[topk], sel_w bf16[topk])."""
    _need_cuda(router_w, gate_exps, up_exps, down_exps, h, gamma)
    h = _bf16(h).reshape(-1)
    gamma = _bf16(gamma).reshape(-1)
    ws = workspace if workspace is not None else moe_layer_workspace(E, H, I, topk, h.device)
    y = out if out is not None else torch.empty(H, dtype=torch.bfloat16, device=h.device)
    if sel_out is None:
        sel = torch.empty(topk, dtype=torch.int32, device=h.device)
        sw = torch.empty(topk, dtype=torch.bfloat16, device=h.device)
    else:
        sel, sw = sel_out
    sg, su, sd = shared if shared is not None else (None, None, None)
    call("aipu_moe_layer_decode", router_type, _ptr(router_w), ggml_type, _ptr(gate_exps), _ptr(up_exps),
         _ptr(down_exps), _ptr(sg), _ptr(su), _ptr(sd), E, H, I, topk, scale_bits, _ptr(h), _ptr(gamma), _ptr(y),
         _ptr(sel), _ptr(sw), _mode(mode), _ptr(ws), ws.numel(), _stream(h))
    return y, sel, sw


def prefill_workspace(M, K, device):
    """A workspace for gemm_prefill(M rows, K): reusable across calls of the same or smaller M."""
    n = _lib.lib().aipu_gemm_prefill_workspace_bytes(M, K)
    if n < 0:
        raise ValueError(f"no prefill workspace for M={M}, K={K}")
    return torch.empty(n, dtype=torch.uint8, device=device)


def gemm_prefill(ggml_type, w, N, K, x, precision=_lib.PREFILL_CODES, out=None, workspace=None, out_f32=False):
    """Prefill GEMM y[M,N] = bf16(x[M,K] . dequant(w)^T) on the matrix cores (tolerance mode).

    With out_f32=True also returns the fp32 accumulators: (y, y_f32)."""
    _need_cuda(w, x)
    x = _bf16(x)
    M = x.shape[0]
    y = out if out is not None else torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    yf = torch.empty((M, N), dtype=torch.float32, device=x.device) if out_f32 else None
    ws = workspace if workspace is not None else prefill_workspace(M, K, x.device)
    call("aipu_gemm_prefill", ggml_type, _ptr(w), N, K, _ptr(x), M, _ptr(y), _ptr(yf), precision, _ptr(ws),
         ws.numel(), _stream(x))
    return (y, yf) if out_f32 else y


def lm_head_workspace(V, device):
    """A workspace for lm_head over a V-row vocabulary (reusable for any V' <= V)."""
    n = _lib.lib().aipu_lm_head_workspace_bytes(V)
    if n < 0:
        raise ValueError(f"no lm_head workspace for V={V}")
    return torch.empty(n, dtype=torch.uint8, device=device)


def lm_head(w, x, logits=True, argmax=True, workspace=None):
    """bf16 LM head in the reference's 7-way interleaved order (bit-exact) and its argmax.

    w: [V, K] bf16 rows; x: [K] bf16.  Returns (logits [V] bf16 or None, argmax [1] int32 or
    None) as device tensors."""
    _need_cuda(w, x)
    w = _bf16(w)
    x = _bf16(x).reshape(-1)
    V, K = w.shape
    if x.numel() != K:
        raise ValueError(f"x has {x.numel()} values, W rows have {K}")
    lg = torch.empty(V, dtype=torch.bfloat16, device=x.device) if logits else None
    am = torch.empty(1, dtype=torch.int32, device=x.device) if argmax else None
    ws = None
    if argmax:
        ws = workspace if workspace is not None else lm_head_workspace(V, x.device)
    call("aipu_lm_head", _ptr(w), V, K, _ptr(x), _ptr(lg), _ptr(am), _ptr(ws), ws.numel() if ws is not None else 0,
         _stream(x))
    return lg, am


def stream_read(buf, sink):
    """Read-bandwidth probe over a uint8 device buffer (bytes multiple of 16)."""
    _need_cuda(buf, sink)
    call("aipu_stream_read", _ptr(buf), buf.numel(), _ptr(sink), _stream(buf))


def measure_gemv(what, w, N, K, x):
    """Launch floors of the M = 1 Q4_K GEMV at (N, K): what = "empty" (an empty kernel of the
    same launch shape) or "copy" (its weight-copy schedule alone)."""
    _need_cuda(w, x)
    call("aipu_measure_gemv", {"empty": 0, "copy": 1}[what], _ptr(w), N, K, _ptr(x), _stream(x))


def wait_timeouts():
    """Whether a bounded wait of a persistent kernel gave up since the last call (its launch's
    result is then wrong); synchronises the current device and clears the flag."""
    flag = ctypes.c_uint32(0)
    call("aipu_wait_timeouts", ctypes.byref(flag))
    return bool(flag.value)
