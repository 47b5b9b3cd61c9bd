"""GPU-backed drop-in for the hot-path entry points of ``tools/glm_model_q4k_ref.py``.

Same names, arguments and value conventions as the reference (bf16 values carried as
bf16-valued np.float32; fp16 headers as ints), with the arithmetic on the GPU:

========================================  ==============================  =====================
reference (tools/glm_model_q4k_ref.py)    here                            C ABI
========================================  ==============================  =====================
fp16_to_f32 :61-63                        fp16_to_f32                     aipu_dequant (F16)
bf16 :76-78 / bf16_bits :68-70            bf16 / bf16_bits                aipu_bf16_round
fp32_rsqrt :96-116                        fp32_rsqrt                      aipu_fp32_rsqrt
glm_sigmoid :293-294, glm_silu :296-299   glm_sigmoid / glm_silu          aipu_glm_sigmoid/silu
matmul_q4k :470-472                       matmul_q4k                      aipu_gemv_f32
QW :491-519                               QW (+ multi-super-block rows)    aipu_dequant / aipu_gemv
moe_router :663-681                       moe_router                      aipu_gemv + aipu_router_topk
swiglu_expert :702-708                    swiglu_expert                   aipu_swiglu_expert
decoder_block MoE half :797-809           moe_ffn                         aipu_moe_swiglu_decode
rmsnorm :451-465                          rmsnorm                         aipu_rmsnorm
decoder_block FFN half :797-810           ffn_block                       aipu_moe_layer_decode
matmul_bf16_dot :476-486                  matmul_bf16_dot                 aipu_lm_head
model_forward LM head :826-834            lm_head                         aipu_lm_head
Config :559-611                           Config (hot-path fields)        --
========================================  ==============================  =====================

``QW`` keeps the reference's constructor (one super-block per output, nin <= 256) and adds
``QW.from_ggml`` for real multi-super-block ggml rows.  Inputs shorter than a whole
super-block are zero-padded to 256: the padded activations are 0, so every padded
product is +-0 and the sequential fp32 sum is unchanged (weights are finite).
All numeric entry points default to the bit-exact reference order (``set_mode('fast')``
switches the GEMV-bearing ones to the streaming kernels).
"""
from __future__ import annotations

import numpy as np
import torch

from . import device as dev
from . import q4k_ref as _q
from ._lib import TYPE_BF16, TYPE_F16, TYPE_Q4_K

F32 = np.float32
U32 = np.uint32
U16 = np.uint16

_MODE = "ref"


def set_mode(mode):
    """'ref' (bit-exact, default) or 'fast' (streaming kernels, tolerance mode)."""
    global _MODE
    if mode not in ("ref", "fast"):
        raise ValueError("mode must be 'ref' or 'fast'")
    _MODE = mode


def _device():
    return _q._device()


# --------------------------------------------------------------- bit helpers
def f32_bits(x):
    return int(F32(x).view(U32))


def bits_f32(u):
    return F32(np.uint32(u & 0xFFFFFFFF).view(np.float32))


def fp16_to_f32(h):
    """exact IEEE half -> single (GPU F16 decoder)."""
    return F32(_q.dequantize_f16(np.array([int(h) & 0xFFFF], np.uint16))[0])


def f32_to_f16bits(x):
    return int(np.frombuffer(np.float16(x).tobytes(), dtype=U16)[0])


def bf16(x):
    """fp32 -> bf16-valued fp32 (RNE, GPU)."""
    return _q.bf16_round(x)


def bf16_bits(x):
    return (f32_bits(bf16(x)) >> 16) & 0xFFFF


def bf16_from_bits(u16):
    return bits_f32((int(u16) & 0xFFFF) << 16)


def b2f(x):
    return F32(x)


def _bits_of(vals):
    """bf16-valued floats -> uint16 patterns (exact: values are bf16 already)."""
    a = np.asarray(vals, np.float32).reshape(-1).view(np.uint32)
    return (a >> 16).astype(np.uint16)


def _vals_of(bits):
    return (np.asarray(bits, np.uint32) << 16).astype(np.uint32).view(np.float32)


def _dev_u16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.int16)).to(_device())


def _host_u16(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


# --------------------------------------------------------------- fp32 / act
def fp32_rsqrt(x):
    y = dev.fp32_rsqrt(torch.tensor([float(F32(x))], dtype=torch.float32, device=_device()))
    return F32(y.cpu().numpy()[0])


def glm_sigmoid(xbf):
    return F32(_vals_of(_host_u16(dev.glm_sigmoid(_dev_u16(_bits_of([xbf])))))[0])


def glm_silu(xbf):
    return F32(_vals_of(_host_u16(dev.glm_silu(_dev_u16(_bits_of([xbf])))))[0])


def f32_bits_key(x):
    """Order-preserving integer key for fp32 (same ordering the GPU router uses)."""
    u = f32_bits(x)
    return (u ^ 0x80000000) if (u >> 31) == 0 else (~u & 0xFFFFFFFF)


# ------------------------------------------------------------------ matmuls
def matmul_q4k(a_row, wdeq_cols):
    """out[o] = bf16(sum_k a[k]*wdeq_cols[o][k]) in sequential fp32 (GPU, bit-exact)."""
    a = np.asarray(a_row, np.float32).reshape(1, -1)
    w = np.stack([np.asarray(c, np.float32) for c in wdeq_cols])
    y = dev.gemv_f32(torch.from_numpy(w).to(_device()), torch.from_numpy(a).to(_device()))
    return list(_vals_of(_host_u16(y))[0])


# ---------------------------------------------------------------- container
def _codes_to_qs(codes256):
    """256 4-bit codes (weight order) -> 128 ggml qs bytes."""
    c = np.asarray(codes256, np.uint8).reshape(4, 2, 32)
    return (c[:, 0, :] | (c[:, 1, :] << 4)).reshape(-1)


class QW:
    """Q4_K weight matrix: ``nout`` outputs x ``nin`` reduction, as ggml row blocks on the GPU.

    ``QW(nout, nin, codes, d, dmin, scales)`` takes the reference's fields (codes[o][k],
    one fp16 d/dmin and one 12-byte scale pack per output, nin <= 256).  ``QW.from_ggml``
    wraps an existing ggml image with any number of super-blocks per row.
    """

    def __init__(self, nout, nin, codes=None, d=None, dmin=None, scales=None, _raw=None):
        self.nout = nout
        self.nin = nin
        self.kpad = (nin + 255) // 256 * 256
        self._deq = None
        if _raw is not None:
            raw = np.asarray(_raw, np.uint8).reshape(nout, self.kpad // 256 * 144)
        else:
            if nin > 256:
                raise ValueError("the reference QW holds one super-block per output (nin <= 256); use QW.from_ggml")
            raw = np.zeros((nout, 144), np.uint8)
            for o in range(nout):
                cc = np.zeros(256, np.uint8)
                cc[:nin] = np.asarray(codes[o][:nin], np.uint8) & 0xF
                raw[o] = _q.q4k_block_bytes(d[o], dmin[o], scales[o], _codes_to_qs(cc))
        self.raw = raw
        self.blocks = torch.from_numpy(raw.reshape(-1).copy()).to(_device())

    @classmethod
    def from_ggml(cls, raw, nout, nin):
        if nin % 256:
            raise ValueError("ggml Q4_K rows hold whole 256-weight super-blocks")
        return cls(nout, nin, _raw=raw)

    def dequant_col(self, o):
        row = self.blocks.view(self.nout, -1)[o]
        return dev.dequantize(TYPE_Q4_K, row).cpu().numpy()[: self.nin]

    def dequant(self):
        if self._deq is None:
            full = dev.dequantize(TYPE_Q4_K, self.blocks).cpu().numpy().reshape(self.nout, self.kpad)
            self._deq = [full[o, : self.nin].copy() for o in range(self.nout)]
        return self._deq


def _pad_x(x_bf, kpad):
    bits = np.zeros(kpad, np.uint16)
    b = _bits_of(x_bf)
    bits[: b.size] = b
    return bits


def _padded_rows(qw, rows):
    """ggml image of `qw` with the output count padded to `rows` (zero blocks: w = 0)."""
    if rows == qw.nout:
        return qw.blocks
    extra = torch.zeros((rows - qw.nout) * qw.raw.shape[1], dtype=torch.uint8, device=qw.blocks.device)
    return torch.cat([qw.blocks, extra])


# ----------------------------------------------------------------- config
class Config:
    """Hot-path subset of the reference Config (:559-611): MoE and FFN shape fields."""

    def __init__(self, **kw):
        self.MODEL_DIM = 128
        self.N_EXPERT = 8
        self.TOPK = 2
        self.INTER_MOE = 64
        self.INTER_DENSE = 256
        self.RSCALE_BITS = 0x40200000
        for k, v in kw.items():
            setattr(self, k, v)


# ---------------------------------------------------------------- operators
def moe_router(cfg, x_bf, Wg):
    """logits = x @ W_g (Q4_K) -> sigmoid -> top-K -> renorm * SCALE, on the GPU.

    Returns (sel_idx list, sel_weight bf16 list, gate_bf list) as the reference does.
    """
    xb = _dev_u16(_pad_x(x_bf, Wg.kpad))[None]
    logits = dev.gemv(TYPE_Q4_K, Wg.blocks, Wg.nout, Wg.kpad, xb, mode=_MODE)
    sel, sw, gates = dev.router_topk(logits.reshape(-1), cfg.TOPK, cfg.RSCALE_BITS, return_gates=True)
    return ([int(v) for v in sel.cpu().numpy()], list(_vals_of(_host_u16(sw))), list(_vals_of(_host_u16(gates))))


def _sum_tree(vals, topk):
    """Balanced fp32 add tree (host helper kept for interface parity; the GPU router
    computes the same tree internally)."""
    import math
    lev = 1 if topk <= 1 else int(math.ceil(math.log2(topk)))
    node = [F32(vals[i]) if i < len(vals) else F32(0.0) for i in range(1 << lev)]
    for _ in range(lev):
        node = [F32(node[2 * i] + node[2 * i + 1]) for i in range(len(node) // 2)]
    return node[0]


def swiglu_expert(cfg, x_bf, Wgate, Wup, Wdown):
    """y = (silu(x @ W_gate) * (x @ W_up)) @ W_down on the GPU; returns HIDDEN bf16 values."""
    H = Wgate.kpad
    I = (Wgate.nout + 255) // 256 * 256
    if Wdown.kpad != I:
        raise ValueError("W_down's reduction length must equal W_gate's output count")
    Hout = (Wdown.nout + 255) // 256 * 256
    if Hout != H:
        raise ValueError("W_down's output count must match W_gate's reduction length")
    y = dev.swiglu_expert(TYPE_Q4_K, _padded_rows(Wgate, I), _padded_rows(Wup, I), _padded_rows(Wdown, H), H, I,
                          _dev_u16(_pad_x(x_bf, H)), mode=_MODE)
    return list(_vals_of(_host_u16(y))[: Wdown.nout])


def moe_ffn(cfg, x_bf, Wg, Mg, Mu, Md, SHg=None, SHu=None, SHd=None):
    """The MoE half of decoder_block (:797-809): router, routed experts in slot order,
    optional shared expert (weight 1), fp32 combine, bf16 out.  Returns
    (fbuf bf16 list, sel list, sel_w list)."""
    E = len(Mg)
    H = Wg.kpad
    I = (Mg[0].nout + 255) // 256 * 256
    gate = torch.cat([_padded_rows(w, I) for w in Mg])
    up = torch.cat([_padded_rows(w, I) for w in Mu])
    down = torch.cat([_padded_rows(w, H) for w in Md])
    shared = None
    if SHg is not None:
        shared = (_padded_rows(SHg, I), _padded_rows(SHu, I), _padded_rows(SHd, H))
    y, sel, sw = dev.moe_swiglu_decode(TYPE_Q4_K, _padded_rows(Wg, Wg.nout), TYPE_Q4_K, gate, up, down, E, H, I,
                                       cfg.TOPK, _dev_u16(_pad_x(x_bf, H)), mode=_MODE, shared=shared,
                                       scale_bits=cfg.RSCALE_BITS)
    return (list(_vals_of(_host_u16(y))[: Md[0].nout]), [int(v) for v in sel.cpu().numpy()],
            list(_vals_of(_host_u16(sw))))


def rmsnorm(x_bf, gamma_bf):
    """y[i] = bf16((x[i]*inv) * gamma[i]), inv = rsqrt(mean(x^2)+eps), on the GPU; reference
    order in 'ref' mode (element-order sum of squares), tree sum in 'fast' mode."""
    x = _dev_u16(_bits_of(x_bf))
    g = _dev_u16(_bits_of(gamma_bf))
    return list(_vals_of(_host_u16(dev.rmsnorm(x, g, mode=_MODE))))


def ffn_block(cfg, h_bf, gamma_bf, Wg, Mg, Mu, Md, SHg=None, SHu=None, SHd=None):
    """The FFN half of decoder_block (:797-810) for a MoE layer: y = bf16(h + MoE(rmsnorm(h))),
    with the router, the routed experts in slot order and the optional shared expert.
    Returns (y bf16 list, sel list, sel_w list)."""
    E = len(Mg)
    H = Wg.kpad
    if len(h_bf) != H:
        raise ValueError("ffn_block needs MODEL_DIM to be a whole number of 256-weight super-blocks")
    I = (Mg[0].nout + 255) // 256 * 256
    gate = torch.cat([_padded_rows(w, I) for w in Mg])
    up = torch.cat([_padded_rows(w, I) for w in Mu])
    down = torch.cat([_padded_rows(w, H) for w in Md])
    shared = None
    if SHg is not None:
        shared = (_padded_rows(SHg, I), _padded_rows(SHu, I), _padded_rows(SHd, H))
    y, sel, sw = dev.moe_layer_decode(TYPE_Q4_K, _padded_rows(Wg, Wg.nout), TYPE_Q4_K, gate, up, down, E, H, I,
                                      cfg.TOPK, _dev_u16(_bits_of(h_bf)), _dev_u16(_bits_of(gamma_bf)), mode=_MODE,
                                      shared=shared, scale_bits=cfg.RSCALE_BITS)
    return (list(_vals_of(_host_u16(y))), [int(v) for v in sel.cpu().numpy()], list(_vals_of(_host_u16(sw))))


def _pad8(bits):
    out = np.zeros((bits.size + 7) // 8 * 8, np.uint16)
    out[: bits.size] = bits
    return out


def matmul_bf16_dot(a_bf, w_bf):
    """One LM-head output: 7 round-robin fp32 partial sums + the fixed add tree (GPU)."""
    a = _pad8(_bits_of(a_bf))
    w = _pad8(_bits_of(w_bf))
    lg, _ = dev.lm_head(_dev_u16(w).view(1, -1), _dev_u16(a), argmax=False)
    return F32(_vals_of(_host_u16(lg))[0])


def lm_head(xn_bf, Wlm):
    """The LM head of model_forward (:826-834): logits[v] = matmul_bf16_dot(xn, Wlm[v]) and the
    strict-greater bf16 argmax with lower-index ties.  Returns (logits list, logits_bits list,
    argmax int).  Rows are zero-padded to a multiple of 8 (zero products leave the sums)."""
    x = _pad8(_bits_of(xn_bf))
    W = np.stack([_pad8(_bits_of(r)) for r in Wlm])
    lg, am = dev.lm_head(_dev_u16(W).view(W.shape[0], -1), _dev_u16(x))
    bits = _host_u16(lg)
    return list(_vals_of(bits)), [int(b) for b in bits], int(am.cpu().numpy()[0])


__all__ = [
    "F32", "f32_bits", "bits_f32", "fp16_to_f32", "f32_to_f16bits", "bf16", "bf16_bits", "bf16_from_bits", "b2f",
    "fp32_rsqrt", "glm_sigmoid", "glm_silu", "f32_bits_key", "matmul_q4k", "QW", "Config", "moe_router",
    "_sum_tree", "swiglu_expert", "moe_ffn", "set_mode", "rmsnorm", "ffn_block", "matmul_bf16_dot", "lm_head",
]
