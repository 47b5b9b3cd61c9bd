"""CPU oracle for the MoE SwiGLU decode step -- TEST INFRASTRUCTURE ONLY.

Imported only by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg, as the checker.  Restates the hot-path subset of the reference's
``tools/glm_model_q4k_ref.py``:

* ``fp32_rsqrt``           -- ``:96-116``  (0x5F3759DF seed + 2 Newton steps, FTZ guards)
* ``glm_sigmoid/glm_silu`` -- ``:214-299`` (clamp +-16, k = round-half-up(z*log2e),
  degree-5 Horner, exponent add with FTZ/clamp, ``1/d = rsqrt(d)^2``)
* ``moe_router`` tail      -- ``:663-699`` (top-K by (fp32 key desc, index asc), balanced
  fp32 add tree, ``rs = rsqrt(s)^2 * SCALE``, bf16 weights)
* ``swiglu_expert``        -- ``:702-708``
* MoE combine              -- ``:797-809`` (slot-ordered fp32 ``facc += g*y``, shared expert
  last with weight 1, bf16 out)
* ``rmsnorm``              -- ``:451-465`` with ``_recip_fp32`` ``:434-449`` (element-order fp32
  sum of squares, ``inv = rsqrt(sumsq*recip(n) + 1e-5)``, ``bf16((x*inv)*gamma)``)
* MoE decoder FFN half     -- ``:797-810`` (rmsnorm -> MoE step -> residual ``bf16(h + fbuf)``)
* batched MoE (M rows)     -- ``src/glm_decoder_block_q4k.v:530-560,836-906``: per-row routing;
  for M > 1 each row combines its own experts in ascending expert index (union-skip scan),
  shared expert last with weight 1; M = 1 keeps the slot order of ``:797-809``
* LM head                  -- ``:476-486`` (``matmul_bf16_dot``: 7 round-robin fp32 partial
  sums, fixed add tree) and the argmax scan of ``model_forward`` ``:826-834`` with
  ``bf16_gt`` ``:138-148``

All fp32 arithmetic is numpy float32 (one IEEE rounding per op, no fusion).  The
scalar forms restate the reference op by op; the vectorised forms (``*_vec``) are checked
equal to the scalar forms on every bf16 input, and both are checked against the committed
golden tables in ``tests/golden/`` that were produced from the reference itself.
"""
from __future__ import annotations

import math

import numpy as np

from . import q4k_oracle as qo

F32 = np.float32
U32 = np.uint32


def _b(u):
    return qo.bits_f32(u)


def _u(x):
    return qo.f32_bits(x)


def fmul(a, b):
    return F32(F32(a) * F32(b))


def fadd(a, b):
    return F32(F32(a) + F32(b))


def fneg(x):
    return _b(_u(x) ^ 0x80000000)


QNAN = 0x7FC00000
_HALF = 0x3F000000
_THREE_HALF = 0x3FC00000
_RSQRT_MAGIC = 0x5F3759DF


# ------------------------------------------------------------------ fp32_rsqrt
def fp32_rsqrt(x):
    """``tools/glm_model_q4k_ref.py:96-116``: magic seed + exactly two Newton steps.

    NaN, negative (incl. -0), zero and subnormal inputs -> quiet NaN; +inf -> +0.
    """
    x = F32(x)
    u = _u(x)
    e = (u >> 23) & 0xFF
    man = u & 0x7FFFFF
    if (e == 0xFF and man != 0) or (u >> 31) == 1 or e == 0:
        return _b(QNAN)
    if e == 0xFF:
        return F32(0.0)
    xhalf = fmul(_b(_HALF), x)
    y = _b((_RSQRT_MAGIC - (u >> 1)) & 0xFFFFFFFF)
    for _ in range(2):
        t = fadd(_b(_THREE_HALF), fneg(fmul(xhalf, fmul(y, y))))
        y = fmul(y, t)
    return y


def fp32_rsqrt_vec(x):
    """Vectorised ``fp32_rsqrt`` over a float32 array (same op order)."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    e = (u >> 23) & 0xFF
    man = u & 0x7FFFFF
    bad = ((e == 0xFF) & (man != 0)) | ((u >> 31) == 1) | (e == 0)
    pinf = (e == 0xFF) & (man == 0) & ((u >> 31) == 0)
    with np.errstate(over="ignore", invalid="ignore"):
        xhalf = np.float32(0.5) * x
        y = ((np.uint32(_RSQRT_MAGIC) - (u >> 1)).astype(np.uint32)).view(np.float32)
        for _ in range(2):
            t = np.float32(1.5) - xhalf * (y * y)
            y = y * t
    y = np.where(bad, _b(QNAN), np.where(pinf, np.float32(0.0), y)).astype(np.float32)
    return y


# ----------------------------------------------------------- sigmoid / silu
_LOG2E = 0x3FB8AA3B
_LN2 = 0x3F317218
_XSAT = 0x41800000            # 16.0
_KMAX = 64
_P5 = 0x3C088889             # 1/120
_P4 = 0x3D2AAAAB             # 1/24
_P3 = 0x3E2AAAAB             # 1/6
_P2 = 0x3F000000             # 1/2
_ONE = 0x3F800000


def _round_half_up_int(f):
    """``glm_model_q4k_ref.py:219-233``: fp32 -> int, magnitude rounded half-up, |f| <~ 23."""
    u = _u(f)
    s = (u >> 31) & 1
    e = (u >> 23) & 0xFF
    m = 0x800000 | (u & 0x7FFFFF)
    if e < 127:
        r = 1 if e == 126 else 0
    else:
        sh = 23 - (e - 127)
        r = ((m >> sh) & 0xFF) + ((m >> (sh - 1)) & 1)
    return -r if s else r


def _sanitize(x):
    """inf/NaN -> signed 16.0 (``:246-250``)."""
    u = _u(x)
    if ((u >> 23) & 0xFF) == 0xFF:
        return _b((u & 0x80000000) | _XSAT)
    return F32(x)


def _clamp16(x):
    """|x| >= 16 -> signed 16.0 (``:252-257``)."""
    u = _u(x)
    if (u & 0x7FFFFFFF) >= _XSAT:
        return _b((u & 0x80000000) | _XSAT)
    return F32(x)


def _exp_poly(r):
    """Degree-5 Horner for exp(r), |r| <= ln2/2 (``:259-266``)."""
    p = fadd(_b(_P4), fmul(r, _b(_P5)))
    p = fadd(_b(_P3), fmul(r, p))
    p = fadd(_b(_P2), fmul(r, p))
    p = fadd(_b(_ONE), fmul(r, p))
    return fadd(_b(_ONE), fmul(r, p))


def _scale_pow2(v, k):
    """2^k * v by exponent add: clamp below inf, flush to signed zero (``:268-277``)."""
    u = _u(v)
    en = ((u >> 23) & 0xFF) + k
    sg = u & 0x80000000
    if en >= 255:
        return _b(sg | (0xFE << 23) | (u & 0x7FFFFF))
    if en <= 0:
        return _b(sg)
    return _b(sg | ((en & 0xFF) << 23) | (u & 0x7FFFFF))


def sigmoid_fp32(x):
    """Unrounded fp32 sigmoid of a bf16-valued fp32 (``:279-291``)."""
    z = fneg(_clamp16(_sanitize(F32(x))))
    k = _round_half_up_int(fmul(z, _b(_LOG2E)))
    k = max(-_KMAX, min(_KMAX, k))
    r = fadd(z, fneg(fmul(F32(k), _b(_LN2))))
    d = fadd(_b(_ONE), _scale_pow2(_exp_poly(r), k))
    t = fp32_rsqrt(d)
    return fmul(t, t)


def glm_sigmoid(x):
    """bf16 sigmoid (``:293-294``); input and output are bf16-valued fp32."""
    return qo.bf16_round(sigmoid_fp32(x))


def glm_silu(x):
    """bf16 silu = bf16(sigmoid(x) * sanitize(x)) (``:296-299``)."""
    return qo.bf16_round(fmul(sigmoid_fp32(x), _sanitize(F32(x))))


def _round_half_up_int_vec(f):
    u = np.asarray(f, np.float32).view(np.uint32).astype(np.int64)
    s = (u >> 31) & 1
    e = (u >> 23) & 0xFF
    m = 0x800000 | (u & 0x7FFFFF)
    sh = np.clip(23 - (e - 127), 1, 31)
    big = ((m >> sh) & 0xFF) + ((m >> (sh - 1)) & 1)
    r = np.where(e < 127, np.where(e == 126, 1, 0), big)
    return np.where(s == 1, -r, r)


def sigmoid_fp32_vec(x):
    """Vectorised ``sigmoid_fp32`` (same ops, same order)."""
    x = np.asarray(x, np.float32)
    u = x.view(np.uint32)
    sgn = u & np.uint32(0x80000000)
    xs = np.where(((u >> 23) & 0xFF) == 0xFF, (sgn | np.uint32(_XSAT)).view(np.float32), x)
    us = xs.view(np.uint32)
    xc = np.where((us & 0x7FFFFFFF) >= _XSAT, ((us & np.uint32(0x80000000)) | np.uint32(_XSAT)).view(np.float32), xs)
    z = (xc.view(np.uint32) ^ np.uint32(0x80000000)).view(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        k = np.clip(_round_half_up_int_vec(z * _b(_LOG2E)), -_KMAX, _KMAX)
        r = z - k.astype(np.float32) * _b(_LN2)
        p = _b(_P4) + r * _b(_P5)
        p = _b(_P3) + r * p
        p = _b(_P2) + r * p
        p = _b(_ONE) + r * p
        p = (_b(_ONE) + r * p).astype(np.float32)
    pu = p.view(np.uint32).astype(np.int64)
    en = ((pu >> 23) & 0xFF) + k
    sg = pu & 0x80000000
    ex = np.where(en >= 255, sg | (0xFE << 23) | (pu & 0x7FFFFF),
                  np.where(en <= 0, sg, sg | ((en & 0xFF) << 23) | (pu & 0x7FFFFF)))
    ex = ex.astype(np.uint32).view(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        d = (_b(_ONE) + ex).astype(np.float32)
        t = fp32_rsqrt_vec(d)
        return (t * t).astype(np.float32)


def glm_sigmoid_bits_vec(x_bits):
    """bf16 bits -> bf16 bits of ``glm_sigmoid``."""
    return qo.bf16_round_bits(sigmoid_fp32_vec(qo.bf16_bits_to_f32(x_bits)))


def glm_silu_bits_vec(x_bits):
    """bf16 bits -> bf16 bits of ``glm_silu``."""
    x = qo.bf16_bits_to_f32(x_bits)
    u = x.view(np.uint32)
    xs = np.where(((u >> 23) & 0xFF) == 0xFF, ((u & np.uint32(0x80000000)) | np.uint32(_XSAT)).view(np.float32), x)
    with np.errstate(over="ignore", invalid="ignore"):
        return qo.bf16_round_bits((sigmoid_fp32_vec(x) * xs).astype(np.float32))


# ----------------------------------------------------------------- router tail
def f32_order_key(x):
    """Order-preserving integer key of an fp32 (``:684-688``)."""
    u = _u(F32(x))
    return (u ^ 0x80000000) if (u >> 31) == 0 else (~u & 0xFFFFFFFF)


def sum_tree(vals, topk):
    """Balanced fp32 add tree of ceil(log2 topk) levels, +0.0 padded (``:691-699``)."""
    lev = 1 if topk <= 1 else int(math.ceil(math.log2(topk)))
    node = [F32(vals[i]) if i < len(vals) else F32(0.0) for i in range(1 << lev)]
    for _ in range(lev):
        node = [fadd(node[2 * i], node[2 * i + 1]) for i in range(len(node) // 2)]
    return node[0]


def router_tail(logits_bits, topk, scale_bits=0x40200000):
    """bf16 logits -> (sel_idx, sel_w bf16 bits, gate bf16 bits).  ``:669-681``.

    gates = glm_sigmoid(logit); order by (fp32 key desc, expert index asc); the first
    ``topk`` win; ``s`` = add tree of the winners; ``rs = f32(f32(rsqrt(s)^2) * SCALE)``;
    ``sel_w = bf16(gate * rs)``.
    """
    logits_bits = np.asarray(logits_bits, np.uint16)
    gate_bits = glm_sigmoid_bits_vec(logits_bits)
    gates = qo.bf16_bits_to_f32(gate_bits)
    E = len(gates)
    order = sorted(range(E), key=lambda e: (f32_order_key(gates[e]), -e), reverse=True)
    sel = order[:topk]
    win = [gates[e] for e in sel]
    s = sum_tree(win, topk)
    rr = fp32_rsqrt(s)
    rs = fmul(fmul(rr, rr), _b(scale_bits))
    sel_w = [qo.bf16_round_bits(fmul(g, rs)) for g in win]
    return np.array(sel, np.int32), np.array(sel_w, np.uint16), gate_bits


# ----------------------------------------------------------------- SwiGLU / MoE
def swiglu_expert(x_bits, wg, wu, wd, ggml_type, H, I):
    """One SwiGLU expert in reference order (``:702-708``).

    ``x_bits`` bf16[H]; ``wg``/``wu`` raw ggml images [I][H/QK]; ``wd`` [H][I/QK].
    gate/up = bf16 GEMVs; ``h = bf16(f32(silu(gate)) * f32(up))``; y = bf16 GEMV(h, down).
    Returns (y_bits uint16[H], h_bits uint16[I]).
    """
    _, g = qo.gemv_quant_ref(ggml_type, wg, I, H, x_bits)
    _, u = qo.gemv_quant_ref(ggml_type, wu, I, H, x_bits)
    sg = qo.bf16_bits_to_f32(glm_silu_bits_vec(g[0]))
    h = qo.bf16_round_bits((sg * qo.bf16_bits_to_f32(u[0])).astype(np.float32))
    _, y = qo.gemv_quant_ref(ggml_type, wd, H, I, h)
    return y[0], h


def moe_combine(sel_w_bits, y_slots_bits, y_shared_bits=None):
    """Slot-ordered fp32 combine (``:799-809``): facc += f32(g*y); + shared; -> bf16."""
    facc = np.zeros(np.asarray(y_slots_bits[0]).shape, np.float32)
    for g_bits, y_bits in zip(sel_w_bits, y_slots_bits):
        g = qo.bf16_bits_to_f32(int(g_bits))
        facc = (facc + (g * qo.bf16_bits_to_f32(y_bits)).astype(np.float32)).astype(np.float32)
    if y_shared_bits is not None:
        facc = (facc + qo.bf16_bits_to_f32(y_shared_bits)).astype(np.float32)
    return qo.bf16_round_bits(facc), facc


def router_logits(router_type, router_w, E, H, x_bits):
    """Router GEMV in reference order (sequential-K fp32 MAC, bf16 logits).

    ``router_type`` is a ggml type id (bf16 weights use ``BF16_TYPE``).
    """
    if router_type == BF16_TYPE:
        rw = np.asarray(router_w)
        rw = rw.view(np.uint16) if rw.dtype == np.uint8 else rw.astype(np.uint16)
        w = qo.bf16_bits_to_f32(rw.reshape(E, H))
        _, y = qo.gemv_ref(w, qo.bf16_bits_to_f32(np.asarray(x_bits, np.uint16))[None, :])
        return y[0]
    _, y = qo.gemv_quant_ref(router_type, router_w, E, H, x_bits)
    return y[0]


#: bf16 weight "type" for the router; ggml's own id for BF16 is 30.
BF16_TYPE = 30


def router_logits_fast_order(rw_bits, E, H, x_bits, dot2="fused"):
    """bf16 router GEMV in the order of the fast-mode router kernel -- a MODEL of this
    repository's kernel (aipu_amd/csrc/route.hpp: router_wave_dot, router_logit), not of the
    reference, used to measure how often fast-mode routing departs from the reference order.

    256 threads per logit; thread t folds the 16-byte chunks c = 8t + 2048u (u = 0, 1, ...)
    in increasing K into two fp32 partials: element pairs (c, c+1) and (c+4, c+5) into s0,
    (c+2, c+3) and (c+6, c+7) into s1, one two-element dot product per pair; then s0 + s1; the
    64 lanes of a wave are summed by a butterfly (xor 32, 16, ..., 1); the four wave sums are
    added in wave order starting from +0; bf16 RNE.  ``dot2`` models the two-element dot
    product: "fused" rounds s + a0*w0 + a1*w1 once, "chain" rounds after each product.
    ``x_bits`` is bf16[H] or bf16[B, H]; returns bf16 logits [E] or [B, E].
    """
    w = qo.bf16_bits_to_f32(np.asarray(rw_bits, np.uint16).reshape(E, H)).astype(np.float64)
    xb = np.asarray(x_bits, np.uint16)
    single = xb.ndim == 1
    x = qo.bf16_bits_to_f32(np.atleast_2d(xb)).astype(np.float64)
    B = x.shape[0]
    T = 256
    s = [np.zeros((B, E, T), np.float32), np.zeros((B, E, T), np.float32)]
    t8 = 8 * np.arange(T)
    with np.errstate(over="ignore", invalid="ignore"):
        for c0 in range(0, H, 2048):
            for pair in range(4):
                idx = c0 + t8 + 2 * pair
                ok = idx < H
                i0, i1 = np.where(ok, idx, 0), np.where(ok, idx + 1, 0)
                p0 = x[:, None, i0] * w[None, :, i0]          # exact: bf16 x bf16
                p1 = x[:, None, i1] * w[None, :, i1]
                p0 = np.where(ok, p0, 0.0)
                p1 = np.where(ok, p1, 0.0)
                acc = s[pair & 1]
                if dot2 == "fused":
                    acc[...] = (acc.astype(np.float64) + (p0 + p1)).astype(np.float32)
                else:
                    acc[...] = (acc + p0.astype(np.float32)).astype(np.float32)
                    acc[...] = (acc + p1.astype(np.float32)).astype(np.float32)
        v = (s[0] + s[1]).astype(np.float32).reshape(B, E, 4, 64)
        lane = np.arange(64)
        for off in (32, 16, 8, 4, 2, 1):
            v = (v + v[..., lane ^ off]).astype(np.float32)
        tot = np.zeros((B, E), np.float32)
        for wv in range(4):
            tot = (tot + v[:, :, wv, 0]).astype(np.float32)
    out = qo.bf16_round_bits(tot)
    return out[0] if single else out


def moe_decode_ref(x_bits, router_type, router_w, experts, ggml_type, E, H, I, topk,
                   scale_bits=0x40200000, shared=None):
    """Whole MoE FFN decode step in reference order.

    ``experts`` = (gate_exps, up_exps, down_exps) flat images [E][...]; ``shared`` an
    optional (gate, up, down) triple.  Returns dict(y, sel_idx, sel_w, logits, facc).
    """
    logits = router_logits(router_type, router_w, E, H, x_bits)
    sel, sel_w, gates = router_tail(logits, topk, scale_bits)
    ge, ue, de = (np.asarray(a, np.uint8).reshape(E, -1) for a in experts)
    ys = []
    for e in sel:
        y, _ = swiglu_expert(x_bits, ge[e], ue[e], de[e], ggml_type, H, I)
        ys.append(y)
    ysh = None
    if shared is not None:
        ysh, _ = swiglu_expert(x_bits, shared[0], shared[1], shared[2], ggml_type, H, I)
    y, facc = moe_combine(sel_w, ys, ysh)
    return dict(y=y, sel_idx=sel, sel_w=sel_w, logits=logits, gates=gates, facc=facc, y_slots=ys)


# ------------------------------------------------------------------ LM head
LM_L = 7   # glm_matmul_pipe interleave (FP_MAC_LAT), tools/glm_model_q4k_ref.py:474


def bf16_dot7_rows(w_bits, x_bits):
    """``matmul_bf16_dot`` (:476-486) for every row of ``w`` at once: numpy float32 with the
    K loop sequential, vectorised across rows.  Returns (bf16 bits [V], fp32 sums [V])."""
    W = qo.bf16_bits_to_f32(np.asarray(w_bits, np.uint16))
    W = np.atleast_2d(W)
    x = qo.bf16_bits_to_f32(np.asarray(x_bits, np.uint16).reshape(-1))
    V, K = W.shape
    ps = np.zeros((LM_L, V), np.float32)
    with np.errstate(invalid="ignore", over="ignore"):      # inf - inf -> nan, as in fp32
        for k in range(K):
            ps[k % LM_L] = ps[k % LM_L] + W[:, k] * x[k]
        a01 = ps[0] + ps[1]
        a23 = ps[2] + ps[3]
        a45 = ps[4] + ps[5]
        a6 = ps[6] + F32(0.0)
        s = (a01 + a23) + (a45 + a6)
    return qo.bf16_round_bits(s), s


def bf16_gt(a, b):
    """``bf16_gt`` (:138-148): strict '>' on bf16 patterns."""
    sa, sb = (a >> 15) & 1, (b >> 15) & 1
    ma, mb = a & 0x7FFF, b & 0x7FFF
    if sa != sb:
        if ma == 0 and mb == 0:
            return False
        return sb == 1
    if sa == 0:
        return ma > mb
    return ma < mb


def lm_argmax(logit_bits):
    """The argmax scan of ``model_forward`` (:826-834): start at -inf (0xFF80) and index 0,
    replace on strict ``bf16_gt`` only (so ties keep the lower index)."""
    best, arg = 0xFF80, 0
    for v, lb in enumerate(np.asarray(logit_bits, np.uint16).tolist()):
        if bf16_gt(lb, best):
            best, arg = lb, v
    return arg


# ------------------------------------------------------------------ RMSNorm + layer
RMS_EPS_BITS = 0x3727C5AC   # 1e-5, :432


def recip_fp32_bits(n):
    """``_recip_fp32`` (:434-449): q = floor(2^60 / n) normalised to 64 bits, 23 mantissa
    bits, guard bit, sticky from the rest of q, round half to even; a mantissa carry shifts
    right and bumps the exponent."""
    q = (1 << 60) // n
    msb = q.bit_length() - 1
    expo = msb - 60 + 127
    qs = q << (63 - msb)
    mant = (qs >> 40) & 0x7FFFFF
    guard = (qs >> 39) & 1
    sticky = 1 if qs & ((1 << 39) - 1) else 0
    mant += guard & (sticky | (mant & 1))
    if mant >> 23:
        mant >>= 1
        expo += 1
    return ((expo & 0xFF) << 23) | (mant & 0x7FFFFF)


def rmsnorm(x_bits, gamma_bits):
    """``rmsnorm`` (:451-465) on bf16 patterns -> bf16 patterns.  The sum of squares is a
    sequential float32 loop; the per-element tail is vectorised (elementwise float32 ops)."""
    x = qo.bf16_bits_to_f32(np.asarray(x_bits, np.uint16).reshape(-1))
    g = qo.bf16_bits_to_f32(np.asarray(gamma_bits, np.uint16).reshape(-1))
    sq = x * x
    s = F32(0.0)
    for v in sq:
        s = F32(s + v)
    meps = fadd(fmul(s, _b(recip_fp32_bits(x.size))), _b(RMS_EPS_BITS))
    inv = fp32_rsqrt(meps)
    with np.errstate(over="ignore", invalid="ignore"):
        return qo.bf16_round_bits((x * inv) * g)


def moe_layer_ref(h_bits, gamma_bits, router_type, router_w, experts, ggml_type, E, H, I, topk,
                  scale_bits=0x40200000, shared=None):
    """FFN half of ``decoder_block`` (:797-810): nrm = rmsnorm(h), fbuf = MoE step on nrm,
    y = bf16(h + fbuf).  Returns dict(y, nrm, fbuf, sel_idx, sel_w)."""
    nrm = rmsnorm(h_bits, gamma_bits)
    r = moe_decode_ref(nrm, router_type, router_w, experts, ggml_type, E, H, I, topk, scale_bits, shared)
    hf = qo.bf16_bits_to_f32(np.asarray(h_bits, np.uint16))
    with np.errstate(over="ignore", invalid="ignore"):
        y = qo.bf16_round_bits(hf + qo.bf16_bits_to_f32(r["y"]))
    return dict(y=y, nrm=nrm, fbuf=r["y"], sel_idx=r["sel_idx"], sel_w=r["sel_w"])


def moe_decode_batched_ref(X_bits, router_type, router_w, experts, ggml_type, E, H, I, topk,
                           scale_bits=0x40200000, shared=None):
    """MoE step for M rows.  Returns dict(y [M][H], sel_idx [M][topk], sel_w [M][topk]) with
    the routing in each row's router order."""
    X = np.atleast_2d(np.asarray(X_bits, np.uint16))
    M = X.shape[0]
    ge, ue, de = (np.asarray(a, np.uint8).reshape(E, -1) for a in experts)
    ysh_cache = {}
    Y = np.zeros((M, H), np.uint16)
    S = np.zeros((M, topk), np.int32)
    W = np.zeros((M, topk), np.uint16)
    for r in range(M):
        x = X[r]
        logits = router_logits(router_type, router_w, E, H, x)
        sel, sel_w, _ = router_tail(logits, topk, scale_bits)
        S[r], W[r] = sel, sel_w
        order = list(range(topk)) if M == 1 else sorted(range(topk), key=lambda t: int(sel[t]))
        ys = [swiglu_expert(x, ge[sel[t]], ue[sel[t]], de[sel[t]], ggml_type, H, I)[0] for t in order]
        ysh = None
        if shared is not None:
            ysh, _ = swiglu_expert(x, shared[0], shared[1], shared[2], ggml_type, H, I)
        Y[r], _ = moe_combine(np.asarray(sel_w)[order], ys, ysh)
    return dict(y=Y, sel_idx=S, sel_w=W)
