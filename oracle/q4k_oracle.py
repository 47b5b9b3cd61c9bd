"""CPU oracle for the Q4_K GEMM core -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import this module, and only as the checker (or, in the bench, as the timed CPU baseline).
The product path (``aipu_amd``) never imports it and has no CPU fallback.

It restates, in numpy, the numeric contract of the reference's Python goldens:

* ``tools/q4k_ref.py``           -- ggml Q4_K / Q6_K / Q8_0 dequant, bf16 RNE, sequential fp32 MAC
* ``tools/q4k_matmul_gen.py``    -- multi-super-block column dequant (K > 256)
* ``tools/gguf_crosscheck.py``   -- ggml block byte layouts (Q4_K 144 B, Q6_K 210 B, Q8_0 34 B)

Every function exists in two forms where it matters:

* a *faithful scalar* form: the same per-element np.float32 loop as the reference
  (used to pin the vectorised form on small inputs and as the CPU timing proxy);
* a *vectorised* form: numpy float32 elementwise ufuncs.  numpy never fuses a multiply
  and an add, and every float32 ufunc is a correctly rounded IEEE-754 binary32 op, so the
  vectorised form is bit-identical to the scalar loop.  The reference-order GEMV keeps
  the K loop sequential and vectorises across output rows only.

How each function is pinned (checked in tests/test_oracle.py):

=======================  =========================================================
fp16 -> fp32             KATs ``test/q4k_prim_tb.v:37-46``; exhaustive 65,536 halves
scale_min_k4 / unpack    KATs ``test/q4k_prim_tb.v:33,49-56``; pack<->unpack bijection
dequant_q4k              brute force (all sc x q x d-sample), position map
                         ``tools/q4k_ref.py:168-178``; scalar == vectorised
dequant_q6k / q8_0 / f16 closed forms, exhaustive int8, edge blocks
                         (``tools/q4k_mixed_gen.py:459-525``); scalar == vectorised;
                         s8 corners ``src/q4k.vh:114-116``
bf16_round               closed-form RNE cases (ties, carry into exponent, overflow,
                         inf/nan truncation)
gemv_ref                 scalar loop == vectorised; K=1 is one rounded product;
                         zero weights -> 0; order-sensitivity probe
=======================  =========================================================
"""
from __future__ import annotations

import numpy as np

QK_K = 256

# ggml type ids (tools/ckpt_pack_q4k.py:58-68 lists F16=1, Q8_0=8, Q4_K=12, Q6_K=14)
GGML_F16 = 1
GGML_Q8_0 = 8
GGML_Q4_K = 12
GGML_Q6_K = 14

#: bytes per block and weights per block for each type (tools/gguf_crosscheck.py:30-31)
BLOCK_BYTES = {GGML_Q4_K: 144, GGML_Q6_K: 210, GGML_Q8_0: 34, GGML_F16: 2}
BLOCK_WEIGHTS = {GGML_Q4_K: 256, GGML_Q6_K: 256, GGML_Q8_0: 32, GGML_F16: 1}

F32 = np.float32


# ----------------------------------------------------------------------------- bits
def f16_bits_to_f32(h):
    """Exact IEEE half -> single on fp16 bit patterns (numpy == ggml GGML_FP16_TO_FP32).

    Follows ``tools/q4k_ref.py:45-46`` (frombuffer as float16, widen to float32).
    Accepts a Python int or an integer array; returns np.float32 / float32 array.
    """
    a = np.asarray(h, dtype=np.uint32).astype(np.uint16)
    out = a.view(np.float16).astype(np.float32)
    return out if out.ndim else F32(out)


def f32_bits(x):
    """float32 value(s) -> uint32 bit pattern(s)."""
    a = np.asarray(x, dtype=np.float32)
    out = a.view(np.uint32)
    return int(out) if out.ndim == 0 else out


def bits_f32(u):
    """uint32 bit pattern(s) -> float32 value(s)."""
    a = np.asarray(u, dtype=np.uint64).astype(np.uint32)
    out = a.view(np.float32)
    return F32(out) if out.ndim == 0 else out


def f32_to_f16_bits(x):
    """float -> fp16 bit pattern (numpy RNE), as ``tools/q4k_ref.py:147-148``."""
    a = np.asarray(x, dtype=np.float64).astype(np.float16).view(np.uint16)
    return int(a) if a.ndim == 0 else a


# ----------------------------------------------------------------------- bf16 RNE
def bf16_round_bits(x):
    """fp32 -> bf16 bit pattern (uint16), round-to-nearest-even on the low 16 bits.

    Restates ``tools/q4k_ref.py:76-84``: finite values round with
    ``(u + 0x7FFF + lsb) & 0xFFFF0000``; inf and NaN keep their sign/exponent and are
    *truncated* (so a NaN whose payload lives only in the low 16 bits becomes inf --
    the reference's quirk, reproduced on purpose).
    """
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    special = (u & 0x7F800000) == 0x7F800000
    lsb = (u >> 16) & 1
    rounded = (u + 0x7FFF + lsb) & 0xFFFF0000
    r = np.where(special, u & 0xFFFF0000, rounded) >> 16
    r = r.astype(np.uint16)
    return int(r) if r.ndim == 0 else r


def bf16_bits_to_f32(b):
    """bf16 bit pattern(s) -> bf16-valued float32 (lossless widen)."""
    a = (np.asarray(b, dtype=np.uint32) & 0xFFFF) << 16
    out = a.astype(np.uint32).view(np.float32)
    return F32(out) if out.ndim == 0 else out


def bf16_round(x):
    """fp32 -> bf16-valued fp32 (``tools/q4k_ref.py:76`` returns the value, not bits)."""
    return bf16_bits_to_f32(bf16_round_bits(x))


def bf16_round_scalar(x):
    """Faithful scalar restatement of ``tools/q4k_ref.py:76-84`` (pins the vector form)."""
    u = int(np.frombuffer(np.float32(x).tobytes(), dtype=np.uint32)[0])
    if (u & 0x7F800000) == 0x7F800000:
        u2 = u & 0xFFFF0000
    else:
        u2 = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return np.float32(np.frombuffer(np.uint32(u2).tobytes(), dtype=np.float32)[0])


# ------------------------------------------------------------ Q4_K 6-bit scales
def scale_min_k4(j, scales):
    """Unpack the j-th (0..7) 6-bit block scale and min from 12 packed bytes.

    Restates ggml ``get_scale_min_k4`` as given in ``tools/q4k_ref.py:27-37``:
    j < 4 reads the low 6 bits of ``scales[j]`` / ``scales[j+4]``; j >= 4 joins the nibble
    of ``scales[j+4]`` with the top two bits of ``scales[j-4]`` (scale) or ``scales[j]`` (min).
    """
    q = [int(v) & 0xFF for v in scales]
    if j < 4:
        return q[j] & 63, q[j + 4] & 63
    sc = (q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4)
    mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4)
    return sc, mn


def unpack_scales_q4k(scales12):
    """Vectorised ``scale_min_k4`` over blocks: uint8[nb,12] -> (sc uint8[nb,8], m uint8[nb,8])."""
    s = np.asarray(scales12, dtype=np.uint8).reshape(-1, 12).astype(np.uint16)
    sc = np.empty((s.shape[0], 8), np.uint16)
    mn = np.empty((s.shape[0], 8), np.uint16)
    sc[:, 0:4] = s[:, 0:4] & 63
    mn[:, 0:4] = s[:, 4:8] & 63
    sc[:, 4:8] = (s[:, 8:12] & 0x0F) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:8] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc.astype(np.uint8), mn.astype(np.uint8)


def pack_scales_q4k(scs, mns):
    """Inverse of ``scale_min_k4``: 8 scales + 8 mins (each 0..63) -> 12 bytes.

    Encoder side used to build synthetic blocks; restates ``tools/q4k_ref.py:132-145``.
    Raises ValueError on out-of-range inputs (the reference asserts).
    """
    scs = [int(v) for v in scs]
    mns = [int(v) for v in mns]
    if len(scs) != 8 or len(mns) != 8 or not all(0 <= v < 64 for v in scs + mns):
        raise ValueError("pack_scales_q4k needs 8 scales and 8 mins in 0..63")
    q = [0] * 12
    for j in range(4):
        q[j] = scs[j]
        q[j + 4] = mns[j]
    for j in range(4, 8):
        q[j + 4] = (scs[j] & 0x0F) | ((mns[j] & 0x0F) << 4)
        q[j - 4] |= ((scs[j] >> 4) & 3) << 6
        q[j] |= ((mns[j] >> 4) & 3) << 6
    return q


# ------------------------------------------------------------------ Q4_K dequant
def q4k_block_fields(raw):
    """Split Q4_K blocks uint8[nb,144] into (d_h, dmin_h, scales[nb,12], qs[nb,128]).

    Byte layout: fp16 d | fp16 dmin | u8 scales[12] | u8 qs[128]
    (``tools/q4k_ref.py:12-16``, offsets ``tools/gguf_crosscheck.py:39-42``).
    """
    r = np.asarray(raw, dtype=np.uint8).reshape(-1, 144)
    d_h = r[:, 0:2].copy().view(np.uint16)[:, 0]
    dm_h = r[:, 2:4].copy().view(np.uint16)[:, 0]
    return d_h, dm_h, r[:, 4:16], r[:, 16:144]


def q4k_codes(qs):
    """qs uint8[nb,128] -> 4-bit codes uint8[nb,256] in weight order.

    For 64-group g the first 32 weights are the low nibbles of ``qs[32g:32g+32]`` and the
    next 32 the high nibbles (``tools/q4k_ref.py:51-60``).
    """
    q = np.asarray(qs, dtype=np.uint8).reshape(-1, 4, 32)
    return np.stack([q & 0x0F, q >> 4], axis=2).reshape(-1, 256)


_SUB_OF_POS = np.arange(QK_K) // 32


def dequant_q4k(raw):
    """Vectorised Q4_K dequant: uint8[nb*144] -> float32[nb*256], bit-exact.

    Per weight ``w = f32(f32(d*sc)*q) - f32(dmin*m)`` with sub-block ``k//32``
    (``tools/q4k_ref.py:45-60``, multi-block form ``tools/q4k_matmul_gen.py:28-40``).
    """
    d_h, dm_h, scales, qs = q4k_block_fields(raw)
    d = f16_bits_to_f32(d_h)
    dm = f16_bits_to_f32(dm_h)
    sc, mn = unpack_scales_q4k(scales)
    with np.errstate(over="ignore", invalid="ignore"):
        D = d[:, None] * sc.astype(np.float32)          # f32(d*sc)   [nb,8]
        M = dm[:, None] * mn.astype(np.float32)         # f32(dmin*m) [nb,8]
        w = D[:, _SUB_OF_POS] * q4k_codes(qs).astype(np.float32) - M[:, _SUB_OF_POS]
    return w.reshape(-1)


def dequant_block_q4k_scalar(d_h, dmin_h, scales, qs):
    """Faithful scalar restatement of ``dequantize_block_q4_K`` (``tools/q4k_ref.py:39-61``)."""
    d = f16_bits_to_f32(int(d_h))
    mn = f16_bits_to_f32(int(dmin_h))
    qs = [int(v) for v in qs]
    y = np.empty(QK_K, dtype=np.float32)
    yi = 0
    for g in range(4):
        sc0, m0 = scale_min_k4(2 * g, scales)
        sc1, m1 = scale_min_k4(2 * g + 1, scales)
        d1 = d * np.float32(sc0)
        mm1 = mn * np.float32(m0)
        d2 = d * np.float32(sc1)
        mm2 = mn * np.float32(m1)
        for l in range(32):
            y[yi] = d1 * np.float32(qs[32 * g + l] & 0xF) - mm1
            yi += 1
        for l in range(32):
            y[yi] = d2 * np.float32(qs[32 * g + l] >> 4) - mm2
            yi += 1
    return y


# ------------------------------------------------------------------ Q6_K dequant
def q6k_block_fields(raw):
    """Split Q6_K blocks uint8[nb,210] into (ql[nb,128], qh[nb,64], sc int8[nb,16], d_h[nb]).

    Byte layout ql | qh | int8 sc[16] | fp16 d (``tools/gguf_crosscheck.py:51-54``).
    """
    r = np.asarray(raw, dtype=np.uint8).reshape(-1, 210)
    return r[:, 0:128], r[:, 128:192], r[:, 192:208].view(np.int8), r[:, 208:210].copy().view(np.uint16)[:, 0]


def q6k_codes(ql, qh):
    """Raw ql/qh -> 6-bit codes uint8[nb,256] (0..63) in ggml y-position order.

    Position ``128h + 32t + l`` takes the low (t<2) or high (t>=2) nibble of
    ``ql[64h + l + 32*(t&1)]`` and bits ``2t..2t+1`` of ``qh[32h + l]``
    (``tools/q4k_ref.py:112-123``; per-position form ``tools/q4k_mixed_gen.py:70-82``).
    """
    ql = np.asarray(ql, dtype=np.uint8).reshape(-1, 2, 2, 32)      # [nb, h, t&1, l]
    qh = np.asarray(qh, dtype=np.uint8).reshape(-1, 2, 32)         # [nb, h, l]
    out = np.empty((ql.shape[0], 2, 4, 32), np.uint8)
    for t in range(4):
        nib = (ql[:, :, t & 1, :] & 0x0F) if t < 2 else (ql[:, :, t & 1, :] >> 4)
        out[:, :, t, :] = nib | (((qh >> (2 * t)) & 3) << 4)
    return out.reshape(-1, 256)


def dequant_q6k(raw):
    """Vectorised Q6_K dequant, bit-exact: ``w = f32(f32(d*sc[p>>4]) * (code-32))``.

    (``tools/q4k_ref.py:105-124``; scale index p>>4 per ``tools/q4k_mixed_gen.py:16-20``.)
    """
    ql, qh, sc, d_h = q6k_block_fields(raw)
    d = f16_bits_to_f32(d_h)
    q = q6k_codes(ql, qh).astype(np.float32) - np.float32(32)     # exact small ints
    with np.errstate(over="ignore", invalid="ignore"):
        ds = d[:, None] * sc.astype(np.float32)                      # [nb,16]
        w = ds[:, np.arange(QK_K) >> 4] * q
    return w.reshape(-1)


def s8(b):
    """Raw byte or signed int -> int8 value (idempotent), as ``tools/q4k_ref.py:99-103``."""
    b = int(b)
    return b - 256 if b > 127 else b


def dequant_block_q6k_scalar(d_h, ql, qh, sc):
    """Faithful scalar restatement of ``dequantize_block_q6_K`` (``tools/q4k_ref.py:105-124``)."""
    d = f16_bits_to_f32(int(d_h))
    ql = [int(v) & 0xFF for v in ql]
    qh = [int(v) & 0xFF for v in qh]
    sc = [s8(v) for v in sc]
    y = np.empty(QK_K, dtype=np.float32)
    for h in range(2):
        bq, bh, bs, by = 64 * h, 32 * h, 8 * h, 128 * h
        for l in range(32):
            i = l // 16
            c = [
                ((ql[bq + l] & 0xF) | (((qh[bh + l] >> 0) & 3) << 4)) - 32,
                ((ql[bq + l + 32] & 0xF) | (((qh[bh + l] >> 2) & 3) << 4)) - 32,
                ((ql[bq + l] >> 4) | (((qh[bh + l] >> 4) & 3) << 4)) - 32,
                ((ql[bq + l + 32] >> 4) | (((qh[bh + l] >> 6) & 3) << 4)) - 32,
            ]
            for t in range(4):
                y[by + l + 32 * t] = d * np.float32(sc[bs + i + 2 * t]) * np.float32(c[t])
    return y


# ------------------------------------------------------------------ Q8_0 / F16
def dequant_q8_0(raw):
    """Vectorised Q8_0 dequant: 34-B blocks (fp16 d, int8 qs[32]) -> ``f32(d * qs)``.

    (``tools/q4k_ref.py:126-129``; layout ``tools/gguf_crosscheck.py:63-64``.)
    """
    r = np.asarray(raw, dtype=np.uint8).reshape(-1, 34)
    d = f16_bits_to_f32(r[:, 0:2].copy().view(np.uint16)[:, 0])
    q = r[:, 2:34].view(np.int8).astype(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        w = d[:, None] * q
    return w.reshape(-1)


def dequant_block_q8_0_scalar(d_h, qs):
    """Faithful scalar restatement of ``dequantize_block_q8_0`` (``tools/q4k_ref.py:126-129``)."""
    d = f16_bits_to_f32(int(d_h))
    return np.array([d * np.float32(s8(q)) for q in qs], dtype=np.float32)


def dequant_f16(raw):
    """F16 passthrough: raw fp16 bytes -> float32 (exact)."""
    h = np.asarray(raw, dtype=np.uint8).reshape(-1).view(np.uint16)
    return f16_bits_to_f32(h)


_DEQUANT = {GGML_Q4_K: dequant_q4k, GGML_Q6_K: dequant_q6k, GGML_Q8_0: dequant_q8_0, GGML_F16: dequant_f16}


def dequant(ggml_type, raw):
    """Dispatch on the ggml type id; raw is the flat byte image of whole blocks."""
    return _DEQUANT[int(ggml_type)](raw)


def row_bytes(ggml_type, K):
    """Bytes of one ggml row of K weights."""
    return K // BLOCK_WEIGHTS[ggml_type] * BLOCK_BYTES[ggml_type]


def dequant_matrix(ggml_type, raw, N, K):
    """Rows of ggml blocks [N][K/QK][B] -> float32[N,K] (row n = output n)."""
    return dequant(ggml_type, np.asarray(raw, np.uint8).reshape(-1)[: N * row_bytes(ggml_type, K)]).reshape(N, K)


# ------------------------------------------------------------- reference GEMV
def dot_ref_scalar(a_row_f32, wdeq_col_f32):
    """Faithful scalar ``matmul_q4k_col`` (``tools/q4k_ref.py:86-92``): fp32 sequential MAC, bf16 out.

    Returns (acc_f32, bf16_value_f32).
    """
    acc = np.float32(0.0)
    for k in range(len(a_row_f32)):
        acc = np.float32(acc + np.float32(a_row_f32[k]) * np.float32(wdeq_col_f32[k]))
    return acc, bf16_round_scalar(acc)


def gemv_ref(wdeq, x):
    """Reference-order GEMV, vectorised over outputs.

    ``wdeq`` float32[N,K] (row n = output n), ``x`` float32[M,K] holding bf16 values.
    For every (m, n): ``acc = f32(acc + f32(x[m,k] * w[n,k]))`` for k = 0..K-1 in order
    (``tools/q4k_ref.py:86-92``; the RTL's streaming order ``src/glm_matmul_q4k.v:261-270``).
    Returns (acc float32[M,N], y_bf16 uint16[M,N]).
    """
    w = np.asarray(wdeq, dtype=np.float32)
    x = np.atleast_2d(np.asarray(x, dtype=np.float32))
    N, K = w.shape
    M = x.shape[0]
    wt = np.ascontiguousarray(w.T)                     # [K,N]
    acc = np.zeros((M, N), dtype=np.float32)
    prod = np.empty((M, N), dtype=np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        for k in range(K):
            np.multiply(x[:, k:k + 1], wt[k][None, :], out=prod)
            np.add(acc, prod, out=acc)
    return acc, bf16_round_bits(acc)


def gemv_quant_ref(ggml_type, raw, N, K, x_bf16):
    """Reference-order GEMV on ggml blocks: dequant exactly, then ``gemv_ref``."""
    w = dequant_matrix(ggml_type, raw, N, K)
    x = bf16_bits_to_f32(np.atleast_2d(np.asarray(x_bf16, np.uint16)))
    return gemv_ref(w, x)


# --------------------------------------------------------- tolerance-mode gate
def tolerance_gate(wdeq, x, acc_test, rel=1e-5):
    """Condition-aware gate for tolerance-mode accumulators.

    ``|acc_test - exact| <= rel * sum_k |x_k w_k|`` with the exact dot computed in fp64.
    Returns (ok, worst_ratio) where worst_ratio = max |delta| / (rel * sum|xw|).
    """
    w = np.asarray(wdeq, dtype=np.float64)
    x = np.atleast_2d(np.asarray(x, dtype=np.float64))
    exact = x @ w.T
    mag = np.abs(x) @ np.abs(w).T
    delta = np.abs(np.asarray(acc_test, np.float64) - exact)
    bound = rel * mag
    with np.errstate(divide="ignore", invalid="ignore"):
        ratio = np.where(bound > 0, delta / np.where(bound > 0, bound, 1), np.where(delta > 0, np.inf, 0))
    return bool(np.all(delta <= bound)), float(np.max(ratio)) if ratio.size else 0.0


def bf16_parity(y_test_bits, acc_ref, wdeq, x, rel=1e-5):
    """bf16 outputs of a reordered sum vs the reference-order accumulators.

    Where the sum is well conditioned (|acc_ref| >= 2^9 * rel * sum|a*w|, so that two
    in-tolerance fp32 results cannot straddle more than one bf16 rounding boundary) the
    outputs must be within 1 bf16 ulp; elsewhere (cancelled sums) they must be within the
    accumulator tolerance plus one ulp.  Returns (ok, max_ulp_well_conditioned, n_cancelled).
    """
    w = np.asarray(wdeq, dtype=np.float64)
    xx = np.atleast_2d(np.asarray(x, dtype=np.float64))
    mag = np.abs(xx) @ np.abs(w).T
    ref_bits = bf16_round_bits(np.asarray(acc_ref, np.float32))
    ulp = bf16_ulp_distance(y_test_bits, ref_bits)
    acc = np.abs(np.asarray(acc_ref, np.float64))
    good = acc >= (2 ** 9) * rel * mag
    yt = bf16_bits_to_f32(y_test_bits).astype(np.float64)
    yr = bf16_bits_to_f32(ref_bits).astype(np.float64)
    loose = np.abs(yt - yr) <= rel * mag + np.abs(yr) * 2.0 ** -7
    ok = bool(np.all(ulp[good] <= 1) and np.all(loose[~good]))
    return ok, int(ulp[good].max()) if good.any() else 0, int((~good).sum())


def bf16_ulp_distance(a_bits, b_bits):
    """|ordered-integer distance| between bf16 bit patterns (sign-magnitude ordering)."""
    def key(b):
        b = np.asarray(b, np.int64) & 0xFFFF
        return np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)
    return np.abs(key(a_bits) - key(b_bits))


# ------------------------------------------------------------ synthetic data
def random_q4k_blocks(rng, nb):
    """BASELINE config-0 distribution: d, dmin = fp16(|N(0,1)| * 2^-8); scales and qs uniform bytes."""
    raw = rng.integers(0, 256, size=(nb, 144), dtype=np.uint8)
    hdr = f32_to_f16_bits(np.abs(rng.standard_normal((nb, 2))) * 2.0 ** -8).astype(np.uint16)
    raw[:, 0:4] = hdr.view(np.uint8).reshape(nb, 4)
    return raw.reshape(-1)


def random_q6k_blocks(rng, nb):
    """Config-3 Q6_K: ql/qh uniform bytes, int8 scales uniform -32..31, d = fp16(|N| * 2^-8)."""
    raw = rng.integers(0, 256, size=(nb, 210), dtype=np.uint8)
    raw[:, 192:208] = rng.integers(-32, 32, size=(nb, 16)).astype(np.int8).view(np.uint8)
    d = f32_to_f16_bits(np.abs(rng.standard_normal(nb)) * 2.0 ** -8).astype(np.uint16)
    raw[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    return raw.reshape(-1)


def random_q8_0_blocks(rng, nb):
    """Config-3 Q8_0: int8 uniform -127..127, d = fp16(|N| * 2^-8)."""
    raw = np.empty((nb, 34), np.uint8)
    raw[:, 2:34] = rng.integers(-127, 128, size=(nb, 32)).astype(np.int8).view(np.uint8)
    d = f32_to_f16_bits(np.abs(rng.standard_normal(nb)) * 2.0 ** -8).astype(np.uint16)
    raw[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    return raw.reshape(-1)


def random_f16_weights(rng, n):
    """Config-3 F16 tiles: N(0, 0.02) as fp16 bytes."""
    return f32_to_f16_bits(rng.standard_normal(n) * 0.02).astype(np.uint16).view(np.uint8)


def random_bf16(rng, shape, scale=1.0):
    """bf16_RNE(N(0, scale^2)) bit patterns."""
    return bf16_round_bits((rng.standard_normal(shape) * scale).astype(np.float32))


RANDOM_BLOCKS = {
    GGML_Q4_K: random_q4k_blocks,
    GGML_Q6_K: random_q6k_blocks,
    GGML_Q8_0: random_q8_0_blocks,
}


def random_weights(rng, ggml_type, N, K):
    """Row-major ggml image [N][K/QK] of the BASELINE distribution for the type."""
    if ggml_type == GGML_F16:
        return random_f16_weights(rng, N * K)
    nb = N * K // BLOCK_WEIGHTS[ggml_type]
    return RANDOM_BLOCKS[ggml_type](rng, nb)
