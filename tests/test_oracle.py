"""Pin the CPU oracle before trusting it (CPU only).

Every oracle function is checked against something that does not restate its own formula:
the reference's literal KATs (test/q4k_prim_tb.v, src/q4k.vh), the golden fixtures written
from the reference itself (tests/golden/), closed forms evaluated exactly in float64, brute
force over small domains, an independent position-map restatement, the second (C) oracle,
and torch as a library.  Mutants with a planted mistake must fail the same checks.
"""
import os

import numpy as np
import pytest

from oracle import c_oracle as co
from oracle import glm_oracle as go
from oracle import q4k_oracle as qo

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def u32(a):
    return np.asarray(a, np.float32).view(np.uint32)


# ----------------------------------------------------------------- fp16 decode
# test/q4k_prim_tb.v:37-46 (signed zero, subnormal min/max, 1.0, max normal, ...)
F16_KAT = [(0x0000, 0x00000000), (0x8000, 0x80000000), (0x3C00, 0x3F800000), (0x211F, 0x3C23E000),
           (0x1D1F, 0x3BA3E000), (0xB400, 0xBE800000), (0x5F00, 0x43E00000), (0x03FF, 0x387FC000),
           (0x0001, 0x33800000), (0x7BFF, 0x477FE000)]


@pytest.mark.parametrize("h,exp", F16_KAT)
def test_fp16_kat(h, exp):
    assert qo.f32_bits(qo.f16_bits_to_f32(h)) == exp
    assert co.lib().oq_f16_to_f32_bits(h) == exp


def test_fp16_exhaustive_numpy_vs_c():
    allh = np.arange(65536, dtype=np.uint16)
    a = u32(qo.f16_bits_to_f32(allh))
    b = np.array([co.lib().oq_f16_to_f32_bits(int(h)) for h in range(0, 65536)], np.uint32)
    assert np.array_equal(a, b)
    # every fp16 value is exactly representable: the conversion is value-preserving
    fin = (allh & 0x7C00) != 0x7C00
    assert np.array_equal(qo.f16_bits_to_f32(allh[fin]).astype(np.float64),
                          allh[fin].view(np.float16).astype(np.float64))


# --------------------------------------------------------------- scale unpack
# test/q4k_prim_tb.v:33,49-56: SC = 96'h6B2A36C53CC261873FE85103, byte i = SC[8i+:8]
SC_HEX = 0x6B2A36C53CC261873FE85103
SC_KAT = [0x1C3, 0x851, 0x0A8, 0xF3F, 0xB05, 0x4D6, 0xCBA, 0x18B]


def _sc_bytes():
    return [(SC_HEX >> (8 * i)) & 0xFF for i in range(12)]


@pytest.mark.parametrize("j", range(8))
def test_scale_min_kat(j):
    sc, m = qo.scale_min_k4(j, _sc_bytes())
    assert (m << 6) | sc == SC_KAT[j]
    c_sc, c_m = __import__("ctypes").c_int(), __import__("ctypes").c_int()
    arr = (__import__("ctypes").c_uint8 * 12)(*_sc_bytes())
    co.lib().oq_scale_min_k4.argtypes = [__import__("ctypes").c_int, __import__("ctypes").c_void_p,
                                         __import__("ctypes").c_void_p, __import__("ctypes").c_void_p]
    co.lib().oq_scale_min_k4(j, arr, __import__("ctypes").byref(c_sc), __import__("ctypes").byref(c_m))
    assert (c_sc.value, c_m.value) == (sc, m)


def test_scale_vectorised_kat():
    sc, m = qo.unpack_scales_q4k(np.array([_sc_bytes()], np.uint8))
    assert [(int(m[0, j]) << 6) | int(sc[0, j]) for j in range(8)] == SC_KAT


def test_scale_pack_unpack_bijection():
    rng = np.random.default_rng(1)
    for _ in range(300):
        scs = [int(v) for v in rng.integers(0, 64, 8)]
        mns = [int(v) for v in rng.integers(0, 64, 8)]
        packed = qo.pack_scales_q4k(scs, mns)
        assert [qo.scale_min_k4(j, packed) for j in range(8)] == list(zip(scs, mns))
    # every value of every field, and uniform bytes <-> uniform fields (12 bytes = 16 x 6 bits)
    for j in range(8):
        for v in range(64):
            scs, mns = [0] * 8, [0] * 8
            scs[j] = v
            mns[7 - j] = 63 - v
            packed = qo.pack_scales_q4k(scs, mns)
            assert qo.scale_min_k4(j, packed)[0] == v
            assert qo.scale_min_k4(7 - j, packed)[1] == 63 - v
    raw = rng.integers(0, 256, size=(500, 12), dtype=np.uint8)
    sc, m = qo.unpack_scales_q4k(raw)
    repacked = np.array([qo.pack_scales_q4k(sc[i], m[i]) for i in range(500)], np.uint8)
    assert np.array_equal(repacked, raw)
    with pytest.raises(ValueError):
        qo.pack_scales_q4k([64] + [0] * 7, [0] * 8)


# -------------------------------------------------------------- Q4_K dequant
def _expected_q4k_weight(raw, pos):
    """Independent per-position restatement (the position map of tools/q4k_ref.py:168-178),
    evaluated exactly in float64: d*sc*q and dmin*m are exact (<= 21 significant bits),
    so the reference's value is one fp32 rounding of their difference."""
    raw = [int(v) for v in raw]
    d = float(np.array([raw[0] | (raw[1] << 8)], np.uint16).view(np.float16)[0])
    dm = float(np.array([raw[2] | (raw[3] << 8)], np.uint16).view(np.float16)[0])
    sub = pos // 32
    grp = sub // 2
    is_ = grp * 2 + (sub & 1)
    sc, m = qo.scale_min_k4(is_, raw[4:16])
    byte = (pos % 32) + (pos // 64) * 32
    q = (raw[16 + byte] & 0xF) if (sub & 1) == 0 else (raw[16 + byte] >> 4)
    return np.float32(d * sc * q - dm * m)


def _position_map_ok(dequant_fn, rng, nblocks=40):
    raw = qo.random_q4k_blocks(rng, nblocks).reshape(nblocks, 144)
    got = dequant_fn(raw.reshape(-1)).reshape(nblocks, 256)
    for b in range(nblocks):
        for pos in range(256):
            if qo.f32_bits(got[b, pos]) != qo.f32_bits(_expected_q4k_weight(raw[b], pos)):
                return False
    return True


def test_q4k_position_map_and_closed_form():
    assert _position_map_ok(qo.dequant_q4k, np.random.default_rng(2))


def test_q4k_brute_force_sc_q():
    """All 64 scales x 16 codes x 64 mins, over a sweep of d/dmin incl. fp16 subnormals."""
    ds = [0x0001, 0x0013, 0x03FF, 0x0400, 0x1C00, 0x2E66, 0x3C00, 0x5800, 0x7BFF]
    blocks = []
    expect = []
    for dh in ds:
        for dmh in (0x0000, 0x0001, 0x1C00, dh):
            for sc in range(64):
                m = (sc * 7 + dh) % 64
                scs = [sc] * 8
                mns = [m] * 8
                codes = np.arange(256) % 16
                qs = (codes.reshape(4, 2, 32)[:, 0, :] | (codes.reshape(4, 2, 32)[:, 1, :] << 4)).reshape(-1)
                blk = np.zeros(144, np.uint8)
                blk[0:2] = np.array([dh], np.uint16).view(np.uint8)
                blk[2:4] = np.array([dmh], np.uint16).view(np.uint8)
                blk[4:16] = qo.pack_scales_q4k(scs, mns)
                blk[16:] = qs
                blocks.append(blk)
                d = float(np.array([dh], np.uint16).view(np.float16)[0])
                dm = float(np.array([dmh], np.uint16).view(np.float16)[0])
                expect.append(np.float32(d * sc * codes.astype(np.float64) - dm * m))
    got = qo.dequant_q4k(np.concatenate(blocks))
    assert np.array_equal(u32(got), u32(np.concatenate(expect)))


def test_q4k_scalar_equals_vectorised():
    rng = np.random.default_rng(3)
    raw = qo.random_q4k_blocks(rng, 64).reshape(64, 144)
    vec = qo.dequant_q4k(raw.reshape(-1)).reshape(64, 256)
    for b in range(64):
        d_h, dm_h, scales, qs = qo.q4k_block_fields(raw[b])
        sca = qo.dequant_block_q4k_scalar(int(d_h[0]), int(dm_h[0]), scales[0], qs[0])
        assert np.array_equal(u32(sca), u32(vec[b]))


def test_q4k_mutants_fail():
    """Planted mistakes in the oracle are caught by the position-map / closed-form check."""
    rng = np.random.default_rng(4)

    def swapped_nibbles(raw):
        r = np.asarray(raw, np.uint8).reshape(-1, 144).copy()
        r[:, 16:] = ((r[:, 16:] >> 4) | (r[:, 16:] << 4)).astype(np.uint8)
        return qo.dequant_q4k(r.reshape(-1))

    def wrong_sub_block(raw):
        d_h, dm_h, scales, qs = qo.q4k_block_fields(raw)
        d = qo.f16_bits_to_f32(d_h)
        dm = qo.f16_bits_to_f32(dm_h)
        sc, mn = qo.unpack_scales_q4k(scales)
        sub = np.arange(256) // 64 * 2            # mistake: k//64*2 instead of k//32
        D = d[:, None] * sc.astype(np.float32)
        M = dm[:, None] * mn.astype(np.float32)
        return (D[:, sub] * qo.q4k_codes(qs).astype(np.float32) - M[:, sub]).reshape(-1)

    def d_times_m(raw):
        d_h, dm_h, scales, qs = qo.q4k_block_fields(raw)
        d = qo.f16_bits_to_f32(d_h)
        sc, mn = qo.unpack_scales_q4k(scales)
        sub = np.arange(256) // 32
        D = d[:, None] * sc.astype(np.float32)
        M = d[:, None] * mn.astype(np.float32)    # mistake: d instead of dmin
        return (D[:, sub] * qo.q4k_codes(qs).astype(np.float32) - M[:, sub]).reshape(-1)

    for mutant in (swapped_nibbles, wrong_sub_block, d_times_m):
        assert not _position_map_ok(mutant, rng, nblocks=4)


# ------------------------------------------------------------- Q6_K / Q8_0
def _q6k_edge_blocks(rng):
    """Edge blocks in the spirit of tools/q4k_mixed_gen.py:459-485 (codes, scales, d corners)."""
    def uniform(nib, hi):
        return [nib | (nib << 4)] * 128, [hi | (hi << 2) | (hi << 4) | (hi << 6)] * 64
    corners = [-128, -1, 0, 127] * 4
    out = []
    for ql, qh in (uniform(0, 0), uniform(0xF, 3), uniform(8, 2)):
        out.append((ql, qh, corners, 0x3C00))
    for sc in ([-128] * 16, [127] * 16, [0] * 16):
        out.append((list(rng.integers(0, 256, 128)), list(rng.integers(0, 256, 64)), sc, 0x3C00))
    for dh in (0x0001, 0x03FF, 0x0400, 0x0000, 0x8000, 0x5800):
        out.append((list(rng.integers(0, 256, 128)), list(rng.integers(0, 256, 64)), corners, dh))
    return out


def _q6k_raw(ql, qh, sc, dh):
    return np.concatenate([np.array(ql, np.uint8), np.array(qh, np.uint8),
                           np.array([s & 0xFF for s in sc], np.uint8), np.array([dh], np.uint16).view(np.uint8)])


def test_q6k_scalar_vectorised_closed_form():
    rng = np.random.default_rng(5)
    blocks = _q6k_edge_blocks(rng)
    raw = np.concatenate([_q6k_raw(*b) for b in blocks] + [qo.random_q6k_blocks(rng, 40)])
    vec = qo.dequant_q6k(raw).reshape(-1, 256)
    r2 = raw.reshape(-1, 210)
    for b in range(r2.shape[0]):
        ql, qh, sc, dh = r2[b, :128], r2[b, 128:192], r2[b, 192:208].view(np.int8), int(r2[b, 208:210].view(np.uint16)[0])
        sca = qo.dequant_block_q6k_scalar(dh, ql, qh, sc)
        assert np.array_equal(u32(sca), u32(vec[b]))
        # closed form: f32(d*sc) is exact, so w = one rounding of d*sc*(code-32) (exact in fp64)
        d = float(np.array([dh], np.uint16).view(np.float16)[0])
        for p in range(0, 256, 7):
            h, t, l = p // 128, (p // 32) % 4, p % 32
            qlb = int(ql[64 * h + l + 32 * (t & 1)])
            nib = (qlb & 0xF) if t < 2 else (qlb >> 4)
            code = nib | (((int(qh[32 * h + l]) >> (2 * t)) & 3) << 4)
            exp = np.float32(d * int(sc[p >> 4]) * (code - 32))
            assert qo.f32_bits(vec[b, p]) == qo.f32_bits(exp), (b, p)


def test_q8_0_exhaustive_closed_form():
    rng = np.random.default_rng(6)
    qs = np.arange(256, dtype=np.uint8)
    ds = np.concatenate([np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0x5800, 0x7BFF], np.uint16),
                         rng.integers(0, 0x7C00, 200).astype(np.uint16)])
    raw = []
    for dh in ds:
        for c in range(8):
            blk = np.empty(34, np.uint8)
            blk[0:2] = np.array([dh], np.uint16).view(np.uint8)
            blk[2:] = qs[32 * c:32 * c + 32]
            raw.append(blk)
    got = qo.dequant_q8_0(np.concatenate(raw)).reshape(len(ds), 256)
    d = np.asarray(ds, np.uint16).view(np.float16).astype(np.float64)
    exp = (d[:, None] * qs.view(np.int8).astype(np.float64)[None, :]).astype(np.float32)
    assert np.array_equal(u32(got), u32(exp))
    # s8 corners, src/q4k.vh:114-116
    for b, bits in [(0x80, 0xC3000000), (0xFF, 0xBF800000), (0x7F, 0x42FE0000), (0x20, 0x42000000),
                    (0xE0, 0xC2000000), (0x00, 0x00000000)]:
        assert qo.f32_bits(np.float32(qo.s8(b))) == bits
    assert qo.s8(-5) == -5 and qo.s8(251) == -5


def test_numpy_vs_c_oracle_all_types():
    rng = np.random.default_rng(7)
    for t, (N, K) in [(qo.GGML_Q4_K, (8, 768)), (qo.GGML_Q6_K, (8, 512)), (qo.GGML_Q8_0, (8, 512)),
                      (qo.GGML_F16, (8, 512))]:
        raw = qo.random_weights(rng, t, N, K)
        assert np.array_equal(u32(qo.dequant(t, raw)), u32(co.dequant(t, raw, N * K)))
        x = qo.random_bf16(rng, (3, K))
        a1, y1 = qo.gemv_quant_ref(t, raw, N, K, x)
        a2, y2 = co.gemv_ref(t, raw, N, K, x)
        assert np.array_equal(u32(a1), u32(a2)) and np.array_equal(y1, y2)


# ----------------------------------------------------------------- bf16 RNE
BF16_CASES = [
    (0x3F800000, 0x3F80), (0x3F808000, 0x3F80), (0x3F818000, 0x3F82), (0x3F808001, 0x3F81),
    (0x3F7FFFFF, 0x3F80), (0x7F7FFFFF, 0x7F80), (0xFF7FFFFF, 0xFF80), (0x7F800000, 0x7F80),
    (0xFF800000, 0xFF80), (0x7FC00001, 0x7FC0), (0x7F800001, 0x7F80), (0x00000001, 0x0000),
    (0x80008000, 0x8000), (0x00018000, 0x0002), (0xBF7FFFFF, 0xBF80),
]


@pytest.mark.parametrize("u,b", BF16_CASES)
def test_bf16_round_cases(u, b):
    assert qo.bf16_round_bits(qo.bits_f32(u)) == b
    assert (qo.f32_bits(qo.bf16_round_scalar(qo.bits_f32(u))) >> 16) == b
    assert co.lib().oq_bf16_round_bits(u) == b


def test_bf16_round_vs_torch_and_scalar():
    import torch
    rng = np.random.default_rng(8)
    u = rng.integers(0, 2 ** 32, 20000, dtype=np.uint64).astype(np.uint32)
    x = u.view(np.float32)
    fin = np.isfinite(x)
    ours = qo.bf16_round_bits(x)
    ref = torch.from_numpy(x[fin].copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours[fin], ref)
    for v in x[:500]:
        assert (qo.f32_bits(qo.bf16_round_scalar(v)) >> 16) == qo.bf16_round_bits(v)


# --------------------------------------------------------------- reference MAC
def test_gemv_ref_scalar_equals_vectorised():
    rng = np.random.default_rng(9)
    for K in (1, 7, 256, 300):
        w = (rng.standard_normal((5, K)) * 0.1).astype(np.float32)
        x = qo.bf16_bits_to_f32(qo.random_bf16(rng, (2, K)))
        acc, y = qo.gemv_ref(w, x)
        for m in range(2):
            for n in range(5):
                a_s, b_s = qo.dot_ref_scalar(x[m], w[n])
                assert qo.f32_bits(a_s) == qo.f32_bits(acc[m, n])
                assert qo.f32_bits(b_s) >> 16 == y[m, n]


def test_gemv_ref_special_cases():
    # K = 1 is one rounded product
    a = np.array([[1.1]], np.float32)
    w = np.array([[3.3]], np.float32)
    acc, _ = qo.gemv_ref(w, a)
    assert qo.f32_bits(acc[0, 0]) == qo.f32_bits(np.float32(np.float32(1.1) * np.float32(3.3)))
    # zero weights give +0
    acc, y = qo.gemv_ref(np.zeros((3, 9), np.float32), np.ones((1, 9), np.float32))
    assert np.all(u32(acc) == 0) and np.all(y == 0)
    # order probe: sequential 2^24 + 1 - 2^24 = 0, any other association gives 1
    w = np.array([[2.0 ** 24, 1.0, -(2.0 ** 24)]], np.float32)
    acc, _ = qo.gemv_ref(w, np.ones((1, 3), np.float32))
    assert acc[0, 0] == 0.0
    acc_rev, _ = qo.gemv_ref(w[:, ::-1].copy(), np.ones((1, 3), np.float32))
    assert acc_rev[0, 0] == 1.0  # the probe does distinguish orders


def test_tolerance_gate_catches_dropped_term():
    rng = np.random.default_rng(10)
    raw = qo.random_q4k_blocks(rng, 8 * 24)
    w = qo.dequant_q4k(raw).reshape(8, 6144)
    x = qo.bf16_bits_to_f32(qo.random_bf16(rng, (1, 6144)))
    acc, _ = qo.gemv_ref(w, x)
    ok, worst = qo.tolerance_gate(w, x, acc)
    assert ok and worst < 0.05
    bad = acc - x[:, 100:101] * w[None, :, 100]     # drop one product
    ok_bad, _ = qo.tolerance_gate(w, x, bad[0][None])
    assert not ok_bad


# ----------------------------------------------------------- golden fixtures
def test_golden_activation_tables():
    t = np.load(os.path.join(GOLD, "act_tables.npz"))
    allb = np.arange(65536, dtype=np.uint16)
    assert np.array_equal(go.glm_silu_bits_vec(allb), t["silu"])
    assert np.array_equal(go.glm_sigmoid_bits_vec(allb), t["sigmoid"])
    L = co.lib()
    idx = np.random.default_rng(11).integers(0, 65536, 4000)
    assert all(L.oq_glm_silu(int(b)) == t["silu"][b] for b in idx)
    assert all(L.oq_glm_sigmoid(int(b)) == t["sigmoid"][b] for b in idx)
    for b in idx[:300]:
        x = qo.bf16_bits_to_f32(b)
        assert qo.bf16_round_bits(go.sigmoid_fp32(x)) == t["sigmoid"][b]
        assert qo.f32_bits(go.glm_silu(x)) >> 16 == t["silu"][b]


def test_golden_rsqrt():
    r = np.load(os.path.join(GOLD, "rsqrt_cases.npz"))
    assert np.array_equal(u32(go.fp32_rsqrt_vec(r["x"].view(np.float32))), r["y"])
    L = co.lib()
    for u, v in zip(r["x"][:800], r["y"][:800]):
        assert qo.f32_bits(go.fp32_rsqrt(qo.bits_f32(int(u)))) == int(v)
        assert L.oq_rsqrt_bits(int(u)) == int(v)


def test_sigmoid_and_rsqrt_accuracy():
    """What the mathematics fixes: 2-step rsqrt ~5e-6 relative; sigmoid close to 1/(1+e^-x)."""
    x = np.linspace(1e-3, 1e3, 5000).astype(np.float32)
    rel = np.abs(go.fp32_rsqrt_vec(x).astype(np.float64) * np.sqrt(x.astype(np.float64)) - 1)
    assert rel.max() < 1e-5
    b = qo.bf16_round_bits(np.linspace(-20, 20, 4001).astype(np.float32))
    xs = qo.bf16_bits_to_f32(b).astype(np.float64)
    s = go.sigmoid_fp32_vec(qo.bf16_bits_to_f32(b)).astype(np.float64)
    # 1/d = rsqrt(d)^2 doubles rsqrt's ~5e-6 relative error
    assert np.max(np.abs(s - 1 / (1 + np.exp(-np.clip(xs, -16, 16))))) < 2e-5


def test_golden_router_cases():
    rc = np.load(os.path.join(GOLD, "router_cases.npz"))
    keys = sorted({k.rsplit("_", 1)[0] for k in rc.files})
    assert len(keys) == 9
    ties = 0
    for k in keys:
        E, topk = (int(v) for v in rc[k + "_E"])
        logits = go.router_logits(qo.GGML_Q4_K, rc[k + "_w"], E, 256, rc[k + "_x"])
        sel, selw, gate = go.router_tail(logits, topk)
        assert np.array_equal(sel, rc[k + "_sel"])
        assert np.array_equal(selw, rc[k + "_selw"])
        assert np.array_equal(gate, rc[k + "_gate"])
        ties += len(gate) - len(np.unique(gate))
    assert ties > 0  # the cases exercise the index tie-break


def test_router_mutant_tie_order_fails():
    rc = np.load(os.path.join(GOLD, "router_cases.npz"))
    caught = False
    for k in sorted({k.rsplit("_", 1)[0] for k in rc.files}):
        E, topk = (int(v) for v in rc[k + "_E"])
        gate = rc[k + "_gate"]
        g = qo.bf16_bits_to_f32(gate)
        order = sorted(range(E), key=lambda e: (go.f32_order_key(g[e]), e), reverse=True)  # mistake: index desc
        if not np.array_equal(np.array(order[:topk], np.int32), rc[k + "_sel"]):
            caught = True
    assert caught


def test_golden_swiglu_cases():
    s = np.load(os.path.join(GOLD, "swiglu_cases.npz"))
    for c in range(2):
        y, _ = go.swiglu_expert(s[f"c{c}_x"], s[f"c{c}_wg"], s[f"c{c}_wu"], s[f"c{c}_wd"], qo.GGML_Q4_K, 256, 256)
        assert np.array_equal(y, s[f"c{c}_y"])


def test_moe_combine_order_and_shared():
    """Combine is sequential in slot order; the shared expert is added last with weight 1."""
    y1 = np.array([qo.bf16_round_bits(np.float32(2.0 ** 9))], np.uint16)
    y2 = np.array([qo.bf16_round_bits(np.float32(1.0))], np.uint16)
    one = qo.bf16_round_bits(np.float32(1.0))
    out, facc = go.moe_combine([one, one], [y1, y2])
    assert facc[0] == np.float32(513.0)
    out_sh, facc_sh = go.moe_combine([one], [y1], y2)
    assert facc_sh[0] == np.float32(513.0)
    # -0 from a single expert is normalised to +0 by the fp32 accumulator starting at +0
    neg0 = np.array([0x8000], np.uint16)
    out0, _ = go.moe_combine([one], [neg0])
    assert out0[0] == 0
