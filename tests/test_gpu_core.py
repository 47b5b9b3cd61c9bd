"""GPU parity for the core numerics through the C ABI: exact dequant of every type, bf16
rounding, glm activations, reference-order GEMV (bit-exact) and the fast streaming GEMV
(tolerance: |acc - exact| <= 1e-5 * sum|a*w|, bf16 within 1 ulp of the reference order)."""
import os

import numpy as np
import pytest
import torch

from aipu_amd import device as dev
from oracle import c_oracle as co
from oracle import glm_oracle as go
from oracle import q4k_oracle as qo

from .gpu_util import assert_bits_equal, d_bf16, d_u8, h_bits, h_f32, note, random_weights_gpu, u32

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")


# ------------------------------------------------------------------- dequant
def test_dequant_f16_exhaustive():
    note("dequant F16 exhaustive")
    allh = np.arange(65536, dtype=np.uint16)
    got = h_f32(dev.dequantize(qo.GGML_F16, d_u8(allh.view(np.uint8))))
    exp = qo.f16_bits_to_f32(allh)
    fin = (allh & 0x7C00) != 0x7C00
    inf = ((allh & 0x7C00) == 0x7C00) & ((allh & 0x3FF) == 0)
    assert_bits_equal(u32(got)[fin | inf], u32(exp)[fin | inf], "F16 finite/inf")
    nan = ~(fin | inf)
    assert np.all(np.isnan(got[nan]))          # NaN stays NaN (payload quieting is not part of the contract)
    assert u32(got)[1] == 0x33800000           # test/q4k_prim_tb.v:45 smallest subnormal KAT


def _q4k_edge_blocks(rng):
    out = []
    for dh, dmh in [(0x0001, 0x0001), (0x03FF, 0x0000), (0x0000, 0x3C00), (0x8000, 0x0400), (0x7BFF, 0x7BFF),
                    (0x5800, 0x0013)]:
        blk = qo.random_q4k_blocks(rng, 1).copy()
        blk[0:2] = np.array([dh], np.uint16).view(np.uint8)
        blk[2:4] = np.array([dmh], np.uint16).view(np.uint8)
        out.append(blk)
    return np.concatenate(out)


@pytest.mark.parametrize("t", [qo.GGML_Q4_K, qo.GGML_Q6_K, qo.GGML_Q8_0, qo.GGML_F16, 30])
def test_dequant_random_bitexact(t):
    note(f"dequant type {t}")
    rng = np.random.default_rng(100 + t)
    if t == 30:
        raw = qo.random_bf16(rng, 4096).view(np.uint8)
        exp = qo.bf16_bits_to_f32(raw.view(np.uint16))
        n = 4096
    else:
        raw = qo.random_weights(rng, t, 64, 4096)
        if t == qo.GGML_Q4_K:
            raw = np.concatenate([raw, _q4k_edge_blocks(rng)])
        n = raw.size // qo.BLOCK_BYTES[t] * qo.BLOCK_WEIGHTS[t]
        exp = qo.dequant(t, raw)
    got = h_f32(dev.dequantize(t, d_u8(raw), n))
    assert_bits_equal(u32(got), u32(exp), f"dequant {t}")


def test_q4k_scale_min_kat_and_random():
    note("scale_min")
    sc_hex = 0x6B2A36C53CC261873FE85103
    kat = [0x1C3, 0x851, 0x0A8, 0xF3F, 0xB05, 0x4D6, 0xCBA, 0x18B]
    blk = np.zeros(144, np.uint8)
    blk[4:16] = [(sc_hex >> (8 * i)) & 0xFF for i in range(12)]
    rng = np.random.default_rng(7)
    raw = np.concatenate([blk, qo.random_q4k_blocks(rng, 500)])
    got = h_bits(dev.q4k_scale_min(d_u8(raw)).view(torch.int16)).astype(np.int64)
    sc, m = qo.unpack_scales_q4k(raw.reshape(-1, 144)[:, 4:16])
    assert np.array_equal(got & 0xFF, sc) and np.array_equal(got >> 8, m)
    assert [int(((v >> 8) << 6) | (v & 0xFF)) for v in got[0]] == kat


def test_bf16_round():
    note("bf16_round")
    rng = np.random.default_rng(8)
    cases = np.array([0x3F800000, 0x3F808000, 0x3F818000, 0x3F7FFFFF, 0x7F7FFFFF, 0xFF7FFFFF, 0x7F800000,
                      0x7FC00001, 0x7F800001, 0x00000001, 0x80008000, 0x00018000], np.uint32)
    u = np.concatenate([cases, rng.integers(0, 2 ** 32, 100000, dtype=np.uint64).astype(np.uint32)])
    got = h_bits(dev.bf16_round(torch.from_numpy(u.view(np.float32).copy()).to("cuda")))
    assert_bits_equal(got, qo.bf16_round_bits(u.view(np.float32)), "bf16")


# ---------------------------------------------------------------- activations
def test_glm_act_tables_exhaustive():
    note("glm_silu / glm_sigmoid exhaustive")
    t = np.load(os.path.join(GOLD, "act_tables.npz"))
    allb = np.arange(65536, dtype=np.uint16)
    assert_bits_equal(h_bits(dev.glm_silu(d_bf16(allb))), t["silu"], "silu")
    assert_bits_equal(h_bits(dev.glm_sigmoid(d_bf16(allb))), t["sigmoid"], "sigmoid")


def test_fp32_rsqrt_golden():
    note("fp32_rsqrt")
    r = np.load(os.path.join(GOLD, "rsqrt_cases.npz"))
    got = h_f32(dev.fp32_rsqrt(torch.from_numpy(r["x"].view(np.float32).copy()).to("cuda")))
    assert_bits_equal(u32(got), r["y"], "rsqrt")


# ------------------------------------------------------- reference-order GEMV
# Q4_K runs on the register kernel (k_gemv_ref_q4k) while K * 4 bytes of staged activations fit
# 128 KB, in passes of up to 8, 4, 2 or 1 rows as the staging allows: 9 rows at K = 256 (8 + 1),
# 8 at K = 6144 (two passes of 4), 5 at K = 8192 (4 + 1), 2 at K = 32768 (one row per pass);
# K = 40960 takes the staged-weights kernel.  Q8_0, F16 and BF16 take their register kernel
# (k_gemv_ref_reg) at K a multiple of 64, Q6_K its own (k_gemv_ref_q6k, blocks alternately 4-B
# aligned and 2 B past a dword) at K a multiple of 512 (K = 1280 stays on the staged kernel).
# Ragged N leaves part of the last wave idle.
REF_CASES = [
    (qo.GGML_Q4_K, 200, 768, 1), (qo.GGML_Q4_K, 131, 512, 3), (qo.GGML_Q4_K, 64, 256, 9),
    (qo.GGML_Q4_K, 130, 6144, 8), (qo.GGML_Q4_K, 33, 8192, 5), (qo.GGML_Q4_K, 70, 32768, 2),
    (qo.GGML_Q4_K, 64, 40960, 1), (qo.GGML_Q8_0, 130, 6144, 8), (qo.GGML_F16, 70, 4096, 3), (30, 33, 8192, 5),
    (qo.GGML_Q6_K, 130, 6144, 8), (qo.GGML_Q6_K, 65, 1024, 1), (qo.GGML_Q6_K, 40, 1280, 2),
    (qo.GGML_Q6_K, 96, 512, 2), (qo.GGML_Q8_0, 70, 512, 1), (qo.GGML_F16, 65, 256, 2), (30, 64, 512, 1),
]


@pytest.mark.parametrize("t,N,K,M", REF_CASES)
def test_gemv_ref_bitexact(t, N, K, M):
    note(f"gemv ref type={t} N={N} K={K} M={M}")
    rng = np.random.default_rng(N * K + M)
    raw = qo.random_bf16(rng, N * K).view(np.uint8) if t == 30 else qo.random_weights(rng, t, N, K)
    x = qo.random_bf16(rng, (M, K))
    y, yf = dev.gemv(t, d_u8(raw), N, K, d_bf16(x), mode="ref", out_f32=True)
    if t == 30:
        acc, ye = qo.gemv_ref(qo.bf16_bits_to_f32(raw.view(np.uint16)).reshape(N, K), qo.bf16_bits_to_f32(x))
    else:
        acc, ye = co.gemv_ref(t, raw, N, K, x)
    assert_bits_equal(u32(h_f32(yf)), u32(acc), "acc")
    assert_bits_equal(h_bits(y), ye, "y")


@pytest.mark.parametrize("t", [qo.GGML_Q4_K, qo.GGML_Q6_K, qo.GGML_Q8_0, qo.GGML_F16])
def test_gemv_ref_unaligned_activations(t):
    """Reference mode asks only 2-byte aligned activations (and, below Q4_K, weights): a vector
    that starts one element into its buffer takes the staged-weights kernel and stays bit-exact."""
    N, K, M = 96, 1024, 2
    note(f"gemv ref unaligned activations type={t}")
    rng = np.random.default_rng(4242 + t)
    raw = qo.random_weights(rng, t, N, K)
    x = qo.random_bf16(rng, (M, K))
    buf = torch.zeros(M * K + 1, dtype=torch.int16, device="cuda")
    buf[1:] = torch.from_numpy(x.reshape(-1).view(np.int16)).to("cuda")
    xd = buf[1:].view(torch.bfloat16).view(M, K)
    assert xd.data_ptr() % 16 == 2
    y, yf = dev.gemv(t, d_u8(raw), N, K, xd, mode="ref", out_f32=True)
    acc, ye = co.gemv_ref(t, raw, N, K, x)
    assert_bits_equal(u32(h_f32(yf)), u32(acc), "acc")
    assert_bits_equal(h_bits(y), ye, "y")


def _random_ref_cases(n=24, seed=20261202):
    """Seeded shapes for the reference-order kernels: every type, ragged N, M = 1..9, K at the
    register kernels' multiples (Q4_K 256, Q6_K 512, Q8_0 / F16 / BF16 64) and off them."""
    rng = np.random.default_rng(seed)
    kinds = [(qo.GGML_Q4_K, 256), (qo.GGML_Q6_K, 256), (qo.GGML_Q8_0, 32), (qo.GGML_F16, 1), (30, 1)]
    cases = []
    for i in range(n):
        t, blk = kinds[i % len(kinds)]
        if t in (qo.GGML_Q4_K, qo.GGML_Q6_K):
            K = 256 * int(rng.integers(1, 25))
        elif t == qo.GGML_Q8_0:
            K = 32 * int(rng.integers(1, 160))
        else:
            K = int(rng.integers(1, 5000)) if i % 2 else 64 * int(rng.integers(1, 80))
        cases.append((t, int(rng.integers(1, 300)), K, int(rng.integers(1, 10))))
    return cases


@pytest.mark.parametrize("t,N,K,M", _random_ref_cases())
def test_gemv_ref_random_shapes(t, N, K, M):
    note(f"gemv ref random type={t} N={N} K={K} M={M}")
    rng = np.random.default_rng(N * 7919 + K * 31 + M)
    raw = qo.random_bf16(rng, N * K).view(np.uint8) if t == 30 else qo.random_weights(rng, t, N, K)
    x = qo.random_bf16(rng, (M, K))
    y, yf = dev.gemv(t, d_u8(raw), N, K, d_bf16(x), mode="ref", out_f32=True)
    if t == 30:
        acc, ye = qo.gemv_ref(qo.bf16_bits_to_f32(raw.view(np.uint16)).reshape(N, K), qo.bf16_bits_to_f32(x))
    else:
        acc, ye = co.gemv_ref(t, raw, N, K, x)
    assert_bits_equal(u32(h_f32(yf)), u32(acc), "acc")
    assert_bits_equal(h_bits(y), ye, "y")


PARTIAL_CASES = [
    (qo.GGML_Q8_0, 70, 288, 1), (qo.GGML_Q8_0, 64, 4128, 3), (qo.GGML_F16, 65, 100, 2), (qo.GGML_F16, 33, 513, 1),
    (30, 64, 264, 4), (30, 17, 7, 1),
]


@pytest.mark.parametrize("mode", ["ref", "fast"])
@pytest.mark.parametrize("t,N,K,M", PARTIAL_CASES)
def test_gemv_k_not_multiple_of_256(t, N, K, M, mode):
    """K a multiple of the type's block but not of 256 (Q8_0: 32; F16 / BF16: any K, odd
    ones included): the last 256-weight stage is partial; both modes run the reference order
    and are bit-exact against the oracle."""
    note(f"gemv partial super-block type={t} N={N} K={K} M={M} {mode}")
    rng = np.random.default_rng(N * K + M + 7)
    raw = qo.random_bf16(rng, N * K).view(np.uint8) if t == 30 else qo.random_weights(rng, t, N, K)
    x = qo.random_bf16(rng, (M, K))
    y, yf = dev.gemv(t, d_u8(raw), N, K, d_bf16(x), mode=mode, out_f32=True)
    if t == 30:
        acc, ye = qo.gemv_ref(qo.bf16_bits_to_f32(raw.view(np.uint16)).reshape(N, K), qo.bf16_bits_to_f32(x))
    else:
        acc, ye = co.gemv_ref(t, raw, N, K, x)
    assert_bits_equal(u32(h_f32(yf)), u32(acc), "acc")
    assert_bits_equal(h_bits(y), ye, "y")


def test_gemv_ref_full_north_star_shape():
    """K = N = 6144, M = 1: every output bit-exact against the C oracle."""
    note("gemv ref 6144x6144")
    rng = np.random.default_rng(6144)
    raw = qo.random_q4k_blocks(rng, 6144 * 24)
    x = qo.random_bf16(rng, (1, 6144))
    y, yf = dev.gemv(qo.GGML_Q4_K, d_u8(raw), 6144, 6144, d_bf16(x), mode="ref", out_f32=True)
    acc, ye = co.gemv_ref(qo.GGML_Q4_K, raw, 6144, 6144, x)
    assert_bits_equal(u32(h_f32(yf)), u32(acc), "acc")
    assert_bits_equal(h_bits(y), ye, "y")


def test_gemv_f32_matmul_q4k_col():
    note("gemv_f32")
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((37, 300)) * 0.05).astype(np.float32)
    x = rng.standard_normal((2, 300)).astype(np.float32)   # not bf16-valued: full fp32 inputs
    y, yf = dev.gemv_f32(torch.from_numpy(w).cuda(), torch.from_numpy(x).cuda(), out_f32=True)
    acc, ye = qo.gemv_ref(w, x)
    assert_bits_equal(u32(h_f32(yf)), u32(acc), "acc")
    assert_bits_equal(h_bits(y), ye, "y")


# ------------------------------------------------------------------ fast GEMV
FAST_CASES = [
    (6144, 6144, 1), (4096, 4096, 1), (6144, 6144, 2), (6144, 6144, 4), (6144, 6144, 8),
    (1001, 2048, 1), (77, 256, 3), (300, 2304, 1), (64, 18432, 1), (2048, 6144, 5),
    # small-batch kernel: K split 3 / 4 blocks per wave, passes of 8 + 4, 4 + 2, and a K
    # too large for it (served by the staged kernel in passes of 4)
    (300, 2304, 8), (129, 8192, 6), (16, 512, 12), (64, 18432, 8),
    # small-batch kernel (2..4 rows): 8 waves x 3 blocks (ragged last tile), 8 x 2, 4 x 2,
    # 6 x 3, 5 x 1, 3 x 1 and 1 x 1 blocks per wave, 2, 3 and 4 rows; the 256-row router
    # shape; passes of 8 + 3 + 1, 7, 6 and 8 + 8 rows
    (6144 + 24, 6144, 2), (4096, 4096, 2), (1001, 2048, 2), (300, 4608, 2), (40, 1280, 2), (77, 768, 2),
    (256, 6144, 2), (6144, 6144, 3), (64, 256, 2), (64, 256, 4), (64, 512, 3), (48, 768, 4),
    (100, 4608, 12), (1000, 6144, 7), (100, 4608, 6), (512, 4096, 16),
    # several weight-copy rounds per wave (3-block groups x 2, 2-block groups x 3): the
    # round loop must run to the end
    (64, 9216, 1), (40, 12288, 1),
    # N / #CUs rows per workgroup (two tiles, the second partly or barely filled)
    (4100, 2048, 1), (7000, 6144, 1),
    # the persistent single-row kernel at its largest K (five copy rounds per tile, two pairs
    # per compute wave): 32 and 29 blocks, and a shape with N > 6144 that reuses tile buffers
    (300, 8192, 1), (64, 7424, 1), (7000, 8192, 1),
]


@pytest.mark.parametrize("N,K,M", FAST_CASES)
def test_gemv_fast_tolerance(N, K, M):
    note(f"gemv fast Q4_K N={N} K={K} M={M}")
    rng = np.random.default_rng(N + K + M)
    raw = qo.random_q4k_blocks(rng, N * K // 256)
    x = qo.random_bf16(rng, (M, K))
    wd = d_u8(raw)
    y, yf = dev.gemv(qo.GGML_Q4_K, wd, N, K, d_bf16(x), mode="fast", out_f32=True)
    _, yrf = dev.gemv(qo.GGML_Q4_K, wd, N, K, d_bf16(x), mode="ref", out_f32=True)
    w = qo.dequant_q4k(raw).reshape(N, K)
    xf = qo.bf16_bits_to_f32(x)
    ok, worst = qo.tolerance_gate(w, xf, h_f32(yf), rel=1e-5)
    note(f"  worst |delta| = {worst:.4f} of the 1e-5*sum|a*w| bound")
    assert ok, f"tolerance gate exceeded: worst {worst:.3f} of the 1e-5*sum|a*w| bound"
    ok, max_ulp, n_cancelled = qo.bf16_parity(h_bits(y), h_f32(yrf), w, xf)
    assert ok, f"bf16 outputs: {max_ulp} ulp on well-conditioned outputs ({n_cancelled} cancelled sums)"
    # deterministic: a second run is bitwise identical
    y2, yf2 = dev.gemv(qo.GGML_Q4_K, wd, N, K, d_bf16(x), mode="fast", out_f32=True)
    assert np.array_equal(u32(h_f32(yf2)), u32(h_f32(yf)))


# Fast-mode batch invariance: the reference gates PE_M = 2 rows bit-exact against per-row
# PE_M = 1 runs (Makefile:1488-1508), and speculative decoding "changes speed, never output"
# (PROJECT_BRIEFING.md:50).  In fast mode every row of an M-row call is bit-identical to the
# one-row call on that row, fp32 accumulators included: the persistent row-pair kernel
# (M = 2..8 at K = 2048/4096/6144), k_gemvs / k_gemvm elsewhere, and a launch per row where no
# multi-row kernel forms rows in the one-row order (K / 256 not split into at most 8 parts of
# at most 4 blocks: 2816, 5632; M = 1 off the persistent kernel: K > 8192), and the streaming
# kernel beyond the matrix-core staging limit.  Two rows share a persistent launch wherever
# nothing else takes them (odd prime block counts such as 23).
# Covers every row count of a verify batch at the BASELINE shape, the other matrix-core shapes
# (ragged N, passes of 8 + remainder), the shapes without a multi-row kernel, and K > 8192.
INVARIANCE_CASES = [(6144, 6144, m) for m in (2, 3, 4, 5, 6, 7, 8)] + [
    (4096, 4096, 4), (1001, 2048, 8), (300, 2304, 3), (512, 4096, 12), (64, 7168, 8), (300, 4096, 9),
    # persistent row-pair kernel: three tiles per CU with a ragged last tile, two tiles per
    # CU, a single tile, and one tile too many for it (the small-batch kernels take over)
    (6100, 6144, 3), (2050, 4096, 6), (8, 2048, 2), (6144 + 24, 6144, 8),
    # one-row calls on the 16-row-tile kernel (k_gemv1) against batches on the row-pair and
    # small-batch kernels
    (4096, 2048, 3), (8192, 4096, 2), (4096, 8192, 2),
    # no multi-row kernel in the one-row order: one launch per row
    (300, 2816, 5), (64, 5632, 2),
    # K > 8192: the one-row kernel is k_gemv1 (several weight-copy rounds); beyond the
    # matrix-core staging limit (K > 30464) every M runs the streaming kernel
    (64, 9216, 3), (40, 12288, 5), (64, 18432, 8), (16, 32768, 3),
    # two rows on the persistent one-row kernel (the M = 2 cases above run there too): an odd
    # block count (a half last pair), a ragged last tile, four tiles per CU, one tile too many
    # for it, a single block
    (100, 2304, 2), (6100, 6144, 2), (8192, 6144, 2), (8200, 4096, 2), (1, 256, 2),
    # block counts that no k_mfma_gemv plan splits (17, 19, 23, 29, 31 blocks): one-row calls on
    # the persistent kernel, batches two rows at a time on it (K <= 6144) or a launch per row;
    # and 37 blocks (K > 8192), where every M runs the streaming kernel
    (2000, 4352, 3), (3000, 4864, 8), (6390, 5888, 6), (2000, 7424, 5), (4100, 7936, 2), (100, 9472, 3)]


def _fast_rows(t, wd, N, K, rows, mode):
    y, yf = dev.gemv(t, wd, N, K, d_bf16(np.ascontiguousarray(rows)), mode=mode, out_f32=True)
    return h_bits(y), u32(h_f32(yf))


@pytest.mark.parametrize("N,K,M", INVARIANCE_CASES)
def test_gemv_fast_batch_invariance(N, K, M):
    note(f"gemv fast batch invariance N={N} K={K} M={M}")
    rng = np.random.default_rng(7 * N + K + M)
    raw = qo.random_q4k_blocks(rng, N * K // 256)
    x = qo.random_bf16(rng, (M, K))
    wd = d_u8(raw)
    yb, yfb = _fast_rows(qo.GGML_Q4_K, wd, N, K, x, "fast")
    for r in range(M):
        y1, yf1 = _fast_rows(qo.GGML_Q4_K, wd, N, K, x[r:r + 1], "fast")
        assert_bits_equal(yf1[0], yfb[r], f"row {r} of M={M}: fp32 accumulators")
        assert_bits_equal(y1[0], yb[r], f"row {r} of M={M}: bf16 outputs")
    # and the batch itself meets the tolerance gate (the one-row kernel's contract)
    w = qo.dequant_q4k(raw).reshape(N, K)
    ok, worst = qo.tolerance_gate(w, qo.bf16_bits_to_f32(x), yfb.view(np.float32), rel=1e-5)
    assert ok, f"batch of M={M}: fp32 accumulators {worst:.3f} of the tolerance"


def _random_fast_cases(n=20, seed=1202):
    """Seeded Q4_K shapes for the fast mode's kernel choice: N from one tile to many per CU, K from
    one block to 8192 (one- and two-pair persistent waves, odd block counts), M = 1..8."""
    rng = np.random.default_rng(seed)
    return [(int(rng.choice([int(rng.integers(1, 64)), int(rng.integers(64, 3000)), int(rng.integers(3000, 9000))])),
             256 * int(rng.integers(1, 33)), int(rng.integers(1, 9))) for _ in range(n)]


@pytest.mark.parametrize("N,K,M", _random_fast_cases())
def test_gemv_fast_random_shapes(N, K, M):
    """Every row of a fast-mode batch equals its one-row launch bit for bit, and the batch meets
    the tolerance gate, at seeded random shapes (whichever kernels the dispatch picks)."""
    note(f"gemv fast random N={N} K={K} M={M}")
    rng = np.random.default_rng(13 * N + K + M)
    raw = qo.random_q4k_blocks(rng, N * K // 256)
    x = qo.random_bf16(rng, (M, K))
    wd = d_u8(raw)
    yb, yfb = _fast_rows(qo.GGML_Q4_K, wd, N, K, x, "fast")
    for r in range(M):
        y1, yf1 = _fast_rows(qo.GGML_Q4_K, wd, N, K, x[r:r + 1], "fast")
        assert_bits_equal(yf1[0], yfb[r], f"row {r} of M={M}: fp32 accumulators")
        assert_bits_equal(y1[0], yb[r], f"row {r} of M={M}: bf16 outputs")
    w = qo.dequant_q4k(raw).reshape(N, K)
    ok, worst = qo.tolerance_gate(w, qo.bf16_bits_to_f32(x), yfb.view(np.float32), rel=1e-5)
    assert ok, f"batch of M={M}: fp32 accumulators {worst:.3f} of the tolerance"
    assert not dev.wait_timeouts(), "a bounded wait gave up"


@pytest.mark.parametrize("N,K,M", [(300, 4096, 2), (513, 6144, 3), (4100, 4096, 4)])
def test_gemv_fast_batch_invariance_bf16(N, K, M):
    """bf16 weights (the router's type) in the streaming kernel: batch rows == one-row calls."""
    note(f"gemv fast bf16 batch invariance N={N} K={K} M={M}")
    rng = np.random.default_rng(11 * N + K + M)
    wb = qo.random_bf16(rng, (N, K), scale=0.05)
    x = qo.random_bf16(rng, (M, K))
    wd = d_u8(wb.view(np.uint8).reshape(-1))
    yb, yfb = _fast_rows(go.BF16_TYPE, wd, N, K, x, "fast")
    for r in range(M):
        y1, yf1 = _fast_rows(go.BF16_TYPE, wd, N, K, x[r:r + 1], "fast")
        assert_bits_equal(yf1[0], yfb[r], f"bf16 row {r} of M={M}: fp32 accumulators")
        assert_bits_equal(y1[0], yb[r], f"bf16 row {r} of M={M}: bf16 outputs")


# AIPU_MODE_FAST_DENSE: Q4_K batches of 2..8 rows at K = 2048/4096/6144 run the dense
# multi-row kernel.  A row agrees with its one-row call within the fast-mode tolerance (fp32
# gate, bf16 within 1 ulp where well conditioned), and its bits depend neither on the other
# rows of the batch nor on its position -- reversing the batch, or sending the row in another
# batch, gives the same bits.  Shapes it does not serve behave as AIPU_MODE_FAST.
def _random_dense_cases(n=10, seed=1909):
    """Seeded (N, K, M) for the dense mode: mostly its K = 2048 / 4096 / 6144, sometimes another K
    (where it behaves as the fast mode), N up to one tile past the dense kernel's limit."""
    rng = np.random.default_rng(seed)
    ks = [2048, 4096, 6144, 2048, 4096, 6144, 1280, 4352]
    return [(int(rng.integers(1, 6169)), int(ks[int(rng.integers(0, len(ks)))]), int(rng.integers(2, 12)))
            for _ in range(n)]


DENSE_CASES = [(6144, 6144, m) for m in (2, 4, 7, 8)] + [
    (6100, 6144, 3), (2050, 4096, 6), (8, 2048, 2), (1001, 2048, 8), (6144 + 24, 6144, 8), (300, 2816, 5)
] + _random_dense_cases()


def _dense_row(N, K, M, r):
    """Whether row r of an M-row dense-mode GEMV is served by the dense multi-row kernel
    (passes of 8 rows; a pass of one row goes to the single-row kernel)."""
    left = min(M - (r // 8) * 8, 8)
    return left >= 2 and K % 2048 == 0 and 2048 <= K <= 6144 and (N + 7) // 8 <= 3 * 256


@pytest.mark.parametrize("N,K,M", DENSE_CASES)
def test_gemv_fast_dense_batch(N, K, M):
    note(f"gemv fast_dense batch N={N} K={K} M={M}")
    rng = np.random.default_rng(7 * N + K + M)
    raw = qo.random_q4k_blocks(rng, N * K // 256)
    x = qo.random_bf16(rng, (M, K))
    wd = d_u8(raw)
    yb, yfb = _fast_rows(qo.GGML_Q4_K, wd, N, K, x, "fast_dense")
    w = qo.dequant_q4k(raw).reshape(N, K)
    xf = qo.bf16_bits_to_f32(x)
    dense = [r for r in range(M) if _dense_row(N, K, M, r)]
    for r in range(M):
        y1, yf1 = _fast_rows(qo.GGML_Q4_K, wd, N, K, x[r:r + 1], "fast_dense")
        if r in dense:
            f = yfb[r].view(np.float32)
            ok, worst = qo.tolerance_gate(w, xf[r:r + 1], f[None, :], rel=1e-5)
            assert ok, f"row {r} of M={M}: fp32 accumulators {worst:.3f} of the tolerance"
            ok, max_ulp, _ = qo.bf16_parity(yb[r][None, :], yf1[0].view(np.float32)[None, :], w, xf[r:r + 1])
            assert ok, f"row {r} of M={M}: bf16 {max_ulp} ulp from the one-row call"
        else:
            assert_bits_equal(yf1[0], yfb[r], f"row {r} of M={M}: fp32 accumulators")
            assert_bits_equal(y1[0], yb[r], f"row {r} of M={M}: bf16 outputs")
    if len(dense) == M and M <= 8:
        # the same rows in reverse order, and each row again beside row 0 in a two-row batch
        yr, yfr = _fast_rows(qo.GGML_Q4_K, wd, N, K, x[::-1], "fast_dense")
        for r in range(M):
            assert_bits_equal(yfr[M - 1 - r], yfb[r], f"row {r} of M={M}, batch reversed: fp32 accumulators")
            assert_bits_equal(yr[M - 1 - r], yb[r], f"row {r} of M={M}, batch reversed: bf16 outputs")
        for r in range(1, M):
            y2, yf2 = _fast_rows(qo.GGML_Q4_K, wd, N, K, np.stack([x[r], x[0]]), "fast_dense")
            assert_bits_equal(yf2[0], yfb[r], f"row {r} of M={M} in a two-row batch: fp32 accumulators")
            assert_bits_equal(yf2[1], yfb[0], f"row 0 of M={M} in a two-row batch: fp32 accumulators")


# Q6_K / Q8_0 / F16 through the mixed-type kernel: shapes where some waves own no blocks
# (K = 256, 768), odd block counts (1280), the largest staged K (15360; larger K is served by
# the exact kernel), ragged row counts and several activation rows.
TYPE_FAST_CASES = [(256, 6144, 1), (37, 768, 1), (100, 256, 2), (300, 1280, 1), (64, 15360, 1), (513, 2048, 3)]


@pytest.mark.parametrize("t", [qo.GGML_Q6_K, qo.GGML_Q8_0, qo.GGML_F16])
@pytest.mark.parametrize("N,K,M", TYPE_FAST_CASES)
def test_gemv_fast_types_tolerance(t, N, K, M):
    note(f"gemv fast type={t} N={N} K={K} M={M}")
    rng = np.random.default_rng(t * 1000 + N + K + M)
    raw = qo.random_weights(rng, t, N, K)
    x = qo.random_bf16(rng, (M, K))
    wd = d_u8(raw)
    y, yf = dev.gemv(t, wd, N, K, d_bf16(x), mode="fast", out_f32=True)
    acc, _ = co.gemv_ref(t, raw, N, K, x)
    w = qo.dequant_matrix(t, raw, N, K)
    xf = qo.bf16_bits_to_f32(x)
    ok, worst = qo.tolerance_gate(w, xf, h_f32(yf), rel=1e-5)
    note(f"  worst |delta| = {worst:.4f} of the 1e-5*sum|a*w| bound")
    assert ok, f"tolerance gate exceeded: worst {worst:.3f} of the 1e-5*sum|a*w| bound"
    ok, max_ulp, n_cancelled = qo.bf16_parity(h_bits(y), acc, w, xf)
    assert ok, f"bf16 outputs: {max_ulp} ulp on well-conditioned outputs ({n_cancelled} cancelled sums)"
    y2, yf2 = dev.gemv(t, wd, N, K, d_bf16(x), mode="fast", out_f32=True)
    assert np.array_equal(u32(h_f32(yf2)), u32(h_f32(yf)))


@pytest.mark.parametrize("t", [qo.GGML_Q6_K, qo.GGML_Q8_0, qo.GGML_F16])
def test_gemv_fast_types_detect_corruption(t):
    """Must-fail twin per type: one changed weight in row 3 moves that output past the gate."""
    note(f"gemv fast type={t} corruption twin")
    rng = np.random.default_rng(40 + t)
    N, K = 32, 1024
    raw = qo.random_weights(rng, t, N, K)
    x = qo.random_bf16(rng, (1, K))
    w = qo.dequant_matrix(t, raw, N, K)
    bad = raw.copy()
    rb = raw.size // N
    if t == qo.GGML_F16:
        bad[3 * rb + 2 * 100:3 * rb + 2 * 100 + 2] = np.asarray(qo.f32_to_f16_bits(np.array([3.0], np.float32)), np.uint16).view(np.uint8)
    elif t == qo.GGML_Q8_0:
        bad[3 * rb + 2 + 7] ^= 0x40
    else:
        bad[3 * rb + 128 + 5] ^= 0x30          # qh bits of one position
    _, yf = dev.gemv(t, d_u8(bad), N, K, d_bf16(x), mode="fast", out_f32=True)
    ok, _ = qo.tolerance_gate(w, qo.bf16_bits_to_f32(x), h_f32(yf))
    assert not ok


def test_gemv_fast_bf16_router_shape():
    note("gemv fast BF16 256x6144")
    rng = np.random.default_rng(11)
    wbits = qo.random_bf16(rng, (256, 6144), scale=0.02)
    x = qo.random_bf16(rng, (1, 6144))
    y, yf = dev.gemv(30, d_u8(wbits.view(np.uint8)), 256, 6144, d_bf16(x), mode="fast", out_f32=True)
    w = qo.bf16_bits_to_f32(wbits)
    ok, worst = qo.tolerance_gate(w, qo.bf16_bits_to_f32(x), h_f32(yf))
    assert ok, worst
    acc, _ = qo.gemv_ref(w, qo.bf16_bits_to_f32(x))
    assert qo.bf16_parity(h_bits(y), acc, w, qo.bf16_bits_to_f32(x))[0]


def test_gemv_fast_detects_corrupted_weights():
    """Must-fail twin: flipping one nibble moves the output beyond the gate."""
    note("gemv fast corruption twin")
    rng = np.random.default_rng(12)
    N, K = 64, 2048
    raw = qo.random_q4k_blocks(rng, N * K // 256)
    off = 5 * 144 * 8                             # row 5, block 0
    raw[off + 4:off + 16] = qo.pack_scales_q4k([32] * 8, [1] * 8)
    raw[off + 16 + 3] &= 0xF0                     # weight 3 has code 0 ...
    x = qo.random_bf16(rng, (1, K))
    x[0, 3] = qo.bf16_round_bits(np.float32(4.0))
    w = qo.dequant_q4k(raw).reshape(N, K)
    bad = raw.copy()
    bad[off + 16 + 3] |= 0x0F                     # ... and 15 in the corrupted copy
    _, yf = dev.gemv(qo.GGML_Q4_K, d_u8(bad), N, K, d_bf16(x), mode="fast", out_f32=True)
    ok, _ = qo.tolerance_gate(w, qo.bf16_bits_to_f32(x), h_f32(yf))
    assert not ok


def test_persistent_waits_complete():
    """No bounded wait of the persistent kernels gives up in normal runs: the give-up flag
    (aipu_wait_timeouts) stays clear across the single-row, row-pair, dense multi-row and MoE
    expert-leg kernels."""
    note("persistent kernels: wait give-up flag")
    dev.wait_timeouts()   # clear whatever earlier tests left
    g = torch.Generator(device="cuda")
    g.manual_seed(17)
    N = K = 6144
    w = random_weights_gpu(qo.GGML_Q4_K, N, K, g)
    x = (torch.randn((8, K), device="cuda", generator=g) * 0.5).to(torch.bfloat16)
    for m, mode in ((1, "fast"), (2, "fast"), (8, "fast"), (8, "fast_dense")):
        dev.gemv(qo.GGML_Q4_K, w, N, K, x[:m], mode=mode)
    E, H, I, topk = 16, 2048, 2048, 8
    ex = [random_weights_gpu(qo.GGML_Q4_K, E * I, H, g), random_weights_gpu(qo.GGML_Q4_K, E * I, H, g),
          random_weights_gpu(qo.GGML_Q4_K, E * H, I, g)]
    rw = (torch.randn((E, H), device="cuda", generator=g) * 0.05).to(torch.bfloat16)
    xm = (torch.randn(H, device="cuda", generator=g) * 0.05).to(torch.bfloat16)
    dev.moe_swiglu_decode(go.BF16_TYPE, rw.view(torch.uint8).reshape(-1), qo.GGML_Q4_K, *ex, E, H, I, topk, xm,
                          mode="fast")
    assert not dev.wait_timeouts()


@pytest.mark.parametrize("N,K", [(6144, 6144), (4096, 4096), (2048, 8192)])
def test_measure_gemv_variants(N, K):
    """The measurement launches (an empty kernel of the M = 1 GEMV's launch shape, its copy
    schedule alone) run to completion, write nothing, and leave no wait given up."""
    note(f"measure_gemv N={N} K={K}")
    dev.wait_timeouts()
    g = torch.Generator(device="cuda")
    g.manual_seed(N + K)
    w = random_weights_gpu(qo.GGML_Q4_K, N, K, g)
    x = torch.zeros((1, K), dtype=torch.bfloat16, device="cuda")
    for what in ("empty", "copy"):
        dev.measure_gemv(what, w, N, K, x)
    torch.cuda.synchronize()
    assert not dev.wait_timeouts()
