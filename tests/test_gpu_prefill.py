"""GPU parity of the matrix-core prefill GEMM (aipu_gemm_prefill) through the C ABI.

Tolerance mode: the fp32 accumulators must satisfy |acc - exact| <= 1e-5 * sum|a*w| against
the fp64 product of the exactly dequantised weights (tools/q4k_ref.py:39-65), and the bf16
outputs must be within 1 ulp of the reference-order result (tools/q4k_ref.py:86-92) wherever
the sum is well conditioned.  Shapes cover ragged M and N, one and odd numbers of
super-blocks, activation rows spanning the whole bf16 exponent range (the per-row fp16
scaling), weight blocks with d = 0, dmin = 0 and subnormal scales, and the full BASELINE
config-4 shape (M=512, K=6144, N=16384) on sampled columns.
"""
import numpy as np
import pytest
import torch

from aipu_amd import device as dev
from oracle import c_oracle as co
from oracle import q4k_oracle as qo

from .gpu_util import assert_bits_equal, d_bf16, d_u8, h_bits, h_f32, note, random_weights_gpu

pytestmark = pytest.mark.gpu
Q4K = qo.GGML_Q4_K


def _prefill(raw, N, K, x_bits, ws=None):
    y, yf = dev.gemm_prefill(Q4K, d_u8(raw), N, K, d_bf16(x_bits), workspace=ws, out_f32=True)
    return h_bits(y), h_f32(yf)


def _check(raw, N, K, x_bits, y, yf, what):
    wdeq = qo.dequant_q4k(raw).reshape(N, K)
    xf = qo.bf16_bits_to_f32(x_bits)
    ok, worst = qo.tolerance_gate(wdeq, xf, yf)
    assert ok, f"{what}: accumulators outside 1e-5*sum|a*w| (worst ratio {worst:.3g})"
    assert_bits_equal(y, qo.bf16_round_bits(yf), f"{what}: bf16 output != bf16(acc)")
    acc, _ = co.gemv_ref(Q4K, raw, N, K, x_bits)
    okb, ulp, ncanc = qo.bf16_parity(y, acc, wdeq, xf)
    assert okb, f"{what}: bf16 outputs {ulp} ulp from reference order ({ncanc} cancelled sums)"
    return worst


@pytest.mark.parametrize("M,N,K", [(130, 300, 512), (128, 256, 256), (1, 17, 768), (257, 520, 1024),
                                   (64, 64, 2048), (200, 1000, 1536),
                                   # the largest K of the one-pass staging kernel, and past it the
                                   # two-kernel staging (row exponents, then packing)
                                   (5, 24, 32768), (3, 40, 33024)])
def test_prefill_tolerance_shapes(M, N, K):
    note(f"prefill M={M} N={N} K={K}")
    rng = np.random.default_rng(M * 7 + N * 3 + K)
    raw = qo.random_q4k_blocks(rng, N * K // 256)
    x = qo.random_bf16(rng, (M, K))
    y, yf = _prefill(raw, N, K, x)
    _check(raw, N, K, x, y, yf, f"M={M} N={N} K={K}")


def test_prefill_activation_range():
    """Rows at very different magnitudes (2^-120 .. 2^100), an all-zero row, a row mixing huge
    and tiny values, negative zeros: the per-row power-of-two scaling keeps them exact."""
    note("prefill activation exponent range")
    rng = np.random.default_rng(77)
    N, K = 96, 768
    raw = qo.random_q4k_blocks(rng, N * K // 256)
    rows = []
    for e in (-120, -60, -20, -3, 0, 7, 20, 60, 100):
        rows.append(rng.standard_normal(K) * 2.0 ** e)
    rows.append(np.zeros(K))
    mixed = rng.standard_normal(K)
    mixed[::7] *= 2.0 ** 40
    mixed[1::5] *= 2.0 ** -40
    rows.append(mixed)
    nz = rng.standard_normal(K)
    nz[::3] = -0.0
    rows.append(nz)
    x = qo.bf16_round_bits(np.stack(rows).astype(np.float32))
    y, yf = _prefill(raw, N, K, x)
    _check(raw, N, K, x, y, yf, "activation range")
    assert np.all(yf[9] == 0.0), "all-zero activation row must give exact zeros"


def test_prefill_weight_edge_blocks():
    """Blocks with d = 0, dmin = 0, subnormal d/dmin, scales all 0 and all 63."""
    note("prefill weight edge blocks")
    rng = np.random.default_rng(78)
    N, K, M = 40, 1024, 70
    raw = qo.random_q4k_blocks(rng, N * K // 256).reshape(-1, 144)
    hdr = raw[:, 0:4].copy().view(np.uint16)
    hdr[0::5, 0] = 0x0000          # d = 0
    hdr[1::5, 1] = 0x0000          # dmin = 0
    hdr[2::5, 0] = 0x0001          # smallest subnormal d
    hdr[3::5, :] = 0x8000          # -0
    raw[:, 0:4] = hdr.view(np.uint8)
    raw[4::7, 4:16] = 0xFF         # every 6-bit scale and min = 63
    raw[5::7, 4:16] = 0x00         # every scale and min = 0
    raw = raw.reshape(-1)
    x = qo.random_bf16(rng, (M, K))
    y, yf = _prefill(raw, N, K, x)
    _check(raw, N, K, x, y, yf, "weight edge blocks")


def test_prefill_workspace_reuse_and_determinism():
    """A workspace sized for a larger M serves a smaller call; repeated calls are bitwise equal."""
    note("prefill workspace reuse")
    rng = np.random.default_rng(79)
    N, K = 320, 1024
    raw = qo.random_q4k_blocks(rng, N * K // 256)
    ws = dev.prefill_workspace(400, K, "cuda")
    x1 = qo.random_bf16(rng, (400, K))
    x2 = qo.random_bf16(rng, (150, K))
    y1, f1 = _prefill(raw, N, K, x1, ws)
    y2, f2 = _prefill(raw, N, K, x2, ws)
    y2b, f2b = _prefill(raw, N, K, x2)
    assert_bits_equal(y2, y2b, "workspace reuse")
    assert_bits_equal(f2.view(np.uint32), f2b.view(np.uint32), "workspace reuse f32")
    y1b, f1b = _prefill(raw, N, K, x1, ws)
    assert_bits_equal(f1.view(np.uint32), f1b.view(np.uint32), "determinism")
    _check(raw, N, K, x2, y2, f2, "M=150 after M=400")


def test_prefill_config4_shape_sampled():
    """BASELINE config 4 (M=512, K=6144, N=16384), weights generated on the device; 48 sampled
    weight rows (all 512 activation rows) checked against fp64 and reference order."""
    note("prefill config-4 shape")
    M, K, N = 512, 6144, 16384
    gen = torch.Generator(device="cuda")
    gen.manual_seed(4)
    w = random_weights_gpu(Q4K, N, K, gen)
    x = (torch.randn((M, K), device="cuda", generator=gen)).to(torch.bfloat16)
    y, yf = dev.gemm_prefill(Q4K, w, N, K, x, out_f32=True)
    torch.cuda.synchronize()
    rng = np.random.default_rng(5)
    cols = np.sort(rng.choice(N, 48, replace=False))
    cols[0], cols[-1] = 0, N - 1
    rb = K // 256 * 144
    raw = w.view(N, rb)[torch.from_numpy(cols).cuda()].cpu().numpy().reshape(-1)
    xb = h_bits(x)
    ys = h_bits(y)[:, cols]
    yfs = h_f32(yf)[:, cols]
    worst = _check(raw, len(cols), K, xb, ys, yfs, "config-4 sampled")
    note(f"config-4 worst tolerance ratio {worst:.3g}")


def test_prefill_detects_corrupted_weights():
    """Must-fail twin: one nibble of row 5 changed from 0 to 15 (under a large scale, against an
    activation of 4 in every row) moves column 5 of every output row past the tolerance gate."""
    note("prefill corruption twin")
    rng = np.random.default_rng(501)
    M, N, K = 64, 96, 768
    raw = qo.random_q4k_blocks(rng, N * K // 256)
    off = 5 * 144 * (K // 256)                      # row 5, block 0
    raw[off + 4:off + 16] = qo.pack_scales_q4k([32] * 8, [1] * 8)
    raw[off + 16 + 3] &= 0xF0                       # weight 3 has code 0 ...
    x = qo.random_bf16(rng, (M, K))
    x[:, 3] = qo.bf16_round_bits(np.float32(4.0))
    wdeq = qo.dequant_q4k(raw).reshape(N, K)
    bad = raw.copy()
    bad[off + 16 + 3] |= 0x0F                       # ... and 15 in the corrupted copy
    y, yf = _prefill(bad, N, K, x)
    ok, _ = qo.tolerance_gate(wdeq, qo.bf16_bits_to_f32(x), yf)
    assert not ok, "the tolerance gate passed a corrupted weight"
    # the clean weights pass the same gate (the twin's other half)
    y, yf = _prefill(raw, N, K, x)
    assert qo.tolerance_gate(wdeq, qo.bf16_bits_to_f32(x), yf)[0]


def _random_prefill_cases(n=10, seed=1606):
    """Seeded (M, N, K): M = 1..600 rows, N = 1..1200 weight rows, K = 256..8192."""
    rng = np.random.default_rng(seed)
    return [(int(rng.integers(1, 601)), int(rng.integers(1, 1201)), 256 * int(rng.integers(1, 33))) for _ in range(n)]


@pytest.mark.parametrize("M,N,K", _random_prefill_cases())
def test_prefill_random_shapes(M, N, K):
    """The prefill GEMM at seeded random shapes (ragged M and N tiles, any super-block count)
    meets the accumulator gate and the bf16 1-ulp bound."""
    note(f"prefill random M={M} N={N} K={K}")
    rng = np.random.default_rng(M * 11 + N * 5 + K)
    raw = qo.random_q4k_blocks(rng, N * K // 256)
    x = qo.random_bf16(rng, (M, K))
    y, yf = _prefill(raw, N, K, x)
    _check(raw, N, K, x, y, yf, f"M={M} N={N} K={K}")
