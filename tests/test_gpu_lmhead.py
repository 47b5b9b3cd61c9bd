"""GPU parity of the bf16 LM head + argmax (aipu_lm_head) through the C ABI: bit-exact
against the C oracle (tools/glm_model_q4k_ref.py:476-486 summation order, :826-834 argmax
with bf16_gt :138-148), including the full vocabulary x MODEL_DIM shape (154,880 x 6,144,
1.9 GB of bf16 rows) checked on every row.

Shapes cover K below, at and between the chunk sizes of both kernels (448 bf16 per chunk for
K <= 6720, 224 for the lane-per-row kernel used above that; ragged tails), vocabularies that end
inside a wave or a workgroup, the order-sensitive cases the oracle is
pinned with, and argmax edge cases (ties, +-0, infinities, NaNs, an all -inf vocabulary).
"""
import numpy as np
import pytest
import torch

from aipu_amd import _lib
from aipu_amd import device as dev
from oracle import c_oracle as co
from oracle import glm_oracle as go
from oracle import q4k_oracle as qo

from .gpu_util import assert_bits_equal, d_bf16, h_bits, note

pytestmark = pytest.mark.gpu


def _run(w_bits, x_bits):
    lg, am = dev.lm_head(d_bf16(w_bits), d_bf16(x_bits))
    return h_bits(lg), int(am.cpu().numpy()[0])


def _check(w_bits, x_bits, what):
    got, am = _run(w_bits, x_bits)
    exp, eam = co.lm_head(w_bits, x_bits)
    assert_bits_equal(got, exp, f"{what}: logits")
    assert am == eam, f"{what}: argmax {am} != {eam}"
    assert am == go.lm_argmax(got), f"{what}: argmax of the device logits"


@pytest.mark.parametrize("V,K", [(1, 8), (63, 56), (64, 64), (65, 112), (129, 152), (200, 104),
                                 (1000, 6144), (777, 2048), (130, 4096 + 48), (37, 448), (36, 6720),
                                 # K > 6720 runs the lane-per-row kernel
                                 (300, 6728), (65, 8192), (130, 12288 + 40)])
def test_lm_head_shapes(V, K):
    note(f"lm_head V={V} K={K}")
    rng = np.random.default_rng(V * 31 + K)
    w = qo.random_bf16(rng, (V, K))
    x = qo.random_bf16(rng, K)
    _check(w, x, f"V={V} K={K}")


def test_lm_head_order_cases():
    """The hand-derived order cases of the oracle pins, padded with zero products to K=16:
    the 7-way interleave (exactly 1 where a sequential sum gives 0) and the add tree."""
    note("lm_head order cases")
    K = 16
    w = np.zeros((3, K), np.float32)
    w[0, 0], w[0, 7], w[0, 1] = 2.0 ** 30, -(2.0 ** 30), 1.0
    w[1, :7] = [2.0 ** 30, 1.0, -(2.0 ** 30), 1.0, 1.0, 0.0, 0.0]
    w[2, :7] = [-(2.0 ** 30), 0.0, 0.0, 0.0, 2.0 ** 30, 64.0, 64.0]
    x = np.zeros(K, np.float32)
    x[:14] = 1.0
    wb, xb = qo.bf16_round_bits(w), qo.bf16_round_bits(x)
    # row 1 and 2 only use k < 7, but x[7..13] = 1 meets w = 0 there: products +0
    got, _ = _run(wb, xb)
    assert got.tolist() == [0x3F80, 0x3F80, 0x0000]
    _check(wb, xb, "order cases")


ARGMAX_CASES = [
    ([0x3F80, 0x4000, 0x4000, 0x3F80], 1),
    ([0xFF80, 0xFF80, 0xFF80], 0),
    ([0xFF80, 0xFF80, 0xBF80], 2),
    ([0x8000, 0x0000], 0),
    ([0xBF80, 0x8000, 0x0000], 1),
    ([0x3F80, 0x7F80], 1),
    ([0xC000, 0xBF80, 0xC040], 1),
]


@pytest.mark.parametrize("logits,expect", ARGMAX_CASES)
def test_lm_head_argmax_cases(logits, expect):
    """x = e0 and W[v][0] = the wanted logit, so logits[v] is exactly that value."""
    note(f"lm_head argmax {logits}")
    K = 8
    V = len(logits)
    w = np.zeros((V, K), np.uint16)
    w[:, 0] = logits
    x = np.zeros(K, np.uint16)
    x[0] = 0x3F80
    got, am = _run(w, x)
    assert got.tolist() == [l if (l & 0x7FFF) else 0 for l in logits]   # -0 * 1 + 0 -> +0
    assert am == expect


def test_lm_head_argmax_across_waves():
    """Maximum ties spread over several 64-row waves and in the last, partial wave: the
    lowest index must win; then a unique maximum in the last row."""
    note("lm_head argmax across waves")
    V, K = 64 * 37 + 5, 16
    w = np.full((V, K), 0, np.uint16)
    w[:, 0] = 0xBF80                       # -1 everywhere
    for v in (2360, 900, 1500, V - 1):
        w[v, 0] = 0x4040                   # 3.0
    x = np.zeros(K, np.uint16)
    x[0] = 0x3F80
    _, am = _run(w, x)
    assert am == 900
    w[V - 1, 0] = 0x4080                   # 4.0
    _, am = _run(w, x)
    assert am == V - 1


def test_lm_head_logits_only_and_argmax_only():
    note("lm_head optional outputs")
    rng = np.random.default_rng(9)
    V, K = 300, 200
    w = d_bf16(qo.random_bf16(rng, (V, K)))
    x = d_bf16(qo.random_bf16(rng, K))
    lg, am = dev.lm_head(w, x)
    lg2, none = dev.lm_head(w, x, argmax=False)
    none2, am2 = dev.lm_head(w, x, logits=False)
    assert none is None and none2 is None
    assert_bits_equal(h_bits(lg2), h_bits(lg), "logits only")
    assert int(am2.cpu()[0]) == int(am.cpu()[0])


def test_lm_head_full_vocabulary():
    """The F4 shape: vocabulary 154,880 x MODEL_DIM 6,144 bf16 rows (1.9 GB), weights drawn on
    the device; every logit bit-exact against the C oracle, argmax equal."""
    V, K = 154880, 6144
    note(f"lm_head full vocabulary V={V} K={K}")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(11)
    w = (torch.randn((V, K), device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
    x = torch.randn(K, device="cuda", generator=gen).to(torch.bfloat16)
    lg, am = dev.lm_head(w, x)
    torch.cuda.synchronize()
    wb = h_bits(w)
    del w
    exp, eam = co.lm_head(wb, h_bits(x))
    assert_bits_equal(h_bits(lg), exp, "full vocabulary logits")
    assert int(am.cpu()[0]) == eam


def test_lm_head_abi_rejects():
    note("lm_head argument checks")
    w = torch.zeros((4, 12), dtype=torch.bfloat16, device="cuda")
    x = torch.zeros(12, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(_lib.AipuError):
        dev.lm_head(w, x)          # K = 12 is not a multiple of 8


def test_lm_head_detects_corrupted_row():
    """Must-fail twin: one bf16 weight of row 17 raised to 8.0 against an activation of 8.0
    changes that logit and makes row 17 the argmax, so both bit-exact checks fail."""
    note("lm_head corruption twin")
    rng = np.random.default_rng(901)
    V, K = 300, 1024
    w = qo.random_bf16(rng, (V, K), scale=0.02)
    x = qo.random_bf16(rng, K)
    x[10] = qo.bf16_round_bits(np.float32(8.0))
    bad = w.copy()
    bad[17, 10] = qo.bf16_round_bits(np.float32(8.0))
    got, am = _run(bad, x)
    exp, eam = co.lm_head(w, x)
    assert not np.array_equal(got, exp), "logits of a corrupted head equal the oracle's"
    assert am == 17 and eam != 17, (am, eam)
    _check(w, x, "clean twin")


def _random_lm_cases(n=10, seed=1707):
    """Seeded (V, K): V = 1..5000 vocabulary rows, K = 8..16384 in steps of 8 (both kernels,
    ragged chunk tails)."""
    rng = np.random.default_rng(seed)
    return [(int(rng.integers(1, 5001)), 8 * int(rng.integers(1, 2049))) for _ in range(n)]


@pytest.mark.parametrize("V,K", _random_lm_cases())
def test_lm_head_random_shapes(V, K):
    note(f"lm_head random V={V} K={K}")
    rng = np.random.default_rng(V * 17 + K)
    w = qo.random_bf16(rng, (V, K))
    x = qo.random_bf16(rng, K)
    _check(w, x, f"V={V} K={K}")
