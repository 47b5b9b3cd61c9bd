"""Pins of the RMSNorm / decoder-FFN-half oracle (oracle/glm_oracle.py recip_fp32_bits,
rmsnorm, moe_layer_ref): the golden cases tests/golden/make_golden.py wrote from the
reference's own rmsnorm (tools/glm_model_q4k_ref.py:451-465), _recip_fp32 (:434-449) and the
FFN half of decoder_block (:797-810) built from its moe_router / swiglu_expert; recip_fp32
against the correctly rounded 1/n; closed forms of rmsnorm."""
import os
from fractions import Fraction

import numpy as np

from oracle import glm_oracle as go
from oracle import q4k_oracle as qo

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "rmsnorm_cases.npz"))


def _rne_f32_bits(fr):
    """Correctly rounded (half to even) fp32 bits of a positive normal rational."""
    e = fr.numerator.bit_length() - fr.denominator.bit_length()
    if Fraction(2) ** e > fr:
        e -= 1
    m = fr / Fraction(2) ** e * (1 << 23)                     # in [2^23, 2^24)
    q, r = divmod(m.numerator, m.denominator)
    if 2 * r > m.denominator or (2 * r == m.denominator and q & 1):
        q += 1
    if q == 1 << 24:
        q >>= 1
        e += 1
    return ((e + 127) << 23) | (q & 0x7FFFFF)


def test_recip_golden():
    for n, b in zip(GOLD["recip_n"], GOLD["recip_bits"]):
        assert go.recip_fp32_bits(int(n)) == int(b), n


def test_recip_is_correctly_rounded_below_2_24():
    """For n < 2^24 the rounding bit sits far above floor(2^60/n)'s lost fraction, so the
    restated rule equals round-to-nearest-even of 1/n (checked on 1..20000 and a sweep)."""
    ns = list(range(1, 20001)) + [int(v) for v in np.random.default_rng(3).integers(20001, 1 << 24, 3000)]
    for n in ns:
        assert go.recip_fp32_bits(n) == _rne_f32_bits(Fraction(1, n)), n


def test_rmsnorm_golden_cases():
    for i in range(int(GOLD["n_cases"][0])):
        got = go.rmsnorm(GOLD[f"n{i}_x"], GOLD[f"n{i}_g"])
        np.testing.assert_array_equal(got, GOLD[f"n{i}_y"], err_msg=f"case {i}")


def test_rmsnorm_closed_forms():
    """x = c (n a power of two, gamma = 1): sumsq = n c^2 exactly, mean = c^2, so y =
    bf16(c * rsqrt(c^2 + 1e-5)); all-zero x gives zeros; gamma = 0 gives (signed) zeros."""
    for c, n in ((1.0, 64), (0.5, 256), (3.0, 1024)):
        x = qo.bf16_round_bits(np.full(n, c, np.float32))
        g = qo.bf16_round_bits(np.ones(n, np.float32))
        inv = go.fp32_rsqrt(go.fadd(np.float32(c * c), qo.bits_f32(go.RMS_EPS_BITS)))
        want = qo.bf16_round_bits(np.float32(np.float32(c) * inv))
        assert np.all(go.rmsnorm(x, g) == want)
    z = np.zeros(32, np.uint16)
    assert np.all(go.rmsnorm(z, qo.bf16_round_bits(np.ones(32, np.float32))) == 0)


def test_moe_layer_golden():
    k = "l0_"
    E, H, I, topk = 4, 256, 256, 2
    sh = tuple(GOLD[k + "sh"][i] for i in range(3))
    r = go.moe_layer_ref(GOLD[k + "h"], GOLD[k + "gamma"], qo.GGML_Q4_K, GOLD[k + "router"],
                         (GOLD[k + "gate"], GOLD[k + "up"], GOLD[k + "down"]), qo.GGML_Q4_K, E, H, I, topk,
                         shared=sh)
    np.testing.assert_array_equal(r["nrm"], GOLD[k + "nrm"])
    assert list(r["sel_idx"]) == list(GOLD[k + "sel"])
    np.testing.assert_array_equal(r["sel_w"], GOLD[k + "selw"])
    np.testing.assert_array_equal(r["fbuf"], GOLD[k + "fbuf"])
    np.testing.assert_array_equal(r["y"], GOLD[k + "y"])
