"""GPU parity of the pre-FFN RMSNorm (aipu_rmsnorm) and the FFN half of a MoE decoder block
(aipu_moe_layer_decode: rmsnorm -> MoE step -> residual) through the C ABI.  Reference mode is
bit-exact against the golden cases from the reference (tools/glm_model_q4k_ref.py:451-465,
:797-810) and the oracle; fast mode is checked against reference mode (RMSNorm within one
bf16 ulp) and against its own pieces run separately at the BASELINE config-2 shape."""
import os

import numpy as np
import pytest
import torch

from aipu_amd import device as dev
from oracle import glm_oracle as go
from oracle import q4k_oracle as qo

from .gpu_util import assert_bits_equal, d_bf16, d_u8, h_bits, note, random_weights_gpu

pytestmark = pytest.mark.gpu
GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "rmsnorm_cases.npz"))
Q4K = qo.GGML_Q4_K
BF16 = 30


def test_rmsnorm_golden_cases_ref():
    note("rmsnorm golden cases")
    for i in range(int(GOLD["n_cases"][0])):
        y = dev.rmsnorm(d_bf16(GOLD[f"n{i}_x"]), d_bf16(GOLD[f"n{i}_g"]), mode="ref")
        assert_bits_equal(h_bits(y), GOLD[f"n{i}_y"], f"golden case {i}")


@pytest.mark.parametrize("n", [1, 33, 4096, 4097, 6144, 12288, 20000])
def test_rmsnorm_random_ref_and_fast(n):
    note(f"rmsnorm n={n}")
    rng = np.random.default_rng(n)
    x = qo.random_bf16(rng, n)
    g = qo.random_bf16(rng, n)
    yr = h_bits(dev.rmsnorm(d_bf16(x), d_bf16(g), mode="ref"))
    assert_bits_equal(yr, go.rmsnorm(x, g), f"ref n={n}")
    yf = h_bits(dev.rmsnorm(d_bf16(x), d_bf16(g), mode="fast"))
    assert qo.bf16_ulp_distance(yf, yr).max() <= 1


def test_moe_layer_golden_ref():
    note("moe layer golden")
    k = "l0_"
    E, H, I, topk = 4, 256, 256, 2
    sh = tuple(d_u8(GOLD[k + "sh"][i]) for i in range(3))
    y, sel, sw = dev.moe_layer_decode(Q4K, d_u8(GOLD[k + "router"]), Q4K, d_u8(GOLD[k + "gate"]),
                                      d_u8(GOLD[k + "up"]), d_u8(GOLD[k + "down"]), E, H, I, topk,
                                      d_bf16(GOLD[k + "h"]), d_bf16(GOLD[k + "gamma"]), mode="ref", shared=sh)
    assert list(sel.cpu().numpy()) == list(GOLD[k + "sel"])
    assert_bits_equal(h_bits(sw), GOLD[k + "selw"], "layer sel_w")
    assert_bits_equal(h_bits(y), GOLD[k + "y"], "layer y")


def test_moe_layer_random_ref():
    note("moe layer random ref")
    E, H, I, topk = 16, 512, 256, 4
    rng = np.random.default_rng(41)
    rw = qo.random_q4k_blocks(rng, E * H // 256)
    ex = tuple(qo.random_q4k_blocks(rng, E * I * H // 256) for _ in range(3))
    sh = tuple(qo.random_q4k_blocks(rng, I * H // 256) for _ in range(3))
    h = qo.random_bf16(rng, H, scale=0.5)
    g = qo.random_bf16(rng, H)
    y, sel, sw = dev.moe_layer_decode(Q4K, d_u8(rw), Q4K, *(d_u8(a) for a in ex), E, H, I, topk, d_bf16(h),
                                      d_bf16(g), mode="ref", shared=tuple(d_u8(a) for a in sh))
    r = go.moe_layer_ref(h, g, Q4K, rw, ex, Q4K, E, H, I, topk, shared=sh)
    assert list(sel.cpu().numpy()) == list(r["sel_idx"])
    assert_bits_equal(h_bits(y), r["y"], "layer y random")


@pytest.mark.parametrize("E,H,I", [(32, 6144, 2048), (256, 6144, 2048), (16, 2304, 256), (16, 8192, 2048)])
def test_moe_layer_fast_c2_shape(E, H, I):
    """Q4_K router and a shared expert, at the config-2 expert shape (32 experts and all 256),
    an odd count of 256-blocks (H = 2304) and two block pairs per router wave (H = 8192): the
    fused call, whose router launch applies the RMSNorm itself, equals rmsnorm -> MoE step ->
    residual run as three separate calls (bitwise), and the fast RMSNorm it starts from is
    within one bf16 ulp of the reference order."""
    topk = 8
    note(f"moe layer fast E={E} H={H} I={I}")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(6 + H + E)
    ge = random_weights_gpu(Q4K, E * I, H, gen)
    ue = random_weights_gpu(Q4K, E * I, H, gen)
    de = random_weights_gpu(Q4K, E * H, I, gen)
    rw = random_weights_gpu(Q4K, E, H, gen)
    sh = (random_weights_gpu(Q4K, I, H, gen), random_weights_gpu(Q4K, I, H, gen), random_weights_gpu(Q4K, H, I, gen))
    rng = np.random.default_rng(6 + H + E)
    h = d_bf16(qo.random_bf16(rng, H, scale=0.5))
    g = d_bf16(qo.random_bf16(rng, H))
    y, sel, sw = dev.moe_layer_decode(Q4K, rw, Q4K, ge, ue, de, E, H, I, topk, h, g, mode="fast", shared=sh)
    nrm = dev.rmsnorm(h, g, mode="fast")
    f, sel2, sw2 = dev.moe_swiglu_decode(Q4K, rw, Q4K, ge, ue, de, E, H, I, topk, nrm, mode="fast", shared=sh)
    want = (h.float() + f.float()).to(torch.bfloat16)     # RNE of an exact fp32 sum of two bf16
    assert torch.equal(sel, sel2)
    assert_bits_equal(h_bits(sw), h_bits(sw2), "sel_w")
    assert_bits_equal(h_bits(y), h_bits(want), "layer = pieces")
    nr = dev.rmsnorm(h, g, mode="ref")
    assert qo.bf16_ulp_distance(h_bits(nrm), h_bits(nr)).max() <= 1


@pytest.mark.parametrize("E,H,I,gamma_off", [(3000, 2304, 256, 0), (32, 6144, 2048, 1)])
def test_moe_layer_fast_router_norm_edges(E, H, I, gamma_off):
    """The RMSNorm in the router's launch at two router tiles per CU (3,000 experts, the one-wave
    routing tail), and the separate RMSNorm launch it falls back to when gamma is not 16-B
    aligned (the norm kernel then takes its unaligned order): the fused call equals rmsnorm ->
    MoE step -> residual run as three separate calls (bitwise) either way."""
    topk = 8
    note(f"moe layer fast router norm E={E} H={H} I={I} gamma offset {gamma_off}")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(E + H)
    ge = random_weights_gpu(Q4K, E * I, H, gen)
    ue = random_weights_gpu(Q4K, E * I, H, gen)
    de = random_weights_gpu(Q4K, E * H, I, gen)
    rw = random_weights_gpu(Q4K, E, H, gen)
    sh = (random_weights_gpu(Q4K, I, H, gen), random_weights_gpu(Q4K, I, H, gen), random_weights_gpu(Q4K, H, I, gen))
    rng = np.random.default_rng(E + H)
    h = d_bf16(qo.random_bf16(rng, H, scale=0.5))
    gbuf = d_bf16(qo.random_bf16(rng, H + 8))
    g = gbuf[gamma_off:gamma_off + H]
    assert (g.data_ptr() % 16 == 0) == (gamma_off == 0)
    y, sel, sw = dev.moe_layer_decode(Q4K, rw, Q4K, ge, ue, de, E, H, I, topk, h, g, mode="fast", shared=sh)
    nrm = dev.rmsnorm(h, g, mode="fast")
    f, sel2, sw2 = dev.moe_swiglu_decode(Q4K, rw, Q4K, ge, ue, de, E, H, I, topk, nrm, mode="fast", shared=sh)
    want = (h.float() + f.float()).to(torch.bfloat16)     # RNE of an exact fp32 sum of two bf16
    assert torch.equal(sel, sel2)
    assert_bits_equal(h_bits(sw), h_bits(sw2), "sel_w")
    assert_bits_equal(h_bits(y), h_bits(want), "layer = pieces")


def test_moe_layer_fast_persistent_legs():
    """A layer without a shared expert and with a bf16 router runs the persistent expert legs,
    the residual added in the down leg's epilogue: the fused call equals rmsnorm -> MoE step ->
    residual run as three separate calls (bitwise)."""
    E, H, I, topk = 16, 2048, 2048, 4
    note("moe layer fast persistent legs")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(16)
    ge = random_weights_gpu(Q4K, E * I, H, gen)
    ue = random_weights_gpu(Q4K, E * I, H, gen)
    de = random_weights_gpu(Q4K, E * H, I, gen)
    rng = np.random.default_rng(16)
    rw = d_u8(qo.random_bf16(rng, (E, H), scale=0.05).view(np.uint8).reshape(-1))
    h = d_bf16(qo.random_bf16(rng, H, scale=0.5))
    g = d_bf16(qo.random_bf16(rng, H))
    y, sel, sw = dev.moe_layer_decode(BF16, rw, Q4K, ge, ue, de, E, H, I, topk, h, g, mode="fast")
    nrm = dev.rmsnorm(h, g, mode="fast")
    f, sel2, sw2 = dev.moe_swiglu_decode(BF16, rw, Q4K, ge, ue, de, E, H, I, topk, nrm, mode="fast")
    want = (h.float() + f.float()).to(torch.bfloat16)     # RNE of an exact fp32 sum of two bf16
    assert torch.equal(sel, sel2)
    assert_bits_equal(h_bits(sw), h_bits(sw2), "sel_w")
    assert_bits_equal(h_bits(y), h_bits(want), "layer = pieces")


def test_glm_mirror_rmsnorm_ffn_block_lm_head():
    """The reference-interface mirrors (aipu_amd/glm_model_q4k_ref.py): rmsnorm and ffn_block
    on the golden cases, matmul_bf16_dot on the 7-way order case, lm_head vs the oracle."""
    from aipu_amd import glm_model_q4k_ref as gm
    from oracle import c_oracle as co
    note("glm mirror rmsnorm / ffn_block / lm_head")
    gm.set_mode("ref")
    x = list(qo.bf16_bits_to_f32(GOLD["n5_x"]))
    g = list(qo.bf16_bits_to_f32(GOLD["n5_g"]))
    y = gm.rmsnorm(x, g)
    assert_bits_equal(np.asarray(y, np.float32).view(np.uint32) >> 16, GOLD["n5_y"], "mirror rmsnorm")
    k = "l0_"
    E, D = 4, 256
    cfg = gm.Config(MODEL_DIM=D, N_EXPERT=E, TOPK=2, INTER_MOE=D)
    Wg = gm.QW.from_ggml(GOLD[k + "router"], E, D)
    per = D * D // 256 * 144
    Mg = [gm.QW.from_ggml(GOLD[k + "gate"][e * per:(e + 1) * per], D, D) for e in range(E)]
    Mu = [gm.QW.from_ggml(GOLD[k + "up"][e * per:(e + 1) * per], D, D) for e in range(E)]
    Md = [gm.QW.from_ggml(GOLD[k + "down"][e * per:(e + 1) * per], D, D) for e in range(E)]
    SH = [gm.QW.from_ggml(GOLD[k + "sh"][i], D, D) for i in range(3)]
    h = list(qo.bf16_bits_to_f32(GOLD[k + "h"]))
    gam = list(qo.bf16_bits_to_f32(GOLD[k + "gamma"]))
    yl, sel, sw = gm.ffn_block(cfg, h, gam, Wg, Mg, Mu, Md, *SH)
    assert sel == list(GOLD[k + "sel"])
    assert_bits_equal(np.asarray(yl, np.float32).view(np.uint32) >> 16, GOLD[k + "y"], "mirror ffn_block")
    ones = [1.0] * 14
    w = [0.0] * 14
    w[0], w[7], w[1] = 2.0 ** 30, -(2.0 ** 30), 1.0
    assert float(gm.matmul_bf16_dot(ones, w)) == 1.0
    rng = np.random.default_rng(12)
    Wb = qo.random_bf16(rng, (50, 100))
    xb = qo.random_bf16(rng, 100)
    logits, lbits, am = gm.lm_head(list(qo.bf16_bits_to_f32(xb)), [list(qo.bf16_bits_to_f32(r)) for r in Wb])
    le, ae = co.lm_head(Wb, xb)
    assert lbits == [int(v) for v in le] and am == ae


def _random_layer_cases(n=8, seed=1808):
    """Seeded FFN-half shapes: E = topk..64, H = 256..4096, I = 256..1536, top-1..8, bf16 or
    Q4_K router, with or without the shared expert."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        topk = int(rng.integers(1, 9))
        out.append((int(rng.integers(topk, 65)), 256 * int(rng.integers(1, 17)), 256 * int(rng.integers(1, 7)), topk,
                    BF16 if rng.integers(0, 2) else Q4K, bool(rng.integers(0, 2))))
    return out


@pytest.mark.parametrize("mode", ["ref", "fast"])
@pytest.mark.parametrize("E,H,I,topk,router_type,shared", _random_layer_cases())
def test_moe_layer_random_shapes(E, H, I, topk, router_type, shared, mode):
    """The FFN half at seeded random shapes: ref mode bit-exact against the oracle; fast mode
    equal (bitwise) to rmsnorm -> MoE step -> residual run as three separate calls."""
    note(f"moe layer random {mode} E={E} H={H} I={I} topk={topk} router={router_type} shared={shared}")
    rng = np.random.default_rng(E * 7 + H + I * 3 + topk)
    if router_type == BF16:
        rw = qo.random_bf16(rng, (E, H), scale=0.05).view(np.uint8).reshape(-1)
    else:
        rw = qo.random_q4k_blocks(rng, E * H // 256)
    ex = tuple(qo.random_q4k_blocks(rng, E * I * H // 256) for _ in range(3))
    sh = tuple(qo.random_q4k_blocks(rng, I * H // 256) for _ in range(3)) if shared else None
    h = qo.random_bf16(rng, H, scale=0.5)
    g = qo.random_bf16(rng, H)
    rwd, exd = d_u8(rw), tuple(d_u8(a) for a in ex)
    shd = tuple(d_u8(a) for a in sh) if sh else None
    y, sel, sw = dev.moe_layer_decode(router_type, rwd, Q4K, *exd, E, H, I, topk, d_bf16(h), d_bf16(g), mode=mode,
                                      shared=shd)
    if mode == "ref":
        r = go.moe_layer_ref(h, g, router_type, rw, ex, Q4K, E, H, I, topk, shared=sh)
        assert list(sel.cpu().numpy()) == list(r["sel_idx"])
        assert_bits_equal(h_bits(y), r["y"], "layer y")
        return
    hd = d_bf16(h)
    nrm = dev.rmsnorm(hd, d_bf16(g), mode="fast")
    f, sel2, sw2 = dev.moe_swiglu_decode(router_type, rwd, Q4K, *exd, E, H, I, topk, nrm, mode="fast", shared=shd)
    want = (hd.float() + f.float()).to(torch.bfloat16)   # RNE of an exact fp32 sum of two bf16
    assert torch.equal(sel, sel2)
    assert_bits_equal(h_bits(sw), h_bits(sw2), "sel_w")
    assert_bits_equal(h_bits(y), h_bits(want), "layer = pieces")
