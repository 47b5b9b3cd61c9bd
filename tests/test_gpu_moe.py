"""GPU parity for the MoE decode path through the C ABI: router tail (golden cases + ties),
SwiGLU expert (golden cases), the whole MoE step in reference order (bit-exact vs the
oracle) and in fast mode (routing = the reference tail of the step's own logits, those logits
within the reference order's rounding, h and y within a two-stage bound around exact fp64
arithmetic), mixed-type tiles, and the reference-interface mirrors."""
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
Q4K = qo.GGML_Q4_K
BF16 = 30


# ---------------------------------------------------------------- router tail
def test_router_golden_cases():
    note("router golden")
    rc = np.load(os.path.join(GOLD, "router_cases.npz"))
    for k in sorted({k.rsplit("_", 1)[0] for k in rc.files}):
        E, topk = (int(v) for v in rc[k + "_E"])
        logits = dev.gemv(Q4K, d_u8(rc[k + "_w"]), E, 256, d_bf16(rc[k + "_x"][None]), mode="ref")
        sel, sw, gates = dev.router_topk(logits.reshape(-1), topk, return_gates=True)
        assert np.array_equal(sel.cpu().numpy(), rc[k + "_sel"]), k
        assert_bits_equal(h_bits(sw), rc[k + "_selw"], k)
        assert_bits_equal(h_bits(gates), rc[k + "_gate"], k)


@pytest.mark.parametrize("E,topk", [(256, 8), (64, 6), (4096, 32), (5, 5), (1, 1)])
def test_router_random_with_ties(E, topk):
    note(f"router E={E} topk={topk}")
    rng = np.random.default_rng(E * 31 + topk)
    # coarse logits -> many exact gate ties
    logits = qo.bf16_round_bits((rng.integers(-8, 9, E) * 0.25).astype(np.float32))
    sel, sw, gates = dev.router_topk(d_bf16(logits), topk, return_gates=True)
    es, ew, eg = go.router_tail(logits, topk)
    assert np.array_equal(sel.cpu().numpy(), es)
    assert_bits_equal(h_bits(sw), ew, "sel_w")
    assert_bits_equal(h_bits(gates), eg, "gates")


# ----------------------------------------------------------------- SwiGLU
def test_swiglu_golden_cases():
    note("swiglu golden")
    s = np.load(os.path.join(GOLD, "swiglu_cases.npz"))
    for c in range(2):
        y = dev.swiglu_expert(Q4K, d_u8(s[f"c{c}_wg"]), d_u8(s[f"c{c}_wu"]), d_u8(s[f"c{c}_wd"]), 256, 256,
                              d_bf16(s[f"c{c}_x"]), mode="ref")
        assert_bits_equal(h_bits(y), s[f"c{c}_y"], f"swiglu case {c}")


def test_swiglu_fast_vs_ref():
    note("swiglu fast 6144/2048")
    rng = np.random.default_rng(21)
    H, I = 6144, 2048
    wg = qo.random_q4k_blocks(rng, I * H // 256)
    wu = qo.random_q4k_blocks(rng, I * H // 256)
    wd = qo.random_q4k_blocks(rng, H * I // 256)
    x = qo.random_bf16(rng, H, scale=0.05)
    yr, hr = dev.swiglu_expert(Q4K, d_u8(wg), d_u8(wu), d_u8(wd), H, I, d_bf16(x), mode="ref", return_h=True)
    yo, ho = go.swiglu_expert(x, wg, wu, wd, Q4K, H, I)
    assert_bits_equal(h_bits(yr), yo, "swiglu ref vs oracle")
    assert_bits_equal(h_bits(hr), ho, "h ref vs oracle")
    yf, hf = dev.swiglu_expert(Q4K, d_u8(wg), d_u8(wu), d_u8(wd), H, I, d_bf16(x), mode="fast", return_h=True)
    assert qo.bf16_ulp_distance(h_bits(hf), ho).max() <= 4
    wdd = qo.dequant_q4k(wd).reshape(H, I)
    hv = qo.bf16_bits_to_f32(ho).astype(np.float64)
    mag = np.abs(wdd) @ np.abs(hv)
    err = np.abs(qo.bf16_bits_to_f32(h_bits(yf)).astype(np.float64) - qo.bf16_bits_to_f32(yo))
    ulp = np.abs(qo.bf16_bits_to_f32(yo).astype(np.float64)) * 2.0 ** -7
    assert np.all(err <= 2.0 ** -7 * mag + 2 * ulp)


# ------------------------------------------------------------------ MoE step
def _moe_case(rng, E, H, I, router_type, shared):
    if router_type == BF16:
        rw = qo.random_bf16(rng, (E, H), scale=0.05).view(np.uint8).reshape(-1)
    else:
        rw = qo.random_q4k_blocks(rng, E * H // 256)
    ge = qo.random_q4k_blocks(rng, E * I * H // 256)
    ue = qo.random_q4k_blocks(rng, E * I * H // 256)
    de = qo.random_q4k_blocks(rng, E * H * I // 256)
    sh = None
    if shared:
        sh = (qo.random_q4k_blocks(rng, I * H // 256), qo.random_q4k_blocks(rng, I * H // 256),
              qo.random_q4k_blocks(rng, H * I // 256))
    x = qo.random_bf16(rng, H, scale=0.05)
    return rw, (ge, ue, de), sh, x


@pytest.mark.parametrize("router_type,shared,topk", [(BF16, False, 4), (Q4K, True, 4), (BF16, True, 8)])
def test_moe_ref_bitexact(router_type, shared, topk):
    E, H, I = 16, 512, 256
    note(f"moe ref router={router_type} shared={shared} topk={topk}")
    rng = np.random.default_rng(topk * 10 + shared)
    rw, ex, sh, x = _moe_case(rng, E, H, I, router_type, shared)
    shd = tuple(d_u8(a) for a in sh) if sh else None
    y, sel, sw = dev.moe_swiglu_decode(router_type, d_u8(rw), Q4K, d_u8(ex[0]), d_u8(ex[1]), d_u8(ex[2]), E, H, I,
                                       topk, d_bf16(x), mode="ref", shared=shd)
    r = go.moe_decode_ref(x, router_type, rw, ex, Q4K, E, H, I, topk, shared=sh)
    assert np.array_equal(sel.cpu().numpy(), r["sel_idx"])
    assert_bits_equal(h_bits(sw), r["sel_w"], "sel_w")
    assert_bits_equal(h_bits(y), r["y"], "y")


@pytest.mark.parametrize("router_type,shared,topk", [(BF16, False, 4), (Q4K, True, 4), (Q4K, True, 8),
                                                    (BF16, True, 7)])
def test_moe_fast_small(router_type, shared, topk):
    """topk = 8 with the shared expert is nine slots: the matrix-core down leg runs as two
    launches handing the fp32 running sum over (routed slots, then the shared slot)."""
    E, H, I = 16, 512, 256
    note(f"moe fast small router={router_type} shared={shared}")
    rng = np.random.default_rng(77 + shared + 100 * topk)
    rw, ex, sh, x = _moe_case(rng, E, H, I, router_type, shared)
    shd = tuple(d_u8(a) for a in sh) if sh else None
    y, sel, sw, lg, hw = _fast_step(router_type, rw, tuple(d_u8(a) for a in ex), E, H, I, topk, x, shd)
    es, ew = _check_routing(router_type, rw, E, H, x, topk, sel, sw, lg)
    _check_moe_tight(y, hw, x, tuple(a.reshape(E, -1)[es] for a in ex), sh, ew, H, I)



@pytest.mark.parametrize("mode", ["ref", "fast"])
def test_moe_detects_corrupted_expert(mode):
    """Must-fail twin: the d of every block in row 0 of the first selected expert's down
    matrix raised to 4.0 moves y[0] past the check (bit-exact in ref mode, the MoE tolerance in
    fast mode); the clean step passes the same check."""
    E, H, I, topk = 16, 512, 256, 4
    note(f"moe corruption twin {mode}")
    rng = np.random.default_rng(4040)
    rw, ex, sh, x = _moe_case(rng, E, H, I, BF16, False)
    r = go.moe_decode_ref(x, BF16, rw, ex, Q4K, E, H, I, topk)
    e0 = int(r["sel_idx"][0])
    bad_down = ex[2].copy().reshape(E, H, I // 256, 144)
    bad_down[e0, 0, :, 0:2] = np.asarray(qo.f32_to_f16_bits(np.array([4.0], np.float32)), np.uint16).view(np.uint8)
    bad = (ex[0], ex[1], bad_down.reshape(-1))
    for weights, expect_pass in ((bad, False), (ex, True)):
        if mode == "ref":
            y, sel, sw = dev.moe_swiglu_decode(BF16, d_u8(rw), Q4K, *(d_u8(a) for a in weights), E, H, I, topk,
                                               d_bf16(x), mode=mode)
            passed = np.array_equal(h_bits(y), r["y"])
        else:
            yb, sel, sw, lg, hw = _fast_step(BF16, rw, tuple(d_u8(a) for a in weights), E, H, I, topk, x)
            es, ew = _check_routing(BF16, rw, E, H, x, topk, sel, sw, lg)
            try:   # checked against the clean weights
                _check_moe_tight(yb, hw, x, tuple(a.reshape(E, -1)[es] for a in ex), None, ew, H, I)
                passed = True
            except AssertionError:
                passed = False
        assert passed == expect_pass, f"{mode}: check {'passed' if passed else 'failed'} on {'clean' if expect_pass else 'corrupted'} weights"

def _fast_step(router_type, rw, ex_d, E, H, I, topk, x, shared_d=None):
    """One fast-mode MoE step with its own workspace.  Returns y, sel, sel_w (host) and the
    step's own router logits and per-slot h, read back from the workspace at the offsets
    include/aipu_q4k.h documents."""
    ws = dev.moe_workspace(E, H, I, topk, "cuda")
    y, sel, sw = dev.moe_swiglu_decode(router_type, d_u8(rw), Q4K, *ex_d, E, H, I, topk, d_bf16(x), mode="fast",
                                       shared=shared_d, workspace=ws)
    lg, hw = dev.moe_workspace_views(ws, E, I, topk + (shared_d is not None))
    return h_bits(y), sel.cpu().numpy(), h_bits(sw), h_bits(lg), h_bits(hw)


def _router_matrix(router_type, rw, E, H):
    if router_type == BF16:
        return qo.bf16_bits_to_f32(np.asarray(rw).view(np.uint16).reshape(E, H))
    return qo.dequant_matrix(router_type, rw, E, H)


def _check_routing(router_type, rw, E, H, x, topk, sel, sw, lg):
    """Fast-mode routing contract: sel / sel_w are exactly the reference's router tail
    (tools/glm_model_q4k_ref.py:669-681) applied to the logits the step itself formed, and those
    logits agree with the reference-order logits (:663-668) within one bf16 ulp where the sum is
    well conditioned and within the accumulator tolerance where it cancels.  For bf16 routers the
    logits are also bit-exact to the oracle's model of the router kernel's summation order."""
    es, ew, _ = go.router_tail(lg, topk)
    assert np.array_equal(sel, es), f"routing {sel} is not the tail of the step's own logits {es}"
    assert_bits_equal(sw, ew, "sel_w")
    w = _router_matrix(router_type, rw, E, H)
    xf = qo.bf16_bits_to_f32(x)[None]
    acc, _ = qo.gemv_ref(w, xf)
    ok, max_ulp, n_c = qo.bf16_parity(lg[None], acc, w, xf)
    assert ok, f"step logits {max_ulp} ulp from the reference order ({n_c} cancelled sums)"
    if router_type == BF16:
        model = {k: go.router_logits_fast_order(np.asarray(rw).view(np.uint16), E, H, x, dot2=k)
                 for k in ("fused", "chain")}
        note("  step logits vs the fast-order model: " + ", ".join(f"{k} {int((lg != v).sum())} differ"
                                                                     for k, v in model.items()))
        assert any(np.array_equal(lg, v) for v in model.values()), "step logits differ from the fast-order model"
    return es, ew


def _silu64(v):
    with np.errstate(over="ignore"):
        return v / (1.0 + np.exp(-v))


def _check_moe_tight(y_bits, h_ws, x, sub, sh, selw, H, I):
    """The step's output against exact fp64 arithmetic, in two stages, using the h the step
    itself formed (read from the workspace):
    - h of every slot within what the gate/up tolerance (1e-5 * sum|x w| on g and u) and the bf16
      roundings of g, u, silu(g) and h allow around silu(g) * u of the exact sums;
    - y within sum_s |g_s| (1e-5 * sum_k |h_sk w_dk| + 2^-8 |y_s|) + 2^-8 |y| (+ fp32 combine
      rounding) of sum_s g_s y_s, y_s the exact down product of the step's own h_s: the down
      legs' tolerance, one bf16 rounding per slot output and one of the combine.
    ``sub`` = (gate, up, down) ggml images of the routed experts in slot order, one row each."""
    xf = qo.bf16_bits_to_f32(x).astype(np.float64)
    slots = [(sub[0][s], sub[1][s], sub[2][s], float(qo.bf16_bits_to_f32(np.uint16(selw[s]))))
             for s in range(len(selw))]
    if sh is not None:
        slots.append((sh[0], sh[1], sh[2], 1.0))
    assert h_ws.shape == (len(slots), I)
    yex = np.zeros(H)
    bound = np.zeros(H)
    gabs = np.zeros(H)
    for s, (wg, wu, wd, g) in enumerate(slots):
        Wg = qo.dequant_q4k(wg).reshape(I, H).astype(np.float64)
        Wu = qo.dequant_q4k(wu).reshape(I, H).astype(np.float64)
        gx, ux = Wg @ xf, Wu @ xf
        eg = 1e-5 * (np.abs(Wg) @ np.abs(xf)) + 2.0 ** -8 * np.abs(gx)
        eu = 1e-5 * (np.abs(Wu) @ np.abs(xf)) + 2.0 ** -8 * np.abs(ux)
        del Wg, Wu
        sx = _silu64(gx)
        bh = (1.1 * eg + 2.0 ** -7 * np.abs(sx)) * (np.abs(ux) + eu) + np.abs(sx) * eu + 2.0 ** -8 * np.abs(sx * ux)
        hs = qo.bf16_bits_to_f32(h_ws[s]).astype(np.float64)
        bad = np.flatnonzero(np.abs(hs - sx * ux) > bh + 1e-30)
        assert bad.size == 0, f"slot {s}: h outside its bound at {bad[:5]}: {hs[bad[:5]]} vs {(sx * ux)[bad[:5]]}"
        Wd = qo.dequant_q4k(wd).reshape(H, I).astype(np.float64)
        ys = Wd @ hs
        yex += g * ys
        bound += abs(g) * (1e-5 * (np.abs(Wd) @ np.abs(hs)) + 2.0 ** -8 * np.abs(ys))
        gabs += np.abs(g * ys)
    bound += 2.0 ** -8 * np.abs(yex) + 2.0 ** -20 * gabs + 1e-30
    yv = qo.bf16_bits_to_f32(y_bits).astype(np.float64)
    bad = np.flatnonzero(np.abs(yv - yex) > bound)
    assert bad.size == 0, f"y outside its bound at {bad[:5]}: {yv[bad[:5]]} vs {yex[bad[:5]]} (bound {bound[bad[:5]]})"


def _expert_rows(t, E, idx):
    """Host copies of experts `idx` (in that order) of a device `_exps` stack, as a new stack."""
    per = t.numel() // E
    return np.concatenate([t[int(e) * per:(int(e) + 1) * per].cpu().numpy() for e in idx])


@pytest.mark.parametrize("mode", ["fast", "ref"])
def test_moe_c2_full_256_experts(mode):
    """BASELINE config 2 at its own size -- the benchmarked step: 256 experts, hidden 6144,
    expert intermediate 2048, top-8, bf16 router (routing in the gate/up kernel in fast mode).
    Fast: the routing is the reference tail of the step's own logits, which agree with the
    reference-order logits, and h and y meet the two-stage bound; ref: routing and y bit-exact
    vs the oracle.  Only the 8 routed experts are copied to the host."""
    E, H, I, topk = 256, 6144, 2048, 8
    note(f"moe C2 E=256 {mode}")
    g = torch.Generator(device="cuda")
    g.manual_seed(256)
    ge = random_weights_gpu(Q4K, E * I, H, g)
    ue = random_weights_gpu(Q4K, E * I, H, g)
    de = random_weights_gpu(Q4K, E * H, I, g)
    rng = np.random.default_rng(256)
    rw = qo.random_bf16(rng, (E, H), scale=0.05).view(np.uint8).reshape(-1)
    x = qo.random_bf16(rng, H, scale=0.05)
    if mode == "fast":
        yb, sel, sw, lg, hw = _fast_step(BF16, rw, (ge, ue, de), E, H, I, topk, x)
        es, ew = _check_routing(BF16, rw, E, H, x, topk, sel, sw, lg)
    else:
        y, sel, sw = dev.moe_swiglu_decode(BF16, d_u8(rw), Q4K, ge, ue, de, E, H, I, topk, d_bf16(x), mode=mode)
        es, ew, _ = go.router_tail(go.router_logits(BF16, rw.view(np.uint16), E, H, x), topk)
        assert np.array_equal(sel.cpu().numpy(), es)
        assert_bits_equal(h_bits(sw), ew, "sel_w")
    sub = tuple(_expert_rows(t, E, es).reshape(topk, -1) for t in (ge, ue, de))   # routed experts in slot order
    if mode == "fast":
        _check_moe_tight(yb, hw, x, sub, None, ew, H, I)
    else:
        ys = [go.swiglu_expert(x, sub[0][s], sub[1][s], sub[2][s], Q4K, H, I)[0] for s in range(topk)]
        yref, _ = go.moe_combine(ew, ys)
        assert_bits_equal(h_bits(y), yref, "moe ref C2 E=256")



def _random_moe_cases(n=10, seed=1404):
    """Seeded MoE shapes: E = topk..96 experts, H = 256..3072, I = 256..1536, top-1..8, bf16 or
    Q4_K router, with or without the shared expert."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        topk = int(rng.integers(1, 9))
        out.append((int(rng.integers(topk, 97)), 256 * int(rng.integers(1, 13)), 256 * int(rng.integers(1, 7)), topk,
                    BF16 if rng.integers(0, 2) else Q4K, bool(rng.integers(0, 2))))
    return out


@pytest.mark.parametrize("mode", ["ref", "fast"])
@pytest.mark.parametrize("E,H,I,topk,router_type,shared", _random_moe_cases())
def test_moe_random_shapes(E, H, I, topk, router_type, shared, mode):
    """One MoE step at seeded random shapes, whichever kernels the dispatch picks: in ref mode
    routing and y bit-exact against the oracle; in fast mode the routing is the reference tail
    of the step's own logits and h and y meet the two-stage bound."""
    note(f"moe random {mode} E={E} H={H} I={I} topk={topk} router={router_type} shared={shared}")
    rng = np.random.default_rng(E * 1000 + H + I + topk + shared)
    rw, ex, sh, x = _moe_case(rng, E, H, I, router_type, shared)
    shd = tuple(d_u8(a) for a in sh) if sh else None
    if mode == "ref":
        y, sel, sw = dev.moe_swiglu_decode(router_type, d_u8(rw), Q4K, d_u8(ex[0]), d_u8(ex[1]), d_u8(ex[2]), E, H,
                                           I, topk, d_bf16(x), mode="ref", shared=shd)
        r = go.moe_decode_ref(x, router_type, rw, ex, Q4K, E, H, I, topk, shared=sh)
        assert np.array_equal(sel.cpu().numpy(), r["sel_idx"])
        assert_bits_equal(h_bits(sw), r["sel_w"], "sel_w")
        assert_bits_equal(h_bits(y), r["y"], "y")
        return
    yb, sel, sw, lg, hw = _fast_step(router_type, rw, tuple(d_u8(a) for a in ex), E, H, I, topk, x, shd)
    es, ew = _check_routing(router_type, rw, E, H, x, topk, sel, sw, lg)
    _check_moe_tight(yb, hw, x, tuple(a.reshape(E, -1)[es] for a in ex), sh, ew, H, I)

def _moe_persistent_case(H, E, topk, seed):
    I = 2048
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    ge = random_weights_gpu(Q4K, E * I, H, g)
    ue = random_weights_gpu(Q4K, E * I, H, g)
    de = random_weights_gpu(Q4K, E * H, I, g)
    rng = np.random.default_rng(seed)
    rw = qo.random_bf16(rng, (E, H), scale=0.05).view(np.uint8).reshape(-1)
    x = qo.random_bf16(rng, H, scale=0.05)
    return I, (ge, ue, de), rw, x


@pytest.mark.parametrize("H,E,topk,shared", [(2048, 16, 1, False), (4096, 64, 5, False), (6144, 32, 2, False),
                                             (2048, 300, 8, False), (2048, 16, 4, True), (6144, 32, 8, True)])
def test_moe_fast_persistent_legs(H, E, topk, shared):
    """Shapes of the persistent expert legs (I = 2048, H = 2048 R): one to eight routed slots
    (whole compute-wave groups idle at one and two slots, unequal groups at five), R = 1, 2, 3,
    an expert count whose routing keys need padding (300), and the shared expert as the last
    slot (five and nine slots).  The routing is the reference tail of the step's own logits, and
    h and y meet the two-stage bound."""
    note(f"moe persistent legs H={H} E={E} topk={topk} shared={shared}")
    I, (ge, ue, de), rw, x = _moe_persistent_case(H, E, topk, H + E + topk + shared)
    shd = sh = None
    if shared:
        g = torch.Generator(device="cuda")
        g.manual_seed(H + topk)
        shd = (random_weights_gpu(Q4K, I, H, g), random_weights_gpu(Q4K, I, H, g), random_weights_gpu(Q4K, H, I, g))
        sh = tuple(t.cpu().numpy() for t in shd)
    yb, sel, sw, lg, hw = _fast_step(BF16, rw, (ge, ue, de), E, H, I, topk, x, shd)
    es, ew = _check_routing(BF16, rw, E, H, x, topk, sel, sw, lg)
    sub = tuple(_expert_rows(t, E, es).reshape(topk, -1) for t in (ge, ue, de))   # routed experts in slot order
    _check_moe_tight(yb, hw, x, sub, sh, ew, H, I)


# The gate/up leg multiplies the high-nibble codes with each activation pair scaled by 2^-e in
# fp16 (e puts the pair's largest magnitude in [2^14, 2^15)).  Activations far below and above 1,
# a vector whose elements span 2^-40..2^40 inside every pair, and one all-zero pair beside
# ordinary ones must still meet the routing contract and the two-stage bound.
@pytest.mark.parametrize("case", ["small", "large", "span", "zero_pair"])
def test_moe_fast_persistent_activation_range(case):
    H, E, topk = 2048, 16, 2
    note(f"moe persistent activation range {case}")
    I, (ge, ue, de), rw, x = _moe_persistent_case(H, E, topk, 7000 + len(case))
    rng = np.random.default_rng(7100 + len(case))
    xf = qo.bf16_bits_to_f32(x).astype(np.float32)
    if case == "small":
        xf *= np.float32(2.0 ** -30)
    elif case == "large":
        xf *= np.float32(2.0 ** 30)
    elif case == "span":
        xf *= np.exp2(rng.integers(-40, 41, H)).astype(np.float32)
    else:
        xf[512:1024] = 0.0
    x = qo.bf16_round_bits(xf)
    yb, sel, sw, lg, hw = _fast_step(BF16, rw, (ge, ue, de), E, H, I, topk, x)
    es, ew = _check_routing(BF16, rw, E, H, x, topk, sel, sw, lg)
    sub = tuple(_expert_rows(t, E, es).reshape(topk, -1) for t in (ge, ue, de))
    _check_moe_tight(yb, hw, x, sub, None, ew, H, I)


def test_moe_persistent_detects_corrupted_expert():
    """Must-fail twin on the persistent legs: d of every block of the first routed expert's down
    matrix 10 % larger (a small error in one slot of the down leg) fails the two-stage bound;
    the clean step passes it."""
    H, E, topk = 2048, 16, 2
    note("moe persistent corruption twin")
    I, (ge, ue, de), rw, x = _moe_persistent_case(H, E, topk, 5150)
    clean = _fast_step(BF16, rw, (ge, ue, de), E, H, I, topk, x)
    es, ew = _check_routing(BF16, rw, E, H, x, topk, *clean[1:4])
    sub = tuple(_expert_rows(t, E, es).reshape(topk, -1) for t in (ge, ue, de))
    bad = de.clone()
    per = bad.numel() // E
    blk = bad[int(es[0]) * per:(int(es[0]) + 1) * per].view(-1, 144)
    dh = blk[:, 0:2].contiguous().cpu().numpy().view(np.uint16).reshape(-1)
    d11 = np.asarray(qo.f32_to_f16_bits(qo.f16_bits_to_f32(dh) * np.float32(1.1)), np.uint16)
    blk[:, 0:2] = torch.from_numpy(d11.view(np.uint8).reshape(-1, 2)).to(bad.device)
    for down, expect_pass in ((bad, False), (de, True)):
        yb, sel, sw, lg, hw = _fast_step(BF16, rw, (ge, ue, down), E, H, I, topk, x)
        assert np.array_equal(sel, es)
        try:
            _check_moe_tight(yb, hw, x, sub, None, ew, H, I)
            passed = True
        except AssertionError:
            passed = False
        assert passed == expect_pass, f"check {'passed' if passed else 'failed'} on {'clean' if expect_pass else 'corrupted'} weights"


@pytest.mark.parametrize("H,E", [(512, 300), (1280, 256), (1536, 512)])
def test_moe_fast_router_wider_than_gateup_plan(H, E):
    """Expert counts that the gate/up plan cannot rank in-kernel (one key per thread and fewer
    threads than keys) take the separate router-tail launch and stay correct."""
    I, topk = 256, 8
    note(f"moe fast wide router H={H} E={E}")
    rng = np.random.default_rng(H + E)
    rw, ex, sh, x = _moe_case(rng, E, H, I, BF16, False)
    yb, sel, sw, lg, hw = _fast_step(BF16, rw, tuple(d_u8(a) for a in ex), E, H, I, topk, x)
    es, ew = _check_routing(BF16, rw, E, H, x, topk, sel, sw, lg)
    _check_moe_tight(yb, hw, x, tuple(a.reshape(E, -1)[es] for a in ex), None, ew, H, I)


# ----------------------------------------------------------------- tiles
@pytest.mark.parametrize("mode", ["ref", "fast"])
def test_mixed_tiles(mode):
    """24 column tiles of 256 rows cycling Q4_K, Q6_K, Q8_0, F16 (BASELINE config 3 at K = 2048)."""
    note(f"tiles {mode}")
    rng = np.random.default_rng(33)
    K, rows = 2048, 256
    types = [Q4K, qo.GGML_Q6_K, qo.GGML_Q8_0, qo.GGML_F16] * 6
    raws = [qo.random_weights(rng, t, rows, K) for t in types]
    tiles = [(t, d_u8(r), i * rows, rows) for i, (t, r) in enumerate(zip(types, raws))]
    N = rows * len(types)
    x = qo.random_bf16(rng, (2, K))
    y, yf = dev.gemv_tiles(tiles, N, K, d_bf16(x), mode=mode, out_f32=True)
    acc = np.concatenate([co.gemv_ref(t, r, rows, K, x)[0] for t, r in zip(types, raws)], axis=1)
    w = np.concatenate([qo.dequant_matrix(t, r, rows, K) for t, r in zip(types, raws)])
    assert set(types) == {Q4K, qo.GGML_Q6_K, qo.GGML_Q8_0, qo.GGML_F16}
    if mode == "ref":
        assert_bits_equal(u32(h_f32(yf)), u32(acc), "tiles acc")
        assert_bits_equal(h_bits(y), qo.bf16_round_bits(acc), "tiles y")
    else:
        ok, worst = qo.tolerance_gate(w, qo.bf16_bits_to_f32(x), h_f32(yf))
        assert ok, worst
        assert qo.bf16_parity(h_bits(y), acc, w, qo.bf16_bits_to_f32(x))[0]


def test_mixed_tiles_c3_full_shape():
    """BASELINE config 3 at its own size: K = N = 6144, 24 tiles of 256 rows, one launch."""
    note("tiles fast C3 K=6144")
    rng = np.random.default_rng(34)
    K, rows = 6144, 256
    types = [Q4K, qo.GGML_Q6_K, qo.GGML_Q8_0, qo.GGML_F16] * 6
    raws = [qo.random_weights(rng, t, rows, K) for t in types]
    tiles = [(t, d_u8(r), i * rows, rows) for i, (t, r) in enumerate(zip(types, raws))]
    N = rows * len(types)
    x = qo.random_bf16(rng, (1, K))
    y, yf = dev.gemv_tiles(tiles, N, K, d_bf16(x), mode="fast", out_f32=True)
    acc = np.concatenate([co.gemv_ref(t, r, rows, K, x)[0] for t, r in zip(types, raws)], axis=1)
    w = np.concatenate([qo.dequant_matrix(t, r, rows, K) for t, r in zip(types, raws)])
    ok, worst = qo.tolerance_gate(w, qo.bf16_bits_to_f32(x), h_f32(yf))
    note(f"  worst |delta| = {worst:.4f} of the 1e-5*sum|a*w| bound")
    assert ok, worst
    assert qo.bf16_parity(h_bits(y), acc, w, qo.bf16_bits_to_f32(x))[0]


# Mixed-type batches share each weight pass: K <= 6144 runs up to four rows per launch (K = 6144
# and 2048: one pass of four or three rows; K = 5120 with six rows: a pass of four, then one of
# two), larger K one row per launch (K = 8192).  Every row must equal its single-row launch bit
# for bit (the rows are formed independently from the same decoded weights) and pass the gate.
@pytest.mark.parametrize("K,M", [(6144, 4), (2048, 3), (5120, 6), (8192, 2)])
def test_mixed_tiles_batch(K, M):
    note(f"tiles fast batch K={K} M={M}")
    rng = np.random.default_rng(K + M)
    rows = 48
    types = [Q4K, qo.GGML_Q6_K, qo.GGML_Q8_0, qo.GGML_F16] * 2
    raws = [qo.random_weights(rng, t, rows, K) for t in types]
    tiles = [(t, d_u8(r), i * rows, rows) for i, (t, r) in enumerate(zip(types, raws))]
    N = rows * len(types)
    x = qo.random_bf16(rng, (M, K))
    y, yf = dev.gemv_tiles(tiles, N, K, d_bf16(x), mode="fast", out_f32=True)
    yb, yfb = h_bits(y), u32(h_f32(yf))
    for r in range(M):
        y1, yf1 = dev.gemv_tiles(tiles, N, K, d_bf16(x[r:r + 1]), mode="fast", out_f32=True)
        assert_bits_equal(u32(h_f32(yf1))[0], yfb[r], f"row {r} of M={M}: fp32 accumulators")
        assert_bits_equal(h_bits(y1)[0], yb[r], f"row {r} of M={M}: bf16 outputs")
    acc = np.concatenate([co.gemv_ref(t, r, rows, K, x)[0] for t, r in zip(types, raws)], axis=1)
    w = np.concatenate([qo.dequant_matrix(t, r, rows, K) for t, r in zip(types, raws)])
    ok, worst = qo.tolerance_gate(w, qo.bf16_bits_to_f32(x), h_f32(yf))
    note(f"  worst |delta| = {worst:.4f} of the 1e-5*sum|a*w| bound")
    assert ok, worst
    assert qo.bf16_parity(h_bits(y), acc, w, qo.bf16_bits_to_f32(x))[0]


def test_mixed_tiles_ragged_fast():
    """Tiles of odd row counts, out of order, with uncovered rows that must stay untouched."""
    note("tiles fast ragged")
    rng = np.random.default_rng(35)
    K = 1280
    spec = [(qo.GGML_F16, 200, 37), (Q4K, 0, 16), (qo.GGML_Q6_K, 20, 100), (qo.GGML_Q8_0, 120, 1),
            (qo.GGML_Q6_K, 121, 17), (Q4K, 250, 33)]
    N = 300
    raws = [qo.random_weights(rng, t, n, K) for t, _, n in spec]
    tiles = [(t, d_u8(r), r0, n) for (t, r0, n), r in zip(spec, raws)]
    x = qo.random_bf16(rng, (1, K))
    y = torch.full((1, N), 7.0, dtype=torch.bfloat16, device="cuda")
    yf = torch.full((1, N), -3.0, dtype=torch.float32, device="cuda")
    dev.gemv_tiles(tiles, N, K, d_bf16(x), mode="fast", out=y, out_f32=yf)
    got_f, got_y = h_f32(yf)[0], h_bits(y)[0]
    covered = np.zeros(N, bool)
    for (t, r0, n), r in zip(spec, raws):
        covered[r0:r0 + n] = True
        w = qo.dequant_matrix(t, r, n, K)
        acc, _ = co.gemv_ref(t, r, n, K, x)
        ok, worst = qo.tolerance_gate(w, qo.bf16_bits_to_f32(x), got_f[None, r0:r0 + n])
        assert ok, (t, r0, n, worst)
        assert qo.bf16_parity(got_y[None, r0:r0 + n], acc, w, qo.bf16_bits_to_f32(x))[0], (t, r0, n)
    assert np.all(got_f[~covered] == np.float32(-3.0))
    assert np.all(got_y[~covered] == qo.bf16_round_bits(np.float32(7.0)))


def _ragged_spec(rng, n_tiles, K):
    """Tiles of every type with uneven row counts, out of order, leaving gaps of uncovered rows."""
    kinds = [Q4K, qo.GGML_Q6_K, qo.GGML_Q8_0, qo.GGML_F16, BF16]
    spec, r0 = [], 0
    for i in range(n_tiles):
        n = int(rng.integers(1, 300)) if i % 5 else int(rng.integers(1, 12))
        spec.append((kinds[i % 5], r0, n))
        r0 += n + int(rng.integers(0, 3))
    order = rng.permutation(n_tiles)
    return [spec[i] for i in order], r0


# Full-size one-row launches against the rows of a two-row batch (one weight pass for both):
# every row must equal its one-row launch bit for bit.  Shapes: C3 (K = 6144), one type over
# all rows at K = 4096 / 2048 / 1024 (four, two and one block per wave, so the last group of a
# Q4_K wave covers blocks past its part), and 40 ragged tiles of all five types, out of order
# and with gaps of uncovered rows, at K = 5120 (five blocks per wave).
LARGE_ONE_ROW_CASES = [("c3", 6144, None), ("q6k", 4096, [(qo.GGML_Q6_K, 0, 4096)]),
              ("q8_0", 2048, [(qo.GGML_Q8_0, 0, 4200)]), ("f16", 1024, [(qo.GGML_F16, 0, 4100)]),
              ("q4k", 4096, [(Q4K, 0, 4352)]), ("ragged", 5120, "ragged")]


@pytest.mark.parametrize("name,K,spec", LARGE_ONE_ROW_CASES)
def test_mixed_tiles_large_one_row(name, K, spec):
    note(f"tiles fast large one-row {name} K={K}")
    rng = np.random.default_rng(K + len(name))
    if spec is None:
        spec = [(t, i * 256, 256) for i, t in enumerate([Q4K, qo.GGML_Q6_K, qo.GGML_Q8_0, qo.GGML_F16] * 6)]
        N = 6144
    elif spec == "ragged":
        spec, N = _ragged_spec(rng, 40, K)
    else:
        N = spec[0][2]
    tw = [_tile_weights(rng, t, n, K) for t, _, n in spec]
    tiles = [(t, d_u8(r), r0, n) for (t, r0, n), (r, _) in zip(spec, tw)]
    x = qo.random_bf16(rng, (2, K))
    y2, yf2 = dev.gemv_tiles(tiles, N, K, d_bf16(x), mode="fast", out_f32=True)
    y = torch.full((1, N), 7.0, dtype=torch.bfloat16, device="cuda")
    yf = torch.full((1, N), -3.0, dtype=torch.float32, device="cuda")
    covered = np.zeros(N, bool)
    for _, r0, n in spec:
        covered[r0:r0 + n] = True
    for r in range(2):
        dev.gemv_tiles(tiles, N, K, d_bf16(x[r:r + 1]), mode="fast", out=y, out_f32=yf)
        got_f, got_y = u32(h_f32(yf))[0], h_bits(y)[0]
        assert_bits_equal(got_f[covered], u32(h_f32(yf2))[r][covered], f"row {r}: fp32 accumulators vs the batch")
        assert_bits_equal(got_y[covered], h_bits(y2)[r][covered], f"row {r}: bf16 outputs vs the batch")
        assert np.all(h_f32(yf)[0][~covered] == np.float32(-3.0)), "rows outside the tiles written"
        assert np.all(got_y[~covered] == qo.bf16_round_bits(np.float32(7.0))), "rows outside the tiles written"
    if name == "c3":
        return   # the oracle comparison at this size: test_mixed_tiles_c3_full_shape
    xf = qo.bf16_bits_to_f32(x[1:])
    for (t, r0, n), (r, wdq) in zip(spec, tw):
        acc, _ = co.gemv_ref(t, r, n, K, x[1:])
        ok, worst = qo.tolerance_gate(wdq, xf, h_f32(yf)[:, r0:r0 + n])
        assert ok, (name, t, r0, n, worst)
        assert qo.bf16_parity(h_bits(y)[:, r0:r0 + n], acc, wdq, xf)[0], (name, t, r0, n)




def _random_tile_cases(n=16, seed=1303):
    """Seeded (K, M, tiles): K from one block to 12288, M = 1..8, 1..10 ragged tiles of all five
    types (on and off the one-launch path, whose limit depends on K)."""
    rng = np.random.default_rng(seed)
    return [(256 * int(rng.integers(1, 49)), int(rng.integers(1, 9)), int(rng.integers(1, 11))) for _ in range(n)]


@pytest.mark.parametrize("K,M,n_tiles", _random_tile_cases())
def test_mixed_tiles_random_shapes(K, M, n_tiles):
    """Fast-mode tile GEMV at seeded random shapes: every row of the batch equals its one-row
    launch bit for bit, rows outside the tiles stay untouched, and each tile meets the gate."""
    note(f"tiles fast random K={K} M={M} tiles={n_tiles}")
    rng = np.random.default_rng(K * 31 + M * 7 + n_tiles)
    spec, N = _ragged_spec(rng, n_tiles, K)
    tw = [_tile_weights(rng, t, n, K) for t, _, n in spec]
    tiles = [(t, d_u8(r), r0, n) for (t, r0, n), (r, _) in zip(spec, tw)]
    x = qo.random_bf16(rng, (M, K))
    covered = np.zeros(N, bool)
    for _, r0, n in spec:
        covered[r0:r0 + n] = True
    yb = torch.full((M, N), 7.0, dtype=torch.bfloat16, device="cuda")
    yfb = torch.full((M, N), -3.0, dtype=torch.float32, device="cuda")
    dev.gemv_tiles(tiles, N, K, d_bf16(x), mode="fast", out=yb, out_f32=yfb)
    bb, bfb = h_bits(yb), u32(h_f32(yfb))
    assert np.all(h_f32(yfb)[:, ~covered] == np.float32(-3.0)), "rows outside the tiles written"
    assert np.all(bb[:, ~covered] == qo.bf16_round_bits(np.float32(7.0))), "rows outside the tiles written"
    for r in range(M):
        y1, yf1 = dev.gemv_tiles(tiles, N, K, d_bf16(x[r:r + 1]), mode="fast", out_f32=True)
        assert_bits_equal(u32(h_f32(yf1))[0][covered], bfb[r][covered], f"row {r} of M={M}: fp32 accumulators")
        assert_bits_equal(h_bits(y1)[0][covered], bb[r][covered], f"row {r} of M={M}: bf16 outputs")
    xf = qo.bf16_bits_to_f32(x)
    for (t, r0, n), (r, wdq) in zip(spec, tw):
        ok, worst = qo.tolerance_gate(wdq, xf, h_f32(yfb)[:, r0:r0 + n])
        assert ok, (t, r0, n, worst)

def _tile_weights(rng, t, rows, K):
    """(raw bytes, dequantised float32[rows, K]) of a tile; BF16 tiles hold N(0, 0.05^2) bf16."""
    if t == BF16:
        bits = qo.random_bf16(rng, (rows, K), scale=0.05)
        return bits.view(np.uint8).reshape(-1), qo.bf16_bits_to_f32(bits)
    raw = qo.random_weights(rng, t, rows, K)
    return raw, qo.dequant_matrix(t, raw, rows, K)


# The fp16-operand types (Q8_0, F16) scale each activation row's part by a power of two that
# puts its largest magnitude in [2^14, 2^15); the bf16-operand types take the activations as
# they are.  Rows far below and above 1, a row whose elements span 2^-40..2^40, and an all-zero
# row, at K = 2048 (four rows per launch) and K = 12288 (two rows per launch, two launches).
@pytest.mark.parametrize("K", [2048, 12288])
def test_mixed_tiles_activation_range(K):
    note(f"tiles fast activation range K={K}")
    rng = np.random.default_rng(37 + K)
    rows = 32
    types = [Q4K, qo.GGML_Q6_K, qo.GGML_Q8_0, qo.GGML_F16, BF16]
    tw = [_tile_weights(rng, t, rows, K) for t in types]
    tiles = [(t, d_u8(r), i * rows, rows) for i, (t, (r, _)) in enumerate(zip(types, tw))]
    N = rows * len(types)
    xf = rng.standard_normal((4, K)).astype(np.float32)
    xf[0] *= np.float32(2.0 ** -60)
    xf[1] *= np.float32(2.0 ** 60)
    xf[2] *= np.exp2(rng.integers(-40, 41, K)).astype(np.float32)
    xf[3] = 0.0
    x = qo.bf16_round_bits(xf)
    y, yf = dev.gemv_tiles(tiles, N, K, d_bf16(x), mode="fast", out_f32=True)
    yb, yfb = h_bits(y), u32(h_f32(yf))
    for r in range(4):
        y1, yf1 = dev.gemv_tiles(tiles, N, K, d_bf16(x[r:r + 1]), mode="fast", out_f32=True)
        assert_bits_equal(u32(h_f32(yf1))[0], yfb[r], f"row {r}: fp32 accumulators vs its one-row launch")
        assert_bits_equal(h_bits(y1)[0], yb[r], f"row {r}: bf16 outputs vs its one-row launch")
    assert np.all(h_f32(yf)[3] == 0.0)
    acc = np.concatenate([co.gemv_ref(t, r, rows, K, x)[0] for t, (r, _) in zip(types, tw)], axis=1)
    w = np.concatenate([wd for _, wd in tw])
    ok, worst = qo.tolerance_gate(w, qo.bf16_bits_to_f32(x), h_f32(yf))
    note(f"  worst |delta| = {worst:.4f} of the 1e-5*sum|a*w| bound")
    assert ok, worst
    assert qo.bf16_parity(h_bits(y), acc, w, qo.bf16_bits_to_f32(x))[0]


def test_mixed_tiles_detect_corruption():
    """Must-fail twin for the tile path: one Q6_K weight of tile 1 changed (its qh bits) moves
    that output past the gate; the clean tiles pass it."""
    note("tiles corruption twin")
    rng = np.random.default_rng(36)
    K, rows = 1024, 64
    types = [Q4K, qo.GGML_Q6_K, qo.GGML_Q8_0, qo.GGML_F16]
    raws = [qo.random_weights(rng, t, rows, K) for t in types]
    N = rows * len(types)
    x = qo.random_bf16(rng, (1, K))
    w = np.concatenate([qo.dequant_matrix(t, r, rows, K) for t, r in zip(types, raws)])
    bad1 = raws[1].copy()
    rb = bad1.size // rows
    bad1[3 * rb + 128 + 5] ^= 0x30
    for rs, expect in ((raws[:1] + [bad1] + raws[2:], False), (raws, True)):
        tiles = [(t, d_u8(r), i * rows, rows) for i, (t, r) in enumerate(zip(types, rs))]
        _, yf = dev.gemv_tiles(tiles, N, K, d_bf16(x), mode="fast", out_f32=True)
        ok, _ = qo.tolerance_gate(w, qo.bf16_bits_to_f32(x), h_f32(yf))
        assert ok == expect, "tile check on " + ("clean" if expect else "corrupted") + " weights"

# --------------------------------------------------- reference-interface mirrors
def test_q4k_ref_mirror_selftest():
    """The reference's own self-test (tools/q4k_ref.py:150-182) run through the GPU mirror."""
    from aipu_amd import q4k_ref as ref
    note("q4k_ref mirror")
    rng = np.random.default_rng(0)
    n = n_fail = 0
    for _ in range(40):
        scs = [int(v) for v in rng.integers(0, 64, 8)]
        mns = [int(v) for v in rng.integers(0, 64, 8)]
        scales = ref._pack_6bit_scales(scs, mns)
        for j in range(0, 8, 3):
            assert ref.get_scale_min_k4(j, scales) == (scs[j], mns[j])
        qs = [int(v) for v in rng.integers(0, 256, 128)]
        d_h = ref._f32_to_f16bits(rng.uniform(0.001, 0.05))
        dm_h = ref._f32_to_f16bits(rng.uniform(0.0, 0.02))
        y = ref.dequantize_block_q4_K(d_h, dm_h, scales, qs)
        exp = qo.dequant_block_q4k_scalar(d_h, dm_h, scales, qs)
        n += 1
        n_fail += int(not np.array_equal(u32(y), u32(exp)))
        q6 = ref.dequantize_block_q6_K(d_h, qs, qs[:64], [int(v) for v in rng.integers(-32, 32, 16)])
        assert q6.shape == (256,)
    assert n_fail == 0
    a = qo.bf16_bits_to_f32(qo.random_bf16(rng, 300))
    w = (rng.standard_normal(300) * 0.1).astype(np.float32)
    assert qo.f32_bits(ref.matmul_q4k_col(a, w)) == qo.f32_bits(qo.dot_ref_scalar(a, w)[1])
    assert qo.f32_bits(ref.bf16_round(np.float32(1.00390625))) == 0x3F800000
    q8 = ref.dequantize_block_q8_0(0x3C00, [-128, -1, 0, 127] * 8)
    assert list(q8[:4]) == [-128.0, -1.0, 0.0, 127.0]


def test_glm_mirror_selftest():
    """tools/glm_model_q4k_ref.py self-test items (a), (b), (f) through the GPU mirror."""
    from aipu_amd import glm_model_q4k_ref as gm
    note("glm mirror")
    rng = np.random.default_rng(0)
    # (a) column dequant == block dequant
    scs = [int(v) for v in rng.integers(0, 64, 8)]
    mns = [int(v) for v in rng.integers(0, 64, 8)]
    s12 = qo.pack_scales_q4k(scs, mns)
    codes = [int(v) for v in rng.integers(0, 16, 256)]
    d_h, dm_h = gm.f32_to_f16bits(0.01), gm.f32_to_f16bits(0.005)
    qw = gm.QW(1, 256, [codes], [d_h], [dm_h], [s12])
    blk = np.zeros(144, np.uint8)
    blk[:] = qw.raw[0]
    assert np.array_equal(u32(qw.dequant_col(0)), u32(qo.dequant_q4k(blk)))
    # (b) matmul_q4k == matmul_q4k_col (sequential fp32)
    a = [gm.bf16(np.float32(v)) for v in rng.uniform(-1.5, 1.5, 256)]
    got = gm.matmul_q4k(a, [qw.dequant_col(0)])[0]
    assert qo.f32_bits(got) == qo.f32_bits(qo.dot_ref_scalar(np.array(a, np.float32), qw.dequant_col(0))[1])
    # (f) router renorm: sum of routed weights ~ SCALE
    cfg = gm.Config(MODEL_DIM=256, N_EXPERT=16, TOPK=4)
    Wg = gm.QW(16, 256, [[int(v) for v in rng.integers(0, 16, 256)] for _ in range(16)],
               [gm.f32_to_f16bits(0.003)] * 16, [gm.f32_to_f16bits(0.003)] * 16,
               [qo.pack_scales_q4k([2] * 8, [15] * 8)] * 16)
    for _ in range(5):
        x = [gm.bf16(np.float32(v)) for v in rng.uniform(-1.5, 1.5, 256)]
        sel, sw, gates = gm.moe_router(cfg, x, Wg)
        assert len(set(sel)) == 4 and abs(sum(float(v) for v in sw) - 2.5) < 0.05
        es, ew, eg = go.router_tail(h_bits(dev.gemv(Q4K, Wg.blocks, 16, 256, d_bf16(np.asarray(x, np.float32).view(np.uint32) >> 16)[None], mode="ref"))[0], 4)
        assert sel == list(es)
    assert gm.glm_silu(gm.bf16_from_bits(0x3F80)) == qo.bf16_bits_to_f32(go.glm_silu_bits_vec(np.array([0x3F80], np.uint16)))[0]
    assert gm.fp32_rsqrt(np.float32(4.0)) == go.fp32_rsqrt(np.float32(4.0))


def test_glm_mirror_swiglu_and_moe_ffn():
    from aipu_amd import glm_model_q4k_ref as gm
    note("glm mirror swiglu / moe_ffn")
    s = np.load(os.path.join(GOLD, "swiglu_cases.npz"))
    cfg = gm.Config(MODEL_DIM=256)
    Wg = gm.QW.from_ggml(s["c0_wg"], 256, 256)
    Wu = gm.QW.from_ggml(s["c0_wu"], 256, 256)
    Wd = gm.QW.from_ggml(s["c0_wd"], 256, 256)
    x = list(qo.bf16_bits_to_f32(s["c0_x"]))
    y = gm.swiglu_expert(cfg, x, Wg, Wu, Wd)
    assert_bits_equal(np.asarray(y, np.float32).view(np.uint32) >> 16, s["c0_y"], "mirror swiglu")
    # MoE FFN half of decoder_block at the reference's committed slice (MODEL_DIM 128, INTER 64)
    rng = np.random.default_rng(9)
    c2 = gm.Config(MODEL_DIM=128, N_EXPERT=8, TOPK=2, INTER_MOE=64)

    def qw(nout, nin):
        return gm.QW(nout, nin, [[int(v) for v in rng.integers(0, 16, nin)] for _ in range(nout)],
                     [gm.f32_to_f16bits(0.004)] * nout, [gm.f32_to_f16bits(0.004)] * nout,
                     [qo.pack_scales_q4k([3] * 8, [22] * 8)] * nout)
    Wr = qw(8, 128)
    Mg = [qw(64, 128) for _ in range(8)]
    Mu = [qw(64, 128) for _ in range(8)]
    Md = [qw(128, 64) for _ in range(8)]
    xin = [gm.bf16(np.float32(v)) for v in rng.uniform(-1, 1, 128)]
    fbuf, sel, sw = gm.moe_ffn(c2, xin, Wr, Mg, Mu, Md, qw(64, 128), qw(64, 128), qw(128, 64))
    assert len(fbuf) == 128 and len(sel) == 2
    # cross-check against per-expert mirror calls + the oracle's combine
    ys = [gm.swiglu_expert(c2, xin, Mg[e], Mu[e], Md[e]) for e in sel]
    assert all(len(v) == 128 for v in ys)
