#!/usr/bin/env python3
"""Write the golden fixtures in tests/golden/ from the reference's own Python golden.

Runs only in the build container (it imports ``/root/reference/tools/glm_model_q4k_ref.py``;
the reference never travels to the GPU box).  Only the functions that no closed form,
KAT or brute force pins are sampled here:

* ``glm_silu`` / ``glm_sigmoid`` over all 65,536 bf16 patterns  -> act_tables.npz
* ``fp32_rsqrt`` over special values and a sweep of fp32 inputs  -> rsqrt_cases.npz
* ``moe_router`` on Q4_K router weights (ties included)           -> router_cases.npz
* ``swiglu_expert`` on one-super-block Q4_K experts               -> swiglu_cases.npz
* ``rmsnorm`` (+ ``_recip_fp32``) on several lengths and ranges, and the FFN half of
  ``decoder_block`` (rmsnorm -> moe_router -> swiglu_expert per slot -> shared expert ->
  combine -> residual) on one-super-block experts               -> rmsnorm_cases.npz
  (``--rmsnorm`` writes only this file)

Inputs come from this script's own seeded generator; weights are passed to the reference
through its ``QW`` container and stored here as raw ggml Q4_K blocks (144 B each), the
layout the product consumes.  Usage: ``python tests/golden/make_golden.py [REF_TOOLS_DIR]``.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_ARGS = [a for a in sys.argv[1:] if not a.startswith("--")]
REF_TOOLS = _ARGS[0] if _ARGS else "/root/reference/tools"


def codes_to_qs(codes):
    """256 4-bit codes (weight order) -> 128 ggml qs bytes: weight k lives in byte
    32*(k//64) + k%32, low nibble when k%64 < 32 (ggml Q4_K packing)."""
    qs = [0] * 128
    for k, c in enumerate(codes):
        byte = 32 * (k // 64) + (k % 32)
        qs[byte] |= (c & 0xF) if (k % 64) < 32 else ((c & 0xF) << 4)
    return qs


def random_qw(ref, rng, nout):
    """A reference ``QW`` (one super-block per output, nin = 256) and its ggml image."""
    codes = [[int(v) for v in rng.integers(0, 16, 256)] for _ in range(nout)]
    d = [int(v) for v in (np.abs(rng.standard_normal(nout)) * 2.0 ** -8).astype(np.float16).view(np.uint16)]
    dmin = [int(v) for v in (np.abs(rng.standard_normal(nout)) * 2.0 ** -8).astype(np.float16).view(np.uint16)]
    scales = [[int(v) for v in rng.integers(0, 256, 12)] for _ in range(nout)]
    qw = ref.QW(nout, 256, codes, d, dmin, scales)
    img = np.zeros((nout, 144), np.uint8)
    for o in range(nout):
        img[o, 0:2] = np.array([d[o]], np.uint16).view(np.uint8)
        img[o, 2:4] = np.array([dmin[o]], np.uint16).view(np.uint8)
        img[o, 4:16] = scales[o]
        img[o, 16:144] = codes_to_qs(codes[o])
    return qw, img.reshape(-1)


def bf16_bits_of(ref, v):
    return ref.bf16_bits(v)


def main():
    sys.path.insert(0, REF_TOOLS)
    import glm_model_q4k_ref as ref  # noqa: E402  (reference golden, build container only)

    F32 = np.float32

    # ---- activation tables over every bf16 pattern ----
    silu = np.empty(65536, np.uint16)
    sig = np.empty(65536, np.uint16)
    for b in range(65536):
        x = ref.bf16_from_bits(b)
        silu[b] = ref.bf16_bits(ref.glm_silu(x))
        sig[b] = ref.bf16_bits(ref.glm_sigmoid(x))
    np.savez_compressed(os.path.join(HERE, "act_tables.npz"), silu=silu, sigmoid=sig)

    # ---- fp32_rsqrt ----
    rng = np.random.default_rng(20261201)
    special = np.array([0x00000000, 0x80000000, 0x00000001, 0x007FFFFF, 0x00800000, 0x3F800000,
                        0x40200000, 0x7F7FFFFF, 0x7F800000, 0xFF800000, 0x7FC00000, 0xBF800000,
                        0x3E800000, 0x41000000, 0x4B000000, 0x3A83126F], np.uint32)
    sweep = np.concatenate([
        rng.integers(0x00800000, 0x7F800000, 4000, dtype=np.uint64).astype(np.uint32),
        (rng.uniform(0.5, 16.0, 2000).astype(np.float32)).view(np.uint32),
    ])
    rin = np.concatenate([special, sweep])
    rout = np.array([ref.f32_bits(ref.fp32_rsqrt(ref.bits_f32(int(u)))) for u in rin], np.uint32)
    np.savez_compressed(os.path.join(HERE, "rsqrt_cases.npz"), x=rin, y=rout)

    # ---- moe_router on Q4_K router weights ----
    cases = {}
    for ci, (E, topk) in enumerate([(64, 8), (32, 6), (16, 2)]):
        cfg = ref.Config(MODEL_DIM=256, N_EXPERT=E, TOPK=topk)
        qw, img = random_qw(ref, rng, E)
        for xi in range(3):
            scale = [1.0, 4.0, 0.25][xi]
            xv = (rng.standard_normal(256) * scale).astype(np.float32)
            x_bf = [ref.bf16(F32(v)) for v in xv]
            sel, sel_w, gate_bf = ref.moe_router(cfg, x_bf, qw)
            key = f"c{ci}_{xi}"
            cases[key + "_E"] = np.array([E, topk], np.int32)
            cases[key + "_w"] = img
            cases[key + "_x"] = np.array([ref.bf16_bits(v) for v in x_bf], np.uint16)
            cases[key + "_sel"] = np.array(sel, np.int32)
            cases[key + "_selw"] = np.array([ref.bf16_bits(v) for v in sel_w], np.uint16)
            cases[key + "_gate"] = np.array([ref.bf16_bits(v) for v in gate_bf], np.uint16)
    np.savez_compressed(os.path.join(HERE, "router_cases.npz"), **cases)

    # ---- swiglu_expert (HIDDEN = INTER = 256, one super-block per row) ----
    sw = {}
    cfg = ref.Config(MODEL_DIM=256)
    for ci in range(2):
        wg, ig = random_qw(ref, rng, 256)
        wu, iu = random_qw(ref, rng, 256)
        wd, idn = random_qw(ref, rng, 256)
        xv = rng.standard_normal(256).astype(np.float32)
        x_bf = [ref.bf16(F32(v)) for v in xv]
        y = ref.swiglu_expert(cfg, x_bf, wg, wu, wd)
        sw[f"c{ci}_x"] = np.array([ref.bf16_bits(v) for v in x_bf], np.uint16)
        sw[f"c{ci}_wg"] = ig
        sw[f"c{ci}_wu"] = iu
        sw[f"c{ci}_wd"] = idn
        sw[f"c{ci}_y"] = np.array([ref.bf16_bits(v) for v in y], np.uint16)
    np.savez_compressed(os.path.join(HERE, "swiglu_cases.npz"), **sw)
    print("wrote act_tables.npz rsqrt_cases.npz router_cases.npz swiglu_cases.npz")


def main_rmsnorm():
    """rmsnorm_cases.npz: rmsnorm goldens and decoder-block FFN-half goldens."""
    sys.path.insert(0, REF_TOOLS)
    import glm_model_q4k_ref as ref  # noqa: E402  (reference golden, build container only)

    F32 = np.float32
    rng = np.random.default_rng(20261202)
    out = {}
    ns = [1, 7, 16, 100, 128, 256, 6144]
    out["recip_n"] = np.array(ns + [3, 5, 1000, 4096, 12288, 65535], np.int64)
    out["recip_bits"] = np.array([ref.f32_bits(ref._recip_fp32(int(n))) for n in out["recip_n"]], np.uint32)

    def bits(vals):
        return np.array([ref.bf16_bits(v) for v in vals], np.uint16)

    ci = 0
    for n in ns:
        for scale in (1.0, 1e-3, 300.0):
            xv = (rng.standard_normal(n) * scale).astype(np.float32)
            gv = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
            if n >= 16 and scale == 1.0:
                xv[0] = 4096.0                      # one large square first: later ones absorbed
            x_bf = [ref.bf16(F32(v)) for v in xv]
            g_bf = [ref.bf16(F32(v)) for v in gv]
            y = ref.rmsnorm(x_bf, g_bf)
            out[f"n{ci}_x"], out[f"n{ci}_g"], out[f"n{ci}_y"] = bits(x_bf), bits(g_bf), bits(y)
            ci += 1
    zero = [ref.bf16(F32(0.0))] * 64
    out[f"n{ci}_x"], out[f"n{ci}_g"], out[f"n{ci}_y"] = bits(zero), bits(zero), bits(ref.rmsnorm(zero, zero))
    out["n_cases"] = np.array([ci + 1], np.int32)

    # FFN half of decoder_block (:797-810), HIDDEN = INTER = 256, E = 4, TOPK = 2, shared expert
    E, TOPK, D = 4, 2, 256
    cfg = ref.Config(MODEL_DIM=D, N_EXPERT=E, TOPK=TOPK, INTER_MOE=D)
    for li in range(1):
        wg_q, wg_img = random_qw(ref, rng, E)
        mg = [random_qw(ref, rng, D) for _ in range(E)]
        mu = [random_qw(ref, rng, D) for _ in range(E)]
        md = [random_qw(ref, rng, D) for _ in range(E)]
        sh = [random_qw(ref, rng, D) for _ in range(3)]
        hv = (rng.standard_normal(D) * 0.5).astype(np.float32)
        gv = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
        h = [ref.bf16(F32(v)) for v in hv]
        gam = [ref.bf16(F32(v)) for v in gv]
        nrm2 = ref.rmsnorm(h, gam)
        sel, sel_w, _ = ref.moe_router(cfg, nrm2, wg_q)
        facc = [F32(0.0)] * D
        for slot in range(TOPK):
            e = sel[slot]
            y_e = ref.swiglu_expert(cfg, nrm2, mg[e][0], mu[e][0], md[e][0])
            gw = ref.b2f(sel_w[slot])
            for d in range(D):
                facc[d] = ref.fadd(facc[d], ref.fmul(gw, ref.b2f(y_e[d])))
        y_sh = ref.swiglu_expert(cfg, nrm2, sh[0][0], sh[1][0], sh[2][0])
        for d in range(D):
            facc[d] = ref.fadd(facc[d], ref.b2f(y_sh[d]))
        fbuf = [ref.bf16(facc[d]) for d in range(D)]
        y = [ref.bf16(ref.fadd(ref.b2f(h[i]), ref.b2f(fbuf[i]))) for i in range(D)]
        k = f"l{li}_"
        out[k + "h"], out[k + "gamma"], out[k + "router"] = bits(h), bits(gam), wg_img
        out[k + "gate"] = np.concatenate([m[1] for m in mg])
        out[k + "up"] = np.concatenate([m[1] for m in mu])
        out[k + "down"] = np.concatenate([m[1] for m in md])
        out[k + "sh"] = np.stack([m[1] for m in sh])
        out[k + "nrm"], out[k + "fbuf"], out[k + "y"] = bits(nrm2), bits(fbuf), bits(y)
        out[k + "sel"] = np.array(sel, np.int32)
        out[k + "selw"] = bits(sel_w)
    np.savez_compressed(os.path.join(HERE, "rmsnorm_cases.npz"), **out)
    print("wrote rmsnorm_cases.npz")


if __name__ == "__main__":
    if "--rmsnorm" in sys.argv:
        main_rmsnorm()
    else:
        main()
