#!/usr/bin/env python3
"""Write the golden fixtures in tests/golden/ from the reference's own Python golden.

Runs only in the build container (it imports ``/root/reference/tools/glm_model_q4k_ref.py``;
the reference never travels to the GPU box).  Only the functions that no closed form,
KAT or brute force pins are sampled here:

* ``glm_silu`` / ``glm_sigmoid`` over all 65,536 bf16 patterns  -> act_tables.npz
* ``fp32_rsqrt`` over special values and a sweep of fp32 inputs  -> rsqrt_cases.npz
* ``moe_router`` on Q4_K router weights (ties included)           -> router_cases.npz
* ``swiglu_expert`` on one-super-block Q4_K experts               -> swiglu_cases.npz

Inputs come from this script's own seeded generator; weights are passed to the reference
through its ``QW`` container and stored here as raw ggml Q4_K blocks (144 B each), the
layout the product consumes.  Usage: ``python tests/golden/make_golden.py [REF_TOOLS_DIR]``.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF_TOOLS = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/tools"


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


if __name__ == "__main__":
    main()
