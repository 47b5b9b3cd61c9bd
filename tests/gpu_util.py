"""Helpers shared by the GPU parity tests (host <-> device, bit comparisons)."""
import sys

import numpy as np
import torch

from oracle import q4k_oracle as qo

DEV = "cuda"


def note(msg):
    """Print (flushed) what the next GPU step is, so a fault names its case."""
    print(f"[gpu-test] {msg}", file=sys.stderr, flush=True)


def d_u8(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint8)).to(DEV)


def d_bf16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.int16)).to(DEV).view(torch.bfloat16)


def h_bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def h_f32(t):
    return t.contiguous().cpu().numpy()


def u32(a):
    return np.asarray(a, np.float32).view(np.uint32)


def assert_bits_equal(got, exp, what=""):
    got = np.asarray(got)
    exp = np.asarray(exp)
    assert got.shape == exp.shape, (what, got.shape, exp.shape)
    bad = np.flatnonzero(got.reshape(-1) != exp.reshape(-1))
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[:5]}: got {got.reshape(-1)[bad[:5]]} exp {exp.reshape(-1)[bad[:5]]}"


def random_weights_gpu(ggml_type, N, K, gen):
    """BASELINE distribution generated on the device (large cases), as a uint8 tensor."""
    if ggml_type == qo.GGML_Q4_K:
        nb = N * K // 256
        raw = torch.randint(0, 256, (nb, 144), dtype=torch.uint8, device=DEV, generator=gen)
        hdr = (torch.randn((nb, 2), device=DEV, generator=gen).abs() * 2.0 ** -8).to(torch.float16)
        raw[:, 0:4] = hdr.view(torch.uint8).view(nb, 4)
        return raw.view(-1)
    raise NotImplementedError(ggml_type)
