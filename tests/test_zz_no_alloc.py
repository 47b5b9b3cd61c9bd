"""The allocation-free MoE decode step (aipu_moe_swiglu_decode_noalloc) through the C ABI:
bit-identical to the workspace entry point aipu_moe_swiglu_decode in both modes, on two calls
in a row on the shared per-GPU scratch array (the second call smaller than the first), with no
torch allocation during the calls; shapes whose scratch exceeds the array are rejected before
any GPU work."""
import ctypes

import numpy as np
import pytest
import torch

from aipu_amd import _lib
from aipu_amd import device as dev
from oracle import q4k_oracle as qo

from .gpu_util import assert_bits_equal, d_bf16, d_u8, h_bits, note, random_weights_gpu

pytestmark = pytest.mark.gpu
Q4K = qo.GGML_Q4_K
BF16 = 30
AIPU_ERR_WORKSPACE = -6


def _case(E, H, I, seed, shared):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    ex = (random_weights_gpu(Q4K, E * I, H, g), random_weights_gpu(Q4K, E * I, H, g),
          random_weights_gpu(Q4K, E * H, I, g))
    sh = (random_weights_gpu(Q4K, I, H, g), random_weights_gpu(Q4K, I, H, g),
          random_weights_gpu(Q4K, H, I, g)) if shared else None
    rng = np.random.default_rng(seed)
    rw = d_u8(qo.random_bf16(rng, (E, H), scale=0.05).view(np.uint8).reshape(-1))
    x = d_bf16(qo.random_bf16(rng, H, scale=0.05))
    return rw, ex, sh, x


@pytest.mark.parametrize("mode", ["fast", "ref"])
def test_noalloc_equals_workspace_entry_point(mode):
    # config 2 with the shared expert (nine slots), then a smaller step on the same scratch
    cases = [(256, 6144, 2048, 8, True, 11), (16, 512, 256, 4, False, 12)]
    for E, H, I, topk, shared, seed in cases:
        note(f"noalloc {mode} E={E} H={H} I={I} topk={topk} shared={shared}")
        rw, ex, sh, x = _case(E, H, I, seed, shared)
        y_ws, sel_ws, sw_ws = dev.moe_swiglu_decode(BF16, rw, Q4K, *ex, E, H, I, topk, x, mode=mode, shared=sh)
        y = torch.empty(H, dtype=torch.bfloat16, device="cuda")
        sel = torch.empty(topk, dtype=torch.int32, device="cuda")
        sw = torch.empty(topk, dtype=torch.bfloat16, device="cuda")
        torch.cuda.synchronize()
        before = torch.cuda.memory_allocated()
        dev.moe_swiglu_decode_noalloc(BF16, rw, Q4K, *ex, E, H, I, topk, x, mode=mode, shared=sh, out=y,
                                      sel_out=(sel, sw))
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated() == before, "the no-alloc call allocated through torch"
        assert np.array_equal(sel.cpu().numpy(), sel_ws.cpu().numpy()), "routing"
        assert_bits_equal(h_bits(sw), h_bits(sw_ws), "sel_w")
        assert_bits_equal(h_bits(y), h_bits(y_ws), "y")


def test_noalloc_rejects_shapes_beyond_its_scratch():
    L = _lib.lib()
    need = L.aipu_moe_workspace_bytes(4096, 16384, 16384, 32)
    assert need > 4 << 20
    rc = L.aipu_moe_swiglu_decode_noalloc(BF16, ctypes.c_void_p(16), Q4K, ctypes.c_void_p(16), ctypes.c_void_p(16),
                                          ctypes.c_void_p(16), None, None, None, 4096, 16384, 16384, 32,
                                          0x40200000, ctypes.c_void_p(16), ctypes.c_void_p(16), None, None, 0, None)
    assert rc == AIPU_ERR_WORKSPACE
    assert b"per-GPU array" in L.aipu_last_error()
