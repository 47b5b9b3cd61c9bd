"""GPU: entry points running at the same time on two streams.

The library's kernels keep their coordination inside a workgroup (LDS counters; no workgroup
waits for another), and every call owns its workspace, so calls on different streams may
overlap on the GPU in any way.  Each stream below runs a sequence of calls into outputs of its
own while the other stream runs another; every output must equal the same call run alone.
"""
import numpy as np
import pytest
import torch

from aipu_amd import device as dev
from oracle import q4k_oracle as qo

from .gpu_util import d_bf16, h_bits, note, random_weights_gpu

pytestmark = pytest.mark.gpu
Q4K = qo.GGML_Q4_K
BF16 = 30
REPEAT = 12


def test_two_streams_overlap():
    note("two streams: GEMV batches beside MoE steps")
    g = torch.Generator(device="cuda")
    g.manual_seed(5151)
    rng = np.random.default_rng(5151)
    N = K = 6144
    w = random_weights_gpu(Q4K, N, K, g)
    xg = [d_bf16(qo.random_bf16(rng, (1 + i % 3, K))) for i in range(REPEAT)]
    E, H, I, topk = 32, 6144, 2048, 8
    ge = random_weights_gpu(Q4K, E * I, H, g)
    ue = random_weights_gpu(Q4K, E * I, H, g)
    de = random_weights_gpu(Q4K, E * H, I, g)
    rw = d_bf16(qo.random_bf16(rng, (E, H), scale=0.05))
    xm = [d_bf16(qo.random_bf16(rng, H, scale=0.05)) for _ in range(REPEAT)]
    wsa = [dev.moe_workspace(E, H, I, topk, "cuda") for _ in range(2)]

    def gemv_seq(outs):
        for i in range(REPEAT):
            dev.gemv(Q4K, w, N, K, xg[i], mode="fast", out=outs[i])

    def moe_seq(outs, ws):
        for i in range(REPEAT):
            dev.moe_swiglu_decode(BF16, rw, Q4K, ge, ue, de, E, H, I, topk, xm[i], mode="fast", workspace=ws,
                                  out=outs[i])

    alone_g = [torch.empty((x.shape[0], N), dtype=torch.bfloat16, device="cuda") for x in xg]
    alone_m = [torch.empty(H, dtype=torch.bfloat16, device="cuda") for _ in range(REPEAT)]
    gemv_seq(alone_g)
    moe_seq(alone_m, wsa[0])
    torch.cuda.synchronize()
    alone_g = [h_bits(t) for t in alone_g]
    alone_m = [h_bits(t) for t in alone_m]

    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    for rnd in range(2):
        og = [torch.full((x.shape[0], N), 3.0, dtype=torch.bfloat16, device="cuda") for x in xg]
        om1 = [torch.full((H,), 3.0, dtype=torch.bfloat16, device="cuda") for _ in range(REPEAT)]
        om2 = [torch.full((H,), 3.0, dtype=torch.bfloat16, device="cuda") for _ in range(REPEAT)]
        torch.cuda.synchronize()
        note(f"  round {rnd}: GEMV and MoE on one stream each, a second MoE sequence after the GEMVs")
        with torch.cuda.stream(s1):
            gemv_seq(og)
            moe_seq(om2, wsa[1])
        with torch.cuda.stream(s2):
            moe_seq(om1, wsa[0])
        torch.cuda.synchronize()
        for i in range(REPEAT):
            assert np.array_equal(h_bits(og[i]), alone_g[i]), f"round {rnd}: GEMV call {i} differs from alone"
            assert np.array_equal(h_bits(om1[i]), alone_m[i]), f"round {rnd}: MoE call {i} (stream 2) differs"
            assert np.array_equal(h_bits(om2[i]), alone_m[i]), f"round {rnd}: MoE call {i} (stream 1) differs"
    assert not dev.wait_timeouts(), "a bounded wait gave up"
