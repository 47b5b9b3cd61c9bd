"""GPU: the entry points inside a captured HIP graph.

Serving loops capture a decode step once and replay it.  Each entry point below is called once
eagerly, then all of them are captured into one graph (on torch's capture stream, with the
workspaces the caller owns), and the graph is replayed several times.  Before every replay the
outputs are overwritten and unrelated eager work (other launches of the same kernels on other
inputs, a host synchronisation) runs; after it every output must equal the eager result bit
for bit.  This covers persistent kernels whose LDS counters and workspace words must start
from the same state on every launch, and workspaces that the library expects zero-filled at
creation and leaves reusable.
"""
import numpy as np
import pytest
import torch

from aipu_amd import device as dev
from oracle import q4k_oracle as qo

from .gpu_util import d_bf16, d_u8, h_bits, note, random_weights_gpu

pytestmark = pytest.mark.gpu
Q4K = qo.GGML_Q4_K
BF16 = 30
REPLAYS = 4


def _ops():
    """(name, closure writing its outputs, list of output tensors, closure running the same kernels
    on other inputs) for every entry point of the decode and prefill paths."""
    g = torch.Generator(device="cuda")
    g.manual_seed(4242)
    rng = np.random.default_rng(4242)
    ops = []

    # Q4_K GEMV, fast: one row (k_gemv1p), two rows (two-row k_gemv1p), eight rows (k_gemvmp); ref mode
    N = K = 6144
    w = random_weights_gpu(Q4K, N, K, g)
    xs = {m: d_bf16(qo.random_bf16(rng, (m, K))) for m in (1, 2, 8)}
    other = d_bf16(qo.random_bf16(rng, (8, K)))
    for m in (1, 2, 8):
        y = torch.empty((m, N), dtype=torch.bfloat16, device="cuda")
        yo = torch.empty((8, N), dtype=torch.bfloat16, device="cuda")
        ops.append((f"gemv fast M={m}", lambda m=m, y=y: dev.gemv(Q4K, w, N, K, xs[m], mode="fast", out=y), [y],
                    lambda m=m, yo=yo: dev.gemv(Q4K, w, N, K, other[:m], mode="fast", out=yo[:m])))
    yr = torch.empty((1, N), dtype=torch.bfloat16, device="cuda")
    ops.append(("gemv ref M=1", lambda: dev.gemv(Q4K, w, N, K, xs[1], mode="ref", out=yr), [yr],
                lambda: dev.gemv(Q4K, w, N, K, other[:1], mode="ref")))

    # mixed-type tiles (one launch over all tiles, three rows)
    Kt, rows = 2048, 256
    types = [Q4K, qo.GGML_Q6_K, qo.GGML_Q8_0, qo.GGML_F16]
    tiles = [(t, d_u8(qo.random_weights(rng, t, rows, Kt)), i * rows, rows) for i, t in enumerate(types)]
    xt = d_bf16(qo.random_bf16(rng, (3, Kt)))
    xto = d_bf16(qo.random_bf16(rng, (3, Kt)))
    yt = torch.empty((3, rows * len(types)), dtype=torch.bfloat16, device="cuda")
    ops.append(("tiles fast M=3", lambda: dev.gemv_tiles(tiles, rows * len(types), Kt, xt, mode="fast", out=yt), [yt],
                lambda: dev.gemv_tiles(tiles, rows * len(types), Kt, xto, mode="fast")))

    # MoE step (config-2 widths, 32 experts), both modes, with caller-owned workspaces
    E, H, I, topk = 32, 6144, 2048, 8
    ge = random_weights_gpu(Q4K, E * I, H, g)
    ue = random_weights_gpu(Q4K, E * I, H, g)
    de = random_weights_gpu(Q4K, E * H, I, g)
    rw = d_bf16(qo.random_bf16(rng, (E, H), scale=0.05))
    xm = d_bf16(qo.random_bf16(rng, H, scale=0.05))
    xmo = d_bf16(qo.random_bf16(rng, H, scale=0.05))
    for mode in ("fast", "ref"):
        ws = dev.moe_workspace(E, H, I, topk, "cuda")
        y = torch.empty(H, dtype=torch.bfloat16, device="cuda")
        sel = torch.empty(topk, dtype=torch.int32, device="cuda")
        sw = torch.empty(topk, dtype=torch.bfloat16, device="cuda")
        ops.append((f"moe {mode}", lambda mode=mode, ws=ws, y=y, sel=sel, sw=sw: dev.moe_swiglu_decode(
            BF16, rw, Q4K, ge, ue, de, E, H, I, topk, xm, mode=mode, workspace=ws, out=y, sel_out=(sel, sw)),
            [y, sel, sw], lambda mode=mode: dev.moe_swiglu_decode(BF16, rw, Q4K, ge, ue, de, E, H, I, topk, xmo,
                                                                  mode=mode)))

    # batched MoE step, three rows, fast
    wsb = dev.moe_batched_workspace(E, H, I, topk, "cuda")
    xb = d_bf16(qo.random_bf16(rng, (3, H), scale=0.05))
    yb = torch.empty((3, H), dtype=torch.bfloat16, device="cuda")
    ops.append(("moe batched fast M=3", lambda: dev.moe_swiglu_decode_batched(
        BF16, rw, Q4K, ge, ue, de, E, H, I, topk, xb, mode="fast", workspace=wsb, out=yb), [yb],
        lambda: dev.moe_swiglu_decode_batched(BF16, rw, Q4K, ge, ue, de, E, H, I, topk, xb[:2], mode="fast")))

    # FFN half (RMSNorm, Q4_K router, experts, residual), fast
    rq = random_weights_gpu(Q4K, E, H, g)
    gam = d_bf16(qo.bf16_round_bits(np.float32(1.0) + np.float32(0.1) * rng.standard_normal(H).astype(np.float32)))
    hl = d_bf16(qo.random_bf16(rng, H, scale=0.5))
    wsl = dev.moe_layer_workspace(E, H, I, topk, "cuda")
    yl = torch.empty(H, dtype=torch.bfloat16, device="cuda")
    sl = torch.empty(topk, dtype=torch.int32, device="cuda")
    swl = torch.empty(topk, dtype=torch.bfloat16, device="cuda")
    ops.append(("moe layer fast", lambda: dev.moe_layer_decode(
        Q4K, rq, Q4K, ge, ue, de, E, H, I, topk, hl, gam, mode="fast", workspace=wsl, out=yl, sel_out=(sl, swl)),
        [yl, sl, swl], lambda: dev.moe_layer_decode(Q4K, rq, Q4K, ge, ue, de, E, H, I, topk, xm, gam, mode="fast")))

    # prefill GEMM
    Mp, Np, Kp = 130, 512, 2048
    wp = random_weights_gpu(Q4K, Np, Kp, g)
    xp = d_bf16(qo.random_bf16(rng, (Mp, Kp)))
    xpo = d_bf16(qo.random_bf16(rng, (Mp, Kp)))
    wsp = dev.prefill_workspace(Mp, Kp, "cuda")
    yp = torch.empty((Mp, Np), dtype=torch.bfloat16, device="cuda")
    ops.append(("prefill", lambda: dev.gemm_prefill(Q4K, wp, Np, Kp, xp, out=yp, workspace=wsp), [yp],
                lambda: dev.gemm_prefill(Q4K, wp, Np, Kp, xpo)))

    # LM head + argmax (outputs allocated by the wrapper: the captured call's tensors are kept)
    V, Kl = 3000, 6144
    wl = d_bf16(qo.random_bf16(rng, (V, Kl)))
    xl = d_bf16(qo.random_bf16(rng, Kl))
    wsh = dev.lm_head_workspace(V, "cuda")
    held = {}

    def lm():
        held["out"] = dev.lm_head(wl, xl, workspace=wsh)
        return held["out"]

    ops.append(("lm head", lm, None, lambda: dev.lm_head(wl, d_bf16(qo.random_bf16(np.random.default_rng(1), Kl)))))

    # RMSNorm, fast
    xn = d_bf16(qo.random_bf16(rng, H, scale=0.5))
    yn = torch.empty(H, dtype=torch.bfloat16, device="cuda")
    ops.append(("rmsnorm fast", lambda: dev.rmsnorm(xn, gam, mode="fast", out=yn), [yn],
                lambda: dev.rmsnorm(xm, gam, mode="fast")))
    return ops, held


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy() if t.dtype == torch.bfloat16 else t.cpu().numpy()


def test_entry_points_in_graph_replays():
    note("graph capture of every entry point")
    ops, held = _ops()
    eager = {}
    for name, fn, outs, _ in ops:
        note(f"  eager {name}")
        r = fn()
        outs = outs if outs is not None else [t for t in r if t is not None]
        eager[name] = [_bits(t) for t in outs]
    torch.cuda.synchronize()
    # warm-up on a side stream, as torch's graph capture expects
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _, fn, _, _ in ops:
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    captured = {}
    note("  capture")
    with torch.cuda.graph(graph):
        for name, fn, outs, _ in ops:
            r = fn()
            captured[name] = outs if outs is not None else [t for t in r if t is not None]
    torch.cuda.synchronize()
    for rep in range(REPLAYS):
        for name in captured:
            for t in captured[name]:
                t.fill_(-7 if t.dtype == torch.int32 else 3.0)
        for name, _, _, other in ops:
            other()
        torch.cuda.synchronize()
        note(f"  replay {rep}")
        graph.replay()
        torch.cuda.synchronize()
        for name in captured:
            got = [_bits(t) for t in captured[name]]
            for i, (a, b) in enumerate(zip(got, eager[name])):
                assert np.array_equal(a, b), f"replay {rep}: {name} output {i} differs from the eager call"
    assert not dev.wait_timeouts(), "a bounded wait gave up"
