"""GPU parity of the batched MoE step (aipu_moe_swiglu_decode_batched) through the C ABI.
Reference mode: bit-exact against the oracle (per-row routing; for M > 1 each row combines
its experts in ascending expert index, src/glm_decoder_block_q4k.v:530-560,836-906), and at
topk = 2 equal to single-row calls (the reference's batch check, Makefile:1490-1508).  Fast
mode (union of experts evaluated once on the matrix cores): routing equal to the reference
tail on the fast logits, outputs within the magnitude bound of the single-row fast tests."""
import numpy as np
import pytest
import torch

from aipu_amd import device as dev
from oracle import glm_oracle as go
from oracle import q4k_oracle as qo

from .gpu_util import assert_bits_equal, d_bf16, d_u8, h_bits, note, random_weights_gpu

pytestmark = pytest.mark.gpu
Q4K = qo.GGML_Q4_K
BF16 = 30


def _case(rng, E, H, I, router_type):
    if router_type == BF16:
        rw = qo.random_bf16(rng, (E, H), scale=0.05).view(np.uint8).reshape(-1)
    else:
        rw = qo.random_q4k_blocks(rng, E * H // 256)
    ex = tuple(qo.random_q4k_blocks(rng, E * I * H // 256) for _ in range(3))
    sh = tuple(qo.random_q4k_blocks(rng, I * H // 256) for _ in range(3))
    return rw, ex, sh


def _run(router_type, rw, ex, sh, E, H, I, topk, X, mode):
    shd = tuple(d_u8(a) for a in sh) if sh is not None else None
    y, sel, sw = dev.moe_swiglu_decode_batched(router_type, d_u8(rw), Q4K, *(d_u8(a) for a in ex), E, H, I, topk,
                                               d_bf16(X), mode=mode, shared=shd)
    return h_bits(y), sel.cpu().numpy(), h_bits(sw)


@pytest.mark.parametrize("M,router_type,shared,topk", [(1, Q4K, True, 4), (2, Q4K, True, 4), (3, BF16, False, 4),
                                                       (5, Q4K, True, 3), (9, BF16, True, 4)])
def test_batched_ref_bitexact(M, router_type, shared, topk):
    E, H, I = 16, 512, 256
    note(f"moe batched ref M={M} router={router_type} shared={shared} topk={topk}")
    rng = np.random.default_rng(M * 13 + topk)
    rw, ex, sh = _case(rng, E, H, I, router_type)
    sh = sh if shared else None
    X = qo.random_bf16(rng, (M, H), scale=0.05)
    y, sel, sw = _run(router_type, rw, ex, sh, E, H, I, topk, X, "ref")
    r = go.moe_decode_batched_ref(X, router_type, rw, ex, Q4K, E, H, I, topk, shared=sh)
    assert np.array_equal(sel, r["sel_idx"])
    assert_bits_equal(sw, r["sel_w"], "sel_w")
    assert_bits_equal(y, r["y"], "y")


def test_batched_ref_topk2_equals_single_rows():
    E, H, I, topk, M = 16, 512, 256, 2, 4
    note("moe batched topk=2 vs single rows")
    rng = np.random.default_rng(5)
    rw, ex, sh = _case(rng, E, H, I, Q4K)
    X = qo.random_bf16(rng, (M, H), scale=0.05)
    y, _, _ = _run(Q4K, rw, ex, sh, E, H, I, topk, X, "ref")
    for r in range(M):
        ys, _, _ = dev.moe_swiglu_decode(Q4K, d_u8(rw), Q4K, *(d_u8(a) for a in ex), E, H, I, topk, d_bf16(X[r]),
                                         mode="ref", shared=tuple(d_u8(a) for a in sh))
        assert_bits_equal(y[r], h_bits(ys), f"row {r}")


def _check_fast(y, sel, sw, X, router_type, rw, ex, sh, E, H, I, topk):
    M = X.shape[0]
    lf = h_bits(dev.gemv(router_type, d_u8(rw), E, H, d_bf16(X), mode="fast"))
    ge, ue, de = (a.reshape(E, -1) for a in ex)
    for r in range(M):
        es, ew, _ = go.router_tail(lf[r], topk)
        assert np.array_equal(sel[r], es), f"row {r} routing"
        assert_bits_equal(sw[r], ew, f"row {r} sel_w")
        order = np.argsort(es, kind="stable")
        ys, mag = [], np.zeros(H)
        slots = [(ge[es[t]], ue[es[t]], de[es[t]], ew[t]) for t in order]
        if sh is not None:
            slots.append((sh[0], sh[1], sh[2], qo.bf16_round_bits(np.float32(1.0))))
        for g_, u_, d_, w in slots:
            yo, ho = go.swiglu_expert(X[r], g_, u_, d_, Q4K, H, I)
            ys.append(yo)
            mag += abs(float(qo.bf16_bits_to_f32(int(w)))) * (np.abs(qo.dequant_q4k(d_).reshape(H, I)) @
                                                             np.abs(qo.bf16_bits_to_f32(ho).astype(np.float64)))
        if sh is not None:
            yref, _ = go.moe_combine(ew[order], ys[:-1], ys[-1])
        else:
            yref, _ = go.moe_combine(ew[order], ys)
        a = qo.bf16_bits_to_f32(y[r]).astype(np.float64)
        b = qo.bf16_bits_to_f32(yref).astype(np.float64)
        assert np.all(np.abs(a - b) <= 2.0 ** -7 * mag + 2.0 ** -6 * np.abs(b)), f"row {r}"


@pytest.mark.parametrize("M,router_type,shared,topk", [(2, Q4K, True, 4), (4, BF16, False, 4), (8, Q4K, True, 8),
                                                       (11, BF16, True, 3), (3, Q4K, False, 8), (6, BF16, True, 4),
                                                       (2, BF16, False, 8)])
def test_batched_fast_small(M, router_type, shared, topk):
    E, H, I = 16, 512, 256
    note(f"moe batched fast M={M} router={router_type} shared={shared} topk={topk}")
    rng = np.random.default_rng(M * 7 + topk + 100)
    rw, ex, sh = _case(rng, E, H, I, router_type)
    sh = sh if shared else None
    X = qo.random_bf16(rng, (M, H), scale=0.05)
    y, sel, sw = _run(router_type, rw, ex, sh, E, H, I, topk, X, "fast")
    _check_fast(y, sel, sw, X, router_type, rw, ex, sh, E, H, I, topk)


@pytest.mark.parametrize("shared", [True, False])
def test_batched_fast_more_experts_than_one_workgroup_routes(shared):
    """E = 600 > 512: a pass routes its rows with the one-wave tail kernel and forms the union
    in a separate launch (the one-workgroup routing-and-union kernel takes E <= 512)."""
    E, H, I, topk, M = 600, 256, 256, 4, 3
    note(f"moe batched fast E={E} shared={shared}")
    rng = np.random.default_rng(600 + shared)
    rw, ex, sh = _case(rng, E, H, I, BF16)
    sh = sh if shared else None
    X = qo.random_bf16(rng, (M, H), scale=0.05)
    y, sel, sw = _run(BF16, rw, ex, sh, E, H, I, topk, X, "fast")
    _check_fast(y, sel, sw, X, BF16, rw, ex, sh, E, H, I, topk)


@pytest.mark.parametrize("M", [2, 4])
def test_batched_fast_c2_shape(M):
    """Config-2 expert shape (6144 <-> 2048, top-8) over 32 experts, shared expert; two rows
    (gate and up of a tile in one workgroup, SwiGLU fused) and four."""
    E, H, I, topk = 32, 6144, 2048, 8
    note(f"moe batched fast C2 shape M={M}")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(8)
    exd = tuple(random_weights_gpu(Q4K, E * I, H, gen) if k < 2 else random_weights_gpu(Q4K, E * H, I, gen)
                for k in range(3))
    shd = (random_weights_gpu(Q4K, I, H, gen), random_weights_gpu(Q4K, I, H, gen), random_weights_gpu(Q4K, H, I, gen))
    rng = np.random.default_rng(8)
    rw = qo.random_bf16(rng, (E, H), scale=0.05).view(np.uint8).reshape(-1)
    X = qo.random_bf16(rng, (M, H), scale=0.05)
    y, sel, sw = dev.moe_swiglu_decode_batched(BF16, d_u8(rw), Q4K, *exd, E, H, I, topk, d_bf16(X), mode="fast",
                                               shared=shd)
    ex = tuple(t.cpu().numpy() for t in exd)
    sh = tuple(t.cpu().numpy() for t in shd)
    _check_fast(h_bits(y), sel.cpu().numpy(), h_bits(sw), X, BF16, rw, ex, sh, E, H, I, topk)


@pytest.mark.parametrize("H,I,topk", [(512, 256, 4), (6144, 2048, 8)])
def test_batched_fast_rows_independent_of_batch(H, I, topk):
    """Fast mode: a row's output, routing and weights do not depend on which other rows share
    its batch (M >= 2, where every row combines its experts in ascending index): the rows of an
    8-row batch equal the same rows run as batches of 2, 3 and 5 (the batch sizes that split
    into different passes), bit for bit."""
    E, M = 32, 8
    note(f"moe batched fast batch composition H={H} I={I} topk={topk}")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(H + topk)
    exd = tuple(random_weights_gpu(Q4K, E * I, H, gen) if k < 2 else random_weights_gpu(Q4K, E * H, I, gen)
                for k in range(3))
    shd = (random_weights_gpu(Q4K, I, H, gen), random_weights_gpu(Q4K, I, H, gen), random_weights_gpu(Q4K, H, I, gen))
    rng = np.random.default_rng(H + topk)
    rw = qo.random_bf16(rng, (E, H), scale=0.05).view(np.uint8).reshape(-1)
    X = qo.random_bf16(rng, (M, H), scale=0.05)

    def run(rows):
        y, sel, sw = dev.moe_swiglu_decode_batched(BF16, d_u8(rw), Q4K, *exd, E, H, I, topk, d_bf16(X[rows]),
                                                   mode="fast", shared=shd)
        return h_bits(y), sel.cpu().numpy(), h_bits(sw)

    y8, sel8, sw8 = run(list(range(M)))
    for rows in ([0, 1], [2, 3, 4], [3, 4, 5, 6, 7], [7, 0]):
        y, sel, sw = run(rows)
        for i, r in enumerate(rows):
            assert np.array_equal(sel[i], sel8[r]), f"row {r} routing in batch {rows}"
            assert_bits_equal(sw[i], sw8[r], f"row {r} sel_w in batch {rows}")
            assert_bits_equal(y[i], y8[r], f"row {r} y in batch {rows}")


@pytest.mark.parametrize("H,topk,shared", [(2048, 4, False), (4096, 8, True), (6144, 3, False), (6144, 8, False)])
def test_batched_fast_two_row_pass_equals_one_row_pass(H, topk, shared):
    """At I = 2048 and H = 2048 R, with and without the shared expert and at topk 3 / 4 / 8: a
    row of a two-row pass (both rows on every union expert) and the same row as the odd row of a
    three-row batch (a one-row pass over its own experts) agree bit for bit in output, routing
    and weights, and the two-row batch passes the fast-mode gate."""
    E, I = 32, 2048
    note(f"moe batched fast two-row pass H={H} topk={topk} shared={shared}")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(H + 10 * topk + shared)
    exd = tuple(random_weights_gpu(Q4K, E * I, H, gen) if k < 2 else random_weights_gpu(Q4K, E * H, I, gen)
                for k in range(3))
    shd = ((random_weights_gpu(Q4K, I, H, gen), random_weights_gpu(Q4K, I, H, gen), random_weights_gpu(Q4K, H, I, gen))
           if shared else None)
    rng = np.random.default_rng(H + topk)
    rw = qo.random_bf16(rng, (E, H), scale=0.05).view(np.uint8).reshape(-1)
    X = qo.random_bf16(rng, (4, H), scale=0.05)

    def run(rows):
        y, sel, sw = dev.moe_swiglu_decode_batched(BF16, d_u8(rw), Q4K, *exd, E, H, I, topk, d_bf16(X[rows]),
                                                   mode="fast", shared=shd)
        return h_bits(y), sel.cpu().numpy(), h_bits(sw)

    y2, sel2, sw2 = run([0, 1])
    for r in (0, 1):
        y3, sel3, sw3 = run([2, 3, r])   # row r alone in the second pass
        assert np.array_equal(sel3[2], sel2[r]), f"row {r} routing"
        assert_bits_equal(sw3[2], sw2[r], f"row {r} sel_w")
        assert_bits_equal(y3[2], y2[r], f"row {r} y")
    ex = tuple(t.cpu().numpy() for t in exd)
    sh = tuple(t.cpu().numpy() for t in shd) if shared else None
    _check_fast(y2, sel2, sw2, X[:2], BF16, rw, ex, sh, E, H, I, topk)


def _random_batched_cases(n=10, seed=1505):
    """Seeded batched MoE shapes: M = 1..9 rows, E = topk..64 experts, H = 256..3072, I = 256..1536,
    top-1..8, bf16 or Q4_K router, with or without the shared expert."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        topk = int(rng.integers(1, 9))
        out.append((int(rng.integers(1, 10)), int(rng.integers(max(topk, 2), 65)), 256 * int(rng.integers(1, 13)),
                    256 * int(rng.integers(1, 7)), topk, BF16 if rng.integers(0, 2) else Q4K, bool(rng.integers(0, 2))))
    return out


@pytest.mark.parametrize("mode", ["ref", "fast"])
@pytest.mark.parametrize("M,E,H,I,topk,router_type,shared", _random_batched_cases())
def test_batched_random_shapes(M, E, H, I, topk, router_type, shared, mode):
    """The batched step at seeded random shapes: ref mode bit-exact against the oracle; fast mode
    routed on its own logits within the fast-mode bound, and (from three rows) each row's bits
    independent of the batch's order."""
    note(f"moe batched random {mode} M={M} E={E} H={H} I={I} topk={topk} router={router_type} shared={shared}")
    rng = np.random.default_rng(M * 100000 + E * 1000 + H + I + topk)
    rw, ex, sh = _case(rng, E, H, I, router_type)
    sh = sh if shared else None
    X = qo.random_bf16(rng, (M, H), scale=0.05)
    y, sel, sw = _run(router_type, rw, ex, sh, E, H, I, topk, X, mode)
    if mode == "ref":
        r = go.moe_decode_batched_ref(X, router_type, rw, ex, Q4K, E, H, I, topk, shared=sh)
        assert np.array_equal(sel, r["sel_idx"])
        assert_bits_equal(sw, r["sel_w"], "sel_w")
        assert_bits_equal(y, r["y"], "y")
        return
    _check_fast(y, sel, sw, X, router_type, rw, ex, sh, E, H, I, topk)
    if M >= 3:
        yr, selr, swr = _run(router_type, rw, ex, sh, E, H, I, topk, X[::-1].copy(), mode)
        assert np.array_equal(selr[::-1], sel), "routing depends on the batch order"
        assert_bits_equal(swr[::-1], sw, "sel_w with the batch reversed")
        assert_bits_equal(yr[::-1], y, "y with the batch reversed")
