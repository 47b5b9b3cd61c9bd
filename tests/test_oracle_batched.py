"""Pins of the batched-MoE oracle (oracle/glm_oracle.py moe_decode_batched_ref): M = 1 is
the single-row step; with topk = 2 the ascending-index combine of M > 1 equals the slot-order
combine (two fp32 adds from +0 commute -- the reference's own batch-vs-single-row check,
Makefile:1490-1508, runs at TOPK = 2); rows are independent of their batch companions; and
a designed combine where order matters shows the ascending order is the one applied."""
import numpy as np

from oracle import glm_oracle as go
from oracle import q4k_oracle as qo

Q4K = qo.GGML_Q4_K


def _case(rng, E, H, I):
    rw = qo.random_q4k_blocks(rng, E * H // 256)
    ex = tuple(qo.random_q4k_blocks(rng, E * I * H // 256) for _ in range(3))
    sh = tuple(qo.random_q4k_blocks(rng, I * H // 256) for _ in range(3))
    return rw, ex, sh


def test_single_row_is_slot_order():
    rng = np.random.default_rng(1)
    E, H, I, topk = 8, 256, 256, 3
    rw, ex, sh = _case(rng, E, H, I)
    x = qo.random_bf16(rng, (1, H), scale=0.1)
    b = go.moe_decode_batched_ref(x, Q4K, rw, ex, Q4K, E, H, I, topk, shared=sh)
    s = go.moe_decode_ref(x[0], Q4K, rw, ex, Q4K, E, H, I, topk, shared=sh)
    np.testing.assert_array_equal(b["y"][0], s["y"])
    assert list(b["sel_idx"][0]) == list(s["sel_idx"])


def test_topk2_batch_equals_single_rows_and_rows_are_independent():
    rng = np.random.default_rng(2)
    E, H, I, topk = 8, 256, 256, 2
    rw, ex, sh = _case(rng, E, H, I)
    X = qo.random_bf16(rng, (3, H), scale=0.1)
    b = go.moe_decode_batched_ref(X, Q4K, rw, ex, Q4K, E, H, I, topk, shared=sh)
    for r in range(3):
        s = go.moe_decode_ref(X[r], Q4K, rw, ex, Q4K, E, H, I, topk, shared=sh)
        np.testing.assert_array_equal(b["y"][r], s["y"])
    b2 = go.moe_decode_batched_ref(X[[2, 0]], Q4K, rw, ex, Q4K, E, H, I, topk, shared=sh)
    np.testing.assert_array_equal(b2["y"][0], b["y"][2])
    np.testing.assert_array_equal(b2["y"][1], b["y"][0])


def test_ascending_combine_is_what_batches_use():
    """For topk = 4 a batched row equals moe_combine over its experts sorted by index, and
    a designed combine shows the two orders can differ: gates 1 on y = (2^24, 1, 1, -2^24)
    in slot order give 0, in the order (2^24, -2^24, 1, 1) give 2."""
    one = qo.bf16_round_bits(np.float32(1.0))
    ys = [qo.bf16_round_bits(np.full(4, v, np.float32)) for v in (2.0 ** 24, 1.0, 1.0, -(2.0 ** 24))]
    y_slot, _ = go.moe_combine([one] * 4, ys)
    y_sorted, _ = go.moe_combine([one] * 4, [ys[0], ys[3], ys[1], ys[2]])
    assert np.all(qo.bf16_bits_to_f32(y_slot) == 0.0) and np.all(qo.bf16_bits_to_f32(y_sorted) == 2.0)
    rng = np.random.default_rng(3)
    E, H, I, topk = 16, 256, 256, 4
    rw, ex, sh = _case(rng, E, H, I)
    X = qo.random_bf16(rng, (2, H), scale=0.1)
    b = go.moe_decode_batched_ref(X, Q4K, rw, ex, Q4K, E, H, I, topk, shared=sh)
    ge, ue, de = (a.reshape(E, -1) for a in ex)
    for r in range(2):
        sel, selw = b["sel_idx"][r], b["sel_w"][r]
        order = np.argsort(sel, kind="stable")
        yo = [go.swiglu_expert(X[r], ge[sel[t]], ue[sel[t]], de[sel[t]], Q4K, H, I)[0] for t in order]
        ysh, _ = go.swiglu_expert(X[r], sh[0], sh[1], sh[2], Q4K, H, I)
        want, _ = go.moe_combine(selw[order], yo, ysh)
        np.testing.assert_array_equal(b["y"][r], want)
