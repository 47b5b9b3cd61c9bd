"""Fast-mode routing against the reference's routing, on the CPU.

The fast MoE step routes from logits that its own router kernel forms in a different fp32
order than the reference's sequential sum (tools/glm_model_q4k_ref.py:663-668).  The oracle
models that order (glm_oracle.router_logits_fast_order; the GPU tests check the kernel's
logits against the model).  Here the model is pinned by cases whose sums are exact in any
order, then used to count, over 1,000 BASELINE config-2 inputs, how often the fast logits and
the reference logits select different experts.
"""
import numpy as np
import pytest

from oracle import glm_oracle as go
from oracle import q4k_oracle as qo


def _ref_logits(rw, x):
    return qo.gemv_ref(qo.bf16_bits_to_f32(rw), qo.bf16_bits_to_f32(np.atleast_2d(x)))[1]


def test_fast_order_model_exact_sums():
    """Small-integer weights and activations: every partial sum is exact in fp32, so any order
    gives the reference's logits -- a dropped, doubled or misplaced element does not."""
    rng = np.random.default_rng(5)
    E, H = 16, 6144
    rw = qo.bf16_round_bits(rng.integers(-3, 4, (E, H)).astype(np.float32))
    x = qo.bf16_round_bits(rng.integers(-2, 3, (3, H)).astype(np.float32))
    assert np.array_equal(go.router_logits_fast_order(rw, E, H, x), _ref_logits(rw, x))
    # a planted mistake in the model's index map (element c + 1 read twice) is caught
    bad = rw.copy().reshape(E, H)
    bad[:, 1::8] = bad[:, 0::8]
    assert not np.array_equal(go.router_logits_fast_order(bad, E, H, x), _ref_logits(rw, x))


@pytest.mark.parametrize("H", [6144, 2048, 1280])
def test_fast_order_model_one_hot(H):
    """x = e_k picks w[:, k] exactly in both orders, for every k of a sweep (each element is
    counted once, with its own weight), including H that leaves threads without a chunk."""
    rng = np.random.default_rng(H)
    E = 8
    rw = qo.random_bf16(rng, (E, H), scale=0.05)
    ks = np.unique(np.concatenate([np.arange(16), rng.integers(0, H, 48), [H - 1]]))
    x = np.zeros((len(ks), H), np.uint16)
    x[np.arange(len(ks)), ks] = 0x3F80                           # 1.0
    got = go.router_logits_fast_order(rw, E, H, x)
    assert np.array_equal(got, rw.reshape(E, H)[:, ks].T)


def test_fast_vs_reference_routing_c2():
    """BASELINE config 2 (E = 256, H = 6144, top-8, bf16 router N(0, 0.05^2), activations
    N(0, 0.05^2), as bench.py draws them): over 1,000 inputs, count logits that differ between
    the fast order and the reference order, and decisions that differ (expert set, slot order,
    slot weights).  The counts are the fast mode's stated routing contract."""
    E, H, topk, n = 256, 6144, 8, 1000
    rng = np.random.default_rng(2026)
    rw = qo.random_bf16(rng, (E, H), scale=0.05)
    X = qo.random_bf16(rng, (n, H), scale=0.05)
    lf = np.concatenate([go.router_logits_fast_order(rw, E, H, X[i:i + 25]) for i in range(0, n, 25)])
    acc_r, lr = qo.gemv_ref(qo.bf16_bits_to_f32(rw), qo.bf16_bits_to_f32(X))
    n_logit = int((lf != lr).sum())
    n_set = n_order = n_weight = 0
    for i in range(n):
        sf, wf, _ = go.router_tail(lf[i], topk)
        sr, wr, _ = go.router_tail(lr[i], topk)
        if set(sf.tolist()) != set(sr.tolist()):
            n_set += 1
        elif not np.array_equal(sf, sr):
            n_order += 1
        elif not np.array_equal(wf, wr):
            n_weight += 1
    print(f"\nfast vs reference routing over {n} inputs: {n_logit} of {n * E} logits differ; "
          f"expert set differs in {n_set}, slot order only in {n_order}, slot weights only in {n_weight}")
    # the orders round the same sums differently: within one bf16 ulp where the sum is well
    # conditioned, within the accumulator tolerance where it cancels
    ok, max_ulp, n_cancelled = qo.bf16_parity(lf, acc_r, qo.bf16_bits_to_f32(rw), qo.bf16_bits_to_f32(X))
    assert ok, f"fast-order logits {max_ulp} ulp from the reference ({n_cancelled} cancelled sums)"
    assert n_logit <= 0.002 * n * E
    assert n_set <= 0.01 * n
