"""Pins the oracle's router decision (model/forward.rs:2658-2705) without
restating its loops: one-hot router rows make each logit exactly x[e], so
the selection must be numpy's stable descending order of x and the
probabilities the float64 softmax; equal logits must select in index order
(first index wins, as torch.topk); the renormalized weights sum to 1; and
the two error variants in the reference's order."""
import numpy as np
import pytest

import oracle


def f64_softmax(z):
    z = np.asarray(z, np.float64)
    e = np.exp(z - z.max())
    return e / e.sum()


@pytest.mark.parametrize("n_experts,top_k", [(8, 2), (128, 8), (5, 5), (64, 1)])
def test_one_hot_router_selects_the_largest_inputs(n_experts, top_k):
    rng = np.random.default_rng(n_experts)
    x = rng.standard_normal(n_experts).astype(np.float32) * 3
    router = np.eye(n_experts, dtype=np.float32)  # logit e = 1 * x[e] + 0 * ... exactly
    ex, w = oracle.router_topk(x, router, n_experts, top_k, False)
    want = np.argsort(-x.astype(np.float64), kind="stable")[:top_k]
    assert list(ex) == list(want)
    p = f64_softmax(x)
    np.testing.assert_allclose(w, p[want], rtol=2e-6, atol=0)
    assert np.all(np.diff(w) <= 0)  # descending probability
    exn, wn = oracle.router_topk(x, router, n_experts, top_k, True)
    assert list(exn) == list(ex)
    assert abs(float(np.sum(wn, dtype=np.float64)) - 1.0) < 4e-7 * top_k
    np.testing.assert_allclose(wn, p[want] / p[want].sum(), rtol=3e-6)


def test_equal_logits_select_in_index_order():
    # All logits equal: probabilities 1/n each, the scan takes 0, 1, 2, ...
    n, k = 16, 6
    router = np.zeros((n, 32), np.float32)
    ex, w = oracle.router_topk(np.ones(32, np.float32), router, n, k, False)
    assert list(ex) == list(range(k))
    assert np.all(w == np.float32(1.0 / n))
    # Two tied maxima: the lower index first.
    x = np.array([0.5, 2.0, 1.0, 2.0], np.float32)
    ex, _ = oracle.router_topk(x, np.eye(4, dtype=np.float32), 4, 3, False)
    assert list(ex) == [1, 3, 2]


def test_random_router_matches_float64_textbook():
    rng = np.random.default_rng(7)
    hidden, n_experts, k = 256, 32, 4
    router = (rng.standard_normal((n_experts, hidden)) * 0.05).astype(np.float32)
    for _ in range(20):
        x = rng.standard_normal(hidden).astype(np.float32)
        logits = router.astype(np.float64) @ x.astype(np.float64)
        ex, w = oracle.router_topk(x, router, n_experts, k, False)
        order = np.argsort(-logits, kind="stable")[:k]
        gaps = np.sort(-logits)[:k + 1]
        if np.min(np.diff(gaps)) > 1e-4:  # selection is unambiguous in f32
            assert list(ex) == list(order)
        np.testing.assert_allclose(w, f64_softmax(logits)[ex], rtol=1e-5)


def test_errors_in_the_reference_order():
    with pytest.raises(oracle.OracleError) as ei:
        oracle.router_topk(np.ones(4, np.float32), np.ones(8, np.float32), 2, 0, False)
    assert ei.value.code == oracle.RV_FWD_INVALID_TOP_K
    with pytest.raises(oracle.OracleError) as ei:
        oracle.router_topk(np.ones(4, np.float32), np.ones(8, np.float32), 2, 3, False)
    assert ei.value.code == oracle.RV_FWD_INVALID_TOP_K
    with pytest.raises(oracle.OracleError) as ei:
        oracle.router_topk(np.zeros(0, np.float32), np.zeros(0, np.float32), 2, 1, False)
    assert ei.value.code == oracle.RV_PRIM_EMPTY
