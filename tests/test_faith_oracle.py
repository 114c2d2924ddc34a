"""Pins of the faithfulness oracle (oracle/faith_oracle.py) on the CPU, and the host-side
validation of `make_faithfulness_loss`."""

import numpy as np
import pytest

from oracle import faith_oracle as fo


def test_mean_of_per_site_relative_errors_reference_values():
    # pd/tests/core/test_faithfulness_normalization.py:47-55
    deltas = {"g": np.stack([np.full((2, 2), 2.0), np.full((2, 2), 1.0)]), "h": np.full((1, 1, 4), 1.0)}
    got = fo.loss_from_deltas(deltas, {"g": (8.0, 16.0), "h": (2.0,)}, 3)
    assert got == pytest.approx((16 / 8.0 + 4 / 16.0 + 4 / 2.0) / 3)


def test_sites_weigh_equally_not_by_parameter_count():
    # pd/tests/core/test_faithfulness_normalization.py:58-62
    deltas = {"g": np.ones((1, 2, 2)), "h": np.zeros((1, 100, 100))}
    assert fo.loss_from_deltas(deltas, {"g": (4.0,), "h": (1.0,)}, 2) == pytest.approx(0.5)


def test_block_factored_deltas_reduce_per_slot():
    # pd/tests/core/test_blocked_factorization.py:396-407: a [1, E, ...] stack per group
    rng = np.random.default_rng(0)
    deltas = {"gate": rng.normal(size=(1, 4, 6, 5)), "down": rng.normal(size=(1, 4, 5, 6))}
    norms = {"gate": (3.0,), "down": (7.0,)}
    want = 0.5 * sum(float((deltas[g] ** 2).sum()) / norms[g][0] for g in ("gate", "down"))
    assert fo.loss_from_deltas(deltas, norms, 2) == pytest.approx(want, rel=1e-12)


def test_deltas_match_brute_force():
    rng = np.random.default_rng(1)
    g, d_in, d_out, C = 2, 5, 3, 4
    W, V, U = rng.normal(size=(g, d_out, d_in)), rng.normal(size=(g, d_in, C)), rng.normal(size=(g, C, d_out))
    d = fo.weight_deltas(W, V, U)
    for s in range(g):
        for o in range(d_out):
            for i in range(d_in):
                assert d[s, o, i] == pytest.approx(W[s, o, i] - sum(V[s, i, c] * U[s, c, o] for c in range(C)))


def test_gradients_finite_differences_and_zero_v_closed_form():
    rng = np.random.default_rng(2)
    g, d_in, d_out, C = 2, 4, 3, 5
    W, V, U = rng.normal(size=(g, d_out, d_in)), rng.normal(size=(g, d_in, C)), rng.normal(size=(g, C, d_out))
    norms = np.array([2.0, 5.0])
    scale = 0.25
    f = lambda VV, UU: scale * fo.site_errors(W, VV, UU, norms).sum()
    dV, dU = fo.grads(W, V, U, norms, scale)
    eps = 1e-6
    for idx in [(0, 0, 0), (1, 3, 4), (0, 2, 1)]:
        Vp, Vm = V.copy(), V.copy()
        Vp[idx] += eps
        Vm[idx] -= eps
        assert (f(Vp, U) - f(Vm, U)) / (2 * eps) == pytest.approx(dV[idx], rel=1e-6, abs=1e-9)
    for idx in [(0, 0, 0), (1, 4, 2), (1, 2, 1)]:
        Up, Um = U.copy(), U.copy()
        Up[idx] += eps
        Um[idx] -= eps
        assert (f(V, Up) - f(V, Um)) / (2 * eps) == pytest.approx(dU[idx], rel=1e-6, abs=1e-9)
    # V = 0: Delta = W, so dV = -2 scale/n W^T U^T and dU = 0
    dV0, dU0 = fo.grads(W, np.zeros_like(V), U, norms, scale)
    np.testing.assert_allclose(dV0, -2 * scale / norms[:, None, None] * np.swapaxes(W, 1, 2) @ np.swapaxes(U, 1, 2))
    np.testing.assert_array_equal(dU0, 0)


def test_make_faithfulness_loss_validates_norm_keys_and_values():
    # pd/tests/core/test_faithfulness_normalization.py:65-73
    from param_decomp_amd.faithfulness import make_faithfulness_loss

    idx = (("s", "s", 0),)
    with pytest.raises(AssertionError):
        make_faithfulness_loss(idx, {"not.a.group": (1.0,)}, {})
    with pytest.raises(AssertionError):
        make_faithfulness_loss(idx, {"s": (1.0, 1.0)}, {})
    for value in (0.0, float("nan"), float("inf")):
        with pytest.raises(AssertionError, match="finite positive"):
            make_faithfulness_loss(idx, {"s": (value,)}, {})
    bound = make_faithfulness_loss((("a", "g", 0), ("b", "g", 1)), {"g": (2.0, 3.0)}, {"g": 1})
    assert bound.padded_sq_norms == {"g": (2.0, 3.0, 1.0)} and bound.n_sites == 2
