"""NumPy restatement of faithfulness (oracle only: test infrastructure, never the product
path; float64 arithmetic). Paths are relative to the reference repository root;
`pd/` = `param_decomp/param_decomp/`.

Pins (tests/test_faith_oracle.py): the reference's hand values
(pd/tests/core/test_faithfulness_normalization.py:47-63) and its block-factored
reduction (pd/tests/core/test_blocked_factorization.py:396-407); brute-force loops for the
deltas; finite differences and the closed form at V = 0 for the gradients.
"""

from __future__ import annotations

import numpy as np


def weight_deltas(W, V, U):
    """`pd/targets/transformer.py:2179-2184`: `W - einsum("gic,gco->goi", V, U)` in fp32
    (here float64). W [g, d_out, d_in] (or [g, e, d_out, d_in] with V [g, e, d_in, c],
    U [g, e, c, d_out])."""
    W, V, U = (np.asarray(a, np.float64) for a in (W, V, U))
    return W - np.swapaxes(V @ U, -1, -2)


def loss_from_deltas(deltas: dict, sq_norms: dict, n_sites: int):
    """`pd/core/faithfulness.py:58-75`: per stack index, the squared Frobenius norm over every
    axis but the first, divided by that index's norm; summed over groups and divided by
    the number of real sites (pads carry norm 1.0 and zero deltas)."""
    total = 0.0
    for group, d in deltas.items():
        d = np.asarray(d, np.float64)
        per = (d ** 2).reshape(d.shape[0], -1).sum(axis=1)
        total += float((per / np.asarray(sq_norms[group], np.float64)).sum())
    return total / n_sites


def site_errors(W, V, U, sq_norms):
    d = weight_deltas(W, V, U)
    return (d ** 2).reshape(d.shape[0], -1).sum(axis=1) / np.asarray(sq_norms, np.float64)


def grads(W, V, U, sq_norms, scale):
    """d(scale * sum_s ||Delta_s||^2 / n_s)/dV and /dU: with Delta = W - (VU)^T,
    dV = -2 scale/n_s Delta^T U^T and dU = -2 scale/n_s V^T Delta^T per matrix."""
    d = weight_deltas(W, V, U)
    V, U = np.asarray(V, np.float64), np.asarray(U, np.float64)
    n = np.asarray(sq_norms, np.float64).reshape((-1,) + (1,) * (V.ndim - 1))
    dT = np.swapaxes(d, -1, -2)
    dV = -2.0 * scale / n * (dT @ np.swapaxes(U, -1, -2))
    dU = -2.0 * scale / n * (np.swapaxes(V, -1, -2) @ dT)
    return dV, dU
