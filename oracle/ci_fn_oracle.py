"""NumPy restatement of the engine's CI functions (oracle only: test infrastructure,
never the product path; float64 arithmetic).

Paths are relative to the reference repository root; `pd/` = `param_decomp/param_decomp/`.

Pins (tests/test_ci_fn_oracle.py):
- `symmetric_leaky_vjp`: the reference's known-answer case
  (pd/tests/core/test_ci_component_conditioning.py:604-614), and finite differences of
  `clip` away from the kinks.
- `site_mlp_fwd` / `site_mlp_bwd` (float64 mode): torch's float64 Linear + exact GELU and
  its autograd on the same inputs (an independent library routine), finite differences,
  and the closed form of a one-hidden-unit stack.
- `readout_fwd` / `readout_bwd`: finite differences of the forward in every parameter
  and in h, the closed form at scale 0, and the clamp limits.
The bf16-storage mode adds only `round_bf16` at the points the GPU kernels round; it is
pinned through the float64 mode (the rounding is the same RNE routine the other oracle
functions use).
"""

from __future__ import annotations

import math

import numpy as np
from scipy.special import erf

from oracle.pd_oracle import round_bf16

ALPHA = 0.01
INV_SQRT_2PI = 1.0 / math.sqrt(2.0 * math.pi)


def _rnd(a, on: bool):
    return round_bf16(a) if on else np.asarray(a, np.float64)


def gelu(z):
    """Exact-erf GELU (`jax.nn.gelu(approximate=False)`, pd/core/ci_fn/implementations/mlp.py:77)."""
    return 0.5 * z * (1.0 + erf(z / math.sqrt(2.0)))


def gelu_grad(z):
    return 0.5 * (1.0 + erf(z / math.sqrt(2.0))) + z * INV_SQRT_2PI * np.exp(-0.5 * z * z)


# ---------------------------------------------------------------- SiteMLP
def init_mlp_stack(dims, rng: np.random.Generator):
    """`pd/core/ci_fn/implementations/mlp.py:81-92`: normal weights [d_in, d_out] scaled by
    gain / sqrt(d_in), gain sqrt 2 on hidden layers and 1 on the head; zero biases."""
    weights, biases = [], []
    for i, (din, dout) in enumerate(zip(dims[:-1], dims[1:])):
        gain = math.sqrt(2.0) if i < len(dims) - 2 else 1.0
        weights.append(rng.normal(size=(din, dout)) * (gain / math.sqrt(din)))
        biases.append(np.zeros(dout))
    return weights, biases


def site_mlp_fwd(x, weights, biases, *, bf16_storage=False):
    """`SiteMLP.__call__` (pd/core/ci_fn/implementations/mlp.py:72-78): z_i = a_i-1 @ W_i + b_i,
    GELU on every layer but the head. With bf16 storage every product, bias sum and GELU
    output is rounded to bf16 (the engine's bf16 compute cast,
    pd/core/ci_fn/implementations/layerwise_mlp.py:108-109,139). Returns (preact, zs, acts)
    with zs/acts the hidden layers' pre-activations and activations."""
    r = bf16_storage
    a = _rnd(x, r)
    zs, acts = [], []
    n = len(weights)
    for i, (w, b) in enumerate(zip(weights, biases)):
        z = _rnd(_rnd(a @ _rnd(w, r), r) + _rnd(b, r), r)
        if i + 1 < n:
            zs.append(z)
            a = _rnd(gelu(z), r)
            acts.append(a)
        else:
            return z, zs, acts
    raise AssertionError("unreachable")


def site_mlp_bwd(x, weights, biases, d_preact, *, bf16_storage=False):
    """Reverse pass of `site_mlp_fwd`: returns (d_weights, d_biases, d_x). With bf16 storage
    the data gradient d_a = d_z @ W^T is rounded, then d_z_prev = round(d_a * GELU'(z));
    weight and bias gradients are unrounded sums of rounded operands."""
    r = bf16_storage
    _, zs, acts = site_mlp_fwd(x, weights, biases, bf16_storage=r)
    n = len(weights)
    dz = _rnd(d_preact, r)
    dW, db = [None] * n, [None] * n
    d_x = None
    for i in range(n - 1, -1, -1):
        a_in = _rnd(x, r) if i == 0 else acts[i - 1]
        dW[i] = a_in.T @ dz
        db[i] = dz.sum(axis=0)
        d_a = _rnd(dz @ _rnd(weights[i], r).T, r)
        if i > 0:
            dz = _rnd(d_a * gelu_grad(zs[i - 1]), r)
        else:
            d_x = d_a
    return dW, db, d_x


# ---------------------------------------------------------------- readout
def symmetric_leaky(x):
    """`pd/core/ci_fn/squashing.py:25-29`: forward `clip(x, 0, 1)`."""
    return np.clip(x, 0.0, 1.0)


def symmetric_leaky_vjp(x, g):
    """`pd/core/ci_fn/squashing.py:32-35`: at or below 0 leak `0.01 g` only for g < 0; at or
    above 1 leak `0.01 g` only for g > 0; pass g inside."""
    below = np.where(g < 0, ALPHA * g, 0.0)
    above = np.where(g > 0, ALPHA * g, 0.0)
    return np.where(x <= 0, below, np.where(x >= 1, above, g))


def readout_fwd(h, params, base=None, *, bf16_storage=False):
    """`ComponentActivationReadout.__call__` with its two `ClampedAffineArm`s
    (pd/core/ci_fn/implementations/transformer/component_conditioning.py:215-243):
    s+ sig(a+ h + b+) + s- sig(a- (-h) + b-) + bias, plus the backbone preactivation
    `base` (:333-338). params [7, C] = a+, b+, s+, a-, b-, s-, bias (rounded to bf16 with
    bf16 storage; the sum is rounded once)."""
    r = bf16_storage
    ap, bp, sp, an, bn, sn, bias = _rnd(params, r)
    hv = _rnd(h, r)
    v = sp * symmetric_leaky(ap * hv + bp) + sn * symmetric_leaky(an * -hv + bn) + bias
    if base is not None:
        v = v + _rnd(base, r)
    return _rnd(v, r)


def readout_bwd(h, params, d_out, *, bf16_storage=False):
    """Reverse pass of `readout_fwd`: returns (d_h, d_params [7, C])."""
    r = bf16_storage
    ap, bp, sp, an, bn, sn, bias = _rnd(params, r)
    hv, g = _rnd(h, r), _rnd(d_out, r)
    xp, xn = ap * hv + bp, an * -hv + bn
    dxp, dxn = symmetric_leaky_vjp(xp, g * sp), symmetric_leaky_vjp(xn, g * sn)
    d_h = ap * dxp - an * dxn
    lead = tuple(range(hv.ndim - 1))
    d_params = np.stack([
        (hv * dxp).sum(lead), dxp.sum(lead), (g * symmetric_leaky(xp)).sum(lead),
        (-hv * dxn).sum(lead), dxn.sum(lead), (g * symmetric_leaky(xn)).sum(lead), g.sum(lead),
    ])
    return _rnd(d_h, r), d_params
