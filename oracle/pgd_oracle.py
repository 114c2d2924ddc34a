"""NumPy restatement of adversarial sources (oracle only: test infrastructure, never the
product path; float64 arithmetic except where a storage dtype fixes a rounding). Paths are
relative to the reference repository root; `pd/` = `param_decomp/param_decomp/`.

Pins (tests/test_pgd_oracle.py): finite differences of the source mask in s and ci,
brute-force broadcasting for the source shapes, the optimizers' closed forms (first Adam
step moves by lr * sign(g) up to eps; SGD and momentum by hand), projection limits, and
the stochastic rounding's unbiasedness over many keys.
"""

from __future__ import annotations

import numpy as np

from oracle import threefry
from oracle.pd_oracle import round_bf16

U16 = 65535.0


def source_view(stored, dtype: str):
    """`pd/core/adversary.py:171-184`: uint16 dequantizes to `u / 65535` (fp32)."""
    if dtype == "uint16":
        return (np.asarray(stored, np.float32) / np.float32(U16)).astype(np.float64)
    return np.asarray(stored, np.float64)


def source_mask(ci, src_view, rows_per_source: int, *, bf16=False):
    """`pd/core/source_mask.py:56-63`: `ci + (1 - ci) * s` with each source row broadcast
    over `rows_per_source` consecutive rows (read in the CI's dtype)."""
    s = np.repeat(np.asarray(src_view, np.float64), rows_per_source, axis=0)
    if bf16:
        s = round_bf16(s)
    ci = np.asarray(ci, np.float64)
    m = ci + (1.0 - ci) * s
    return round_bf16(m) if bf16 else m


def source_mask_vjp(g, ci, src_view, rows_per_source: int):
    """(d_sources, d_ci): the broadcast's reduction of `g (1 - ci)` and `g (1 - s)`."""
    g, ci = np.asarray(g, np.float64), np.asarray(ci, np.float64)
    rows, C = ci.shape
    d_src = (g * (1.0 - ci)).reshape(rows // rows_per_source, rows_per_source, C).sum(axis=1)
    s = np.repeat(np.asarray(src_view, np.float64), rows_per_source, axis=0)
    return d_src, g * (1.0 - s)


def sgd(values, g, lr):
    """`pd/core/adversary.py:392-403`."""
    return np.clip(values + lr * g, 0.0, 1.0)


def momentum_sgd(values, g, velocity, lr, momentum):
    """`pd/core/adversary.py:406-428`: v = momentum v + g; s += lr v; clip."""
    v = momentum * velocity + g
    return np.clip(values + lr * v, 0.0, 1.0), v


def adam(values, g, m, v, step_count, lr, beta1=0.9, beta2=0.999, eps=1e-8):
    """`pd/core/adversary.py:463-496` (step_count is the count after this update), exact
    arithmetic: the fp32-moment form."""
    m = beta1 * m + (1 - beta1) * g
    v = beta2 * v + (1 - beta2) * g * g
    bc1, bc2 = 1 - beta1 ** step_count, 1 - beta2 ** step_count
    return np.clip(values + lr * (m / bc1) / (np.sqrt(v / bc2) + eps), 0.0, 1.0), m, v


def adam_bf16(values, g, m, v, step_count, lr, beta1=0.9, beta2=0.999, eps=1e-8):
    """The same ascent with bf16 sources and moments, rounding where the reference's
    dtypes round (`pd/core/adversary.py:463-496`): the gradient is cast to the moment
    dtype; the Python-float coefficients beta and (1 - beta) meet bf16 moments as weak
    scalars and so are rounded to bf16 (bf16(0.9) = 0.8984375, bf16(0.999) = 1.0); every
    bf16 product and sum rounds; the bias corrections are fp32 on fp32(beta); the update
    is formed in fp32 and cast to bf16 before the add and the clip."""
    rb = round_bf16
    f32 = lambda a: np.asarray(a, np.float32).astype(np.float64)  # noqa: E731
    g = rb(g)
    b1, omb1, b2, omb2 = rb(beta1), rb(1.0 - beta1), rb(beta2), rb(1.0 - beta2)
    m = rb(rb(b1 * m) + rb(omb1 * g))
    v = rb(rb(b2 * v) + rb(rb(omb2 * g) * g))
    bc1 = f32(1.0 - f32(f32(beta1) ** step_count))
    bc2 = f32(1.0 - f32(f32(beta2) ** step_count))
    upd = f32(f32(lr) * f32(f32(m) / bc1) / f32(f32(np.sqrt(f32(v / bc2))) + f32(eps)))
    return np.clip(rb(values + rb(upd)), 0.0, 1.0), m, v


def sign_ascent(values, g, step_size):
    """`pd/core/train.py:788-800`."""
    return np.clip(values + step_size * np.sign(g), 0.0, 1.0)


def quantize_stochastic(values, key, *, partitionable=True):
    """`pd/core/adversary.py:186-194`: floor(v 65535) plus a carry when a uniform of `key`
    (one per element, fp32) falls below the fractional part."""
    scaled = (np.clip(np.asarray(values, np.float32), 0.0, 1.0) * np.float32(U16)).astype(np.float32)
    low = np.floor(scaled)
    u = threefry.uniform(key, scaled.shape, "float32", partitionable=partitionable)
    up = (u < (scaled - low)).astype(np.float32)
    return np.clip(low + up, 0.0, U16).astype(np.uint16)
