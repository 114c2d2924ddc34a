"""The bf16 dense step's binned gate, as mathematics (numpy, float64).

The step replaces each component's token sums sum_t dg_t f(h_t) (f = the 48 gate-parameter
summands) by 8 Chebyshev moments per bin, M_m = sum_t dg_t T_m(tau_t), and the node weights
w_k = (2/8) (M_0 / 2 + sum_{m>=1} T_m(x_k) M_m) at the Chebyshev nodes x_k = cos((2k+1)
pi / 16). These tests pin that identity independently of the kernel: it must be exact for
every polynomial of degree <= 7 in the bin coordinate (discrete orthogonality), keep
sum_k w_k = sum_t dg_t, and stay within the documented interpolation bounds for GELU, GELU'
and h GELU' at the fallback limit dz = 3. The table half of the scheme (degree-7 power
form from the 8 node values) is pinned the same way: exact on degree-7 polynomials.
"""

import numpy as np
import pytest
from scipy.special import erf

NC = 8
NODES = np.cos((2 * np.arange(NC) + 1) * np.pi / 16)


def cheb_T(m, x):
    return np.polynomial.chebyshev.chebval(x, np.eye(NC)[m])


def moments(dg, tau):
    return np.array([(dg * cheb_T(m, tau)).sum() for m in range(NC)])


def node_weights(M):
    Tk = np.stack([cheb_T(m, NODES) for m in range(NC)])  # [m, k]
    return 0.25 * (0.5 * M[0] + M[1:] @ Tk[1:])


def table_coeffs(fvals):
    """Power-form coefficients of the degree-7 interpolant through f(x_k) (the table
    kernel's construction: Chebyshev coefficients, then T_m's monomial coefficients)."""
    cm = np.array([0.25 * (fvals * cheb_T(m, NODES)).sum() for m in range(NC)])
    cm[0] *= 0.5
    return np.polynomial.chebyshev.cheb2poly(cm)


def gelu(z):
    return z * 0.5 * (1 + erf(z / np.sqrt(2)))


def dgelu(z):
    return 0.5 * (1 + erf(z / np.sqrt(2))) + z * np.exp(-z * z / 2) / np.sqrt(2 * np.pi)


@pytest.mark.parametrize("seed", range(4))
def test_node_weights_are_exact_on_degree_7_polynomials(seed):
    rng = np.random.default_rng(seed)
    tau = rng.uniform(-1, 1, size=500)
    dg = rng.normal(size=500)
    w = node_weights(moments(dg, tau))
    for _ in range(5):
        p = rng.normal(size=NC)  # any degree-7 polynomial
        exact = (dg * np.polynomial.polynomial.polyval(tau, p)).sum()
        assert np.isclose((w * np.polynomial.polynomial.polyval(NODES, p)).sum(), exact, rtol=1e-10, atol=1e-10)
    # a degree-8 term is not reproduced: the identity is not vacuous
    t8 = (dg * tau**8).sum()
    assert abs((w * NODES**8).sum() - t8) > 1e-6
    assert np.isclose(w.sum(), dg.sum(), rtol=1e-12)


def test_table_power_form_is_exact_on_degree_7_polynomials():
    rng = np.random.default_rng(7)
    p = rng.normal(size=NC)
    a = table_coeffs(np.polynomial.polynomial.polyval(NODES, p))
    np.testing.assert_allclose(a, p, rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("dz,bounds", [(2.0, (7.7e-6, 2.0e-5)), (3.0, (1.6e-4, 4.0e-4))])
def test_moment_interpolation_error_bounds_for_gelu(dz, bounds):
    """Worst case over the bin's position in z of |f - p| for the degree-7 interpolant on a
    bin of z-width dz: the bounds the kernel's comments and the header state."""
    t = np.linspace(-1, 1, 801)
    worst = [0.0, 0.0]
    for z0 in np.linspace(-8, 8, 161):
        for i, f in enumerate((gelu, dgelu)):
            a = table_coeffs(f(z0 + dz / 2 * NODES))
            err = np.abs(np.polynomial.polynomial.polyval(t, a) - f(z0 + dz / 2 * t)).max()
            worst[i] = max(worst[i], err)
    assert worst[0] <= bounds[0] * 1.05 and worst[1] <= bounds[1] * 1.05, worst
    assert worst[0] > bounds[0] / 3  # the stated bound is tight, not a loose guess


def test_binned_gate_sums_match_exact_sums_at_benchmark_scale():
    """One component as the step sees it (T = 4096, h ~ N(0, 1), w_in ~ N(0, 2), 16 moment
    bins over [min h, max h]): the 48 summands' token sums from the node weights against the
    exact sums, relative to sum_t |dg_t f(h_t)|."""
    rng = np.random.default_rng(3)
    T = 4096
    h = rng.normal(size=T)
    dg = rng.normal(size=T)
    wi, bi, wo = rng.normal(size=16) * 2**0.5, rng.normal(size=16) * 0.3, rng.normal(size=16) * 0.35
    lo, hi = h.min(), h.max()
    bw = (hi - lo) / 16
    assert np.abs(wi).max() * bw <= 3.0  # not a flagged component
    s = (h - lo) / bw
    mb = np.clip(np.floor(s).astype(int), 0, 15)
    tau = 2 * (s - mb) - 1
    hv, wv = [], []
    for b in range(16):
        sel = mb == b
        wv.append(node_weights(moments(dg[sel], tau[sel])))
        hv.append(lo + bw * (b + 0.5 + 0.5 * NODES))
    hv, wv = np.concatenate(hv), np.concatenate(wv)

    def sums(hh, ww):
        z = np.outer(hh, wi) + bi
        return np.stack([(ww[:, None] * wo * dgelu(z) * hh[:, None]).sum(0), (ww[:, None] * wo * dgelu(z)).sum(0),
                         (ww[:, None] * gelu(z)).sum(0)])

    def scale(hh, ww):
        z = np.outer(hh, wi) + bi
        return np.stack([np.abs(ww[:, None] * wo * dgelu(z) * hh[:, None]).sum(0),
                         np.abs(ww[:, None] * wo * dgelu(z)).sum(0), np.abs(ww[:, None] * gelu(z)).sum(0)])

    err = np.abs(sums(hv, wv) - sums(h, dg)) / scale(h, dg)
    assert err.max() < 1e-5, err.max()
