"""Pins of the adversarial-source oracle (oracle/pgd_oracle.py) on the CPU."""

import numpy as np
import pytest

from oracle import pgd_oracle as po
from oracle import threefry


@pytest.mark.parametrize("rps", [1, 4, 12])
def test_source_mask_broadcast_and_vjp_by_finite_differences(rps):
    rng = np.random.default_rng(rps)
    rows, C = 12, 5
    ci = rng.uniform(size=(rows, C))
    s = rng.uniform(size=(rows // rps, C))
    m = po.source_mask(ci, s, rps)
    for r in range(rows):
        for c in range(C):
            assert m[r, c] == pytest.approx(ci[r, c] + (1 - ci[r, c]) * s[r // rps, c])
    g = rng.normal(size=(rows, C))
    d_src, d_ci = po.source_mask_vjp(g, ci, s, rps)
    f = lambda cc, ss: float((po.source_mask(cc, ss, rps) * g).sum())
    eps = 1e-6
    for idx in [(0, 0), (rows // rps - 1, C - 1)]:
        sp, sm = s.copy(), s.copy()
        sp[idx] += eps
        sm[idx] -= eps
        assert (f(ci, sp) - f(ci, sm)) / (2 * eps) == pytest.approx(d_src[idx], rel=1e-6)
    for idx in [(0, 1), (rows - 1, 2)]:
        cp, cm = ci.copy(), ci.copy()
        cp[idx] += eps
        cm[idx] -= eps
        assert (f(cp, s) - f(cm, s)) / (2 * eps) == pytest.approx(d_ci[idx], rel=1e-6)


def test_first_adam_step_moves_by_lr_times_sign():
    # bias-corrected first step: m_hat = g, v_hat = g^2, so the step is lr * g / (|g| + eps)
    g = np.array([0.3, -2.0, 1e-3, 0.0])
    vals = np.full(4, 0.5)
    new, m, v = po.adam(vals, g, np.zeros(4), np.zeros(4), 1.0, lr=0.1)
    np.testing.assert_allclose(new, 0.5 + 0.1 * g / (np.abs(g) + 1e-8), rtol=1e-12)
    np.testing.assert_allclose(m, 0.1 * g)
    np.testing.assert_allclose(v, 0.001 * g * g)


def test_bf16_adam_takes_the_coefficients_at_the_moment_dtype():
    # bf16 moments meet the Python-float betas as weak scalars: bf16(0.9) = 0.8984375,
    # bf16(0.1) = 0.10009765625, bf16(0.999) = 1.0, bf16(0.001) = 131/128 * 2^-10 = 0.00099945068359375.
    # Hand-rounded values for g = 1 over two steps from zero moments:
    #   m1 = 0.10009765625; v1 = 0.00099945068359375
    #   m2 = bf16(bf16(0.8984375 * m1) + m1) = bf16(0.08984375 + 0.10009765625)
    #      = bf16(0.18994140625) = 0.189453125 (a tie, to even)
    #   v2 = bf16(1.0 * v1 + v1) = 2 v1 exactly: v never decays
    g = np.array([1.0])
    s1, m1, v1 = po.adam_bf16(np.array([0.25]), g, np.zeros(1), np.zeros(1), 1.0, lr=0.01)
    assert m1[0] == 0.10009765625 and v1[0] == 0.00099945068359375
    s2, m2, v2 = po.adam_bf16(s1, g, m1, v1, 2.0, lr=0.01)
    assert m2[0] == 0.189453125 and v2[0] == 2 * v1[0]
    # the exact (fp32-moment) form differs exactly where the rounding bites
    _, me, ve = po.adam(np.array([0.25]), g, np.array([0.1]), np.array([0.001]), 2.0, lr=0.01)
    assert me[0] == pytest.approx(0.19) and ve[0] == pytest.approx(0.001999)


def test_sgd_momentum_sign_and_projection():
    vals = np.array([0.0, 0.5, 0.95, 1.0])
    g = np.array([-1.0, 2.0, 1.0, 3.0])
    np.testing.assert_allclose(po.sgd(vals, g, 0.1), [0.0, 0.7, 1.0, 1.0])
    new, v = po.momentum_sgd(vals, g, np.array([1.0, -1.0, 0.0, 0.0]), 0.1, 0.5)
    np.testing.assert_allclose(v, [-0.5, 1.5, 1.0, 3.0])
    np.testing.assert_allclose(new, [0.0, 0.65, 1.0, 1.0])
    np.testing.assert_allclose(po.sign_ascent(vals, np.array([-1.0, 0.0, 2.0, -3.0]), 0.1), [0.0, 0.5, 1.0, 0.9])


def test_uint16_view_and_stochastic_rounding_is_unbiased():
    assert po.source_view(np.array([0, 65535, 32768], np.uint16), "uint16")[1] == 1.0
    # exact grid points never move; a value a quarter step above a grid point rounds up
    # about a quarter of the time over many keys
    grid = np.array([0.0, 1.0, 100 / 65535], np.float32)
    q = po.quantize_stochastic(grid, (0, 7))
    np.testing.assert_array_equal(q, [0, 65535, 100])
    x = np.full(4096, (1000 + 0.25) / 65535, np.float32)
    ups = [po.quantize_stochastic(x, threefry.fold_in((1, 2), k)).astype(np.int64) - 1000 for k in range(4)]
    frac = float(np.mean(ups))
    assert 0.22 < frac < 0.28
    assert set(np.unique(np.concatenate(ups))) <= {0, 1}
