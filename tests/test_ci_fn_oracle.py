"""Pins of the CI-function oracle (oracle/ci_fn_oracle.py) on the CPU: the reference's
known-answer case for the symmetric clamp, torch's float64 Linear/GELU autograd as an
independent library routine for the MLP, finite differences, and closed forms."""

import math

import numpy as np
import pytest
import torch

from oracle import ci_fn_oracle as co


def test_symmetric_clamp_known_answer():
    # pd/tests/core/test_ci_component_conditioning.py:604-614
    x = np.array([-0.5, 0.25, 1.5, -0.5, 0.25, 1.5])
    g = np.array([-1.0, -1.0, -1.0, 1.0, 1.0, 1.0])
    np.testing.assert_array_equal(co.symmetric_leaky(x), [0, 0.25, 1, 0, 0.25, 1])
    np.testing.assert_allclose(co.symmetric_leaky_vjp(x, g), [-0.01, -1, 0, 0, 1, 0.01], rtol=1e-12)


def test_symmetric_clamp_boundaries_take_the_leaky_branches():
    # x == 0 and x == 1 are outside the pass-through band of the symmetric rule
    # (pd/core/ci_fn/squashing.py:32-35: `x <= 0`, then `x >= 1`)
    x = np.array([0.0, 0.0, 1.0, 1.0])
    g = np.array([-2.0, 2.0, -2.0, 2.0])
    np.testing.assert_allclose(co.symmetric_leaky_vjp(x, g), [-0.02, 0.0, 0.0, 0.02])


def _torch_mlp(x, weights, biases):
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    ws = [torch.tensor(w, dtype=torch.float64, requires_grad=True) for w in weights]
    bs = [torch.tensor(b, dtype=torch.float64, requires_grad=True) for b in biases]
    a = xt
    for i, (w, b) in enumerate(zip(ws, bs)):
        a = torch.nn.functional.linear(a, w.T, b)
        if i + 1 < len(ws):
            a = torch.nn.functional.gelu(a, approximate="none")
    return xt, ws, bs, a


@pytest.mark.parametrize("dims", [(16, 32, 8), (24, 40, 32, 16), (8, 8, 8, 8, 8)])
def test_site_mlp_matches_torch_float64_autograd(dims):
    rng = np.random.default_rng(sum(dims))
    weights, biases = co.init_mlp_stack(dims, rng)
    biases = [rng.normal(size=b.shape) * 0.3 for b in biases]
    x = rng.normal(size=(37, dims[0]))
    d_out = rng.normal(size=(37, dims[-1]))
    pre, zs, acts = co.site_mlp_fwd(x, weights, biases)
    xt, ws, bs, yt = _torch_mlp(x, weights, biases)
    np.testing.assert_allclose(pre, yt.detach().numpy(), rtol=1e-12, atol=1e-12)
    assert len(zs) == len(acts) == len(dims) - 2
    (yt * torch.tensor(d_out)).sum().backward()
    dW, db, dx = co.site_mlp_bwd(x, weights, biases, d_out)
    np.testing.assert_allclose(dx, xt.grad.numpy(), rtol=1e-10, atol=1e-12)
    for i in range(len(weights)):
        np.testing.assert_allclose(dW[i], ws[i].grad.numpy(), rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(db[i], bs[i].grad.numpy(), rtol=1e-10, atol=1e-12)


def test_site_mlp_one_unit_closed_form():
    # preact = w2 GELU(w1 x + b1) + b2, GELU(z) = z Phi(z)
    w1, b1, w2, b2 = 1.7, -0.3, -0.8, 0.25
    x = np.array([[-1.5], [0.0], [0.4], [2.0]])
    pre, _, _ = co.site_mlp_fwd(x, [np.array([[w1]]), np.array([[w2]])], [np.array([b1]), np.array([b2])])
    z = w1 * x[:, 0] + b1
    phi = 0.5 * (1 + np.array([math.erf(v / math.sqrt(2)) for v in z]))
    np.testing.assert_allclose(pre[:, 0], w2 * z * phi + b2, rtol=1e-14)


def test_site_mlp_backward_finite_differences():
    rng = np.random.default_rng(5)
    dims = (8, 16, 8)
    weights, biases = co.init_mlp_stack(dims, rng)
    biases = [rng.normal(size=b.shape) * 0.2 for b in biases]
    x = rng.normal(size=(5, 8))
    d_out = rng.normal(size=(5, 8))
    f = lambda ws, bs, xx: float((co.site_mlp_fwd(xx, ws, bs)[0] * d_out).sum())
    dW, db, dx = co.site_mlp_bwd(x, weights, biases, d_out)
    eps = 1e-6
    for layer in range(2):
        for idx in [(0, 0), (3, 5), (7, 7)]:
            wp = [w.copy() for w in weights]
            wm = [w.copy() for w in weights]
            wp[layer][idx] += eps
            wm[layer][idx] -= eps
            fd = (f(wp, biases, x) - f(wm, biases, x)) / (2 * eps)
            assert abs(fd - dW[layer][idx]) < 1e-6 * max(1, abs(fd))
    i = (2, 3)
    xp, xm = x.copy(), x.copy()
    xp[i] += eps
    xm[i] -= eps
    assert abs((f(weights, biases, xp) - f(weights, biases, xm)) / (2 * eps) - dx[i]) < 1e-6


def test_site_mlp_bf16_mode_tracks_float64():
    rng = np.random.default_rng(9)
    dims = (32, 64, 16)
    weights, biases = co.init_mlp_stack(dims, rng)
    x = rng.normal(size=(50, 32))
    exact = co.site_mlp_fwd(x, weights, biases)[0]
    rounded = co.site_mlp_fwd(x, weights, biases, bf16_storage=True)[0]
    assert np.abs(rounded - exact).max() < 3e-2 * np.abs(exact).max()
    np.testing.assert_array_equal(rounded, co.round_bf16(rounded))


def _readout_case(rng, N=40, C=12):
    h = rng.normal(size=(N, C)) * 1.5
    params = np.stack([rng.uniform(0.5, 1.5, C), rng.normal(size=C) * 0.3, rng.normal(size=C),
                       rng.uniform(0.5, 1.5, C), rng.normal(size=C) * 0.3, rng.normal(size=C), rng.normal(size=C)])
    return h, params


def test_readout_finite_differences_in_every_parameter_and_h():
    rng = np.random.default_rng(3)
    h, params = _readout_case(rng)
    d_out = rng.normal(size=h.shape)
    f = lambda hh, pp: float((co.readout_fwd(hh, pp) * d_out).sum())
    d_h, d_params = co.readout_bwd(h, params, d_out)
    eps = 1e-7

    def away_from_kinks(hh, pp, c):
        xp = pp[0, c] * hh[:, c] + pp[1, c]
        xn = -pp[3, c] * hh[:, c] + pp[4, c]
        return min(np.abs(xp).min(), np.abs(xp - 1).min(), np.abs(xn).min(), np.abs(xn - 1).min()) > 1e-4

    for k in range(7):
        for c in range(params.shape[1]):
            if k != 6 and k != 2 and k != 5 and not away_from_kinks(h, params, c):
                continue
            pp, pm = params.copy(), params.copy()
            pp[k, c] += eps
            pm[k, c] -= eps
            fd = (f(h, pp) - f(h, pm)) / (2 * eps)
            # inside the band the clamp's pullback is the derivative; outside it is 0 or
            # the leak, so compare only components whose every x is inside or outside with
            # a zero-leak cotangent sign; the leak itself is checked below
            xp = params[0, c] * h[:, c] + params[1, c]
            xn = -params[3, c] * h[:, c] + params[4, c]
            inside = ((xp > 0) & (xp < 1)).all() and ((xn > 0) & (xn < 1)).all()
            if k in (2, 5, 6) or inside:
                assert abs(fd - d_params[k, c]) < 1e-5 * max(1, abs(fd)), (k, c, fd, d_params[k, c])
    # h: entries whose both arms are strictly inside the band
    for (n, c) in [(0, 0), (5, 3), (17, 8), (39, 11)]:
        xp = params[0, c] * h[n, c] + params[1, c]
        xn = -params[3, c] * h[n, c] + params[4, c]
        if 0 < xp < 1 and 0 < xn < 1:
            hp, hm = h.copy(), h.copy()
            hp[n, c] += eps
            hm[n, c] -= eps
            assert abs((f(hp, params) - f(hm, params)) / (2 * eps) - d_h[n, c]) < 1e-5


def test_readout_in_band_gradients_equal_the_derivative():
    # every arm input inside (0, 1): the readout is affine in h per arm, the VJP is exact
    rng = np.random.default_rng(4)
    N, C = 30, 5
    h = rng.uniform(-0.2, 0.2, size=(N, C))
    params = np.stack([np.full(C, 1.0), np.full(C, 0.5), rng.normal(size=C), np.full(C, 1.0), np.full(C, 0.5),
                       rng.normal(size=C), rng.normal(size=C)])
    g = rng.normal(size=(N, C))
    d_h, d_params = co.readout_bwd(h, params, g)
    sp, sn = params[2], params[5]
    np.testing.assert_allclose(d_h, g * sp - g * sn, rtol=1e-12)
    np.testing.assert_allclose(d_params[0], (g * sp * h).sum(0), rtol=1e-12)
    np.testing.assert_allclose(d_params[1], (g * sp).sum(0), rtol=1e-12)
    np.testing.assert_allclose(d_params[2], (g * (h + 0.5)).sum(0), rtol=1e-12)
    np.testing.assert_allclose(d_params[3], (g * sn * -h).sum(0), rtol=1e-12)
    np.testing.assert_allclose(d_params[6], g.sum(0), rtol=1e-12)


def test_readout_saturation_and_zero_scale():
    C = 4
    params = np.stack([np.ones(C), np.zeros(C), np.full(C, 2.0), np.ones(C), np.zeros(C), np.full(C, 3.0),
                       np.full(C, -0.5)])
    h = np.array([[10.0, -10.0, 0.5, 0.0]])
    base = np.array([[1.0, 1.0, 1.0, 1.0]])
    # positive arm clamps h, negative arm clamps -h
    np.testing.assert_allclose(co.readout_fwd(h, params, base)[0], [1 + 2 - 0.5, 1 + 3 - 0.5, 1 + 1 - 0.5, 0.5])
    params[2] = params[5] = 0
    np.testing.assert_allclose(co.readout_fwd(h, params, base)[0], [0.5] * 4)


def test_planted_sign_error_in_the_readout_vjp_is_caught():
    # the negative arm reads -h: dropping that sign must fail the finite-difference check
    rng = np.random.default_rng(11)
    h = rng.uniform(-0.2, 0.2, size=(10, 3))
    params = np.stack([np.ones(3), np.full(3, 0.5), np.ones(3), np.ones(3), np.full(3, 0.5), np.full(3, 2.0),
                       np.zeros(3)])
    g = rng.normal(size=h.shape)
    d_h, _ = co.readout_bwd(h, params, g)
    wrong = params[0] * co.symmetric_leaky_vjp(h + 0.5, g) + params[3] * co.symmetric_leaky_vjp(-h + 0.5, g * 2.0)
    eps = 1e-7
    hp, hm = h.copy(), h.copy()
    hp[0, 0] += eps
    hm[0, 0] -= eps
    fd = float(((co.readout_fwd(hp, params) - co.readout_fwd(hm, params)) * g).sum() / (2 * eps))
    assert abs(fd - d_h[0, 0]) < 1e-6
    assert abs(fd - wrong[0, 0]) > 1e-2
