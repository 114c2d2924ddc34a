"""Pins the CPU oracle against known answers, closed forms, brute force and finite
differences — never against a retyped copy of its own formula.

Known answers come from: Random123's published threefry2x32-20 vectors; JAX's
documentation values of `split(PRNGKey(0))` (original layout, and the partitionable
layout that JAX >= 0.5 defaults to); and the reference's own tests
(`param_decomp/param_decomp/tests/core/test_lower_leaky_hard_grad.py:18-30`,
`tests/core/test_imp_min.py`, `tests/core/test_frequency_minimality.py:52-75`,
`tests/core/test_hidden_acts_reconstruction.py:87-125`, `tests/routed/test_experts.py`).
"""

import math

import numpy as np
import pytest

from oracle import pd_oracle as po
from oracle import threefry as tf

# ------------------------------------------------------------------ Threefry


@pytest.mark.parametrize(
    "key, ctr, expected",
    [
        ((0, 0), (0, 0), (0x6B200159, 0x99BA4EFE)),
        ((0xFFFFFFFF, 0xFFFFFFFF), (0xFFFFFFFF, 0xFFFFFFFF), (0x1CB996FC, 0xBB002BE7)),
        ((0x13198A2E, 0x03707344), (0x243F6A88, 0x85A308D3), (0xC4923A9C, 0x483DF7A0)),
    ],
)
def test_threefry_random123_kat(key, ctr, expected):
    y0, y1 = tf.threefry2x32(key, np.uint32(ctr[0]), np.uint32(ctr[1]))
    assert (int(y0), int(y1)) == expected


def test_split_matches_jax_documentation_original_layout():
    assert tf.split(tf.prng_key(0), 2, partitionable=False) == [(4146024105, 967050713), (2718843009, 1272950319)]


def test_split_partitionable_layout():
    """First subkey = the Random123 vector at key (0,0), counter (0,0) (pinned); the
    second row is a regression vector of this restatement (split(k)[1] == fold_in(k, 1),
    checked generally in the next test)."""
    got = tf.split(tf.prng_key(0), 2, partitionable=True)
    assert got[0] == (0x6B200159, 0x99BA4EFE)
    assert got == [(1797259609, 2579123966), (928981903, 3453687069)]


def test_fp32_uniform_matches_reference_stored_jax_draws():
    """The reference's stored PPGD sources are fp32 `jax.random.uniform` draws, one per
    site, under `split(PRNGKey(3), 9)` in site order
    (`tests/targets/stacked_parity/gen_stacked_fixtures.py:102`, `core/adversary.py:283-303`):
    they pin the partitionable split, the per-element counter layout and the fp32
    bits->[0,1) map bit for bit."""
    import os

    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "stacked_sources.npz"))
    names = list(z.keys())
    assert len(names) == 9 and all(n.startswith("src::") for n in names)
    keys = tf.split(tf.prng_key(3), len(names), partitionable=True)
    for key, name in zip(keys, names):
        want = z[name]
        got = tf.uniform(key, want.shape, "float32", partitionable=True).astype(np.float32)
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32), err_msg=name)


def test_partitionable_split_is_foldlike():
    key = tf.fold_in(tf.prng_key(7), 3)
    subs = tf.split(key, 5, partitionable=True)
    assert subs == [tf.fold_in(key, i) for i in range(5)]


def test_original_layout_bits_are_the_split_counter_stream():
    """The original layout's 32-bit draw of n words is the block applied to counter
    halves; split(key, n) reads the same stream reshaped [n, 2]."""
    key = (12345, 678)
    words = tf.random_bits(key, 32, (8,), partitionable=False)
    flat = np.array(tf.split(key, 4, partitionable=False), np.uint32).reshape(-1)
    np.testing.assert_array_equal(words, flat)


def test_original_layout_subword_bits_are_little_endian_bytes():
    key = (3, 9)
    words = tf.random_bits(key, 32, (4,), partitionable=False)
    bytes_ = tf.random_bits(key, 8, (16,), partitionable=False)
    np.testing.assert_array_equal(bytes_, words.view(np.uint8))


def test_uniform_ranges_and_grids():
    key = tf.fold_in(tf.prng_key(1), 0)
    u32 = tf.uniform(key, (4096,), "float32")
    u16 = tf.uniform(key, (4096,), "bfloat16")
    assert u32.min() >= 0 and u32.max() < 1 and u16.min() >= 0 and u16.max() < 1
    assert np.all(u32 * 2**23 == np.round(u32 * 2**23))
    assert np.all(u16 * 2**7 == np.round(u16 * 2**7))
    # bf16 uses the low byte, fp32 the top 23 bits of the same x0^x1 word
    bits = tf.random_bits(key, 32, (4096,))
    np.testing.assert_array_equal(u16, ((bits & 0xFF) >> 1) / 128.0)
    # a fair draw: the mean of 4096 uniforms is near 1/2
    assert abs(u32.mean() - 0.5) < 0.03


@pytest.mark.parametrize("bf16", [False, True])
def test_c_uniform_matches_numpy(bf16):
    from oracle import cpu

    key = tf.fold_in(tf.split(tf.prng_key(5))[1], 2)
    n = 10007
    got = cpu.uniform(key, n, bf16)
    want = tf.uniform(key, (n,), "bfloat16" if bf16 else "float32")
    np.testing.assert_array_equal(got, want.astype(np.float32))


# ------------------------------------------------------------------ squashing

ALPHA = 0.01
LHS_CASES = [
    (-2.0, -3.0, ALPHA * -3.0),
    (-2.0, 3.0, 0.0),
    (0.5, -3.0, -3.0),
    (0.5, 3.0, 3.0),
    (4.0, -3.0, 0.0),
    (4.0, 3.0, 0.0),
    (0.0, -3.0, ALPHA * -3.0),
    (0.0, 3.0, 0.0),
    (1.0, -3.0, -3.0),
    (1.0, 3.0, 3.0),
]


@pytest.mark.parametrize("x, g, expected", LHS_CASES)
def test_lower_leaky_cotangent_reference_cases(x, g, expected):
    assert po.lower_leaky_vjp(np.float64(x), np.float64(g)) == pytest.approx(expected, abs=0)


def test_upper_leaky_forward_and_grad_finite_difference():
    xs = np.array([-1.5, -0.2, 0.3, 0.7, 1.2, 3.0])
    want = np.array([0.0, 0.0, 0.3, 0.7, 1.002, 1.02])
    np.testing.assert_allclose(po.upper_leaky(xs), want, rtol=1e-12)
    eps = 1e-6
    fd = (po.upper_leaky(xs + eps) - po.upper_leaky(xs - eps)) / (2 * eps)
    np.testing.assert_allclose(po.upper_leaky_vjp(xs, np.ones_like(xs)), fd, atol=1e-6)
    # clip's ties: JAX's max/min JVP splits the cotangent evenly at x == 0 and x == 1
    np.testing.assert_array_equal(po.upper_leaky_vjp(np.array([0.0, 1.0]), np.array([2.0, 2.0])), [1.0, 1.0])


# ------------------------------------------------------------------ imp-min


def test_smooth_l0_shape_invariants():
    for gamma in (1.0, 0.1):
        assert po.smooth_l0_psi(0.0, gamma) == 0.0
        assert abs(po.smooth_l0_psi(gamma, gamma) - 0.5) < 1e-12
        assert po.smooth_l0_psi(10 * gamma, gamma) > 0.99
        cs = np.linspace(0, 5 * gamma, 4096)
        gr = np.abs(po.smooth_l0_psi_grad(cs, gamma))
        assert gr.max() <= 0.65 / gamma + 1e-3
        assert abs(cs[np.argmax(gr)] - gamma / math.sqrt(3)) < 0.02 * gamma
        assert po.smooth_l0_psi_grad(0.0, gamma) == 0.0


def test_smooth_l0_terms_reference_closed_forms():
    ci = [np.array([[1.0, 2.0], [3.0, 4.0]])]
    act, freq = po.importance_minimality_terms(ci, 1.0, 8)
    f0 = (1 / 2 + 9 / 10) / 2
    f1 = (4 / 5 + 16 / 17) / 2
    assert math.isclose(act, f0 + f1, rel_tol=1e-12)
    assert math.isclose(freq, f0 * math.log2(1 + 8 * f0) + f1 * math.log2(1 + 8 * f1), rel_tol=1e-12)
    act, freq = po.importance_minimality_terms([np.ones((3, 2))], 1.0, 8, normalize_at_one=True)
    assert act == pytest.approx(2.0) and freq == pytest.approx(2.0 * math.log2(9.0))
    for gamma in (1.0, 0.1):
        act, _ = po.importance_minimality_terms([np.ones((1, 2))], gamma, None, normalize_at_one=True)
        assert act == pytest.approx(2.0)


def test_pnorm_impmin_brute_force_and_grad():
    rng = np.random.default_rng(0)
    up = rng.uniform(0.0, 1.3, size=(5, 4))
    for p in (1.0, 2.0, 0.7):
        total = 0.0
        for b in range(5):
            for c in range(4):
                total += abs(up[b, c]) ** p
        assert po.impmin_pnorm(up, p) == pytest.approx(total / 5, rel=1e-12)
        for beta in (0.0, 0.3):
            g = po.impmin_pnorm_grad(up, p, eps=0.0, beta=beta)
            eps = 1e-6
            for idx in [(0, 0), (3, 2), (4, 3)]:
                a = up.copy()
                a[idx] += eps
                b_ = up.copy()
                b_[idx] -= eps
                fd = (po.impmin_pnorm(a, p, beta=beta) - po.impmin_pnorm(b_, p, beta=beta)) / (2 * eps)
                assert g[idx] == pytest.approx(fd, rel=1e-5, abs=1e-9)


# ------------------------------------------------------------------ recon losses


def test_relative_squared_error_reference_values():
    assert po.relative_squared_error(np.array([[[3.0, 0.0]]]), np.array([[[3.0, 4.0]]])) == pytest.approx(16 / 25)
    assert po.relative_squared_error(np.ones((2, 4, 8)) * 1.25, np.ones((2, 4, 8))) == 0.0625
    clean = np.array([[[1.0], [3.0]], [[2.0], [4.0]]])
    masked = np.array([[[2.0], [3.0]], [[2.0], [0.0]]])
    assert po.relative_squared_error(masked, clean) == pytest.approx((1.0 + 0 + 0 + 1.0) / 4)


def test_mse_brute_force():
    rng = np.random.default_rng(1)
    a, b = rng.normal(size=(4, 5)), rng.normal(size=(4, 5))
    assert po.mse(a, b) == pytest.approx(sum((a[i, j] - b[i, j]) ** 2 for i in range(4) for j in range(5)) / 20)


def test_kl_closed_form_and_grad():
    # two categories: KL(p||q) = p log(p/q) + (1-p) log((1-p)/(1-q))
    clean = np.array([[0.0, math.log(3.0)]])  # p = (1/4, 3/4)
    masked = np.array([[0.0, 0.0]])  # q = (1/2, 1/2)
    want = 0.25 * math.log(0.5) + 0.75 * math.log(1.5)
    assert po.categorical_kl(masked, clean) == pytest.approx(want, rel=1e-12)
    assert po.categorical_kl(clean, clean) == pytest.approx(0.0, abs=1e-15)
    rng = np.random.default_rng(2)
    m, c = rng.normal(size=(3, 7)), rng.normal(size=(3, 7))
    g = po.categorical_kl_grad(m, c)
    eps = 1e-6
    for idx in [(0, 0), (1, 4), (2, 6)]:
        a, b = m.copy(), m.copy()
        a[idx] += eps
        b[idx] -= eps
        assert g[idx] == pytest.approx((po.categorical_kl(a, c) - po.categorical_kl(b, c)) / (2 * eps), rel=1e-6)


# ------------------------------------------------------------------ gate MLP


def _gate(rng, C, H=16):
    return po.GateParams(rng.normal(size=(C, H)) * 0.7, rng.normal(size=(C, H)) * 0.3,
                         rng.normal(size=(C, H)) * 0.4, rng.normal(size=C) * 0.2)


def test_gelu_matches_erf_definition_brute_force():
    zs = np.linspace(-6, 6, 101)
    want = np.array([0.5 * z * (1 + math.erf(z / math.sqrt(2))) for z in zs])
    np.testing.assert_allclose(po.gelu(zs), want, rtol=1e-13, atol=1e-15)
    eps = 1e-6
    np.testing.assert_allclose(po.gelu_grad(zs), (po.gelu(zs + eps) - po.gelu(zs - eps)) / (2 * eps), atol=1e-8)


def test_gate_forward_brute_force_and_backward_finite_difference():
    rng = np.random.default_rng(3)
    T, C, H = 3, 4, 16
    p = _gate(rng, C, H)
    h = rng.normal(size=(T, C))
    g = po.gate_forward(h, p)
    for t in range(T):
        for c in range(C):
            s = p.b_out[c]
            for j in range(H):
                z = p.w_in[c, j] * h[t, c] + p.b_in[c, j]
                s += p.w_out[c, j] * 0.5 * z * (1 + math.erf(z / math.sqrt(2)))
            assert g[t, c] == pytest.approx(s, rel=1e-12)
    dg = rng.normal(size=(T, C))
    dh, dwi, dbi, dwo, dbo = po.gate_backward(h, p, dg)
    f = lambda hh, pp: float(np.sum(po.gate_forward(hh, pp) * dg))
    eps = 1e-6
    for t, c in [(0, 0), (2, 3)]:
        a, b = h.copy(), h.copy()
        a[t, c] += eps
        b[t, c] -= eps
        assert dh[t, c] == pytest.approx((f(a, p) - f(b, p)) / (2 * eps), rel=1e-6)
    for name, grad in (("w_in", dwi), ("b_in", dbi), ("w_out", dwo)):
        for idx in [(0, 0), (3, 15), (1, 7)]:
            pa = po.GateParams(*(np.copy(v) for v in (p.w_in, p.b_in, p.w_out, p.b_out)))
            pb = po.GateParams(*(np.copy(v) for v in (p.w_in, p.b_in, p.w_out, p.b_out)))
            getattr(pa, name)[idx] += eps
            getattr(pb, name)[idx] -= eps
            assert grad[idx] == pytest.approx((f(h, pa) - f(h, pb)) / (2 * eps), rel=1e-6, abs=1e-10)
    pa = po.GateParams(p.w_in, p.b_in, p.w_out, p.b_out + np.eye(C)[1] * eps)
    pb = po.GateParams(p.w_in, p.b_in, p.w_out, p.b_out - np.eye(C)[1] * eps)
    assert dbo[1] == pytest.approx((f(h, pa) - f(h, pb)) / (2 * eps), rel=1e-6)


# ------------------------------------------------------------------ decomposed linear


def test_site_forward_equals_per_token_masked_weight():
    """The paper's statement: W'_b = U^T diag(m_b) V^T per token (with the delta channel
    adding d_b * (W - (V U)^T)), and route falls back to the target weight."""
    rng = np.random.default_rng(4)
    T, din, dout, C = 5, 6, 7, 9
    x = rng.normal(size=(T, din))
    W = rng.normal(size=(dout, din))
    V = rng.normal(size=(din, C))
    U = rng.normal(size=(C, dout))
    m = rng.uniform(size=(T, C))
    d = rng.uniform(size=T)
    route = np.array([True, False, True, True, False])
    y0, xV = po.site_forward(x, W, V, U, m, None, None)
    y1, _ = po.site_forward(x, W, V, U, m, d, None)
    y2, _ = po.site_forward(x, W, V, U, m, d, route)
    for t in range(T):
        Wp = (V @ np.diag(m[t]) @ U).T
        np.testing.assert_allclose(y0[t], Wp @ x[t], rtol=1e-12)
        Wd = Wp + d[t] * (W - (V @ U).T)
        np.testing.assert_allclose(y1[t], Wd @ x[t], rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(y2[t], (Wd if route[t] else W) @ x[t], rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(xV, x @ V)


@pytest.mark.parametrize("with_delta,with_route", [(False, False), (True, False), (True, True)])
def test_site_backward_finite_difference(with_delta, with_route):
    rng = np.random.default_rng(5)
    T, din, dout, C = 4, 3, 5, 6
    x, W = rng.normal(size=(T, din)), rng.normal(size=(dout, din))
    V, U = rng.normal(size=(din, C)), rng.normal(size=(C, dout))
    m = rng.uniform(size=(T, C))
    d = rng.uniform(size=T) if with_delta else None
    r = np.array([True, False, True, True]) if with_route else None
    go = rng.normal(size=(T, dout))
    dx, dV, dU, dm = po.site_backward(x, W, V, U, m, d, r, go)
    f = lambda x_, V_, U_, m_: float(np.sum(po.site_forward(x_, W, V_, U_, m_, d, r)[0] * go))
    eps = 1e-6
    for arr, grad, pos in ((x, dx, 0), (V, dV, 1), (U, dU, 2), (m, dm, 3)):
        for idx in [(0, 0), (arr.shape[0] - 1, arr.shape[1] - 1)]:
            args = [x, V, U, m]
            a = [v.copy() for v in args]
            b = [v.copy() for v in args]
            a[pos][idx] += eps
            b[pos][idx] -= eps
            assert grad[idx] == pytest.approx((f(*a) - f(*b)) / (2 * eps), rel=1e-6, abs=1e-9)


@pytest.mark.parametrize("with_route", [False, True])
def test_site_delta_grad_finite_difference_and_exact_factorization(with_route):
    """The delta cotangent: central differences of <site_forward, g> in each delta_t;
    unrouted positions get 0; and with V@U = W^T the blend is delta-independent, so the
    cotangent vanishes (a dropped target term or a sign flip breaks one of them)."""
    rng = np.random.default_rng(8)
    T, din, dout, C = 5, 3, 4, 6
    x, W = rng.normal(size=(T, din)), rng.normal(size=(dout, din))
    V, U = rng.normal(size=(din, C)), rng.normal(size=(C, dout))
    m = rng.uniform(size=(T, C))
    d = rng.uniform(size=T)
    r = np.array([True, False, True, True, False]) if with_route else None
    go = rng.normal(size=(T, dout))
    dd = po.site_delta_grad(x, W, V, U, m, d, r, go)
    eps = 1e-6
    for t in range(T):
        dp, dm_ = d.copy(), d.copy()
        dp[t] += eps
        dm_[t] -= eps
        fd = (np.sum(po.site_forward(x, W, V, U, m, dp, r)[0] * go)
              - np.sum(po.site_forward(x, W, V, U, m, dm_, r)[0] * go)) / (2 * eps)
        assert dd[t] == pytest.approx(fd, rel=1e-6, abs=1e-9)
    if with_route:
        assert dd[1] == 0.0 and dd[4] == 0.0
    # exact factorization: W^T = V @ U (C >= d_in, so V has a right inverse)
    U2 = np.linalg.lstsq(V, W.T, rcond=None)[0]
    np.testing.assert_allclose(V @ U2, W.T, atol=1e-10)
    assert np.abs(po.site_delta_grad(x, W, V, U2, m, d, r, go)).max() < 1e-9
    assert np.abs(dd).max() > 1e-3


@pytest.mark.parametrize("contraction", ["fused_output", "fused_input"])
def test_blocked_site_delta_grad_finite_difference(contraction):
    rng = np.random.default_rng(9)
    T, E, d_in, d_out, c = 4, 3, 2, 3, 2
    site_in = d_in * (E if contraction == "fused_input" else 1)
    site_out = d_out * (E if contraction == "fused_output" else 1)
    x, W = rng.normal(size=(T, site_in)), rng.normal(size=(site_out, site_in))
    V, U = rng.normal(size=(E, d_in, c)), rng.normal(size=(E, c, d_out))
    m, d = rng.uniform(size=(T, E * c)), rng.uniform(size=T)
    r = np.array([True, True, False, True])
    go = rng.normal(size=(T, site_out))
    dd = po.blocked_site_delta_grad(x, W, V, U, m, d, r, contraction, go)
    eps = 1e-6
    for t in range(T):
        dp, dm_ = d.copy(), d.copy()
        dp[t] += eps
        dm_[t] -= eps
        fd = (np.sum(po.blocked_site_forward(x, W, V, U, m, dp, r, contraction)[0] * go)
              - np.sum(po.blocked_site_forward(x, W, V, U, m, dm_, r, contraction)[0] * go)) / (2 * eps)
        assert dd[t] == pytest.approx(fd, rel=1e-6, abs=1e-9)
    assert dd[2] == 0.0 and np.abs(dd).max() > 1e-3


def test_dense_step_gradients_finite_difference():
    """The whole single-site step: loss(V, U, gate) with the mask uniforms fixed by the
    key — central differences on V, U and every gate parameter family. The lower
    squashing's custom VJP equals the true derivative only on (0, 1) (its leak below
    zero is pinned by the known-answer cases above), so the gate output is kept there."""
    rng = np.random.default_rng(6)
    T, din, dout, C = 6, 5, 4, 7
    x, W = rng.normal(size=(T, din)), rng.normal(size=(dout, din))
    V, U = rng.normal(size=(din, C)) * 0.5, rng.normal(size=(C, dout)) * 0.5
    gp = _gate(rng, C)
    gp.w_out = gp.w_out * 0.1
    gp.b_out = np.full(C, 0.5)
    key = tf.prng_key(11)
    for use_delta in (False, True):
        kw = dict(p=2.0, imp_coeff=0.3, recon_coeff=1.7, mask_dtype="float32", use_delta=use_delta)
        r = po.dense_site_step(x, W, V, U, gp, key, **kw)
        assert np.all((r.g_raw > 0) & (r.g_raw < 1))
        loss = lambda V_, U_, g_: po.dense_site_step(x, W, V_, U_, g_, key, **kw).loss
        eps = 1e-6
        for idx in [(0, 0), (4, 6), (2, 3)]:
            a, b = V.copy(), V.copy()
            a[idx] += eps
            b[idx] -= eps
            assert r.dV[idx] == pytest.approx((loss(a, U, gp) - loss(b, U, gp)) / (2 * eps), rel=2e-5, abs=1e-8)
        for idx in [(0, 0), (6, 3)]:
            a, b = U.copy(), U.copy()
            a[idx] += eps
            b[idx] -= eps
            assert r.dU[idx] == pytest.approx((loss(V, a, gp) - loss(V, b, gp)) / (2 * eps), rel=2e-5, abs=1e-8)
        names = ("w_in", "b_in", "w_out", "b_out")
        for k, name in enumerate(names):
            idx = (3, 5) if name != "b_out" else (3,)
            pa = po.GateParams(*(np.copy(getattr(gp, n)) for n in names))
            pb = po.GateParams(*(np.copy(getattr(gp, n)) for n in names))
            getattr(pa, name)[idx] += eps
            getattr(pb, name)[idx] -= eps
            fd = (loss(V, U, pa) - loss(V, U, pb)) / (2 * eps)
            assert r.dgate[k][idx] == pytest.approx(fd, rel=2e-5, abs=1e-8)


@pytest.mark.parametrize("use_delta", [False, True])
def test_c_dense_step_matches_numpy(use_delta):
    from oracle import cpu

    rng = np.random.default_rng(7)
    T, din, dout, C = 64, 24, 40, 48
    x = rng.normal(size=(T, din)).astype(np.float32).astype(np.float64)
    W = (rng.normal(size=(dout, din)) / 5).astype(np.float32).astype(np.float64)
    V = (rng.normal(size=(din, C)) / 5).astype(np.float32).astype(np.float64)
    U = (rng.normal(size=(C, dout)) / 7).astype(np.float32).astype(np.float64)
    gp = _gate(rng, C)
    gp = po.GateParams(*(v.astype(np.float32).astype(np.float64) for v in (gp.w_in, gp.b_in, gp.w_out, gp.b_out)))
    gp.b_out = gp.b_out + 0.25
    key = tf.prng_key(3)
    r = po.dense_site_step(x, W, V, U, gp, key, p=2.0, imp_coeff=0.5, use_delta=use_delta, mask_dtype="bfloat16")
    mk, dk = po.site_keys(key, 0)
    losses, dV, dU, dg = cpu.dense_step(x, W, V, U, gp, mk, dk, use_delta=use_delta, bf16_mask=True, p=2.0,
                                        imp_coeff=0.5)
    np.testing.assert_allclose(losses, [r.loss, r.recon, r.imp], rtol=2e-5)
    np.testing.assert_allclose(dV, r.dV, rtol=1e-4, atol=1e-6 * np.abs(r.dV).max())
    np.testing.assert_allclose(dU, r.dU, rtol=1e-4, atol=1e-6 * np.abs(r.dU).max())
    for got, want in zip(dg, r.dgate):
        np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-6 * max(np.abs(want).max(), 1e-30))


# ------------------------------------------------------------------ routing (reference fixture shapes)

E, K, T_R = 8, 2, 24


def _fixture_top_idx():
    first = np.arange(T_R) % (E - 2)
    return np.stack([first, (first + 1) % (E - 2)], axis=1).astype(np.int32)


def test_routed_jobs_reference_fixture():
    top = _fixture_top_idx()
    jobs = po.routed_jobs(top, E)
    np.testing.assert_array_equal(jobs.group_sizes, np.bincount(top.ravel(), minlength=E))
    np.testing.assert_array_equal(jobs.group_sizes[-2:], [0, 0])
    flat = top.reshape(-1)
    # brute force stable bucketing: experts ascending, job ids ascending inside
    want = [j for e in range(E) for j in range(flat.size) if flat[j] == e]
    np.testing.assert_array_equal(jobs.sort_idx, want)
    np.testing.assert_array_equal(jobs.sort_idx[jobs.inv_sort_idx], np.arange(flat.size))


def test_select_experts_descending_lowest_index_on_ties():
    probs = np.array([[0.1, 0.3, 0.3, 0.05, 0.25, 0.0], [0.2, 0.2, 0.2, 0.2, 0.1, 0.1]])
    np.testing.assert_array_equal(po.select_experts(probs, 3), [[1, 2, 4], [0, 1, 2]])
    w = po.expert_mixing_weights(probs, po.select_experts(probs, 3))
    np.testing.assert_allclose(w.sum(-1), 1.0)
    np.testing.assert_allclose(w[0], np.array([0.3, 0.3, 0.25]) / 0.85)


def test_routed_moe_matches_dense_oracle():
    """Routed (sort -> grouped matmuls -> combine) vs every-expert dense compute with
    the routing vector, the reference's own oracle shape (`tests/routed/test_experts.py:53-96`)."""
    rng = np.random.default_rng(8)
    D, DI = 16, 24
    x = rng.normal(size=(T_R, D))
    wg = rng.normal(size=(E, D, DI)) / 4
    wu = rng.normal(size=(E, D, DI)) / 4
    wd = rng.normal(size=(E, DI, D)) / 5
    top = _fixture_top_idx()
    tw = po.softmax(rng.normal(size=(T_R, K)))
    jobs = po.routed_jobs(top, E)
    xj = po.gather_tokens(x, jobs)
    g = po.grouped_matmul(xj, wg, jobs.group_sizes)
    u = po.grouped_matmul(xj, wu, jobs.group_sizes)
    silu = lambda v: v / (1 + np.exp(-v))
    routed = po.combine_jobs(po.grouped_matmul(silu(g) * u, wd, jobs.group_sizes), jobs, tw)
    routing = np.zeros((T_R, E))
    for t in range(T_R):
        for s in range(K):
            routing[t, top[t, s]] += tw[t, s]
    gd = np.einsum("td,edh->teh", x, wg)
    ud = np.einsum("td,edh->teh", x, wu)
    dense = np.einsum("teh,ehd->td", silu(gd) * ud * routing[..., None], wd)
    np.testing.assert_allclose(routed, dense, rtol=1e-12, atol=1e-12)


def test_transposed_grouped_matmul_ragged_sizes_and_empty_groups():
    sizes = np.array([7, 0, 19, 1, 0, 26, 37, 0])
    rng = np.random.default_rng(9)
    n = int(sizes.sum())
    lhs, dout = rng.normal(size=(n, 8)), rng.normal(size=(n, 12))
    out = po.transposed_grouped_matmul(lhs, dout, sizes)
    starts = np.concatenate([[0], np.cumsum(sizes)])
    for e in range(len(sizes)):
        want = np.zeros((8, 12))
        for j in range(starts[e], starts[e + 1]):
            want += np.outer(lhs[j], dout[j])
        np.testing.assert_allclose(out[e], want, rtol=1e-12, atol=1e-12)
    assert np.all(out[sizes == 0] == 0.0)


def test_gather_tokens_vjp_is_the_adjoint():
    rng = np.random.default_rng(10)
    top = _fixture_top_idx()
    jobs = po.routed_jobs(top, E)
    x = rng.normal(size=(T_R, 5))
    g = rng.normal(size=(T_R * K, 5))
    lhs = float(np.sum(po.gather_tokens(x, jobs) * g))
    rhs = float(np.sum(x * po.gather_tokens_vjp(g, jobs)))
    assert lhs == pytest.approx(rhs, rel=1e-12)
    y = rng.normal(size=(T_R * K, 3))
    np.testing.assert_allclose(po.sum_jobs(y, jobs), np.stack(
        [sum(y[np.where(jobs.sort_idx == t * K + s)[0][0]] for s in range(K)) for t in range(T_R)]))


# ---------------------------------------------------------------- routing samplers
@pytest.mark.parametrize("partitionable", [True, False])
@pytest.mark.parametrize("minval,maxval", [(1, 2), (1, 8), (0, 25), (3, 68), (5, 5), (7, 2)])
def test_randint_is_the_64_bit_value_mod_span(partitionable, minval, maxval):
    """randint's 32-bit remainder steps equal (hi * 2^32 + lo) mod span computed with
    exact integers; span 1 (maxval <= minval) returns minval."""
    key = (7, 1234)
    n = 4000
    k1, k2 = tf.split(key, partitionable=partitionable)
    hi = tf.random_bits(k1, 32, (n,), partitionable=partitionable)
    lo = tf.random_bits(k2, 32, (n,), partitionable=partitionable)
    span = maxval - minval if maxval > minval else 1
    want = np.array([minval + ((int(h) << 32) + int(l)) % span for h, l in zip(hi, lo)], dtype=np.int64)
    got = tf.randint(key, (n,), minval, maxval, partitionable=partitionable)
    assert got.dtype == np.int32
    np.testing.assert_array_equal(got.astype(np.int64), want)


@pytest.mark.parametrize("partitionable", [True, False])
def test_uniform_k_routing_subset_sizes_and_uniformity(partitionable):
    """Each position routes exactly k sites, k = randint(1, S + 1) from the first split
    key; k is uniform over 1..S (chi-square) and each site is routed with probability
    (S + 1) / (2 S)."""
    S, n = 6, 30000
    key = (0, 99)
    routes = po.uniform_k_routing(key, S, (n,), partitionable=partitionable)
    k_key, _ = tf.split(key, partitionable=partitionable)
    k = tf.randint(k_key, (n,), 1, S + 1, partitionable=partitionable)
    np.testing.assert_array_equal(routes.sum(axis=0), k)
    counts = np.bincount(k, minlength=S + 1)[1:]
    chi2 = float(np.sum((counts - n / S) ** 2 / (n / S)))
    assert chi2 < 25.0  # 5 dof; p ~ 1e-4
    np.testing.assert_allclose(routes.mean(axis=1), (S + 1) / (2 * S), atol=0.02)


def test_uniform_k_routing_brute_force_small():
    """S = 3 by hand: routed[j] = (index of the j-th smallest u) < k, stable on ties."""
    key = (3, 4)
    S, n = 3, 50
    k_key, perm_key = tf.split(key)
    k = tf.randint(k_key, (n,), 1, S + 1)
    u = tf.uniform(perm_key, (S, n), "float32")
    routes = po.uniform_k_routing(key, S, (n,))
    for pos in range(n):
        order = sorted(range(S), key=lambda s: (u[s, pos], s))
        for j in range(S):
            assert bool(routes[j, pos]) == (order[j] < k[pos])


def test_static_probability_routing_limits_and_rate():
    key = (1, 2)
    n = 20000
    assert not po.static_probability_routing(key, 3, 0.0, (n,)).any()
    assert po.static_probability_routing(key, 3, 1.0, (n,)).all()
    r = po.static_probability_routing(key, 4, 0.3, (n,))
    np.testing.assert_allclose(r.mean(axis=1), 0.3, atol=0.015)
    u1 = tf.uniform(tf.fold_in(key, 1), (n,), "float32")
    np.testing.assert_array_equal(r[1], u1 < np.float32(0.3))


# ---------------------------------------------------------------- streamed-vocab KL
@pytest.mark.parametrize("n_chunks", [1, 3, 8])
def test_streamed_kl_equals_materialized_kl(n_chunks):
    """The paired online-softmax recurrence equals KL on the materialized logits, for
    any chunking (the result is invariant to the running max)."""
    rng = np.random.default_rng(n_chunks)
    N, d, V = 37, 16, 48
    aq, ap = rng.normal(size=(N, d)), rng.normal(size=(N, d))
    head = rng.normal(size=(V, d))
    kl, stats = po.streamed_position_kl(aq, head, ap, head, n_chunks)
    want = po.kl_per_position(aq @ head.T, ap @ head.T)
    np.testing.assert_allclose(kl, want, rtol=1e-10, atol=1e-13)
    # stats: m_p is the row max, m_p + log s_p the clean log-partition
    zp = ap @ head.T
    np.testing.assert_allclose(stats[:, 0], zp.max(axis=-1), rtol=0, atol=0)
    np.testing.assert_allclose(stats[:, 0] + np.log(stats[:, 1]), np.log(np.exp(zp).sum(axis=-1)), rtol=1e-12)
    assert np.all(kl >= -1e-12)


def test_streamed_kl_vjp_finite_differences():
    rng = np.random.default_rng(0)
    N, d, V = 5, 4, 12
    aq, ap = rng.normal(size=(N, d)), rng.normal(size=(N, d))
    hq, hp = rng.normal(size=(V, d)), rng.normal(size=(V, d))
    g = rng.normal(size=N)
    grad = po.streamed_position_kl_vjp(aq, hq, ap, hp, g)
    eps = 1e-6
    for n in range(N):
        for j in range(d):
            a1, a2 = aq.copy(), aq.copy()
            a1[n, j] += eps
            a2[n, j] -= eps
            f1 = np.dot(g, po.streamed_position_kl(a1, hq, ap, hp, 3)[0])
            f2 = np.dot(g, po.streamed_position_kl(a2, hq, ap, hp, 3)[0])
            assert grad[n, j] == pytest.approx((f1 - f2) / (2 * eps), rel=1e-6, abs=1e-9)


# ---------------------------------------------------------------- block-factored site
@pytest.mark.parametrize("contraction", ["fused_output", "fused_input"])
@pytest.mark.parametrize("with_delta_and_route", [False, True])
def test_blocked_site_einsum_form_matches_per_block_loop(contraction, with_delta_and_route):
    rng = np.random.default_rng(4)
    E, d_in, d_out, c, T = 3, 5, 4, 2, 11
    site_in = d_in * (E if contraction == "fused_input" else 1)
    site_out = d_out * (E if contraction == "fused_output" else 1)
    x = rng.normal(size=(T, site_in))
    V = rng.normal(size=(E, d_in, c)) * 0.3
    U = rng.normal(size=(E, c, d_out)) * 0.3
    W = rng.normal(size=(site_out, site_in))
    mask = rng.uniform(size=(T, E * c))
    delta = rng.uniform(size=T) if with_delta_and_route else None
    route = (rng.uniform(size=T) < 0.5) if with_delta_and_route else None
    got = po.blocked_site_forward(x, W, V, U, mask, delta, route, contraction)
    want = po.blocked_site_forward_loop(x, W, V, U, mask, delta, route, contraction)
    np.testing.assert_allclose(got[0], want[0], rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(got[1], want[1], rtol=1e-12, atol=1e-13)


@pytest.mark.parametrize("contraction", ["fused_output", "fused_input"])
def test_blocked_site_backward_finite_differences(contraction):
    rng = np.random.default_rng(9)
    E, d_in, d_out, c, T = 2, 3, 4, 2, 5
    site_in = d_in * (E if contraction == "fused_input" else 1)
    site_out = d_out * (E if contraction == "fused_output" else 1)
    x = rng.normal(size=(T, site_in))
    V = rng.normal(size=(E, d_in, c))
    U = rng.normal(size=(E, c, d_out))
    W = rng.normal(size=(site_out, site_in))
    mask = rng.uniform(size=(T, E * c))
    delta = rng.uniform(size=T)
    route = rng.uniform(size=T) < 0.6
    G = rng.normal(size=(T, site_out))
    grads = po.blocked_site_backward(x, W, V, U, mask, delta, route, contraction, G)

    def f(x_, V_, U_, m_):
        return float(np.sum(G * po.blocked_site_forward(x_, W, V_, U_, m_, delta, route, contraction)[0]))

    for which, arr in enumerate((x, V, U, mask)):
        for _ in range(4):
            idx = tuple(rng.integers(0, n) for n in arr.shape)
            args = [x, V, U, mask]
            a1, a2 = arr.copy(), arr.copy()
            a1[idx] += 1e-6
            a2[idx] -= 1e-6
            args[which] = a1
            f1 = f(*args)
            args[which] = a2
            f2 = f(*args)
            assert grads[(0, 1, 2, 3)[which]][idx] == pytest.approx((f1 - f2) / 2e-6, rel=1e-6, abs=1e-8)
