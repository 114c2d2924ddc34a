"""The oracle's EMA frequency estimator against the reference's own closed-form EMA
tests (pd/tests/core/test_frequency_minimality.py:169-300), restated on the oracle:
step-0 identity at the half-life cap, bounded fp32 drift of the update form over a full
run, stationary batches, the varying-batch closed form, settling near Phi(mean f), and
the surrogate gradient's scale at stationarity. The site-level EMA arm of the imp-min
(`impmin_site_terms_ema`) is then pinned against the plain batch arm at step 0 and against
torch autograd of the reference's surrogate spelling."""

import math

import numpy as np
import pytest

from oracle import pd_oracle as po

GAMMA = 1.0


def _freqs(ci, gamma=GAMMA, normalize=False):
    return po.smooth_l0_psi(np.asarray(ci, np.float64), gamma, normalize).mean(axis=0)


def test_ema_finite_at_extreme_halflife():
    # the expm1 form stays finite at the 1e6 cap; step 0 reproduces the batch penalty
    f = _freqs([[0.2, 0.8], [0.4, 0.1]])
    value, new = po.ema_frequency_penalty({"a": f}, {"a": np.zeros(2)}, 0.0, 1e6, 64)
    batch = float(np.sum(po.frequency_curve(f, 64)))
    assert math.isfinite(value) and np.isfinite(new["a"]).all()
    assert math.isclose(value, batch, rel_tol=1e-4)
    # the subtractive form would cancel: 1 - 2^(-1/h) is representable only via expm1
    alpha, debias = po.ema_decay_terms(0.0, 1e6)
    assert alpha > 0 and debias > 0 and math.isclose(alpha, debias)


@pytest.mark.parametrize("halflife,bound", [(1e6, 1e-4), (1e4, 1e-3)])
def test_ema_long_scan_rounding_bounded(halflife, bound):
    """400k constant-f updates of the recurrence in fp32, as the kernels run it
    (new = e + alpha (f - e), alpha rounded to fp32), debiased exactly in double."""
    f = np.float32(0.5)
    alpha = np.float32(-math.expm1(-math.log(2.0) / halflife))
    e = np.float32(0.0)
    steps = 400_000
    for _ in range(steps):
        e = np.float32(e + np.float32(alpha * np.float32(f - e)))
    debias = -math.expm1(-math.log(2.0) / halflife * steps)
    assert abs(float(e) / debias - 0.5) <= bound * 0.5, (halflife, float(e) / debias)


def test_ema_stationary_equals_batch_penalty():
    f = _freqs([[0.2, 0.8], [0.4, 0.1]])
    ema = {"a": np.zeros(2)}
    batch = float(np.sum(po.frequency_curve(f, 64)))
    for step in range(6):
        value, ema = po.ema_frequency_penalty({"a": f}, ema, float(step), 8.0, 64)
        assert math.isclose(value, batch, rel_tol=1e-5), step


def test_ema_matches_closed_form():
    halflife, a = 4.0, 32
    decay = 0.5 ** (1.0 / halflife)
    fs = [np.array([0.1, 0.5]), np.array([0.3, 0.2]), np.array([0.05, 0.9])]
    ema = {"a": np.zeros(2)}
    value = 0.0
    for step, f in enumerate(fs):
        value, ema = po.ema_frequency_penalty({"a": f}, ema, float(step), halflife, a)
    expected = (1 - decay) * sum(decay ** (2 - i) * f for i, f in enumerate(fs))
    np.testing.assert_allclose(ema["a"], expected, rtol=1e-12)
    f_hat = expected / (1 - decay**3)
    assert math.isclose(value, float(np.sum(f_hat * np.log2(1 + a * f_hat))), rel_tol=1e-12)


def test_ema_smooths_toward_mean():
    halflife, a = 16.0, 1024

    def phi(f):
        return float(np.sum(f * np.log2(1 + a * f)))

    f_hi, f_lo = np.array([0.2]), np.array([0.0])
    f_mean = (f_hi + f_lo) / 2
    ema = {"a": np.zeros(1)}
    value = 0.0
    for step in range(300):
        value, ema = po.ema_frequency_penalty({"a": f_hi if step % 2 == 0 else f_lo}, ema, float(step), halflife, a)
    assert abs(value - phi(f_mean)) < 0.1 * (phi(f_hi) - phi(f_mean))


def test_ema_gradient_matches_unsmoothed_at_stationarity():
    """Step 0 with a zero estimate: f_hat = f, so the site arm's value and CI gradient equal
    the batch arm's at full scale (no shrink by 1 - decay)."""
    rng = np.random.default_rng(0)
    up = rng.uniform(0.0, 1.1, size=(64, 12))
    spec = po.ImpMin("smooth_l0", coeff=0.7, gamma=0.3, normalize_at_one=True, freq_coeff=0.4, ref_count=64.0,
                     ema_halflife=50.0)
    a0, f0, g0 = po.impmin_site_terms(up, spec, 64)
    a1, f1, g1, new, fb = po.impmin_site_terms_ema(up, spec, 64, ema=np.zeros(12), count=0.0)
    assert math.isclose(a0, a1) and math.isclose(f0, f1, rel_tol=1e-12) and math.isclose(fb, f0, rel_tol=1e-12)
    np.testing.assert_allclose(g1, g0, rtol=1e-12)
    alpha, _ = po.ema_decay_terms(0.0, 50.0)
    np.testing.assert_allclose(new, alpha * po.smooth_l0_psi(up, 0.3, True).mean(0), rtol=1e-12)


def test_ema_counts_observations_in_the_debias():
    """Three observations, then one: the estimate debiased by its own count (the
    reference's test_ema_counts_its_own_observations) reproduces a constant batch."""
    f = np.full(2, 0.3)
    ema = {"a": np.zeros(2)}
    for step, v in enumerate((0.2, 0.7, 0.4)):
        _, ema = po.ema_frequency_penalty({"a": np.full(2, v)}, ema, float(step), 4.0, 64)
    value, _ = po.ema_frequency_penalty({"a": f}, {"a": np.zeros(2)}, 0.0, 4.0, 64)
    assert math.isclose(value, float(np.sum(po.frequency_curve(f, 64))), rel_tol=1e-12)
    # the frequent estimator's next value differs from its batch value (it remembers)
    v3, _ = po.ema_frequency_penalty({"a": f}, ema, 3.0, 4.0, 64)
    assert not math.isclose(v3, float(np.sum(po.frequency_curve(f, 64))), rel_tol=1e-3)


@pytest.mark.parametrize("groups", [None, "experts"])
def test_site_ema_gradient_equals_autograd_of_the_surrogate(groups):
    """The hand-written slope Phi'(f_hat) / n psi'(up) equals torch autograd (float64) of
    the reference's spelling Phi(f_hat) + Phi'(f_hat) (f - sg(f)) with f_hat from the
    stop-gradded f, on a mid-run estimate (count 5), also with expert-grouped rows."""
    import torch

    rng = np.random.default_rng(1)
    n, c, E = 48, 8, 3
    up = rng.uniform(0.0, 1.2, size=(n, 2, c))
    g = rng.integers(0, E, size=(n, 2)) if groups else None
    n_groups = E if groups else 1
    spec = po.ImpMin("smooth_l0", coeff=0.5, gamma=0.25, normalize_at_one=False, freq_coeff=0.3, ref_count=200.0,
                     ema_halflife=6.0)
    ema = rng.uniform(0.0, 0.4, size=n_groups * c)
    act, freq, grad, new, fb = po.impmin_site_terms_ema(up, spec, n, g, n_groups, ema=ema, count=5.0)

    t_up = torch.tensor(up, dtype=torch.float64, requires_grad=True)
    psi = t_up**2 / (t_up**2 + spec.gamma**2)
    idx = torch.zeros(n * 2, dtype=torch.long) if g is None else torch.as_tensor(g.reshape(-1), dtype=torch.long)
    F = torch.zeros(n_groups, c, dtype=torch.float64).index_add(0, idx, psi.reshape(-1, c)) / n
    fr = F.reshape(-1)
    alpha, debias = po.ema_decay_terms(5.0, 6.0)
    f_sg = fr.detach()
    prev = torch.tensor(ema)
    f_hat = (prev + alpha * (f_sg - prev)) / debias
    a = spec.ref_count
    slope = torch.log2(1 + a * f_hat) + a * f_hat / ((1 + a * f_hat) * math.log(2.0))
    value = f_hat * torch.log2(1 + a * f_hat) + slope * (fr - f_sg)
    loss = spec.coeff * fr.sum() + spec.freq_coeff * value.sum()
    (want,) = torch.autograd.grad(loss, t_up)
    np.testing.assert_allclose(grad, want.numpy(), rtol=1e-10, atol=1e-14)
    assert math.isclose(freq, float(value.detach().sum()), rel_tol=1e-12)
    np.testing.assert_allclose(new, (prev + alpha * (f_sg - prev)).numpy(), rtol=1e-12)
    assert math.isclose(fb, float((f_sg * torch.log2(1 + a * f_sg)).sum()), rel_tol=1e-12)
    assert math.isclose(act, float(fr.detach().sum()), rel_tol=1e-12)
