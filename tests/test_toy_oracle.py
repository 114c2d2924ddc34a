"""CPU checks of the toy-target oracle: finite differences of the whole step loss pin its
backward (gates held in their linear range, where the lower sigmoid's custom VJP equals
the true derivative), plus target invariants."""

import numpy as np
import pytest

from oracle import pd_oracle as po
from oracle import toy_oracle as to


def _linear_gates(sites, rng):
    """Gate operating point inside (0, 1): small output weights around b_out = 0.5."""
    for s in sites:
        C, H = s.gate.w_in.shape
        s.gate = po.GateParams(rng.normal(size=(C, H)), rng.normal(size=(C, H)) * 0.3,
                               rng.normal(size=(C, H)) * 0.05, 0.5 + rng.normal(size=C) * 0.05)


def _loss(kind, target, sites, x, key, **kw):
    return to.toy_step(kind, target, sites, x, key, **kw)["loss"]


def _fd_check(kind, target, sites, x, key, rng, **kw):
    res = to.toy_step(kind, target, sites, x, key, **kw)
    for i, s in enumerate(sites):
        assert all(np.all((g > 0.02) & (g < 0.98)) for g in res["g_raw"]), "gate left its linear range"
        params = [("V", s.V, res["dV"][i]), ("U", s.U, res["dU"][i]),
                  ("w_in", s.gate.w_in, res["dgate"][i][0]), ("b_in", s.gate.b_in, res["dgate"][i][1]),
                  ("w_out", s.gate.w_out, res["dgate"][i][2]), ("b_out", s.gate.b_out, res["dgate"][i][3])]
        for name, arr, grad in params:
            for _ in range(3):
                idx = tuple(rng.integers(0, n) for n in arr.shape)
                old = arr[idx]
                eps = 1e-6
                arr[idx] = old + eps
                lp = _loss(kind, target, sites, x, key, **kw)
                arr[idx] = old - eps
                lm = _loss(kind, target, sites, x, key, **kw)
                arr[idx] = old
                fd = (lp - lm) / (2 * eps)
                assert grad[idx] == pytest.approx(fd, rel=2e-4, abs=1e-9), f"{s.name}.{name}{idx}"


@pytest.mark.parametrize("use_delta,routed", [(False, False), (True, False), (True, True)])
def test_tms_step_finite_differences(use_delta, routed):
    rng = np.random.default_rng(5)
    cfg = to.TMSConfig(n_features=5, n_hidden=2, C=6, batch=40, feature_probability=1.0)
    target, sites = to.tms_init(cfg, rng)
    target["b2"] = rng.normal(size=5) * 0.3
    _linear_gates(sites, rng)
    x = to.tms_batch(cfg, rng)
    routes = None
    if routed:
        routes = [rng.uniform(size=cfg.batch) < 0.6 for _ in sites]
    _fd_check("tms", target, sites, x, (0, 11), rng, p=1.0, imp_coeff=0.7, recon_coeff=1.3, use_delta=use_delta,
              routes=routes)


@pytest.mark.parametrize("use_delta", [False, True])
def test_resid_mlp_step_finite_differences(use_delta):
    rng = np.random.default_rng(6)
    cfg = to.ResidMLPConfig(n_features=6, d_embed=10, d_mlp=4, n_layers=2, C=5, batch=24, feature_probability=0.7)
    target, sites = to.resid_mlp_init(cfg, rng)
    _linear_gates(sites, rng)
    x = to.resid_mlp_batch(cfg, rng)
    _fd_check("resid_mlp", target, sites, x, (3, 4), rng, p=2.0, imp_coeff=0.4, recon_coeff=2.0,
              use_delta=use_delta)


def test_toy_targets_invariants():
    rng = np.random.default_rng(0)
    target, sites = to.tms_init(to.TMSConfig(), rng)
    np.testing.assert_array_equal(sites[1].W, sites[0].W.T)
    assert np.all(np.abs(sites[0].W) <= 1 / np.sqrt(5))
    rt, rs = to.resid_mlp_init(to.ResidMLPConfig(n_features=20, d_embed=30, d_mlp=8, C=4), rng)
    np.testing.assert_allclose(np.linalg.norm(rt["W_E"], axis=-1), 1.0, rtol=1e-12)
    np.testing.assert_array_equal(rt["W_U"], rt["W_E"].T)
    assert [s.name for s in rs] == ["layers.0.mlp_in", "layers.0.mlp_out"]


def test_toy_step_with_full_masks_reproduces_clean_output():
    """Masks of all ones, no delta and V@U = W^T make the masked forward the clean one
    (recon 0), whatever the gate says: mask = lower + (1 - lower) * u = 1 when lower = 1."""
    rng = np.random.default_rng(1)
    cfg = to.TMSConfig(n_features=5, n_hidden=2, C=5, batch=16, feature_probability=1.0)
    target, sites = to.tms_init(cfg, rng)
    for s in sites:
        d_out, d_in = s.W.shape
        s.V = np.eye(d_in, cfg.C)
        s.U = np.zeros((cfg.C, d_out))
        s.U[:d_in] = s.W.T
        C, H = s.gate.w_in.shape
        s.gate = po.GateParams(np.zeros((C, H)), np.zeros((C, H)), np.zeros((C, H)), np.full(C, 3.0))
    x = to.tms_batch(cfg, rng)
    res = to.toy_step("tms", target, sites, x, (0, 1))
    assert res["recon"] == pytest.approx(0.0, abs=1e-24)
    np.testing.assert_allclose(res["out"], res["clean"], rtol=1e-12, atol=1e-15)
    # upper = 1 + 0.01 * (3 - 1) for every component of both sites: imp = 2 * C * 1.02^p
    assert res["imp"] == pytest.approx(2 * cfg.C * 1.02, rel=1e-12)
