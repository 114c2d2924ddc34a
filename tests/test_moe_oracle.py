"""Pins the MoE-stack oracle: central finite differences of its loss against its
hand-written backward (V, U of every site, the CI preactivations and the stack input),
and the routed forward against an every-expert dense spelling of the same layer."""

import numpy as np
import pytest

from oracle import moe_oracle as mo
from oracle import pd_oracle as po


def _setup(seed=0, L=2):
    cfg = mo.MoEConfig(T=12, d=8, f=6, E=5, k=2, c=4, L=L)
    rng = np.random.default_rng(seed)
    params, x0, _ = mo.init_moe(cfg, rng)
    # CI in (0, 1): there the lower squashing's custom VJP is the true derivative
    ci = [{s: rng.uniform(0.05, 0.95, size=(cfg.T, cfg.k, cfg.c)) for s in mo.SITES} for _ in range(L)]
    return cfg, params, x0, ci


def _loss(cfg, params, x0, ci):
    return mo.moe_stack_step(cfg, params, x0, ci, (0, 3), p=2.0, imp_coeff=0.3, recon_coeff=1.7)["loss"]


def test_moe_backward_matches_finite_differences():
    cfg, params, x0, ci = _setup()
    res = mo.moe_stack_step(cfg, params, x0, ci, (0, 3), p=2.0, imp_coeff=0.3, recon_coeff=1.7)
    eps = 1e-6
    rng = np.random.default_rng(1)
    for l in range(cfg.L):
        for name in ("Vg", "Ug", "Vu", "Uu", "Vd", "Ud"):
            arr = params[l][name]
            for _ in range(3):
                idx = tuple(int(rng.integers(0, s)) for s in arr.shape)
                old = arr[idx]
                arr[idx] = old + eps
                lp = _loss(cfg, params, x0, ci)
                arr[idx] = old - eps
                lm = _loss(cfg, params, x0, ci)
                arr[idx] = old
                assert res["grads"][l][name][idx] == pytest.approx((lp - lm) / (2 * eps), rel=1e-5, abs=1e-9), (l, name)
        for s in mo.SITES:
            arr = ci[l][s]
            for _ in range(3):
                idx = tuple(int(rng.integers(0, n)) for n in arr.shape)
                old = arr[idx]
                arr[idx] = old + eps
                lp = _loss(cfg, params, x0, ci)
                arr[idx] = old - eps
                lm = _loss(cfg, params, x0, ci)
                arr[idx] = old
                assert res["d_ci_pre"][l][s][idx] == pytest.approx((lp - lm) / (2 * eps), rel=1e-5, abs=1e-9)


def test_moe_input_gradient_through_router_and_norm():
    """dL/dx0 through the masked pass only (the clean pass is detached): perturb x0 in
    the masked pass alone by holding the clean pass's inputs fixed."""
    cfg, params, x0, ci = _setup(seed=2)
    base = mo.moe_stack_step(cfg, params, x0, ci, (0, 3), p=2.0, imp_coeff=0.3, recon_coeff=1.7)
    eps = 1e-6

    def masked_loss(x):
        # clean pass on the unperturbed x0: rerun with the clean residual replaced
        r = mo.moe_stack_step(cfg, params, x, ci, (0, 3), p=2.0, imp_coeff=0.3, recon_coeff=1.7)
        assert all(np.array_equal(a, b) for a, b in zip(r["top_idx"], base["top_idx"]))
        return np.mean((r["r_final"] - base["rc_final"]) ** 2) * 1.7 + 0.3 * r["imp"]

    for idx in [(0, 0), (5, 3), (11, 7)]:
        xp, xm = x0.copy(), x0.copy()
        xp[idx] += eps
        xm[idx] -= eps
        assert base["dx0"][idx] == pytest.approx((masked_loss(xp) - masked_loss(xm)) / (2 * eps), rel=1e-5, abs=1e-9)


def test_moe_layer_routed_equals_dense_spelling():
    """One decomposed layer, routed job space vs computing every expert densely and
    masking by the routing (the reference's `dense_masked` arm is its numerical oracle,
    `pd/core/README.md:241-247`)."""
    cfg, params, x0, ci = _setup(seed=3, L=1)
    P = params[0]
    res = mo.moe_stack_step(cfg, params, x0, ci, (0, 3))
    idx = res["top_idx"][0]
    h2, _ = mo.rms_norm_zero_centered(x0, P["ln"], cfg.eps)
    probs = po.softmax(h2 @ P["router"].T)
    w = po.expert_mixing_weights(probs, idx)
    keys = mo.site_mask_keys((0, 3), 0)
    from oracle import threefry as tf

    m = {}
    for s in mo.SITES:
        lo = po.lower_leaky(ci[0][s])
        u = tf.uniform(keys[s], (cfg.T, cfg.k * cfg.c), "bfloat16").reshape(cfg.T, cfg.k, cfg.c)
        m[s] = lo + (1 - lo) * u
    out = x0.copy()
    for t in range(cfg.T):
        acc = np.zeros(cfg.d)
        for slot in range(cfg.k):
            e = idx[t, slot]
            g = ((h2[t] @ P["Vg"][e]) * m["gate"][t, slot]) @ P["Ug"][e]
            u_ = ((h2[t] @ P["Vu"][e]) * m["up"][t, slot]) @ P["Uu"][e]
            din = mo.silu(g) * u_ * w[t, slot]
            acc += ((din @ P["Vd"][e]) * m["down"][t, slot]) @ P["Ud"][e]
        out[t] += acc
    np.testing.assert_allclose(res["r_final"], out, rtol=1e-12, atol=1e-12)
