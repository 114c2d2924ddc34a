"""Pins the MoE-stack oracle: central finite differences of its loss against its
hand-written backward (V, U of every site, the CI preactivations and the stack input),
the routed forward against a per-token, per-expert spelling of the same layer (mask,
delta draws and frozen channel included), and the delta channel's defining identity:
with every component live (m = 1) and V_e U_e = W_e the masked stack reproduces the
clean one for any delta draw."""

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
    dkeys = mo.site_delta_keys((0, 3), 0)
    from oracle import threefry as tf

    m, dl = {}, {}
    for s in mo.SITES:
        lo = po.lower_leaky(ci[0][s])
        u = tf.uniform(keys[s], (cfg.T, cfg.k * cfg.c), "bfloat16").reshape(cfg.T, cfg.k, cfg.c)
        m[s] = lo + (1 - lo) * u
        # one bf16 draw per token, from the second half of the split draw key
        dl[s] = tf.uniform(dkeys[s], (cfg.T,), "bfloat16")
        assert np.all((dl[s] >= 0) & (dl[s] < 1)) and np.all(dl[s] * 128 == np.round(dl[s] * 128))
        np.testing.assert_array_equal(res["deltas"][0][s], dl[s])
    out = x0.copy()
    for t in range(cfg.T):
        acc = np.zeros(cfg.d)
        for slot in range(cfg.k):
            e = idx[t, slot]
            g = (((h2[t] @ P["Vg"][e]) * (m["gate"][t, slot] - dl["gate"][t])) @ P["Ug"][e]
                 + dl["gate"][t] * (h2[t] @ P["Wg"][e]))
            u_ = (((h2[t] @ P["Vu"][e]) * (m["up"][t, slot] - dl["up"][t])) @ P["Uu"][e]
                  + dl["up"][t] * (h2[t] @ P["Wu"][e]))
            din = mo.silu(g) * u_ * w[t, slot]
            acc += (((din @ P["Vd"][e]) * (m["down"][t, slot] - dl["down"][t])) @ P["Ud"][e]
                    + dl["down"][t] * (din @ P["Wd"][e]))
        out[t] += acc
    np.testing.assert_allclose(res["r_final"], out, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("v", [0.0, 0.375])
def test_moe_constant_sources_gradients_and_ci_masked_form(v):
    """Constant sources u = d = v: central differences of the loss in V, U and the CI,
    and at v = 0 (the CI-masked recon) the masked layer is the per-token spelling with
    m = lower(ci) and no frozen share."""
    cfg, params, x0, ci = _setup(seed=4, L=1)
    kw = dict(p=2.0, imp_coeff=0.3, recon_coeff=1.7, source_value=v)
    res = mo.moe_stack_step(cfg, params, x0, ci, (0, 3), **kw)
    eps = 1e-6
    rng = np.random.default_rng(7)
    for arr, grad in ((params[0]["Vg"], res["grads"][0]["Vg"]), (params[0]["Ud"], res["grads"][0]["Ud"]),
                      (ci[0]["up"], res["d_ci_pre"][0]["up"])):
        for _ in range(3):
            idx = tuple(int(rng.integers(0, n)) for n in arr.shape)
            old = arr[idx]
            arr[idx] = old + eps
            lp = mo.moe_stack_step(cfg, params, x0, ci, (0, 3), **kw)["loss"]
            arr[idx] = old - eps
            lm = mo.moe_stack_step(cfg, params, x0, ci, (0, 3), **kw)["loss"]
            arr[idx] = old
            assert grad[idx] == pytest.approx((lp - lm) / (2 * eps), rel=1e-5, abs=1e-9)
    if v == 0.0:
        P = params[0]
        idx = res["top_idx"][0]
        h2, _ = mo.rms_norm_zero_centered(x0, P["ln"], cfg.eps)
        w = po.expert_mixing_weights(po.softmax(h2 @ P["router"].T), idx)
        m = {s: po.lower_leaky(ci[0][s]) for s in mo.SITES}
        out = x0.copy()
        for t in range(cfg.T):
            for slot in range(cfg.k):
                e = idx[t, slot]
                g = ((h2[t] @ P["Vg"][e]) * m["gate"][t, slot]) @ P["Ug"][e]
                u_ = ((h2[t] @ P["Vu"][e]) * m["up"][t, slot]) @ P["Uu"][e]
                din = mo.silu(g) * u_ * w[t, slot]
                out[t] += ((din @ P["Vd"][e]) * m["down"][t, slot]) @ P["Ud"][e]
        np.testing.assert_allclose(res["r_final"], out, rtol=1e-12, atol=1e-12)


def test_moe_delta_channel_restores_the_target_when_every_component_is_live():
    """ci >= 1 (lower(ci) = 1, m = 1) and exact factorizations V_e U_e = W_e: the site
    output (h (1 - d)) U + d x W = x W whatever d is, so the masked stack equals the clean
    one and the recon term vanishes. Dropping the frozen term, flipping the coefficient's
    sign or using the mask draw for d all break it (the delta draws are far from 0)."""
    cfg = mo.MoEConfig(T=16, d=8, f=6, E=4, k=2, c=8, L=2)
    rng = np.random.default_rng(5)
    params, x0, _ = mo.init_moe(cfg, rng)
    for P in params:
        for s, (din_, dout_) in (("g", (cfg.d, cfg.f)), ("u", (cfg.d, cfg.f)), ("d", (cfg.f, cfg.d))):
            V = P["V" + s][:, :din_, :]
            # c >= d_in: V_e invertible on its leading d_in components; U_e solves V_e U_e = W_e
            U = np.zeros((cfg.E, cfg.c, dout_))
            for e in range(cfg.E):
                U[e] = np.linalg.lstsq(V[e], P["W" + s][e], rcond=None)[0]
            P["U" + s] = U
            np.testing.assert_allclose(np.einsum("eic,eco->eio", V, U), P["W" + s], atol=1e-10)
    ci = [{s: np.full((cfg.T, cfg.k, cfg.c), 1.2) for s in mo.SITES} for _ in range(cfg.L)]
    res = mo.moe_stack_step(cfg, params, x0, ci, (0, 7), p=2.0, imp_coeff=0.0, recon_coeff=1.0)
    assert min(float(d.max()) for layer in res["deltas"] for d in layer.values()) > 0.5
    np.testing.assert_allclose(res["r_final"], res["rc_final"], rtol=1e-10, atol=1e-10)
    assert res["recon"] < 1e-20
    # a stack whose factorization is off reconstructs only approximately: the identity
    # above is not vacuous
    bent = [dict(P) for P in params]
    bent[0]["Vg"] = bent[0]["Vg"] * 1.1
    res2 = mo.moe_stack_step(cfg, bent, x0, ci, (0, 7), p=2.0, imp_coeff=0.0, recon_coeff=1.0)
    assert res2["recon"] > 1e-6
    # with the bent factorization the delta draw matters: d x (W - V U) differs per draw
    res3 = mo.moe_stack_step(cfg, bent, x0, ci, (0, 7), p=2.0, imp_coeff=0.0, recon_coeff=1.0, use_delta=False)
    assert abs(res3["recon"] - res2["recon"]) > 1e-3 * res2["recon"]


def test_selection_within_ulps_accepts_only_near_ties():
    # 0.999 rounds to bf16 1.0: experts 0 and 2 tie, so either order is a valid top-2
    raw = np.array([1.0, 0.5, 0.999, 0.2, -1.0])
    assert mo.selection_within_ulps(raw, [0, 2], 2) and mo.selection_within_ulps(raw, [2, 0], 2)
    # 0.9 is 13 ulps below 1.0: only the exact order is accepted
    raw = np.array([1.0, 0.5, 0.9, 0.2, -1.0])
    assert mo.selection_within_ulps(raw, [0, 2], 2)
    assert not mo.selection_within_ulps(raw, [2, 0], 2)
    assert not mo.selection_within_ulps(raw, [0, 1], 2)  # a wrong member
    assert not mo.selection_within_ulps(raw, [0, 0], 2)  # a repeated expert
    # each logit may move one ulp, so values one or two ulps apart may swap; three may not
    raw = np.array([1.0, 1.0078125, 1.0234375, -3.0])
    assert mo.selection_within_ulps(raw, [2, 1, 0], 3) and mo.selection_within_ulps(raw, [2, 0, 1], 3)
    assert mo.selection_within_ulps(raw, [1, 2, 0], 3)  # two ulps: a tie, broken by the lower index
    assert not mo.selection_within_ulps(raw, [0, 2, 1], 3)  # three ulps apart
    assert not mo.selection_within_ulps(raw, [0, 1, 2], 3)


def test_pinned_routing_reproduces_the_oracles_own_step():
    cfg = mo.MoEConfig(T=40, d=16, f=8, E=6, k=2, c=4, L=2)
    params, x0, ci = mo.init_moe(cfg, np.random.default_rng(3))
    a = mo.moe_stack_step(cfg, params, x0, ci, (1, 2), bf16_storage=True)
    b = mo.moe_stack_step(cfg, params, x0, ci, (1, 2), bf16_storage=True, pinned_top_idx=a["own_top_idx"])
    assert a["loss"] == b["loss"]
    for l in range(cfg.L):
        np.testing.assert_array_equal(a["top_idx"][l], b["top_idx"][l])
        np.testing.assert_array_equal(a["grads"][l]["Vd"], b["grads"][l]["Vd"])


def test_torch_restatement_matches_the_numpy_oracle():
    """The torch (autograd) restatement used for the CPU baseline equals the NumPy
    oracle's hand-written backward in float64: loss, every V/U gradient and the CI
    preactivation gradients (CI kept away from the squashing kinks, where the torch
    form's plain clamp derivative and the reference's custom lower VJP agree)."""
    cfg = mo.MoEConfig(T=48, d=16, f=8, E=6, k=2, c=4, L=2)
    rng = np.random.default_rng(11)
    params, x0, _ = mo.init_moe(cfg, rng)
    ci = [{s: rng.uniform(0.05, 0.95, size=(cfg.T, cfg.k, cfg.c)) for s in mo.SITES} for _ in range(cfg.L)]
    a = mo.moe_stack_step(cfg, params, x0, ci, (3, 4), p=2.0, imp_coeff=0.5, recon_coeff=1.5)
    b = mo.moe_stack_step_torch(cfg, params, x0, ci, (3, 4), p=2.0, imp_coeff=0.5, recon_coeff=1.5)
    assert b["loss"] == pytest.approx(a["loss"], rel=1e-10)
    for l in range(cfg.L):
        np.testing.assert_array_equal(a["top_idx"][l], b["top_idx"][l])
        for n in ("Vg", "Ug", "Vu", "Uu", "Vd", "Ud"):
            np.testing.assert_allclose(b["grads"][l][n], a["grads"][l][n], rtol=1e-8, atol=1e-12)
        for s in mo.SITES:
            np.testing.assert_allclose(b["d_ci_pre"][l][s], a["d_ci_pre"][l][s], rtol=1e-8, atol=1e-12)


@pytest.mark.parametrize("normalize", [False, True])
@pytest.mark.parametrize("ref_count", [0.0, 64.0])
def test_selected_smooth_l0_equals_the_dense_reference_form(normalize, ref_count):
    """A selected-emitting site's smooth-L0 terms (values [T, k, c] scattered to their
    expert's block of the [E * c] components) equal the reference's dense formula on the
    scattered [T, E * c] upper CI (zeros where unselected, psi(0) = 0), and the gradient
    matches central differences of activity + frequency."""
    rng = np.random.default_rng(5)
    T, k, c, E = 40, 3, 4, 6
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)])
    up = rng.uniform(0.0, 1.2, size=(T, k, c))
    spec = po.ImpMin("smooth_l0", coeff=0.7, gamma=0.3, normalize_at_one=normalize, freq_coeff=0.4,
                     ref_count=ref_count)
    act, freq, grad = po.impmin_site_terms(up, spec, T, idx, E)
    dense = np.zeros((T, E, c))
    for t in range(T):
        for s_ in range(k):
            dense[t, idx[t, s_]] = up[t, s_]
    wa, wf = po.importance_minimality_terms([dense.reshape(T, E * c)], 0.3, ref_count if ref_count else None,
                                            normalize)
    assert act == pytest.approx(wa, rel=1e-12) and freq == pytest.approx(wf, rel=1e-12, abs=1e-15)

    def loss(u):
        a_, f_, _ = po.impmin_site_terms(u, spec, T, idx, E)
        return spec.loss(a_, f_)

    for ii in [(0, 0, 0), (7, 2, 3), (39, 1, 1), (12, 0, 2)]:
        e = 1e-6
        upp, upm = up.copy(), up.copy()
        upp[ii] += e
        upm[ii] -= e
        assert grad[ii] == pytest.approx((loss(upp) - loss(upm)) / (2 * e), rel=1e-5, abs=1e-9)


def test_smooth_l0_moe_step_matches_the_autograd_restatement():
    """The NumPy oracle's smooth-L0 + frequency backward (per-expert frequency slopes)
    against torch autograd through the reference's scatter form, in float64."""
    cfg = mo.MoEConfig(T=48, d=16, f=8, E=6, k=2, c=4, L=2)
    rng = np.random.default_rng(13)
    params, x0, _ = mo.init_moe(cfg, rng)
    ci = [{s: rng.uniform(0.05, 0.95, size=(cfg.T, cfg.k, cfg.c)) for s in mo.SITES} for _ in range(cfg.L)]
    spec = po.ImpMin("smooth_l0", coeff=0.5, gamma=0.2, normalize_at_one=True, freq_coeff=0.3, ref_count=96.0)
    a = mo.moe_stack_step(cfg, params, x0, ci, (3, 4), recon_coeff=1.5, imp_min=spec)
    b = mo.moe_stack_step_torch(cfg, params, x0, ci, (3, 4), recon_coeff=1.5, imp_min=spec)
    assert b["loss"] == pytest.approx(a["loss"], rel=1e-10)
    assert b["imp"] == pytest.approx(a["imp"], rel=1e-10) and b["freq"] == pytest.approx(a["freq"], rel=1e-10)
    assert a["freq"] > 0
    for l in range(cfg.L):
        for n in ("Vg", "Ug", "Vu", "Uu", "Vd", "Ud"):
            np.testing.assert_allclose(b["grads"][l][n], a["grads"][l][n], rtol=1e-8, atol=1e-12)
        for s in mo.SITES:
            np.testing.assert_allclose(b["d_ci_pre"][l][s], a["d_ci_pre"][l][s], rtol=1e-8, atol=1e-12)


def test_smooth_l0_ema_moe_step_matches_the_autograd_restatement():
    """With the EMA frequency estimate (mid-run: count 4, a nonzero estimate per expert
    block) the NumPy oracle's slope Phi'(f_hat) equals torch autograd of the reference's
    surrogate Phi(f_hat) + Phi'(f_hat) (f - sg(f)) through the scatter form, and the new
    estimate is ema + alpha (f - ema) per (layer, site)."""
    cfg = mo.MoEConfig(T=48, d=16, f=8, E=6, k=2, c=4, L=2)
    rng = np.random.default_rng(17)
    params, x0, _ = mo.init_moe(cfg, rng)
    ci = [{s: rng.uniform(0.05, 0.95, size=(cfg.T, cfg.k, cfg.c)) for s in mo.SITES} for _ in range(cfg.L)]
    spec = po.ImpMin("smooth_l0", coeff=0.5, gamma=0.2, normalize_at_one=True, freq_coeff=0.3, ref_count=96.0,
                     ema_halflife=5.0)
    ema = rng.uniform(0.0, 0.3, size=(cfg.L, 3, cfg.E * cfg.c))
    a = mo.moe_stack_step(cfg, params, x0, ci, (3, 4), recon_coeff=1.5, imp_min=spec, freq_ema=ema, ema_count=4.0)
    b = mo.moe_stack_step_torch(cfg, params, x0, ci, (3, 4), recon_coeff=1.5, imp_min=spec, freq_ema=ema,
                                ema_count=4.0)
    batch = mo.moe_stack_step(cfg, params, x0, ci, (3, 4), recon_coeff=1.5, imp_min=spec)
    assert b["loss"] == pytest.approx(a["loss"], rel=1e-10) and b["freq"] == pytest.approx(a["freq"], rel=1e-10)
    assert a["freq_batch"] == pytest.approx(batch["freq"], rel=1e-12) and abs(a["freq"] - batch["freq"]) > 1e-3
    for l in range(cfg.L):
        for n in ("Vg", "Ug", "Vu", "Uu", "Vd", "Ud"):
            np.testing.assert_allclose(b["grads"][l][n], a["grads"][l][n], rtol=1e-8, atol=1e-12)
        for si, s in enumerate(mo.SITES):
            np.testing.assert_allclose(b["d_ci_pre"][l][s], a["d_ci_pre"][l][s], rtol=1e-8, atol=1e-12)
            up = po.upper_leaky(ci[l][s])
            F = np.zeros((cfg.E, cfg.c))
            np.add.at(F, batch["top_idx"][l].reshape(-1), po.smooth_l0_psi(up, 0.2, True).reshape(-1, cfg.c))
            alpha, _ = po.ema_decay_terms(4.0, 5.0)
            np.testing.assert_allclose(a["freq_ema"][l, si], ema[l, si] + alpha * (F.reshape(-1) / cfg.T - ema[l, si]),
                                       rtol=1e-12)


@pytest.mark.parametrize("use_delta", [True, False])
def test_routed_moe_step_matches_the_autograd_restatement(use_delta):
    """Per-token site routes (`where(route, decomposed + d frozen, frozen)` per job,
    pd/targets/qwen36_moe.py:2822-2827): the NumPy oracle's hand-written backward equals
    torch autograd of the routed forward in float64; every route on reproduces the unrouted
    step, every route off reproduces the frozen model (recon 0, CI gradient = the imp-min
    pullback alone)."""
    cfg = mo.MoEConfig(T=48, d=16, f=8, E=6, k=2, c=4, L=2)
    rng = np.random.default_rng(23)
    params, x0, _ = mo.init_moe(cfg, rng)
    ci = [{s: rng.uniform(0.05, 0.95, size=(cfg.T, cfg.k, cfg.c)) for s in mo.SITES} for _ in range(cfg.L)]
    routes = [{s: rng.uniform(size=cfg.T) < 0.6 for s in mo.SITES} for _ in range(cfg.L)]
    kw = dict(p=2.0, imp_coeff=0.5, recon_coeff=1.5, use_delta=use_delta)
    a = mo.moe_stack_step(cfg, params, x0, ci, (3, 4), routes=routes, **kw)
    b = mo.moe_stack_step_torch(cfg, params, x0, ci, (3, 4), routes=routes, **kw)
    assert b["loss"] == pytest.approx(a["loss"], rel=1e-10)
    for l in range(cfg.L):
        for n in ("Vg", "Ug", "Vu", "Uu", "Vd", "Ud"):
            np.testing.assert_allclose(b["grads"][l][n], a["grads"][l][n], rtol=1e-8, atol=1e-12)
        for s in mo.SITES:
            np.testing.assert_allclose(b["d_ci_pre"][l][s], a["d_ci_pre"][l][s], rtol=1e-8, atol=1e-12)
    plain = mo.moe_stack_step(cfg, params, x0, ci, (3, 4), **kw)
    on = mo.moe_stack_step(cfg, params, x0, ci, (3, 4), routes=[{s: np.ones(cfg.T, bool) for s in mo.SITES}
                                                                 for _ in range(cfg.L)], **kw)
    assert on["loss"] == pytest.approx(plain["loss"], rel=1e-12)
    off = mo.moe_stack_step(cfg, params, x0, ci, (3, 4), routes=[{s: np.zeros(cfg.T, bool) for s in mo.SITES}
                                                                  for _ in range(cfg.L)], **kw)
    assert off["recon"] == pytest.approx(0.0, abs=1e-24)
    for l in range(cfg.L):
        for s in mo.SITES:
            up = po.upper_leaky(ci[l][s])
            _, _, dup = po.impmin_site_terms(up, po.ImpMin("pnorm", p=2.0, coeff=0.5), cfg.T)
            np.testing.assert_allclose(off["d_ci_pre"][l][s], po.upper_leaky_vjp(ci[l][s], dup), rtol=1e-12)


@pytest.mark.parametrize("rps", [48, 12, 1])
def test_persistent_sources_match_the_autograd_restatement(rps):
    """Persistent source tables (the `c`, `bc` and `bsc` shapes: 48, 12 and 1 tokens per
    source row): the hand-written source gradients (the scatter of dm (1 - lower) into
    each row's [E, c] table and the delta cotangent summed over each row's tokens) and
    every model gradient equal torch autograd with the tables as leaves, in float64."""
    cfg = mo.MoEConfig(T=48, d=16, f=8, E=6, k=2, c=4, L=2)
    rng = np.random.default_rng(21)
    params, x0, _ = mo.init_moe(cfg, rng)
    ci = [{s: rng.uniform(0.05, 0.95, size=(cfg.T, cfg.k, cfg.c)) for s in mo.SITES} for _ in range(cfg.L)]
    S = cfg.T // rps
    src = [{s: rng.uniform(size=(S, cfg.E, cfg.c)) for s in mo.SITES} for _ in range(cfg.L)]
    srcd = [{s: rng.uniform(size=S) for s in mo.SITES} for _ in range(cfg.L)]
    a = mo.moe_stack_step(cfg, params, x0, ci, (3, 4), p=2.0, imp_coeff=0.0, recon_coeff=1.5,
                          sources=(src, srcd, rps))
    b = mo.moe_stack_step_torch(cfg, params, x0, ci, (3, 4), p=2.0, imp_coeff=0.0, recon_coeff=1.5,
                                sources=(src, srcd, rps))
    assert b["loss"] == pytest.approx(a["loss"], rel=1e-10)
    for l in range(cfg.L):
        for n in ("Vg", "Ug", "Vu", "Uu", "Vd", "Ud"):
            np.testing.assert_allclose(b["grads"][l][n], a["grads"][l][n], rtol=1e-8, atol=1e-12)
        for s in mo.SITES:
            np.testing.assert_allclose(b["d_ci_pre"][l][s], a["d_ci_pre"][l][s], rtol=1e-8, atol=1e-12)
            np.testing.assert_allclose(b["d_src"][l][s], a["d_src"][l][s], rtol=1e-8, atol=1e-12)
            np.testing.assert_allclose(b["d_src_delta"][l][s], a["d_src_delta"][l][s], rtol=1e-8, atol=1e-12)
    # the tables were really read: a source row's gradient is nonzero only where its
    # tokens routed, and unselected experts of a bsc row stay exactly zero
    if rps == 1:
        for s in mo.SITES:
            sel = np.zeros((cfg.T, cfg.E), bool)
            for t in range(cfg.T):
                sel[t, a["top_idx"][0][t]] = True
            assert np.all(a["d_src"][0][s][~sel] == 0.0)


def test_c_restatement_matches_the_numpy_oracle():
    """The compiled fp32 C/OpenMP restatement (the CPU baseline) against the NumPy
    oracle in float64: same expert selection, losses and every gradient to fp32
    precision (CI away from the squashing kinks)."""
    from oracle import cpu

    cfg = mo.MoEConfig(T=64, d=32, f=16, E=7, k=3, c=8, L=2)
    rng = np.random.default_rng(12)
    params, x0, _ = mo.init_moe(cfg, rng)
    ci = [{s: rng.uniform(0.05, 0.95, size=(cfg.T, cfg.k, cfg.c)) for s in mo.SITES} for _ in range(cfg.L)]
    a = mo.moe_stack_step(cfg, params, x0, ci, (3, 4), p=2.0, imp_coeff=0.5, recon_coeff=1.5)
    b = cpu.moe_step(cfg, params, x0, ci, (3, 4), p=2.0, imp_coeff=0.5, recon_coeff=1.5)
    assert b["loss"] == pytest.approx(a["loss"], rel=1e-5)
    assert b["recon"] == pytest.approx(a["recon"], rel=1e-4)
    for l in range(cfg.L):
        np.testing.assert_array_equal(b["top_idx"][l], a["top_idx"][l])
        for n in ("Vg", "Ug", "Vu", "Uu", "Vd", "Ud"):
            w = a["grads"][l][n]
            np.testing.assert_allclose(b["grads"][l][n], w, rtol=2e-4, atol=2e-5 * np.abs(w).max())
        for s in mo.SITES:
            w = a["d_ci_pre"][l][s]
            np.testing.assert_allclose(b["d_ci_pre"][l][s], w, rtol=2e-4, atol=2e-5 * np.abs(w).max())
