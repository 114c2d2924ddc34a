"""GPU parity of the EMA frequency estimator (pd/core/losses.py:425-458, 522-543) against
the oracle over three consecutive steps, threading the estimate: pd_impmin through the
host `EmaFrequency`, and the dense, MoE and LM fused steps through their step objects
(each call reads and rewrites the estimate on the device and advances its count). Every
step's losses (including the batch penalty), gradients and the new estimate are compared
with the oracle fed the oracle's own running estimate. The first observation from a zero
estimate reproduces the batch-estimate step."""

import numpy as np
import pytest
import torch

from oracle import pd_oracle as po
from oracle import threefry as tf

pytestmark = pytest.mark.gpu

HALFLIFE = 3.0


def np64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _close(got, want, rtol, floor, what, worst=None):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = max(np.abs(want).max(), 1e-30)
    err = np.abs(got - want)
    if worst is not None:
        worst.append((what, float((err / np.maximum(np.abs(want), floor * scale)).max())))
    bad = err > rtol * np.abs(want) + floor * scale
    assert not bad.any(), f"{what}: {bad.sum()}/{bad.size} off, worst {err.max():.3e} scale {scale:.3e}"


def test_impmin_ema_three_steps(device):
    """pd_impmin with the estimate (fp32 CI): activity, the penalty at f_hat, the batch
    penalty, the new estimate and the CI gradient through autograd, at rtol 1e-5."""
    from param_decomp_amd.losses import init_frequency_estimator

    rng = np.random.default_rng(2)
    sites = {"a": 24, "b": 40}
    est = init_frequency_estimator(HALFLIFE, sites, device)
    ema = {n: np.zeros(C) for n, C in sites.items()}
    # the loss act + 0.5 * penalty: the oracle's coefficients are coeff 1, freq_coeff 0.5
    spec = po.ImpMin("smooth_l0", coeff=1.0, gamma=0.3, normalize_at_one=True, freq_coeff=0.5, ref_count=128.0,
                     ema_halflife=HALFLIFE)
    worst = []
    for step in range(3):
        ci = {n: rng.uniform(0.0, 1.05, size=(96, C)) * (0.5 + 0.4 * step) for n, C in sites.items()}
        tci = {n: torch.tensor(v, dtype=torch.float32, device=device, requires_grad=True) for n, v in ci.items()}
        act, pen, est = est.evaluate_ci(tci, 0.3, 128, normalize_at_one=True)
        (act + 0.5 * pen.value).backward()
        want_a = want_f = want_b = 0.0
        for n in sites:
            up = np64(tci[n])  # the same fp32 values
            a_, f_, g_, new, fb = po.impmin_site_terms_ema(up, spec, 96, ema=ema[n], count=float(step))
            want_a, want_f, want_b = want_a + a_, want_f + f_, want_b + fb
            ema[n] = new
            _close(np64(tci[n].grad), g_, 1e-5, 1e-7, f"grad {n} step {step}", worst)
            _close(np64(est.estimate[n]), new, 1e-5, 1e-7, f"estimate {n} step {step}", worst)
        _close(float(act.detach()), want_a, 1e-5, 0.0, f"activity step {step}", worst)
        _close(float(pen.value), want_f, 1e-5, 0.0, f"penalty step {step}", worst)
        _close(float(pen.batch_value), want_b, 1e-5, 0.0, f"batch penalty step {step}", worst)
        assert est.count == step + 1
    print("worst relative error", max(worst, key=lambda w: w[1]))


def _dense_inputs(rng, T, d_in, d_out, C):
    x = rng.normal(size=(T, d_in))
    W = rng.normal(size=(d_out, d_in)) / np.sqrt(d_in)
    V = rng.normal(size=(d_in, C)) / np.sqrt(d_in)
    U = rng.normal(size=(C, d_out)) / np.sqrt(C)
    gp = po.GateParams(rng.normal(size=(C, 16)) * 1.4, np.zeros((C, 16)), rng.normal(size=(C, 16)) * 0.35,
                       np.full(C, 0.3))
    return x, W, V, U, gp


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_dense_step_ema_three_steps(device, dtype):
    from param_decomp_amd.dense_step import DenseSiteStep
    from param_decomp_amd.losses import ImpMin

    rng = np.random.default_rng(13)
    T, d_in, d_out, C = 256, 64, 96, 192
    x, W, V, U, gp = _dense_inputs(rng, T, d_in, d_out, C)
    if dtype == torch.bfloat16:
        cv = lambda a: torch.tensor(np.asarray(a, np.float32), device=device).to(torch.bfloat16)  # noqa: E731
    else:
        cv = lambda a: torch.tensor(np.asarray(a, np.float32), device=device)  # noqa: E731
    tx, tW, tV, tU = (cv(a) for a in (x, W, V, U))
    gate = tuple(torch.tensor(np.asarray(a, np.float32), device=device) for a in (gp.w_in, gp.b_in, gp.w_out,
                                                                                   gp.b_out))
    spec = po.ImpMin("smooth_l0", coeff=0.7, gamma=0.2, normalize_at_one=True, freq_coeff=0.4, ref_count=300.0,
                     ema_halflife=HALFLIFE)
    imp = ImpMin.smooth_l0(0.7, 0.2, normalize_at_one=True, frequency_coeff=0.4, reference_datapoint_count=300.0,
                           ema_halflife_steps=HALFLIFE)
    step = DenseSiteStep(T, d_in, d_out, C, dtype=dtype, device=device, recon_coeff=1.3, use_delta=True,
                         imp_min=imp)
    batch_step = DenseSiteStep(T, d_in, d_out, C, dtype=dtype, device=device, recon_coeff=1.3, use_delta=True,
                               imp_min=ImpMin.smooth_l0(0.7, 0.2, normalize_at_one=True, frequency_coeff=0.4,
                                                        reference_datapoint_count=300.0))
    gp64 = po.GateParams(*(np64(t) for t in gate))
    ema = np.zeros(C)
    bf = dtype == torch.bfloat16
    rtol, floor = (2e-2, 1e-2) if bf else (1e-5, 1e-5)  # fp32: the smooth-L0 floor of the dense parity test
    for s in range(3):
        draw_key = tf.fold_in(tf.prng_key(5), 1 + s)
        mk, dk = step.site_keys(draw_key, 0)
        g = step.step(tx, tW, tV, tU, gate, mk, dk)
        torch.cuda.synchronize()
        r = po.dense_site_step(np64(tx), np64(tW), np64(tV), np64(tU), gp64, draw_key, recon_coeff=1.3,
                               mask_dtype="bfloat16" if bf else "float32", use_delta=True, bf16_storage=bf,
                               imp_min=spec, freq_ema=ema, ema_count=float(s))
        np.testing.assert_allclose(g.losses.cpu().numpy(), [r.loss, r.recon, r.imp, r.freq, r.freq_batch],
                                   rtol=rtol, atol=1e-7)
        _close(np64(step.frequency.values), r.freq_ema, 1e-5 if not bf else rtol, 1e-6, f"estimate step {s}")
        _close(np64(g.dU), r.dU, rtol, floor, f"dU step {s}")
        _close(np64(g.dV), r.dV, rtol, floor, f"dV step {s}")
        for got, want, name in zip((g.dw_in, g.db_in, g.dw_out, g.db_out), r.dgate,
                                   ("dw_in", "db_in", "dw_out", "db_out")):
            _close(np64(got), want, rtol, floor, f"{name} step {s}")
        if s == 0:  # the first observation from a zero estimate is the batch-estimate step
            gb = batch_step.step(tx, tW, tV, tU, gate, mk, dk)
            torch.cuda.synchronize()
            torch.testing.assert_close(g.losses[:4], gb.losses, rtol=1e-6, atol=0.0)
            torch.testing.assert_close(g.dV, gb.dV, rtol=1e-5, atol=1e-6 * float(gb.dV.abs().max()))
            torch.testing.assert_close(g.db_out, gb.db_out, rtol=1e-5, atol=1e-6 * float(gb.db_out.abs().max()))
        ema = r.freq_ema
    assert step.frequency.count == 3


def test_moe_step_ema_three_steps(device):
    from routing_checks import assert_routing_matches
    from test_gpu_moe import _make

    from oracle import moe_oracle as mo
    from param_decomp_amd.losses import ImpMin
    from param_decomp_amd.moe_step import MoEStackStep

    cfg = mo.MoEConfig(T=200, d=48, f=40, E=13, k=4, c=24, L=3)
    params, x0, ci, w, ci_t, x0_t = _make(cfg, 0, device)
    spec = po.ImpMin("smooth_l0", coeff=0.5, gamma=0.3, normalize_at_one=True, freq_coeff=0.25, ref_count=4096.0,
                     ema_halflife=HALFLIFE)
    imp = ImpMin.smooth_l0(0.5, 0.3, normalize_at_one=True, frequency_coeff=0.25, reference_datapoint_count=4096.0,
                           ema_halflife_steps=HALFLIFE)
    step = MoEStackStep(cfg.T, cfg.d, cfg.f, cfg.E, cfg.k, cfg.c, cfg.L, device=device, recon_coeff=1.5, imp_min=imp)
    ema = np.zeros((cfg.L, 3, cfg.E * cfg.c))
    for s in range(3):
        key = (0, 17 + s)
        step.step(x0_t, w, ci_t, key)
        torch.cuda.synchronize()
        got_idx = step.top_idx.cpu().numpy()
        ref = mo.moe_stack_step(cfg, params, x0, ci, key, recon_coeff=1.5, bf16_storage=True, pinned_top_idx=got_idx,
                                imp_min=spec, freq_ema=ema, ema_count=float(s))
        for l in range(cfg.L):
            assert_routing_matches(got_idx[l], ref, l, cfg.k)
        np.testing.assert_allclose(step.losses.cpu().numpy(),
                                   [ref["loss"], ref["recon"], ref["imp"], ref["freq"], ref["freq_batch"]],
                                   rtol=2e-2, atol=1e-7)
        _close(np64(step.frequency.values).reshape(ema.shape), ref["freq_ema"], 2e-2, 1e-3, f"estimate step {s}")
        for l in range(cfg.L):
            for site, vn, un in (("gate", "Vg", "Ug"), ("up", "Vu", "Uu"), ("down", "Vd", "Ud")):
                _close(np64(step.dV[site][l]), ref["grads"][l][vn], 2e-2, 1e-2, f"{vn}[{l}] step {s}")
                _close(np64(step.dU[site][l]), ref["grads"][l][un], 2e-2, 1e-2, f"{un}[{l}] step {s}")
            got = np64(step.d_ci_pre[l])
            for si, site in enumerate(mo.SITES):
                _close(got[si], ref["d_ci_pre"][l][site], 2e-2, 1e-2, f"d_ci_pre[{l}][{site}] step {s}")
        ema = ref["freq_ema"]
    assert step.frequency.count == 3


def test_lm_step_ema_three_steps(device):
    from test_gpu_lm import _close as lm_close
    from test_gpu_lm import _setup

    from oracle import lm_oracle as lo
    from param_decomp_amd.lm_step import KINDS, LMStackStep
    from param_decomp_amd.losses import ImpMin

    B, T = 2, 128
    cfg = lo.LMConfig(n_layers=2, d=128, n_head=2, n_kv_head=2, d_mlp=256, vocab=384,
                      C={"q_proj": 64, "k_proj": 48, "v_proj": 64, "o_proj": 32, "c_fc": 128, "down_proj": 96})
    params, tokens, ci, w, ci_t, tok_t = _setup(cfg, B, T, 6, device)
    spec = po.ImpMin("smooth_l0", coeff=0.05, gamma=0.4, normalize_at_one=False, freq_coeff=0.02, ref_count=2048.0,
                     ema_halflife=HALFLIFE)
    imp = ImpMin.smooth_l0(0.05, 0.4, frequency_coeff=0.02, reference_datapoint_count=2048.0,
                           ema_halflife_steps=HALFLIFE)
    step = LMStackStep(B, T, cfg.d, cfg.n_head, cfg.n_kv_head, cfg.d_mlp, cfg.vocab, cfg.n_layers, cfg.C,
                       device=device, n_kl_chunks=3, recon_coeff=3.0, imp_min=imp)
    ema = [{k: np.zeros(cfg.C[k]) for k in KINDS} for _ in range(cfg.n_layers)]
    for s in range(3):
        key = (5, 23 + s)
        step.step(tok_t, w, ci_t, key)
        torch.cuda.synchronize()
        ref = lo.lm_stack_step(cfg, params, tokens, ci, key, bf16_storage=True, recon_coeff=3.0, imp_min=spec,
                               freq_ema=ema, ema_count=float(s))
        np.testing.assert_allclose(step.losses.cpu().numpy(),
                                   [ref["loss"], ref["recon"], ref["imp"], ref["freq"], ref["freq_batch"]],
                                   rtol=2e-2, atol=1e-7)
        got_ema = np64(step.frequency.values)
        off = 0
        for l in range(cfg.n_layers):  # layer-major, kinds in KIND_ORDER
            for k in KINDS:
                _close(got_ema[off:off + cfg.C[k]], ref["freq_ema"][l][k], 1e-5, 1e-6, f"estimate [{l}][{k}] step {s}")
                off += cfg.C[k]
        stats = []
        for l in range(cfg.n_layers):
            for k in KINDS:
                lm_close(np64(step.dV[k][l]), ref["dV"][l][k], f"dV[{l}][{k}] step {s}", stats)
                lm_close(np64(step.dU[k][l]), ref["dU"][l][k], f"dU[{l}][{k}] step {s}", stats)
                lm_close(np64(step.d_ci_pre[k][l]), ref["d_ci_pre"][l][k], f"d_ci_pre[{l}][{k}] step {s}", stats)
        ema = ref["freq_ema"]
    assert step.frequency.count == 3


def test_ema_arguments_are_checked(device):
    """An estimate without the frequency term, or a half-life outside (0, 1e6], is
    rejected before any launch."""
    from param_decomp_amd import _lib as L
    from param_decomp_amd import ops

    ci = torch.rand(16, 8, device=device)
    ema = torch.zeros(8, device=device)
    with pytest.raises(L.PDError, match="frequency term"):
        ops.impmin(ci, kind=L.IMPMIN_SMOOTH_L0, ref_count=0.0, ema=ema, ema_halflife=4.0)
    with pytest.raises(L.PDError, match="half-life"):
        ops.impmin(ci, kind=L.IMPMIN_SMOOTH_L0, ref_count=8.0, ema=ema, ema_halflife=2e6)
    with pytest.raises(L.PDError, match="needs freq_ema_in"):
        ops.impmin(ci, kind=L.IMPMIN_SMOOTH_L0, ref_count=8.0, ema_out=ema, ema_halflife=4.0)
