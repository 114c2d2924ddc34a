"""GPU parity of the fused MoE stack step against the MoE oracle (same bf16 storage
points): routing bit-exact up to bf16 near-ties of the router products, losses and
every gradient within rtol 2e-2 on the same routing."""

import numpy as np
import pytest
import torch

from oracle import moe_oracle as mo
from oracle import pd_oracle as po
from routing_checks import assert_routing_matches

pytestmark = pytest.mark.gpu


def _close(got, want, rtol, floor, what):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = max(np.abs(want).max(), 1e-30)
    bad = np.abs(got - want) > rtol * np.abs(want) + floor * scale
    assert not bad.any(), f"{what}: {bad.sum()}/{bad.size} off, worst {np.abs(got - want).max():.3e} scale {scale:.3e}"


def _make(cfg, seed, device):
    rng = np.random.default_rng(seed)
    params, x0, ci = mo.init_moe(cfg, rng)
    rb = po.round_bf16
    params = [{k: (v.astype(np.float32).astype(np.float64) if k == "ln" else rb(v)) for k, v in P.items()}
              for P in params]
    x0 = rb(x0)
    ci = [{s: rb(v) for s, v in layer.items()} for layer in ci]
    from param_decomp_amd.moe_step import MoEWeights

    def stack(name, dt=torch.bfloat16):
        return torch.tensor(np.stack([P[name] for P in params]).astype(np.float32), device=device).to(dt)

    w = MoEWeights(ln=stack("ln", torch.float32), router=stack("router"), Wg=stack("Wg"), Wu=stack("Wu"),
                   Wd=stack("Wd"), Vg=stack("Vg"), Ug=stack("Ug"), Vu=stack("Vu"), Uu=stack("Uu"), Vd=stack("Vd"),
                   Ud=stack("Ud"))
    ci_t = torch.tensor(np.stack([np.stack([layer[s] for s in mo.SITES]) for layer in ci]).astype(np.float32),
                        device=device).to(torch.bfloat16)
    x0_t = torch.tensor(x0.astype(np.float32), device=device).to(torch.bfloat16)
    return params, x0, ci, w, ci_t, x0_t


# the engine's smooth-L0 imp-min with its frequency penalty (per-expert component frequencies)
SL0 = dict(kind="smooth_l0", coeff=0.5, gamma=0.3, normalize_at_one=True, freq_coeff=0.25, ref_count=4096.0)


@pytest.mark.parametrize("cfg,partitionable,use_delta,source_value,sl0", [
    (mo.MoEConfig(T=256, d=64, f=32, E=8, k=2, c=16, L=2), True, True, None, None),
    (mo.MoEConfig(T=128, d=32, f=24, E=6, k=2, c=16, L=1), True, True, None, None),  # no clean layer on the helper stream
    (mo.MoEConfig(T=200, d=48, f=40, E=13, k=4, c=24, L=3), True, True, None, None),
    (mo.MoEConfig(T=120, d=32, f=24, E=6, k=3, c=40, L=2), False, True, None, None),
    (mo.MoEConfig(T=256, d=64, f=32, E=8, k=2, c=16, L=2), True, False, None, None),
    (mo.MoEConfig(T=200, d=48, f=40, E=13, k=4, c=24, L=3), False, False, None, None),
    (mo.MoEConfig(T=200, d=48, f=40, E=13, k=4, c=24, L=3), True, True, 0.0, None),
    (mo.MoEConfig(T=256, d=64, f=32, E=8, k=2, c=16, L=2), True, True, 0.375, None),
    (mo.MoEConfig(T=200, d=48, f=40, E=13, k=4, c=24, L=3), True, True, None, SL0),
    (mo.MoEConfig(T=256, d=64, f=32, E=8, k=2, c=72, L=2), False, True, None, dict(SL0, ref_count=0.0,
                                                                                 normalize_at_one=False)),
    # more than 64 experts: several experts per lane in the router, pinned-weight and
    # token-backward kernels; the grouped products' group scan in 64-expert steps
    (mo.MoEConfig(T=256, d=64, f=32, E=100, k=6, c=16, L=2), True, True, None, None),
    (mo.MoEConfig(T=192, d=32, f=16, E=300, k=8, c=8, L=2), True, True, None, SL0)])
def test_moe_stack_step_matches_oracle(device, cfg, partitionable, use_delta, source_value, sl0):
    """sl0: the smooth-L0 term (per (tile, expert) column sums of psi in the mask pass,
    per-expert frequencies and slopes in between, the slope in the mask backward)."""
    from param_decomp_amd import _lib as L
    from param_decomp_amd.losses import ImpMin
    from param_decomp_amd.moe_step import MoEStackStep

    params, x0, ci, w, ci_t, x0_t = _make(cfg, 0, device)
    key = (0, 17)
    spec = po.ImpMin(**sl0) if sl0 else po.ImpMin("pnorm", p=2.0, coeff=0.5)
    imp = ImpMin(spec.kind, spec.p, spec.coeff, spec.gamma, spec.normalize_at_one, spec.freq_coeff, spec.ref_count)
    step = MoEStackStep(cfg.T, cfg.d, cfg.f, cfg.E, cfg.k, cfg.c, cfg.L, device=device, recon_coeff=1.5,
                        layout=L.LAYOUT_PARTITIONABLE if partitionable else L.LAYOUT_ORIGINAL,
                        use_delta=use_delta, source_value=-1.0 if source_value is None else source_value, imp_min=imp)
    step.step(x0_t, w, ci_t, key)
    torch.cuda.synchronize()
    got_idx = step.top_idx.cpu().numpy()
    ref = mo.moe_stack_step(cfg, params, x0, ci, key, recon_coeff=1.5, bf16_storage=True,
                            partitionable=partitionable, use_delta=use_delta, source_value=source_value,
                            pinned_top_idx=got_idx, imp_min=spec)
    for l in range(cfg.L):
        assert_routing_matches(got_idx[l], ref, l, cfg.k)
    losses = step.losses.cpu().numpy()
    np.testing.assert_allclose(losses, [ref["loss"], ref["recon"], ref["imp"], ref["freq"]], rtol=2e-2, atol=1e-7)
    for l in range(cfg.L):
        for s, vn, un in (("gate", "Vg", "Ug"), ("up", "Vu", "Uu"), ("down", "Vd", "Ud")):
            _close(step.dV[s][l].cpu().numpy(), ref["grads"][l][vn], 2e-2, 1e-2, f"{vn}[{l}]")
            _close(step.dU[s][l].cpu().numpy(), ref["grads"][l][un], 2e-2, 1e-2, f"{un}[{l}]")
        got = step.d_ci_pre[l].float().cpu().numpy()
        for si, s in enumerate(mo.SITES):
            _close(got[si], ref["d_ci_pre"][l][s], 2e-2, 1e-2, f"d_ci_pre[{l}][{s}]")


@pytest.mark.parametrize("use_delta", [True, False])
def test_moe_stack_step_with_routes_matches_oracle(device, use_delta):
    """Per-token site routes from the uniform-k-subset sampler (pd/core/recon.py:218-231)
    over the stack's 3L sites (site = layer * 3 + kind): an unrouted token's jobs take the
    frozen output at that site (pd/targets/qwen36_moe.py:2822-2827), also without the
    delta draws (the frozen channel then runs for the routes alone)."""
    from param_decomp_amd import ops
    from param_decomp_amd.moe_step import MoEStackStep

    cfg = mo.MoEConfig(T=200, d=48, f=40, E=13, k=4, c=24, L=3)
    params, x0, ci, w, ci_t, x0_t = _make(cfg, 2, device)
    key = (0, 31)
    rt = ops.route_uniform_k((5, 6), 3 * cfg.L, cfg.T, device).reshape(cfg.L, 3, cfg.T)
    assert 0.2 < float(rt.float().mean()) < 0.9
    step = MoEStackStep(cfg.T, cfg.d, cfg.f, cfg.E, cfg.k, cfg.c, cfg.L, device=device, recon_coeff=1.5, p=2.0,
                        imp_coeff=0.5, use_delta=use_delta)
    step.step(x0_t, w, ci_t, key, routes=rt)
    torch.cuda.synchronize()
    got_idx = step.top_idx.cpu().numpy()
    rnp = rt.cpu().numpy().astype(bool)
    ref = mo.moe_stack_step(cfg, params, x0, ci, key, p=2.0, imp_coeff=0.5, recon_coeff=1.5, bf16_storage=True,
                            use_delta=use_delta, pinned_top_idx=got_idx,
                            routes=[{s: rnp[l, i] for i, s in enumerate(mo.SITES)} for l in range(cfg.L)])
    for l in range(cfg.L):
        assert_routing_matches(got_idx[l], ref, l, cfg.k)
    np.testing.assert_allclose(step.losses.cpu().numpy(), [ref["loss"], ref["recon"], ref["imp"], ref["freq"]],
                               rtol=2e-2, atol=1e-7)
    for l in range(cfg.L):
        for s, vn, un in (("gate", "Vg", "Ug"), ("up", "Vu", "Uu"), ("down", "Vd", "Ud")):
            _close(step.dV[s][l].cpu().numpy(), ref["grads"][l][vn], 2e-2, 1e-2, f"{vn}[{l}]")
            _close(step.dU[s][l].cpu().numpy(), ref["grads"][l][un], 2e-2, 1e-2, f"{un}[{l}]")
        got = step.d_ci_pre[l].float().cpu().numpy()
        for si, s in enumerate(mo.SITES):
            _close(got[si], ref["d_ci_pre"][l][s], 2e-2, 1e-2, f"d_ci_pre[{l}][{s}]")
    # every route on is the unrouted step, bit for bit
    ones = torch.ones_like(rt)
    step.step(x0_t, w, ci_t, key, routes=ones)
    l1, d1 = step.losses.clone(), step.dV["down"].clone()
    step.step(x0_t, w, ci_t, key)
    if use_delta:  # without the delta draws the routed call also runs the frozen channel (d = 0 blend)
        assert torch.equal(step.losses, l1) and torch.equal(step.dV["down"], d1)
    else:
        torch.testing.assert_close(step.losses, l1, rtol=1e-6, atol=0.0)


def test_moe_stack_step_full_size_properties(device):
    """The Qwen3.5-MoE-shaped stack (T=8192, width 512, 42 experts top-8, SwiGLU
    512->256->512, c=512 per expert, 4 layers): finite losses, deterministic run to
    run (also when calls with other inputs are queued back to back), and every expert's
    bucket size equals its routed job count (the per-layer routing is a permutation: all
    T*k jobs land)."""
    from param_decomp_amd.moe_step import MoEStackStep, MoEWeights

    T, d, f, E, k, c, Ln = 8192, 512, 256, 42, 8, 512, 4
    g = torch.Generator(device=device).manual_seed(0)

    def rn(*shape, scale):
        return (torch.randn(*shape, device=device, generator=g) * scale).to(torch.bfloat16)

    w = MoEWeights(ln=torch.zeros(Ln, d, device=device), router=rn(Ln, E, d, scale=d**-0.5),
                   Wg=rn(Ln, E, d, f, scale=d**-0.5), Wu=rn(Ln, E, d, f, scale=d**-0.5),
                   Wd=rn(Ln, E, f, d, scale=f**-0.5), Vg=rn(Ln, E, d, c, scale=d**-0.5),
                   Ug=rn(Ln, E, c, f, scale=(E * c)**-0.5), Vu=rn(Ln, E, d, c, scale=d**-0.5),
                   Uu=rn(Ln, E, c, f, scale=(E * c)**-0.5), Vd=rn(Ln, E, f, c, scale=f**-0.5),
                   Ud=rn(Ln, E, c, d, scale=(E * c)**-0.5))
    x0 = rn(T, d, scale=1.0)
    ci = (torch.rand(Ln, 3, T, k, c, device=device, generator=g) * 1.6 - 0.3).to(torch.bfloat16)
    step = MoEStackStep(T, d, f, E, k, c, Ln, device=device)
    step.step(x0, w, ci, (0, 1))
    l1 = step.losses.clone()
    dv1 = step.dV["down"].clone()
    dci1 = step.d_ci_pre.clone()
    step.step(x0, w, ci, (0, 1))
    assert torch.isfinite(l1).all() and float(l1[1]) > 0 and float(l1[2]) > 0
    assert torch.equal(step.losses, l1) and torch.equal(step.dV["down"], dv1) and torch.equal(step.d_ci_pre, dci1)
    # back to back with another input and no host synchronization in between: the helper
    # stream's work of one call must neither see the other call's buffers nor be seen by it
    x1 = rn(T, d, scale=1.0)
    step.step(x1, w, ci, (0, 2))
    lb, dvb, dcib = step.losses.clone(), step.dV["down"].clone(), step.d_ci_pre.clone()
    step.step(x0, w, ci, (0, 1))
    la, dva, dcia = step.losses.clone(), step.dV["down"].clone(), step.d_ci_pre.clone()
    torch.cuda.synchronize()
    assert torch.equal(la, l1) and torch.equal(dva, dv1) and torch.equal(dcia, dci1)
    step.step(x1, w, ci, (0, 2))
    torch.cuda.synchronize()
    assert torch.equal(step.losses, lb) and torch.equal(step.dV["down"], dvb) and torch.equal(step.d_ci_pre, dcib)
    assert not torch.equal(lb, l1)
    step.step(x0, w, ci, (0, 1))
    for l in range(Ln):
        counts = torch.bincount(step.top_idx[l].reshape(-1).long(), minlength=E)
        assert int(counts.sum()) == T * k
        # each token's k experts are distinct
        srt, _ = torch.sort(step.top_idx[l], dim=-1)
        assert bool((srt[:, 1:] != srt[:, :-1]).all())
