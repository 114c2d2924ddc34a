"""GPU parity of the toy decomposition steps (TMS 5-2, ResidMLP-1L) against the float64
toy oracle fed the same fp32 values.

Tolerance: losses rtol 1e-5; outputs and gradients rtol 1e-5 with an absolute floor of
1e-6 x max|oracle|: fp32 GEMMs and batch reductions over 2048-4096 rows against float64
round at about 1e-7 of the largest magnitude (measured need at rtol 1e-5: at most 1.2e-7).
Each comparison prints the floor it needed."""

import numpy as np
import pytest
import torch

from oracle import pd_oracle as po
from oracle import toy_oracle as to

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().double().cpu().numpy()


def _close(got, want, rtol, floor, what):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = max(np.abs(want).max(), 1e-30)
    err = np.abs(got - want)
    need = max(0.0, float(((err - 1e-5 * np.abs(want)) / scale).max()))
    print(f"[fp32] {what}: floor needed at rtol 1e-5 {need:.2e}")
    bad = err > rtol * np.abs(want) + floor * scale
    assert not bad.any(), f"{what}: {bad.sum()}/{bad.size} off, worst {np.abs(got - want).max():.3e} (scale {scale:.3e})"


def _vary_gates(sites, g):
    """Spread the gates' operating points over both squashing kinks."""
    with torch.no_grad():
        for s in sites:
            s.gate.b_in.copy_(torch.randn(s.gate.b_in.shape, device=s.V.device, generator=g) * 0.5)
            s.gate.b_out.copy_(torch.randn(s.gate.b_out.shape, device=s.V.device, generator=g) * 0.4 + 0.3)


def _oracle_sites(sites):
    return [to.ToySite(s.name, _np(s.W), _np(s.V), _np(s.U),
                       po.GateParams(_np(s.gate.w_in), _np(s.gate.b_in), _np(s.gate.w_out), _np(s.gate.b_out)))
            for s in sites]


def _compare(res, sites, want):
    for k in ("loss", "recon", "imp"):
        assert float(res[k]) == pytest.approx(want[k], rel=1e-5), k
    _close(_np(res["out"]), want["out"], 1e-5, 1e-6, "masked output")
    for i, s in enumerate(sites):
        _close(_np(s.V.grad), want["dV"][i], 1e-5, 1e-6, f"{s.name} dV")
        _close(_np(s.U.grad), want["dU"][i], 1e-5, 1e-6, f"{s.name} dU")
        for prm, w, nm in zip((s.gate.w_in, s.gate.b_in, s.gate.w_out, s.gate.b_out), want["dgate"][i],
                              ("w_in", "b_in", "w_out", "b_out")):
            _close(_np(prm.grad), w, 1e-5, 1e-6, f"{s.name} gate {nm}")


@pytest.mark.parametrize("use_delta,routed", [(False, False), (True, False), (True, True)])
def test_tms_5_2_step_matches_oracle(device, use_delta, routed):
    from param_decomp_amd import toys
    from param_decomp_amd.routing import UniformKRouting

    g = torch.Generator(device=device).manual_seed(0)
    target, sites = toys.init_tms(5, 2, 20, device=device, generator=g)
    with torch.no_grad():
        target.b2.copy_(torch.randn(5, device=device, generator=g) * 0.1)
    _vary_gates(sites, g)
    x = toys.sparse_features(4096, 5, 0.05, 0.0, device=device, generator=g)
    key = (0, 2024)
    routes = None
    if routed:
        r = UniformKRouting(tuple(s.name for s in sites), device)((7, 8), (4096,))
        routes = [r[s.name] for s in sites]
    step = toys.ToyDecompositionStep(target, sites, p=1.0, imp_coeff=0.3, recon_coeff=1.0, use_delta=use_delta)
    res = step.step(x, key, routes)
    torch.cuda.synchronize()
    want = to.toy_step("tms", {"W1": _np(target.W1), "b2": _np(target.b2)}, _oracle_sites(sites), _np(x), key, p=1.0,
                       imp_coeff=0.3, recon_coeff=1.0, use_delta=use_delta,
                       routes=None if routes is None else [r.cpu().numpy() for r in routes])
    _compare(res, sites, want)


@pytest.mark.parametrize("use_delta,routed,B", [(False, False, 4096), (True, False, 4096), (True, True, 4096),
                                                (False, False, 1000)])
def test_tms_fused_step_matches_oracle(device, use_delta, routed, B):
    """The one-launch TMS step (pd_tms_step) against the same oracle, incl. a batch that
    is not a multiple of the 64-row wave; then bit-identical on a second call."""
    from param_decomp_amd import toys
    from param_decomp_amd.routing import UniformKRouting

    g = torch.Generator(device=device).manual_seed(0)
    target, sites = toys.init_tms(5, 2, 20, device=device, generator=g)
    with torch.no_grad():
        target.b2.copy_(torch.randn(5, device=device, generator=g) * 0.1)
    _vary_gates(sites, g)
    x = toys.sparse_features(B, 5, 0.05, 0.0, device=device, generator=g)
    key = (0, 2024)
    routes = None
    if routed:
        r = UniformKRouting(tuple(s.name for s in sites), device)((7, 8), (B,))
        routes = [r[s.name] for s in sites]
    step = toys.TMSFusedStep(target, sites, p=1.0, imp_coeff=0.3, recon_coeff=1.0, use_delta=use_delta)
    res = step.step(x, key, routes)
    torch.cuda.synchronize()
    want = to.toy_step("tms", {"W1": _np(target.W1), "b2": _np(target.b2)}, _oracle_sites(sites), _np(x), key, p=1.0,
                       imp_coeff=0.3, recon_coeff=1.0, use_delta=use_delta,
                       routes=None if routes is None else [r.cpu().numpy() for r in routes])
    for k in ("loss", "recon", "imp"):
        assert float(res[k]) == pytest.approx(want[k], rel=1e-5), k
    for i, s in enumerate(sites):
        _close(_np(s.V.grad), want["dV"][i], 1e-5, 1e-6, f"{s.name} dV")
        _close(_np(s.U.grad), want["dU"][i], 1e-5, 1e-6, f"{s.name} dU")
        for prm, w, nm in zip((s.gate.w_in, s.gate.b_in, s.gate.w_out, s.gate.b_out), want["dgate"][i],
                              ("w_in", "b_in", "w_out", "b_out")):
            _close(_np(prm.grad), w, 1e-5, 1e-6, f"{s.name} gate {nm}")
    flat = step.flat.clone()
    step.step(x, key, routes)
    torch.cuda.synchronize()
    assert torch.equal(step.flat, flat)


@pytest.mark.parametrize("use_delta", [False, True])
def test_resid_mlp_1l_step_matches_oracle(device, use_delta):
    from param_decomp_amd import toys

    g = torch.Generator(device=device).manual_seed(1)
    target, sites = toys.init_resid_mlp(100, 1000, 50, 1, 100, device=device, generator=g)
    _vary_gates(sites, g)
    x = toys.sparse_features(2048, 100, 0.01, -1.0, device=device, generator=g)
    key = (5, 6)
    step = toys.ToyDecompositionStep(target, sites, p=2.0, imp_coeff=0.1, recon_coeff=1.0, use_delta=use_delta)
    res = step.step(x, key)
    torch.cuda.synchronize()
    tgt = {"W_E": _np(target.W_E), "W_U": _np(target.W_U), "layers": [{"b_in": None, "b_out": None}]}
    want = to.toy_step("resid_mlp", tgt, _oracle_sites(sites), _np(x), key, p=2.0, imp_coeff=0.1, recon_coeff=1.0,
                       use_delta=use_delta)
    _compare(res, sites, want)


@pytest.mark.parametrize("n_layers,B", [(1, 2048), (2, 1003)])
def test_resid_mlp_fused_step_matches_oracle(device, n_layers, B):
    """The native ResidMLP step (pd_resid_mlp_step) against the same oracle: the benchmark
    shape, and two layers (the second mlp_in's masked input differs from its clean gate
    input, and the residual cotangent flows through the first layer) with a batch that is
    not a multiple of the site passes' 8-row chunks; then bit-identical on a second call."""
    from param_decomp_amd import toys

    g = torch.Generator(device=device).manual_seed(1)
    target, sites = toys.init_resid_mlp(100, 1000, 50, n_layers, 100, device=device, generator=g)
    _vary_gates(sites, g)
    x = toys.sparse_features(B, 100, 0.01, -1.0, device=device, generator=g)
    key = (5, 6)
    step = toys.ResidMLPFusedStep(target, sites, p=2.0, imp_coeff=0.1, recon_coeff=1.0)
    res = step.step(x, key)
    torch.cuda.synchronize()
    tgt = {"W_E": _np(target.W_E), "W_U": _np(target.W_U), "layers": [{"b_in": None, "b_out": None}] * n_layers}
    want = to.toy_step("resid_mlp", tgt, _oracle_sites(sites), _np(x), key, p=2.0, imp_coeff=0.1, recon_coeff=1.0)
    _compare(res, sites, want)
    flat, out = step.flat.clone(), res["out"].clone()
    res = step.step(x, key)
    torch.cuda.synchronize()
    assert torch.equal(step.flat, flat) and torch.equal(res["out"], out)


def test_resid_mlp_graphed_step_matches_eager(device):
    """The ResidMLP-1L step captured into a HIP graph (mask keys read from a device buffer
    the host rewrites before each replay) against the eager step with the same draw keys:
    losses, output and every gradient bit-identical on each of four replays, with eager
    steps run between the replays, and a batch change between replays picked up."""
    from param_decomp_amd import prng, toys

    g = torch.Generator(device=device).manual_seed(5)
    target, sites = toys.init_resid_mlp(100, 1000, 50, 1, 100, device=device, generator=g)
    _vary_gates(sites, g)
    xs = [toys.sparse_features(2048, 100, 0.01, -1.0, device=device, generator=g) for _ in range(2)]
    eager = toys.ToyDecompositionStep(target, sites, p=2.0)
    graphed = toys.GraphedToyStep(toys.ToyDecompositionStep(target, sites, p=2.0), xs[0])
    params = [prm for s in sites for prm in s.parameters()]
    outs = []
    for i in range(4):
        key, x = prng.fold_in((0, 7), i), xs[i // 2]
        res = graphed.step(x, key)
        got = {k: res[k].clone() for k in ("loss", "recon", "imp", "out")}
        got_grads = [prm.grad.clone() for prm in params]
        want = eager.step(x, key)
        torch.cuda.synchronize()
        for k in got:
            assert torch.equal(got[k], want[k]), f"replay {i}: {k}"
        for prm, gg in zip(params, got_grads):
            assert torch.equal(gg, prm.grad), f"replay {i}: a gradient differs"
        outs.append(got["out"])
    for i in range(3):  # each replay drew its own masks
        assert not torch.equal(outs[i], outs[i + 1])
