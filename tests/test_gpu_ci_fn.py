"""GPU parity of the engine's CI functions (SiteMLP and the component-activation readout)
against the oracle (oracle/ci_fn_oracle.py) in its bf16-storage mode.

Tolerances: preactivations and data gradients within 2e-2 of the largest magnitude
(bf16 storage, one ulp is 2^-8 relative); parameter gradients by relative Frobenius error
3e-2, the bound the reference's own readout-gradient test uses
(pd/tests/core/test_ci_component_conditioning.py:389-394)."""

import numpy as np
import pytest
import torch

from oracle import ci_fn_oracle as co
from param_decomp_amd import _lib as L
from param_decomp_amd import ci_fn, ops

pytestmark = pytest.mark.gpu


def _bf(a, dev):
    return torch.tensor(np.asarray(a, np.float32), device=dev).to(torch.bfloat16)


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _maxrel(got, want):
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


def _frob(got, want):
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


MLP_CASES = [
    (300, (24, 40, 32, 16)),      # ragged tokens and K < 64
    (1024, (64, 128, 128, 64)),   # whole tiles
    (777, (136, 256, 200)),       # one hidden layer, ragged widths
    (64, (8, 8, 8)),              # smallest widths
]


@pytest.mark.parametrize("N,dims", MLP_CASES)
def test_site_mlp_matches_oracle(device, N, dims):
    print(f"site_mlp N={N} dims={dims}", flush=True)
    rng = np.random.default_rng(N + sum(dims))
    weights, biases = co.init_mlp_stack(dims, rng)
    biases = [rng.normal(size=b.shape) * 0.2 for b in biases]
    x = rng.normal(size=(N, dims[0]))
    d_pre = rng.normal(size=(N, dims[-1]))
    xb, wb, bb, gb = _bf(x, device), [_bf(w, device) for w in weights], [_bf(b, device) for b in biases], _bf(d_pre,
                                                                                                            device)
    pre, ws = ops.ci_mlp_fwd(xb, wb, bb)
    dW, db, dx = ops.ci_mlp_bwd(xb, wb, gb, ws, True)
    torch.cuda.synchronize()
    f = lambda ts: [_np(t) for t in ts]
    xr, wr, br, gr = _np(xb), f(wb), f(bb), _np(gb)
    want_pre, _, _ = co.site_mlp_fwd(xr, wr, br, bf16_storage=True)
    want_dW, want_db, want_dx = co.site_mlp_bwd(xr, wr, br, gr, bf16_storage=True)
    assert _maxrel(_np(pre), want_pre) < 2e-2
    assert _maxrel(_np(dx), want_dx) < 2e-2
    for i in range(len(dims) - 1):
        assert _frob(_np(dW[i]), want_dW[i]) < 3e-2, i
        assert _frob(_np(db[i]), want_db[i]) < 3e-2, i


def test_site_mlp_backward_is_deterministic_and_skips_dx(device):
    rng = np.random.default_rng(1)
    dims = (64, 256, 96)
    N = 5000
    weights, biases = co.init_mlp_stack(dims, rng)
    xb = _bf(rng.normal(size=(N, 64)), device)
    wb, bb = [_bf(w, device) for w in weights], [_bf(b, device) for b in biases]
    gb = _bf(rng.normal(size=(N, 96)), device)
    _, ws = ops.ci_mlp_fwd(xb, wb, bb)
    a = ops.ci_mlp_bwd(xb, wb, gb, ws, True)
    b = ops.ci_mlp_bwd(xb, wb, gb, ws, False)
    assert b[2] is None
    for u, v in zip(a[0] + a[1], b[0] + b[1]):
        assert torch.equal(u, v)


def test_site_mlp_module_autograd(device):
    gen = torch.Generator(device=device).manual_seed(0)
    mlp = ci_fn.SiteMLP((32, 64, 48), device=device, generator=gen)
    x = torch.randn(200, 32, device=device, generator=gen, requires_grad=True)
    pre = mlp(x)
    assert pre.dtype == torch.bfloat16 and pre.shape == (200, 48)
    g = torch.randn(200, 48, device=device, generator=gen)
    pre.backward(g.to(torch.bfloat16))
    wr = [_np(w.detach().to(torch.bfloat16)) for w in mlp.weights]
    br = [_np(b.detach().to(torch.bfloat16)) for b in mlp.biases]
    xr = _np(x.detach().to(torch.bfloat16))
    dW, db, dx = co.site_mlp_bwd(xr, wr, br, _np(g.to(torch.bfloat16)), bf16_storage=True)
    assert x.grad.dtype == torch.float32
    assert _maxrel(_np(x.grad), dx) < 2e-2
    for i in range(2):
        assert mlp.weights[i].grad.dtype == torch.float32
        assert _frob(_np(mlp.weights[i].grad), dW[i]) < 3e-2
        assert _frob(_np(mlp.biases[i].grad), db[i]) < 3e-2


def test_layerwise_mlp_ci_fn(device):
    gen = torch.Generator(device=device).manual_seed(3)
    fn = ci_fn.LayerwiseMLPCIFn(("in.a", "in.b"), (("a", 32, 64), ("b", 48, 128)), (64,), device=device,
                                generator=gen)
    taps = {"in.a": torch.randn(4, 10, 32, device=device, generator=gen),
            "in.b": torch.randn(4, 10, 48, device=device, generator=gen)}
    ci = fn(taps)
    assert set(ci.preactivations) == {"a", "b"}
    assert ci.lower["a"].shape == (4, 10, 64) and ci.upper["b"].shape == (4, 10, 128)
    # positions are independent: one token's preactivations do not depend on the others
    single = fn.site_preactivations({k: v[1:2, 3:4] for k, v in taps.items()})
    assert torch.equal(single["a"][0, 0], ci.preactivations["a"][1, 3])
    with pytest.raises(ValueError):
        fn.site_preactivations({"in.a": taps["in.a"]})


def test_site_mlp_rejects_bad_widths(device):
    xb = torch.zeros(16, 12, dtype=torch.bfloat16, device=device)
    w = [torch.zeros(12, 16, dtype=torch.bfloat16, device=device)]
    b = [torch.zeros(16, dtype=torch.bfloat16, device=device)]
    with pytest.raises(L.PDError, match="multiple of 8"):
        ops.ci_mlp_fwd(xb, w, b)


def _readout_case(rng, N, C):
    h = rng.normal(size=(N, C)) * 1.5
    params = np.stack([rng.uniform(0.5, 1.5, C), rng.normal(size=C) * 0.3, rng.normal(size=C),
                       rng.uniform(0.5, 1.5, C), rng.normal(size=C) * 0.3, rng.normal(size=C), rng.normal(size=C)])
    return h, params


@pytest.mark.parametrize("N,C", [(1000, 72), (256, 64), (3, 8), (4096, 512), (77, 8), (500, 20), (300, 1)])
def test_readout_matches_oracle(device, N, C):
    print(f"readout N={N} C={C}", flush=True)
    rng = np.random.default_rng(N * 7 + C)
    h, params = _readout_case(rng, N, C)
    base = rng.normal(size=(N, C))
    g = rng.normal(size=(N, C))
    hb, bb, gb = _bf(h, device), _bf(base, device), _bf(g, device)
    pt = torch.tensor(params, dtype=torch.float32, device=device)
    out = ops.ci_readout_fwd(hb, pt, bb)
    d_h, d_params = ops.ci_readout_bwd(hb, pt, gb)
    torch.cuda.synchronize()
    pr = params.astype(np.float32).astype(np.float64)
    want = co.readout_fwd(_np(hb), pr, _np(bb), bf16_storage=True)
    want_dh, want_dp = co.readout_bwd(_np(hb), pr, _np(gb), bf16_storage=True)
    assert _maxrel(_np(out), want) < 2e-2
    assert _maxrel(_np(d_h), want_dh) < 2e-2
    for k in range(7):
        assert _frob(_np(d_params[k]), want_dp[k]) < 3e-2, k
    # fixed-order sums: a second call is bit-identical
    assert torch.equal(ops.ci_readout_bwd(hb, pt, gb)[1], d_params)


def test_readout_symmetric_clamp_known_answer(device):
    # pd/tests/core/test_ci_component_conditioning.py:604-614 through the readout: the
    # positive arm with unit scale and no bias is the clamp itself, the negative arm is off
    C = 6
    params = torch.zeros(7, C, device=device)
    params[0] = 1.0
    params[2] = 1.0
    h = torch.tensor([[-0.5, 0.25, 1.5, -0.5, 0.25, 1.5]], device=device).to(torch.bfloat16)
    g = torch.tensor([[-1.0, -1.0, -1.0, 1.0, 1.0, 1.0]], device=device).to(torch.bfloat16)
    out = ops.ci_readout_fwd(h, params)
    d_h, _ = ops.ci_readout_bwd(h, params, g)
    np.testing.assert_array_equal(_np(out)[0], [0, 0.25, 1, 0, 0.25, 1])
    np.testing.assert_allclose(_np(d_h)[0], [-0.01, -1, 0, 0, 1, 0.01], rtol=1e-2)


def test_readout_module_autograd(device):
    C = 40
    ro = ci_fn.ComponentActivationReadout(C, 0.5, device=device)
    with torch.no_grad():
        ro.params[1].uniform_(-0.3, 0.3)
    h = torch.randn(3, 50, C, device=device, requires_grad=True)
    base = torch.randn(3, 50, C, device=device).to(torch.bfloat16).requires_grad_()
    y = ro(h, base)
    g = torch.randn_like(y)
    y.backward(g)
    assert torch.equal(base.grad, g)
    hr = _np(h.detach().to(torch.bfloat16)).reshape(-1, C)
    want_dh, want_dp = co.readout_bwd(hr, _np(ro.params.detach()), _np(g).reshape(-1, C), bf16_storage=True)
    assert _maxrel(_np(h.grad).reshape(-1, C), want_dh) < 2e-2
    assert _frob(_np(ro.params.grad), want_dp) < 3e-2


def test_global_mlp_ci_fn_is_one_mlp_over_the_joined_taps(device):
    gen = torch.Generator(device=device).manual_seed(4)
    fn = ci_fn.GlobalMLPCIFn((("t1", 16), ("t0", 24)), (("a", 32), ("b", 8), ("c", 24)), (48,), device=device,
                             generator=gen)
    taps = {"t0": torch.randn(70, 24, device=device, generator=gen),
            "t1": torch.randn(70, 16, device=device, generator=gen)}
    ci = fn(taps)
    joined = torch.cat([taps["t1"], taps["t0"]], dim=-1).to(torch.bfloat16)
    wr = [_np(w.detach().to(torch.bfloat16)) for w in fn.mlp.weights]
    br = [_np(b.detach().to(torch.bfloat16)) for b in fn.mlp.biases]
    want, _, _ = co.site_mlp_fwd(_np(joined), wr, br, bf16_storage=True)
    got = np.concatenate([_np(ci.preactivations[k]) for k in ("a", "b", "c")], axis=-1)
    assert _maxrel(got, want) < 2e-2
    assert ci.preactivations["b"].shape == (70, 8)
    (ci.lower["a"].float().sum() + ci.upper["c"].float().sum()).backward()
    assert all(w.grad is not None for w in fn.mlp.weights)


def test_site_mlp_pads_toy_widths_exactly(device):
    # TMS-sized layerwise CI fn (hidden 50 over 5 inputs, C=20): widths not multiples of 8
    gen = torch.Generator(device=device).manual_seed(6)
    mlp = ci_fn.SiteMLP((5, 50, 20), device=device, generator=gen)
    with torch.no_grad():
        for b in mlp.biases:
            b.normal_(0, 0.3, generator=gen)
    x = torch.randn(64, 5, device=device, generator=gen, requires_grad=True)
    pre = mlp(x)
    assert pre.shape == (64, 20)
    g = torch.randn(64, 20, device=device, generator=gen).to(torch.bfloat16)
    pre.backward(g)
    wr = [_np(w.detach().to(torch.bfloat16)) for w in mlp.weights]
    br = [_np(b.detach().to(torch.bfloat16)) for b in mlp.biases]
    xr = _np(x.detach().to(torch.bfloat16))
    want = co.site_mlp_fwd(xr, wr, br, bf16_storage=True)[0]
    dW, db, dx = co.site_mlp_bwd(xr, wr, br, _np(g), bf16_storage=True)
    assert _maxrel(_np(pre), want) < 2e-2
    assert _maxrel(_np(x.grad), dx) < 2e-2
    for i in range(2):
        assert mlp.weights[i].grad.shape == mlp.weights[i].shape
        assert _frob(_np(mlp.weights[i].grad), dW[i]) < 3e-2
        assert _frob(_np(mlp.biases[i].grad), db[i]) < 3e-2
