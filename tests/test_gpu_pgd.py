"""GPU parity of adversarial sources (pd_source_mask_fwd/bwd, pd_source_ascend) and of the
dense-site persistent-PGD step against the oracle (oracle/pgd_oracle.py).

Tolerances: fp32 paths within 1e-5 of the float64 oracle (relative to the largest
magnitude); bf16 masks within one bf16 ulp; uint16 stores bit-exact except where the fp32
sum val + lr*g lands within an ulp of a rounding threshold (at most 0.1% of elements,
off by one count)."""

import numpy as np
import pytest
import torch

from oracle import pd_oracle as pdo
from oracle import pgd_oracle as po
from oracle import threefry
from param_decomp_amd import _lib as L
from param_decomp_amd import adversary as A
from param_decomp_amd import ops

pytestmark = pytest.mark.gpu

SRC_DT = {"float32": torch.float32, "bfloat16": torch.bfloat16, "uint16": torch.uint16}


def _np(t):
    if t.dtype == torch.uint16:
        return t.to(torch.int32).cpu().numpy()
    return t.detach().float().cpu().numpy().astype(np.float64)


def _rel(got, want):
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


def _sources(rng, n, C, sdt, device):
    v = rng.uniform(size=(n, C)).astype(np.float32)
    if sdt == "uint16":
        return torch.tensor(np.round(v * 65535).astype(np.int32), device=device).to(torch.uint16)
    return torch.tensor(v, device=device).to(SRC_DT[sdt])


@pytest.mark.parametrize("sdt", ["float32", "bfloat16", "uint16"])
@pytest.mark.parametrize("cdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,C,rps", [(256, 72, 1), (256, 72, 64), (300, 40, 300), (400, 300, 100)])
def test_source_mask_matches_oracle(device, sdt, cdt, rows, C, rps):
    print(f"source_mask {sdt} {cdt} rows={rows} C={C} rps={rps}", flush=True)
    rng = np.random.default_rng(rows + C + rps)
    ci = torch.tensor(rng.uniform(size=(rows, C)).astype(np.float32), device=device).to(cdt)
    src = _sources(rng, rows // rps, C, sdt, device)
    g = torch.tensor(rng.normal(size=(rows, C)).astype(np.float32), device=device).to(cdt)
    m = ops.source_mask_fwd(ci, src, rps)
    d_src, d_ci = ops.source_mask_bwd(g, ci, src, rps, want_dci=True)
    torch.cuda.synchronize()
    view = po.source_view(_np(src), sdt)
    bf = cdt == torch.bfloat16
    want = po.source_mask(_np(ci), view, rps, bf16=bf)
    assert np.abs(_np(m) - want).max() <= (2 ** -8 if bf else 1e-6)
    s_in_frame = po.round_bf16(view) if bf else view
    want_src, want_ci = po.source_mask_vjp(_np(g), _np(ci), s_in_frame, rps)
    assert _rel(_np(d_src), want_src) < (1e-5 if not bf else 1e-4)
    assert _rel(_np(d_ci), want_ci) < (1e-6 if not bf else 2 ** -8)
    # fixed-order reduction: bit-identical on a second call
    assert torch.equal(ops.source_mask_bwd(g, ci, src, rps)[0], d_src)


def test_source_ascents_fp32_match_oracle(device):
    rng = np.random.default_rng(3)
    n = 5000
    vals = rng.uniform(size=n).astype(np.float32)
    g = (rng.normal(size=n) * 0.5).astype(np.float32)
    gt = torch.tensor(g, device=device)
    f = lambda a: torch.tensor(a, device=device)
    # SGD
    s = f(vals.copy())
    ops.source_ascend(L.PGD_SGD, s, gt, lr=0.05)
    assert _rel(_np(s), po.sgd(vals, g, 0.05)) < 1e-6
    # momentum, two steps
    s, vel = f(vals.copy()), torch.zeros(n, device=device)
    ops.source_ascend(L.PGD_MOMENTUM, s, gt, vel, lr=0.05, momentum=0.7)
    ops.source_ascend(L.PGD_MOMENTUM, s, gt, vel, lr=0.05, momentum=0.7)
    w1, v1 = po.momentum_sgd(vals.astype(np.float64), g, np.zeros(n), 0.05, 0.7)
    w2, v2 = po.momentum_sgd(w1, g, v1, 0.05, 0.7)
    assert _rel(_np(s), w2) < 1e-6 and _rel(_np(vel), v2) < 1e-6
    # Adam, two steps
    s, m, v = f(vals.copy()), torch.zeros(n, device=device), torch.zeros(n, device=device)
    for step in (1.0, 2.0):
        ops.source_ascend(L.PGD_ADAM, s, gt, m, v, step_count=step, lr=0.01)
    w, mm, vv = vals.astype(np.float64), np.zeros(n), np.zeros(n)
    for step in (1.0, 2.0):
        w, mm, vv = po.adam(w, g, mm, vv, step, lr=0.01)
    assert _rel(_np(s), w) < 1e-5 and _rel(_np(m), mm) < 1e-5 and _rel(_np(v), vv) < 1e-5
    # fresh-PGD sign step
    s = f(vals.copy())
    A.fresh_pgd_ascend(s, gt, 0.1)
    assert _rel(_np(s), po.sign_ascent(vals, g, 0.1)) < 1e-6


def test_source_ascents_bf16_storage(device):
    rng = np.random.default_rng(4)
    n = 3000
    vals = po.round_bf16(rng.uniform(size=n))
    g = rng.normal(size=n) * 0.3
    s = torch.tensor(vals, dtype=torch.float32, device=device).to(torch.bfloat16)
    m, v = torch.zeros_like(s), torch.zeros_like(s)
    ops.source_ascend(L.PGD_ADAM, s, torch.tensor(g, dtype=torch.float32, device=device), m, v, step_count=1.0, lr=0.01)
    want, _, _ = po.adam(vals, po.round_bf16(g), 0, 0, 1.0, lr=0.01)
    assert np.abs(_np(s) - want).max() <= 2 ** -8  # one bf16 ulp on [0, 1]
    vel = torch.zeros(n, dtype=torch.bfloat16, device=device)
    s2 = torch.tensor(vals, dtype=torch.float32, device=device).to(torch.bfloat16)
    ops.source_ascend(L.PGD_MOMENTUM, s2, torch.tensor(g, dtype=torch.float32, device=device), vel, lr=0.05,
                      momentum=0.9)
    want2, _ = po.momentum_sgd(vals, po.round_bf16(g), 0, 0.05, 0.9)
    assert np.abs(_np(s2) - want2).max() <= 2 ** -8


def test_adam_bf16_moments_over_several_steps(device):
    """bf16 sources and moments over four steps from nonzero moments, against the
    oracle's bf16 Adam (coefficients at the moment dtype: bf16(0.999) = 1, so v does not
    decay; a one-step test from zero moments cannot tell this from fp32 coefficients)."""
    rng = np.random.default_rng(6)
    n = 5000
    vals = po.round_bf16(rng.uniform(0.2, 0.8, size=n))
    m0 = po.round_bf16(rng.normal(size=n) * 0.05)
    v0 = po.round_bf16(rng.uniform(0.0, 0.01, size=n))
    bf = lambda a: torch.tensor(np.asarray(a, np.float32), device=device).to(torch.bfloat16)  # noqa: E731
    s, m, v = bf(vals), bf(m0), bf(v0)
    w, mm, vv = vals, m0, v0
    for step in (3.0, 4.0, 5.0, 6.0):
        g = rng.normal(size=n) * 0.3
        ops.source_ascend(L.PGD_ADAM, s, torch.tensor(g, dtype=torch.float32, device=device), m, v,
                          step_count=step, lr=0.01)
        w, mm, vv = po.adam_bf16(w, g, mm, vv, step, lr=0.01)
    assert np.abs(_np(m) - mm).max() <= 1e-6 * np.abs(mm).max() + 1e-30
    assert np.abs(_np(v) - vv).max() <= 1e-6 * np.abs(vv).max()
    assert np.abs(_np(s) - w).max() <= 2 ** -8  # one bf16 ulp on [0, 1]
    # the fp32-coefficient spelling would have decayed v: it is measurably different
    _, _, v_f32 = po.adam(vals, po.round_bf16(g), m0, v0, 3.0, lr=0.01)
    assert np.abs(v_f32 - po.adam_bf16(vals, g, m0, v0, 3.0, lr=0.01)[2]).max() > 1e-6


@pytest.mark.parametrize("opt", [L.PGD_SGD, L.PGD_MOMENTUM])
def test_uint16_storage_rounds_stochastically_with_the_leaf_key(device, opt):
    rng = np.random.default_rng(5)
    n = 20000
    u = rng.integers(0, 65536, size=n).astype(np.int64)
    g = (rng.normal(size=n) * 1e-4).astype(np.float32)
    key = (123, 456)
    s = torch.tensor(u.astype(np.int32), device=device).to(torch.uint16)
    vel = torch.zeros(n, dtype=torch.bfloat16, device=device) if opt == L.PGD_MOMENTUM else None
    ops.source_ascend(opt, s, torch.tensor(g, device=device), vel, lr=0.5, momentum=0.0, key=key)
    view = (u.astype(np.float32) / np.float32(65535.0)).astype(np.float32)
    step = g if opt == L.PGD_SGD else po.round_bf16(g).astype(np.float32)
    new = np.clip(view + np.float32(0.5) * step, 0, 1).astype(np.float32)
    want = po.quantize_stochastic(new, key).astype(np.int64)
    got = _np(s).astype(np.int64)
    diff = np.abs(got - want)
    assert diff.max() <= 1 and (diff > 0).mean() <= 1e-3
    # unbiased: the mean of the stored values tracks the fp32 target
    assert abs((got / 65535.0 - new).mean()) < 2e-6


def test_adam_refuses_uint16_storage(device):
    s = torch.zeros(8, dtype=torch.uint16, device=device)
    with pytest.raises(L.PDError, match="uint16"):
        ops.source_ascend(L.PGD_ADAM, s, torch.zeros(8, device=device), s, s, step_count=1.0)
    with pytest.raises(ValueError):
        A.PersistentAdversary(s.reshape(1, 8), A.AdamPGDConfig(), 2, 4)


def _oracle_step(x, V, U, ci, target, src, rps, n_warmup, lr, W=None, dsrc=None):
    """float64 persistent-PGD step with Adam (fp32 storage): warmups then the final. With
    delta sources (dsrc [n_sources, 1]) the site output is (xV (m - d)) @ U + d (x @ W^T)
    and the delta leaf ascends beside the components."""

    def recon(s, sd):
        m = po.source_mask(ci, s, rps)
        xV = x @ V
        d = np.zeros(x.shape[0]) if sd is None else np.repeat(sd[:, 0], rps)
        coef = m - d[:, None]
        out = (xV * coef) @ U
        if sd is not None:
            out = out + d[:, None] * (x @ W.T)
        g_out = 2 * (out - target) / out.size
        da = g_out @ U.T
        dm = da * xV
        d_src, d_ci = po.source_mask_vjp(dm, ci, s, rps)
        d_sd = None
        if sd is not None:
            dd = pdo.site_delta_grad(x, W, V, U, m, d, None, g_out)
            d_sd = dd.reshape(-1, rps).sum(axis=1, keepdims=True)
        dU = (xV * coef).T @ g_out
        dV = x.T @ (da * coef)
        return float(((out - target) ** 2).mean()), d_src, d_ci, dV, dU, d_sd

    state = {"s": (src.copy(), np.zeros_like(src), np.zeros_like(src))}
    if dsrc is not None:
        state["d"] = (dsrc.copy(), np.zeros_like(dsrc), np.zeros_like(dsrc))
    step = 0.0

    def ascend(d_src, d_sd):
        s_, m_, v_ = state["s"]
        state["s"] = po.adam(s_, d_src, m_, v_, step, lr=lr)
        if dsrc is not None:
            s_, m_, v_ = state["d"]
            state["d"] = po.adam(s_, d_sd, m_, v_, step, lr=lr)

    cur = lambda k: None if k not in state else state[k][0]
    for _ in range(n_warmup):
        _, d_src, _, _, _, d_sd = recon(cur("s"), cur("d"))
        step += 1
        ascend(d_src, d_sd)
    loss, d_src, d_ci, dV, dU, d_sd = recon(cur("s"), cur("d"))
    step += 1
    ascend(d_src, d_sd)
    return loss, dV, dU, d_ci, cur("s"), cur("d")


@pytest.mark.parametrize("rps,with_delta", [(256, False), (32, False), (1, False), (32, True), (1, True)])
def test_dense_site_ppgd_step_matches_oracle(device, rps, with_delta):
    print(f"ppgd step rps={rps} delta={with_delta}", flush=True)
    rng = np.random.default_rng(rps)
    T, d_in, d_out, C = 256, 64, 48, 96
    x = rng.normal(size=(T, d_in)).astype(np.float32)
    V = (rng.normal(size=(d_in, C)) / 8).astype(np.float32)
    U = (rng.normal(size=(C, d_out)) / 10).astype(np.float32)
    W = (rng.normal(size=(d_out, d_in)) / 8).astype(np.float32)
    ci = rng.uniform(size=(T, C)).astype(np.float32)
    target = (x @ V @ U + rng.normal(size=(T, d_out)) * 0.1).astype(np.float32)
    src = rng.uniform(size=(T // rps, C)).astype(np.float32)
    dsrc = rng.uniform(size=(T // rps, 1)).astype(np.float32) if with_delta else None
    f = lambda a: torch.tensor(a, device=device)
    adv = A.PersistentAdversary(f(src.copy()), A.AdamPGDConfig(), n_warmup=2, rows_per_source=rps)
    dadv = None
    if with_delta:
        dadv = A.PersistentAdversary(f(dsrc.copy()), A.AdamPGDConfig(), n_warmup=2, rows_per_source=rps, leaf_index=1)
    res = A.DenseSitePPGDStep(adv, dadv).step(f(x), f(V), f(U), f(ci), f(target), lr=0.01, key=(0, 1),
                                              W=f(W) if with_delta else None)
    torch.cuda.synchronize()
    d64 = lambda a: None if a is None else a.astype(np.float64)
    loss, dV, dU, d_ci, s_final, d_final = _oracle_step(d64(x), d64(V), d64(U), d64(ci), d64(target), d64(src), rps,
                                                        2, 0.01, W=d64(W), dsrc=d64(dsrc))
    assert float(res.loss[0]) == pytest.approx(loss, rel=1e-4)
    assert len(res.warmup_losses) == 2
    assert _rel(_np(res.dV), dV) < 1e-4 and _rel(_np(res.dU), dU) < 1e-4 and _rel(_np(res.d_ci), d_ci) < 1e-4
    # Adam's steps are ~lr sign(g): a source whose gradient is within rounding of zero may
    # step the other way, so allow a few of those
    off = np.abs(_np(adv.sources) - s_final) > 1e-3
    assert off.mean() <= 1e-3
    assert adv.step_count == 3.0
    if with_delta:
        # the delta leaf moved, and by the oracle's Adam steps
        assert np.abs(_np(dadv.sources) - dsrc).max() > 5e-3
        assert (np.abs(_np(dadv.sources) - d_final) > 1e-3).mean() <= 2e-2
        assert dadv.step_count == 3.0


def test_dense_site_ppgd_step_bf16_runs_at_full_site_shape(device):
    gen = torch.Generator(device=device).manual_seed(0)
    T, d_in, d_out, C = 4096, 768, 3072, 4096
    x = torch.randn(T, d_in, device=device, generator=gen).to(torch.bfloat16)
    V = (torch.randn(d_in, C, device=device, generator=gen) / d_in ** 0.5).to(torch.bfloat16)
    U = (torch.randn(C, d_out, device=device, generator=gen) / C ** 0.5).to(torch.bfloat16)
    ci = torch.rand(T, C, device=device, generator=gen).to(torch.bfloat16)
    target = torch.randn(T, d_out, device=device, generator=gen).to(torch.bfloat16)
    src = A.store_unit_float(torch.rand(1, C, device=device, generator=gen), torch.uint16)
    adv = A.PersistentAdversary(src, A.MomentumSgdPGDConfig(0.9), n_warmup=2, rows_per_source=T)
    before = adv.float_sources.clone()
    res = A.DenseSitePPGDStep(adv).step(x, V, U, ci, target, lr=0.01, key=(3, 4))
    torch.cuda.synchronize()
    assert torch.isfinite(res.loss).all() and torch.isfinite(res.dV.float()).all()
    after = adv.float_sources
    assert ((after >= 0) & (after <= 1)).all() and not torch.equal(before, after)
    assert all(torch.isfinite(w).all() for w in res.warmup_losses)
