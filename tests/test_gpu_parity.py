"""GPU parity: every C-ABI entry point against the CPU oracle on the same seeded inputs.

Bars: bit-exact for Threefry bits/uniforms, routing indices and bucketing; fp32
kernels within rtol 1e-5 (looser only where an fp32 reduction order differs, stated per
test); bf16 kernels within rtol 2e-2 against a float64 oracle fed the same
bf16-rounded inputs.
"""

import numpy as np
import pytest
import torch

from oracle import pd_oracle as po
from oracle import threefry as tf

pytestmark = pytest.mark.gpu

BF16_RTOL = 2e-2


def np64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def bf(a, device):
    return torch.tensor(np.asarray(a, np.float32), device=device).to(torch.bfloat16)


def f32(a, device):
    return torch.tensor(np.asarray(a, np.float32), device=device)


def assert_close(got, want, rtol, atol_frac=1e-3, what=""):
    """|got - want| <= rtol*|want| + atol_frac*max|want| (the absolute floor scales with
    the tensor so near-zero entries of a bf16 product are judged at its precision)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = max(np.abs(want).max(), 1e-30)
    err = np.abs(got - want)
    if rtol <= 1e-4:  # fp32: the floor that rtol 1e-5 alone would need (0: 1e-5 holds as is)
        need = max(0.0, float(((err - 1e-5 * np.abs(want)) / scale).max()))
        print(f"[fp32] {what}: max rel {float((err / np.maximum(np.abs(want), 1e-30)).max()):.2e}, "
              f"floor needed at rtol 1e-5 {need:.2e}")
    bound = rtol * np.abs(want) + atol_frac * scale
    bad = err > bound
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} off; worst {err.max():.3e} (scale {scale:.3e})"


# ------------------------------------------------------------------ Threefry draws


@pytest.mark.parametrize("draw", ["float32", "bfloat16"])
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("n", [1, 7, 4096, 100003])
def test_uniform_bit_exact(device, draw, layout, n):
    from param_decomp_amd import ops

    key = tf.fold_in(tf.split(tf.prng_key(42))[0], 3)
    dt = torch.float32 if draw == "float32" else torch.bfloat16
    got = ops.uniform(key, (n,), dt, device, out_dtype=torch.float32, layout=layout)
    want = tf.uniform(key, (n,), draw, partitionable=(layout == 0))
    np.testing.assert_array_equal(got.cpu().numpy().astype(np.float64), want)


def test_uniform_reproduces_reference_stored_jax_draws(device):
    """pd_uniform (fp32 draw, partitionable layout) reproduces the reference's stored
    fp32 `jax.random.uniform` sources under `split(PRNGKey(3), 9)`
    (`tests/targets/stacked_parity/gen_stacked_fixtures.py:102`), bit for bit."""
    import os

    from param_decomp_amd import ops, prng

    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "stacked_sources.npz"))
    names = list(z.keys())
    keys = prng.split(prng.PRNGKey(3), len(names), partitionable=True)
    for key, name in zip(keys, names):
        want = z[name]
        got = ops.uniform(key, want.shape, torch.float32, device).cpu().numpy()
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32), err_msg=name)


def test_prng_host_matches_oracle():
    from param_decomp_amd import prng

    for seed in (0, 1, 12345):
        k = prng.PRNGKey(seed)
        assert prng.split(k) == tf.split(tf.prng_key(seed))
        assert prng.split(k, 3, partitionable=False) == tf.split(tf.prng_key(seed), 3, partitionable=False)
        assert prng.fold_in(k, 77) == tf.fold_in(tf.prng_key(seed), 77)


# ------------------------------------------------------------------ squashing / masks


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_squash_and_reference_cotangents(device, dtype):
    from param_decomp_amd.squashing import lower_leaky_hard_sigmoid, upper_leaky_hard_sigmoid

    xs = [-2.0, -2.0, 0.5, 0.5, 4.0, 4.0, 0.0, 0.0, 1.0, 1.0]
    gs = [-3.0, 3.0, -3.0, 3.0, -3.0, 3.0, -3.0, 3.0, -3.0, 3.0]
    x = torch.tensor(xs, device=device, dtype=dtype, requires_grad=True)
    # fp32: exact equality with the float32 value of each known answer, as the
    # reference's own test asserts (`cotangent == jnp.float32(expected)`)
    rtol = 1e-2 if dtype == torch.bfloat16 else 0
    cast = (lambda a: a) if dtype == torch.bfloat16 else (lambda a: np.asarray(a, np.float32).astype(np.float64))
    lo = lower_leaky_hard_sigmoid(x)
    (glo,) = torch.autograd.grad(lo, x, torch.tensor(gs, device=device, dtype=dtype))
    np.testing.assert_allclose(np64(glo), cast(po.lower_leaky_vjp(np.array(xs), np.array(gs))), rtol=rtol)
    up = upper_leaky_hard_sigmoid(x)
    (gup,) = torch.autograd.grad(up, x, torch.tensor(gs, device=device, dtype=dtype))
    # upper: 1 + 0.01*(x-1) is evaluated in fp32 (one rounding per op), so 1 ulp
    rtol_up = 1e-2 if dtype == torch.bfloat16 else 1e-6
    np.testing.assert_allclose(np64(up), po.upper_leaky(np.array(xs)), rtol=rtol_up)
    np.testing.assert_allclose(np64(gup), po.upper_leaky_vjp(np.array(xs), np.array(gs)), rtol=rtol_up)


def test_component_mask_fwd_bwd(device):
    from param_decomp_amd.masking import sample_component_mask

    rng = np.random.default_rng(0)
    ci = rng.uniform(size=(33, 70)).astype(np.float32)
    key = tf.fold_in(tf.prng_key(9), 1)
    x = f32(ci, device).requires_grad_(True)
    m = sample_component_mask(x, key)
    u = tf.uniform(key, ci.shape, "float32")
    np.testing.assert_allclose(np64(m), po.component_mask(ci.astype(np.float64), u), rtol=1e-6, atol=1e-7)
    g = rng.normal(size=ci.shape)
    (d,) = torch.autograd.grad(m, x, f32(g, device))
    np.testing.assert_allclose(np64(d), g * (1 - u), rtol=1e-6, atol=1e-7)


# ------------------------------------------------------------------ gate MLP


def _gate_np(rng, C, H=16):
    return po.GateParams(*(a.astype(np.float32).astype(np.float64) for a in (
        rng.normal(size=(C, H)) * 1.4, rng.normal(size=(C, H)) * 0.2, rng.normal(size=(C, H)) * 0.35,
        rng.normal(size=C) * 0.2 + 0.3)))


@pytest.mark.parametrize("precise", [True, False])
def test_gate_fwd_bwd_fp32(device, precise):
    from param_decomp_amd import ops

    rng = np.random.default_rng(1)
    T, C = 130, 75
    gp = _gate_np(rng, C)
    h = rng.normal(size=(T, C)).astype(np.float32).astype(np.float64)
    tp = [f32(a, device) for a in (gp.w_in, gp.b_in, gp.w_out, gp.b_out)]
    g = ops.gate_fwd(f32(h, device), *tp, precise)
    want = po.gate_forward(h, gp)
    # fast path: A&S 7.1.26 erf (|err| <= 1.5e-7) -> per-value error <= ~1e-6 absolute
    assert_close(np64(g), want, 1e-5, 1e-6 if precise else 3e-6, "gate fwd")
    dg = rng.normal(size=(T, C))
    dh, dwi, dbi, dwo, dbo = ops.gate_bwd(f32(h, device), *tp, f32(dg, device), precise)
    w = po.gate_backward(h, gp, dg)
    for got, want_, name in zip((dh, dwi, dbi, dwo, dbo), w, ("dh", "dw_in", "db_in", "dw_out", "db_out")):
        # precise: rtol 1e-5 with a 1e-6 floor (measured need <= 8e-8 of the largest
        # magnitude); the fast path's erf (A&S 7.1.26, |error| <= 1.5e-7) keeps 3e-5
        assert_close(np64(got), want_, 1e-5, 1e-6 if precise else 3e-5, name)


def test_gate_bf16_h(device):
    from param_decomp_amd import ops

    rng = np.random.default_rng(2)
    T, C = 96, 128
    gp = _gate_np(rng, C)
    hb = bf(rng.normal(size=(T, C)), device)
    tp = [f32(a, device) for a in (gp.w_in, gp.b_in, gp.w_out, gp.b_out)]
    g = ops.gate_fwd(hb, *tp, False)
    assert_close(np64(g), po.gate_forward(np64(hb), gp), BF16_RTOL, 1e-3, "gate fwd bf16")


# ------------------------------------------------------------------ losses


@pytest.mark.parametrize("p,beta", [(1.0, 0.0), (2.0, 0.0), (0.9, 0.2)])
def test_impmin_pnorm(device, p, beta):
    from param_decomp_amd import _lib as L
    from param_decomp_amd import ops

    rng = np.random.default_rng(3)
    up = rng.uniform(0.0, 1.2, size=(300, 37)).astype(np.float32).astype(np.float64)
    out, grad = ops.impmin(f32(up, device), kind=L.IMPMIN_PNORM, p=p, eps=1e-3, beta=beta, world_size=2.0,
                           want_grad=True)
    assert float(out[0]) == pytest.approx(po.impmin_pnorm(up, p, 1e-3, beta, 2), rel=1e-5)
    assert_close(np64(grad), po.impmin_pnorm_grad(up, p, 1e-3, beta, 2), 1e-5, 1e-6, "pnorm grad")


@pytest.mark.parametrize("normalize", [False, True])
def test_impmin_smooth_l0(device, normalize):
    from param_decomp_amd.losses import importance_minimality_terms

    rng = np.random.default_rng(4)
    a = rng.uniform(0.0, 1.1, size=(257, 40)).astype(np.float32).astype(np.float64)
    b = rng.uniform(0.0, 1.1, size=(257, 9)).astype(np.float32).astype(np.float64)
    ta, tb = f32(a, device).requires_grad_(True), f32(b, device).requires_grad_(True)
    act, freq = importance_minimality_terms({"a": ta, "b": tb}, 0.3, 64, normalize_at_one=normalize)
    wa, wf = po.importance_minimality_terms([a, b], 0.3, 64, normalize)
    assert float(act) == pytest.approx(wa, rel=1e-5)
    assert float(freq) == pytest.approx(wf, rel=1e-5)
    (ga,) = torch.autograd.grad(act + 0.5 * freq, ta)
    # finite differences of the oracle objective at a few entries
    f = lambda arr: sum(po.importance_minimality_terms([arr, b], 0.3, 64, normalize) * np.array([1.0, 0.5]))
    for idx in [(0, 0), (100, 17), (256, 39)]:
        e = 1e-6
        ap, am = a.copy(), a.copy()
        ap[idx] += e
        am[idx] -= e
        assert float(ga[idx]) == pytest.approx((f(ap) - f(am)) / (2 * e), rel=1e-3, abs=1e-7)


def test_reference_smooth_l0_closed_forms_on_gpu(device):
    from param_decomp_amd.losses import importance_minimality_terms

    act, freq = importance_minimality_terms({"a": f32([[1.0, 2.0], [3.0, 4.0]], device)}, 1.0, 8,
                                            normalize_at_one=False)
    f0, f1 = (1 / 2 + 9 / 10) / 2, (4 / 5 + 16 / 17) / 2
    assert float(act) == pytest.approx(f0 + f1, rel=1e-6)
    assert float(freq) == pytest.approx(f0 * np.log2(1 + 8 * f0) + f1 * np.log2(1 + 8 * f1), rel=1e-6)
    act, _ = importance_minimality_terms({"a": f32([[1.0, 1.0]], device)}, 0.1, None, normalize_at_one=True)
    assert float(act) == pytest.approx(2.0, rel=1e-6)


def test_mse_and_kl(device):
    from param_decomp_amd.losses import categorical_kl_from_logits, mse

    rng = np.random.default_rng(5)
    a, b = rng.normal(size=(50, 33)), rng.normal(size=(50, 33))
    ta = f32(a, device).requires_grad_(True)
    loss = mse(ta, f32(b, device))
    a32, b32 = a.astype(np.float32).astype(np.float64), b.astype(np.float32).astype(np.float64)
    assert float(loss) == pytest.approx(po.mse(a32, b32), rel=1e-5)
    (g,) = torch.autograd.grad(loss, ta)
    assert_close(np64(g), 2 * (a32 - b32) / a.size, 1e-5, 1e-7, "mse grad")
    m, c = rng.normal(size=(9, 1001)) * 3, rng.normal(size=(9, 1001)) * 3
    tm = f32(m, device).requires_grad_(True)
    kl = categorical_kl_from_logits(tm, f32(c, device))
    m32, c32 = m.astype(np.float32).astype(np.float64), c.astype(np.float32).astype(np.float64)
    assert float(kl) == pytest.approx(po.categorical_kl(m32, c32), rel=1e-4)
    (gk,) = torch.autograd.grad(kl, tm)
    assert_close(np64(gk), po.categorical_kl_grad(m32, c32), 1e-4, 1e-6, "kl grad")


# ------------------------------------------------------------------ GEMM


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(128, 128, 64), (200, 136, 72), (256, 384, 768), (8, 8, 8), (1000, 776, 1096),
                                   (136, 264, 520)])
def test_gemm_bf16_layouts(device, ta, tb, M, N, K):
    """Every operand layout runs the buffer-fed kernel (an MN-major operand's fragments
    transposed on their way out of LDS); ragged tiles and a k-tail stage."""
    from param_decomp_amd import ops

    rng = np.random.default_rng(M + N + K + 2 * ta + tb)
    A = rng.normal(size=(K, M) if ta else (M, K))
    B = rng.normal(size=(N, K) if tb else (K, N))
    Ab, Bb = bf(A, device), bf(B, device)
    out = ops.gemm(Ab, Bb, trans_a=bool(ta), trans_b=bool(tb), out_dtype=torch.float32)
    An, Bn = np64(Ab), np64(Bb)
    want = (An.T if ta else An) @ (Bn.T if tb else Bn)
    assert_close(np64(out), want, 1e-5, 1e-6, f"gemm ta={ta} tb={tb}")  # fp32 out: accumulation order only
    out16 = ops.gemm(Ab, Bb, trans_a=bool(ta), trans_b=bool(tb))
    assert_close(np64(out16), want, BF16_RTOL, 1e-3, "gemm bf16 out")


@pytest.mark.parametrize("ta,tb", [(0, 1), (1, 0), (1, 1), (0, 0)])
def test_gemm_bf16_padded_leading_dims(device, ta, tb):
    """Leading dimensions past the operand extents (column blocks of wider tensors): the
    columns an MN-major tile reads past M or N only feed outputs that are never stored."""
    from param_decomp_amd import _lib as L

    rng = np.random.default_rng(40 + 2 * ta + tb)
    M, N, K, pad = 264, 200, 328, 24
    A = bf(rng.normal(size=(K, M + pad) if ta else (M, K + pad)), device)
    B = bf(rng.normal(size=(N, K + pad) if tb else (K, N + pad)), device)
    C = torch.full((M, N + 8), 7.0, dtype=torch.float32, device=device)
    L.call("pd_gemm", L.BF16, M, N, K, L.ptr(A), A.shape[1], ta, L.ptr(B), B.shape[1], tb, L.ptr(C), N + 8, L.F32,
           1.0, 0.0, L.stream())
    a, b = np64(A), np64(B)
    a = a[:, :M].T if ta else a[:, :K]
    b = b[:, :K].T if tb else b[:, :N]
    assert_close(np64(C)[:, :N], a @ b, 1e-5, 1e-6, f"padded gemm ta={ta} tb={tb}")
    assert torch.all(C[:, N:] == 7.0)


@pytest.mark.parametrize("ta,tb", [(0, 1), (1, 0), (1, 1), (0, 0)])
@pytest.mark.parametrize("M,N,K", [(264, 200, 328), (70, 90, 1200), (40, 33, 3002)])
@pytest.mark.parametrize("pad,off", [(24, 0), (3, 1)])
def test_gemm_fp32_padded_and_offset(device, ta, tb, M, N, K, pad, off):
    """fp32 operands inside wider tensors: padded leading dimensions, and (off = 1) base
    pointers and leading dimensions that are not 16-byte multiples, where the direct form
    reads K-contiguous rows as dwords instead of 16-byte vectors; contraction split over 8
    and 16 waves, K % 4 != 0 at K = 3002."""
    from param_decomp_amd import _lib as L

    rng = np.random.default_rng(M + N + K + 2 * ta + tb + pad)
    A = f32(rng.normal(size=(K, M + pad) if ta else (M, K + pad)), device)
    B = f32(rng.normal(size=(N, K + pad) if tb else (K, N + pad)), device)
    C = torch.full((M, N + 8), 7.0, dtype=torch.float32, device=device)
    L.call("pd_gemm", L.F32, M, N, K, L.ptr(A) + 4 * off, A.shape[1], ta, L.ptr(B) + 4 * off, B.shape[1], tb, L.ptr(C),
           N + 8, L.F32,
           1.0, 0.0, L.stream())
    a, b = np64(A)[:, off:], np64(B)[:, off:]
    a = a[:, :M].T if ta else a[:, :K]
    b = b[:, :K].T if tb else b[:, :N]
    assert_close(np64(C)[:, :N], a @ b, 1e-5, 1e-6, f"padded fp32 gemm ta={ta} tb={tb} pad={pad} off={off}")
    assert torch.all(C[:, N:] == 7.0)


def test_gemm_alpha_beta_and_fp32(device):
    from param_decomp_amd import ops

    rng = np.random.default_rng(11)
    A, B, C0 = rng.normal(size=(70, 50)), rng.normal(size=(50, 90)), rng.normal(size=(70, 90))
    c = f32(C0, device)
    ops.gemm(f32(A, device), f32(B, device), out=c, alpha=0.5, beta=2.0)
    A32, B32, C32 = (x.astype(np.float32).astype(np.float64) for x in (A, B, C0))
    assert_close(np64(c), 0.5 * A32 @ B32 + 2 * C32, 1e-5, 1e-6, "fp32 gemm")


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(2048, 100, 1000), (1000, 100, 2048), (100, 1000, 2048), (2048, 1000, 100),
                                   (70, 50, 5), (33, 65, 97), (2048, 50, 1000)])
def test_gemm_fp32_matrix_core_layouts(device, ta, tb, M, N, K):
    """The fp32 MFMA kernel at the residual-MLP target's product shapes (its forward
    contractions and weight gradients over 2048 rows) and ragged edges in every
    dimension, every operand layout: fp32 accumulation-order error of a float64 product."""
    from param_decomp_amd import ops

    rng = np.random.default_rng(M * 7 + N * 3 + K + 2 * ta + tb)
    A = f32(rng.normal(size=(K, M) if ta else (M, K)), device)
    B = f32(rng.normal(size=(N, K) if tb else (K, N)), device)
    out = ops.gemm(A, B, trans_a=bool(ta), trans_b=bool(tb))
    An, Bn = np64(A), np64(B)
    want = (An.T if ta else An) @ (Bn.T if tb else Bn)
    assert_close(np64(out), want, 1e-5, 1e-6, f"fp32 gemm ta={ta} tb={tb} {M}x{N}x{K}")
    again = ops.gemm(A, B, trans_a=bool(ta), trans_b=bool(tb))
    assert torch.equal(out, again)  # fixed summation order


# ------------------------------------------------------------------ masked linear (site_forward)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("with_delta,with_route", [(False, False), (True, False), (True, True), (False, True)])
@pytest.mark.parametrize("shape", [(3, 40, 64, 96, 128), (2, 150, 200, 136, 520)])
def test_site_forward_and_backward(device, dtype, with_delta, with_route, shape):
    """bf16 runs the fused seam (the mask step in the x @ V and g @ U^T epilogues, the
    target blend inside one k loop over [W^T ; U]); the second shape has several k
    stages and k tails in every product."""
    from param_decomp_amd.decomposed_linear import SiteWeights, site_forward

    rng = np.random.default_rng(12)
    B_, S, d_in, d_out, C = shape
    x = rng.normal(size=(B_, S, d_in))
    W = rng.normal(size=(d_out, d_in)) / 8
    V = rng.normal(size=(d_in, C)) / 8
    U = rng.normal(size=(C, d_out)) / 11
    m = rng.uniform(size=(B_, S, C))
    d = rng.uniform(size=(B_, S)) if with_delta else None
    r = rng.uniform(size=(B_, S)) > 0.3 if with_route else None
    cv = (lambda a: bf(a, device)) if dtype == torch.bfloat16 else (lambda a: f32(a, device))
    tx, tV, tU, tm = (cv(a).requires_grad_(True) for a in (x, V, U, m))
    tW = cv(W)
    td = None if d is None else cv(d).requires_grad_(True)
    tr = None if r is None else torch.tensor(r, device=device)
    res = site_forward(tx, SiteWeights(tW, tV, tU), tm, td, tr)
    xs, Ws, Vs, Us, ms = (np64(t) for t in (tx, tW, tV, tU, tm))
    ds = None if td is None else np64(td)
    want, want_xV = po.site_forward(xs, Ws, Vs, Us, ms, ds, r)
    # fp32: rtol 1e-5 with a floor of 1e-6 of the tensor's largest magnitude, the rounding
    # of an fp32 reduction against float64 (measured need <= 1.2e-7 on these shapes)
    rtol = 1e-5 if dtype == torch.float32 else BF16_RTOL
    assert_close(np64(res.output), want, rtol, 1e-6 if dtype == torch.float32 else 4e-3, "site out")
    assert_close(np64(res.component_activation), want_xV, rtol, 1e-6 if dtype == torch.float32 else 4e-3, "xV")
    go = rng.normal(size=want.shape)
    inputs = (tx, tV, tU, tm) + (() if td is None else (td,))
    grads = torch.autograd.grad(res.output, inputs, cv(go))
    dx, dV, dU, dm = po.site_backward(xs, Ws, Vs, Us, ms, ds, r, np64(cv(go)))
    wants = (dx, dV, dU, dm)
    if td is not None:  # the weight-delta cotangent (the delta sources of adversarial masking)
        wants = wants + (po.site_delta_grad(xs, Ws, Vs, Us, ms, ds, r, np64(cv(go))),)
    for got, w, name in zip(grads, wants, ("dx", "dV", "dU", "dmask", "d_delta")):
        assert_close(np64(got), w, rtol, 1e-6 if dtype == torch.float32 else 5e-3, name)


@pytest.mark.parametrize("blocked", [False, True])
def test_site_forward_casts_fp32_mask_and_delta_to_bf16(device, blocked):
    """An fp32 mask or delta (e.g. uniforms drawn in fp32) with bf16 activations is cast
    to x's dtype, as the reference's arithmetic promotes it: the result equals the
    all-bf16 call bit for bit, gradients included (returned in the input's dtype)."""
    from param_decomp_amd.decomposed_linear import (BlockedSiteWeights, SiteWeights, blocked_site_forward,
                                                    site_forward)

    rng = np.random.default_rng(31)
    T, d_in, d_out = 48, 64, 80
    if blocked:
        E, c = 3, 16
        C = E * c
        W, V, U = rng.normal(size=(E * d_out, d_in)) / 8, rng.normal(size=(E, d_in, c)) / 8, rng.normal(
            size=(E, c, d_out)) / 8
        run = lambda x, m, d: blocked_site_forward(x, BlockedSiteWeights(tW, tV, tU), m, d, None,  # noqa: E731
                                                   "fused_output").output
    else:
        C = 96
        W, V, U = rng.normal(size=(d_out, d_in)) / 8, rng.normal(size=(d_in, C)) / 8, rng.normal(size=(C, d_out)) / 8
        run = lambda x, m, d: site_forward(x, SiteWeights(tW, tV, tU), m, d, None).output  # noqa: E731
    tW, tV, tU = bf(W, device), bf(V, device), bf(U, device)
    x = bf(rng.normal(size=(T, d_in)), device)
    m32 = f32(po.round_bf16(rng.uniform(size=(T, C))), device).requires_grad_(True)
    d32 = f32(po.round_bf16(rng.uniform(size=T)), device).requires_grad_(True)
    m16 = m32.detach().to(torch.bfloat16).requires_grad_(True)
    d16 = d32.detach().to(torch.bfloat16).requires_grad_(True)
    y32, y16 = run(x, m32, d32), run(x, m16, d16)
    assert torch.equal(y32, y16)
    g = bf(rng.normal(size=tuple(y16.shape)), device)
    gm32, gd32 = torch.autograd.grad(y32, (m32, d32), g)
    gm16, gd16 = torch.autograd.grad(y16, (m16, d16), g)
    assert gm32.dtype == torch.float32 and gd32.dtype == torch.float32
    assert torch.equal(gm32, gm16.float()) and torch.equal(gd32, gd16.float())


# ------------------------------------------------------------------ fused dense step


def _dense_inputs(rng, T, d_in, d_out, C):
    x = rng.normal(size=(T, d_in))
    W = rng.normal(size=(d_out, d_in)) / np.sqrt(d_in)
    V = rng.normal(size=(d_in, C)) / np.sqrt(d_in)
    U = rng.normal(size=(C, d_out)) / np.sqrt(C)
    gp = po.GateParams(rng.normal(size=(C, 16)) * 1.4, np.zeros((C, 16)), rng.normal(size=(C, 16)) * 0.35,
                       np.full(C, 0.3))
    return x, W, V, U, gp


@pytest.mark.parametrize("use_delta,sl0", [(False, False), (True, False), (True, True)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_dense_step_matches_oracle(device, dtype, use_delta, sl0):
    """sl0: the engine's smooth-L0 term with its frequency penalty (each 64-token chunk's
    column sums of psi in the gate pass, frequencies and slopes in between, the slope in
    the gate backward)."""
    from param_decomp_amd.dense_step import DenseSiteStep
    from param_decomp_amd.losses import ImpMin

    rng = np.random.default_rng(13)
    T, d_in, d_out, C = 256, 64, 96, 192
    x, W, V, U, gp = _dense_inputs(rng, T, d_in, d_out, C)
    cv = (lambda a: bf(a, device)) if dtype == torch.bfloat16 else (lambda a: f32(a, device))
    tx, tW, tV, tU = (cv(a) for a in (x, W, V, U))
    gate = tuple(f32(a, device) for a in (gp.w_in, gp.b_in, gp.w_out, gp.b_out))
    draw_key = tf.fold_in(tf.prng_key(5), 1)
    spec = (po.ImpMin("smooth_l0", coeff=0.7, gamma=0.2, normalize_at_one=True, freq_coeff=0.4, ref_count=300.0)
            if sl0 else po.ImpMin("pnorm", p=2.0, coeff=0.7))
    imp = ImpMin(spec.kind, spec.p, spec.coeff, spec.gamma, spec.normalize_at_one, spec.freq_coeff, spec.ref_count)
    step = DenseSiteStep(T, d_in, d_out, C, dtype=dtype, device=device, recon_coeff=1.3, use_delta=use_delta,
                         imp_min=imp)
    mk, dk = step.site_keys(draw_key, 0)
    g = step.step(tx, tW, tV, tU, gate, mk, dk)
    torch.cuda.synchronize()
    gp64 = po.GateParams(*(np64(t) for t in gate))
    r = po.dense_site_step(np64(tx), np64(tW), np64(tV), np64(tU), gp64, draw_key, recon_coeff=1.3,
                           mask_dtype="bfloat16" if dtype == torch.bfloat16 else "float32",
                           use_delta=use_delta, bf16_storage=dtype == torch.bfloat16, imp_min=spec)
    rtol = 1e-5 if dtype == torch.float32 else BF16_RTOL
    losses = g.losses.cpu().numpy()
    np.testing.assert_allclose(losses, [r.loss, r.recon, r.imp, r.freq], rtol=rtol, atol=1e-7)
    # fp32 floor: 1e-6 of the largest magnitude (fp32 reductions against float64; measured
    # need <= 1.3e-7), 1e-5 with smooth-L0, where one dV entry measured 4.3e-6: a gate value
    # within fp32 rounding of a squashing kink takes the other backward branch
    floor = (1e-5 if sl0 else 1e-6) if dtype == torch.float32 else 1e-2
    assert_close(np64(g.dU), r.dU, rtol, floor, "dU")
    assert_close(np64(g.dV), r.dV, rtol, floor, "dV")
    for got, want, name in zip((g.dw_in, g.db_in, g.dw_out, g.db_out), r.dgate, ("dw_in", "db_in", "dw_out", "db_out")):
        assert_close(np64(got), want, rtol, floor, name)


def test_dense_step_bf16_exact_gate_components(device):
    """The bf16 step's binned gate falls back to the exact per-element gate for components
    with a hidden unit wider than 3 in z over one moment bin. Four components get w_in x8
    (two share a 32-component block with unflagged ones, so flagged and unflagged lanes run
    in one wave); the whole step must still match the oracle at the bf16 tolerance."""
    from param_decomp_amd.dense_step import DenseSiteStep

    rng = np.random.default_rng(21)
    T, d_in, d_out, C = 256, 64, 96, 192
    x, W, V, U, gp = _dense_inputs(rng, T, d_in, d_out, C)
    wide = [0, 5, 33, 100]
    gp.w_in[wide] *= 8.0
    tx, tW, tV, tU = (bf(a, device) for a in (x, W, V, U))
    gate = tuple(f32(a, device) for a in (gp.w_in, gp.b_in, gp.w_out, gp.b_out))
    # which components the step flags (moment-bin width = range(h) / 16)
    h = np64(tx) @ np64(tV)
    dz = np.abs(np64(gate[0])).max(1) * (h.max(0) - h.min(0)) / 16
    assert (dz[wide] > 4).all() and (np.delete(dz, wide) < 2.5).all(), dz
    draw_key = tf.fold_in(tf.prng_key(9), 1)
    step = DenseSiteStep(T, d_in, d_out, C, dtype=torch.bfloat16, device=device, recon_coeff=1.3, use_delta=True)
    mk, dk = step.site_keys(draw_key, 0)
    g = step.step(tx, tW, tV, tU, gate, mk, dk)
    torch.cuda.synchronize()
    gp64 = po.GateParams(*(np64(t) for t in gate))
    r = po.dense_site_step(np64(tx), np64(tW), np64(tV), np64(tU), gp64, draw_key, recon_coeff=1.3,
                           mask_dtype="bfloat16", use_delta=True, bf16_storage=True)
    np.testing.assert_allclose(g.losses.cpu().numpy(), [r.loss, r.recon, r.imp, r.freq], rtol=BF16_RTOL, atol=1e-7)
    assert_close(np64(g.dU), r.dU, BF16_RTOL, 1e-2, "dU")
    assert_close(np64(g.dV), r.dV, BF16_RTOL, 1e-2, "dV")
    for got, want, name in zip((g.dw_in, g.db_in, g.dw_out, g.db_out), r.dgate, ("dw_in", "db_in", "dw_out", "db_out")):
        assert_close(np64(got), want, BF16_RTOL, 1e-2, name)
        # the flagged components alone, at their own scale
        assert_close(np64(got)[wide], want[wide], BF16_RTOL, 1e-2, name + "[flagged]")


def test_dense_step_full_size_properties(device):
    """At the full single-linear shape (T=4096, 768->3072, C=4096): the step is
    deterministic run to run, losses are finite and positive, and the gradient of
    the recon term scales linearly with recon_coeff (the MSE pullback is linear in its
    coefficient and imp_coeff=0 removes the other term)."""
    from param_decomp_amd.dense_step import DenseSiteStep

    T, d_in, d_out, C = 4096, 768, 3072, 4096
    gen = torch.Generator(device=device).manual_seed(0)
    x = torch.randn(T, d_in, device=device, generator=gen).to(torch.bfloat16)
    W = (torch.randn(d_out, d_in, device=device, generator=gen) / d_in**0.5).to(torch.bfloat16)
    V = (torch.randn(d_in, C, device=device, generator=gen) / d_in**0.5).to(torch.bfloat16)
    U = (torch.randn(C, d_out, device=device, generator=gen) / C**0.5).to(torch.bfloat16)
    gate = (torch.randn(C, 16, device=device, generator=gen) * 1.4, torch.zeros(C, 16, device=device),
            torch.randn(C, 16, device=device, generator=gen) * 0.35, torch.full((C,), 0.3, device=device))
    mk, dk = DenseSiteStep.site_keys((0, 7), 0)
    s1 = DenseSiteStep(T, d_in, d_out, C, device=device, imp_coeff=0.0, recon_coeff=1.0)
    a = s1.step(x, W, V, U, gate, mk, dk)
    dV1, dU1, l1 = a.dV.clone(), a.dU.clone(), a.losses.clone()
    a = s1.step(x, W, V, U, gate, mk, dk)
    assert torch.equal(a.dV, dV1) and torch.equal(a.dU, dU1) and torch.equal(a.losses, l1)
    assert torch.isfinite(l1).all() and float(l1[1]) > 0
    s2 = DenseSiteStep(T, d_in, d_out, C, device=device, imp_coeff=0.0, recon_coeff=2.0)
    b = s2.step(x, W, V, U, gate, mk, dk)
    torch.testing.assert_close(b.dU, 2 * dU1, rtol=2e-2, atol=1e-3 * float(dU1.abs().max()))


# ------------------------------------------------------------------ routing


@pytest.mark.parametrize("E,k", [(42, 8), (100, 6), (256, 8), (500, 16)])
def test_router_topk_bit_exact_indices(device, E, k):
    """E > 64 puts several experts on each lane (lane l holds experts l + 64 i)."""
    from param_decomp_amd.routed.experts import route_tokens

    rng = np.random.default_rng(14 + E)
    T = 1000
    logits = rng.normal(size=(T, E)).astype(np.float32)
    logits[3, [5, 9, 11]] = 2.5  # exact ties: lowest index first
    logits[4, :] = 0.0
    probs, idx, w = route_tokens(f32(logits, device), k)
    p_or = po.softmax(logits.astype(np.float64))
    want_idx = po.select_experts(p_or, k)
    np.testing.assert_array_equal(idx.cpu().numpy(), want_idx)
    np.testing.assert_allclose(probs.cpu().numpy(), p_or, rtol=2e-6, atol=1e-7)
    np.testing.assert_allclose(w.cpu().numpy(), po.expert_mixing_weights(p_or, want_idx), rtol=1e-5)


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("S,n", [(7, 1000), (24, 4096), (1, 5), (64, 300), (12, 8192)])
def test_route_uniform_k_bit_exact(device, layout, S, n):
    from param_decomp_amd.routing import UniformKRouting

    key = (5, 77 + S)
    sites = tuple(f"s{j}" for j in range(S))
    got = UniformKRouting(sites, device, layout)(key, (n,))
    want = po.uniform_k_routing(key, S, (n,), partitionable=layout == 0)
    for j, name in enumerate(sites):
        assert got[name].dtype == torch.bool
        np.testing.assert_array_equal(got[name].cpu().numpy(), want[j], err_msg=name)


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("p", [0.0, 0.3, 0.5, 1.0])
def test_route_static_p_bit_exact(device, layout, p):
    from param_decomp_amd.routing import AllRouting, StaticProbabilityRouting

    key = (9, 31)
    sites = ("a", "b", "c")
    got = StaticProbabilityRouting(sites, p, device, layout)(key, (3, 700))
    want = po.static_probability_routing(key, 3, p, (3, 700), partitionable=layout == 0)
    for j, name in enumerate(sites):
        np.testing.assert_array_equal(got[name].cpu().numpy(), want[j])
    assert AllRouting()(key, (3, 700)) is None


@pytest.mark.parametrize("T,k,E", [(24, 2, 8), (8192, 8, 42), (1000, 3, 5), (7, 1, 64), (3001, 5, 1000)])
def test_routed_jobs_bit_exact(device, T, k, E):
    from param_decomp_amd.routed.experts import routed_jobs

    if (T, k, E) == (24, 2, 8):
        first = np.arange(T) % (E - 2)
        top = np.stack([first, (first + 1) % (E - 2)], axis=1).astype(np.int32)
    else:
        rng = np.random.default_rng(T)
        top = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    jobs = routed_jobs(torch.tensor(top, device=device), E)
    want = po.routed_jobs(top, E)
    np.testing.assert_array_equal(jobs.sort_idx.cpu().numpy(), want.sort_idx)
    np.testing.assert_array_equal(jobs.inv_sort_idx.cpu().numpy(), want.inv_sort_idx)
    np.testing.assert_array_equal(jobs.group_sizes.cpu().numpy(), want.group_sizes)
    np.testing.assert_array_equal(jobs.group_offsets.cpu().numpy(), np.concatenate([[0], np.cumsum(want.group_sizes)]))


def test_gather_combine_and_vjp(device):
    from param_decomp_amd.routed.experts import combine_jobs, gather_tokens, routed_jobs, sum_jobs

    rng = np.random.default_rng(15)
    T, k, E, D = 300, 4, 10, 48
    top = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    jobs = routed_jobs(torch.tensor(top, device=device), E)
    oj = po.routed_jobs(top, E)
    x = rng.normal(size=(T, D))
    tx = f32(x, device).requires_grad_(True)
    xj = gather_tokens(tx, jobs)
    np.testing.assert_array_equal(np64(xj), po.gather_tokens(x.astype(np.float32).astype(np.float64), oj))
    g = rng.normal(size=(T * k, D))
    (gx,) = torch.autograd.grad(xj, tx, f32(g, device))
    assert_close(np64(gx), po.gather_tokens_vjp(g.astype(np.float32).astype(np.float64), oj), 1e-6, 1e-7, "vjp")
    y = rng.normal(size=(T * k, D)).astype(np.float32).astype(np.float64)
    w = po.softmax(rng.normal(size=(T, k))).astype(np.float32).astype(np.float64)
    assert_close(np64(sum_jobs(f32(y, device), jobs)), po.sum_jobs(y, oj), 1e-6, 1e-7, "sum_jobs")
    assert_close(np64(combine_jobs(f32(y, device), jobs, f32(w, device))), po.combine_jobs(y, oj, w), 1e-6, 1e-7,
                 "combine")


@pytest.mark.parametrize("sizes", [[7, 0, 19, 1, 0, 26, 37, 0], [0, 0, 300, 5], [129, 128, 127, 1]])
def test_grouped_matmul_fwd_bwd(device, sizes):
    from param_decomp_amd.routed.experts import grouped_matmul, transposed_grouped_matmul

    rng = np.random.default_rng(sum(sizes))
    E, K, N = len(sizes), 64, 136
    J = int(sum(sizes)) + 5  # 5 trailing rows past sum(group_sizes)
    offsets = torch.tensor(np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32), device=device)
    lhs = bf(rng.normal(size=(J, K)), device).requires_grad_(True)
    rhs = bf(rng.normal(size=(E, K, N)) / 8, device).requires_grad_(True)
    out = grouped_matmul(lhs, rhs, offsets)
    want = po.grouped_matmul(np64(lhs), np64(rhs), sizes)
    assert_close(np64(out), want, BF16_RTOL, 4e-3, "grouped fwd")
    assert np.all(np64(out)[sum(sizes):] == 0)
    g = bf(rng.normal(size=(J, N)), device)
    dl, dr = torch.autograd.grad(out, (lhs, rhs), g)
    gn = np64(g)
    gn[sum(sizes):] = 0.0
    want_dl = po.grouped_matmul(gn, np.transpose(np64(rhs), (0, 2, 1)), sizes)
    assert_close(np64(dl), want_dl, BF16_RTOL, 4e-3, "grouped d_lhs")
    want_dr = po.transposed_grouped_matmul(np64(lhs), gn, sizes)
    assert_close(np64(dr), want_dr, BF16_RTOL, 4e-3, "grouped d_rhs")
    dw = transposed_grouped_matmul(lhs.detach(), g, offsets, out_dtype=torch.float32)
    assert_close(np64(dw), want_dr, 1e-5, 1e-6, "dw fp32")
    for e, s in enumerate(sizes):
        if s == 0:
            assert torch.count_nonzero(dw[e]) == 0 and torch.count_nonzero(dr[e]) == 0


@pytest.mark.parametrize("sizes", [[7, 0, 19, 1, 0, 26, 37, 0], [0, 0, 300, 5], [129, 128, 127, 1]])
@pytest.mark.parametrize("K", [72, 512])
def test_grouped_gemm_kmajor_rhs(device, sizes, K):
    """Grouped forward with the per-group weights stored [E, N, K] (K-contiguous): ragged
    groups, a contraction that is not a multiple of the 64-wide k tile, trailing rows."""
    from param_decomp_amd import ops

    rng = np.random.default_rng(11 + K + sum(sizes))
    E, N = len(sizes), 136
    used = int(sum(sizes))
    J = used + 5
    offsets = torch.tensor(np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32), device=device)
    lhs = bf(rng.normal(size=(J, K)), device)
    rhsT = bf(rng.normal(size=(E, N, K)) / 8, device)
    out = ops.grouped_gemm(lhs, rhsT, offsets, trans_rhs=True)
    want = po.grouped_matmul(np64(lhs)[:used], np.transpose(np64(rhsT), (0, 2, 1)), sizes)
    assert_close(np64(out)[:used], want, BF16_RTOL, 4e-3, "grouped kmajor rhs")
    assert np.all(np64(out)[used:] == 0)


@pytest.mark.parametrize("sizes", [[7, 0, 19, 1, 0, 26, 37, 0], [0, 0, 300, 5], [129, 128, 127, 1], [3, 5]])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_grouped_gemm_dw_kmajor(device, sizes, out_dtype):
    """Ragged-contraction dW from job-contiguous operands: unaligned group starts and
    empty groups (exact zeros); trailing jobs past the last offset are ignored."""
    from param_decomp_amd import ops

    rng = np.random.default_rng(7 + sum(sizes))
    E, K, N = len(sizes), 72, 136
    used = int(sum(sizes))
    J = (used + 5 + 7) // 8 * 8
    offsets = torch.tensor(np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32), device=device)
    lhs = bf(rng.normal(size=(J, K)), device)
    dout = bf(rng.normal(size=(J, N)), device)
    dw = ops.grouped_gemm_dw_kmajor(lhs.t().contiguous(), dout.t().contiguous(), offsets, E, out_dtype=out_dtype)
    want = po.transposed_grouped_matmul(np64(lhs)[:used], np64(dout)[:used], sizes)
    if out_dtype == torch.float32:
        assert_close(np64(dw), want, 1e-5, 1e-6, "dw kmajor fp32")
    else:
        assert_close(np64(dw), want, BF16_RTOL, 4e-3, "dw kmajor bf16")
    ref = ops.grouped_gemm_dw(lhs, dout, offsets, E, out_dtype=torch.float32)
    if out_dtype == torch.float32:
        assert_close(np64(dw), np64(ref), 1e-6, 1e-6, "dw kmajor vs row-major")
    for e, s in enumerate(sizes):
        if s == 0:
            assert torch.count_nonzero(dw[e]) == 0


@pytest.mark.parametrize("sizes", [[700, 0, 300, 1025], [7, 0, 19, 1, 0, 26, 37, 0], [129, 128, 127, 1]])
def test_grouped_gemm_dw_row_major(device, sizes):
    """Ragged-contraction dW straight from the token-row operands (both MN-major: the
    k axis is the row index): multi-stage groups, unaligned starts, empty groups."""
    from param_decomp_amd import ops

    rng = np.random.default_rng(70 + sum(sizes))
    E, K, N = len(sizes), 200, 264
    used = int(sum(sizes))
    J = used + 3
    offsets = torch.tensor(np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32), device=device)
    lhs = bf(rng.normal(size=(J, K)), device)
    dout = bf(rng.normal(size=(J, N)), device)
    dw = ops.grouped_gemm_dw(lhs, dout, offsets, E, out_dtype=torch.float32)
    want = po.transposed_grouped_matmul(np64(lhs)[:used], np64(dout)[:used], sizes)
    assert_close(np64(dw), want, 1e-5, 1e-6, "dw row-major fp32")
    for e, s_ in enumerate(sizes):
        if s_ == 0:
            assert torch.count_nonzero(dw[e]) == 0


@pytest.mark.parametrize("K", [200, 520])
def test_grouped_gemm_mn_rhs_multistage(device, K):
    """Grouped forward with each expert's weight stored [K, N] (MN-major) over several k
    stages and a k tail."""
    from param_decomp_amd import ops

    sizes = [300, 0, 129, 77]
    rng = np.random.default_rng(K)
    E, N = len(sizes), 392
    used = int(sum(sizes))
    offsets = torch.tensor(np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32), device=device)
    lhs = bf(rng.normal(size=(used + 4, K)), device)
    rhs = bf(rng.normal(size=(E, K, N)) / 8, device)
    out = ops.grouped_gemm(lhs, rhs, offsets, trans_rhs=False, out_dtype=torch.float32)
    want = po.grouped_matmul(np64(lhs)[:used], np64(rhs), sizes)
    assert_close(np64(out)[:used], want, 1e-5, 1e-6, "grouped mn rhs")
    assert torch.count_nonzero(out[used:]) == 0


# ------------------------------------------------------------------ streamed-vocab KL


@pytest.mark.parametrize("dtype,n_chunks,V,d,shared", [(torch.float32, 1, 1200, 64, False),
                                                       (torch.float32, 3, 1200, 64, False),
                                                       (torch.float32, 8, 1200, 64, False),
                                                       (torch.bfloat16, 8, 4096, 128, False),
                                                       (torch.bfloat16, 2, 4096, 128, False),
                                                       (torch.bfloat16, 3, 4101, 128, False),
                                                       (torch.bfloat16, 1, 2011, 128, False),
                                                       (torch.bfloat16, 3, 999, 72, False),
                                                       (torch.bfloat16, 3, 4101, 128, True),
                                                       (torch.bfloat16, 1, 2011, 128, True),
                                                       (torch.bfloat16, 3, 999, 72, True)])
def test_streamed_kl_fwd_bwd(device, dtype, n_chunks, V, d, shared):
    """Per-position KL and the masked-activation gradient against the float64 oracle on
    the same (dtype-rounded) inputs. fp32: |err| <= 1e-4 |want| + 2e-6 max|want| (fp32
    logits accumulated over d, exp/log in fp32). bf16: the gradient's (q - p) g passes
    through bf16 on its way into the GEMM, so rtol 2e-2. V = 4101 (3 x 1367) and 2011 (prime)
    give bf16 chunk widths that are not multiples of 8: the kernels stream 8-aligned chunks
    and a ragged last one (the reference's LM vocab 50277 = 3 x 16759 is such a case).
    `shared`: one head tensor for both sides (a tied head), the bf16 passes' 128 x 256
    tiles."""
    from param_decomp_amd.losses import streamed_kl_per_position, streamed_position_kl

    rng = np.random.default_rng(n_chunks + V)
    N = 300 if dtype == torch.float32 else 512
    cast = (lambda a: f32(a, device)) if dtype == torch.float32 else (lambda a: bf(a, device))
    aq = cast(rng.normal(size=(N, d)) * 0.5).requires_grad_(True)
    ap = cast(rng.normal(size=(N, d)) * 0.5)
    hq = cast(rng.normal(size=(V, d)) * 0.3)
    hp = hq if shared else cast(rng.normal(size=(V, d)) * 0.3)
    kl = streamed_position_kl(aq, hq, ap, hp, n_chunks)
    want, _ = po.streamed_position_kl(np64(aq), np64(hq), np64(ap), np64(hp), n_chunks)
    if dtype == torch.float32:
        assert_close(np64(kl), want, 1e-4, 2e-6, "position kl")
    else:
        assert_close(np64(kl), want, 1e-3, 1e-4, "position kl bf16")
    g = rng.normal(size=N)
    (da,) = torch.autograd.grad(kl, aq, f32(g, device))
    want_da = po.streamed_position_kl_vjp(np64(aq), np64(hq), np64(ap), np64(hp), g)
    if dtype == torch.float32:
        assert_close(np64(da), want_da, 1e-4, 1e-5, "d act_masked")
    else:
        assert_close(np64(da), want_da, BF16_RTOL, 1e-2, "d act_masked bf16")
    mean = streamed_kl_per_position(aq, hq, ap, hp, n_chunks)
    assert float(mean) == pytest.approx(float(np.mean(want)), rel=1e-3)


# ------------------------------------------------------------------ strided-batched GEMM / blocked site


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("ta,tb,shared_a", [(0, 0, False), (1, 0, True), (0, 1, False), (1, 1, False)])
def test_gemm_strided_batched(device, dtype, ta, tb, shared_a):
    from param_decomp_amd import _lib as L

    rng = np.random.default_rng(ta * 4 + tb * 2 + int(shared_a))
    Bt, M, N, K = 5, 72, 40, 56
    cast = (lambda a: f32(a, device)) if dtype == torch.float32 else (lambda a: bf(a, device))
    A = cast(rng.normal(size=(1 if shared_a else Bt,) + ((K, M) if ta else (M, K))))
    B = cast(rng.normal(size=(Bt,) + ((N, K) if tb else (K, N))))
    C = torch.empty((Bt, M, N), dtype=torch.float32, device=device)
    lda = M if ta else K
    ldb = K if tb else N
    L.call("pd_gemm_strided_batched", L.dtype_code(dtype), Bt, M, N, K, L.ptr(A), lda, 0 if shared_a else M * K, ta,
           L.ptr(B), ldb, N * K, tb, L.ptr(C), N, M * N, L.F32, 1.0, 0.0, L.stream())
    a, b = np64(A), np64(B)
    a = np.broadcast_to(a, (Bt,) + a.shape[1:])
    want = np.einsum("zmk,zkn->zmn", np.swapaxes(a, 1, 2) if ta else a, np.swapaxes(b, 1, 2) if tb else b)
    assert_close(np64(C), want, 1e-5 if dtype == torch.float32 else 1e-5, 1e-6, "batched")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("contraction", ["fused_output", "fused_input"])
@pytest.mark.parametrize("with_delta_and_route", [False, True])
def test_blocked_site_forward_backward(device, dtype, contraction, with_delta_and_route):
    from param_decomp_amd.decomposed_linear import BlockedSiteWeights, blocked_site_forward

    rng = np.random.default_rng(2 + int(with_delta_and_route))
    E, d_in, d_out, c, T = 6, 32, 24, 16, 150
    site_in = d_in * (E if contraction == "fused_input" else 1)
    site_out = d_out * (E if contraction == "fused_output" else 1)
    cast = (lambda a: f32(a, device)) if dtype == torch.float32 else (lambda a: bf(a, device))
    x = cast(rng.normal(size=(T, site_in))).requires_grad_(True)
    V = cast(rng.normal(size=(E, d_in, c)) / np.sqrt(d_in)).requires_grad_(True)
    U = cast(rng.normal(size=(E, c, d_out)) / np.sqrt(E * c)).requires_grad_(True)
    W = cast(rng.normal(size=(site_out, site_in)) / np.sqrt(site_in))
    mask = cast(rng.uniform(size=(T, E * c))).requires_grad_(True)
    delta = cast(rng.uniform(size=T)).requires_grad_(True) if with_delta_and_route else None
    route = torch.tensor(rng.uniform(size=T) < 0.6, device=device) if with_delta_and_route else None
    sf = blocked_site_forward(x, BlockedSiteWeights(W, V, U), mask, delta, route, contraction)
    want_out, want_xv = po.blocked_site_forward(np64(x), np64(W), np64(V), np64(U), np64(mask),
                                                None if delta is None else np64(delta),
                                                None if route is None else route.cpu().numpy(), contraction)
    rt, fl = (1e-5, 1e-6) if dtype == torch.float32 else (BF16_RTOL, 4e-3)
    assert_close(np64(sf.output), want_out, rt, fl, "blocked out")
    assert_close(np64(sf.component_activation), want_xv, rt, fl, "blocked xV")
    G = rng.normal(size=want_out.shape)
    Gx = rng.normal(size=want_xv.shape) * 0.1
    dx, dV, dU, dm = torch.autograd.grad((sf.output, sf.component_activation), (x, V, U, mask),
                                         (cast(G), cast(Gx)))
    wdx, wdV, wdU, wdm = po.blocked_site_backward(np64(x), np64(W), np64(V), np64(U), np64(mask),
                                                  None if delta is None else np64(delta),
                                                  None if route is None else route.cpu().numpy(), contraction,
                                                  np64(cast(G)))
    gx = np64(cast(Gx))
    xe = np64(x) if contraction == "fused_output" else np64(x).reshape(T, E, d_in)
    gxe = gx.reshape(T, E, c)
    if contraction == "fused_output":
        wdV = wdV + np.einsum("ti,tej->eij", xe, gxe)
        wdx = wdx + np.einsum("tej,eij->ti", gxe, np64(V))
    else:
        wdV = wdV + np.einsum("tei,tej->eij", xe, gxe)
        wdx = wdx + np.einsum("tej,eij->tei", gxe, np64(V)).reshape(T, -1)
    rt, fl = (1e-4, 1e-5) if dtype == torch.float32 else (BF16_RTOL, 1e-2)
    for got, want, name in ((dx, wdx, "dx"), (dV, wdV, "dV"), (dU, wdU, "dU"), (dm, wdm, "dmask")):
        assert_close(np64(got), want, rt, fl, f"blocked {name}")
    if delta is not None:  # the weight-delta cotangent (delta sources of adversarial masking)
        (dd,) = torch.autograd.grad(
            blocked_site_forward(x, BlockedSiteWeights(W, V, U), mask, delta, route, contraction).output, (delta,),
            cast(G))
        want_dd = po.blocked_site_delta_grad(np64(x), np64(W), np64(V), np64(U), np64(mask), np64(delta),
                                             route.cpu().numpy(), contraction, np64(cast(G)))
        assert_close(np64(dd), want_dd, rt, fl, "blocked d_delta")
