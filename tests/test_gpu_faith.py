"""GPU parity of faithfulness (pd_faithfulness_fwd/bwd) against the oracle
(oracle/faith_oracle.py). fp32 arithmetic: losses, deltas and gradients within 1e-5 of
the float64 oracle (relative to the largest magnitude), the fp32 bound of the path."""

import numpy as np
import pytest
import torch

from oracle import faith_oracle as fo
from param_decomp_amd import faithfulness as F
from param_decomp_amd import ops

pytestmark = pytest.mark.gpu


def _t(a, dev, dtype=torch.float32):
    return torch.tensor(np.asarray(a, np.float32), device=dev).to(dtype)


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _rel(got, want):
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


CASES = [
    # (n_mats, per_site, d_in, d_out, C, W dtype)
    (1, 1, 96, 80, 40, torch.float32),        # ragged tiles, vector staging
    (3, 1, 256, 128, 160, torch.bfloat16),    # bf16 frozen weights
    (6, 3, 64, 48, 24, torch.float32),        # block-factored: 2 sites of 3 experts
    (1, 1, 5, 2, 20, torch.float32),          # TMS 5-2: scalar staging
    (2, 1, 130, 66, 7, torch.float32),        # odd C and widths
    (1, 1, 64, 64, 2048, torch.bfloat16),     # few tiles, long C: 4 k splits
    (1, 1, 30, 10, 1100, torch.float32),      # 2 k splits, ragged split, scalar delta pass
]


@pytest.mark.parametrize("n,per,d_in,d_out,C,wdt", CASES)
def test_faithfulness_matches_oracle(device, n, per, d_in, d_out, C, wdt):
    print(f"faith n={n} per={per} d_in={d_in} d_out={d_out} C={C} {wdt}", flush=True)
    rng = np.random.default_rng(n * 1000 + d_in + C)
    W = rng.normal(size=(n, d_out, d_in))
    V = rng.normal(size=(n, d_in, C)) / np.sqrt(d_in)
    U = rng.normal(size=(n, C, d_out)) / np.sqrt(C)
    Wt = _t(W, device, wdt)
    Wr = _np(Wt)
    norms = np.array([(Wr[s * per:(s + 1) * per] ** 2).sum() for s in range(n // per)])
    scale = 1.0 / 7
    Vt, Ut, nt = _t(V, device), _t(U, device), _t(norms, device)
    loss, site_err, delta = ops.faithfulness_fwd(Wt, Vt, Ut, nt, per, scale, keep_delta=True)
    g = torch.tensor([2.5], device=device)
    dV, dU = ops.faithfulness_bwd(delta, Vt, Ut, nt, per, scale, g)
    torch.cuda.synchronize()
    Vr, Ur, nr = _np(Vt), _np(Ut), _np(nt)
    want_delta = fo.weight_deltas(Wr, Vr, Ur)
    per_mat = (want_delta ** 2).reshape(n, -1).sum(1)
    want_site = per_mat.reshape(-1, per).sum(1) / nr
    assert _rel(_np(delta), want_delta) < 1e-5
    np.testing.assert_allclose(_np(site_err), want_site, rtol=1e-5)
    assert float(loss[0]) == pytest.approx(scale * want_site.sum(), rel=1e-5)
    mat_norms = np.repeat(nr, per)
    want_dV, want_dU = fo.grads(Wr, Vr, Ur, mat_norms, scale * 2.5)
    assert _rel(_np(dV), want_dV) < 1e-5
    assert _rel(_np(dU), want_dU) < 1e-5


def test_reference_hand_values_through_the_kernel(device):
    # pd/tests/core/test_faithfulness_normalization.py:47-55 on precomputed deltas
    loss = F.make_faithfulness_loss((("a", "g", 0), ("b", "g", 1), ("c", "h", 0)), {"g": (8.0, 16.0), "h": (2.0,)},
                                    {})
    deltas = {"g": torch.stack([torch.full((2, 2), 2.0), torch.full((2, 2), 1.0)]).to(device),
              "h": torch.full((1, 1, 4), 1.0, device=device)}
    assert float(loss.from_deltas(deltas)) == pytest.approx((16 / 8.0 + 4 / 16.0 + 4 / 2.0) / 3, rel=1e-6)


def test_bound_loss_autograd_over_dense_and_blocked_groups(device):
    rng = np.random.default_rng(5)
    dense = (rng.normal(size=(2, 24, 32)), rng.normal(size=(2, 32, 16)) / 6, rng.normal(size=(2, 16, 24)) / 4)
    blocked = (rng.normal(size=(1, 3, 8, 16)), rng.normal(size=(1, 3, 16, 8)) / 4, rng.normal(size=(1, 3, 8, 8)) / 3)
    norms = {"attn": tuple(float((dense[0][i] ** 2).sum()) for i in range(2)),
             "experts": (float((blocked[0] ** 2).sum()),)}
    idx = (("l0.q", "attn", 0), ("l1.q", "attn", 1), ("l0.experts", "experts", 0))
    loss_fn = F.make_faithfulness_loss(idx, norms, {})
    tens = {k: [_t(a, device) for a in v] for k, v in (("attn", dense), ("experts", blocked))}
    for k in tens:
        for a in tens[k][1:]:
            a.requires_grad_()
    loss = loss_fn({k: tuple(v) for k, v in tens.items()})
    (3.0 * loss).backward()
    deltas = {"attn": fo.weight_deltas(*dense), "experts": fo.weight_deltas(*blocked)}
    want = fo.loss_from_deltas(deltas, norms, 3)
    assert float(loss) == pytest.approx(want, rel=1e-5)
    dVa, dUa = fo.grads(*dense, np.array(norms["attn"]), 3.0 / 3)
    assert _rel(_np(tens["attn"][1].grad), dVa) < 1e-5
    assert _rel(_np(tens["attn"][2].grad), dUa) < 1e-5
    dVe, dUe = fo.grads(blocked[0][0], blocked[1][0], blocked[2][0], np.repeat(norms["experts"], 3), 3.0 / 3)
    assert _rel(_np(tens["experts"][1].grad)[0], dVe) < 1e-5
    assert _rel(_np(tens["experts"][2].grad)[0], dUe) < 1e-5


def test_faithfulness_is_deterministic_at_the_dense_site_shape(device):
    gen = torch.Generator(device=device).manual_seed(0)
    W = torch.randn(1, 3072, 768, device=device, generator=gen).to(torch.bfloat16)
    V = torch.randn(1, 768, 4096, device=device, generator=gen) / 768 ** 0.5
    U = torch.randn(1, 4096, 3072, device=device, generator=gen) / 64
    nt = (W.float() ** 2).sum().reshape(1)
    a = ops.faithfulness_fwd(W, V, U, nt, 1, 1.0, keep_delta=True)
    b = ops.faithfulness_fwd(W, V, U, nt, 1, 1.0, keep_delta=True)
    assert torch.equal(a[0], b[0]) and torch.equal(a[2], b[2])
    ga = ops.faithfulness_bwd(a[2], V, U, nt, 1, 1.0, None)
    gb = ops.faithfulness_bwd(b[2], V, U, nt, 1, 1.0, None)
    assert torch.equal(ga[0], gb[0]) and torch.equal(ga[1], gb[1])
    # a size-independent identity: sum Delta^2 / ||W||^2 recomputed from the kept deltas
    assert float(a[0][0]) == pytest.approx(float((a[2].double() ** 2).sum() / nt.double()), rel=1e-5)
