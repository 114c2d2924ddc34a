"""Importance-minimality and reconstruction losses on the GPU (fp32 accumulation).

Mirrors:
- `importance_minimality_terms(ci_upper, gamma, reference_datapoint_count,
  normalize_at_one)` — smooth-L0 activity `sum_sites sum_c mean psi(c)`,
  `psi = c^2/(c^2+gamma^2)`, and the frequency term `sum f log2(1 + a' f)`
  (`param_decomp/param_decomp/core/losses.py:357-485`).
- `importance_minimality_pnorm(ci_upper, p, eps, beta, world_size)` — the L_p form of the
  SPD paper (algorithm step 4) with the `eps`/`beta` extension of
  `nano_param_decomp/run.py:413-429`.
- `mse(masked, clean)` — `pd/targets/tms.py:380-388`, `pd/targets/resid_mlp.py:411-418`.
- `categorical_kl_from_logits(masked, clean)` — KL(clean || masked) per position,
  clean frozen (`pd/core/losses.py:80-92`).
"""

from __future__ import annotations

import torch

from param_decomp_amd import _lib as L
from param_decomp_amd import ops


class _ImpMin(torch.autograd.Function):
    @staticmethod
    def forward(ctx, ci, kw):
        out, _ = ops.impmin(ci.contiguous(), **kw)
        ctx.save_for_backward(ci)
        ctx.kw = kw
        return out[0], out[1]

    @staticmethod
    def backward(ctx, g_act, g_freq):
        (ci,) = ctx.saved_tensors
        kw = dict(ctx.kw)
        # device scalars -> host coefficients (the backward is outside the hot loop of
        # the fused steps, which call the C ABI directly)
        kw["coeff_act"] = float(g_act) if g_act is not None else 0.0
        kw["coeff_freq"] = float(g_freq) if g_freq is not None else 0.0
        _, grad = ops.impmin(ci.contiguous(), want_grad=True, **kw)
        return grad, None


def importance_minimality_terms(ci_upper: dict, gamma: float, reference_datapoint_count: int | None, *,
                                normalize_at_one: bool) -> tuple[torch.Tensor, torch.Tensor]:
    act = None
    freq = None
    for v in ci_upper.values():
        kw = dict(kind=L.IMPMIN_SMOOTH_L0, gamma=float(gamma), normalize_at_one=normalize_at_one,
                  ref_count=float(reference_datapoint_count or 0))
        a, f = _ImpMin.apply(v, kw)
        act = a if act is None else act + a
        freq = f if freq is None else freq + f
    return act, freq


def importance_minimality_pnorm(ci_upper: dict, p: float, *, eps: float = 0.0, beta: float = 0.0,
                                world_size: int = 1) -> torch.Tensor:
    total = None
    for v in ci_upper.values():
        kw = dict(kind=L.IMPMIN_PNORM, p=float(p), eps=float(eps), beta=float(beta), world_size=float(world_size))
        a, _ = _ImpMin.apply(v, kw)
        total = a if total is None else total + a
    return total


class _MSE(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a, b):
        out, grad = ops.mse(a.contiguous(), b.contiguous(), want_grad=True)
        ctx.save_for_backward(grad)
        return out[0]

    @staticmethod
    def backward(ctx, g):
        (grad,) = ctx.saved_tensors
        return grad * g.to(grad.dtype), None


def mse(masked: torch.Tensor, clean: torch.Tensor) -> torch.Tensor:
    return _MSE.apply(masked, clean.detach())


class _KL(torch.autograd.Function):
    @staticmethod
    def forward(ctx, masked, clean):
        out, grad = ops.kl(masked.contiguous(), clean.contiguous(), want_grad=True)
        ctx.save_for_backward(grad)
        return out[0]

    @staticmethod
    def backward(ctx, g):
        (grad,) = ctx.saved_tensors
        return grad * g.to(grad.dtype), None


def categorical_kl_from_logits(masked_logits: torch.Tensor, clean_logits: torch.Tensor) -> torch.Tensor:
    return _KL.apply(masked_logits, clean_logits.detach())
