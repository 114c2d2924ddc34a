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
- `streamed_position_kl` / `streamed_kl_per_position` — the same KL over the factored
  lm-head edge, streamed over vocab chunks (`pd/targets/losses.py:101-170`).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from param_decomp_amd import _lib as L
from param_decomp_amd import ops


@dataclass(frozen=True)
class ImpMin:
    """The imp-min term of the fused steps (`pd_dense_step`, `pd_moe_stack_step`,
    `pd_lm_stack_step`). `kind="pnorm"`: `coeff * sum upper^p / n`. `kind="smooth_l0"`:
    the engine's `ImportanceMinimalityLoss` (`pd/core/configs.py:186-206`,
    `pd/core/objective.py:101-131`): `coeff * sum_c f_c + frequency_coeff * sum_c f_c
    log2(1 + reference_datapoint_count * f_c)` with `f_c = sum psi(upper) / n`,
    `psi = c^2 / (c^2 + gamma^2)` (times `1 + gamma^2` with `normalize_at_one`), the
    frequency term off when `reference_datapoint_count` is 0 (a single-batch estimate:
    the EMA estimator's state lives outside the step). gamma is the schedule's value
    at this step."""

    kind: str = "pnorm"
    p: float = 2.0
    coeff: float = 1.0
    gamma: float = 1.0
    normalize_at_one: bool = False
    frequency_coeff: float = 0.0
    reference_datapoint_count: float = 0.0

    @classmethod
    def smooth_l0(cls, coeff: float, gamma: float, *, normalize_at_one: bool = False, frequency_coeff: float = 0.0,
                  reference_datapoint_count: float = 0.0) -> "ImpMin":
        return cls("smooth_l0", 2.0, coeff, gamma, normalize_at_one, frequency_coeff, reference_datapoint_count)

    def c_args(self) -> list:
        """(kind, p, gamma, normalize_at_one, coeff, freq_coeff, ref_count) for the C ABI."""
        if self.kind not in ("pnorm", "smooth_l0"):
            raise L.PDError(f"ImpMin: unknown kind {self.kind!r}")
        kind = L.IMPMIN_SMOOTH_L0 if self.kind == "smooth_l0" else L.IMPMIN_PNORM
        return [kind, float(self.p), float(self.gamma), int(self.normalize_at_one), float(self.coeff),
                float(self.frequency_coeff), float(self.reference_datapoint_count)]


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
        # the gradient of each term at unit coefficient, scaled by the upstream device
        # scalar: no host read of g_act / g_freq, so the backward can be graph-captured
        grad = None
        for g, unit in ((g_act, dict(coeff_act=1.0, coeff_freq=0.0)), (g_freq, dict(coeff_act=0.0, coeff_freq=1.0))):
            if g is None or (unit["coeff_freq"] and ctx.kw["kind"] != L.IMPMIN_SMOOTH_L0):
                continue  # only the smooth-L0 form has a frequency term
            _, d = ops.impmin(ci.contiguous(), want_grad=True, **dict(ctx.kw, **unit))
            d = d * g.to(d.dtype)
            grad = d if grad is None else grad + d
        return (grad if grad is not None else torch.zeros_like(ci)), None


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


class _StreamedKL(torch.autograd.Function):
    @staticmethod
    def forward(ctx, act_masked, head_masked, act_clean, head_clean, n_chunks):
        N, d = act_masked.shape
        V = head_masked.shape[0]
        dt = L.dtype_code(act_masked.dtype)
        kl = torch.empty(N, dtype=torch.float32, device=act_masked.device)
        stats = torch.empty((N, 5), dtype=torch.float32, device=act_masked.device)
        ws = L.workspace(L.load().pd_streamed_kl_workspace_size(dt, N, d, V, n_chunks), act_masked.device)
        args = (dt, N, d, V, n_chunks, L.ptr(act_masked), L.ptr(head_masked), L.ptr(act_clean), L.ptr(head_clean))
        L.call("pd_streamed_kl_fwd", *args, L.ptr(kl), L.ptr(stats), L.ptr(ws), ws.numel(), L.stream())
        ctx.save_for_backward(act_masked, head_masked, act_clean, head_clean, stats)
        ctx.n_chunks = n_chunks
        return kl

    @staticmethod
    def backward(ctx, g):
        act_masked, head_masked, act_clean, head_clean, stats = ctx.saved_tensors
        N, d = act_masked.shape
        V = head_masked.shape[0]
        dt = L.dtype_code(act_masked.dtype)
        d_act = torch.empty((N, d), dtype=torch.float32, device=act_masked.device)
        ws = L.workspace(L.load().pd_streamed_kl_workspace_size(dt, N, d, V, ctx.n_chunks), act_masked.device)
        L.call("pd_streamed_kl_bwd", dt, N, d, V, ctx.n_chunks, L.ptr(act_masked), L.ptr(head_masked),
               L.ptr(act_clean), L.ptr(head_clean), L.ptr(stats), L.ptr(g.float().contiguous()), L.ptr(d_act),
               L.ptr(ws), ws.numel(), L.stream())
        return d_act.to(act_masked.dtype), None, None, None, None


def streamed_position_kl(act_masked: torch.Tensor, head_masked: torch.Tensor, act_clean: torch.Tensor,
                         head_clean: torch.Tensor, n_chunks: int) -> torch.Tensor:
    """Per-position KL(clean || masked) over the factored lm-head edge, streamed over
    `n_chunks` vocab chunks (`param_decomp/param_decomp/targets/losses.py:101-163`);
    differentiable w.r.t. the masked activations (the clean side is the target)."""
    lead = act_masked.shape[:-1]
    am = act_masked.reshape(-1, act_masked.shape[-1]).contiguous()
    ac = act_clean.detach().reshape(-1, act_clean.shape[-1]).contiguous()
    kl = _StreamedKL.apply(am, head_masked.detach().contiguous(), ac, head_clean.detach().contiguous(), int(n_chunks))
    return kl.reshape(lead)


def streamed_kl_per_position(act_masked, head_masked, act_clean, head_clean, n_chunks: int) -> torch.Tensor:
    """`streamed_kl_per_position` (`targets/losses.py:166-170`): the mean over positions."""
    return streamed_position_kl(act_masked, head_masked, act_clean, head_clean, n_chunks).mean()
