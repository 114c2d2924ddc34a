"""Importance-minimality and reconstruction losses on the GPU (fp32 accumulation).

Mirrors:
- `importance_minimality_terms(ci_upper, gamma, reference_datapoint_count,
  normalize_at_one)` — smooth-L0 activity `sum_sites sum_c mean psi(c)`,
  `psi = c^2/(c^2+gamma^2)`, and the frequency term `sum f log2(1 + a' f)`
  (`param_decomp/param_decomp/core/losses.py:357-485`).
- `EmaFrequency` / `init_frequency_estimator` — the frequency penalty at a debiased EMA
  estimate across steps (`pd/core/losses.py:425-458, 500-561`).
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
from typing import NamedTuple

import torch

from param_decomp_amd import _lib as L
from param_decomp_amd import ops


@dataclass(frozen=True)
class ImpMin:
    """The imp-min term of the fused steps (`pd_dense_step`, `pd_moe_stack_step`,
    `pd_lm_stack_step`). `kind="pnorm"`: `coeff * sum upper^p / n`. `kind="smooth_l0"`:
    the engine's `ImportanceMinimalityLoss` (`pd/core/configs.py:165-206`,
    `pd/core/objective.py:101-131`): `coeff * sum_c f_c + frequency_coeff * sum_c Phi(f_c)`,
    `Phi(f) = f log2(1 + reference_datapoint_count * f)`, with `f_c = sum psi(upper) / n`,
    `psi = c^2 / (c^2 + gamma^2)` (times `1 + gamma^2` with `normalize_at_one`), the
    frequency term off when `reference_datapoint_count` is 0. `ema_halflife_steps` (the
    frequency config's field, `pd/core/configs.py:182`) evaluates the frequency term at
    the debiased EMA estimate of `f_c` across steps (`pd/core/losses.py:425-458`); the
    step objects then keep that estimate (`StepFrequencyEstimate`) and advance it on
    every step. gamma is the schedule's value at this step."""

    kind: str = "pnorm"
    p: float = 2.0
    coeff: float = 1.0
    gamma: float = 1.0
    normalize_at_one: bool = False
    frequency_coeff: float = 0.0
    reference_datapoint_count: float = 0.0
    ema_halflife_steps: float | None = None

    @classmethod
    def smooth_l0(cls, coeff: float, gamma: float, *, normalize_at_one: bool = False, frequency_coeff: float = 0.0,
                  reference_datapoint_count: float = 0.0, ema_halflife_steps: float | None = None) -> "ImpMin":
        return cls("smooth_l0", 2.0, coeff, gamma, normalize_at_one, frequency_coeff, reference_datapoint_count,
                   ema_halflife_steps)

    @property
    def uses_ema(self) -> bool:
        return self.ema_halflife_steps is not None

    def new_estimate(self, n_components: int, device) -> "StepFrequencyEstimate | None":
        """The zero-initialized running estimate of a step with `n_components` components
        in all (`init_frequency_estimator`, `pd/core/losses.py:549-561`), or None without
        the EMA."""
        if not self.uses_ema:
            return None
        if self.kind != "smooth_l0" or not self.reference_datapoint_count > 0:
            raise L.PDError("ImpMin: the EMA estimate needs the smooth-L0 frequency term")
        if not 0.0 < float(self.ema_halflife_steps) <= 1e6:
            raise L.PDError("ImpMin: ema_halflife_steps must be in (0, 1e6]")
        return StepFrequencyEstimate(float(self.ema_halflife_steps),
                                     torch.zeros(int(n_components), dtype=torch.float32, device=device))

    def c_args(self, estimate: "StepFrequencyEstimate | None" = None) -> list:
        """(kind, p, gamma, normalize_at_one, coeff, freq_coeff, ref_count, freq_ema_in,
        freq_ema_out, ema_count, ema_halflife) for the C ABI; the estimate is updated in
        place by the call (advance its count afterwards)."""
        if self.kind not in ("pnorm", "smooth_l0"):
            raise L.PDError(f"ImpMin: unknown kind {self.kind!r}")
        kind = L.IMPMIN_SMOOTH_L0 if self.kind == "smooth_l0" else L.IMPMIN_PNORM
        base = [kind, float(self.p), float(self.gamma), int(self.normalize_at_one), float(self.coeff),
                float(self.frequency_coeff), float(self.reference_datapoint_count)]
        if estimate is None:
            return base + [None, None, 0.0, 0.0]
        return base + [L.ptr(estimate.values), L.ptr(estimate.values), float(estimate.count),
                       float(estimate.halflife_steps)]


@dataclass
class StepFrequencyEstimate:
    """A fused step's EMA frequency state (`EmaFrequency`, `pd/core/losses.py:522-543`):
    one fp32 vector over every component of the step's sites, in the layout of the step's
    entry point, and the number of earlier observations. Each step call reads and
    rewrites `values` on the device; `count` advances on the host."""

    halflife_steps: float
    values: torch.Tensor
    count: int = 0


class EmaFrequencyPenalty(NamedTuple):
    """`pd/core/losses.py:501-503`: the penalty at the smoothed estimate and the
    single-batch diagnostic."""

    value: torch.Tensor
    batch_value: torch.Tensor


class EmaFrequency:
    """The reference's `EmaFrequency` (`pd/core/losses.py:522-543`) over per-site fp32
    estimates: `evaluate_ci` computes each site's frequencies from its upper CI, returns
    the activity, the penalty `sum Phi(f_hat)` (gradient `Phi'(f_hat) df`, no gradient
    into the estimate) with its batch value, and the estimator after this observation."""

    def __init__(self, halflife_steps: float, estimate: dict, count: int = 0):
        if not 0.0 < float(halflife_steps) <= 1e6:
            raise L.PDError("EmaFrequency: halflife_steps must be in (0, 1e6]")
        self.halflife_steps = float(halflife_steps)
        self.estimate = dict(estimate)
        self.count = int(count)

    def evaluate_ci(self, ci_upper: dict, gamma: float, reference_datapoint_count: int, *,
                    normalize_at_one: bool) -> tuple[torch.Tensor, EmaFrequencyPenalty, "EmaFrequency"]:
        if not reference_datapoint_count or reference_datapoint_count <= 0:
            raise L.PDError("EmaFrequency: a positive reference_datapoint_count is required")
        act = freq = batch = None
        new = {}
        for name, v in ci_upper.items():
            kw = dict(kind=L.IMPMIN_SMOOTH_L0, gamma=float(gamma), normalize_at_one=normalize_at_one,
                      ref_count=float(reference_datapoint_count), ema=self.estimate[name].contiguous(),
                      ema_count=float(self.count), ema_halflife=self.halflife_steps)
            a, f, b, e = _ImpMin.apply(v, kw)
            new[name] = e
            act = a if act is None else act + a
            freq = f if freq is None else freq + f
            batch = b if batch is None else batch + b
        return act, EmaFrequencyPenalty(freq, batch), EmaFrequency(self.halflife_steps, new, self.count + 1)


def init_frequency_estimator(halflife_steps: float | None, sites: dict, device="cuda") -> EmaFrequency | None:
    """`pd/core/losses.py:549-561`: zero estimates per site (`sites`: name -> C), or None
    (the single-batch estimate) without a half-life."""
    if halflife_steps is None:
        return None
    return EmaFrequency(halflife_steps, {n: torch.zeros(int(C), dtype=torch.float32, device=device)
                                         for n, C in sites.items()})


class _ImpMin(torch.autograd.Function):
    """(activity, frequency, batch frequency, new EMA estimate) of one site; only the
    first two carry gradients. kw["ema"] (the estimate before this batch) switches the
    frequency term to the EMA estimate."""

    @staticmethod
    def forward(ctx, ci, kw):
        ema = kw.get("ema")
        new = torch.empty_like(ema) if ema is not None else None
        out, _ = ops.impmin(ci.contiguous(), ema_out=new, **kw)
        ctx.save_for_backward(ci)
        ctx.kw = kw
        if new is None:
            new = torch.zeros(0, dtype=torch.float32, device=ci.device)
        batch = out[2].clone()
        ctx.mark_non_differentiable(batch, new)
        return out[0], out[1], batch, new

    @staticmethod
    def backward(ctx, g_act, g_freq, g_batch, g_new):
        (ci,) = ctx.saved_tensors
        # each term's gradient at unit coefficient in fp32 (bf16 CI values are exact in
        # fp32, so the kernel's arithmetic is the same), scaled by the upstream device
        # scalar in fp32, summed in fp32 and rounded to the CI dtype once; no host read
        # of g_act / g_freq, so the backward can be graph-captured
        grad = None
        cif = ci.contiguous().float()
        for g, unit in ((g_act, dict(coeff_act=1.0, coeff_freq=0.0)), (g_freq, dict(coeff_act=0.0, coeff_freq=1.0))):
            if g is None or (unit["coeff_freq"] and ctx.kw["kind"] != L.IMPMIN_SMOOTH_L0):
                continue  # only the smooth-L0 form has a frequency term
            _, d = ops.impmin(cif, want_grad=True, **dict(ctx.kw, **unit))
            d = d * g.float()
            grad = d if grad is None else grad + d
        return (grad.to(ci.dtype) if grad is not None else torch.zeros_like(ci)), None


def importance_minimality_terms(ci_upper: dict, gamma: float, reference_datapoint_count: int | None, *,
                                normalize_at_one: bool) -> tuple[torch.Tensor, torch.Tensor]:
    act = None
    freq = None
    for v in ci_upper.values():
        kw = dict(kind=L.IMPMIN_SMOOTH_L0, gamma=float(gamma), normalize_at_one=normalize_at_one,
                  ref_count=float(reference_datapoint_count or 0))
        a, f, _, _ = _ImpMin.apply(v, kw)
        act = a if act is None else act + a
        freq = f if freq is None else freq + f
    return act, freq


def importance_minimality_pnorm(ci_upper: dict, p: float, *, eps: float = 0.0, beta: float = 0.0,
                                world_size: int = 1) -> torch.Tensor:
    total = None
    for v in ci_upper.values():
        kw = dict(kind=L.IMPMIN_PNORM, p=float(p), eps=float(eps), beta=float(beta), world_size=float(world_size))
        a, _, _, _ = _ImpMin.apply(v, kw)
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
