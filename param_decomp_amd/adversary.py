"""Adversarial sources on the GPU: persistent PGD (warmup ascents and the final ascent)
and fresh PGD sign ascents.

Mirrors `param_decomp/param_decomp/core/adversary.py`:
- source storage `float32` / `bfloat16` / `uint16` (`u / 65535`, stored back with
  unbiased stochastic rounding; `:150-214`), `source_values_to_float`, `velocity_dtype`;
- the source optimizers `AdamPGDConfig`, `SgdPGDConfig`, `MomentumSgdPGDConfig`
  (`pd/core/configs.py:347-375`) and their projected ascents (`:392-470`);
- `PersistentAdversary.warmup_ascend` / `after_one_ascent` / `final_ascend` (`:487-560`);
- fresh PGD's sign ascent (`pd/core/train.py:788-800`);
and the source masks `ci + (1 - ci) s` (`pd/core/source_mask.py:56-63`).

A source tensor is `[n_sources, C]`; each source row covers `rows_per_source`
consecutive CI rows (`bsc`: 1, `bc`: the positions of a sample, `c`: every row).
`DenseSitePPGDStep` runs the persistent-PGD step of one dense site through the
masked-linear kernels: `n_warmup` source ascents on the detached reconstruction loss,
then the final reconstruction (model gradients) whose source gradient makes the final
ascent (`pd/core/train.py:693-811`).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from param_decomp_amd import _lib as L
from param_decomp_amd import ops, prng

UINT16_UNIT_SCALE = 65535.0


@dataclass(frozen=True)
class AdamPGDConfig:
    beta1: float = 0.9
    beta2: float = 0.999
    eps: float = 1e-8


@dataclass(frozen=True)
class SgdPGDConfig:
    pass


@dataclass(frozen=True)
class MomentumSgdPGDConfig:
    momentum: float = 0.9


def velocity_dtype(storage: torch.dtype) -> torch.dtype:
    """fp32 velocity for fp32 sources, bf16 for either 16-bit storage (`:270-274`)."""
    return torch.float32 if storage == torch.float32 else torch.bfloat16


def store_unit_float(value: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Init-time store of [0, 1] values: uint16 rounds to nearest, floats cast (`:159-168`)."""
    if dtype == torch.uint16:
        return torch.round(value.float() * UINT16_UNIT_SCALE).to(torch.int32).to(torch.uint16)
    return value.to(dtype)


def source_values_to_float(sources: torch.Tensor) -> torch.Tensor:
    """The float view: uint16 dequantizes to fp32 `u / 65535`; floats pass through."""
    if sources.dtype == torch.uint16:
        return sources.to(torch.int32).float() / UINT16_UNIT_SCALE
    return sources


def source_mask(ci: torch.Tensor, sources: torch.Tensor, rows_per_source: int) -> torch.Tensor:
    return ops.source_mask_fwd(ci.contiguous(), sources, rows_per_source)


def source_mask_grad(g_mask, ci, sources, rows_per_source: int, want_dci: bool = False):
    """(d_sources fp32, d_ci): the pullback of `source_mask`."""
    return ops.source_mask_bwd(g_mask.contiguous(), ci.contiguous(), sources, rows_per_source, want_dci)


class PersistentAdversary:
    """Persistent sources, optimizer state and ascent configuration of one source leaf."""

    def __init__(self, sources: torch.Tensor, optimizer, n_warmup: int, rows_per_source: int, leaf_index: int = 0):
        if isinstance(optimizer, AdamPGDConfig) and sources.dtype == torch.uint16:
            raise ValueError("uint16 fixed-point source storage pairs with source optimizer sgd/momentum_sgd; "
                             "adam stores its moments at the source dtype")
        self.sources = sources.contiguous()
        self.optimizer = optimizer
        self.n_warmup = n_warmup
        self.rows_per_source = rows_per_source
        self.leaf_index = leaf_index
        self.step_count = 0.0
        self.state_a = self.state_b = None
        if isinstance(optimizer, AdamPGDConfig):
            self.state_a = torch.zeros_like(self.sources)
            self.state_b = torch.zeros_like(self.sources)
        elif isinstance(optimizer, MomentumSgdPGDConfig):
            self.state_a = torch.zeros(self.sources.shape, dtype=velocity_dtype(self.sources.dtype),
                                       device=self.sources.device)

    @property
    def float_sources(self) -> torch.Tensor:
        return source_values_to_float(self.sources)

    def mask(self, ci: torch.Tensor) -> torch.Tensor:
        return source_mask(ci, self.sources, self.rows_per_source)

    def after_one_ascent(self, grad: torch.Tensor, lr: float, key) -> "PersistentAdversary":
        """One projected ascent along the float-view gradient; `key` is the ascent's key,
        folded with this leaf's index for the uint16 rounding draw (`:197-214`)."""
        opt = self.optimizer
        leaf_key = prng.fold_in(key, self.leaf_index)
        if isinstance(opt, AdamPGDConfig):
            self.step_count += 1.0
            ops.source_ascend(L.PGD_ADAM, self.sources, grad.contiguous(), self.state_a, self.state_b,
                              step_count=self.step_count, lr=lr, beta1=opt.beta1, beta2=opt.beta2, eps=opt.eps,
                              key=leaf_key)
        elif isinstance(opt, MomentumSgdPGDConfig):
            ops.source_ascend(L.PGD_MOMENTUM, self.sources, grad.contiguous(), self.state_a, lr=lr,
                              momentum=opt.momentum, key=leaf_key)
        else:
            ops.source_ascend(L.PGD_SGD, self.sources, grad.contiguous(), lr=lr, key=leaf_key)
        return self

    def warmup_ascend(self, scoring_grad, lr: float, key) -> "PersistentAdversary":
        """`n_warmup` projected ascents; `scoring_grad(self)` returns the source gradient of
        the detached reconstruction loss at the current sources (`:519-539`)."""
        for ascent_key in prng.split(key, self.n_warmup) if self.n_warmup else []:
            self.after_one_ascent(scoring_grad(self), lr, ascent_key)
        return self

    final_ascend = after_one_ascent


def fresh_pgd_ascend(sources: torch.Tensor, grad: torch.Tensor, step_size: float) -> torch.Tensor:
    """`clip(s + step_size * sign(g), 0, 1)` in place (fp32 sources)."""
    return ops.source_ascend(L.PGD_SIGN, sources, grad.contiguous(), lr=step_size)


@dataclass
class PPGDStepResult:
    loss: torch.Tensor  # fp32 [1], the final reconstruction loss
    dV: torch.Tensor
    dU: torch.Tensor
    d_ci: torch.Tensor
    warmup_losses: list


class DenseSitePPGDStep:
    """The persistent-PGD reconstruction step of one dense site (bf16 compute):
    `n_warmup` ascents of the adversary on `mse(site(x, m(s)), target)` with the model
    detached (only the mask gradient is formed), then the final forward whose backward
    gives dV, dU, the CI gradient and the source gradient of the final ascent. The loss and
    gradients are the unscaled term's: the term coefficient scales only the model side
    when the caller assembles the objective, so the sources ascend even at coefficient 0
    (pd/core/adversary.py:553-560).

    `delta_adversary` adds the explicit weight-delta source of the site
    (`SiteSource.delta`, pd/core/adversary.py:74-82): one value per token group, `[n_sources,
    1]` with the components' `rows_per_source`, read as the site's delta mask
    (`SourceMaskIngredients.delta_mask`, pd/core/source_mask.py:61-63), so the site output
    becomes `(xV (m - d)) @ U + d (x @ W^T)`. It is the next leaf after the components
    (`SourceStack` field order), so its uint16 rounding draws fold in `leaf_index + 1`.
    The delta values are formed by the source-mask kernel at ci = 0 (`0 + (1 - 0) s = s`),
    and their gradient is that kernel's pullback of the masked linear's delta cotangent."""

    def __init__(self, adversary: PersistentAdversary, delta_adversary: PersistentAdversary | None = None):
        self.adv = adversary
        self.dadv = delta_adversary
        if delta_adversary is not None:
            if delta_adversary.rows_per_source != adversary.rows_per_source or delta_adversary.n_warmup != adversary.n_warmup:
                raise ValueError("delta sources share the component sources' shape and warmup count")
            if delta_adversary.sources.shape[-1] != 1:
                raise ValueError("delta sources are [n_sources, 1]: one value per token group")

    def _delta(self, zeros):
        return None if self.dadv is None else source_mask(zeros, self.dadv.sources, self.dadv.rows_per_source)

    def _grads(self, x, V, U, W, ci, target, zeros, *, final: bool):
        mask = self.adv.mask(ci)
        d = self._delta(zeros)
        dvec = None if d is None else d.reshape(-1)
        out, xV, acts = ops.masked_linear_fwd(x, V, U, mask, W=W, delta=dvec)
        loss, g_out = ops.mse(out, target, 1.0, want_grad=True)
        _, dV, dU, dm, dd = ops.masked_linear_bwd(x, V, U, mask, xV, acts, g_out, W=W, delta=dvec, want_dvu=final,
                                                  want_ddelta=d is not None)
        d_src, d_ci = source_mask_grad(dm, ci, self.adv.sources, self.adv.rows_per_source, want_dci=final)
        d_dsrc = None
        if d is not None:
            d_dsrc, _ = source_mask_grad(dd.reshape(-1, 1), zeros, self.dadv.sources, self.dadv.rows_per_source)
        return loss, dV, dU, d_ci, d_src, d_dsrc

    def _ascend(self, d_src, d_dsrc, lr, key):
        self.adv.after_one_ascent(d_src, lr, key)
        if self.dadv is not None:
            self.dadv.after_one_ascent(d_dsrc, lr, key)

    def step(self, x, V, U, ci, target, lr: float, key, adv_index: int = 0, W=None) -> PPGDStepResult:
        """`key` is the step's adversary key: the warmup ascents take
        fold_in(fold_in(key, 0x51C), adv_index) (pd/core/train.py:746-753) and the final
        ascent fold_in(fold_in(fold_in(key, 0x51C), 0x51D), adv_index) (:1004-1007, 1291).
        W [d_out, d_in] is the site's target weight, needed with delta sources."""
        if self.dadv is not None and W is None:
            raise ValueError("delta sources need the site's target weight W")
        quantize_key = prng.fold_in(key, 0x51C)
        warm_key = prng.fold_in(quantize_key, adv_index)
        final_key = prng.fold_in(prng.fold_in(quantize_key, 0x51D), adv_index)
        zeros = None
        if self.dadv is not None:
            zeros = torch.zeros((ci.shape[0], 1), dtype=ci.dtype, device=ci.device)
        warmup_losses = []
        n = self.adv.n_warmup
        for ascent_key in prng.split(warm_key, n) if n else []:
            loss, _, _, _, d_src, d_dsrc = self._grads(x, V, U, W, ci, target, zeros, final=False)
            warmup_losses.append(loss)
            self._ascend(d_src, d_dsrc, lr, ascent_key)
        loss, dV, dU, d_ci, d_src, d_dsrc = self._grads(x, V, U, W, ci, target, zeros, final=True)
        self._ascend(d_src, d_dsrc, lr, final_key)
        return PPGDStepResult(loss=loss, dV=dV, dU=dU, d_ci=d_ci, warmup_losses=warmup_losses)


class MoEPPGDStep:
    """The persistent-PGD reconstruction step over every expert site of the MoE stack
    (`pd/core/train.py:693-811`, `pd/core/adversary.py:463-567`, the source-masking arm of
    `pd/targets/qwen36_moe.py:2151-2163`), on `pd_moe_stack_step_sources`: `n_warmup`
    ascents of the adversary on the detached reconstruction loss (only the source
    gradients are formed), then the final step, whose backward gives the model and CI
    gradients and the source gradients of the final ascent.

    `adversary.sources` is the stacked component-source leaf [L, 3, S, E, c] (sites gate,
    up, down; every row covering `step.rows_per_source` tokens), `delta_adversary.sources`
    the delta leaf [L, 3, S] (the next leaf, so its uint16 rounding draws fold in
    `leaf_index + 1`). Keys as `DenseSitePPGDStep.step`."""

    def __init__(self, step, adversary: PersistentAdversary, delta_adversary: PersistentAdversary | None = None):
        self.step_fn = step
        self.adv = adversary
        self.dadv = delta_adversary
        if step.rows_per_source is None:
            raise ValueError("the MoE step must be constructed with rows_per_source")
        if delta_adversary is not None and delta_adversary.n_warmup != adversary.n_warmup:
            raise ValueError("delta sources share the component sources' warmup count")

    def _run(self, x0, w, ci_pre, final: bool, reuse_clean: bool):
        self.step_fn.step_sources(x0, w, ci_pre, self.adv.sources, None if self.dadv is None else self.dadv.sources,
                                  want_weight_grads=final, reuse_clean=reuse_clean)
        return self.step_fn.losses[0].clone()

    def _ascend(self, lr, key):
        self.adv.after_one_ascent(self.step_fn.d_src, lr, key)
        if self.dadv is not None:
            self.dadv.after_one_ascent(self.step_fn.d_src_delta, lr, key)

    def step(self, x0, w, ci_pre, lr: float, key, adv_index: int = 0) -> PPGDStepResult:
        quantize_key = prng.fold_in(key, 0x51C)
        warm_key = prng.fold_in(quantize_key, adv_index)
        final_key = prng.fold_in(prng.fold_in(quantize_key, 0x51D), adv_index)
        warmup_losses = []
        n = self.adv.n_warmup
        # the frozen clean pass depends only on x0 and the frozen weights: the first call of
        # the step forms it, the later ones reuse it from the step's workspace
        for i, ascent_key in enumerate(prng.split(warm_key, n) if n else []):
            warmup_losses.append(self._run(x0, w, ci_pre, final=False, reuse_clean=i > 0))
            self._ascend(lr, ascent_key)
        loss = self._run(x0, w, ci_pre, final=True, reuse_clean=n > 0)
        self._ascend(lr, final_key)
        s = self.step_fn
        return PPGDStepResult(loss=loss, dV=s.dV, dU=s.dU, d_ci=s.d_ci_pre, warmup_losses=warmup_losses)


class LMPPGDStep:
    """The persistent-PGD reconstruction step over every decomposed matrix of the LM stack
    (`pd/core/train.py:693-811`, `pd/core/adversary.py:463-567`), on
    `pd_lm_stack_step_sources`: `n_warmup` ascents of the adversary on the detached KL
    reconstruction loss (only the source gradients are formed), then the final step, whose
    backward gives the model and CI gradients and the source gradients of the final ascent.

    `adversaries[kind].sources` is that kind's component-source leaf [L, S, C_kind] (every
    row covering `step.rows_per_source` tokens of the [B*T] order), `delta_adversary.sources`
    the delta leaf [L, 6, S]; each leaf folds its own `leaf_index` into the uint16 rounding
    draws. A pooled adversary (one particle per sample drawn from a pool,
    `pd/core/masking.py:221-257`) gathers its drawn particles into `bc` tables (rows of T
    tokens) before the step and scatters the gradients back. Keys as
    `DenseSitePPGDStep.step`."""

    def __init__(self, step, adversaries: dict, delta_adversary: PersistentAdversary | None = None):
        from param_decomp_amd.lm_step import KINDS

        self.step_fn = step
        self.kinds = KINDS
        self.adv = {k: adversaries[k] for k in KINDS}
        self.dadv = delta_adversary
        if step.rows_per_source is None:
            raise ValueError("the LM step must be constructed with rows_per_source")
        counts = {a.n_warmup for a in self.adv.values()} | ({delta_adversary.n_warmup} if delta_adversary else set())
        if len(counts) != 1:
            raise ValueError("every source leaf of the step shares one warmup count")
        self.n_warmup = counts.pop()

    def _run(self, tokens, w, ci_pre, final: bool, reuse_clean: bool):
        self.step_fn.step_sources(tokens, w, ci_pre, {k: a.sources for k, a in self.adv.items()},
                                  None if self.dadv is None else self.dadv.sources, want_weight_grads=final,
                                  reuse_clean=reuse_clean)
        return self.step_fn.losses[0].clone()

    def _ascend(self, lr, key):
        for k, a in self.adv.items():
            a.after_one_ascent(self.step_fn.d_src[k], lr, key)
        if self.dadv is not None:
            self.dadv.after_one_ascent(self.step_fn.d_src_delta, lr, key)

    def step(self, tokens, w, ci_pre, lr: float, key, adv_index: int = 0) -> PPGDStepResult:
        quantize_key = prng.fold_in(key, 0x51C)
        warm_key = prng.fold_in(quantize_key, adv_index)
        final_key = prng.fold_in(prng.fold_in(quantize_key, 0x51D), adv_index)
        warmup_losses = []
        n = self.n_warmup
        # the frozen forward depends only on the tokens and the frozen weights: the first
        # call of the step forms it, the later ones reuse it from the step's workspace
        for i, ascent_key in enumerate(prng.split(warm_key, n) if n else []):
            warmup_losses.append(self._run(tokens, w, ci_pre, final=False, reuse_clean=i > 0))
            self._ascend(lr, ascent_key)
        loss = self._run(tokens, w, ci_pre, final=True, reuse_clean=n > 0)
        self._ascend(lr, final_key)
        s = self.step_fn
        return PPGDStepResult(loss=loss, dV=s.dV, dU=s.dU, d_ci=s.d_ci_pre, warmup_losses=warmup_losses)
