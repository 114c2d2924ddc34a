"""CI squashings with their gradient rules, on the GPU.

Mirrors `param_decomp/param_decomp/core/ci_fn/squashing.py:8-45` and
`CI.from_preactivations` (`core/ci_fn/interface.py:35-41`):
- `lower_leaky_hard_sigmoid`: forward `clip(x, 0, 1)`; custom VJP leaks `0.01*g` below
  zero only for `g < 0`, passes `g` on (0, 1], blocks above 1.
- `upper_leaky_hard_sigmoid`: `x > 1 ? 1 + 0.01(x-1) : clip(x, 0, 1)` with the plain
  autodiff VJP (half the cotangent at the exact clip ties x == 0 and x == 1).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from param_decomp_amd import ops


class _Lower(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        ctx.save_for_backward(x)
        return ops.squash_fwd(x.contiguous(), lower=True, upper=False)[0]

    @staticmethod
    def backward(ctx, g):
        (x,) = ctx.saved_tensors
        return ops.squash_bwd(x.contiguous(), g.contiguous(), None)


class _Upper(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        ctx.save_for_backward(x)
        return ops.squash_fwd(x.contiguous(), lower=False, upper=True)[1]

    @staticmethod
    def backward(ctx, g):
        (x,) = ctx.saved_tensors
        return ops.squash_bwd(x.contiguous(), None, g.contiguous())


def lower_leaky_hard_sigmoid(x: torch.Tensor) -> torch.Tensor:
    return _Lower.apply(x)


def upper_leaky_hard_sigmoid(x: torch.Tensor) -> torch.Tensor:
    return _Upper.apply(x)


@dataclass(frozen=True)
class CI:
    """The CI fn output: raw preactivations and both squashings, keyed by site."""

    preactivations: dict
    lower: dict
    upper: dict

    @staticmethod
    def from_preactivations(preactivations) -> "CI":
        pre = dict(preactivations)
        return CI(
            preactivations=pre,
            lower={k: lower_leaky_hard_sigmoid(v) for k, v in pre.items()},
            upper={k: upper_leaky_hard_sigmoid(v) for k, v in pre.items()},
        )
