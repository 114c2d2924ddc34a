"""Stochastic masks drawn on the GPU from JAX-compatible threefry keys.

Mirrors `param_decomp/param_decomp/core/masking.py:135-171` and `uniform_like`
(`core/linear_plan.py:80-106`):
- `uniform_like(key, reference, drop_last_axis, dtype)`: `jax.random.uniform` in the
  reference's shape and dtype (bf16 and fp32 draws from one key are different samples).
- `sample_component_mask(ci, key)`: `m = ci + (1 - ci) * uniform_like(key, ci)`; the
  VJP w.r.t. ci is `g * (1 - u)` with u regenerated from the key, never stored.
- `sample_delta_mask(ci, key)`: one uniform per leading position.
- `materialize_masking(ci_lower, draw_key)`: `mask_key, delta_key = split(draw_key)`,
  then `fold_in(., site_idx)` in the CI mapping's insertion order.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from param_decomp_amd import _lib as L
from param_decomp_amd import ops, prng
from param_decomp_amd.prng import Key

LAYOUT = L.LAYOUT_PARTITIONABLE


def uniform_like(key: Key, reference: torch.Tensor, *, drop_last_axis: bool = False,
                 dtype: torch.dtype | None = None) -> torch.Tensor:
    shape = reference.shape[:-1] if drop_last_axis else reference.shape
    dt = dtype or reference.dtype
    return ops.uniform(key, shape, dt, reference.device, layout=LAYOUT)


class _ComponentMask(torch.autograd.Function):
    @staticmethod
    def forward(ctx, ci, key):
        ctx.key = key
        ctx.draw_dtype = ci.dtype
        return ops.component_mask_fwd(ci.contiguous(), key, ci.dtype, LAYOUT)

    @staticmethod
    def backward(ctx, g):
        return ops.component_mask_bwd(g.contiguous(), ctx.key, ctx.draw_dtype, LAYOUT), None


def sample_component_mask(ci: torch.Tensor, key) -> torch.Tensor:
    """`key`: a host pair, or a device tensor of two 32-bit words that the mask kernels read
    when they run (what a captured graph rewrites before each replay)."""
    return _ComponentMask.apply(ci, key if isinstance(key, torch.Tensor) else (int(key[0]), int(key[1])))


def sample_delta_mask(ci: torch.Tensor, key: Key) -> torch.Tensor:
    return uniform_like(key, ci, drop_last_axis=True)


@dataclass
class MaterializedMasking:
    component_masks: dict = field(default_factory=dict)
    weight_delta_masks: dict | None = None


def materialize_masking(ci_lower: dict, draw_key: Key) -> MaterializedMasking:
    mask_key, delta_key = prng.split(draw_key)
    masks, deltas = {}, {}
    for site_idx, (site, ci) in enumerate(ci_lower.items()):
        masks[site] = sample_component_mask(ci, prng.fold_in(mask_key, site_idx))
        deltas[site] = sample_delta_mask(ci, prng.fold_in(delta_key, site_idx))
    return MaterializedMasking(component_masks=masks, weight_delta_masks=deltas)
