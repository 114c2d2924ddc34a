"""Target-relative parameter faithfulness on the GPU.

Mirrors `param_decomp/param_decomp/core/faithfulness.py:16-75` (`make_faithfulness_loss`:
the mean over sites of `||W_s - V_s U_s||^2_F / ||W_s||^2_F`) composed with the targets'
`weight_deltas` (`pd/targets/transformer.py:2134-2184`: fp32 `W - einsum("gic,gco->goi",
V, U)` per stack), as the train step calls them together
(`faithfulness(faithfulness_weight_deltas(model, c))`, `pd/core/train.py:1194-1196`).
`pd_faithfulness_fwd` forms the deltas inside a GEMM epilogue and reduces them; the
backward is two fp32 GEMMs against the kept deltas.

A stack is `(W, V, U)` with W `[g, d_out, d_in]` (bf16 or fp32 frozen weights), V fp32
`[g, d_in, C]`, U fp32 `[g, C, d_out]`, or the block-factored spelling W
`[g, expert, d_out, d_in]`, V `[g, expert, d_in, c]`, U `[g, expert, c, d_out]`, whose
blocks partition each site matrix.
"""

from __future__ import annotations

import math

import torch

from param_decomp_amd import ops


class _FaithFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, V, U, W, norms, per_site, scale):
        loss, _, delta = ops.faithfulness_fwd(W, V, U, norms, per_site, scale, keep_delta=True)
        ctx.save_for_backward(delta, V, U, norms)
        ctx.per_site, ctx.scale = per_site, scale
        return loss.reshape(())

    @staticmethod
    def backward(ctx, g):
        delta, V, U, norms = ctx.saved_tensors
        dV, dU = ops.faithfulness_bwd(delta, V, U, norms, ctx.per_site, ctx.scale,
                                      g.detach().float().reshape(1).contiguous())
        return dV, dU, None, None, None, None


def _flat_stack(W, V, U):
    """(W, V, U) as [n_mats, ...] matrices with the number of matrices per site."""
    if W.dim() == 3:
        return W.contiguous(), V.contiguous(), U.contiguous(), 1
    if W.dim() == 4:
        g, e = W.shape[:2]
        return (W.reshape(g * e, *W.shape[2:]).contiguous(), V.reshape(g * e, *V.shape[2:]).contiguous(),
                U.reshape(g * e, *U.shape[2:]).contiguous(), e)
    raise ValueError(f"a stack is [g, d_out, d_in] or [g, expert, d_out, d_in], got {tuple(W.shape)}")


class FaithfulnessLoss:
    """The bound loss: `__call__(stacks)` takes `{group: (W, V, U)}` and returns the scalar
    loss (fp32, differentiable in every V and U); `from_deltas(deltas)` takes precomputed
    fp32 deltas `{group: [g, ...]}`, the reference loss's own input."""

    def __init__(self, stack_names: dict, padded_sq_norms: dict, n_sites: int):
        self.stack_names = stack_names
        self.padded_sq_norms = padded_sq_norms
        self.n_sites = n_sites
        self._norm_tensors: dict = {}

    def _norms(self, group, device):
        key = (group, str(device))
        if key not in self._norm_tensors:
            self._norm_tensors[key] = torch.tensor(self.padded_sq_norms[group], dtype=torch.float32, device=device)
        return self._norm_tensors[key]

    def __call__(self, stacks: dict) -> torch.Tensor:
        if set(stacks) != set(self.padded_sq_norms):
            raise ValueError(f"stack groups {sorted(stacks)} != bound groups {sorted(self.padded_sq_norms)}")
        total = None
        for group in sorted(stacks):
            W, V, U, per_site = _flat_stack(*stacks[group])
            norms = self._norms(group, W.device)
            if W.shape[0] != per_site * norms.numel():
                raise ValueError(f"group {group}: {W.shape[0] // per_site} stack entries, {norms.numel()} norms")
            loss = _FaithFn.apply(V, U, W, norms, per_site, 1.0 / self.n_sites)
            total = loss if total is None else total + loss
        return total

    def from_deltas(self, deltas: dict) -> torch.Tensor:
        out = None
        for group in sorted(deltas):
            d = deltas[group].float()
            flat = d.reshape(d.shape[0] * (d.shape[1] if d.dim() == 4 else 1), *d.shape[-2:]).contiguous()
            per_site = d.shape[1] if d.dim() == 4 else 1
            n, d_out, d_in = flat.shape
            zV = torch.zeros((n, d_in, 1), dtype=torch.float32, device=d.device)
            zU = torch.zeros((n, 1, d_out), dtype=torch.float32, device=d.device)
            loss, _, _ = ops.faithfulness_fwd(flat, zV, zU, self._norms(group, d.device), per_site,
                                              1.0 / self.n_sites, keep_delta=False)
            out = loss[0] if out is None else out + loss[0]
        return out


def _names_by_stack(site_stack_indices) -> dict:
    """Per stack group, its site names in stack order. Each group's indices must count
    0, 1, 2, ... in the order the sites are listed."""
    names: dict = {}
    for name, group, index in site_stack_indices:
        seq = names.setdefault(group, [])
        if index != len(seq):
            raise AssertionError(f"stack {group!r}: site {name!r} has stack index {index}, expected {len(seq)}")
        seq.append(name)
    return names


def make_faithfulness_loss(site_stack_indices, target_sq_norms: dict, stack_pads: dict | None = None):
    """`pd/core/faithfulness.py:16-75`: validate and bind the per-stack-index `||W_s||^2`
    (finite and positive), pad persist-stack pads with 1.0 (their deltas are exactly
    zero), and average over the real sites. Bad inputs raise AssertionError, as the
    reference's checks do (its test matches the words "finite positive")."""
    pads = dict(stack_pads or {})
    names = _names_by_stack(site_stack_indices)
    if set(target_sq_norms) != set(names):
        raise AssertionError(f"||W||^2 stack groups {sorted(target_sq_norms)} differ from the sites' {sorted(names)}")
    for group, norms in target_sq_norms.items():
        values = [float(v) for v in norms]
        if len(values) != len(names[group]):
            raise AssertionError(f"stack {group!r}: {len(values)} norms for {len(names[group])} sites")
        invalid = {n: v for n, v in zip(names[group], values) if not (math.isfinite(v) and v > 0.0)}
        if invalid:
            raise AssertionError(f"each ||W_s||^2 must be a finite positive number; stack {group!r} has {invalid}")
    unknown = set(pads) - set(names)
    if unknown:
        raise AssertionError(f"pads for unknown stack groups {sorted(unknown)}")
    padded = {group: tuple(float(v) for v in norms) + (1.0,) * int(pads.get(group, 0))
              for group, norms in target_sq_norms.items()}
    return FaithfulnessLoss(names, padded, len(site_stack_indices))
