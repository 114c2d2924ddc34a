"""Routed sparse expert compute on the GPU: bucket -> grouped matmul -> unsort.

Mirrors `param_decomp/param_decomp/routed/experts.py:98-369` with one more
`GroupedMatmulBackend` arm, `"hip"` (the reference's only backend-dispatch seam,
`:70`): job j = (token j // k, slot j % k); `sort_idx` lists job ids grouped by expert
(stable, so token order survives inside an expert), `inv_sort_idx` is its inverse,
`group_sizes[e]` counts expert e's jobs. The gathers carry the reference's
inverse-gather VJPs; `grouped_matmul`'s backward is the transposed-rhs grouped matmul
(d_input) and the ragged-contracting `transposed_grouped_matmul` (d_weights).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Literal

import torch

from param_decomp_amd import ops

GroupedMatmulBackend = Literal["hip"]


@dataclass(frozen=True)
class RoutedJobs:
    top_idx: torch.Tensor  # [T, k] int32
    sort_idx: torch.Tensor  # [J] int32
    inv_sort_idx: torch.Tensor  # [J] int32
    group_sizes: torch.Tensor  # [E] int32
    group_offsets: torch.Tensor  # [E+1] int32 (exclusive prefix of group_sizes)

    @property
    def experts_per_token(self) -> int:
        return self.top_idx.shape[-1]


def routed_jobs(top_idx: torch.Tensor, n_experts: int) -> RoutedJobs:
    ti = top_idx.to(torch.int32).contiguous()
    sort_idx, inv, sizes, offsets = ops.routed_jobs(ti, n_experts)
    return RoutedJobs(ti, sort_idx, inv, sizes, offsets)


class _GatherTokens(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, sort_idx, inv, k):
        ctx.save_for_backward(inv)
        ctx.k = k
        return ops.gather_rows(x.contiguous(), sort_idx, k)

    @staticmethod
    def backward(ctx, g):
        (inv,) = ctx.saved_tensors
        T = inv.numel() // ctx.k
        return ops.combine_jobs(g.contiguous(), inv, None, T, ctx.k), None, None, None


class _PermuteRows(torch.autograd.Function):
    @staticmethod
    def forward(ctx, y, perm, inverse_perm):
        ctx.save_for_backward(inverse_perm)
        return ops.gather_rows(y.contiguous(), perm, 1)

    @staticmethod
    def backward(ctx, g):
        (inv,) = ctx.saved_tensors
        return ops.gather_rows(g.contiguous(), inv, 1), None, None


def gather_tokens(x: torch.Tensor, jobs: RoutedJobs) -> torch.Tensor:
    return _GatherTokens.apply(x, jobs.sort_idx, jobs.inv_sort_idx, jobs.experts_per_token)


def unsort_jobs(y: torch.Tensor, jobs: RoutedJobs) -> torch.Tensor:
    T, k = jobs.top_idx.shape
    return _PermuteRows.apply(y, jobs.inv_sort_idx, jobs.sort_idx).reshape(T, k, y.shape[-1])


def sort_jobs(values: torch.Tensor, jobs: RoutedJobs) -> torch.Tensor:
    return _PermuteRows.apply(values.reshape(-1, 1), jobs.sort_idx, jobs.inv_sort_idx).reshape(-1)


def sort_job_values(values: torch.Tensor, jobs: RoutedJobs) -> torch.Tensor:
    T, k = jobs.top_idx.shape
    return _PermuteRows.apply(values.reshape(T * k, -1), jobs.sort_idx, jobs.inv_sort_idx)


class _Combine(torch.autograd.Function):
    @staticmethod
    def forward(ctx, y, inv, sort_idx, weights, k):
        T = inv.numel() // k
        ctx.save_for_backward(sort_idx, inv, weights if weights is not None else torch.empty(0, device=y.device), y)
        ctx.k = k
        ctx.has_w = weights is not None
        return ops.combine_jobs(y.contiguous(), inv, None if weights is None else weights.float().contiguous(), T, k)

    @staticmethod
    def backward(ctx, g):
        sort_idx, inv, weights, y = ctx.saved_tensors
        k = ctx.k
        # d y[j] = w[job] * g[token(job)]: gather g rows by sort_idx // k, then scale
        gy = ops.gather_rows(g.contiguous(), sort_idx, k)
        dw = None
        if ctx.has_w:
            wj = weights.reshape(-1)[sort_idx.long()].to(gy.dtype)
            if ctx.needs_input_grad[3]:
                per = ops.gather_rows(y.contiguous(), inv, 1).float().reshape(-1, k, y.shape[-1])
                dw = (per * g.float()[:, None, :]).sum(-1)
            gy = gy * wj[:, None]
        return gy, None, None, dw, None


def sum_jobs(y: torch.Tensor, jobs: RoutedJobs) -> torch.Tensor:
    return _Combine.apply(y, jobs.inv_sort_idx, jobs.sort_idx, None, jobs.experts_per_token)


def combine_jobs(y: torch.Tensor, jobs: RoutedJobs, weights: torch.Tensor) -> torch.Tensor:
    return _Combine.apply(y, jobs.inv_sort_idx, jobs.sort_idx, weights, jobs.experts_per_token)


class _GroupedMatmul(torch.autograd.Function):
    @staticmethod
    def forward(ctx, lhs, rhs, offsets):
        ctx.save_for_backward(lhs, rhs, offsets)
        return ops.grouped_gemm(lhs.contiguous(), rhs.contiguous(), offsets)

    @staticmethod
    def backward(ctx, g):
        lhs, rhs, offsets = ctx.saved_tensors
        g = g.contiguous()
        d_lhs = ops.grouped_gemm(g, rhs.contiguous(), offsets, trans_rhs=True) if ctx.needs_input_grad[0] else None
        d_rhs = ops.grouped_gemm_dw(lhs.contiguous(), g, offsets, rhs.shape[0], out_dtype=rhs.dtype) \
            if ctx.needs_input_grad[1] else None
        return d_lhs, d_rhs, None


def grouped_matmul(lhs: torch.Tensor, rhs: torch.Tensor, jobs_or_offsets, backend: GroupedMatmulBackend = "hip"):
    """`lhs`'s e-th contiguous group of rows times `rhs[e]` (`rhs` is `[E, d_in, d_out]`)."""
    if backend != "hip":
        raise ValueError(f"unknown grouped-matmul backend {backend!r}")
    offsets = jobs_or_offsets.group_offsets if isinstance(jobs_or_offsets, RoutedJobs) else jobs_or_offsets
    return _GroupedMatmul.apply(lhs, rhs, offsets)


def transposed_grouped_matmul(lhs: torch.Tensor, dout: torch.Tensor, jobs_or_offsets, out_dtype=None):
    """`out[e] = lhs[block_e]^T @ dout[block_e]`; empty groups are exactly zero."""
    offsets = jobs_or_offsets.group_offsets if isinstance(jobs_or_offsets, RoutedJobs) else jobs_or_offsets
    return ops.grouped_gemm_dw(lhs.contiguous(), dout.contiguous(), offsets, offsets.numel() - 1, out_dtype=out_dtype)


def route_tokens(logits: torch.Tensor, k: int):
    """Softmax over experts (fp32), top-k descending with lowest index on ties, and the
    renormalized mixing weights (`pd/targets/qwen36_moe.py:473-514`). Returns
    (probs [T,E], top_idx [T,k] int32, weights [T,k] fp32)."""
    return ops.router_topk(logits.float().contiguous(), k)
