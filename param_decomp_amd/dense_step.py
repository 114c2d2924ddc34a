"""The fused single-site stochastic-recon step (the dense hot path) on the GPU.

One call = one fwd+bwd of one decomposed linear whose input is the clean input:
clean target `x@W^T` (detached), inner activations `h = x@V`, paper-form gate on h,
lower/upper squashing, mask `m = lower + (1-lower)*u` with u drawn from the site's
mask key (`pd/core/masking.py:148-167` key chain), optional weight-delta channel,
`y = (h*(m-d))@U + d*(x@W^T)`, MSE recon, the imp-min term (L_p, or the engine's
smooth-L0 with its frequency penalty), and the gradients w.r.t. V, U
and the gate parameters (the gate reads `h = x@V` with V live, so dV carries both
pullbacks, as `pd/core/train.py:624-655` pulls the CI VJP back onto the components).

All buffers are allocated once at construction; `step()` only enqueues kernels.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from param_decomp_amd import _lib as L
from param_decomp_amd import prng
from param_decomp_amd.losses import ImpMin
from param_decomp_amd.prng import Key


@dataclass
class DenseStepGrads:
    dV: torch.Tensor  # [d_in, C] fp32
    dU: torch.Tensor  # [C, d_out] fp32
    dw_in: torch.Tensor
    db_in: torch.Tensor
    dw_out: torch.Tensor
    db_out: torch.Tensor
    losses: torch.Tensor  # [4] fp32: loss, recon, activity, frequency (+ the batch frequency with the EMA)


class DenseSiteStep:
    def __init__(self, T: int, d_in: int, d_out: int, C: int, *, dtype=torch.bfloat16, device="cuda", H: int = 16,
                 p: float = 2.0, imp_coeff: float = 1.0, recon_coeff: float = 1.0, use_delta: bool = False,
                 draw_dtype: torch.dtype | None = None, layout: int = L.LAYOUT_PARTITIONABLE,
                 imp_min: ImpMin | None = None):
        self.T, self.d_in, self.d_out, self.C, self.H = T, d_in, d_out, C, H
        self.dtype = dtype
        self.dt = L.dtype_code(dtype)
        self.draw = L.dtype_code(draw_dtype or dtype)
        self.layout = layout
        self.recon_coeff, self.use_delta = recon_coeff, use_delta
        # the imp-min term: L_p (p, imp_coeff) unless a smooth-L0 ImpMin is given
        self.imp_min = imp_min if imp_min is not None else ImpMin("pnorm", p=p, coeff=imp_coeff)
        dev = torch.device(device)
        f32 = dict(dtype=torch.float32, device=dev)
        # the EMA frequency estimate over the site's C components (None: the batch estimate)
        self.frequency = self.imp_min.new_estimate(C, dev)
        self.grads = DenseStepGrads(torch.empty(d_in, C, **f32), torch.empty(C, d_out, **f32), torch.empty(C, H, **f32),
                                    torch.empty(C, H, **f32), torch.empty(C, H, **f32), torch.empty(C, **f32),
                                    torch.empty(5 if self.frequency else 4, **f32))
        nbytes = L.load().pd_dense_step_workspace_size(self.dt, T, d_in, d_out, C, H)
        self.workspace = L.workspace(nbytes, dev)

    PHASES = ("delta_draw", "gemm_target", "gemm_xV", "gate_mask_fwd", "gemm_actsU", "recon", "loss_final",
              "gemm_dU", "gemm_da", "gate_mask_bwd", "gate_grad_reduce", "gemm_dV")

    def step(self, x, W, V, U, gate, mask_key: Key, delta_key: Key, *, events=None) -> DenseStepGrads:
        """`gate` is (w_in, b_in, w_out, b_out) fp32; keys are the site's folded keys.
        `events` (a ctypes array of len(PHASES)+1 hipEvent_t) records phase boundaries."""
        w_in, b_in, w_out, b_out = gate
        g = self.grads
        args = [self.dt, self.T, self.d_in, self.d_out, self.C, self.H, L.ptr(x), L.ptr(W), L.ptr(V), L.ptr(U),
                L.ptr(w_in), L.ptr(b_in), L.ptr(w_out), L.ptr(b_out), mask_key[0], mask_key[1], delta_key[0],
                delta_key[1], int(self.use_delta), self.draw, self.layout, *self.imp_min.c_args(self.frequency),
                self.recon_coeff,
                L.ptr(g.losses), L.ptr(g.dV), L.ptr(g.dU), L.ptr(g.dw_in), L.ptr(g.db_in), L.ptr(g.dw_out),
                L.ptr(g.db_out), L.ptr(self.workspace), self.workspace.numel(), L.stream()]
        if events is None:
            L.call("pd_dense_step", *args)
        else:
            L.call("pd_dense_step_timed", *args, events)
        if self.frequency is not None:
            self.frequency.count += 1
        return g

    @staticmethod
    def site_keys(draw_key: Key, site_idx: int = 0) -> tuple[Key, Key]:
        """`mask_key, delta_key = split(draw_key)`, each folded with the site index."""
        mk, dk = prng.split(draw_key)
        return prng.fold_in(mk, site_idx), prng.fold_in(dk, site_idx)
