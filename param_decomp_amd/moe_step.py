"""The decomposed MoE stack step (the routed-expert hot path end to end) on the GPU.

One call = the clean forward on the frozen experts (pinning each layer's expert
indices), the masked forward with every routed expert matrix decomposed (with the
frozen delta channel the reference's stochastic masking draws, unless `use_delta` is
off), MSE recon of
the final residual + the imp-min term over the selected CI (L_p or the engine's
smooth-L0 with its frequency penalty), and the full backward to the
V/U factors of every site and to the CI preactivations. See `pd_moe_stack_step` in
include/pd_mi355x.h for the reference citations and layouts.

All buffers are allocated once at construction; `step()` only enqueues kernels.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from param_decomp_amd import _lib as L
from param_decomp_amd.losses import ImpMin
from param_decomp_amd.prng import Key

SITE_NAMES = ("gate", "up", "down")
CATEGORIES = ("clean_fwd", "norm_route", "gemm_fwd", "mask_fwd", "swiglu", "combine_loss", "gemm_dx", "gemm_dw",
              "mask_bwd", "token_bwd", "wait", "gemm_dx_mask")


@dataclass
class MoEWeights:
    """bf16 tensors in the layouts of the C ABI (ln is fp32)."""

    ln: torch.Tensor  # [L, d] fp32
    router: torch.Tensor  # [L, E, d]
    Wg: torch.Tensor  # [L, E, d, f]
    Wu: torch.Tensor  # [L, E, d, f]
    Wd: torch.Tensor  # [L, E, f, d]
    Vg: torch.Tensor  # [L, E, d, c]
    Ug: torch.Tensor  # [L, E, c, f]
    Vu: torch.Tensor  # [L, E, d, c]
    Uu: torch.Tensor  # [L, E, c, f]
    Vd: torch.Tensor  # [L, E, f, c]
    Ud: torch.Tensor  # [L, E, c, d]


class MoEStackStep:
    def __init__(self, T: int, d: int, f: int, E: int, k: int, c: int, n_layers: int, *, device="cuda",
                 p: float = 2.0, imp_coeff: float = 1.0, recon_coeff: float = 1.0,
                 layout: int = L.LAYOUT_PARTITIONABLE, use_delta: bool = True, source_value: float = -1.0,
                 imp_min: ImpMin | None = None, rows_per_source: int | None = None):
        """rows_per_source: tokens per row of persistent source tables (`step_sources`; T
        is the `c` shape, a sample's positions `bc`, 1 `bsc`)."""
        self.dims = (T, d, f, E, k, c, n_layers)
        # the imp-min term: L_p (p, imp_coeff) unless a smooth-L0 ImpMin is given
        self.imp_min = imp_min if imp_min is not None else ImpMin("pnorm", p=p, coeff=imp_coeff)
        self.recon_coeff, self.layout = recon_coeff, layout
        self.use_delta = bool(use_delta)
        # < 0: Threefry mask and delta draws (stochastic recon); v in [0, 1]: constant
        # sources u = d = v (0: the CI-masked recon)
        self.source_value = float(source_value)
        dev = torch.device(device)
        f32 = dict(dtype=torch.float32, device=dev)
        Ln = n_layers
        # the EMA frequency estimate over every site's [E * c] components, [L, 3, E * c]
        # (None: the batch estimate); advanced by `step` and the final (weight-gradient)
        # call of `step_sources`, not by the adversary's warmup ascents
        self.frequency = self.imp_min.new_estimate(Ln * 3 * E * c, dev)
        # loss, recon, activity, frequency (+ the batch frequency with the EMA)
        self.losses = torch.empty(5 if self.frequency else 4, **f32)
        self.dV = {"gate": torch.empty(Ln, E, d, c, **f32), "up": torch.empty(Ln, E, d, c, **f32),
                   "down": torch.empty(Ln, E, f, c, **f32)}
        self.dU = {"gate": torch.empty(Ln, E, c, f, **f32), "up": torch.empty(Ln, E, c, f, **f32),
                   "down": torch.empty(Ln, E, c, d, **f32)}
        self.d_ci_pre = torch.empty(Ln, 3, T, k, c, dtype=torch.bfloat16, device=dev)
        self.top_idx = torch.empty(Ln, T, k, dtype=torch.int32, device=dev)
        self.rows_per_source = rows_per_source
        if rows_per_source is None:
            nbytes = L.load().pd_moe_stack_workspace_size(T, d, f, E, k, c, Ln)
        else:
            if rows_per_source <= 0 or T % rows_per_source:
                raise L.PDError("MoEStackStep: rows_per_source must divide T")
            S = T // rows_per_source
            nbytes = L.load().pd_moe_stack_sources_workspace_size(T, d, f, E, k, c, Ln, rows_per_source)
            self.d_src = torch.empty(Ln, 3, S, E, c, **f32)
            self.d_src_delta = torch.empty(Ln, 3, S, **f32)
        self.workspace = L.workspace(nbytes, dev)

    def _args(self, x0, w: MoEWeights, ci_pre, draw_key: Key, routes=None):
        T, d, f, E, k, c, Ln = self.dims
        rt = None
        if routes is not None:
            if isinstance(routes, dict):  # site -> [L, T]
                routes = torch.stack([routes[s] for s in SITE_NAMES], 1)
            if tuple(routes.shape) != (Ln, 3, T):
                raise L.PDError("MoEStackStep: routes are [L, 3, T]")
            rt = routes.to(torch.uint8).contiguous()
            self._routes = rt  # kept alive until the next call
        return [T, d, f, E, k, c, Ln, L.ptr(x0), L.ptr(w.ln), L.ptr(w.router), L.ptr(w.Wg), L.ptr(w.Wu), L.ptr(w.Wd),
                L.ptr(w.Vg), L.ptr(w.Ug), L.ptr(w.Vu), L.ptr(w.Uu), L.ptr(w.Vd), L.ptr(w.Ud), L.ptr(ci_pre),
                draw_key[0], draw_key[1], int(self.use_delta), L.ptr(rt), self.source_value, self.layout,
                *self.imp_min.c_args(self.frequency), self.recon_coeff, L.ptr(self.losses),
                L.ptr(self.dV["gate"]), L.ptr(self.dU["gate"]), L.ptr(self.dV["up"]), L.ptr(self.dU["up"]),
                L.ptr(self.dV["down"]), L.ptr(self.dU["down"]), L.ptr(self.d_ci_pre), L.ptr(self.top_idx),
                L.ptr(self.workspace), self.workspace.numel(), L.stream()]

    def step_sources(self, x0: torch.Tensor, w: MoEWeights, ci_pre: torch.Tensor, src: torch.Tensor,
                     src_delta: torch.Tensor | None = None, *, want_weight_grads: bool = True,
                     reuse_clean: bool = False):
        """The step with persistent source tables in place of the draws: src [L, 3, S, E, c]
        and src_delta [L, 3, S] (float32, bfloat16 or uint16 storage; None = no delta
        channel). Fills `d_src`, `d_src_delta` (and the model gradients when
        `want_weight_grads`). `reuse_clean` takes the frozen clean pass from this object's
        workspace as the previous call left it: only for repeated calls on the same x0 and
        frozen weights (ln, router, Wg, Wu, Wd) with no other step on this object between."""
        if self.rows_per_source is None:
            raise L.PDError("MoEStackStep: construct with rows_per_source for source tables")
        T, d, f, E, k, c, Ln = self.dims
        S = T // self.rows_per_source
        if tuple(src.shape) != (Ln, 3, S, E, c) or (src_delta is not None and tuple(src_delta.shape) != (Ln, 3, S)):
            raise L.PDError("step_sources: src [L, 3, S, E, c], src_delta [L, 3, S]")
        g = want_weight_grads
        P = lambda t: L.ptr(t) if g else None  # noqa: E731
        L.call("pd_moe_stack_step_sources", T, d, f, E, k, c, Ln, L.ptr(x0), L.ptr(w.ln), L.ptr(w.router),
               L.ptr(w.Wg), L.ptr(w.Wu), L.ptr(w.Wd), L.ptr(w.Vg), L.ptr(w.Ug), L.ptr(w.Vu), L.ptr(w.Uu), L.ptr(w.Vd),
               L.ptr(w.Ud), L.ptr(ci_pre), L.ptr(src), L.dtype_code(src.dtype),
               None if src_delta is None else L.ptr(src_delta),
               L.F32 if src_delta is None else L.dtype_code(src_delta.dtype), self.rows_per_source,
               *self.imp_min.c_args(self.frequency if g else None), self.recon_coeff, int(g), int(reuse_clean),
               L.ptr(self.losses),
               P(self.dV["gate"]),
               P(self.dU["gate"]), P(self.dV["up"]), P(self.dU["up"]), P(self.dV["down"]), P(self.dU["down"]),
               L.ptr(self.d_ci_pre), L.ptr(self.d_src), L.ptr(self.d_src_delta), L.ptr(self.top_idx),
               L.ptr(self.workspace), self.workspace.numel(), L.stream())
        if g:
            self._advance()
        return self

    def _advance(self):
        if self.frequency is not None:
            self.frequency.count += 1

    def step(self, x0: torch.Tensor, w: MoEWeights, ci_pre: torch.Tensor, draw_key: Key, routes=None):
        """routes: per-token site routes, uint8/bool [L, 3, T] or site -> [L, T] (None:
        every token routed); an unrouted token's jobs take the frozen output."""
        L.call("pd_moe_stack_step", *self._args(x0, w, ci_pre, draw_key, routes))
        self._advance()
        return self

    def step_timed(self, x0, w, ci_pre, draw_key, events: ctypes.Array, categories: torch.Tensor) -> int:
        """Records phase events; returns the number recorded (categories is an int32 CPU
        tensor of the events' capacity)."""
        n = ctypes.c_int(0)
        L.call("pd_moe_stack_step_timed", *self._args(x0, w, ci_pre, draw_key), events,
               ctypes.c_void_p(categories.data_ptr()), len(events), ctypes.byref(n))
        self._advance()
        return n.value
