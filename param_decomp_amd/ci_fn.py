"""Per-component causal-importance gate MLP (the SPD paper's CI function), on the GPU.

`papers/Stochastic_Parameter_Decomposition/spd_paper.md`, appendix "Architecture of
Causal Importance Function MLPs": every component c has its own scalar-input MLP,
`g_c = W_out,c GELU(W_in,c h_c + b_in,c) + b_out,c` with hidden width d_gate = 16,
reading the component's inner activation `h_c = x@V_c`. GELU is the exact-erf form the
engine uses (`param_decomp/param_decomp/core/ci_fn/implementations/mlp.py:77`). The
returned preactivations feed `CI.from_preactivations` (lower/upper squashings). Init:
Kaiming-normal (gain sqrt 2) weights and zero biases, as `init_mlp_stack`
(`core/ci_fn/implementations/mlp.py:81-92`) does for the engine's MLPs.
"""

from __future__ import annotations

import math

import torch

from param_decomp_amd import ops
from param_decomp_amd.squashing import CI

D_GATE = 16


class _Gate(torch.autograd.Function):
    @staticmethod
    def forward(ctx, h, w_in, b_in, w_out, b_out, precise):
        hc = h.contiguous()
        ctx.save_for_backward(hc, w_in, b_in, w_out, b_out)
        ctx.precise = precise
        return ops.gate_fwd(hc, w_in, b_in, w_out, b_out, precise)

    @staticmethod
    def backward(ctx, g):
        h, w_in, b_in, w_out, b_out = ctx.saved_tensors
        dh, dwi, dbi, dwo, dbo = ops.gate_bwd(h, w_in, b_in, w_out, b_out, g.float().contiguous(), ctx.precise)
        return dh, dwi, dbi, dwo, dbo, None


class ComponentGateMLP(torch.nn.Module):
    """Gate parameters for C components: `w_in, b_in, w_out` `[C, 16]`, `b_out` `[C]`
    (fp32 masters). `forward(h)` returns fp32 preactivations of h's shape."""

    def __init__(self, C: int, *, device=None, generator: torch.Generator | None = None):
        super().__init__()
        self.w_in = torch.nn.Parameter(torch.randn(C, D_GATE, device=device, generator=generator) * math.sqrt(2.0))
        self.b_in = torch.nn.Parameter(torch.zeros(C, D_GATE, device=device))
        self.w_out = torch.nn.Parameter(
            torch.randn(C, D_GATE, device=device, generator=generator) * math.sqrt(2.0 / D_GATE))
        self.b_out = torch.nn.Parameter(torch.zeros(C, device=device))

    def forward(self, h: torch.Tensor, *, precise: bool | None = None) -> torch.Tensor:
        pr = (h.dtype == torch.float32) if precise is None else precise
        return _Gate.apply(h, self.w_in, self.b_in, self.w_out, self.b_out, pr)

    def ci(self, site_acts: dict) -> CI:
        """Per-site preactivations from component activations, squashed into `CI`."""
        return CI.from_preactivations({k: self(v) for k, v in site_acts.items()})
