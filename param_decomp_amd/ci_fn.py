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


# ---------------------------------------------------------------- the engine's CI functions
def _bf16(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16).contiguous()


class _SiteMLPFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, n_layers, *params):
        weights = [_bf16(w) for w in params[:n_layers]]
        biases = [_bf16(b) for b in params[n_layers:]]
        xb = _bf16(x)
        out, ws = ops.ci_mlp_fwd(xb, weights, biases)
        ctx.save_for_backward(xb, ws, *weights)
        ctx.n_layers, ctx.x_dtype = n_layers, x.dtype
        return out

    @staticmethod
    def backward(ctx, g):
        xb, ws, *weights = ctx.saved_tensors
        dW, db, dx = ops.ci_mlp_bwd(xb, weights, _bf16(g), ws, ctx.needs_input_grad[0])
        return (dx.to(ctx.x_dtype) if dx is not None else None), None, *dW, *db


class SiteMLP(torch.nn.Module):
    """One site's CI MLP (`pd/core/ci_fn/implementations/mlp.py:57-78`): Linear+GELU(erf)
    hidden layers and a linear head over widths `dims = (d_in, *hidden, C)`. fp32 master
    weights [d_i, d_i+1] and biases, cast to bf16 for compute as the engine's `prepare`
    does (`layerwise_mlp.py:108-109`); the forward returns bf16 preactivations. Init as
    `init_mlp_stack` (`mlp.py:81-92`): normal weights times gain / sqrt(d_in), gain sqrt 2
    on the hidden layers and 1 on the head, zero biases. Widths that are not multiples of 8
    are zero-padded around the kernels."""

    def __init__(self, dims, *, device=None, generator: torch.Generator | None = None):
        super().__init__()
        dims = tuple(int(d) for d in dims)
        if len(dims) < 2:
            raise ValueError("SiteMLP needs at least an input and an output width")
        self.dims = dims
        self.weights = torch.nn.ParameterList()
        self.biases = torch.nn.ParameterList()
        for i, (din, dout) in enumerate(zip(dims[:-1], dims[1:])):
            gain = math.sqrt(2.0) if i < len(dims) - 2 else 1.0
            w = torch.randn(din, dout, device=device, generator=generator) * (gain / math.sqrt(din))
            self.weights.append(torch.nn.Parameter(w))
            self.biases.append(torch.nn.Parameter(torch.zeros(dout, device=device)))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if all(d % 8 == 0 for d in self.dims):
            return _SiteMLPFn.apply(x, len(self.weights), *self.weights, *self.biases)
        # The kernels take widths in multiples of 8. Zero padding is exact: padded input
        # columns meet zero weight rows, padded hidden units have zero weights and bias, so
        # z = 0 and GELU(0) = 0, and padded outputs are dropped.
        pd8 = [(-d) % 8 for d in self.dims]
        F = torch.nn.functional
        ws = [F.pad(w, (0, pd8[i + 1], 0, pd8[i])) for i, w in enumerate(self.weights)]
        bs = [F.pad(b, (0, pd8[i + 1])) for i, b in enumerate(self.biases)]
        out = _SiteMLPFn.apply(F.pad(x, (0, pd8[0])), len(ws), *ws, *bs)
        return out[..., :self.dims[-1]]


class LayerwiseMLPCIFn(torch.nn.Module):
    """One `SiteMLP` per output site reading the input tap at the same position
    (`pd/core/ci_fn/implementations/layerwise_mlp.py:90-140`): `site_preactivations(taps)`
    maps each input tap to its site's preactivations, `forward(taps)` squashes them into
    `CI` (`CI.from_preactivations`). Taps are cast to bf16 first. At least one hidden layer,
    as `init_layerwise_mlp_ci_fn` requires."""

    def __init__(self, input_names, sites, hidden_dims, *, device=None, generator=None):
        """`sites`: (name, d_in, C) per site, in output order."""
        super().__init__()
        if not hidden_dims:
            raise ValueError("MLP CI fn needs at least one hidden layer")
        self.input_names = tuple(input_names)
        self.output_names = tuple(name for name, _, _ in sites)
        if len(self.input_names) != len(self.output_names) or len(set(self.input_names)) != len(self.input_names):
            raise ValueError(f"one distinct input per site: {self.input_names} -> {self.output_names}")
        self.site_mlps = torch.nn.ModuleDict({
            name: SiteMLP((d_in, *hidden_dims, C), device=device, generator=generator) for name, d_in, C in sites
        })

    def site_preactivations(self, taps: dict) -> dict:
        if set(taps) != set(self.input_names):
            raise ValueError(f"tap keys {sorted(taps)} != CI fn inputs {sorted(self.input_names)}")
        return {out: self.site_mlps[out](_bf16_keep_grad(taps[inp]))
                for inp, out in zip(self.input_names, self.output_names)}

    def forward(self, taps: dict) -> CI:
        return CI.from_preactivations(self.site_preactivations(taps))


class GlobalMLPCIFn(torch.nn.Module):
    """ONE `SiteMLP` over every tap (`pd/core/ci_fn/implementations/global_mlp.py:90-154`):
    the taps are concatenated in `input_taps` order into `[..., sum width]`, mapped to
    `[..., sum C]` and split back per site in `sites` order, so every site's
    preactivations depend on every tap. `input_taps`: (key, width); `sites`: (name, C)."""

    def __init__(self, input_taps, sites, hidden_dims, *, device=None, generator=None):
        super().__init__()
        if not hidden_dims:
            raise ValueError("global MLP CI fn needs at least one hidden layer")
        self.input_taps = tuple((str(k), int(w)) for k, w in input_taps)
        keys = [k for k, _ in self.input_taps]
        if not keys or len(set(keys)) != len(keys):
            raise ValueError(f"distinct tap keys required: {keys}")
        self.output_names = tuple(name for name, _ in sites)
        self.c_sizes = tuple(int(c) for _, c in sites)
        dims = (sum(w for _, w in self.input_taps), *hidden_dims, sum(self.c_sizes))
        self.mlp = SiteMLP(dims, device=device, generator=generator)

    def site_preactivations(self, taps: dict) -> dict:
        if set(taps) != {k for k, _ in self.input_taps}:
            raise ValueError(f"tap keys {sorted(taps)} != CI fn inputs {sorted(k for k, _ in self.input_taps)}")
        for k, w in self.input_taps:
            if taps[k].shape[-1] != w:
                raise ValueError(f"tap {k} width {taps[k].shape[-1]} != expected {w}")
        joined = torch.cat([_bf16_keep_grad(taps[k]) for k, _ in self.input_taps], dim=-1)
        pre = self.mlp(joined)
        out, off = {}, 0
        for name, c in zip(self.output_names, self.c_sizes):
            out[name] = pre[..., off:off + c]
            off += c
        return out

    def forward(self, taps: dict) -> CI:
        return CI.from_preactivations(self.site_preactivations(taps))


def _bf16_keep_grad(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.bfloat16 else t.to(torch.bfloat16)


class _ReadoutFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, h, params, base):
        hb = _bf16(h)
        out = ops.ci_readout_fwd(hb, params.contiguous(), None if base is None else _bf16(base))
        ctx.save_for_backward(hb, params)
        ctx.h_dtype, ctx.has_base = h.dtype, base is not None
        return out

    @staticmethod
    def backward(ctx, g):
        hb, params = ctx.saved_tensors
        gb = _bf16(g)
        d_h, d_params = ops.ci_readout_bwd(hb, params.contiguous(), gb, want_dh=ctx.needs_input_grad[0])
        d_base = gb if ctx.has_base and ctx.needs_input_grad[2] else None
        return (d_h.to(ctx.h_dtype) if d_h is not None else None), d_params, d_base


class ComponentActivationReadout(torch.nn.Module):
    """One site's readout of its component activations h
    (`pd/core/ci_fn/implementations/transformer/component_conditioning.py:215-243`):
    `s+ sig(a+ h + b+) + s- sig(a- (-h) + b-) + bias`, sig the symmetric leaky hard
    sigmoid. `params` [7, C] fp32 = rows a+, b+, s+, a-, b-, s-, bias; init as
    `ConditionedCIFnArch.initialize_backbone` and `_uncalibrated_arm` (:136-172): unit
    input scales, zero input biases, `output_scale_init` output scales, zero bias.
    `forward(h, base)` adds the backbone's preactivations `base` (:333-338)."""

    A_POS, B_POS, S_POS, A_NEG, B_NEG, S_NEG, BIAS = range(7)

    def __init__(self, C: int, output_scale_init: float, *, device=None):
        super().__init__()
        p = torch.zeros(7, C, device=device)
        p[self.A_POS] = 1.0
        p[self.A_NEG] = 1.0
        p[self.S_POS] = output_scale_init
        p[self.S_NEG] = output_scale_init
        self.params = torch.nn.Parameter(p)

    def forward(self, h: torch.Tensor, base: torch.Tensor | None = None) -> torch.Tensor:
        return _ReadoutFn.apply(h, self.params, base)
