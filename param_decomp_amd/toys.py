"""Toy targets (TMS, ResidMLP) and their decomposition step on the GPU.

Mirrors the reference's toy targets:
- TMS (`param_decomp/param_decomp/targets/tms.py`): `clean_output` (`:254-258`),
  `site_inputs` (`:261-271`), the masked forward `_run_masked` (`:311-359`:
  `linear1` -> `linear2` + b2 -> ReLU, every site decomposed), `tms_mse` (`:380-388`),
  the tied untrained target (`:569-581`) and `sample_sparse_features` (`:584-609`).
- ResidMLP (`targets/resid_mlp.py`): `clean_output` / `site_inputs` (`:266-333`), the
  masked forward (`:336-390`: `resid += mlp_out(act(mlp_in(resid)))`, `out = resid @
  W_U`), `resid_mlp_mse` (`:411-418`), Kaiming-uniform blocks and the fixed unit-norm
  embedding (`:596-628`), `sample_sparse_features` (`:643-662`).

`ToyDecompositionStep.step` is one fwd+bwd of the stochastic-recon + importance-minimality
objective (`core/train.py:1182-1258`): clean forward, per-site CI from the gate MLP on
`clean_input @ V`, masks drawn from `split(draw_key)` -> `fold_in(., site_idx)`
(`core/masking.py:148-167`), masked forward through `site_forward`, MSE recon, p-norm
imp-min summed over sites, gradients left on V, U and the gate parameters. Every
product, gate, squashing, mask and loss runs in the HIP library (fp32 kernels); ReLU,
bias and residual adds are the only torch elementwise ops.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from param_decomp_amd import losses, masking, ops, prng
from param_decomp_amd.ci_fn import ComponentGateMLP
from param_decomp_amd.decomposed_linear import SiteWeights, site_out
from param_decomp_amd.prng import Key
from param_decomp_amd.squashing import lower_leaky_hard_sigmoid, upper_leaky_hard_sigmoid


class _Product(torch.autograd.Function):
    """`a @ b` through the HIP GEMM (fp32 or bf16), differentiable in both operands."""

    @staticmethod
    def forward(ctx, a, b):
        ctx.save_for_backward(a, b)
        return ops.gemm(a.contiguous(), b.contiguous())

    @staticmethod
    def backward(ctx, g):
        a, b = ctx.saved_tensors
        g = g.contiguous()
        da = ops.gemm(g, b.contiguous(), trans_b=True) if ctx.needs_input_grad[0] else None
        db = ops.gemm(a.contiguous(), g, trans_a=True) if ctx.needs_input_grad[1] else None
        return da, db


def product(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    return _Product.apply(a, b)


@dataclass
class ToySite:
    """One decomposed site: frozen `W [d_out, d_in]`, trainable `V [d_in, C]`, `U [C, d_out]`
    and the per-component gate."""

    name: str
    W: torch.Tensor
    V: torch.Tensor
    U: torch.Tensor
    gate: ComponentGateMLP

    def parameters(self):
        return [self.V, self.U, *self.gate.parameters()]


@dataclass
class TMSTarget:
    W1: torch.Tensor  # [n_hidden, n_features]; linear2's weight is W1^T (tied)
    b2: torch.Tensor  # [n_features]


@dataclass
class ResidMLPTarget:
    W_E: torch.Tensor  # [n_features, d_embed]
    W_U: torch.Tensor  # [d_embed, n_features]
    b_in: list = field(default_factory=list)  # per layer, None = no bias
    b_out: list = field(default_factory=list)


def make_site(name: str, W: torch.Tensor, C: int, *, generator=None) -> ToySite:
    """V ~ N(0, 1/d_in), U ~ N(0, 1/C) (`core/components.py:650-677`)."""
    d_out, d_in = W.shape
    dev = W.device
    V = (torch.randn(d_in, C, device=dev, generator=generator) / math.sqrt(d_in)).requires_grad_(True)
    U = (torch.randn(C, d_out, device=dev, generator=generator) / math.sqrt(C)).requires_grad_(True)
    return ToySite(name, W, V, U, ComponentGateMLP(C, device=dev, generator=generator))


def init_tms(n_features: int = 5, n_hidden: int = 2, C: int = 20, *, device="cuda", generator=None):
    """Untrained tied TMS target with zero bias (`tms.py:569-581`) and sites linear1, linear2."""
    b = 1.0 / math.sqrt(n_features)
    W1 = (torch.rand(n_hidden, n_features, device=device, generator=generator) * 2 - 1) * b
    target = TMSTarget(W1, torch.zeros(n_features, device=device))
    return target, [make_site("linear1", W1, C, generator=generator),
                    make_site("linear2", W1.t().contiguous(), C, generator=generator)]


def init_resid_mlp(n_features: int = 100, d_embed: int = 1000, d_mlp: int = 50, n_layers: int = 1, C: int = 100, *,
                   device="cuda", generator=None):
    """Fixed random unit-norm embedding (`W_U = W_E^T`) and Kaiming-uniform bias-free
    blocks (`resid_mlp.py:596-628`); sites `layers.{i}.mlp_in`, `layers.{i}.mlp_out`."""
    raw = torch.randn(n_features, d_embed, device=device, generator=generator)
    W_E = raw / raw.norm(dim=-1, keepdim=True)
    target = ResidMLPTarget(W_E, W_E.t().contiguous(), [None] * n_layers, [None] * n_layers)
    sites = []
    for i in range(n_layers):
        bi, bo = 1.0 / math.sqrt(d_embed), 1.0 / math.sqrt(d_mlp)
        W_in = (torch.rand(d_mlp, d_embed, device=device, generator=generator) * 2 - 1) * bi
        W_out = (torch.rand(d_embed, d_mlp, device=device, generator=generator) * 2 - 1) * bo
        sites += [make_site(f"layers.{i}.mlp_in", W_in, C, generator=generator),
                  make_site(f"layers.{i}.mlp_out", W_out, C, generator=generator)]
    return target, sites


def sparse_features(batch: int, n_features: int, p: float, low: float, *, device="cuda", generator=None):
    """`at_least_zero_active` batches: U(low, 1) values gated by U(0,1) < p (TMS low=0,
    ResidMLP low=-1)."""
    v = torch.rand(batch, n_features, device=device, generator=generator) * (1.0 - low) + low
    return v * (torch.rand(batch, n_features, device=device, generator=generator) < p)


def _bias(a, b):
    return a if b is None else a + b


@torch.no_grad()
def clean_forward(target, sites, x):
    """The all-frozen forward and each site's clean input."""
    if isinstance(target, TMSTarget):
        hidden = ops.gemm(x, sites[0].W, trans_b=True)
        return torch.relu(ops.gemm(hidden, sites[1].W, trans_b=True) + target.b2), [x, hidden]
    r = ops.gemm(x, target.W_E)
    inputs = []
    for i in range(len(sites) // 2):
        hid = torch.relu(_bias(ops.gemm(r, sites[2 * i].W, trans_b=True), target.b_in[i]))
        inputs += [r, hid]
        r = r + _bias(ops.gemm(hid, sites[2 * i + 1].W, trans_b=True), target.b_out[i])
    return ops.gemm(r, target.W_U), inputs


def masked_forward(target, sites, x, masks, deltas=None, routes=None):
    """The masked forward with every site decomposed (`tms.py:311-359`;
    `resid_mlp.py:336-390`)."""
    def site(i, a):
        s = sites[i]
        return site_out(a, SiteWeights(s.W, s.V, s.U), masks[i], None if deltas is None else deltas[i],
                        None if routes is None else routes[i])

    if isinstance(target, TMSTarget):
        return torch.relu(site(1, site(0, x)) + target.b2)
    r = ops.gemm(x, target.W_E)
    for i in range(len(sites) // 2):
        hid = torch.relu(_bias(site(2 * i, r), target.b_in[i]))
        r = r + _bias(site(2 * i + 1, hid), target.b_out[i])
    return product(r, target.W_U)


class ToyDecompositionStep:
    """One fwd+bwd of the toy decomposition objective; gradients accumulate into `.grad`
    of each site's V, U and gate parameters (zeroed at the start of every step)."""

    def __init__(self, target, sites, *, p: float = 1.0, imp_coeff: float = 1.0, recon_coeff: float = 1.0,
                 use_delta: bool = False):
        self.target, self.sites = target, sites
        self.p, self.imp_coeff, self.recon_coeff, self.use_delta = p, imp_coeff, recon_coeff, use_delta

    def step(self, x: torch.Tensor, draw_key: Key, routes=None) -> dict:
        for s in self.sites:
            for prm in s.parameters():
                prm.grad = None
        mask_key, delta_key = prng.split(draw_key)
        n = len(self.sites)
        deltas = [prng.fold_in(delta_key, i) for i in range(n)] if self.use_delta else None
        return self._body(x, [prng.fold_in(mask_key, i) for i in range(n)], deltas, routes)

    def _body(self, x, mask_keys, delta_keys, routes) -> dict:
        """The step given each site's mask key (host pairs, or device key tensors) and
        delta key (host pairs or None)."""
        clean, cin = clean_forward(self.target, self.sites, x)
        g = [s.gate(product(cin[i], s.V)) for i, s in enumerate(self.sites)]
        lower = [lower_leaky_hard_sigmoid(a) for a in g]
        upper = {s.name: upper_leaky_hard_sigmoid(a) for s, a in zip(self.sites, g)}
        masks = [masking.sample_component_mask(lo, mask_keys[i]) for i, lo in enumerate(lower)]
        deltas = None
        if delta_keys is not None:
            deltas = [masking.sample_delta_mask(lo, delta_keys[i]) for i, lo in enumerate(lower)]
        out = masked_forward(self.target, self.sites, x, masks, deltas, routes)
        recon = losses.mse(out, clean)
        imp = losses.importance_minimality_pnorm(upper, self.p)
        loss = self.recon_coeff * recon + self.imp_coeff * imp
        loss.backward()
        return {"loss": loss.detach(), "recon": recon.detach(), "imp": imp.detach(), "out": out.detach(),
                "clean": clean, "g_raw": [a.detach() for a in g]}


class GraphedToyStep:
    """`ToyDecompositionStep` captured once into a HIP graph and replayed every step: the
    host launches one graph instead of ~90 kernels through autograd (at the ResidMLP-1L
    shape the eager step is bound by that host work, not by its GPU time).

    Each step writes that step's per-site mask keys (`fold_in(split(draw_key)[0], site)`)
    into a device buffer the mask kernels read when they run, and copies the batch into the
    captured input buffer, so a replay draws that step's masks over that step's batch; the
    kernels and their order are those of the eager step, so results are bit-identical to
    it. The returned tensors and the parameters' `.grad` are the graph's own buffers,
    overwritten by the next step. Not for the weight-delta channel or routes (their draws
    take host keys)."""

    def __init__(self, step: ToyDecompositionStep, x_example: torch.Tensor, *, warmup: int = 2):
        if step.use_delta:
            raise ValueError("GraphedToyStep: the weight-delta channel draws with host keys")
        self.inner, self.warmup = step, warmup
        self.x = x_example.detach().clone()
        self.keys = torch.zeros((len(step.sites), 2), dtype=torch.int32, device=self.x.device)
        self.params = [prm for s in step.sites for prm in s.parameters()]
        self.graph = None

    def _set_keys(self, draw_key: Key):
        import numpy as np

        mask_key, _ = prng.split(draw_key)
        ks = np.array([prng.fold_in(mask_key, i) for i in range(len(self.inner.sites))], dtype=np.uint32)
        self.keys.copy_(torch.from_numpy(ks.view(np.int32)))  # stream-ordered after the last replay

    def _capture(self):
        keys = [self.keys[i] for i in range(self.keys.shape[0])]
        side = torch.cuda.Stream(device=self.x.device)
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):  # autograd's own set-up happens outside the capture
            for _ in range(self.warmup):
                for prm in self.params:
                    prm.grad = None
                self.inner._body(self.x, keys, None, None)
        torch.cuda.current_stream().wait_stream(side)
        for prm in self.params:
            prm.grad = None
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.out = self.inner._body(self.x, keys, None, None)
        self.grads = [prm.grad for prm in self.params]

    def step(self, x: torch.Tensor, draw_key: Key) -> dict:
        self._set_keys(draw_key)
        if x is not self.x:
            self.x.copy_(x)
        if self.graph is None:
            self._capture()
        self.graph.replay()
        for prm, gr in zip(self.params, self.grads):
            prm.grad = gr
        return self.out


class ResidMLPFusedStep:
    """The ResidMLP decomposition step of `ToyDecompositionStep` (same objective, draws and
    gradients; bias-free blocks, no weight-delta channel or routes) as one native call
    (`pd_resid_mlp_step`): the fp32 MFMA products plus one fused CI / mask pass per site
    forward and one backward, about a third of the composed step's launches. The gradients
    land in the sites' `.grad` as views of one flat buffer; `out` is the masked output."""

    def __init__(self, target: ResidMLPTarget, sites, *, p: float = 1.0, imp_coeff: float = 1.0,
                 recon_coeff: float = 1.0, layout: int | None = None):
        from param_decomp_amd import _lib as L

        if any(b is not None for b in target.b_in + target.b_out):
            raise L.PDError("ResidMLPFusedStep: bias-free blocks only (the composed step takes biases)")
        self.target, self.sites = target, sites
        self.F, self.D = target.W_E.shape
        self.L = len(sites) // 2
        self.M = sites[0].W.shape[0]
        self.C = sites[0].V.shape[1]
        self.p, self.imp_coeff, self.recon_coeff = p, imp_coeff, recon_coeff
        self.layout = L.LAYOUT_PARTITIONABLE if layout is None else layout
        dev = target.W_E.device
        D, M, C = self.D, self.M, self.C
        self.flat = torch.zeros(L.load().pd_resid_mlp_step_grads_size(D, M, C, self.L), dtype=torch.float32,
                                device=dev)
        self.losses = torch.zeros(3, dtype=torch.float32, device=dev)
        self.views = []
        o = 0
        for i in range(len(sites)):
            din, dout = (M, D) if i % 2 else (D, M)
            dV = self.flat[o:o + din * C].view(din, C)
            o += din * C
            dU = self.flat[o:o + C * dout].view(C, dout)
            o += C * dout
            gv = []
            for shape in ((C, 16), (C, 16), (C, 16), (C,)):
                k = shape[0] * (shape[1] if len(shape) > 1 else 1)
                gv.append(self.flat[o:o + k].view(*shape))
                o += k
            self.views.append((dV, dU, gv))
        self._ws = None
        self._out = None
        self._keep = None

    def step(self, x: torch.Tensor, draw_key: Key) -> dict:
        import ctypes

        from param_decomp_amd import _lib as L

        B = x.shape[0]
        lib = L.load()
        nbytes = lib.pd_resid_mlp_step_workspace_size(B, self.F, self.D, self.M, self.C, self.L)
        if self._ws is None or self._ws.numel() < nbytes:
            self._ws = L.workspace(nbytes, x.device)
        if self._out is None or self._out.shape[0] != B:
            self._out = torch.empty(B, self.F, dtype=torch.float32, device=x.device)
        sites = self.sites
        arrays = (L.host_array(ctypes.c_void_p, [L.ptr(sites[2 * i].W) for i in range(self.L)]),
                  L.host_array(ctypes.c_void_p, [L.ptr(sites[2 * i + 1].W) for i in range(self.L)]),
                  L.host_array(ctypes.c_void_p, [L.ptr(s.V) for s in sites]),
                  L.host_array(ctypes.c_void_p, [L.ptr(s.U) for s in sites]),
                  L.host_array(ctypes.c_void_p, [L.ptr(t) for s in sites for t in
                                                 (s.gate.w_in, s.gate.b_in, s.gate.w_out, s.gate.b_out)]))
        self._keep = arrays
        L.call("pd_resid_mlp_step", B, self.F, self.D, self.M, self.C, self.L, L.ptr(x.contiguous()),
               L.ptr(self.target.W_E), L.ptr(self.target.W_U), *arrays, draw_key[0], draw_key[1], self.layout,
               self.p, self.imp_coeff, self.recon_coeff, L.ptr(self.flat), L.ptr(self.losses), L.ptr(self._out),
               L.ptr(self._ws), self._ws.numel(), L.stream())
        for s, (dV, dU, gv) in zip(sites, self.views):
            s.V.grad, s.U.grad = dV, dU
            for prm, g in zip(s.gate.parameters(), gv):
                prm.grad = g
        return {"loss": self.losses[0], "recon": self.losses[1], "imp": self.losses[2], "out": self._out}


class TMSFusedStep:
    """The TMS decomposition step of `ToyDecompositionStep` (same objective, draws and
    gradients) as one fused launch plus one reduction (`pd_tms_step`): each wave owns 64
    batch rows end to end, parameters in LDS, gradients summed over rows in a fixed order.
    Compiled for the 5-2 target with 20 components per site; the gradients land in the
    sites' `.grad` as views of one flat buffer."""

    F, H, C = 5, 2, 20

    def __init__(self, target: TMSTarget, sites, *, p: float = 1.0, imp_coeff: float = 1.0, recon_coeff: float = 1.0,
                 use_delta: bool = False, layout: int | None = None):
        from param_decomp_amd import _lib as L

        H, F = target.W1.shape
        C = sites[0].V.shape[1]
        if (F, H, C) != (self.F, self.H, self.C) or len(sites) != 2:
            raise L.PDError(f"TMSFusedStep: compiled for the 5-2 target with 20 components (got {F}-{H}, C={C})")
        self.target, self.sites = target, sites
        self.p, self.imp_coeff, self.recon_coeff, self.use_delta = p, imp_coeff, recon_coeff, use_delta
        self.layout = L.LAYOUT_PARTITIONABLE if layout is None else layout
        dev = target.W1.device
        n = L.load().pd_tms_step_grads_size(F, H, C)
        self.flat = torch.zeros(n, dtype=torch.float32, device=dev)
        self.losses = torch.zeros(3, dtype=torch.float32, device=dev)
        G = 16
        o = 0
        views = []
        for shape in ((F, C), (C, H), (H, C), (C, F)):
            views.append(self.flat[o:o + shape[0] * shape[1]].view(*shape))
            o += shape[0] * shape[1]
        self.gate_views = []
        for _ in range(2):
            gv = []
            for shape in ((C, G), (C, G), (C, G), (C,)):
                k = shape[0] * (shape[1] if len(shape) > 1 else 1)
                gv.append(self.flat[o:o + k].view(*shape))
                o += k
            self.gate_views.append(gv)
        self.dV = [views[0], views[2]]
        self.dU = [views[1], views[3]]
        self._ws = None
        self._keep = None

    def _workspace(self, B, dev):
        from param_decomp_amd import _lib as L

        nbytes = L.load().pd_tms_step_workspace_size(B, self.F, self.H, self.C)
        if self._ws is None or self._ws.numel() < nbytes:
            self._ws = L.workspace(nbytes, dev)
        return self._ws

    def step(self, x: torch.Tensor, draw_key: Key, routes=None) -> dict:
        import ctypes

        from param_decomp_amd import _lib as L

        B = x.shape[0]
        s0, s1 = self.sites
        gates = L.host_array(ctypes.c_void_p, [L.ptr(t) for s in self.sites for t in
                                              (s.gate.w_in, s.gate.b_in, s.gate.w_out, s.gate.b_out)])
        rt = None
        if routes is not None:
            rt = torch.stack([r.to(torch.uint8) for r in routes]).contiguous()
        self._keep = (gates, rt)
        ws = self._workspace(B, x.device)
        # the library derives the sites' mask / delta keys from draw_key on the host side
        L.call("pd_tms_step", B, self.F, self.H, self.C, L.ptr(x.contiguous()), L.ptr(self.target.W1),
               L.ptr(self.target.b2), L.ptr(s0.V), L.ptr(s0.U), L.ptr(s1.V), L.ptr(s1.U), gates, draw_key[0],
               draw_key[1], int(self.use_delta), self.layout, None if rt is None else L.ptr(rt), self.p, self.imp_coeff,
               self.recon_coeff, L.ptr(self.flat), L.ptr(self.losses), L.ptr(ws), ws.numel(), L.stream())
        for i, s in enumerate(self.sites):
            s.V.grad, s.U.grad = self.dV[i], self.dU[i]
            for prm, g in zip(s.gate.parameters(), self.gate_views[i]):
                prm.grad = g
        return {"loss": self.losses[0], "recon": self.losses[1], "imp": self.losses[2]}
