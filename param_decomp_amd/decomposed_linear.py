"""The decomposed-linear primitive on the GPU: `((x@V)*(m-d))@U + d*(x@W^T)`.

Mirrors `param_decomp/param_decomp/core/decomposed_linear.py`:
- `SiteWeights(W, V, U)` (`:96-107`; the placement fields are single-GPU and absent),
- `site_forward(x, weights, mask, delta, route) -> SiteForward(output,
  component_activation)` (`:142-175`), `site_out` (`:178-181`),
- `component_coefficients` / `blend_target_output` semantics (`:65-85`): `delta` and
  `route` carry the leading axes only; None is the identity (d = 0, every position
  routed) and skips the target product.

`site_forward` is differentiable w.r.t. x, V, U and mask (W is frozen; delta and route
are samples). Forward and backward run as bf16 (or fp32) MFMA GEMMs through the C ABI.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from param_decomp_amd import _lib as L


@dataclass(frozen=True)
class SiteWeights:
    W: torch.Tensor  # [d_out, d_in]
    V: torch.Tensor  # [d_in, C]
    U: torch.Tensor  # [C, d_out]


@dataclass(frozen=True)
class SiteForward:
    output: torch.Tensor
    component_activation: torch.Tensor


def component_coefficients(mask: torch.Tensor, delta: torch.Tensor | None) -> torch.Tensor:
    return mask if delta is None else mask - delta


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise L.PDError(msg)


def _check_operands(x, V, U, W, mask, v_shape, u_shape, w_shape, c_total):
    """The kernels read every operand in x's dtype: the factors and the target weight
    must already be in it (the reference casts them once per step,
    `pd/core/model.py:479-483`); the mask and delta are cast here, as the reference's
    arithmetic promotes them (`pd/core/decomposed_linear.py:65-85`)."""
    for name, t, shape in (("V", V, v_shape), ("U", U, u_shape), ("W", W, w_shape)):
        if t is None:
            continue
        _require(t.dtype == x.dtype, f"site_forward: {name} is {t.dtype}, x is {x.dtype}")
        _require(tuple(t.shape) == tuple(shape), f"site_forward: {name} has shape {tuple(t.shape)}, expected "
                                                 f"{tuple(shape)}")
    _require(mask.shape[-1] == c_total and mask.numel() == x.numel() // x.shape[-1] * c_total,
             f"site_forward: mask shape {tuple(mask.shape)} does not match x {tuple(x.shape)} and C={c_total}")


class _MaskedLinear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, V, U, mask, W, delta, route):
        lead = x.shape[:-1]
        T = int(math.prod(lead))
        d_in, C = V.shape
        d_out = U.shape[1]
        dt = L.dtype_code(x.dtype)
        _require(x.shape[-1] == d_in, f"site_forward: x has {x.shape[-1]} features, V expects {d_in}")
        _check_operands(x, V, U, W, mask, (d_in, C), (C, d_out), (d_out, d_in), C)
        x2 = x.reshape(T, d_in).contiguous()
        m2 = mask.reshape(T, C).to(x.dtype).contiguous()
        d2 = None if delta is None else delta.reshape(T).to(x.dtype).contiguous()
        r2 = None if route is None else route.reshape(T).to(torch.uint8).contiguous()
        Wc = None if W is None else W.contiguous()
        out = torch.empty((T, d_out), dtype=x.dtype, device=x.device)
        xV = torch.empty((T, C), dtype=x.dtype, device=x.device)
        acts = torch.empty((T, C), dtype=x.dtype, device=x.device)
        L.call("pd_masked_linear_fwd", dt, T, d_in, d_out, C, L.ptr(x2), L.ptr(V.contiguous()), L.ptr(U.contiguous()),
               L.ptr(Wc), L.ptr(m2), L.ptr(d2), L.ptr(r2), L.ptr(out), L.ptr(xV), L.ptr(acts), L.stream())
        ctx.save_for_backward(x2, V, U, m2, Wc if Wc is not None else torch.empty(0, device=x.device),
                              d2 if d2 is not None else torch.empty(0, device=x.device),
                              r2 if r2 is not None else torch.empty(0, device=x.device), xV, acts)
        ctx.has = (W is not None, delta is not None, route is not None)
        ctx.lead = lead
        ctx.set_materialize_grads(False)
        return out.reshape(*lead, d_out), xV.reshape(*lead, C)

    @staticmethod
    def backward(ctx, g_out, g_xV):
        x2, V, U, m2, W, d2, r2, xV, acts = ctx.saved_tensors
        has_w, has_d, has_r = ctx.has
        W = W if has_w else None
        d2 = d2 if has_d else None
        r2 = r2 if has_r else None
        T, d_in = x2.shape
        C = V.shape[1]
        d_out = U.shape[1]
        dt = L.dtype_code(x2.dtype)
        if g_out is None:
            g_out = torch.zeros((T, d_out), dtype=x2.dtype, device=x2.device)
        g = g_out.reshape(T, d_out).contiguous()
        need_x, need_v, need_u, need_m = ctx.needs_input_grad[:4]
        need_d = ctx.needs_input_grad[5] and W is not None
        dx = torch.empty_like(x2) if need_x else None
        dd = torch.empty((T,), dtype=x2.dtype, device=x2.device) if need_d else None
        dV = torch.empty((d_in, C), dtype=x2.dtype, device=x2.device)
        dU = torch.empty((C, d_out), dtype=x2.dtype, device=x2.device)
        dm = torch.empty_like(m2) if need_m else None
        ws = L.workspace(L.load().pd_masked_linear_bwd_workspace_size(dt, T, d_out, C), x2.device)
        L.call("pd_masked_linear_bwd", dt, T, d_in, d_out, C, L.ptr(x2), L.ptr(V.contiguous()), L.ptr(U.contiguous()),
               L.ptr(W), L.ptr(m2), L.ptr(d2), L.ptr(r2), L.ptr(xV), L.ptr(acts), L.ptr(g), L.ptr(dx), L.ptr(dV),
               L.ptr(dU), L.ptr(dm), L.ptr(dd), L.ptr(ws), ws.numel(), L.stream())
        if g_xV is not None:
            # component_activation = x@V is also an output (the CI tap): its cotangent
            # adds x^T g_xV to dV and g_xV V^T to dx.
            from param_decomp_amd import ops

            gx = g_xV.reshape(T, C).contiguous().to(x2.dtype)
            ops.gemm(x2, gx, trans_a=True, out=dV, beta=1.0)
            if dx is not None:
                ops.gemm(gx, V.contiguous(), trans_b=True, out=dx, beta=1.0)
        lead = ctx.lead
        return (None if dx is None else dx.reshape(*lead, d_in), dV if need_v else None, dU if need_u else None,
                None if dm is None else dm.reshape(*lead, C), None, None if dd is None else dd.reshape(lead), None)


def site_forward(x: torch.Tensor, weights: SiteWeights, mask: torch.Tensor, delta: torch.Tensor | None,
                 route: torch.Tensor | None) -> SiteForward:
    """`where(route, ((x@V)*m)@U + d*(x@(W - V@U)^T), x@W^T)` per position."""
    W = weights.W if (delta is not None or route is not None) else None
    out, xV = _MaskedLinear.apply(x, weights.V, weights.U, mask, W, delta, route)
    return SiteForward(output=out, component_activation=xV)


def site_out(x, weights, mask, delta, route) -> torch.Tensor:
    return site_forward(x, weights, mask, delta, route).output


# ---------------------------------------------------------------- block-factored sites
@dataclass(frozen=True)
class BlockedSiteWeights:
    """A block-factored site (`pd/core/decomposed_linear.py:197-206`): the fused target
    weight `W`, per-block factors `V [E, d_in, c]` and `U [E, c, d_out]`."""

    W: torch.Tensor
    V: torch.Tensor
    U: torch.Tensor


_CONTRACTIONS = {"fused_output": L.BLOCK_FUSED_OUTPUT, "fused_input": L.BLOCK_FUSED_INPUT}


class _BlockedMaskedLinear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, V, U, mask, W, delta, route, contraction):
        E, d_in, c = V.shape
        d_out = U.shape[2]
        lead = x.shape[:-1]
        x2 = x.reshape(-1, x.shape[-1]).contiguous()
        T = x2.shape[0]
        fo = contraction == "fused_output"
        _require(x.shape[-1] == (d_in if fo else E * d_in),
                 f"blocked_site_forward: x has {x.shape[-1]} features for {E} blocks of d_in={d_in} ({contraction})")
        _check_operands(x, V, U, W, mask, (E, d_in, c), (E, c, d_out),
                        (E * d_out, d_in) if fo else (d_out, E * d_in), E * c)
        m2 = mask.reshape(T, E * c).to(x.dtype).contiguous()
        d2 = None if delta is None else delta.reshape(T).to(x.dtype).contiguous()
        r2 = None if route is None else route.reshape(T).to(torch.uint8).contiguous()
        Wc = None if W is None else W.contiguous()
        code = _CONTRACTIONS[contraction]
        DO = E * d_out if contraction == "fused_output" else d_out
        out = torch.empty((T, DO), dtype=x.dtype, device=x.device)
        xV = torch.empty((T, E * c), dtype=x.dtype, device=x.device)
        acts = torch.empty_like(xV)
        L.call("pd_blocked_site_fwd", L.dtype_code(x.dtype), code, T, E, d_in, d_out, c, L.ptr(x2),
               L.ptr(V.contiguous()), L.ptr(U.contiguous()), L.ptr(Wc), L.ptr(m2), L.ptr(d2), L.ptr(r2), L.ptr(out),
               L.ptr(xV), L.ptr(acts), L.stream())
        empty = torch.empty(0, device=x.device)
        ctx.save_for_backward(x2, V, U, m2, Wc if Wc is not None else empty, d2 if d2 is not None else empty,
                              r2 if r2 is not None else empty, xV, acts)
        ctx.has = (Wc is not None, d2 is not None, r2 is not None)
        ctx.meta = (lead, code, T, E, d_in, d_out, c)
        ctx.set_materialize_grads(False)
        return out.reshape(*lead, DO), xV.reshape(*lead, E * c)

    @staticmethod
    def backward(ctx, g_out, g_xV):
        x2, V, U, m2, W, d2, r2, xV, acts = ctx.saved_tensors
        has_w, has_d, has_r = ctx.has
        W, d2, r2 = (W if has_w else None), (d2 if has_d else None), (r2 if has_r else None)
        lead, code, T, E, d_in, d_out, c = ctx.meta
        dt = L.dtype_code(x2.dtype)
        DO = E * d_out if code == L.BLOCK_FUSED_OUTPUT else d_out
        if g_out is None:
            g_out = torch.zeros((T, DO), dtype=x2.dtype, device=x2.device)
        g = g_out.reshape(T, DO).contiguous()
        need_x, need_v, need_u, need_m = ctx.needs_input_grad[:4]
        need_d = ctx.needs_input_grad[5] and W is not None
        dx = torch.empty_like(x2) if need_x else None
        dV = torch.empty_like(V)
        dU = torch.empty_like(U)
        dm = torch.empty_like(m2) if need_m else None
        dd = torch.empty((T,), dtype=x2.dtype, device=x2.device) if need_d else None
        ws = L.workspace(L.load().pd_blocked_site_bwd_workspace_size(dt, code, T, E, d_in, d_out, c), x2.device)
        L.call("pd_blocked_site_bwd", dt, code, T, E, d_in, d_out, c, L.ptr(x2), L.ptr(V.contiguous()),
               L.ptr(U.contiguous()), L.ptr(W), L.ptr(m2), L.ptr(d2), L.ptr(r2), L.ptr(xV), L.ptr(acts), L.ptr(g),
               L.ptr(dx), L.ptr(dV), L.ptr(dU), L.ptr(dm), L.ptr(dd), L.ptr(ws), ws.numel(), L.stream())
        if g_xV is not None:
            # the flat component activation is also an output (the CI tap)
            from param_decomp_amd import ops

            gx = g_xV.reshape(T, E * c).contiguous().to(x2.dtype)
            fo = code == L.BLOCK_FUSED_OUTPUT
            DI = d_in if fo else E * d_in
            L.call("pd_gemm_strided_batched", dt, E, d_in, c, T, L.ptr(x2), DI, 0 if fo else d_in, 1, L.ptr(gx),
                   E * c, c, 0, L.ptr(dV), c, d_in * c, dt, 1.0, 1.0, L.stream())
            if dx is not None:
                if fo:
                    for e in range(E):
                        ops.gemm(gx[:, e * c:(e + 1) * c].contiguous(), V[e].contiguous(), trans_b=True, out=dx,
                                 beta=1.0)
                else:
                    L.call("pd_gemm_strided_batched", dt, E, T, d_in, c, L.ptr(gx), E * c, c, 0,
                           L.ptr(V.contiguous()), c, d_in * c, 1, L.ptr(dx), DI, d_in, dt, 1.0, 1.0, L.stream())
        return (None if dx is None else dx.reshape(*lead, x2.shape[1]), dV if need_v else None,
                dU if need_u else None, None if dm is None else dm.reshape(*lead, E * c), None,
                None if dd is None else dd.reshape(lead), None, None)


def blocked_site_forward(x: torch.Tensor, weights: BlockedSiteWeights, mask: torch.Tensor,
                         delta: torch.Tensor | None, route: torch.Tensor | None, contraction: str) -> SiteForward:
    """`blocked_site_forward` (`pd/core/decomposed_linear.py:209-271`), dense over every
    block: "fused_output" concatenates the blocks' outputs (gate/up), "fused_input"
    splits x per block and sums the outputs (down); mask / delta / route and the returned
    component activation use the flat block-major component axis `C = E*c`."""
    W = weights.W if (delta is not None or route is not None) else None
    out, xV = _BlockedMaskedLinear.apply(x, weights.V, weights.U, mask, W, delta, route, contraction)
    return SiteForward(output=out, component_activation=xV)
