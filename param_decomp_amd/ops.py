"""Tensor-level wrappers over the C ABI: shape checks, output allocation, streams.

Each function maps one-to-one onto an `include/pd_mi355x.h` entry point. Higher-level
modules (`masking`, `decomposed_linear`, `losses`, `routed.experts`) add autograd.
"""

from __future__ import annotations

import ctypes
import math

import torch

from param_decomp_amd import _lib as L
from param_decomp_amd.prng import Key


def _flat_rows(t: torch.Tensor) -> tuple[int, int]:
    return int(math.prod(t.shape[:-1])), int(t.shape[-1])


def uniform(key: Key, shape, draw_dtype: torch.dtype, device, *, out_dtype: torch.dtype | None = None,
            layout: int = L.LAYOUT_PARTITIONABLE) -> torch.Tensor:
    out = torch.empty(tuple(shape), dtype=out_dtype or draw_dtype, device=device)
    L.call("pd_uniform", key[0], key[1], out.numel(), L.dtype_code(draw_dtype), layout, L.ptr(out),
           L.dtype_code(out.dtype), L.stream())
    return out


def squash_fwd(pre: torch.Tensor, lower: bool = True, upper: bool = True):
    lo = torch.empty_like(pre) if lower else None
    up = torch.empty_like(pre) if upper else None
    L.call("pd_squash_fwd", L.ptr(pre), L.dtype_code(pre.dtype), pre.numel(), L.ptr(lo), L.ptr(up), L.stream())
    return lo, up


def squash_bwd(pre, g_lower, g_upper):
    d = torch.empty_like(pre)
    L.call("pd_squash_bwd", L.ptr(pre), L.ptr(g_lower), L.ptr(g_upper), L.dtype_code(pre.dtype), pre.numel(),
           L.ptr(d), L.stream())
    return d


def _device_key(key) -> bool:
    """A key given as a device tensor of two 32-bit words (read when the kernel runs: the
    form a captured graph replays with fresh keys) rather than a host pair."""
    if isinstance(key, torch.Tensor):
        if key.dtype not in (torch.int32, torch.uint32) or key.numel() != 2 or not key.is_cuda:
            raise L.PDError("a device key is a CUDA tensor of two 32-bit words")
        return True
    return False


def component_mask_fwd(ci, key, draw_dtype: torch.dtype, layout=L.LAYOUT_PARTITIONABLE):
    m = torch.empty_like(ci)
    if _device_key(key):
        L.call("pd_component_mask_fwd_dkey", L.ptr(ci), L.dtype_code(ci.dtype), ci.numel(), L.ptr(key),
               L.dtype_code(draw_dtype), layout, L.ptr(m), L.stream())
    else:
        L.call("pd_component_mask_fwd", L.ptr(ci), L.dtype_code(ci.dtype), ci.numel(), key[0], key[1],
               L.dtype_code(draw_dtype), layout, L.ptr(m), L.stream())
    return m


def component_mask_bwd(g_mask, key, draw_dtype: torch.dtype, layout=L.LAYOUT_PARTITIONABLE):
    d = torch.empty_like(g_mask)
    if _device_key(key):
        L.call("pd_component_mask_bwd_dkey", L.ptr(g_mask), L.dtype_code(g_mask.dtype), g_mask.numel(), L.ptr(key),
               L.dtype_code(draw_dtype), layout, L.ptr(d), L.stream())
    else:
        L.call("pd_component_mask_bwd", L.ptr(g_mask), L.dtype_code(g_mask.dtype), g_mask.numel(), key[0], key[1],
               L.dtype_code(draw_dtype), layout, L.ptr(d), L.stream())
    return d


def gate_fwd(h, w_in, b_in, w_out, b_out, precise: bool):
    rows, C = _flat_rows(h)
    g = torch.empty(h.shape, dtype=torch.float32, device=h.device)
    L.call("pd_gate_fwd", L.ptr(h), L.dtype_code(h.dtype), rows, C, w_in.shape[1], L.ptr(w_in), L.ptr(b_in),
           L.ptr(w_out), L.ptr(b_out), int(precise), L.ptr(g), L.stream())
    return g


def gate_bwd(h, w_in, b_in, w_out, b_out, dg_raw, precise: bool):
    rows, C = _flat_rows(h)
    H = w_in.shape[1]
    dh = torch.empty_like(h)
    dwi, dbi, dwo = torch.empty_like(w_in), torch.empty_like(b_in), torch.empty_like(w_out)
    dbo = torch.empty_like(b_out)
    lib = L.load()
    ws = L.workspace(lib.pd_gate_bwd_workspace_size(rows, C, H), h.device)
    L.call("pd_gate_bwd", L.ptr(h), L.dtype_code(h.dtype), rows, C, H, L.ptr(w_in), L.ptr(b_in), L.ptr(w_out),
           L.ptr(b_out), L.ptr(dg_raw.contiguous()), int(precise), L.ptr(dh), L.ptr(dwi), L.ptr(dbi), L.ptr(dwo),
           L.ptr(dbo), L.ptr(ws), ws.numel(), L.stream())
    return dh, dwi, dbi, dwo, dbo


def impmin(ci_upper, *, kind: int, p=1.0, eps=0.0, beta=0.0, world_size=1.0, gamma=1.0, normalize_at_one=False,
           ref_count=0.0, coeff_act=1.0, coeff_freq=0.0, want_grad=False, ema=None, ema_out=None, ema_count=0.0,
           ema_halflife=0.0):
    """out[0] = activity, out[1] = frequency penalty, out[2] = the batch penalty when
    `ema` (the fp32 [C] estimate before this batch) is given; `ema_out` receives the new
    estimate (may be `ema` itself)."""
    rows, C = _flat_rows(ci_upper)
    out = torch.zeros(3, dtype=torch.float32, device=ci_upper.device)
    grad = torch.empty_like(ci_upper) if want_grad else None
    ws = L.workspace(L.load().pd_impmin_workspace_size(rows, C), ci_upper.device)
    L.call("pd_impmin", L.ptr(ci_upper), L.dtype_code(ci_upper.dtype), rows, C, kind, p, eps, beta, world_size, gamma,
           int(normalize_at_one), ref_count, L.ptr(ema), L.ptr(ema_out), float(ema_count), float(ema_halflife),
           coeff_act, coeff_freq, L.ptr(out), L.ptr(grad), L.ptr(ws), ws.numel(), L.stream())
    return out, grad


def mse(a, b, coeff=1.0, want_grad=False):
    out = torch.empty(1, dtype=torch.float32, device=a.device)
    grad = torch.empty_like(a) if want_grad else None
    ws = L.workspace(L.load().pd_mse_workspace_size(a.numel()), a.device)
    L.call("pd_mse", L.ptr(a), L.ptr(b), L.dtype_code(a.dtype), a.numel(), coeff, L.ptr(out), L.ptr(grad), L.ptr(ws),
           ws.numel(), L.stream())
    return out, grad


def kl(masked_logits, clean_logits, coeff=1.0, want_grad=False):
    rows, V = _flat_rows(masked_logits)
    out = torch.empty(1, dtype=torch.float32, device=masked_logits.device)
    grad = torch.empty_like(masked_logits) if want_grad else None
    ws = L.workspace(L.load().pd_kl_workspace_size(rows), masked_logits.device)
    L.call("pd_kl", L.ptr(masked_logits), L.ptr(clean_logits), L.dtype_code(masked_logits.dtype), rows, V, coeff,
           L.ptr(out), L.ptr(grad), L.ptr(ws), ws.numel(), L.stream())
    return out, grad


def gemm(a: torch.Tensor, b: torch.Tensor, *, trans_a=False, trans_b=False, out: torch.Tensor | None = None,
         out_dtype: torch.dtype | None = None, alpha=1.0, beta=0.0) -> torch.Tensor:
    """`alpha * op(a) @ op(b) + beta * out` for 2-D row-major tensors."""
    M = a.shape[1] if trans_a else a.shape[0]
    K = a.shape[0] if trans_a else a.shape[1]
    N = b.shape[0] if trans_b else b.shape[1]
    Kb = b.shape[1] if trans_b else b.shape[0]
    if K != Kb:
        raise L.PDError(f"gemm shape mismatch {tuple(a.shape)} {tuple(b.shape)}")
    if a.dtype != b.dtype:
        raise L.PDError("gemm operands must share a dtype")
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype or a.dtype, device=a.device)
    L.call("pd_gemm", L.dtype_code(a.dtype), M, N, K, L.ptr(a), a.shape[1], int(trans_a), L.ptr(b), b.shape[1],
           int(trans_b), L.ptr(out), N, L.dtype_code(out.dtype), alpha, beta, L.stream())
    return out


def route_uniform_k(key: Key, n_sites: int, n_positions: int, device, layout: int = L.LAYOUT_PARTITIONABLE):
    routes = torch.empty((n_sites, n_positions), dtype=torch.uint8, device=device)
    L.call("pd_route_uniform_k", key[0], key[1], n_positions, n_sites, layout, L.ptr(routes), L.stream())
    return routes


def route_static_p(key: Key, n_sites: int, p: float, n_positions: int, device, layout: int = L.LAYOUT_PARTITIONABLE):
    routes = torch.empty((n_sites, n_positions), dtype=torch.uint8, device=device)
    L.call("pd_route_static_p", key[0], key[1], n_positions, n_sites, p, layout, L.ptr(routes), L.stream())
    return routes


def router_topk(logits: torch.Tensor, k: int):
    T, E = logits.shape
    probs = torch.empty_like(logits)
    idx = torch.empty((T, k), dtype=torch.int32, device=logits.device)
    w = torch.empty((T, k), dtype=torch.float32, device=logits.device)
    L.call("pd_router_topk", L.ptr(logits), T, E, k, L.ptr(probs), L.ptr(idx), L.ptr(w), L.stream())
    return probs, idx, w


def routed_jobs(top_idx: torch.Tensor, n_experts: int):
    T, k = top_idx.shape
    n = T * k
    dev = top_idx.device
    sort_idx = torch.empty(n, dtype=torch.int32, device=dev)
    inv = torch.empty(n, dtype=torch.int32, device=dev)
    sizes = torch.empty(n_experts, dtype=torch.int32, device=dev)
    offsets = torch.empty(n_experts + 1, dtype=torch.int32, device=dev)
    ws = L.workspace(L.load().pd_routed_jobs_workspace_size(n, n_experts), dev)
    L.call("pd_routed_jobs", L.ptr(top_idx), T, k, n_experts, L.ptr(sort_idx), L.ptr(inv), L.ptr(sizes),
           L.ptr(offsets), L.ptr(ws), ws.numel(), L.stream())
    return sort_idx, inv, sizes, offsets


def gather_rows(src: torch.Tensor, idx: torch.Tensor, div: int) -> torch.Tensor:
    out = torch.empty((idx.numel(), src.shape[-1]), dtype=src.dtype, device=src.device)
    L.call("pd_gather_rows", L.ptr(src), L.dtype_code(src.dtype), src.shape[-1], L.ptr(idx), div, idx.numel(),
           L.ptr(out), L.stream())
    return out


def combine_jobs(y: torch.Tensor, inv: torch.Tensor, weights: torch.Tensor | None, T: int, k: int) -> torch.Tensor:
    out = torch.empty((T, y.shape[-1]), dtype=y.dtype, device=y.device)
    L.call("pd_combine_jobs", L.ptr(y), L.dtype_code(y.dtype), y.shape[-1], L.ptr(inv), L.ptr(weights), T, k,
           L.ptr(out), L.stream())
    return out


def grouped_gemm(lhs, rhs, offsets, *, trans_rhs=False, out_dtype=None):
    J, K = lhs.shape
    E = rhs.shape[0]
    N = rhs.shape[1] if trans_rhs else rhs.shape[2]
    out = torch.empty((J, N), dtype=out_dtype or lhs.dtype, device=lhs.device)
    L.call("pd_grouped_gemm", L.ptr(lhs), L.ptr(rhs), L.ptr(offsets), J, E, K, N, int(trans_rhs), L.ptr(out),
           L.dtype_code(out.dtype), L.stream())
    return out


def grouped_gemm_dw_kmajor(lhsT, doutT, offsets, n_groups: int, *, out_dtype=None):
    """`out[e] = lhsT[:, rows_e] @ doutT[:, rows_e]^T` from job-contiguous operands."""
    K, J = lhsT.shape
    N = doutT.shape[0]
    out = torch.empty((n_groups, K, N), dtype=out_dtype or lhsT.dtype, device=lhsT.device)
    L.call("pd_grouped_gemm_dw_kmajor", L.ptr(lhsT), L.ptr(doutT), L.ptr(offsets), J, n_groups, K, N, L.ptr(out),
           L.dtype_code(out.dtype), L.stream())
    return out


def grouped_gemm_dw(lhs, dout, offsets, n_groups: int, *, out_dtype=None):
    J, K = lhs.shape
    N = dout.shape[1]
    out = torch.empty((n_groups, K, N), dtype=out_dtype or lhs.dtype, device=lhs.device)
    L.call("pd_grouped_gemm_dw", L.ptr(lhs), L.ptr(dout), L.ptr(offsets), J, n_groups, K, N, L.ptr(out),
           L.dtype_code(out.dtype), L.stream())
    return out


def ci_mlp_fwd(x: torch.Tensor, weights, biases):
    """SiteMLP preactivations of bf16 `x` [..., d_0] with bf16 weights[i] [d_i, d_i+1] and
    biases[i] [d_i+1]. Returns (preact [..., d_n], workspace); the workspace holds the
    hidden activations and feeds `ci_mlp_bwd`."""
    rows, d0 = _flat_rows(x)
    dims = [d0] + [w.shape[1] for w in weights]
    for i, w in enumerate(weights):
        if w.shape[0] != dims[i] or biases[i].shape != (dims[i + 1],):
            raise L.PDError(f"ci_mlp layer {i}: weight {tuple(w.shape)} / bias {tuple(biases[i].shape)} mismatch")
    cdims = L.host_array(ctypes.c_int64, dims)
    out = torch.empty((*x.shape[:-1], dims[-1]), dtype=torch.bfloat16, device=x.device)
    ws = L.workspace(L.load().pd_ci_mlp_workspace_size(len(weights), cdims, rows), x.device)
    L.call("pd_ci_mlp_fwd", len(weights), cdims, rows, L.ptr(x), L.host_array(ctypes.c_void_p, map(L.ptr, weights)),
           L.host_array(ctypes.c_void_p, map(L.ptr, biases)), L.ptr(out), L.ptr(ws), ws.numel(), L.stream())
    return out, ws


def ci_mlp_bwd(x: torch.Tensor, weights, d_preact: torch.Tensor, ws: torch.Tensor, want_dx: bool):
    """Gradients of `ci_mlp_fwd` from bf16 `d_preact`, reusing its workspace: fp32
    d_weights and d_biases, and bf16 d_x (None unless asked)."""
    rows, d0 = _flat_rows(x)
    dims = [d0] + [w.shape[1] for w in weights]
    cdims = L.host_array(ctypes.c_int64, dims)
    dW = [torch.empty(w.shape, dtype=torch.float32, device=x.device) for w in weights]
    db = [torch.empty(w.shape[1], dtype=torch.float32, device=x.device) for w in weights]
    dx = torch.empty_like(x) if want_dx else None
    L.call("pd_ci_mlp_bwd", len(weights), cdims, rows, L.ptr(x), L.host_array(ctypes.c_void_p, map(L.ptr, weights)),
           L.ptr(d_preact), L.host_array(ctypes.c_void_p, map(L.ptr, dW)), L.host_array(ctypes.c_void_p, map(L.ptr, db)),
           L.ptr(dx), L.ptr(ws), ws.numel(), L.stream())
    return dW, db, dx


def ci_readout_fwd(h: torch.Tensor, params: torch.Tensor, base: torch.Tensor | None = None) -> torch.Tensor:
    """Component-activation readout of bf16 `h` [..., C] with fp32 params [7, C], added to
    bf16 `base` when given."""
    rows, C = _flat_rows(h)
    if params.shape != (7, C) or params.dtype != torch.float32:
        raise L.PDError("readout params must be fp32 [7, C]")
    out = torch.empty_like(h)
    L.call("pd_ci_readout_fwd", rows, C, L.ptr(h), L.ptr(params), L.ptr(base), L.ptr(out), L.stream())
    return out


def ci_readout_bwd(h: torch.Tensor, params: torch.Tensor, d_out: torch.Tensor, want_dh: bool = True):
    rows, C = _flat_rows(h)
    d_h = torch.empty_like(h) if want_dh else None
    d_params = torch.empty((7, C), dtype=torch.float32, device=h.device)
    ws = L.workspace(L.load().pd_ci_readout_workspace_size(rows, C), h.device)
    L.call("pd_ci_readout_bwd", rows, C, L.ptr(h), L.ptr(params), L.ptr(d_out), L.ptr(d_h), L.ptr(d_params), L.ptr(ws),
           ws.numel(), L.stream())
    return d_h, d_params


def faithfulness_fwd(W, V, U, w_sq_norms, mats_per_site: int, scale: float, keep_delta: bool):
    """Stacked faithfulness forward: W [n, d_out, d_in] (bf16/fp32), V fp32 [n, d_in, C],
    U fp32 [n, C, d_out], w_sq_norms fp32 [n / mats_per_site]. Returns (loss [1],
    site_errors, delta or None)."""
    n, d_out, d_in = W.shape
    C = V.shape[-1]
    if V.shape != (n, d_in, C) or U.shape != (n, C, d_out) or V.dtype != torch.float32 or U.dtype != torch.float32:
        raise L.PDError(f"faithfulness shapes: W {tuple(W.shape)} V {tuple(V.shape)} U {tuple(U.shape)} (fp32 V/U)")
    dev = W.device
    loss = torch.empty(1, dtype=torch.float32, device=dev)
    site_err = torch.empty(n // mats_per_site, dtype=torch.float32, device=dev)
    delta = torch.empty((n, d_out, d_in), dtype=torch.float32, device=dev) if keep_delta else None
    ws = L.workspace(L.load().pd_faithfulness_workspace_size(n, d_in, d_out, C), dev)
    L.call("pd_faithfulness_fwd", n, mats_per_site, d_in, d_out, C, L.ptr(W), L.dtype_code(W.dtype), L.ptr(V), L.ptr(U),
           L.ptr(w_sq_norms), scale, L.ptr(loss), L.ptr(site_err), L.ptr(delta), L.ptr(ws), ws.numel(), L.stream())
    return loss, site_err, delta


def faithfulness_bwd(delta, V, U, w_sq_norms, mats_per_site: int, scale: float, d_loss: torch.Tensor | None):
    n, d_out, d_in = delta.shape
    C = V.shape[-1]
    dV = torch.empty_like(V)
    dU = torch.empty_like(U)
    L.call("pd_faithfulness_bwd", n, mats_per_site, d_in, d_out, C, L.ptr(delta), L.ptr(V), L.ptr(U), L.ptr(w_sq_norms),
           scale, L.ptr(d_loss), L.ptr(dV), L.ptr(dU), L.stream())
    return dV, dU


def masked_linear_fwd(x, V, U, mask, W=None, delta=None):
    """`pd_masked_linear_fwd` without route: (out, xV, acts) with acts = xV * (mask - delta)
    and, with a delta [T], out = acts @ U + delta * (x @ W^T)."""
    T, d_in = x.shape
    C, d_out = U.shape
    out = torch.empty((T, d_out), dtype=x.dtype, device=x.device)
    xV = torch.empty((T, C), dtype=x.dtype, device=x.device)
    acts = torch.empty((T, C), dtype=x.dtype, device=x.device)
    L.call("pd_masked_linear_fwd", L.dtype_code(x.dtype), T, d_in, d_out, C, L.ptr(x), L.ptr(V), L.ptr(U), L.ptr(W),
           L.ptr(mask), L.ptr(delta), None, L.ptr(out), L.ptr(xV), L.ptr(acts), L.stream())
    return out, xV, acts


def masked_linear_bwd(x, V, U, mask, xV, acts, g_out, *, W=None, delta=None, want_dx=False, want_dvu=True,
                      want_dmask=True, want_ddelta=False):
    """`pd_masked_linear_bwd` without route; each output optional. Returns
    (dx, dV, dU, dmask, d_delta); d_delta [T] needs W."""
    T, d_in = x.shape
    C, d_out = U.shape
    dx = torch.empty_like(x) if want_dx else None
    dV = torch.empty_like(V) if want_dvu else None
    dU = torch.empty_like(U) if want_dvu else None
    dm = torch.empty_like(mask) if want_dmask else None
    dd = torch.empty((T,), dtype=x.dtype, device=x.device) if want_ddelta else None
    dt = L.dtype_code(x.dtype)
    ws = L.workspace(L.load().pd_masked_linear_bwd_workspace_size(dt, T, d_out, C), x.device)
    L.call("pd_masked_linear_bwd", dt, T, d_in, d_out, C, L.ptr(x), L.ptr(V), L.ptr(U), L.ptr(W), L.ptr(mask),
           L.ptr(delta), None, L.ptr(xV), L.ptr(acts), L.ptr(g_out), L.ptr(dx), L.ptr(dV), L.ptr(dU), L.ptr(dm),
           L.ptr(dd), L.ptr(ws), ws.numel(), L.stream())
    return dx, dV, dU, dm, dd


def source_mask_fwd(ci, sources, rows_per_source: int):
    """m = ci + (1 - ci) s for ci [rows, C] and sources [rows / rows_per_source, C]."""
    rows, C = _flat_rows(ci)
    mask = torch.empty_like(ci)
    L.call("pd_source_mask_fwd", L.ptr(ci), L.dtype_code(ci.dtype), rows, C, L.ptr(sources),
           L.dtype_code(sources.dtype), rows_per_source, L.ptr(mask), L.stream())
    return mask


def source_mask_bwd(g_mask, ci, sources, rows_per_source: int, want_dci: bool = False):
    rows, C = _flat_rows(ci)
    d_src = torch.empty((rows // rows_per_source, C), dtype=torch.float32, device=ci.device)
    d_ci = torch.empty_like(ci) if want_dci else None
    ws = L.workspace(L.load().pd_source_mask_bwd_workspace_size(rows, C, rows_per_source), ci.device)
    L.call("pd_source_mask_bwd", L.ptr(g_mask), L.ptr(ci), L.dtype_code(ci.dtype), rows, C, L.ptr(sources),
           L.dtype_code(sources.dtype), rows_per_source, L.ptr(d_src), L.ptr(d_ci), L.ptr(ws), ws.numel(), L.stream())
    return d_src, d_ci


def source_ascend(opt: int, sources, grad, state_a=None, state_b=None, *, step_count=0.0, lr=1.0, beta1=0.9,
                  beta2=0.999, eps=1e-8, momentum=0.0, key: Key = (0, 0), layout: int = L.LAYOUT_PARTITIONABLE):
    """One projected ascent of `sources` in place (see pd_source_ascend)."""
    L.call("pd_source_ascend", opt, L.dtype_code(sources.dtype), sources.numel(), L.ptr(sources), L.ptr(grad),
           L.ptr(state_a), L.ptr(state_b), step_count, lr, beta1, beta2, eps, momentum, key[0], key[1], layout,
           L.stream())
    return sources
