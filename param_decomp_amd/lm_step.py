"""The decomposed Llama-style LM step (every q/k/v/o/c_fc/down_proj matrix of a
LlamaSimpleMLP-form target decomposed) on the GPU.

One call = the frozen forward (the KL target), the masked forward with stochastic masks
drawn in-block per (kind, layer) and the weight-delta channel, the streamed KL over the
tied head plus the L_p imp-min, and the full backward to every site's V/U and CI
preactivations. See `pd_lm_stack_step` in include/pd_mi355x.h for the reference
citations and layouts.

All buffers are allocated once at construction; `step()` only enqueues kernels.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from param_decomp_amd import _lib as L
from param_decomp_amd.losses import ImpMin
from param_decomp_amd.prng import Key

KINDS = ("q_proj", "k_proj", "v_proj", "o_proj", "c_fc", "down_proj")  # KIND_ORDER (pd/targets/llama_simple_mlp.py)
CATEGORIES = ("prep", "clean_fwd", "gemm_fwd", "mask_fwd", "attention", "elementwise", "kl", "gemm_dx", "gemm_dw",
              "mask_bwd", "wait")
HEAD_DIM = 64


@dataclass
class LMWeights:
    """bf16 tensors in the C ABI's layouts (norm weights fp32)."""

    wte: torch.Tensor  # [V, d] embedding and tied head
    ln1: torch.Tensor  # [L, d] fp32
    ln2: torch.Tensor  # [L, d] fp32
    norm: torch.Tensor  # [d] fp32
    W: dict  # kind -> [L, d_out, d_in]
    V: dict  # kind -> [L, d_in, C]
    U: dict  # kind -> [L, C, d_out]


def site_dims(kind: str, d: int, n_head: int, n_kv_head: int, d_mlp: int) -> tuple[int, int]:
    qd, kvd = n_head * HEAD_DIM, n_kv_head * HEAD_DIM
    return {"q_proj": (d, qd), "k_proj": (d, kvd), "v_proj": (d, kvd), "o_proj": (qd, d), "c_fc": (d, d_mlp),
            "down_proj": (d_mlp, d)}[kind]


class LMStackStep:
    def __init__(self, B: int, T: int, d: int, n_head: int, n_kv_head: int, d_mlp: int, vocab: int, n_layers: int,
                 C: dict, *, device="cuda", p: float = 2.0, imp_coeff: float = 1.0, recon_coeff: float = 1.0,
                 layout: int = L.LAYOUT_PARTITIONABLE, use_delta: bool = True, n_kl_chunks: int = 1,
                 eps: float = 1e-6, rope_base: float = 10000.0, imp_min: ImpMin | None = None,
                 routed: bool = False, rows_per_source: int | None = None):
        """routed: the step takes per-token site routes (`step(..., routes=...)`).
        rows_per_source: tokens per row of persistent source tables (`step_sources`; B*T is
        the `c` shape, T a sample's positions `bc`, 1 `bsc`)."""
        if d != n_head * HEAD_DIM:
            raise L.PDError(f"LMStackStep: head_dim must be {HEAD_DIM} (d = {HEAD_DIM} * n_head)")
        self.dims = (B, T, d, n_head, n_kv_head, d_mlp, vocab, n_layers)
        self.C = {k: int(C[k]) for k in KINDS}
        # the imp-min term: L_p (p, imp_coeff) unless a smooth-L0 ImpMin is given
        self.imp_min = imp_min if imp_min is not None else ImpMin("pnorm", p=p, coeff=imp_coeff)
        self.recon_coeff, self.layout = recon_coeff, layout
        self.use_delta, self.n_kl_chunks, self.eps, self.rope_base = bool(use_delta), n_kl_chunks, eps, rope_base
        self.routed = bool(routed)
        dev = torch.device(device)
        N = B * T
        f32 = dict(dtype=torch.float32, device=dev)
        # the EMA frequency estimate, [L][kind][C_kind] layer-major (None: the batch estimate)
        self.frequency = self.imp_min.new_estimate(n_layers * sum(self.C.values()), dev)
        # total, kl, activity, frequency (+ the batch frequency with the EMA)
        self.losses = torch.empty(5 if self.frequency else 4, **f32)
        self.dV, self.dU, self.d_ci_pre = {}, {}, {}
        for k in KINDS:
            din, dout = site_dims(k, d, n_head, n_kv_head, d_mlp)
            self.dV[k] = torch.empty(n_layers, din, self.C[k], **f32)
            self.dU[k] = torch.empty(n_layers, self.C[k], dout, **f32)
            self.d_ci_pre[k] = torch.empty(n_layers, N, self.C[k], dtype=torch.bfloat16, device=dev)
        self._cs = L.host_array(ctypes.c_int32, [self.C[k] for k in KINDS])
        self.rows_per_source = rows_per_source
        if rows_per_source is None:
            nbytes = L.load().pd_lm_stack_workspace_size(B, T, d, n_head, n_kv_head, d_mlp, vocab, n_layers,
                                                         self._cs, int(self.use_delta or self.routed), n_kl_chunks)
        else:
            if rows_per_source <= 0 or N % rows_per_source:
                raise L.PDError("LMStackStep: rows_per_source must divide B*T")
            S = N // rows_per_source
            nbytes = L.load().pd_lm_stack_sources_workspace_size(B, T, d, n_head, n_kv_head, d_mlp, vocab,
                                                                 n_layers, self._cs, int(self.use_delta),
                                                                 n_kl_chunks, rows_per_source)
            self.d_src = {k: torch.empty(n_layers, S, self.C[k], **f32) for k in KINDS}
            self.d_src_delta = torch.empty(n_layers, len(KINDS), S, **f32)
            self._dsrc = L.host_array(ctypes.c_void_p, [L.ptr(self.d_src[k]) for k in KINDS])
        if nbytes == 0:
            raise L.PDError("pd_lm_stack_workspace_size: bad dimensions")
        self.workspace = L.workspace(nbytes, dev)
        P = ctypes.c_void_p
        self._dV = L.host_array(P, [L.ptr(self.dV[k]) for k in KINDS])
        self._dU = L.host_array(P, [L.ptr(self.dU[k]) for k in KINDS])
        self._dci = L.host_array(P, [L.ptr(self.d_ci_pre[k]) for k in KINDS])

    def _args(self, tokens, w: LMWeights, ci_pre: dict, draw_key: Key, routes=None):
        B, T, d, H, KV, f, V, Ln = self.dims
        P = ctypes.c_void_p
        for k in KINDS:
            if ci_pre[k].dtype != torch.bfloat16 or w.W[k].dtype != torch.bfloat16:
                raise L.PDError("pd_lm_stack_step: weights and CI preactivations are bf16")
        self._keep = (L.host_array(P, [L.ptr(w.W[k]) for k in KINDS]), L.host_array(P, [L.ptr(w.V[k]) for k in KINDS]),
                      L.host_array(P, [L.ptr(w.U[k]) for k in KINDS]),
                      L.host_array(P, [L.ptr(ci_pre[k]) for k in KINDS]))
        Wa, Va, Ua, Ca = self._keep
        rt = None
        if routes is not None:
            if not self.routed:
                raise L.PDError("LMStackStep: construct with routed=True to pass routes")
            if isinstance(routes, dict):  # kind -> [L, N]
                routes = torch.stack([routes[k] for k in KINDS], 1)
            if tuple(routes.shape) != (Ln, len(KINDS), B * T):
                raise L.PDError("LMStackStep: routes are [L, 6, N]")
            rt = routes.to(torch.uint8).contiguous()
            self._keep = self._keep + (rt,)
        return [B, T, d, H, KV, f, V, Ln, self._cs, L.ptr(tokens), L.ptr(w.wte), L.ptr(w.ln1), L.ptr(w.ln2),
                L.ptr(w.norm), self.eps, self.rope_base, Wa, Va, Ua, Ca, draw_key[0], draw_key[1], int(self.use_delta),
                L.ptr(rt), self.layout, *self.imp_min.c_args(self.frequency), self.recon_coeff, self.n_kl_chunks, L.ptr(self.losses), self._dV,
                self._dU, self._dci, L.ptr(self.workspace), self.workspace.numel(), L.stream()]

    def step(self, tokens: torch.Tensor, w: LMWeights, ci_pre: dict, draw_key: Key, routes=None):
        """routes: per-token site routes, uint8/bool [L, 6, N] or kind -> [L, N] (None:
        every token routed); an unrouted token's site output is the target's."""
        L.call("pd_lm_stack_step", *self._args(tokens, w, ci_pre, draw_key, routes))
        self._advance()
        return self

    def step_sources(self, tokens: torch.Tensor, w: LMWeights, ci_pre: dict, src: dict,
                     src_delta: torch.Tensor | None = None, *, want_weight_grads: bool = True,
                     reuse_clean: bool = False):
        """The step with persistent source tables in place of the draws: src kind -> [L, S,
        C_k] (one storage dtype: float32, bfloat16 or uint16) and src_delta [L, 6, S] (None =
        no delta channel; construct with use_delta=True to size for one). Fills `d_src`,
        `d_src_delta` (and the model gradients when `want_weight_grads`). `reuse_clean` takes
        the frozen forward's final activations from this object's workspace as the previous
        call left them: only for repeated calls on the same tokens, wte and frozen weights
        with no other step on this object between."""
        if self.rows_per_source is None:
            raise L.PDError("LMStackStep: construct with rows_per_source for source tables")
        B, T, d, H, KV, f, V, Ln = self.dims
        S = B * T // self.rows_per_source
        dts = {src[k].dtype for k in KINDS}
        if len(dts) != 1 or any(tuple(src[k].shape) != (Ln, S, self.C[k]) for k in KINDS):
            raise L.PDError("step_sources: src[kind] [L, S, C_kind], one dtype")
        if src_delta is not None and (tuple(src_delta.shape) != (Ln, len(KINDS), S) or not self.use_delta):
            raise L.PDError("step_sources: src_delta [L, 6, S], on a step constructed with use_delta=True")
        g = want_weight_grads
        P = ctypes.c_void_p
        Wa = L.host_array(P, [L.ptr(w.W[k]) for k in KINDS])
        Va = L.host_array(P, [L.ptr(w.V[k]) for k in KINDS])
        Ua = L.host_array(P, [L.ptr(w.U[k]) for k in KINDS])
        Ca = L.host_array(P, [L.ptr(ci_pre[k]) for k in KINDS])
        Sa = L.host_array(P, [L.ptr(src[k]) for k in KINDS])
        L.call("pd_lm_stack_step_sources", B, T, d, H, KV, f, V, Ln, self._cs, L.ptr(tokens), L.ptr(w.wte),
               L.ptr(w.ln1), L.ptr(w.ln2), L.ptr(w.norm), self.eps, self.rope_base, Wa, Va, Ua, Ca, Sa,
               L.dtype_code(dts.pop()), None if src_delta is None else L.ptr(src_delta),
               L.F32 if src_delta is None else L.dtype_code(src_delta.dtype), self.rows_per_source,
               *self.imp_min.c_args(self.frequency if g else None), self.recon_coeff, self.n_kl_chunks, int(g),
               int(reuse_clean), L.ptr(self.losses), self._dV if g else None, self._dU if g else None, self._dci,
               self._dsrc, L.ptr(self.d_src_delta), L.ptr(self.workspace), self.workspace.numel(), L.stream())
        if g:
            self._advance()
        return self

    def _advance(self):
        if self.frequency is not None:
            self.frequency.count += 1

    def step_timed(self, tokens, w, ci_pre, draw_key, events: ctypes.Array, categories: torch.Tensor) -> int:
        n = ctypes.c_int(0)
        L.call("pd_lm_stack_step_timed", *self._args(tokens, w, ci_pre, draw_key), events,
               ctypes.c_void_p(categories.data_ptr()), len(events), ctypes.byref(n))
        self._advance()
        return n.value
