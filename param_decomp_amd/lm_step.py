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
                 routed: bool = False):
        """routed: the step takes per-token site routes (`step(..., routes=...)`)."""
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
        nbytes = L.load().pd_lm_stack_workspace_size(B, T, d, n_head, n_kv_head, d_mlp, vocab, n_layers, self._cs,
                                                     int(self.use_delta or self.routed), n_kl_chunks)
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

    def _advance(self):
        if self.frequency is not None:
            self.frequency.count += 1

    def step_timed(self, tokens, w, ci_pre, draw_key, events: ctypes.Array, categories: torch.Tensor) -> int:
        n = ctypes.c_int(0)
        L.call("pd_lm_stack_step_timed", *self._args(tokens, w, ci_pre, draw_key), events,
               ctypes.c_void_p(categories.data_ptr()), len(events), ctypes.byref(n))
        self._advance()
        return n.value
