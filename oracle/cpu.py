"""ctypes binding of the oracle's C restatement (`oracle/cpu_step.c`) — test
infrastructure and the timed CPU baseline only."""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "libpdoracle.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-C", _HERE, "-B", "_build/libpdoracle.so"], check=True, capture_output=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
        u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
        _lib.or_uniform.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int64, ctypes.c_int, f32p]
        _lib.or_uniform.restype = None
        _lib.or_dense_step.argtypes = [ctypes.c_int] * 5 + [f32p] * 8 + [u32p, u32p] + [ctypes.c_int] * 2 + [
            ctypes.c_float] * 3 + [f32p] * 4
        _lib.or_dense_step.restype = ctypes.c_int
        _lib.or_num_threads.restype = ctypes.c_int
        i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
        _lib.or_moe_step.argtypes = [ctypes.c_int] * 7 + [f32p] * 13 + [u32p, u32p, ctypes.c_int] + [
            ctypes.c_float] * 3 + [f32p] * 8 + [i32p]
        _lib.or_moe_step.restype = ctypes.c_int
    return _lib


def uniform(key, n: int, bf16: bool) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().or_uniform(key[0], key[1], n, int(bf16), out)
    return out


def num_threads() -> int:
    return lib().or_num_threads()


def dense_step(x, W, V, U, gate, mask_key, delta_key, *, use_delta=False, bf16_mask=True, p=2.0,
               imp_coeff=1.0, recon_coeff=1.0):
    """Runs `or_dense_step`; returns (losses[3], dV, dU, (dw_in, db_in, dw_out, db_out))."""
    f = lambda a: np.ascontiguousarray(a, dtype=np.float32)
    T, din = x.shape
    dout = W.shape[0]
    C = V.shape[1]
    H = gate.w_in.shape[1]
    losses = np.zeros(3, np.float32)
    dV = np.zeros((din, C), np.float32)
    dU = np.zeros((C, dout), np.float32)
    dgate = np.zeros(3 * C * H + C, np.float32)
    rc = lib().or_dense_step(T, din, dout, C, H, f(x), f(W), f(V), f(U), f(gate.w_in), f(gate.b_in),
                             f(gate.w_out), f(gate.b_out), np.asarray(mask_key, np.uint32),
                             np.asarray(delta_key, np.uint32), int(use_delta), int(bf16_mask), p, imp_coeff,
                             recon_coeff, losses, dV, dU, dgate)
    assert rc == 0
    CH = C * H
    dg = (dgate[:CH].reshape(C, H), dgate[CH:2 * CH].reshape(C, H), dgate[2 * CH:3 * CH].reshape(C, H),
          dgate[3 * CH:])
    return losses, dV, dU, dg


def pack_moe(cfg, params, x0, ci_pre, draw_key):
    """The fp32 arrays `or_moe_step` reads (stacked over layers) and the per-(layer, site)
    mask and delta keys (partitionable counter layout)."""
    from oracle import moe_oracle as mo

    f32 = lambda a: np.ascontiguousarray(a, dtype=np.float32)  # noqa: E731
    L = cfg.L
    st = {n: f32(np.stack([P[n] for P in params])) for n in ("ln", "router", "Wg", "Wu", "Wd", "Vg", "Ug", "Vu",
                                                               "Uu", "Vd", "Ud")}
    st["x0"] = f32(x0)
    st["ci"] = f32(np.stack([np.stack([ci_pre[l][s] for s in mo.SITES]) for l in range(L)]))
    st["mkeys"] = np.array([[mo.site_mask_keys(draw_key, l)[s] for s in mo.SITES] for l in range(L)],
                           np.uint32).reshape(-1)
    st["dkeys"] = np.array([[mo.site_delta_keys(draw_key, l)[s] for s in mo.SITES] for l in range(L)],
                           np.uint32).reshape(-1)
    return st


def run_moe(cfg, st, *, p=2.0, imp_coeff=1.0, recon_coeff=1.0, use_delta=True):
    """`or_moe_step` on packed inputs; returns dict(loss, recon, imp, grads, d_ci_pre, top_idx)."""
    from oracle import moe_oracle as mo

    T, d, f, E, k, c, L = cfg.T, cfg.d, cfg.f, cfg.E, cfg.k, cfg.c, cfg.L
    losses = np.zeros(3, np.float32)
    g = {n: np.zeros(st[n].shape, np.float32) for n in ("Vg", "Ug", "Vu", "Uu", "Vd", "Ud")}
    d_ci = np.zeros_like(st["ci"])
    top = np.zeros((L, T, k), np.int32)
    rc = lib().or_moe_step(T, d, f, E, k, c, L, st["x0"], st["ln"], st["router"], st["Wg"], st["Wu"], st["Wd"],
                           st["Vg"], st["Ug"], st["Vu"], st["Uu"], st["Vd"], st["Ud"], st["ci"], st["mkeys"],
                           st["dkeys"], int(use_delta), p, imp_coeff, recon_coeff, losses, g["Vg"], g["Ug"], g["Vu"],
                           g["Uu"], g["Vd"], g["Ud"], d_ci, top)
    assert rc == 0
    grads = [{n: g[n][l] for n in g} for l in range(L)]
    return dict(loss=float(losses[0]), recon=float(losses[1]), imp=float(losses[2]), grads=grads,
                d_ci_pre=[{s: d_ci[l, i] for i, s in enumerate(mo.SITES)} for l in range(L)], top_idx=top)


def moe_step(cfg, params, x0, ci_pre, draw_key, *, p=2.0, imp_coeff=1.0, recon_coeff=1.0, use_delta=True):
    """Runs `or_moe_step` (the fp32 C restatement of oracle.moe_oracle.moe_stack_step
    without the bf16 storage model; partitionable counter layout). params / ci_pre as
    moe_stack_step takes them."""
    return run_moe(cfg, pack_moe(cfg, params, x0, ci_pre, draw_key), p=p, imp_coeff=imp_coeff,
                   recon_coeff=recon_coeff, use_delta=use_delta)
