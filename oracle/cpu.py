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
