"""ctypes binding of `libpd_mi355x.so` (the C ABI in include/pd_mi355x.h).

Tensors are torch tensors on the GPU; their device pointers and the current HIP
stream are passed through. There is no fallback: a missing library or a non-GPU
tensor raises.
"""

from __future__ import annotations

import ctypes
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libpd_mi355x.so")

F32, BF16, U16 = 0, 1, 2
PGD_SGD, PGD_MOMENTUM, PGD_ADAM, PGD_SIGN = 0, 1, 2, 3
LAYOUT_PARTITIONABLE, LAYOUT_ORIGINAL = 0, 1
IMPMIN_PNORM, IMPMIN_SMOOTH_L0 = 0, 1
BLOCK_FUSED_OUTPUT, BLOCK_FUSED_INPUT = 0, 1

_c_i64, _c_i32, _c_u32, _c_f32, _c_p, _c_sz = (ctypes.c_int64, ctypes.c_int, ctypes.c_uint32, ctypes.c_float,
                                                ctypes.c_void_p, ctypes.c_size_t)

# name -> (restype, argtypes)
# imp-min arguments of the fused steps: kind, p, gamma, normalize_at_one, coeff, freq_coeff, ref_count,
# freq_ema_in, freq_ema_out, ema_count, ema_halflife
_IMP_ARGS = [_c_i32, _c_f32, _c_f32, _c_i32, _c_f32, _c_f32, _c_f32, _c_p, _c_p, _c_f32, _c_f32]

_SIGNATURES = {
    "pd_last_error": (ctypes.c_char_p, []),
    "pd_abi_version": (_c_i32, []),
    "pd_uniform": (_c_i32, [_c_u32, _c_u32, _c_i64, _c_i32, _c_i32, _c_p, _c_i32, _c_p]),
    "pd_squash_fwd": (_c_i32, [_c_p, _c_i32, _c_i64, _c_p, _c_p, _c_p]),
    "pd_squash_bwd": (_c_i32, [_c_p, _c_p, _c_p, _c_i32, _c_i64, _c_p, _c_p]),
    "pd_component_mask_fwd": (_c_i32, [_c_p, _c_i32, _c_i64, _c_u32, _c_u32, _c_i32, _c_i32, _c_p, _c_p]),
    "pd_component_mask_bwd": (_c_i32, [_c_p, _c_i32, _c_i64, _c_u32, _c_u32, _c_i32, _c_i32, _c_p, _c_p]),
    "pd_component_mask_fwd_dkey": (_c_i32, [_c_p, _c_i32, _c_i64, _c_p, _c_i32, _c_i32, _c_p, _c_p]),
    "pd_component_mask_bwd_dkey": (_c_i32, [_c_p, _c_i32, _c_i64, _c_p, _c_i32, _c_i32, _c_p, _c_p]),
    "pd_gate_fwd": (_c_i32, [_c_p, _c_i32, _c_i64, _c_i64, _c_i32, _c_p, _c_p, _c_p, _c_p, _c_i32, _c_p, _c_p]),
    "pd_gate_bwd_workspace_size": (_c_sz, [_c_i64, _c_i64, _c_i32]),
    "pd_gate_bwd": (_c_i32, [_c_p, _c_i32, _c_i64, _c_i64, _c_i32, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i32, _c_p, _c_p,
                             _c_p, _c_p, _c_p, _c_p, _c_sz, _c_p]),
    "pd_impmin_workspace_size": (_c_sz, [_c_i64, _c_i64]),
    "pd_impmin": (_c_i32, [_c_p, _c_i32, _c_i64, _c_i64, _c_i32, _c_f32, _c_f32, _c_f32, _c_f32, _c_f32, _c_i32,
                           _c_f32, _c_p, _c_p, _c_f32, _c_f32, _c_f32, _c_f32, _c_p, _c_p, _c_p, _c_sz, _c_p]),
    "pd_mse_workspace_size": (_c_sz, [_c_i64]),
    "pd_mse": (_c_i32, [_c_p, _c_p, _c_i32, _c_i64, _c_f32, _c_p, _c_p, _c_p, _c_sz, _c_p]),
    "pd_kl_workspace_size": (_c_sz, [_c_i64]),
    "pd_kl": (_c_i32, [_c_p, _c_p, _c_i32, _c_i64, _c_i64, _c_f32, _c_p, _c_p, _c_p, _c_sz, _c_p]),
    "pd_streamed_kl_workspace_size": (_c_sz, [_c_i32, _c_i64, _c_i64, _c_i64, _c_i32]),
    "pd_streamed_kl_fwd": (_c_i32, [_c_i32, _c_i64, _c_i64, _c_i64, _c_i32] + [_c_p] * 6 + [_c_p, _c_sz, _c_p]),
    "pd_streamed_kl_bwd": (_c_i32, [_c_i32, _c_i64, _c_i64, _c_i64, _c_i32] + [_c_p] * 7 + [_c_p, _c_sz, _c_p]),
    "pd_gemm": (_c_i32, [_c_i32, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_i32, _c_p, _c_i64, _c_i32, _c_p, _c_i64,
                         _c_i32, _c_f32, _c_f32, _c_p]),
    "pd_gemm_strided_batched": (_c_i32, [_c_i32, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_i32, _c_p,
                                         _c_i64, _c_i64, _c_i32, _c_p, _c_i64, _c_i64, _c_i32, _c_f32, _c_f32, _c_p]),
    "pd_blocked_site_fwd": (_c_i32, [_c_i32, _c_i32] + [_c_i64] * 5 + [_c_p] * 11),
    "pd_blocked_site_bwd_workspace_size": (_c_sz, [_c_i32, _c_i32] + [_c_i64] * 5),
    "pd_blocked_site_bwd": (_c_i32, [_c_i32, _c_i32] + [_c_i64] * 5 + [_c_p] * 16 + [_c_sz, _c_p]),
    "pd_masked_linear_fwd": (_c_i32, [_c_i32, _c_i64, _c_i64, _c_i64, _c_i64] + [_c_p] * 11),
    "pd_masked_linear_bwd_workspace_size": (_c_sz, [_c_i32, _c_i64, _c_i64, _c_i64]),
    "pd_masked_linear_bwd": (_c_i32, [_c_i32, _c_i64, _c_i64, _c_i64, _c_i64] + [_c_p] * 16 + [_c_sz, _c_p]),
    "pd_masked_linear_bwd_noalloc": (_c_i32, [_c_i32, _c_i64, _c_i64, _c_i64, _c_i64] + [_c_p] * 16),
    "pd_dense_step_workspace_size": (_c_sz, [_c_i32, _c_i64, _c_i64, _c_i64, _c_i64, _c_i32]),
    "pd_dense_step": (_c_i32, [_c_i32, _c_i64, _c_i64, _c_i64, _c_i64, _c_i32] + [_c_p] * 8 + [_c_u32] * 4 +
                      [_c_i32] * 3 + _IMP_ARGS + [_c_f32] + [_c_p] * 7 + [_c_p, _c_sz, _c_p]),
    "pd_dense_step_timed": (_c_i32, [_c_i32, _c_i64, _c_i64, _c_i64, _c_i64, _c_i32] + [_c_p] * 8 + [_c_u32] * 4 +
                            [_c_i32] * 3 + _IMP_ARGS + [_c_f32] + [_c_p] * 7 + [_c_p, _c_sz, _c_p, _c_p]),
    "pd_route_uniform_k": (_c_i32, [_c_u32, _c_u32, _c_i64, _c_i32, _c_i32, _c_p, _c_p]),
    "pd_route_static_p": (_c_i32, [_c_u32, _c_u32, _c_i64, _c_i32, _c_f32, _c_i32, _c_p, _c_p]),
    "pd_router_topk": (_c_i32, [_c_p, _c_i64, _c_i32, _c_i32, _c_p, _c_p, _c_p, _c_p]),
    "pd_routed_jobs_workspace_size": (_c_sz, [_c_i64, _c_i32]),
    "pd_routed_jobs": (_c_i32, [_c_p, _c_i64, _c_i32, _c_i32, _c_p, _c_p, _c_p, _c_p, _c_p, _c_sz, _c_p]),
    "pd_gather_rows": (_c_i32, [_c_p, _c_i32, _c_i64, _c_p, _c_i32, _c_i64, _c_p, _c_p]),
    "pd_gather_rows_vjp": (_c_i32, [_c_p, _c_i32, _c_i64, _c_p, _c_i64, _c_i32, _c_p, _c_p]),
    "pd_combine_jobs": (_c_i32, [_c_p, _c_i32, _c_i64, _c_p, _c_p, _c_i64, _c_i32, _c_p, _c_p]),
    "pd_grouped_gemm": (_c_i32, [_c_p, _c_p, _c_p, _c_i64, _c_i32, _c_i64, _c_i64, _c_i32, _c_p, _c_i32, _c_p]),
    "pd_grouped_gemm_dw": (_c_i32, [_c_p, _c_p, _c_p, _c_i64, _c_i32, _c_i64, _c_i64, _c_p, _c_i32, _c_p]),
    "pd_grouped_gemm_dw_kmajor": (_c_i32, [_c_p, _c_p, _c_p, _c_i64, _c_i32, _c_i64, _c_i64, _c_p, _c_i32, _c_p]),
    "pd_moe_stack_workspace_size": (_c_sz, [_c_i64] + [_c_i32] * 6),
    "pd_moe_stack_step": (_c_i32, [_c_i64] + [_c_i32] * 6 + [_c_p] * 13 +
                          [_c_u32, _c_u32, _c_i32, _c_p, _c_f32, _c_i32] + _IMP_ARGS + [_c_f32] + [_c_p] * 9 +
                          [_c_p, _c_sz, _c_p]),
    "pd_moe_stack_step_timed": (_c_i32, [_c_i64] + [_c_i32] * 6 + [_c_p] * 13 +
                                [_c_u32, _c_u32, _c_i32, _c_p, _c_f32, _c_i32] + _IMP_ARGS + [_c_f32] + [_c_p] * 9 +
                                [_c_p, _c_sz, _c_p, _c_p, _c_p, _c_i32, _c_p]),
    "pd_moe_stack_sources_workspace_size": (_c_sz, [_c_i64] + [_c_i32] * 6 + [_c_i64]),
    "pd_moe_stack_step_sources": (_c_i32, [_c_i64] + [_c_i32] * 6 + [_c_p] * 13 + [_c_p, _c_i32, _c_p, _c_i32, _c_i64] +
                                  _IMP_ARGS + [_c_f32, _c_i32, _c_i32] + [_c_p] * 12 + [_c_sz, _c_p]),
    "pd_tms_step_workspace_size": (_c_sz, [_c_i64, _c_i32, _c_i32, _c_i32]),
    "pd_tms_step_grads_size": (_c_i32, [_c_i32, _c_i32, _c_i32]),
    "pd_tms_step": (_c_i32, [_c_i64] + [_c_i32] * 3 + [_c_p] * 7 + [_c_p, _c_u32, _c_u32, _c_i32, _c_i32, _c_p] +
                    [_c_f32] * 3 + [_c_p, _c_p, _c_p, _c_sz, _c_p]),
    "pd_resid_mlp_step_workspace_size": (_c_sz, [_c_i64] + [_c_i32] * 5),
    "pd_resid_mlp_step_grads_size": (_c_i64, [_c_i32] * 4),
    "pd_resid_mlp_step": (_c_i32, [_c_i64] + [_c_i32] * 5 + [_c_p] * 8 + [_c_u32, _c_u32, _c_i32] + [_c_f32] * 3 +
                          [_c_p] * 4 + [_c_sz, _c_p]),
    "pd_lm_stack_workspace_size": (_c_sz, [_c_i64, _c_i64] + [_c_i32] * 4 + [_c_i64, _c_i32, _c_p, _c_i32, _c_i32]),
    "pd_lm_stack_step": (_c_i32,
                         [_c_i64, _c_i64] + [_c_i32] * 4 + [_c_i64, _c_i32] + [_c_p] * 6 + [_c_f32, _c_f32] +
                         [_c_p] * 4 + [_c_u32, _c_u32, _c_i32, _c_p, _c_i32] + _IMP_ARGS + [_c_f32, _c_i32] +
                         [_c_p] * 5 + [_c_sz, _c_p]),
    "pd_lm_stack_step_timed": (_c_i32,
                               [_c_i64, _c_i64] + [_c_i32] * 4 + [_c_i64, _c_i32] + [_c_p] * 6 + [_c_f32, _c_f32] +
                               [_c_p] * 4 + [_c_u32, _c_u32, _c_i32, _c_p, _c_i32] + _IMP_ARGS + [_c_f32, _c_i32] +
                               [_c_p] * 5 + [_c_sz, _c_p, _c_p, _c_p, _c_i32, _c_p]),
    "pd_lm_stack_sources_workspace_size": (_c_sz, [_c_i64, _c_i64] + [_c_i32] * 4 +
                                           [_c_i64, _c_i32, _c_p, _c_i32, _c_i32, _c_i64]),
    "pd_lm_stack_step_sources": (_c_i32,
                                 [_c_i64, _c_i64] + [_c_i32] * 4 + [_c_i64, _c_i32] + [_c_p] * 6 + [_c_f32, _c_f32] +
                                 [_c_p] * 4 + [_c_p, _c_i32, _c_p, _c_i32, _c_i64] + _IMP_ARGS +
                                 [_c_f32, _c_i32, _c_i32, _c_i32] + [_c_p] * 7 + [_c_sz, _c_p]),
    "pd_ci_mlp_workspace_size": (_c_sz, [_c_i32, _c_p, _c_i64]),
    "pd_ci_mlp_fwd": (_c_i32, [_c_i32, _c_p, _c_i64] + [_c_p] * 5 + [_c_sz, _c_p]),
    "pd_ci_mlp_bwd": (_c_i32, [_c_i32, _c_p, _c_i64] + [_c_p] * 7 + [_c_sz, _c_p]),
    "pd_ci_readout_fwd": (_c_i32, [_c_i64, _c_i64] + [_c_p] * 5),
    "pd_ci_readout_workspace_size": (_c_sz, [_c_i64, _c_i64]),
    "pd_ci_readout_bwd": (_c_i32, [_c_i64, _c_i64] + [_c_p] * 6 + [_c_sz, _c_p]),
    "pd_source_mask_fwd": (_c_i32, [_c_p, _c_i32, _c_i64, _c_i64, _c_p, _c_i32, _c_i64, _c_p, _c_p]),
    "pd_source_mask_bwd_workspace_size": (_c_sz, [_c_i64] * 3),
    "pd_source_mask_bwd": (_c_i32, [_c_p, _c_p, _c_i32, _c_i64, _c_i64, _c_p, _c_i32, _c_i64, _c_p, _c_p, _c_p, _c_sz,
                                    _c_p]),
    "pd_source_ascend": (_c_i32, [_c_i32, _c_i32, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_f32, _c_f32, ctypes.c_double,
                                  ctypes.c_double, _c_f32, _c_f32, _c_u32, _c_u32, _c_i32, _c_p]),
    "pd_faithfulness_workspace_size": (_c_sz, [_c_i64] * 4),
    "pd_faithfulness_fwd": (_c_i32, [_c_i64] * 5 + [_c_p, _c_i32] + [_c_p] * 3 + [_c_f32] + [_c_p] * 4 +
                            [_c_sz, _c_p]),
    "pd_faithfulness_bwd": (_c_i32, [_c_i64] * 5 + [_c_p] * 4 + [_c_f32] + [_c_p] * 4),
}

_lib = None


class PDError(RuntimeError):
    pass


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise PDError(f"HIP library not built: {LIB_PATH} is missing (run `python -m param_decomp_amd.builder`)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        raise PDError(f"pd error {rc}: {load().pd_last_error().decode()}")


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args))


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return F32
    if dt == torch.bfloat16:
        return BF16
    if dt == torch.uint16:
        return U16
    raise PDError(f"unsupported dtype {dt}")


def ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise PDError("pd kernels take GPU tensors")
    if not t.is_contiguous():
        raise PDError("pd kernels take contiguous tensors")
    return t.data_ptr()


def host_array(ctype, values):
    """A host array of `ctype` (the C ABI's `const int64_t*` / `const void* const*` lists)."""
    values = list(values)
    return (ctype * len(values))(*values)


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=device)
