"""ctypes binding of liblewi_surge.so (the gfx950 HIP library, C ABI in include/lewi_surge.h).

torch-ROCm provides device memory and the current HIP stream; every computation runs in the HIP library.
There is no fallback: if the library is missing or fails to load, `lib()` raises.
"""
from __future__ import annotations

import ctypes
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liblewi_surge.so")

F32, BF16, F16 = 0, 1, 2
_DT = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_sz = ctypes.c_size_t


class MoeShape(ctypes.Structure):
    _fields_ = [("t", _i64), ("d", _i64), ("e", _i64), ("k", _i64), ("f", _i64), ("fs", _i64)]


class MoeParams(ctypes.Structure):
    _fields_ = [(n, _p) for n in ("x", "w_r", "bias", "w_gate", "w_up", "w_down", "ws_gate", "ws_up", "ws_down")]


class MoeGrads(ctypes.Structure):
    _fields_ = [(n, _p) for n in ("dx", "dw_r", "dw_gate", "dw_up", "dw_down", "dws_gate", "dws_up", "dws_down",
                                  "dweights")]


class MoeSavedViews(ctypes.Structure):
    _fields_ = [(n, _p) for n in ("logits", "sel", "weights", "group_sizes", "offsets", "block_off", "order", "pos",
                                  "slot", "row_src", "blk_expert", "blk_rows", "num_blocks", "h_gate", "h_up",
                                  "h", "y_pad")]


# name -> (restype, argtypes)
_SIGS = {
    "lsurge_abi_version": (_int, []),
    "lsurge_test_fail_launch": (_int, [_int, _int]),
    "lsurge_test_helpers_idle": (_int, []),
    "lsurge_last_error": (ctypes.c_char_p, []),
    "lsurge_set_concurrency": (_int, [_int]),
    "lsurge_get_concurrency": (_int, []),
    "lsurge_set_gemm_variant": (_int, [_int]),
    "lsurge_get_gemm_variant": (_int, []),
    "lsurge_gather_rows": (_int, [_p, _i64, _i64, _int, _p, _i64, _p, _p, _p]),
    "lsurge_gather_reduce": (_int, [_p, _i64, _i64, _int, _p, _i64, _i64, _p, _p, _int, _p]),
    "lsurge_gather_dot": (_int, [_p, _i64, _i64, _int, _p, _i64, _i64, _p, _int, _p, _p]),
    "lsurge_combine_bwd": (_int, [_p, _int, _p, _p, _i64, _i64, _i64, _p, _int, _p, _p, _p]),
    "lsurge_invert_permutation": (_int, [_p, _i64, _p, _p]),
    "lsurge_sort_indices_workspace_bytes": (_sz, [_i64, _i64]),
    "lsurge_sort_indices": (_int, [_p, _i64, _i64, _p, _p, _p, _p, _sz, _p]),
    "lsurge_router_topk": (_int, [_p, _p, _p, _i64, _i64, _i64, _i64, _p, _p, _p, _p]),
    "lsurge_max_blocks": (_i64, [_i64, _i64]),
    "lsurge_layout_workspace_bytes": (_sz, [_i64, _i64]),
    "lsurge_build_layout": (_int, [_p, _i64, _i64] + [_p] * 10 + [_p, _sz, _p]),
    "lsurge_ragged_dot_workspace_bytes": (_sz, [_i64, _i64]),
    "lsurge_ragged_dot_f32_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64]),
    "lsurge_ragged_dot_bwd_f32_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64]),
    "lsurge_ragged_dot": (_int, [_p, _p, _p, _i64, _i64, _i64, _i64, _int, _p, _int, _p, _sz, _p]),
    "lsurge_ragged_dot_noalloc_max_rows": (_sz, []),
    "lsurge_ragged_dot_noalloc_max_groups": (_sz, []),
    "lsurge_ragged_dot_noalloc": (_int, [_p, _p, _p, _i64, _i64, _i64, _i64, _int, _p, _int, _p]),
    "lsurge_ragged_dot_bwd": (_int, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _int, _p, _p, _p, _sz, _p]),
    "lsurge_ragged_dot_bwd_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64]),
    "lsurge_moe_saved_bytes": (_sz, [ctypes.POINTER(MoeShape)]),
    "lsurge_moe_saved_bytes_fp8": (_sz, [ctypes.POINTER(MoeShape)]),
    "lsurge_moe_fwd_workspace_bytes": (_sz, [ctypes.POINTER(MoeShape)]),
    "lsurge_moe_bwd_workspace_bytes": (_sz, [ctypes.POINTER(MoeShape)]),
    "lsurge_moe_fwd": (_int, [ctypes.POINTER(MoeShape), ctypes.POINTER(MoeParams), _p, _p, _sz, _p, _sz, _p]),
    "lsurge_moe_bwd": (_int, [ctypes.POINTER(MoeShape), ctypes.POINTER(MoeParams), _p, _p, ctypes.POINTER(MoeGrads),
                              _p, _sz, _p]),
    "lsurge_moe_saved_layout": (_int, [ctypes.POINTER(MoeShape), _p, ctypes.POINTER(MoeSavedViews)]),
    "lsurge_fp8_quantize_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "lsurge_fp8_quantize": (_int, [_p, _i64, _i64, _i64, _int, _p, _p, _p, _sz, _p]),
    "lsurge_ragged_dot_fp8": (_int, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p, _int, _p, _sz, _p]),
    "lsurge_moe_fp8_weights_bytes": (_sz, [ctypes.POINTER(MoeShape)]),
    "lsurge_moe_fp8_quantize_weights_workspace_bytes": (_sz, [ctypes.POINTER(MoeShape)]),
    "lsurge_moe_fp8_quantize_weights": (_int, [ctypes.POINTER(MoeShape), ctypes.POINTER(MoeParams), _p, _sz, _p, _sz,
                                               _p]),
    "lsurge_moe_fwd_fp8_workspace_bytes": (_sz, [ctypes.POINTER(MoeShape)]),
    "lsurge_moe_fwd_fp8": (_int, [ctypes.POINTER(MoeShape), ctypes.POINTER(MoeParams), _p, _sz, _p, _p, _sz, _p, _sz,
                                  _p]),
    "lsurge_moe_bwd_fp8_workspace_bytes": (_sz, [ctypes.POINTER(MoeShape)]),
    "lsurge_moe_bwd_fp8": (_int, [ctypes.POINTER(MoeShape), ctypes.POINTER(MoeParams), _p, _sz, _p, _p,
                                  ctypes.POINTER(MoeGrads), _p, _sz, _p]),
    "lsurge_fp8_cast_workspace_bytes": (_sz, []),
    "lsurge_fp8_cast_transpose": (_int, [_p, _i64, _i64, _int, _p, _p, _i64, _p, _p, _sz, _p]),
    "lsurge_causal_conv1d": (_int, [_p, _p, _i64, _i64, _i64, _i64, _p, _p]),
    "lsurge_causal_conv1d_bwd_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64]),
    "lsurge_causal_conv1d_bwd": (_int, [_p, _p, _p, _i64, _i64, _i64, _i64, _p, _p, _p, _sz, _p]),
    "lsurge_gdn_chunked_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _i64]),
    "lsurge_gdn_chunked_fwd": (_int, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _sz, _p]),
    "lsurge_gdn_chunked_bwd_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _i64]),
    "lsurge_l2norm_rows": (_int, [_p, _i64, _i64, ctypes.c_float, _p, _p, _p]),
    "lsurge_l2norm_rows_bwd": (_int, [_p, _p, _p, _i64, _i64, _p, _p]),
    "lsurge_gdn_chunked_bwd": (_int, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p, _p, _p,
                                      _p, _p, _sz, _p]),
    "lsurge_gdn_chunked_fwd_save": (_int, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _sz, _p]),
    "lsurge_gdn_chunked_saved_bytes": (_sz, [_i64, _i64, _i64, _i64, _i64]),
    "lsurge_gdn_chunked_bwd_saved_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _i64]),
    "lsurge_gdn_chunked_bwd_saved": (_int, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p, _p, _p,
                                            _p, _sz, _p, _sz, _p]),
    "lsurge_mfma_rate_probe_out_floats": (_sz, []),
    "lsurge_mfma_rate_probe": (_int, [_int, _int, _p, _p]),
    "lsurge_prof_enable": (_int, [_int]),
    "lsurge_prof_collect": (_int, []),
    "lsurge_prof_kernel_count": (_int, []),
    "lsurge_prof_kernel_name": (ctypes.c_char_p, [_int]),
    "lsurge_prof_read": (_int, [_int, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_i64)]),
    "lsurge_prof_reset": (None, []),
}

_lib = None


def lib():
    """Load the HIP library (raises if it is not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"lewi-surge HIP library not built: {LIB_PATH} missing "
                               "(run `python lewi-surge_amd/build.py` or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def exported_symbols():
    return list(_SIGS)


def check(rc, what=""):
    if rc != 0:
        msg = lib().lsurge_last_error().decode(errors="replace")
        raise RuntimeError(f"lewi-surge {what} failed ({rc}): {msg}")


def dt(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; expected float32, bfloat16 or float16") from None


def ptr(t):
    if t is None:
        return None
    return ctypes.c_void_p(t.data_ptr())


def stream(device=None):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def require_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("lewi-surge kernels need tensors on a ROCm device (got a CPU tensor)")


def contig(t):
    return t if t is None or t.is_contiguous() else t.contiguous()


def workspace(nbytes, device):
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)
