"""ctypes binding of ``libfmoe.so`` (the C ABI declared in ``include/fmoe.h``).

The library is loaded from this package directory.  There is no fallback: if
it is missing or fails to load, every op raises ``RuntimeError`` naming the
build step, so a run can never silently use another implementation.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libfmoe.so")

FMOE_OK = 0
FMOE_ERR_INVALID = 1
FMOE_ERR_UNSUPPORTED = 2
FMOE_ERR_WORKSPACE = 3
FMOE_ERR_HIP = 4

W_BF16, W_FP8, W_INT4, W_MXFP4, W_INT4_TILED, W_MXFP4_TILED = 0, 1, 2, 3, 4, 5
ACT_SILU, ACT_GELU, ACT_SWIGLU = 0, 1, 2

c_i32p = ctypes.POINTER(ctypes.c_int32)
c_f32p = ctypes.POINTER(ctypes.c_float)
vp = ctypes.c_void_p


class AlignOut(ctypes.Structure):
    _fields_ = [(n, vp) for n in (
        "expt_indx", "expt_scal", "topk_indx", "gate_indx", "gate_scal", "hist", "offs_raw",
        "offs_pad", "tile_map", "n_tiles", "sorted_token_ids", "expert_ids",
        "num_tokens_post_padded")]


class Routing(ctypes.Structure):
    _fields_ = [
        ("topk_indx", vp), ("gate_indx", vp), ("gate_scal", vp), ("offs_raw", vp),
        ("offs_pad", vp), ("tile_map", vp), ("n_tiles", vp), ("n_tokens", ctypes.c_int64), ("top_k", ctypes.c_int32),
        ("n_experts", ctypes.c_int32), ("block_m", ctypes.c_int32), ("max_tiles", ctypes.c_int32),
    ]


class Epilogue(ctypes.Structure):
    _fields_ = [("activation", ctypes.c_int32), ("bias", vp), ("alpha", ctypes.c_float),
                ("limit", ctypes.c_float)]


class FusedArgs(ctypes.Structure):
    _fields_ = [
        ("wtype", ctypes.c_int32), ("x", vp), ("M", ctypes.c_int64), ("K", ctypes.c_int64),
        ("N", ctypes.c_int64), ("E", ctypes.c_int32), ("top_k", ctypes.c_int32), ("w13", vp),
        ("w2", vp), ("w13_scale", vp), ("w2_scale", vp), ("w13_zero", vp), ("w2_zero", vp),
        ("group_size", ctypes.c_int32), ("topk_weights", vp), ("topk_ids", vp),
        ("apply_router_weight_on_input", ctypes.c_int32), ("routed_scaling_factor", ctypes.c_float),
        ("path", ctypes.c_int32), ("out", vp), ("workspace", vp), ("workspace_bytes", ctypes.c_size_t),
        ("activation", ctypes.c_int32), ("b13", vp), ("b2", vp), ("alpha", ctypes.c_float),
        ("limit", ctypes.c_float), ("expert_map", vp), ("n_global", ctypes.c_int32),
    ]


# name -> (restype, argtypes)
_SIGS = {
    "fmoe_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "fmoe_last_error": (ctypes.c_char_p, []),
    "fmoe_abi_version": (ctypes.c_int, []),
    "fmoe_topk_softmax": (ctypes.c_int, [vp, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp, vp]),
    "fmoe_grouped_topk": (ctypes.c_int, [vp, vp, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp, vp]),
    "fmoe_max_tiles": (ctypes.c_int64, [ctypes.c_int64, ctypes.c_int]),
    "fmoe_sorted_ids_len": (ctypes.c_int64, [ctypes.c_int64, ctypes.c_int, ctypes.c_int]),
    "fmoe_align_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64, ctypes.c_int, ctypes.c_int]),
    "fmoe_align": (ctypes.c_int, [vp, vp, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                  ctypes.POINTER(AlignOut), vp, ctypes.c_size_t, vp]),
    "fmoe_align_ex": (ctypes.c_int, [vp, vp, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     vp, ctypes.c_int, ctypes.POINTER(AlignOut), vp, ctypes.c_size_t,
                                     vp]),
    "fmoe_expt_data": (ctypes.c_int, [vp, ctypes.c_int, ctypes.c_int64, ctypes.c_int, vp, vp, vp, vp, vp]),
    "fmoe_quant_fp8_group": (ctypes.c_int, [vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, vp, vp, vp]),
    "fmoe_gemm1": (ctypes.c_int, [ctypes.c_int, vp, vp, vp, vp, vp, ctypes.c_int64, ctypes.c_int64,
                                  ctypes.POINTER(Routing), ctypes.c_int, vp, ctypes.c_int, vp]),
    "fmoe_gemm2": (ctypes.c_int, [ctypes.c_int, vp, vp, vp, vp, vp, ctypes.c_int64, ctypes.c_int64,
                                  ctypes.POINTER(Routing), ctypes.c_int, vp, ctypes.c_int, ctypes.c_int, vp]),
    "fmoe_gemm1_ex": (ctypes.c_int, [ctypes.c_int, vp, vp, vp, vp, vp, ctypes.c_int64, ctypes.c_int64,
                                     ctypes.POINTER(Routing), ctypes.c_int, ctypes.POINTER(Epilogue), vp,
                                     ctypes.c_int, vp]),
    "fmoe_gemm2_ex": (ctypes.c_int, [ctypes.c_int, vp, vp, vp, vp, vp, ctypes.c_int64, ctypes.c_int64,
                                     ctypes.POINTER(Routing), ctypes.c_int, vp, vp, ctypes.c_int,
                                     ctypes.c_int, vp]),
    "fmoe_gemm2_splits": (ctypes.c_int, [ctypes.c_int, ctypes.c_int64, ctypes.c_int64,
                                         ctypes.POINTER(Routing), ctypes.c_int]),
    "fmoe_choose_block_m": (ctypes.c_int, [ctypes.c_int, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "fmoe_fused_block_m": (ctypes.c_int, [ctypes.c_int, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int64, ctypes.c_int64]),
    "fmoe_moe_sum": (ctypes.c_int, [vp, ctypes.c_int, vp, ctypes.c_int64, ctypes.c_int, ctypes.c_int64,
                                    ctypes.c_float, vp, vp]),
    "fmoe_fused_experts_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(FusedArgs)]),
    "fmoe_fused_experts": (ctypes.c_int, [ctypes.POINTER(FusedArgs), vp]),
    "fmoe_fused_experts_noalloc": (ctypes.c_int, [ctypes.POINTER(FusedArgs), vp]),
    "fmoe_repack_int4": (ctypes.c_int, [ctypes.c_int, vp, vp, vp, ctypes.c_int64, ctypes.c_int64,
                                        ctypes.c_int64, ctypes.c_int, vp, vp, vp, vp, vp]),
    "fmoe_tile_int4": (ctypes.c_int, [vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, vp, vp]),
}

EXPORTED = tuple(_SIGS)

_lib = None
_lock = threading.Lock()


def lib():
    """Load (once) and return the ctypes handle; raise if the build is missing."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise RuntimeError(
                        f"flaggems_sglang: HIP library not built ({LIB_PATH} missing); "
                        "run `python -c 'import __graft_entry__ as g; g.build()'` at the repo root")
                h = ctypes.CDLL(LIB_PATH)
                for name, (res, args) in _SIGS.items():
                    fn = getattr(h, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = h
    return _lib


class FmoeError(RuntimeError):
    pass


def check(status: int, what: str) -> None:
    """Map a status code to the reference's error convention: unsupported
    features raise AssertionError("... is not supported") like the reference's
    asserts (ops/fused_moe.py:154-170), bad arguments ValueError, the rest
    RuntimeError."""
    if status == FMOE_OK:
        return
    msg = lib().fmoe_last_error().decode(errors="replace")
    text = f"{what}: {msg}"
    if status == FMOE_ERR_UNSUPPORTED:
        raise AssertionError(text)
    if status == FMOE_ERR_INVALID:
        raise ValueError(text)
    raise FmoeError(f"{text} (status {status})")


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def require_cuda(*ts) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("flaggems_sglang fused MoE runs on the GPU: every tensor must be on a HIP device")
