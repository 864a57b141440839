"""CPU checks of the C-ABI boundary: libfmoe.so loads, exports every function
``include/fmoe.h`` declares (and ctypes binds exactly those), and the
host-only entry points (sizes, argument validation) behave.  No kernel is
launched: argument errors are detected before any HIP call."""

import ctypes
import os
import re

import pytest

from flaggems_sglang import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fmoe.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fmoe_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_expected_entries():
    names = _declared()
    for n in ("fmoe_align", "fmoe_gemm1", "fmoe_gemm2", "fmoe_moe_sum", "fmoe_fused_experts",
              "fmoe_topk_softmax", "fmoe_grouped_topk", "fmoe_quant_fp8_group"):
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for n in _declared():
        assert hasattr(lib, n), n
    assert sorted(_lib.EXPORTED) == _declared()


def test_host_queries():
    L = _lib.lib()
    assert L.fmoe_abi_version() == 2
    assert L.fmoe_status_string(2) == b"not supported"
    assert L.fmoe_max_tiles(8, 256) == 8
    assert L.fmoe_max_tiles(65536, 256) == 255 + (65536 - 256 + 1 + 15) // 16
    assert L.fmoe_sorted_ids_len(128, 8, 16) == 128 + 8 * 15
    assert L.fmoe_choose_block_m(_lib.W_INT4, 4096, 2, 8, 0) == 16
    assert L.fmoe_choose_block_m(_lib.W_BF16, 1, 2, 8, 0) == 16
    assert L.fmoe_choose_block_m(_lib.W_BF16, 4096, 2, 8, 0) == 256
    assert L.fmoe_choose_block_m(_lib.W_BF16, 1024, 8, 128, 0) == 128
    assert L.fmoe_choose_block_m(_lib.W_BF16, 400, 8, 128, 0) == 64
    # fp8: 160-row tiles where the mean + 2 sd load per expert needs fewer of
    # them than of 128-row tiles (DSV3 M=4096: 128 +- 11 slots per expert)
    assert L.fmoe_choose_block_m(_lib.W_FP8, 4096, 8, 256, 0) == 160
    assert L.fmoe_choose_block_m(_lib.W_FP8, 8192, 8, 256, 0) == 160
    assert L.fmoe_choose_block_m(_lib.W_FP8, 3072, 8, 256, 0) == 128
    assert L.fmoe_choose_block_m(_lib.W_FP8, 6400, 8, 256, 0) == 128
    # the fused path's choice: fp8 160-row tiles only while K, N <= 8192
    assert L.fmoe_fused_block_m(_lib.W_FP8, 4096, 8, 256, 0, 7168, 2048) == 160
    assert L.fmoe_fused_block_m(_lib.W_FP8, 4096, 8, 256, 0, 8448, 2048) == 128
    assert L.fmoe_fused_block_m(_lib.W_FP8, 4096, 8, 256, 0, 7168, 8320) == 128
    assert L.fmoe_fused_block_m(_lib.W_BF16, 1024, 8, 64, 0, 16384, 16384) == 160


def test_argument_errors_map_to_reference_convention():
    L = _lib.lib()
    st = L.fmoe_topk_softmax(None, 4, 8, 0, 1, None, None, None)
    assert st == _lib.FMOE_ERR_INVALID
    with pytest.raises(ValueError, match="topk_softmax"):
        _lib.check(st, "topk_softmax")
    ao = _lib.AlignOut()
    st = L.fmoe_align(None, None, 4, 2, 8, 48, ctypes.byref(ao), None, 0, None)
    assert st == _lib.FMOE_ERR_UNSUPPORTED
    with pytest.raises(AssertionError, match="is not supported"):
        _lib.check(st, "align")
    fa = _lib.FusedArgs()
    fa.wtype, fa.M, fa.K, fa.N, fa.E, fa.top_k = 0, 4, 100, 256, 8, 2
    assert L.fmoe_fused_experts_workspace_bytes(ctypes.byref(fa)) == 0
    assert L.fmoe_fused_experts(ctypes.byref(fa), None) == _lib.FMOE_ERR_UNSUPPORTED
    fa.K = 128
    assert L.fmoe_fused_experts_workspace_bytes(ctypes.byref(fa)) > 0
    assert L.fmoe_fused_experts(ctypes.byref(fa), None) == _lib.FMOE_ERR_INVALID  # null pointers
    # int4 weights take SiLU / GELU only (no SWIGLU row pairing)
    fa.wtype, fa.group_size, fa.activation = _lib.W_INT4_TILED, 128, _lib.ACT_SWIGLU
    assert L.fmoe_fused_experts_workspace_bytes(ctypes.byref(fa)) == 0
    assert L.fmoe_fused_experts(ctypes.byref(fa), None) == _lib.FMOE_ERR_UNSUPPORTED
    assert b"SWIGLU" in L.fmoe_last_error()
    fa.activation = _lib.ACT_SILU
    assert L.fmoe_fused_experts_workspace_bytes(ctypes.byref(fa)) > 0
