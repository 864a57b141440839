"""Fused MoE for MI355X: the host side of FlagGems-sglang's fused-MoE path.

Mirrors ``flaggems_sglang.ops.fused_moe`` of the reference
(``src/flaggems_sglang/ops/fused_moe.py``): the same entry points
(``triton_kernel_fused_experts``, ``fused_moe_flagos``), argument meaning and
error behaviour (``AssertionError("<name> is not supported")``,
``ValueError`` for an unknown activation).  Every op calls the HIP library
``libfmoe.so`` through its C ABI (``include/fmoe.h``); nothing here computes
the MoE in torch.

Additions the reference does not have (its fp8 arguments are asserted off,
``ops/fused_moe.py:154-169``, and it has no int4 path): the SGLang-style
plain-tensor ``fused_experts`` with fp8 block-scale W8A8 and int4 W4A16
weights, the routers ``topk_softmax`` / ``grouped_topk`` and SGLang's
``moe_align_block_size``.
"""

from __future__ import annotations

import ctypes
import logging
from dataclasses import dataclass, field
from types import SimpleNamespace
from typing import Optional

import torch

from .. import _lib
from .._lib import (W_BF16, W_FP8, W_INT4, W_INT4_TILED, W_MXFP4, W_MXFP4_TILED, check, lib, ptr,
                    require_cuda, stream_of)

logger = logging.getLogger(__name__)

_UNSUPPORTED_FEATURE_MSG = "{name} is not supported"


# ---------------------------------------------------------------------------
# routing containers (field names of triton_kernels.routing, which the
# reference builds at ops/fused_moe.py:125-130)
# ---------------------------------------------------------------------------
@dataclass
class ExptData:
    hist: torch.Tensor
    token_offs_raw: torch.Tensor
    token_offs_pad: dict = field(default_factory=dict)   # block_m -> [E+1] (tiles)
    block_pid_map: dict = field(default_factory=dict)    # block_m -> [max_tiles]
    n_tiles: dict = field(default_factory=dict)          # block_m -> [1] device int32


@dataclass
class RoutingData:
    gate_scal: torch.Tensor
    expt_hist: torch.Tensor
    n_expts_tot: int
    n_expts_act: int
    expt_data: Optional[ExptData] = None


@dataclass
class GatherIndx:
    src_indx: torch.Tensor
    dst_indx: torch.Tensor


@dataclass
class ScatterIndx:
    src_indx: torch.Tensor
    dst_indx: torch.Tensor


@dataclass
class CombineInput:
    """Stand-in for SGLang's StandardCombineInput when SGLang is absent."""
    hidden_states: torch.Tensor


# ---------------------------------------------------------------------------
# routers
# ---------------------------------------------------------------------------
def topk_softmax(gating_output: torch.Tensor, topk: int, renormalize: bool = True):
    """softmax -> top-k -> renormalise (tests/test_fused_moe.py:24-27).

    Returns ``(topk_weights fp32 [M, k], topk_ids int32 [M, k])``, descending."""
    require_cuda(gating_output)
    x = gating_output.float().contiguous()
    M, E = x.shape
    w = torch.empty(M, topk, dtype=torch.float32, device=x.device)
    ids = torch.empty(M, topk, dtype=torch.int32, device=x.device)
    check(lib().fmoe_topk_softmax(ptr(x), M, E, topk, int(renormalize), ptr(w), ptr(ids),
                                  stream_of(x)), "topk_softmax")
    return w, ids


def grouped_topk(gating_output: torch.Tensor, topk: int, num_expert_group: int,
                 topk_group: int, correction_bias: Optional[torch.Tensor] = None,
                 renormalize: bool = True, scoring_func: str = "sigmoid"):
    """DeepSeek-V3 grouped top-k (SGLang biased_grouped_topk semantics)."""
    require_cuda(gating_output, correction_bias)
    if scoring_func not in ("sigmoid", "softmax"):
        raise ValueError(f"Unsupported scoring function: {scoring_func}")
    x = gating_output.float().contiguous()
    b = None if correction_bias is None else correction_bias.float().contiguous()
    M, E = x.shape
    w = torch.empty(M, topk, dtype=torch.float32, device=x.device)
    ids = torch.empty(M, topk, dtype=torch.int32, device=x.device)
    check(lib().fmoe_grouped_topk(ptr(x), ptr(b), M, E, topk, num_expert_group, topk_group,
                                  0 if scoring_func == "sigmoid" else 1, int(renormalize),
                                  ptr(w), ptr(ids), stream_of(x)), "grouped_topk")
    return w, ids


# ---------------------------------------------------------------------------
# alignment
# ---------------------------------------------------------------------------
@dataclass
class _Align:
    expt_indx: torch.Tensor
    expt_scal: torch.Tensor
    topk_indx: torch.Tensor
    gate_indx: torch.Tensor
    gate_scal: torch.Tensor
    hist: torch.Tensor
    offs_raw: torch.Tensor
    offs_pad: torch.Tensor
    tile_map: torch.Tensor
    n_tiles: torch.Tensor
    sorted_token_ids: Optional[torch.Tensor]
    expert_ids: Optional[torch.Tensor]
    num_tokens_post_padded: Optional[torch.Tensor]
    block_m: int


def _ids_i32(topk_ids: torch.Tensor) -> torch.Tensor:
    return topk_ids if topk_ids.dtype == torch.int32 and topk_ids.is_contiguous() else \
        topk_ids.to(torch.int32).contiguous()


def _align(topk_weights, topk_ids, n_experts: int, block_m: int, sglang_format: bool,
           expert_map: Optional[torch.Tensor] = None) -> _Align:
    require_cuda(topk_weights, topk_ids, expert_map)
    L = lib()
    ids = _ids_i32(topk_ids)
    w = topk_weights.float().contiguous()
    M, k = ids.shape
    n = M * k
    dev = ids.device
    i32 = dict(dtype=torch.int32, device=dev)
    max_tiles = L.fmoe_max_tiles(n, n_experts)
    a = _Align(
        expt_indx=torch.empty(n, **i32), expt_scal=torch.empty(n, dtype=torch.float32, device=dev),
        topk_indx=torch.empty(n, **i32), gate_indx=torch.empty(n, **i32),
        gate_scal=torch.empty(n, dtype=torch.float32, device=dev), hist=torch.empty(n_experts, **i32),
        offs_raw=torch.empty(n_experts + 1, **i32), offs_pad=torch.empty(n_experts + 1, **i32),
        tile_map=torch.empty(max_tiles, **i32), n_tiles=torch.empty(1, **i32),
        sorted_token_ids=None, expert_ids=None, num_tokens_post_padded=None, block_m=block_m)
    if sglang_format:
        cap = L.fmoe_sorted_ids_len(n, n_experts, block_m)
        a.sorted_token_ids = torch.empty(cap, **i32)
        a.expert_ids = torch.empty(cap // block_m + 1, **i32)
        a.num_tokens_post_padded = torch.empty(1, **i32)
    o = _lib.AlignOut(*[ptr(getattr(a, f)) for f, _ in _lib.AlignOut._fields_])
    ws_bytes = L.fmoe_align_workspace_bytes(M, k, n_experts)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    emap = None if expert_map is None else _ids_i32(expert_map.view(1, -1)).view(-1)
    check(L.fmoe_align_ex(ptr(ids), ptr(w), M, k, n_experts, block_m, ptr(emap),
                          0 if emap is None else emap.numel(), ctypes.byref(o), ptr(ws), ws_bytes,
                          stream_of(ids)), "moe_align")
    return a


def moe_align_block_size(topk_ids: torch.Tensor, block_size: int, num_experts: int):
    """SGLang ``moe_align_block_size``: returns ``(sorted_token_ids, expert_ids,
    num_tokens_post_padded)``; token order inside an expert is ascending
    (stable), padding uses the sentinel ``topk_ids.numel()``."""
    w = torch.zeros(topk_ids.shape, dtype=torch.float32, device=topk_ids.device)
    a = _align(w, topk_ids, num_experts, block_size, sglang_format=True)
    return a.sorted_token_ids, a.expert_ids, a.num_tokens_post_padded


def _block_m(wtype: int, M: int, k: int, E: int, path: int, K: int, N: int) -> int:
    """The fused path's tile height for a K x N layer (fmoe_fused_block_m: the
    library's own choice, so stage-path routing always matches it)."""
    return lib().fmoe_fused_block_m(wtype, M, k, E, path, K, N)


def _standard_topk_to_triton_kernels(topk_weights, topk_ids, n_expts_tot, block_m: Optional[int] = None):
    """Convert standard top-k output to routing data (ops/fused_moe.py:103-130).

    The expert-sorted permutation, its inverse, the sorted gate weights, the
    histogram and ExptData come from one HIP alignment pass.  ExptData holds
    the tile map for ``block_m`` (default: the tile height the GEMMs will use);
    other tile heights are derived from the histogram on demand."""
    M, k = topk_ids.shape
    if block_m is None:
        block_m = lib().fmoe_choose_block_m(W_BF16, M, k, n_expts_tot, 0)
    a = _align(topk_weights, topk_ids, n_expts_tot, block_m, sglang_format=False)
    ed = ExptData(hist=a.hist, token_offs_raw=a.offs_raw, token_offs_pad={block_m: a.offs_pad},
                  block_pid_map={block_m: a.tile_map}, n_tiles={block_m: a.n_tiles})
    routing_data = RoutingData(a.gate_scal, a.hist, n_expts_tot, k, ed)
    gather_indx = GatherIndx(src_indx=a.topk_indx, dst_indx=a.gate_indx)
    scatter_indx = ScatterIndx(src_indx=a.gate_indx, dst_indx=a.topk_indx)
    return routing_data, gather_indx, scatter_indx


def _expt_data_for(routing_data: RoutingData, n_slots: int, block_m: int):
    """(offs_raw, offs_pad, tile_map, n_tiles) for ``block_m``: reuse the
    routing's own ExptData when it has this tile height, else derive it from
    the histogram (compute_expt_data_torch, ops/fused_moe.py:124)."""
    ed = routing_data.expt_data
    if ed is not None and block_m in getattr(ed, "block_pid_map", {}) and block_m in getattr(ed, "n_tiles", {}):
        return ed.token_offs_raw, ed.token_offs_pad[block_m], ed.block_pid_map[block_m], ed.n_tiles[block_m]
    L = lib()
    E = routing_data.n_expts_tot
    hist = routing_data.expt_hist.to(torch.int32).contiguous()
    dev = hist.device
    i32 = dict(dtype=torch.int32, device=dev)
    offs_raw = torch.empty(E + 1, **i32)
    offs_pad = torch.empty(E + 1, **i32)
    tile_map = torch.empty(L.fmoe_max_tiles(n_slots, E), **i32)
    n_tiles = torch.empty(1, **i32)
    check(L.fmoe_expt_data(ptr(hist), E, n_slots, block_m, ptr(offs_raw), ptr(offs_pad),
                           ptr(tile_map), ptr(n_tiles), stream_of(hist)), "expt_data")
    if isinstance(ed, ExptData):  # cache on this package's own containers only
        ed.token_offs_pad[block_m] = offs_pad
        ed.block_pid_map[block_m] = tile_map
        ed.n_tiles[block_m] = n_tiles
    return offs_raw, offs_pad, tile_map, n_tiles


# ---------------------------------------------------------------------------
# quantization
# ---------------------------------------------------------------------------
def per_token_group_quant_fp8(x: torch.Tensor, group_size: int = 128):
    """Dynamic 1 x group fp8-e4m3fn activation quant: ``(q, scale)`` with
    ``scale = max(amax, 1e-10) / 448`` per group."""
    require_cuda(x)
    x = x.contiguous()
    if x.dtype != torch.bfloat16:
        raise ValueError("per_token_group_quant_fp8: x must be bfloat16")
    M, K = x.shape
    q = torch.empty(M, K, dtype=torch.float8_e4m3fn, device=x.device)
    s = torch.empty(M, K // group_size, dtype=torch.float32, device=x.device)
    check(lib().fmoe_quant_fp8_group(ptr(x), M, K, group_size, ptr(q), ptr(s), stream_of(x)),
          "per_token_group_quant_fp8")
    return q, s


# ---------------------------------------------------------------------------
# GEMM stages over reference-format routing
# ---------------------------------------------------------------------------
def _wtype_and_check(use_fp8_w8a8, use_int4_w4a16, w1, w2, w1_scale, w2_scale, w1_zp, w2_zp,
                     block_shape, per_channel_quant, use_mxfp4_w4a16=False):
    assert per_channel_quant is False, _UNSUPPORTED_FEATURE_MSG.format(name="per_channel_quant")
    if int(bool(use_fp8_w8a8)) + int(bool(use_int4_w4a16)) + int(bool(use_mxfp4_w4a16)) > 1:
        raise ValueError("use_fp8_w8a8, use_int4_w4a16 and use_mxfp4_w4a16 are exclusive")
    if use_mxfp4_w4a16:
        assert block_shape is None or list(block_shape) in ([0, 32], [32]), \
            _UNSUPPORTED_FEATURE_MSG.format(name=f"block_shape={block_shape}")
        assert w1.dtype == torch.uint8 and w2.dtype == torch.uint8, "mxfp4 weights are packed uint8"
        assert w1_scale is not None and w2_scale is not None, "mxfp4 needs w1_scale and w2_scale"
        assert w1_scale.dtype in (torch.uint8, torch.float8_e8m0fnu) and \
            w2_scale.dtype in (torch.uint8, torch.float8_e8m0fnu), "mxfp4 scales are e8m0 bytes"
        assert w1_zp is None and w2_zp is None, _UNSUPPORTED_FEATURE_MSG.format(name="mxfp4 zero points")
        # 4-D weights: tiled by quant.tile_mxfp4 (both or neither)
        assert w1.dim() == w2.dim() and w1.dim() in (3, 4), \
            "mxfp4 weights must both be row-major [E, R, C/2] or both tiled [E, R/16, C/128, 1024]"
        return W_MXFP4_TILED if w1.dim() == 4 else W_MXFP4
    if use_fp8_w8a8:
        assert block_shape is not None and list(block_shape) == [128, 128], \
            _UNSUPPORTED_FEATURE_MSG.format(name=f"block_shape={block_shape}")
        assert w1.dtype == torch.float8_e4m3fn and w2.dtype == torch.float8_e4m3fn, \
            "fp8 weights must be float8_e4m3fn"
        assert w1_scale is not None and w2_scale is not None, "fp8 needs w1_scale and w2_scale"
        return W_FP8
    if use_int4_w4a16:
        assert block_shape is None or list(block_shape) in ([0, 128], [128]), \
            _UNSUPPORTED_FEATURE_MSG.format(name=f"block_shape={block_shape}")
        assert w1.dtype == torch.uint8 and w2.dtype == torch.uint8, "int4 weights are packed uint8"
        assert w1_scale is not None and w2_scale is not None and w1_zp is not None and w2_zp is not None, \
            "int4 needs w1_scale, w2_scale, w1_zp and w2_zp"
        # 4-D weights: the tiled layout of quant.tile_int4 (both or neither)
        assert w1.dim() == w2.dim() and w1.dim() in (3, 4), \
            "int4 weights must both be row-major [E, R, C/2] or both tiled [E, R/16, C/128, 1024]"
        return W_INT4_TILED if w1.dim() == 4 else W_INT4
    assert w1_scale is None, _UNSUPPORTED_FEATURE_MSG.format(name="w1_scale")
    assert w2_scale is None, _UNSUPPORTED_FEATURE_MSG.format(name="w2_scale")
    assert block_shape is None, _UNSUPPORTED_FEATURE_MSG.format(name="block_shape")
    assert w1.dtype == torch.bfloat16, "w1 must be bfloat16"
    assert w2.dtype == torch.bfloat16, "w2 must be bfloat16"
    return W_BF16


_ACTIVATIONS = {"silu": _lib.ACT_SILU, "gelu": _lib.ACT_GELU}


def _act_code(activation: str) -> int:
    """silu / gelu (ops/fused_moe.py:198-206); anything else raises the
    reference's ValueError."""
    if activation not in _ACTIVATIONS:
        raise ValueError(f"Unsupported FusedMoe activation: {activation}")
    return _ACTIVATIONS[activation]


def _weight_dims(w, wtype):
    """(experts, rows, reduction length) of a weight tensor in any layout."""
    if wtype in (W_INT4_TILED, W_MXFP4_TILED):
        assert w.shape[3] == 1024, "tiled 4-bit weights must be [E, R/16, C/128, 1024]"
        return w.shape[0], w.shape[1] * 16, w.shape[2] * 128
    nib = wtype in (W_INT4, W_MXFP4)
    return w.shape[0], w.shape[1], w.shape[2] * (2 if nib else 1)


def _run_stages(x, w13, w2, wtype, w13_scale, w2_scale, w13_zp, w2_zp, n_tokens, top_k,
                n_experts, topk_indx, gate_indx, gate_scal, offs_raw, offs_pad, tile_map, n_tiles,
                block_m, apply_router_weight_on_input, scale, combine=True, act=_lib.ACT_SILU,
                b13=None, b2=None, alpha=1.0, limit=0.0, slot_order=None):
    """GEMM1+activation -> GEMM2 -> top-k sum on prepared routing, SGLang
    layouts ``w13 [E, 2N, K]``, ``w2 [E, K, N]``; ``b13 [E, 2N]`` / ``b2 [E, K]``
    fp32 biases (bias path).

    ``combine=False`` returns the per-slot rows ``[M, k, K]`` bf16 instead of
    their sum: row ``(t, j)`` is token t's j-th slot in the routing's flat
    order (each token's experts ascending, the order of ``expt_indx``), or,
    with ``slot_order [M, k]`` (the rank of original column j in that order),
    token t's choice ``topk_ids[t, j]``.  A slot whose expert was dropped
    (expert map) is zero."""
    L = lib()
    M, K = x.shape
    N = _weight_dims(w2, wtype)[2]
    dev = x.device
    st = stream_of(x)
    r = _lib.Routing(ptr(topk_indx), ptr(gate_indx), ptr(gate_scal), ptr(offs_raw), ptr(offs_pad),
                     ptr(tile_map), ptr(n_tiles), n_tokens, top_k, n_experts, block_m,
                     L.fmoe_max_tiles(n_tokens * top_k, n_experts))
    slots = n_tokens * top_k
    # fp8: the prefill kernels take pre-quantized activations; the decode
    # kernels (block_m 16) quantize bf16 rows in-kernel
    quant_acts = wtype == W_FP8 and block_m != 16
    xa, xs = x, None
    if quant_acts:
        xa, xs = per_token_group_quant_fp8(x, 128)
    act_buf = torch.empty(slots, N, dtype=torch.bfloat16, device=dev)
    ep = _lib.Epilogue(act, ptr(b13), float(alpha), float(limit))
    check(L.fmoe_gemm1_ex(wtype, ptr(xa), ptr(xs), ptr(w13), ptr(w13_scale), ptr(w13_zp), K, N,
                          ctypes.byref(r), int(apply_router_weight_on_input), ctypes.byref(ep),
                          ptr(act_buf), 0, st), "gemm1")
    a2, a2s = act_buf, None
    if quant_acts:
        a2, a2s = per_token_group_quant_fp8(act_buf, 128)
    splits = L.fmoe_gemm2_splits(wtype, K, N, ctypes.byref(r), 0)
    y = torch.empty(splits, slots, K, dtype=torch.float32, device=dev)
    check(L.fmoe_gemm2_ex(wtype, ptr(a2), ptr(a2s), ptr(w2), ptr(w2_scale), ptr(w2_zp), K, N,
                          ctypes.byref(r), int(not apply_router_weight_on_input), ptr(b2), ptr(y),
                          splits, 0, st), "gemm2")
    if not combine:
        # per-slot rows: moe_sum over "tokens" = slots with one choice each
        # (split planes summed in fixed order, dropped slots -> 0)
        g = gate_indx if slot_order is None else \
            gate_indx.view(n_tokens, top_k).gather(1, slot_order).contiguous()
        per = torch.empty(n_tokens * top_k, K, dtype=torch.bfloat16, device=dev)
        check(L.fmoe_moe_sum(ptr(y), splits, ptr(g), n_tokens * top_k, 1, K, 1.0, ptr(per), st),
              "moe_sum")
        return per.view(n_tokens, top_k, K)
    out = torch.empty(M, K, dtype=torch.bfloat16, device=dev)
    check(L.fmoe_moe_sum(ptr(y), splits, ptr(gate_indx), M, top_k, K, float(scale), ptr(out), st),
          "moe_sum")
    return out


def _as_sglang_layout(w: torch.Tensor) -> torch.Tensor:
    """matmul_ogs layout [E, K_in, N_out] -> kernel layout [E, N_out, K_in].
    A transposed view of a contiguous SGLang tensor is used as is; a truly
    [E, K_in, N_out]-contiguous tensor is transposed once here (the reference
    pays the same copy in fused_moe_flagos, ops/fused_moe.py:326-327)."""
    t = w.transpose(-1, -2)
    return t if t.is_contiguous() else t.contiguous()


def triton_kernel_fused_experts(
    hidden_states: torch.Tensor,
    w1: torch.Tensor,
    w2: torch.Tensor,
    routing_data,
    gather_indx,
    scatter_indx,
    inplace: bool = False,
    activation: str = "silu",
    apply_router_weight_on_input: bool = False,
    use_fp8_w8a8: bool = False,
    per_channel_quant: bool = False,
    global_num_experts: int = -1,
    expert_map: Optional[torch.Tensor] = None,
    w1_scale: Optional[torch.Tensor] = None,
    w2_scale: Optional[torch.Tensor] = None,
    a1_scale: Optional[torch.Tensor] = None,
    a2_scale: Optional[torch.Tensor] = None,
    block_shape: Optional[list[int]] = None,
) -> torch.Tensor:
    """Drop-in for ``triton_kernel_fused_experts`` (ops/fused_moe.py:133-216).

    ``w1 [E, K, 2N]`` and ``w2 [E, N, K]`` in matmul_ogs layout (or transposed
    views of SGLang-layout tensors); routing objects as built by
    ``_standard_topk_to_triton_kernels``.  With ``use_fp8_w8a8`` and
    ``block_shape=[128, 128]`` the fp8 block path runs (weights fp8 in the same
    layouts, scales ``[E, 2N/128, K/128]`` / ``[E, K/128, N/128]``); the
    reference asserts this off.  ``scatter_indx=None`` returns the per-slot
    outputs ``[M, k, K]`` (token-major, experts ascending) without combining.
    """
    logger.debug("FLAGGEMS_SGLANG FUSED_MOE")
    assert expert_map is None, _UNSUPPORTED_FEATURE_MSG.format(name="expert_map")
    assert a1_scale is None, _UNSUPPORTED_FEATURE_MSG.format(name="a1_scale")
    assert a2_scale is None, _UNSUPPORTED_FEATURE_MSG.format(name="a2_scale")
    assert inplace is False, "Inplace is not supported"
    if not use_fp8_w8a8:
        assert w1_scale is None, _UNSUPPORTED_FEATURE_MSG.format(name="w1_scale")
        assert w2_scale is None, _UNSUPPORTED_FEATURE_MSG.format(name="w2_scale")
        assert block_shape is None, _UNSUPPORTED_FEATURE_MSG.format(name="block_shape")
    assert hidden_states.ndim == 2, "hidden_states must be 2D"
    assert hidden_states.dtype == torch.bfloat16, "hidden_states must be bfloat16"
    if not use_fp8_w8a8:
        assert w1.dtype == torch.bfloat16, "w1 must be bfloat16"
        assert w2.dtype == torch.bfloat16, "w2 must be bfloat16"
    assert hidden_states.shape[-1] == w1.shape[-2], "hidden size mismatch"
    assert w2.shape[-1] == w1.shape[1], "intermediate size mismatch"
    act = _act_code(activation)
    wtype = _wtype_and_check(use_fp8_w8a8, False, w1, w2, w1_scale, w2_scale, None, None,
                             block_shape, per_channel_quant)
    require_cuda(hidden_states, w1, w2)

    x = hidden_states.contiguous()
    M = x.shape[0]
    k = routing_data.n_expts_act
    E = routing_data.n_expts_tot
    w13 = _as_sglang_layout(w1)
    w2t = _as_sglang_layout(w2)
    s13 = None if w1_scale is None else _as_sglang_layout(w1_scale)
    s2 = None if w2_scale is None else _as_sglang_layout(w2_scale)
    bm = _block_m(wtype, M, k, E, 0, x.shape[1], w2.shape[1])
    offs_raw, offs_pad, tile_map, n_tiles = _expt_data_for(routing_data, M * k, bm)
    topk_indx = gather_indx.src_indx.to(torch.int32).contiguous()
    gate_indx = gather_indx.dst_indx.to(torch.int32).contiguous()
    gate_scal = routing_data.gate_scal.float().contiguous()
    return _run_stages(x, w13, w2t, wtype, s13, s2, None, None, M, k, E, topk_indx, gate_indx,
                       gate_scal, offs_raw, offs_pad, tile_map, n_tiles, bm,
                       apply_router_weight_on_input, 1.0, combine=scatter_indx is not None, act=act)


def triton_kernel_fused_experts_with_bias(
    hidden_states: torch.Tensor,
    w1: torch.Tensor,
    w1_pcg,
    b1: torch.Tensor,
    w2: torch.Tensor,
    w2_pcg,
    b2: torch.Tensor,
    routing_data,
    gather_indx,
    scatter_indx,
    inplace: bool = False,
    activation: str = "silu",
    apply_router_weight_on_input: bool = False,
    global_num_experts: int = -1,
    gemm1_alpha: Optional[float] = None,
    gemm1_clamp_limit: Optional[float] = None,
) -> torch.Tensor:
    """Drop-in for ``triton_kernel_fused_experts_with_bias`` (ops/fused_moe.py:219-309).

    ``w1 [E, K, 2N]`` with interleaved gate / linear columns (gate 2j, linear
    2j+1), ``b1 [E, 2N]``, ``w2 [E, N, K]``, ``b2 [E, K]``; ``activation="silu"``
    selects the fused swiglu of the reference (:258-259):
    ``g = min(x_2j + b, limit)``, ``l = clamp(x_2j+1 + b, -limit, limit)``,
    ``act = g * sigmoid(alpha * g) * (l + 1)`` on the fp32 GEMM1 result, then
    the routing weight when applied on the input; GEMM2 adds ``b2`` before the
    routing weight.  ``gemm1_alpha=None`` means 1, ``gemm1_clamp_limit=None`` no
    clamp.

    ``w1_pcg`` / ``w2_pcg`` (matmul_ogs precision configs): None for bf16
    weights; for MXFP4 weights (OCP e2m1 + e8m0 block scales, W4A16) objects
    whose ``weight_scale`` holds the block scales as plain row-major tensors,
    ``[E, K/32, 2N]`` / ``[E, N/32, K]`` uint8 (or float8_e8m0fnu), with
    ``w1 [E, K/2, 2N]`` / ``w2 [E, N/2, K]`` uint8 packed along the reduction
    dim (low nibble = even element).  triton_kernels' swizzled value / scale
    layouts are not accepted.
    """
    logger.debug("FLAGGEMS_SGLANG FUSED_MOE_WITH_BIAS")
    assert inplace is False, "Inplace is not supported"
    assert hidden_states.dtype == torch.bfloat16, "hidden_states must be bfloat16"
    if activation != "silu":
        raise ValueError(f"Unsupported FusedMoe activation: {activation}")
    assert hidden_states.ndim == 2, "hidden_states must be 2D"
    mx = w1_pcg is not None or w2_pcg is not None
    if mx:
        assert w1_pcg is not None and w2_pcg is not None, "w1_pcg and w2_pcg go together"
        s1, s2 = _pcg_scale(w1_pcg, "w1_pcg"), _pcg_scale(w2_pcg, "w2_pcg")
        assert w1.dtype == torch.uint8 and w2.dtype == torch.uint8, "mxfp4 weights are packed uint8"
        Kh = w1.shape[1] * 2
    else:
        assert w1.dtype == torch.bfloat16, "w1 must be bfloat16"
        assert w2.dtype == torch.bfloat16, "w2 must be bfloat16"
        Kh = w1.shape[1]
    assert hidden_states.shape[-1] == Kh, "hidden size mismatch"
    assert w2.shape[-1] == Kh, "intermediate size mismatch"
    assert b1 is not None and b2 is not None, "Bias execution requires both w13_bias and w2_bias"
    E = routing_data.n_expts_tot
    assert tuple(b1.shape) == (E, w1.shape[2]) and tuple(b2.shape) == (E, w2.shape[2]), \
        "bias shape mismatch"
    require_cuda(hidden_states, w1, w2, b1, b2)
    x = hidden_states.contiguous()
    M = x.shape[0]
    k = routing_data.n_expts_act
    w13 = _as_sglang_layout(w1)
    w2t = _as_sglang_layout(w2)
    wtype, s13, s2t = _lib.W_BF16, None, None
    if mx:
        wtype = W_MXFP4
        s13, s2t = _as_sglang_layout(s1.view(torch.uint8)), _as_sglang_layout(s2.view(torch.uint8))
        N2 = w13.shape[1]
        assert tuple(s13.shape) == (E, N2, Kh // 32) and tuple(s2t.shape) == (E, Kh, w2t.shape[2] * 2 // 32), \
            "mxfp4 scale shapes do not match the weights"
        require_cuda(s13, s2t)
    bm = lib().fmoe_choose_block_m(wtype, M, k, E, 0)
    offs_raw, offs_pad, tile_map, n_tiles = _expt_data_for(routing_data, M * k, bm)
    topk_indx = gather_indx.src_indx.to(torch.int32).contiguous()
    gate_indx = gather_indx.dst_indx.to(torch.int32).contiguous()
    gate_scal = routing_data.gate_scal.float().contiguous()
    return _run_stages(x, w13, w2t, wtype, s13, s2t, None, None, M, k, E, topk_indx,
                       gate_indx, gate_scal, offs_raw, offs_pad, tile_map, n_tiles, bm,
                       apply_router_weight_on_input, 1.0, combine=scatter_indx is not None,
                       act=_lib.ACT_SWIGLU, b13=b1.float().contiguous(), b2=b2.float().contiguous(),
                       alpha=1.0 if gemm1_alpha is None else float(gemm1_alpha),
                       limit=0.0 if gemm1_clamp_limit is None else float(gemm1_clamp_limit))


def _pcg_scale(pcg, name):
    """The MXFP4 block scales of a precision config (``weight_scale``)."""
    sc = getattr(pcg, "weight_scale", None)
    assert isinstance(sc, torch.Tensor), _UNSUPPORTED_FEATURE_MSG.format(
        name=f"{name} without a plain weight_scale tensor")
    assert sc.dtype in (torch.uint8, torch.float8_e8m0fnu), f"{name}.weight_scale must be e8m0 bytes"
    return sc


# ---------------------------------------------------------------------------
# plain-tensor entry point (SGLang fused_experts style, SGLang layouts)
# ---------------------------------------------------------------------------
def fused_experts(
    hidden_states: torch.Tensor,
    w1: torch.Tensor,
    w2: torch.Tensor,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    inplace: bool = False,
    activation: str = "silu",
    apply_router_weight_on_input: bool = False,
    use_fp8_w8a8: bool = False,
    use_int4_w4a16: bool = False,
    per_channel_quant: bool = False,
    w1_scale: Optional[torch.Tensor] = None,
    w2_scale: Optional[torch.Tensor] = None,
    w1_zp: Optional[torch.Tensor] = None,
    w2_zp: Optional[torch.Tensor] = None,
    a1_scale: Optional[torch.Tensor] = None,
    a2_scale: Optional[torch.Tensor] = None,
    block_shape: Optional[list[int]] = None,
    routed_scaling_factor: Optional[float] = None,
    no_combine: bool = False,
    path: int = 0,
    expert_map: Optional[torch.Tensor] = None,
    global_num_experts: int = -1,
    use_mxfp4_w4a16: bool = False,
) -> torch.Tensor:
    """Whole fused MoE in one C call (align -> GEMM1+SiLU -> GEMM2 -> top-k sum).

    Layouts (SGLang layer): ``w1 [E, 2N, K]``, ``w2 [E, K, N]``;
      fp8  (``use_fp8_w8a8``, ``block_shape=[128,128]``): float8_e4m3fn weights,
           ``w1_scale [E, 2N/128, K/128]``, ``w2_scale [E, K/128, N/128]`` fp32;
           activations quantized per 1x128 group inside the call;
      int4 (``use_int4_w4a16``, group 128): ``w1 [E, 2N, K/2]`` / ``w2 [E, K, N/2]``
           uint8 (two uint4 per byte, low nibble first), ``w1_scale [E, K/128, 2N]``
           / ``w2_scale [E, N/128, K]`` fp16, ``w1_zp [E, K/128, N]`` /
           ``w2_zp [E, N/128, K/2]`` uint8 (two uint4 zeros per byte);
           The same weights tiled by ``quant.tile_int4`` (4-D ``[E, R/16,
           C/128, 1024]``, scales and zeros unchanged) take the decode kernels'
           contiguous-block loads (MXFP4 likewise, ``quant.tile_mxfp4``);
      mxfp4 (``use_mxfp4_w4a16``): OCP MXFP4 ``w1 [E, 2N, K/2]`` / ``w2 [E, K, N/2]``
           uint8 (two e2m1 per byte, low nibble first), ``w1_scale [E, 2N, K/32]`` /
           ``w2_scale [E, K, N/32]`` e8m0 bytes; bf16 activations (the streaming
           kernels, like int4).
    ``path``: 0 choose, 1 prefill kernels, 2 decode kernels.
    ``expert_map`` (expert parallel): ``topk_ids`` hold global expert ids,
    ``expert_map [global_num_experts]`` int maps each to a local expert (index
    into ``w1`` / ``w2``) or -1; choices of non-local experts are dropped, so
    each token gets the sum over its local experts only.
    """
    assert inplace is False, "Inplace is not supported"
    assert a1_scale is None, _UNSUPPORTED_FEATURE_MSG.format(name="a1_scale")
    assert a2_scale is None, _UNSUPPORTED_FEATURE_MSG.format(name="a2_scale")
    act = _act_code(activation)
    assert hidden_states.ndim == 2 and hidden_states.dtype == torch.bfloat16, \
        "hidden_states must be 2D bfloat16"
    wtype = _wtype_and_check(use_fp8_w8a8, use_int4_w4a16, w1, w2, w1_scale, w2_scale, w1_zp,
                             w2_zp, block_shape, per_channel_quant, use_mxfp4_w4a16)
    require_cuda(hidden_states, w1, w2, topk_weights, topk_ids, w1_scale, w2_scale, w1_zp, w2_zp)
    x = hidden_states.contiguous()
    M, K = x.shape
    E, rows1, kin = _weight_dims(w1, wtype)
    _, rows2, N = _weight_dims(w2, wtype)
    k = topk_ids.shape[1]
    if wtype in (W_MXFP4, W_MXFP4_TILED):
        assert tuple(w1_scale.shape) == (E, 2 * N, K // 32) and tuple(w2_scale.shape) == (E, K, N // 32), \
            "mxfp4 scales must be [E, 2N, K/32] and [E, K, N/32]"
        w1_scale, w2_scale = w1_scale.view(torch.uint8), w2_scale.view(torch.uint8)
    assert kin == K and rows1 == 2 * N and rows2 == K and w2.shape[0] == E, "weight shapes do not match"
    for t in (w1, w2, w1_scale, w2_scale, w1_zp, w2_zp):
        if t is not None:
            assert t.is_contiguous(), "weights and scales must be contiguous"
    scale = 1.0 if routed_scaling_factor is None else float(routed_scaling_factor)
    emap = None
    if expert_map is not None:
        require_cuda(expert_map)
        n_global = global_num_experts if global_num_experts > 0 else expert_map.numel()
        assert expert_map.numel() == n_global, "expert_map must have global_num_experts entries"
        emap = _ids_i32(expert_map.view(1, -1)).view(-1)
    if no_combine:
        # SGLang's no_combine contract: [M, k, K] with slot (t, j) = the
        # expert topk_ids[t, j] (routed_scaling_factor not applied, as in the
        # reference hook, ops/fused_moe.py:399-404)
        a = _align(topk_weights, topk_ids, E, _block_m(wtype, M, k, E, path, K, N), False,
                   expert_map=emap)
        return _run_stages(x, w1, w2, wtype, w1_scale, w2_scale, w1_zp, w2_zp, M, k, E,
                           a.topk_indx, a.gate_indx, a.gate_scal, a.offs_raw, a.offs_pad, a.tile_map,
                           a.n_tiles, a.block_m, apply_router_weight_on_input, 1.0, combine=False,
                           act=act, slot_order=_slot_order(topk_ids, emap))
    ids = _ids_i32(topk_ids)
    tw = topk_weights.float().contiguous()
    out = torch.empty(M, K, dtype=torch.bfloat16, device=x.device)
    args = _lib.FusedArgs(
        wtype, ptr(x), M, K, N, E, k, ptr(w1), ptr(w2), ptr(w1_scale), ptr(w2_scale), ptr(w1_zp),
        ptr(w2_zp), 128, ptr(tw), ptr(ids), int(apply_router_weight_on_input), scale, path,
        ptr(out), None, 0, act, None, None, 1.0, 0.0, ptr(emap), 0 if emap is None else emap.numel())
    L = lib()
    nbytes = L.fmoe_fused_experts_workspace_bytes(ctypes.byref(args))
    if nbytes == 0:
        # the size query refuses invalid arguments: run the call for its error
        check(L.fmoe_fused_experts(ctypes.byref(args), stream_of(x)), "fused_experts")
        raise RuntimeError("fused_experts: workspace query failed")
    ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    args.workspace = ptr(ws)
    args.workspace_bytes = nbytes
    check(L.fmoe_fused_experts(ctypes.byref(args), stream_of(x)), "fused_experts")
    return out


def _slot_order(topk_ids: torch.Tensor, emap: Optional[torch.Tensor]) -> torch.Tensor:
    """[M, k] int64: the position of column j of ``topk_ids`` in its row after
    the stable per-row sort by (local) expert id that the routing applies
    (ops/fused_moe.py:113; ids dropped by the expert map sort as -1)."""
    ids = topk_ids.long()
    if emap is not None:
        ok = (ids >= 0) & (ids < emap.numel())
        ids = torch.where(ok, emap.long()[ids.clamp(0, emap.numel() - 1)], torch.full_like(ids, -1))
    order = torch.sort(ids, dim=1, stable=True).indices
    return torch.argsort(order, dim=1)


# ---------------------------------------------------------------------------
# SGLang runner hook
# ---------------------------------------------------------------------------
def _is_triton_routing(topk_output) -> bool:
    """SGLang's TopKOutputChecker.format_is_triton_kernels (ops/fused_moe.py:339),
    by structure rather than class: a ``(routing_data, gather_indx,
    scatter_indx)`` triple whose routing data has the triton_kernels
    ``RoutingData`` fields and whose indices have ``src_indx`` / ``dst_indx``
    (SGLang's TritonKernelTopKOutput, this package's own containers, or any
    other object with those fields)."""
    fmt = getattr(topk_output, "format", None)
    if fmt is not None and getattr(fmt, "name", None) == "TRITON_KERNEL":
        return True
    if not isinstance(topk_output, (tuple, list)) or len(topk_output) != 3:
        return False
    rd, gi, si = topk_output
    return (all(hasattr(rd, f) for f in ("gate_scal", "expt_hist", "n_expts_tot", "n_expts_act"))
            and all(hasattr(o, f) for o in (gi, si) for f in ("src_indx", "dst_indx")))


def _combine_input(hidden_states):
    try:
        from sglang.srt.layers.moe.token_dispatcher.standard import StandardCombineInput
    except Exception:
        return CombineInput(hidden_states=hidden_states)
    return StandardCombineInput(hidden_states=hidden_states)


def fused_moe_flagos(obj, layer: torch.nn.Module, dispatch_output):
    """SGLang integration wrapper (ops/fused_moe.py:312-406).

    Reads the same fields: ``layer.w13_weight [E, 2N, K]`` and
    ``layer.w2_weight [E, K, N]`` (used in place, no per-call transpose),
    optional ``w13_weight_bias``/``w2_weight_bias`` (bias path, fused swiglu with
    ``gemm1_alpha`` / ``gemm1_clamp_limit`` from the config),
    ``dispatch_output.hidden_states`` and ``.topk_output`` (either
    ``topk_weights``/``topk_ids`` or a triton_kernels-format
    ``(routing_data, gather_indx, scatter_indx)`` triple), and
    ``obj.runner.config`` (``num_experts``, ``no_combine``, ``activation``,
    ``apply_router_weight_on_input``, ``routed_scaling_factor``).
    fp8 block-scale layers carry ``w13_weight_scale_inv``/``w2_weight_scale_inv``;
    int4 layers ``w13_qweight``/``w13_scales``/``w13_qzeros`` and the w2 ones,
    in the W4A16 layout -- or in a checkpoint layout named by
    ``layer.fmoe_int4_checkpoint_format`` ("awq", "gptq", "gptq_v2"), which the
    first call converts in place (``formats.repack_layer_int4``).
    """
    cfg = obj.runner.config
    b13 = getattr(layer, "w13_weight_bias", None)
    b2 = getattr(layer, "w2_weight_bias", None)
    hidden_states = dispatch_output.hidden_states
    topk_output = dispatch_output.topk_output
    no_combine = bool(getattr(cfg, "no_combine", False))
    rsf = getattr(cfg, "routed_scaling_factor", None)
    scale = None if (rsf is None or rsf == 1.0 or no_combine) else rsf
    activation = getattr(cfg, "activation", "silu")
    on_input = bool(getattr(cfg, "apply_router_weight_on_input", False))

    if hasattr(layer, "w13_qweight"):
        ckpt_format = getattr(layer, "fmoe_int4_checkpoint_format", None)
        if ckpt_format is not None:
            from flaggems_sglang.formats import repack_layer_int4

            repack_layer_int4(layer, ckpt_format)
        quant = dict(use_int4_w4a16=True, w1_scale=layer.w13_scales, w2_scale=layer.w2_scales,
                     w1_zp=layer.w13_qzeros, w2_zp=layer.w2_qzeros)
        w13, w2 = layer.w13_qweight, layer.w2_qweight
    elif layer.w13_weight.dtype == torch.uint8 and getattr(layer, "w13_weight_scale", None) is not None:
        # MXFP4 layer (SGLang Mxfp4 naming): e2m1 [E, 2N, K/2] + e8m0 [E, 2N, K/32]
        quant = dict(use_mxfp4_w4a16=True, w1_scale=layer.w13_weight_scale, w2_scale=layer.w2_weight_scale)
        w13, w2 = layer.w13_weight, layer.w2_weight
    elif getattr(layer, "w13_weight_scale_inv", None) is not None:
        quant = dict(use_fp8_w8a8=True, block_shape=[128, 128], w1_scale=layer.w13_weight_scale_inv,
                     w2_scale=layer.w2_weight_scale_inv)
        w13, w2 = layer.w13_weight, layer.w2_weight
    else:
        quant = {}
        w13, w2 = layer.w13_weight, layer.w2_weight

    if b13 is not None or b2 is not None:
        # bias path (ops/fused_moe.py:364-383): fused swiglu, bf16 or MXFP4 weights
        assert b13 is not None and b2 is not None, "Bias execution requires both w13_bias and w2_bias"
        assert not quant or quant.get("use_mxfp4_w4a16"), \
            _UNSUPPORTED_FEATURE_MSG.format(name="fp8 / int4 weights with bias")
        pcg13 = pcg2 = None
        if quant:
            # matmul_ogs orientation views of the SGLang-layout scales (no copy)
            pcg13 = SimpleNamespace(weight_scale=quant["w1_scale"].transpose(-1, -2))
            pcg2 = SimpleNamespace(weight_scale=quant["w2_scale"].transpose(-1, -2))
        if _is_triton_routing(topk_output):
            routing_data, gather_indx, scatter_indx = topk_output
        else:
            routing_data, gather_indx, scatter_indx = _standard_topk_to_triton_kernels(
                topk_output.topk_weights, topk_output.topk_ids, cfg.num_experts)
        out = triton_kernel_fused_experts_with_bias(
            hidden_states, w13.transpose(-1, -2), pcg13, b13, w2.transpose(-1, -2), pcg2, b2,
            routing_data, gather_indx, None if no_combine else scatter_indx, activation=activation,
            apply_router_weight_on_input=on_input, gemm1_alpha=getattr(cfg, "gemm1_alpha", None),
            gemm1_clamp_limit=getattr(cfg, "gemm1_clamp_limit", None))
        if scale is not None:
            out.mul_(scale)
    elif _is_triton_routing(topk_output):
        routing_data, gather_indx, scatter_indx = topk_output
        assert not quant.get("use_int4_w4a16"), _UNSUPPORTED_FEATURE_MSG.format(
            name="int4 with triton_kernels routing")
        out = triton_kernel_fused_experts(
            hidden_states, w13.transpose(-1, -2), w2.transpose(-1, -2), routing_data, gather_indx,
            None if no_combine else scatter_indx, activation=activation,
            apply_router_weight_on_input=on_input,
            use_fp8_w8a8=bool(quant.get("use_fp8_w8a8")),
            w1_scale=None if not quant else quant["w1_scale"].transpose(-1, -2),
            w2_scale=None if not quant else quant["w2_scale"].transpose(-1, -2),
            block_shape=quant.get("block_shape"))
        if scale is not None:
            out.mul_(scale)
    else:
        out = fused_experts(
            hidden_states, w13, w2, topk_output.topk_weights, topk_output.topk_ids,
            activation=activation, apply_router_weight_on_input=on_input,
            routed_scaling_factor=scale, no_combine=no_combine, **quant)
    return _combine_input(out)
