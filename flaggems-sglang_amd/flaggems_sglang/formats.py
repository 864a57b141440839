"""Checkpoint weight formats of the W4A16 MoE path, converted once at load.

SGLang loads int4 MoE layers from AWQ (AutoAWQ "gemm" packing) and GPTQ
(AutoGPTQ packing, format v1 or v2) checkpoints.  The W4A16 kernels read
their own layout (``qweight [E, N, K/2] u8``, ``scales [E, K/g, N] fp16``,
``zeros [E, K/g, N/2] u8``; N = output rows, K = reduction dim); the
functions here repack a checkpoint's stacked expert tensors into it with one
HIP pass per weight (``fmoe_repack_int4``), so nothing is re-laid out per
forward -- unlike the reference's per-call ``transpose().contiguous()``
(ops/fused_moe.py:326-327).  The converted weights dequantize to exactly the
checkpoint's values.

For GEMM1 the checkpoint's gate and up projections are stacked along the
output dim (gate rows first), as SGLang's ``w13`` parameters are.
"""

from __future__ import annotations

import torch

from flaggems_sglang._lib import check, lib, ptr, require_cuda, stream_of

FMOE_INT4_AWQ, FMOE_INT4_GPTQ_V1, FMOE_INT4_GPTQ_V2 = 0, 1, 2
_GPTQ_VERSIONS = {"gptq": FMOE_INT4_GPTQ_V1, "gptq_v1": FMOE_INT4_GPTQ_V1, "gptq_v2": FMOE_INT4_GPTQ_V2}


def _check_int32(name, t, ndim=3):
    if t.dtype != torch.int32 or t.dim() != ndim:
        raise ValueError(f"{name} must be an int32 tensor with {ndim} dims, got {t.dtype} {tuple(t.shape)}")


def _repack(fmt, qweight, qzeros, scales, K, N, group):
    require_cuda(qweight, qzeros, scales)
    if scales.dtype != torch.float16:
        raise ValueError(f"scales must be float16, got {scales.dtype}")
    E = qweight.shape[0]
    if tuple(scales.shape) != (E, K // group, N) or tuple(qzeros.shape) != (E, K // group, N // 8):
        raise ValueError(f"scales {tuple(scales.shape)} / qzeros {tuple(qzeros.shape)} do not match "
                         f"E={E}, K={K}, N={N}, group={group}")
    dev = qweight.device
    q = torch.empty(E, N, K // 2, dtype=torch.uint8, device=dev)
    sc = torch.empty(E, K // group, N, dtype=torch.float16, device=dev)
    z = torch.empty(E, K // group, N // 2, dtype=torch.uint8, device=dev)
    bad = torch.zeros(1, dtype=torch.int32, device=dev)
    qweight, qzeros, scales = qweight.contiguous(), qzeros.contiguous(), scales.contiguous()
    check(lib().fmoe_repack_int4(fmt, ptr(qweight), ptr(qzeros), ptr(scales), E, K, N, group,
                                 ptr(q), ptr(sc), ptr(z), ptr(bad), stream_of(qweight)),
          "repack_int4")
    return q, sc, z, bad


def repack_awq_moe(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor):
    """AWQ expert weights -> the W4A16 layout.

    ``qweight int32 [E, K, N/8]``, ``qzeros int32 [E, K/g, N/8]``, ``scales
    fp16 [E, K/g, N]`` (word j of a row holds columns 8j..8j+7, nibble i =
    column 8j + (0, 2, 4, 6, 1, 3, 5, 7)[i]; w = (q - z) * s).  The group size
    follows from the shapes.  Returns ``(qweight [E, N, K/2] u8, scales
    [E, K/g, N] fp16, zeros [E, K/g, N/2] u8)``."""
    _check_int32("qweight", qweight)
    _check_int32("qzeros", qzeros)
    E, K, N8 = qweight.shape
    N = N8 * 8
    if qzeros.shape[1] == 0 or K % qzeros.shape[1]:
        raise ValueError(f"qzeros groups {qzeros.shape[1]} do not divide K={K}")
    group = K // qzeros.shape[1]
    q, sc, z, _ = _repack(FMOE_INT4_AWQ, qweight, qzeros, scales, K, N, group)
    return q, sc, z


def repack_gptq_moe(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor,
                    g_idx: torch.Tensor | None = None, checkpoint_format: str = "gptq"):
    """GPTQ expert weights -> the W4A16 layout.

    ``qweight int32 [E, K/8, N]`` (nibble j of word i = row 8i + j),
    ``qzeros int32 [E, K/g, N/8]`` (nibble j of word c = column 8c + j),
    ``scales fp16 [E, K/g, N]``.  ``checkpoint_format`` "gptq" (v1: zeros
    stored minus one) or "gptq_v2" (zeros stored as is).  Act-order
    checkpoints (``g_idx`` other than ``k // g``) are not supported.  A v1
    zero of 16 (stored 15) cannot be held in 4 bits and raises ValueError."""
    if checkpoint_format not in _GPTQ_VERSIONS:
        raise ValueError(f"unknown GPTQ checkpoint format {checkpoint_format!r}")
    _check_int32("qweight", qweight)
    _check_int32("qzeros", qzeros)
    E, K8, N = qweight.shape
    K = K8 * 8
    if qzeros.shape[1] == 0 or K % qzeros.shape[1]:
        raise ValueError(f"qzeros groups {qzeros.shape[1]} do not divide K={K}")
    group = K // qzeros.shape[1]
    if g_idx is not None:
        want = torch.arange(K, device=g_idx.device, dtype=torch.int64) // group
        gi = g_idx.to(torch.int64)
        if gi.shape[-1] != K or not bool((gi == want).all()):
            raise AssertionError("GPTQ act-order (desc_act) is not supported")
    q, sc, z, bad = _repack(_GPTQ_VERSIONS[checkpoint_format], qweight, qzeros, scales, K, N, group)
    if checkpoint_format != "gptq_v2" and int(bad.item()):
        raise ValueError(f"GPTQ v1 checkpoint holds {int(bad.item())} zero point(s) of 16, "
                         "which 4-bit zeros cannot represent")
    return q, sc, z


def repack_layer_int4(layer: torch.nn.Module, checkpoint_format: str, tiled: bool = True) -> None:
    """Convert an int4 MoE layer's checkpoint tensors in place, once.

    Reads ``w13_qweight`` / ``w13_qzeros`` / ``w13_scales`` and the ``w2_``
    ones in ``checkpoint_format`` ("awq", "gptq", "gptq_v2"; optional
    ``w13_g_idx`` / ``w2_g_idx``) and replaces them with the W4A16 layout that
    ``fused_moe_flagos`` passes to the kernels -- with ``tiled`` (default) the
    weights in the tiled layout of ``quant.tile_int4``, which the decode
    kernels stream faster; marks the layer so a second call is a no-op."""
    if getattr(layer, "fmoe_int4_repacked", False):
        return
    for pre in ("w13", "w2"):
        qw = getattr(layer, f"{pre}_qweight")
        qz = getattr(layer, f"{pre}_qzeros")
        sc = getattr(layer, f"{pre}_scales")
        if checkpoint_format == "awq":
            q, s, z = repack_awq_moe(qw, qz, sc)
        else:
            q, s, z = repack_gptq_moe(qw, qz, sc, getattr(layer, f"{pre}_g_idx", None), checkpoint_format)
        if tiled:
            from .quant import tile_int4

            q = tile_int4(q)
        for name, t in (("qweight", q), ("scales", s), ("qzeros", z)):
            old = getattr(layer, f"{pre}_{name}")
            if isinstance(old, torch.nn.Parameter):
                t = torch.nn.Parameter(t, requires_grad=False)
            setattr(layer, f"{pre}_{name}", t)
    layer.fmoe_int4_repacked = True
