"""Weight preparation for the quantized fused-MoE paths (load time, not the
hot path): fp8-e4m3fn 128x128 block quantization, uint4 group and MXFP4
quantization into the layouts ``fused_experts`` reads (plain torch, on
whatever device the weights live), and the tiling of int4 weights for the
decode kernels (``tile_int4``, a HIP kernel).
"""

from __future__ import annotations

import torch

from . import _lib

FP8_MAX = 448.0
FP8_EPS = 1e-10


def quantize_fp8_block(w: torch.Tensor, block=(128, 128)):
    """``w [E, R, C]`` -> (float8_e4m3fn ``[E, R, C]``, fp32 scales
    ``[E, R/bR, C/bC]``) with scale = max(amax, 1e-10) / 448 per block."""
    E, R, C = w.shape
    bR, bC = block
    if R % bR or C % bC:
        raise ValueError(f"quantize_fp8_block: {R}x{C} is not a multiple of {bR}x{bC}")
    wf = w.float().view(E, R // bR, bR, C // bC, bC)
    amax = wf.abs().amax(dim=(2, 4)).clamp_min(FP8_EPS)
    # tensor / tensor: a true (correctly rounded) division on every device;
    # torch turns "/ python_scalar" into a reciprocal multiply on the GPU
    s = amax / torch.full_like(amax, FP8_MAX)
    q = (wf / s[:, :, None, :, None]).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return q.view(E, R, C), s


def _pack_u4(q: torch.Tensor) -> torch.Tensor:
    if q.shape[-1] % 2:
        q = torch.nn.functional.pad(q, (0, 1))
    return (q[..., 0::2] | (q[..., 1::2] << 4)).contiguous()


def quantize_int4_group(w: torch.Tensor, group: int = 128):
    """Asymmetric uint4 quantization of ``w [E, R, C]`` in groups of ``group``
    along C (the reduction dim).

    scale = fp16((max - min) / 15, floored at 1e-8), zero = clamp(round(-min /
    scale), 0, 15), q = clamp(round(w / scale) + zero, 0, 15).  Returns
    ``(qweight [E, R, C/2] u8, scales [E, C/group, R] fp16, zeros
    [E, C/group, ceil(R/2)] u8)``; two nibbles per byte, low nibble first."""
    E, R, C = w.shape
    if C % group:
        raise ValueError(f"quantize_int4_group: {C} is not a multiple of {group}")
    G = C // group
    wf = w.float().view(E, R, G, group)
    mn = wf.amin(dim=-1)
    mx = wf.amax(dim=-1)
    sc = ((mx - mn) / torch.full_like(mx, 15.0)).clamp_min(1e-8).to(torch.float16)
    scf = sc.float()
    z = torch.clamp(torch.round(-mn / scf), 0, 15)
    q = torch.clamp(torch.round(wf / scf[..., None]) + z[..., None], 0, 15).to(torch.uint8)
    return (_pack_u4(q.view(E, R, C)), sc.transpose(1, 2).contiguous(),
            _pack_u4(z.to(torch.uint8).transpose(1, 2).contiguous()))


_E2M1_CUTS = (0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0)


def quantize_mxfp4(w: torch.Tensor, block: int = 32):
    """OCP MXFP4 quantization of ``w [E, R, C]`` along C (the reduction dim):
    one e8m0 scale per 32 elements with the RCEIL rule of torch's reference
    MX quantizer (exponent = ceil(log2(amax / 6)), clamped to [-127, 127]; no
    element saturates), elements rounded to E2M1 (nearest, ties to the even
    code).  Returns ``(qweight [E, R, C/2] u8, scales [E, R, C/32] u8)``, two
    elements per byte, low nibble first."""
    E, R, C = w.shape
    if C % block:
        raise ValueError(f"quantize_mxfp4: {C} is not a multiple of {block}")
    g = w.float().view(E, R, C // block, block)
    amax = g.abs().amax(dim=-1)
    ex = torch.ceil(torch.log2(amax / torch.full_like(amax, 6.0)))
    ex = torch.where(torch.isfinite(ex), ex, torch.full_like(ex, -127.0)).clamp(-127, 127)
    scale = (ex + 127).to(torch.uint8)
    inv = torch.where(scale == 0, torch.ones_like(ex), torch.exp2(-ex))
    a = g * inv[..., None]
    m = a.abs()
    # code = number of E2M1 decision points passed; ties go to the even code
    c = torch.zeros_like(m, dtype=torch.uint8)
    for i, cut in enumerate(_E2M1_CUTS):
        passed = (m >= cut) if i % 2 == 1 else (m > cut)
        c = torch.where(passed, torch.full_like(c, i + 1), c)
    c = c | (torch.signbit(a).to(torch.uint8) << 3)
    c = c.view(E, R, C)
    return (c[..., 0::2] | (c[..., 1::2] << 4)).contiguous(), scale.contiguous()


def tile_int4(q: torch.Tensor) -> torch.Tensor:
    """Row-major int4 weights ``q [E, R, C/2]`` u8 (as ``quantize_int4_group``
    returns them) -> the tiled layout ``[E, R/16, C/128, 1024]`` that
    ``fused_experts`` streams with one contiguous 1 KiB read per 16 rows x one
    128-element group (``fmoe_tile_int4``, on the GPU).  Scales and zeros
    keep their layout.  Needs R % 16 == 0 and C % 128 == 0."""
    _lib.require_cuda(q)
    assert q.dtype == torch.uint8 and q.dim() == 3, "tile_int4 takes packed uint8 [E, R, C/2]"
    q = q.contiguous()
    E, R, half = q.shape
    K = 2 * half
    out = torch.empty(E, R // 16, K // 128, 1024, dtype=torch.uint8, device=q.device)
    _lib.check(_lib.lib().fmoe_tile_int4(_lib.ptr(q), E, R, K, _lib.ptr(out), _lib.stream_of(q)),
               "tile_int4")
    return out


def tile_mxfp4(q: torch.Tensor) -> torch.Tensor:
    """MXFP4 weight bytes ``q [E, R, C/2]`` (as ``quantize_mxfp4`` returns them)
    -> the same tiled layout as ``tile_int4`` (both pack two 4-bit elements per
    byte along C; the e8m0 scales keep their layout)."""
    return tile_int4(q)
