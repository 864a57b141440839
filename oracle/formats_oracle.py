"""CPU oracle of the int4 checkpoint formats (test infrastructure only).

Only tests/ may import this module: it is the checker for
``fmoe_repack_int4`` / ``flaggems_sglang.formats``, never a product path.

The reference has no int4 path; its SGLang integration loads W4A16 MoE
layers from AWQ and GPTQ checkpoints, whose packings are defined by
third-party libraries absent here:
  * AutoAWQ (0.2.x, "gemm" version: ``awq/modules/linear/gemm.py`` pack, the
    ``order_map = [0, 2, 4, 6, 1, 3, 5, 7]``): qweight int32 [K, N/8], word j
    of row k holds columns 8j + order_map[i] in nibble i; qzeros int32
    [K/g, N/8] the same; scales fp16 [K/g, N]; w = (q - z) * s.
  * AutoGPTQ (0.7.x, ``qlinear_cuda_old`` / exllama packing, no act-order):
    qweight int32 [K/8, N], nibble j of word i = row 8i + j; qzeros int32
    [K/g, N/8], nibble j of word c = column 8c + j, holding z - 1 (format v1)
    or z (v2, GPTQModel); scales fp16 [K/g, N]; w = (q - z) * s.
These are restated from the libraries' published packers.  Parity against
the libraries themselves is unpinned (they cannot be run here); the oracle
is pinned by known-answer words derived from the published order maps, by
pack / unpack round trips and by dequantization invariance (a checkpoint and
its repacked form dequantize to identical values), all in
tests/test_formats.py.

The tiled int4 layout (``fmoe_tile_int4``, FMOE_W_INT4_TILED) has no
counterpart in the reference or in those libraries; ``tile_int4`` restates
its definition, and tests/test_int4_tiled.py pins it by known-answer
positions, the round trip through ``untile_int4``, and bit-identical
fused-MoE outputs from tiled and row-major weights.

Target layout (the W4A16 kernels, ``fused_moe_oracle.quant_int4``):
qweight [N, K/2] u8 (element 2i low nibble), scales [K/g, N] fp16, zeros
[K/g, N/2] u8 (row 2j low nibble).
"""

from __future__ import annotations

import numpy as np

AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)  # nibble i holds column AWQ_ORDER[i] of its 8


def _as_i32(words_u32: np.ndarray) -> np.ndarray:
    return words_u32.astype(np.uint32).view(np.int32)


def awq_pack(q: np.ndarray) -> np.ndarray:
    """uint4 values ``[..., R, C]`` (C % 8 == 0) -> AWQ words ``[..., R, C/8]``."""
    q = q.astype(np.uint32)
    *lead, R, C = q.shape
    g = q.reshape(*lead, R, C // 8, 8)
    w = np.zeros((*lead, R, C // 8), dtype=np.uint32)
    for i, col in enumerate(AWQ_ORDER):
        w |= g[..., col] << np.uint32(4 * i)
    return _as_i32(w)


def awq_unpack(w: np.ndarray) -> np.ndarray:
    """AWQ words ``[..., R, C/8]`` -> uint4 values ``[..., R, C]`` (uint8)."""
    u = w.view(np.uint32)
    *lead, R, C8 = u.shape
    out = np.zeros((*lead, R, C8, 8), dtype=np.uint8)
    for i, col in enumerate(AWQ_ORDER):
        out[..., col] = (u >> np.uint32(4 * i)) & np.uint32(15)
    return out.reshape(*lead, R, C8 * 8)


def seq_pack(q: np.ndarray, axis: int) -> np.ndarray:
    """Sequential nibble packing along ``axis`` (GPTQ): element 8i + j of
    that axis goes to nibble j of word i."""
    q = np.moveaxis(q.astype(np.uint32), axis, -1)
    *lead, L = q.shape
    g = q.reshape(*lead, L // 8, 8)
    w = np.zeros((*lead, L // 8), dtype=np.uint32)
    for j in range(8):
        w |= g[..., j] << np.uint32(4 * j)
    return np.moveaxis(_as_i32(w), -1, axis)


def seq_unpack(w: np.ndarray, axis: int) -> np.ndarray:
    u = np.moveaxis(w.view(np.uint32), axis, -1)
    *lead, L8 = u.shape
    out = np.zeros((*lead, L8, 8), dtype=np.uint8)
    for j in range(8):
        out[..., j] = (u >> np.uint32(4 * j)) & np.uint32(15)
    return np.moveaxis(out.reshape(*lead, L8 * 8), -1, axis)


def pack_u4_last(q: np.ndarray) -> np.ndarray:
    """Two per byte along the last dim, even index in the low nibble."""
    q = q.astype(np.uint8)
    return (q[..., 0::2] | (q[..., 1::2] << 4)).astype(np.uint8)


def unpack_u4_last(p: np.ndarray) -> np.ndarray:
    out = np.empty((*p.shape[:-1], p.shape[-1] * 2), dtype=np.uint8)
    out[..., 0::2] = p & 15
    out[..., 1::2] = p >> 4
    return out


# ---------------------------------------------------------------- checkpoints
def make_awq(q_kn: np.ndarray, z_gn: np.ndarray, s_gn: np.ndarray):
    """Stacked ``q [E, K, N]``, ``z [E, G, N]`` (uint4), ``s [E, G, N]`` fp16 ->
    AWQ tensors (qweight, qzeros, scales)."""
    return awq_pack(q_kn), awq_pack(z_gn), s_gn.astype(np.float16)


def make_gptq(q_kn: np.ndarray, z_gn: np.ndarray, s_gn: np.ndarray, version: int = 1):
    """GPTQ tensors; v1 stores z - 1 (mod 16), v2 stores z."""
    zs = (z_gn.astype(np.int64) - (1 if version == 1 else 0)) & 15
    return seq_pack(q_kn, axis=-2), seq_pack(zs.astype(np.uint8), axis=-1), s_gn.astype(np.float16)


def unpack_awq(qweight, qzeros, scales):
    """AWQ -> (q [E, K, N], z [E, G, N], s [E, G, N])."""
    return awq_unpack(qweight), awq_unpack(qzeros), scales


def unpack_gptq(qweight, qzeros, scales, version: int = 1):
    """GPTQ -> (q [E, K, N], z [E, G, N], s [E, G, N]); v1 zeros are stored
    minus one, so z = stored + 1 (16 is not representable)."""
    z = seq_unpack(qzeros, axis=-1).astype(np.int64)
    if version == 1:
        z = z + 1
    return seq_unpack(qweight, axis=-2), z, scales


def to_fmoe(q_kn, z_gn, s_gn):
    """Unpacked (q [E, K, N], z [E, G, N], s [E, G, N]) -> the W4A16 layout
    (qweight [E, N, K/2] u8, scales [E, G, N] fp16, zeros [E, G, N/2] u8)."""
    q_nk = np.ascontiguousarray(np.swapaxes(q_kn, -1, -2))
    return pack_u4_last(q_nk), s_gn.astype(np.float16), pack_u4_last(np.asarray(z_gn) & 15)


def repack_awq(qweight, qzeros, scales):
    return to_fmoe(*unpack_awq(qweight, qzeros, scales))


def repack_gptq(qweight, qzeros, scales, version: int = 1):
    return to_fmoe(*unpack_gptq(qweight, qzeros, scales, version))


def dequant_checkpoint(q_kn, z_gn, s_gn, group: int):
    """Textbook dequantization w[k, n] = (q - z[k // g]) * s[k // g] -> fp32
    ``[E, N, K]`` (output rows first, like the fused-MoE weights)."""
    zk = np.repeat(np.asarray(z_gn, dtype=np.float32), group, axis=-2)
    sk = np.repeat(np.asarray(s_gn, dtype=np.float32), group, axis=-2)
    w = (q_kn.astype(np.float32) - zk) * sk
    return np.ascontiguousarray(np.swapaxes(w, -1, -2))


# ------------------------------------------------------------ tiled layout
def tile_int4(q: np.ndarray) -> np.ndarray:
    """Row-major ``q [E, R, K/2]`` u8 -> ``[E, R/16, K/128, 1024]``: block
    (b, c) holds rows 16b..16b+15 x bytes 64c..64c+63; byte 16 (16 g + r) + i
    of the block = byte 64c + 16g + i of row 16b + r."""
    E, R, half = q.shape
    K = 2 * half
    v = q.reshape(E, R // 16, 16, K // 128, 4, 16)     # e, b, r, c, g, i
    return np.ascontiguousarray(v.transpose(0, 1, 3, 4, 2, 5)).reshape(E, R // 16, K // 128, 1024)


def untile_int4(t: np.ndarray) -> np.ndarray:
    E, B, C, _ = t.shape
    v = t.reshape(E, B, C, 4, 16, 16)                   # e, b, c, g, r, i
    return np.ascontiguousarray(v.transpose(0, 1, 4, 2, 3, 5)).reshape(E, B * 16, C * 64)
