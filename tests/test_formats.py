"""int4 checkpoint formats (AWQ, GPTQ v1/v2) -> the W4A16 layout.

CPU: the oracle's packers against known-answer words that follow from the
published packing definitions, pack/unpack round trips, and the invariant
that a checkpoint and its repacked form dequantize to identical values
(through the fused-MoE oracle's own dequantizer); host-side argument checks.
GPU (marked ``gpu``): ``fmoe_repack_int4`` through the C ABI, bit-exact
against the oracle, and end to end: weights quantized for the W4A16 kernels,
written out as AWQ / GPTQ checkpoints and repacked come back bit-identical,
so ``fused_experts`` gives identical outputs.
"""

import numpy as np
import pytest
import torch

from oracle import formats_oracle as FO
from oracle import fused_moe_oracle as O


def _rand_ckpt(E, K, N, group, seed):
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 16, size=(E, K, N), dtype=np.uint8)
    z = rng.integers(0, 16, size=(E, K // group, N), dtype=np.uint8)
    s = (rng.random((E, K // group, N)) * 0.05 + 1e-3).astype(np.float16)
    return q, z, s


# ------------------------------------------------------------ known answers
def test_awq_known_words():
    # columns 0..7 holding their own index: nibble i = column (0,2,4,6,1,3,5,7)[i]
    q = np.arange(8, dtype=np.uint8)[None, :]
    assert FO.awq_pack(q).view(np.uint32)[0, 0] == 0x75316420
    # a lone 15 in column 1 sits in nibble 4, column 6 in nibble 3, column 5 in nibble 6
    for col, word in ((1, 0x000F0000), (7, 0xF0000000), (0, 0x0000000F), (6, 0x0000F000), (5, 0x0F000000)):
        q = np.zeros((1, 8), dtype=np.uint8)
        q[0, col] = 15
        assert FO.awq_pack(q).view(np.uint32)[0, 0] == word, col


def test_gptq_known_words():
    # rows 0..7 of one column holding their index: nibble j = row j
    q = np.arange(8, dtype=np.uint8)[:, None]
    assert FO.seq_pack(q, axis=0).view(np.uint32)[0, 0] == 0x76543210
    # zeros are packed along columns, v1 stores z - 1 (so z = 0 wraps to 15)
    z = np.array([[1, 2, 3, 4, 5, 6, 7, 0]], dtype=np.uint8)
    _, qz, _ = FO.make_gptq(np.zeros((8, 8), np.uint8), z, np.ones((1, 8), np.float16), version=1)
    assert qz.view(np.uint32)[0, 0] == 0xF6543210
    _, qz2, _ = FO.make_gptq(np.zeros((8, 8), np.uint8), z, np.ones((1, 8), np.float16), version=2)
    assert qz2.view(np.uint32)[0, 0] == 0x07654321


def test_target_layout_known_bytes():
    # one output row n, reduction elements 0..3 = 1, 2, 3, 4 -> bytes 0x21, 0x43
    q_kn = np.zeros((1, 8, 8), np.uint8)
    q_kn[0, :4, 5] = [1, 2, 3, 4]
    z = np.zeros((1, 1, 8), np.uint8)
    z[0, 0, 2], z[0, 0, 3] = 9, 10
    qo, _, zo = FO.to_fmoe(q_kn, z, np.ones((1, 1, 8), np.float16))
    assert qo.shape == (1, 8, 4) and list(qo[0, 5]) == [0x21, 0x43, 0, 0]
    assert zo.shape == (1, 1, 4) and zo[0, 0, 1] == 0xA9


# ------------------------------------------------------------ round trips
@pytest.mark.parametrize("E,K,N,group", [(1, 128, 8, 128), (3, 192, 72, 32), (2, 256, 136, 64)])
def test_round_trips(E, K, N, group):
    q, z, s = _rand_ckpt(E, K, N, group, E + K + N)
    qw, qz, sc = FO.make_awq(q, z, s)
    assert qw.shape == (E, K, N // 8) and qw.dtype == np.int32
    q2, z2, s2 = FO.unpack_awq(qw, qz, sc)
    assert np.array_equal(q2, q) and np.array_equal(z2, z) and np.array_equal(s2, s)
    for v in (1, 2):
        zz = np.maximum(z, 1) if v == 1 else z  # v1 cannot hold z = 0 (it would wrap to 16)
        gw, gz, gs = FO.make_gptq(q, zz, s, version=v)
        assert gw.shape == (E, K // 8, N)
        q3, z3, _ = FO.unpack_gptq(gw, gz, gs, version=v)
        assert np.array_equal(q3, q) and np.array_equal(z3, zz)
    packed = FO.pack_u4_last(q)
    assert np.array_equal(FO.unpack_u4_last(packed), q)


@pytest.mark.parametrize("fmt", ["awq", "gptq", "gptq_v2"])
def test_repack_preserves_dequantized_weights(fmt):
    """A checkpoint and its W4A16 form dequantize to the same values: the
    textbook dequantization of the checkpoint vs the fused-MoE oracle's
    dequantizer on the repacked tensors."""
    E, K, N, group = 2, 256, 48, 64
    q, z, s = _rand_ckpt(E, K, N, group, 7)
    if fmt == "gptq":
        z = np.maximum(z, 1)
    if fmt == "awq":
        ck = FO.make_awq(q, z, s)
        qo, so, zo = FO.repack_awq(*ck)
        uq, uz, us = FO.unpack_awq(*ck)
    else:
        v = 1 if fmt == "gptq" else 2
        ck = FO.make_gptq(q, z, s, version=v)
        qo, so, zo = FO.repack_gptq(*ck, version=v)
        uq, uz, us = FO.unpack_gptq(*ck, version=v)
    want = FO.dequant_checkpoint(uq, uz, us, group)
    for e in range(E):
        got = O.dequant_int4(torch.from_numpy(qo[e]), torch.from_numpy(so[e]),
                             torch.from_numpy(zo[e]), group).numpy()
        assert np.array_equal(got, want[e]), e
    # and the checkpoint values are the generator's
    assert np.array_equal(want, FO.dequant_checkpoint(q, z, s, group))


# ------------------------------------------------------------ host checks
def test_host_argument_checks():
    from flaggems_sglang import formats as F

    with pytest.raises(ValueError):
        F.repack_awq_moe(torch.zeros(1, 128, 1), torch.zeros(1, 1, 1, dtype=torch.int32),
                         torch.zeros(1, 1, 8, dtype=torch.float16))
    with pytest.raises(ValueError):
        F.repack_gptq_moe(torch.zeros(1, 16, 8, dtype=torch.int32), torch.zeros(1, 3, 1, dtype=torch.int32),
                          torch.zeros(1, 3, 8, dtype=torch.float16))
    with pytest.raises(ValueError):
        F.repack_gptq_moe(torch.zeros(1, 16, 8, dtype=torch.int32), torch.zeros(1, 1, 1, dtype=torch.int32),
                          torch.zeros(1, 1, 8, dtype=torch.float16), checkpoint_format="marlin")
    with pytest.raises(ValueError):  # CPU tensors: the repack runs on the GPU only
        F.repack_awq_moe(torch.zeros(1, 128, 1, dtype=torch.int32), torch.zeros(1, 1, 1, dtype=torch.int32),
                         torch.zeros(1, 1, 8, dtype=torch.float16))


# ------------------------------------------------------------ GPU
DEV = "cuda"


def _gpu_repack(fmt, ck):
    from flaggems_sglang import formats as F

    t = [torch.from_numpy(np.ascontiguousarray(a)).to(DEV) for a in ck]
    if fmt == "awq":
        out = F.repack_awq_moe(*t)
    else:
        out = F.repack_gptq_moe(*t, checkpoint_format=fmt)
    return [o.cpu().numpy() for o in out]


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["awq", "gptq", "gptq_v2"])
@pytest.mark.parametrize("E,K,N,group", [(1, 128, 8, 128), (3, 192, 72, 32), (2, 256, 136, 64),
                                         (2, 4096, 1024, 128), (1, 1024, 200, 128)])
def test_gpu_repack_bit_exact(fmt, E, K, N, group):
    q, z, s = _rand_ckpt(E, K, N, group, E * K + N)
    if fmt == "gptq":
        z = np.maximum(z, 1)
    if fmt == "awq":
        ck = FO.make_awq(q, z, s)
        want = FO.repack_awq(*ck)
    else:
        v = 1 if fmt == "gptq" else 2
        ck = FO.make_gptq(q, z, s, version=v)
        want = FO.repack_gptq(*ck, version=v)
    got = _gpu_repack(fmt, ck)
    for name, g, w in zip(("qweight", "scales", "zeros"), got, want):
        assert g.shape == w.shape, name
        assert np.array_equal(g.view(np.uint8), np.ascontiguousarray(w).view(np.uint8)), name


@pytest.mark.gpu
def test_gpu_gptq_rejects_v1_zero_16_and_act_order():
    from flaggems_sglang import formats as F

    q, z, s = _rand_ckpt(1, 128, 16, 128, 3)
    z[0, 0, 5] = 0  # stored as 15 in v1 -> a zero of 16 after the +1
    ck = [torch.from_numpy(a).to(DEV) for a in FO.make_gptq(q, z, s, version=1)]
    with pytest.raises(ValueError):
        F.repack_gptq_moe(*ck)
    g_idx = (torch.arange(128, device=DEV) % 2).int()  # act-order: not k // 128
    with pytest.raises(AssertionError):
        F.repack_gptq_moe(*ck, g_idx=g_idx)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["awq", "gptq_v2"])
def test_gpu_checkpoint_to_fused_experts_end_to_end(fmt):
    """Quantize for the W4A16 kernels, write the weights out as a checkpoint,
    repack on the GPU: identical tensors, identical fused_experts output."""
    import flaggems_sglang
    from flaggems_sglang import quant as Q

    M, K, N, E, k = 5, 512, 256, 4, 2
    d = O.make_inputs(M, K, N, E, k, wscale=0.02)
    packs = [Q.quantize_int4_group(d[n].to(DEV)) for n in ("w13", "w2")]
    repacked = []
    for qw, sc, zp in packs:
        R, C = qw.shape[1], qw.shape[2] * 2
        q_nk = FO.unpack_u4_last(qw.cpu().numpy())              # [E, R, C]
        z_gr = FO.unpack_u4_last(zp.cpu().numpy())[..., :R]     # [E, G, R]
        q_kn = np.ascontiguousarray(np.swapaxes(q_nk, -1, -2))  # [E, C, R]
        ck = FO.make_awq(q_kn, z_gr, sc.cpu().numpy()) if fmt == "awq" else \
            FO.make_gptq(q_kn, z_gr, sc.cpu().numpy(), version=2)
        got = [torch.from_numpy(a).to(DEV) for a in _gpu_repack(fmt, ck)]
        assert torch.equal(got[0], qw) and torch.equal(got[1], sc) and torch.equal(got[2], zp)
        assert C == (K if len(repacked) == 0 else N)
        repacked.append(got)
    args = (d["x"].to(DEV), d["topk_weights"].to(DEV), d["topk_ids"].to(DEV))

    def run(p13, p2):
        return flaggems_sglang.fused_experts(args[0], p13[0], p2[0], args[1], args[2], use_int4_w4a16=True,
                                             w1_scale=p13[1], w2_scale=p2[1], w1_zp=p13[2], w2_zp=p2[2])

    assert torch.equal(run(*packs), run(*repacked))


@pytest.mark.gpu
def test_gpu_flagos_hook_repacks_awq_layer_once():
    """fused_moe_flagos on a layer holding AWQ checkpoint tensors: converted
    (and tiled) on the first call, reused after, same output as the
    row-major W4A16-layout layer."""
    from types import SimpleNamespace

    from flaggems_sglang import quant as Q
    from flaggems_sglang.ops.fused_moe import fused_moe_flagos

    M, K, N, E, k = 3, 256, 128, 4, 2
    d = O.make_inputs(M, K, N, E, k, wscale=0.02)
    native = torch.nn.Module()
    awq = torch.nn.Module()
    for pre in ("w13", "w2"):
        qw, sc, zp = Q.quantize_int4_group(d[pre].to(DEV))
        native.register_parameter(f"{pre}_qweight", torch.nn.Parameter(qw, requires_grad=False))
        native.register_parameter(f"{pre}_scales", torch.nn.Parameter(sc, requires_grad=False))
        native.register_parameter(f"{pre}_qzeros", torch.nn.Parameter(zp, requires_grad=False))
        R = qw.shape[1]
        q_kn = np.ascontiguousarray(np.swapaxes(FO.unpack_u4_last(qw.cpu().numpy()), -1, -2))
        z_gr = FO.unpack_u4_last(zp.cpu().numpy())[..., :R]
        ck = FO.make_awq(q_kn, z_gr, sc.cpu().numpy())
        for n_, a in zip(("qweight", "qzeros", "scales"), ck):
            awq.register_parameter(f"{pre}_{n_}", torch.nn.Parameter(torch.from_numpy(a).to(DEV),
                                                                     requires_grad=False))
    awq.fmoe_int4_checkpoint_format = "awq"
    cfg = SimpleNamespace(num_experts=E, no_combine=False, activation="silu",
                          apply_router_weight_on_input=False, routed_scaling_factor=None)
    obj = SimpleNamespace(runner=SimpleNamespace(config=cfg))
    disp = SimpleNamespace(hidden_states=d["x"].to(DEV),
                           topk_output=SimpleNamespace(topk_weights=d["topk_weights"].to(DEV),
                                                       topk_ids=d["topk_ids"].to(DEV)))
    ref = fused_moe_flagos(obj, native, disp).hidden_states
    out1 = fused_moe_flagos(obj, awq, disp).hidden_states
    assert awq.fmoe_int4_repacked and awq.w13_qweight.dtype == torch.uint8
    # repacked into the tiled layout (quant.tile_int4) by default
    assert awq.w13_qweight.shape == (E, 2 * N // 16, K // 128, 1024)
    assert awq.w2_qweight.shape == (E, K // 16, N // 128, 1024)
    out2 = fused_moe_flagos(obj, awq, disp).hidden_states
    assert torch.equal(out1, ref) and torch.equal(out2, ref)
