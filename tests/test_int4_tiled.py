"""Tiled 4-bit weights (``quant.tile_int4`` / ``tile_mxfp4`` /
``fmoe_tile_int4``, weight types FMOE_W_INT4_TILED and FMOE_W_MXFP4_TILED):
the layout the decode kernels read with one contiguous 1 KiB load per 16 rows
x one 128-element quant group.

CPU: the oracle's tile / untile against known-answer positions and its round
trip; the host check that both weights use the same layout.  GPU: the tiling
kernel bit-exact against the oracle (and its argument checks), and the fused
op on tiled weights bit-identical to the same weights row-major (same
kernels, same reduction order: only the weight addresses change), across
decode and larger batches, both activations, an expert map, no_combine and
the stage-level C ABI.
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle import formats_oracle as FO

DEV = "cuda"


# ----------------------------------------------------------------- CPU
def test_oracle_tile_known_positions():
    # every 16-byte chunk of q holds (row, chunk) so its destination names it
    E, R, K = 2, 48, 384
    half = K // 2
    q = np.zeros((E, R, half), dtype=np.uint8)
    for e in range(E):
        for r in range(R):
            for ch in range(half // 16):
                q[e, r, 16 * ch:16 * ch + 16] = [e, r, ch] + [0xA5] * 13
    t = FO.tile_int4(q)
    assert t.shape == (E, R // 16, K // 128, 1024)
    flat = t.reshape(E, -1)
    # row 17, chunk 5 = group c 1, lane group g 1; block b 1, r 1:
    # byte offset ((b * K/128 + c) * 1024) + (16 g + r) * 16
    off = (1 * (K // 128) + 1) * 1024 + (16 * 1 + 1) * 16
    assert list(flat[1, off:off + 3]) == [1, 17, 5]
    # row 0, chunk 0 -> offset 0; row 15, chunk 3 (c 0, g 3) -> (48 + 15) * 16
    assert list(flat[0, 0:3]) == [0, 0, 0]
    assert list(flat[0, 63 * 16:63 * 16 + 3]) == [0, 15, 3]
    # row 47, last chunk (c 2, g 3), block 2
    off = (2 * 3 + 2) * 1024 + (48 + 15) * 16
    assert list(flat[1, off:off + 3]) == [1, 47, half // 16 - 1]
    # each 1 KiB block holds 16 distinct rows x 4 chunks of one group
    blk = t[0, 1, 2].reshape(64, 16)
    assert sorted({(int(c[1]), int(c[2])) for c in blk}) == sorted(
        (16 + r, 4 * 2 + g) for r in range(16) for g in range(4))


def test_oracle_tile_round_trip():
    rng = np.random.default_rng(7)
    for E, R, K in [(1, 16, 128), (3, 64, 512), (2, 32, 1152)]:
        q = rng.integers(0, 256, (E, R, K // 2), dtype=np.uint8)
        t = FO.tile_int4(q)
        assert np.array_equal(FO.untile_int4(t), q)
        # a permutation: same byte multiset per expert
        assert np.array_equal(np.sort(t.reshape(E, -1), axis=1), np.sort(q.reshape(E, -1), axis=1))


def test_host_rejects_mixed_layouts():
    from flaggems_sglang.ops.fused_moe import _wtype_and_check
    w3 = torch.zeros(2, 256, 64, dtype=torch.uint8)
    w4 = torch.zeros(2, 16, 1, 1024, dtype=torch.uint8)
    s = torch.zeros(1)
    with pytest.raises(AssertionError, match="both be row-major"):
        _wtype_and_check(False, True, w3, w4, s, s, s, s, None, False)
    from flaggems_sglang._lib import W_INT4, W_INT4_TILED
    assert _wtype_and_check(False, True, w4, w4, s, s, s, s, None, False) == W_INT4_TILED
    assert _wtype_and_check(False, True, w3, w3, s, s, s, s, None, False) == W_INT4


# ----------------------------------------------------------------- GPU
@pytest.mark.gpu
@pytest.mark.parametrize("E,R,K", [(1, 16, 128), (3, 64, 512), (2, 48, 1152), (8, 256, 4096)])
def test_tile_kernel_matches_oracle(E, R, K):
    from flaggems_sglang import quant as Q
    g = torch.Generator().manual_seed(E * 1000 + R + K)
    q = torch.randint(0, 256, (E, R, K // 2), dtype=torch.uint8, generator=g)
    t = Q.tile_int4(q.to(DEV))
    torch.cuda.synchronize()
    assert np.array_equal(t.cpu().numpy(), FO.tile_int4(q.numpy()))


@pytest.mark.gpu
def test_tile_kernel_argument_checks():
    from flaggems_sglang import _lib
    L = _lib.lib()
    q = torch.zeros(1, 32, 128, dtype=torch.uint8, device=DEV)
    out = torch.empty_like(q)
    st = torch.cuda.current_stream().cuda_stream
    assert L.fmoe_tile_int4(q.data_ptr(), 1, 32, 256, out.data_ptr(), st) == 0
    assert L.fmoe_tile_int4(q.data_ptr(), 1, 24, 256, out.data_ptr(), st) != 0  # R % 16
    assert L.fmoe_tile_int4(q.data_ptr(), 1, 32, 192, out.data_ptr(), st) != 0  # K % 128
    assert L.fmoe_tile_int4(q.data_ptr(), 1, 32, 256, q.data_ptr() + 1024, st) != 0  # overlap
    assert b"overlap" in L.fmoe_last_error()
    assert L.fmoe_tile_int4(None, 1, 32, 256, out.data_ptr(), st) != 0
    torch.cuda.synchronize()


# batches up to this many tokens on tiled int4 weights run as one launch
# (GEMM1 -> act -> GEMM2 per 128-column slice) plus the plane sum
ONE_LAUNCH_MAX_M = 1


def _rel_below(out, ref, tol):
    out, ref = out.float().cpu(), ref.float().cpu()
    rel = float((out - ref).norm() / ref.norm().clamp_min(1e-30))
    assert rel < tol, f"relative difference {rel:.3e}"


def _int4_layer(M, K, N, E, k):
    from flaggems_sglang import quant as Q
    from oracle import fused_moe_oracle as O
    d = O.make_inputs(M, K, N, E, k, wscale=0.05)
    q1, s1, z1 = Q.quantize_int4_group(d["w13"].to(DEV))
    q2, s2, z2 = Q.quantize_int4_group(d["w2"].to(DEV))
    kw = dict(use_int4_w4a16=True, w1_scale=s1, w2_scale=s2, w1_zp=z1, w2_zp=z2)
    return d, q1, q2, Q.tile_int4(q1), Q.tile_int4(q2), kw


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N,E,k", [(1, 512, 384, 8, 2), (5, 256, 256, 4, 2), (16, 1024, 768, 8, 2),
                                       (64, 512, 384, 16, 4), (300, 256, 512, 8, 2), (1, 128, 128, 1, 1)])
@pytest.mark.parametrize("activation", ["silu", "gelu"])
def test_fused_tiled_equals_row_major(M, K, N, E, k, activation):
    import flaggems_sglang
    d, q1, q2, t1, t2, kw = _int4_layer(M, K, N, E, k)
    x, tw, ti = d["x"].to(DEV), d["topk_weights"].to(DEV), d["topk_ids"].to(DEV)
    ref = flaggems_sglang.fused_experts(x, q1, q2, tw, ti, activation=activation, **kw)
    out = flaggems_sglang.fused_experts(x, t1, t2, tw, ti, activation=activation, **kw)
    if M <= ONE_LAUNCH_MAX_M:
        # tiled weights take the one-launch route here: GEMM2 summed in other
        # fp32 partials (N / 128 planes), so equal to a few bf16 ulps
        _rel_below(out, ref, 2e-3)
    else:
        assert torch.equal(out, ref)
    if M == 16 and activation == "silu":
        # and against the dequantizing oracle, as the row-major int4 tests do
        from oracle import fused_moe_oracle as O
        o = O.fused_experts_w4a16(d["x"], q1.cpu(), kw["w1_scale"].cpu(), kw["w1_zp"].cpu(), q2.cpu(),
                                  kw["w2_scale"].cpu(), kw["w2_zp"].cpu(), d["topk_weights"], d["topk_ids"])
        rel = float((out.float().cpu() - o.float()).norm() / o.float().norm())
        assert rel < 5e-2 / 4


@pytest.mark.gpu
def test_fused_tiled_expert_map_and_no_combine():
    import flaggems_sglang
    M, K, N, E, k = 9, 512, 384, 16, 4
    d, q1, q2, t1, t2, kw = _int4_layer(M, K, N, E, k)
    x, tw, ti = d["x"].to(DEV), d["topk_weights"].to(DEV), d["topk_ids"].to(DEV)
    emap = torch.arange(E, dtype=torch.int32, device=DEV)
    emap[3] = -1
    a = flaggems_sglang.fused_experts(x, q1, q2, tw, ti, expert_map=emap, global_num_experts=E, **kw)
    b = flaggems_sglang.fused_experts(x, t1, t2, tw, ti, expert_map=emap, global_num_experts=E, **kw)
    assert torch.equal(a, b)
    a = flaggems_sglang.fused_experts(x, q1, q2, tw, ti, no_combine=True, **kw)
    b = flaggems_sglang.fused_experts(x, t1, t2, tw, ti, no_combine=True, **kw)
    assert torch.equal(a, b)


@pytest.mark.gpu
@pytest.mark.parametrize("tiled", [False, True])
def test_paired_row_split_odd_tiles_and_expert_map(tiled):
    """int4 decode batches of >= 24 slots per expert take the row-split kernel
    with paired 16-slot tiles (the workgroup of tile 2i computes 2i and 2i + 1,
    the odd tile's workgroup exits).  Skewed routing gives experts an odd
    number of tiles (a lone last tile) and experts of <= 16 slots (one tile,
    the pair's second half empty); an expert map drops two experts.  Both
    against the dequantizing oracle."""
    import flaggems_sglang
    from flaggems_sglang import quant as Q
    from oracle import fused_moe_oracle as O
    M, K, N, E, k = 300, 512, 384, 8, 2
    d = O.make_inputs(M, K, N, E, k, wscale=0.05, expert_bias_std=1.0)
    counts = torch.bincount(d["topk_ids"].flatten().long(), minlength=E)
    tiles = (counts + 15) // 16
    assert bool((tiles % 2 == 1).any()) and int(counts.min()) <= 16 and int(counts.max()) > 32, counts
    q1, s1, z1 = Q.quantize_int4_group(d["w13"].to(DEV))
    q2, s2, z2 = Q.quantize_int4_group(d["w2"].to(DEV))
    kw = dict(use_int4_w4a16=True, w1_scale=s1, w2_scale=s2, w1_zp=z1, w2_zp=z2)
    w1, w2 = (Q.tile_int4(q1), Q.tile_int4(q2)) if tiled else (q1, q2)
    x, tw, ti = d["x"].to(DEV), d["topk_weights"].to(DEV), d["topk_ids"].to(DEV)

    def ref(tw_, ti_):
        return O.fused_experts_w4a16(d["x"], q1.cpu(), s1.cpu(), z1.cpu(), q2.cpu(), s2.cpu(), z2.cpu(),
                                     tw_, ti_)

    out = flaggems_sglang.fused_experts(x, w1, w2, tw, ti, **kw)
    _rel_below(out, ref(d["topk_weights"], d["topk_ids"]), 5e-2 / 4)
    emap = torch.arange(E, dtype=torch.int32)
    emap[1] = -1
    emap[int(counts.argmax())] = -1
    out = flaggems_sglang.fused_experts(x, w1, w2, tw, ti, expert_map=emap.to(DEV), global_num_experts=E, **kw)
    ltw, lti = O.ep_localize(d["topk_weights"], d["topk_ids"], emap)
    _rel_below(out, ref(ltw, lti), 5e-2 / 4)


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N,E,k", [(1, 512, 384, 8, 2), (16, 1024, 768, 8, 2), (300, 256, 512, 8, 2)])
def test_fused_mxfp4_tiled_equals_row_major(M, K, N, E, k):
    import flaggems_sglang
    from flaggems_sglang import quant as Q
    from oracle import fused_moe_oracle as O
    d = O.make_inputs(M, K, N, E, k, wscale=0.05)
    q1, s1 = Q.quantize_mxfp4(d["w13"].to(DEV))
    q2, s2 = Q.quantize_mxfp4(d["w2"].to(DEV))
    x, tw, ti = d["x"].to(DEV), d["topk_weights"].to(DEV), d["topk_ids"].to(DEV)
    kw = dict(use_mxfp4_w4a16=True, w1_scale=s1, w2_scale=s2)
    ref = flaggems_sglang.fused_experts(x, q1, q2, tw, ti, **kw)
    out = flaggems_sglang.fused_experts(x, Q.tile_mxfp4(q1), Q.tile_mxfp4(q2), tw, ti, **kw)
    assert torch.equal(out, ref)


def _w_bf16_from_oracle(fmt, q, s, z):
    """The weights the large-batch path computes with: the oracle's dequantized
    values rounded once to bf16 (exact for MXFP4; int4 (q - z) * s is exact in
    fp32 before that rounding)."""
    from oracle import fused_moe_oracle as O
    q, s = q.cpu(), s.cpu()
    if fmt in ("int4t", "mxfp4t"):
        q = torch.from_numpy(FO.untile_int4(q.numpy()))
    if fmt.startswith("int4"):
        z = z.cpu()
        w = torch.stack([O.dequant_int4(q[e], s[e], z[e]) for e in range(q.shape[0])])
    else:
        w = O.mxfp4_dequant(q, s).float()
    return w.to(torch.bfloat16)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["int4", "int4t", "mxfp4", "mxfp4t"])
def test_large_batch_dequant_path(fmt):
    """Experts averaging >= 128 slots: the 4-bit weights are dequantized once
    to bf16 and the bf16 prefill kernels run.  Bit-identical to the bf16 path
    on the oracle-dequantized weights, within tolerance of the oracle and of
    the decode kernels (path=2); path=1 forces it at small M."""
    import flaggems_sglang
    from flaggems_sglang import quant as Q
    from oracle import fused_moe_oracle as O
    M, K, N, E, k = 600, 256, 256, 4, 2
    d = O.make_inputs(M, K, N, E, k, wscale=0.05)
    x, tw, ti = d["x"].to(DEV), d["topk_weights"].to(DEV), d["topk_ids"].to(DEV)
    if fmt.startswith("int4"):
        q1, s1, z1 = Q.quantize_int4_group(d["w13"].to(DEV))
        q2, s2, z2 = Q.quantize_int4_group(d["w2"].to(DEV))
        if fmt == "int4t":
            q1, q2 = Q.tile_int4(q1), Q.tile_int4(q2)
        kw = dict(use_int4_w4a16=True, w1_scale=s1, w2_scale=s2, w1_zp=z1, w2_zp=z2)
        tol = 5e-2
    else:
        q1, s1 = Q.quantize_mxfp4(d["w13"].to(DEV))
        q2, s2 = Q.quantize_mxfp4(d["w2"].to(DEV))
        z1 = z2 = None
        if fmt == "mxfp4t":
            q1, q2 = Q.tile_mxfp4(q1), Q.tile_mxfp4(q2)
        kw = dict(use_mxfp4_w4a16=True, w1_scale=s1, w2_scale=s2)
        tol = 2e-2
    out = flaggems_sglang.fused_experts(x, q1, q2, tw, ti, **kw)
    w13b = _w_bf16_from_oracle(fmt, q1, s1, z1).to(DEV)
    w2b = _w_bf16_from_oracle(fmt, q2, s2, z2).to(DEV)
    ref_bf16 = flaggems_sglang.fused_experts(x, w13b, w2b, tw, ti, path=1)
    assert torch.equal(out, ref_bf16)
    dec = flaggems_sglang.fused_experts(x, q1, q2, tw, ti, path=2, **kw)
    rel = float((out.float() - dec.float()).norm() / dec.float().norm())
    assert rel < tol / 4, rel
    o = O.fused_experts(d["x"], w13b.cpu().float(), w2b.cpu().float(), d["topk_weights"], d["topk_ids"])
    rel = float((out.float().cpu() - o.float()).norm() / o.float().norm())
    assert rel < tol / 4, rel
    # path=1 takes the same route at a decode-sized batch
    small = flaggems_sglang.fused_experts(x[:5], q1, q2, tw[:5], ti[:5], path=1, **kw)
    ref_small = flaggems_sglang.fused_experts(x[:5], w13b, w2b, tw[:5], ti[:5], path=1)
    assert torch.equal(small, ref_small)


# ------------------------------------------- one-launch decode (tiled int4)
@pytest.mark.gpu
@pytest.mark.parametrize("K,N,E,k", [(512, 384, 8, 2), (1024, 256, 4, 1), (256, 1152, 16, 4),
                                     (4096, 14336, 8, 2)])
def test_one_launch_decode_matches_oracle(K, N, E, k):
    """Tiled int4 at M = 1: GEMM1, the activation and GEMM2 of each 128-column
    slice of the intermediate in one workgroup, N / 128 partial planes added
    by moe_sum_planes.  Against the dequantizing oracle (north_star int4
    tolerance 5e-2, as test_mixtral_w4a16), against the two-launch path on
    the same weights row-major, and run to run bit-identical."""
    import flaggems_sglang
    from oracle import fused_moe_oracle as O
    from test_gpu_fused_moe import _close
    d, q1, q2, t1, t2, kw = _int4_layer(1, K, N, E, k)
    x, tw, ti = d["x"].to(DEV), d["topk_weights"].to(DEV), d["topk_ids"].to(DEV)
    out = flaggems_sglang.fused_experts(x, t1, t2, tw, ti, **kw)
    o = O.fused_experts_w4a16(d["x"], q1.cpu(), kw["w1_scale"].cpu(), kw["w1_zp"].cpu(), q2.cpu(),
                              kw["w2_scale"].cpu(), kw["w2_zp"].cpu(), d["topk_weights"], d["topk_ids"])
    _close(out, o, 5e-2)
    _rel_below(out, flaggems_sglang.fused_experts(x, q1, q2, tw, ti, **kw), 2e-3)
    assert torch.equal(out, flaggems_sglang.fused_experts(x, t1, t2, tw, ti, **kw))


@pytest.mark.gpu
@pytest.mark.parametrize("activation,on_input", [("silu", False), ("gelu", False), ("silu", True)])
def test_one_launch_decode_activation_gamma_scaling(activation, on_input):
    """GELU, the routing weight on the input (top-1), routed scaling: the
    one-launch route (tiled) against the two-launch route (row-major)."""
    import flaggems_sglang
    K, N, E, k = 512, 640, 8, 1 if on_input else 2
    d, q1, q2, t1, t2, kw = _int4_layer(1, K, N, E, k)
    x, tw, ti = d["x"].to(DEV), d["topk_weights"].to(DEV), d["topk_ids"].to(DEV)
    args = dict(activation=activation, apply_router_weight_on_input=on_input, routed_scaling_factor=1.5, **kw)
    out = flaggems_sglang.fused_experts(x, t1, t2, tw, ti, **args)
    ref = flaggems_sglang.fused_experts(x, q1, q2, tw, ti, **args)
    _rel_below(out, ref, 2e-3)


@pytest.mark.gpu
def test_one_launch_decode_routing_paths_bit_exact():
    """At M = 1 the tiles come from the top-k ids inside the workgroup (no
    align launch); with an identity expert map from the align kernels.  Same
    tiles, same sums: bit-identical.  With an expert dropped by the map its
    slot contributes nothing (two-launch route on row-major weights as the
    check)."""
    import flaggems_sglang
    K, N, E, k = 512, 384, 16, 4
    d, q1, q2, t1, t2, kw = _int4_layer(1, K, N, E, k)
    x, tw, ti = d["x"].to(DEV), d["topk_weights"].to(DEV), d["topk_ids"].to(DEV)
    plain = flaggems_sglang.fused_experts(x, t1, t2, tw, ti, **kw)
    emap = torch.arange(E, dtype=torch.int32, device=DEV)
    mapped = flaggems_sglang.fused_experts(x, t1, t2, tw, ti, expert_map=emap, global_num_experts=E, **kw)
    assert torch.equal(plain, mapped)
    emap[int(d["topk_ids"][0, 1])] = -1
    a = flaggems_sglang.fused_experts(x, t1, t2, tw, ti, expert_map=emap, global_num_experts=E, **kw)
    b = flaggems_sglang.fused_experts(x, q1, q2, tw, ti, expert_map=emap, global_num_experts=E, **kw)
    _rel_below(a, b, 2e-3)
    assert not torch.equal(a, plain)


@pytest.mark.gpu
def test_tiled_m1_with_down_bias_takes_two_launch_route():
    """A GEMM2 bias with SiLU is accepted by the C ABI; the one-launch kernel
    applies no bias, so such single-token calls on tiled weights take the
    two-launch route and match the row-major weights with the same bias."""
    import flaggems_sglang  # noqa: F401
    from flaggems_sglang import _lib
    K, N, E, k = 512, 384, 8, 2
    d, q1, q2, t1, t2, kw = _int4_layer(1, K, N, E, k)
    x, tw, ti = d["x"].to(DEV), d["topk_weights"].to(DEV), d["topk_ids"].to(DEV)
    b2 = (torch.randn(E, K, generator=torch.Generator().manual_seed(5)) * 0.5).to(DEV)
    L = _lib.lib()
    st = torch.cuda.current_stream().cuda_stream

    def run(wt, w13, w2, bias):
        out = torch.empty(1, K, dtype=torch.bfloat16, device=DEV)
        a = _lib.FusedArgs(wt, x.data_ptr(), 1, K, N, E, k, w13.data_ptr(), w2.data_ptr(),
                           kw["w1_scale"].data_ptr(), kw["w2_scale"].data_ptr(), kw["w1_zp"].data_ptr(),
                           kw["w2_zp"].data_ptr(), 128, tw.data_ptr(), ti.data_ptr(), 0, 1.0, 0,
                           out.data_ptr(), None, 0, _lib.ACT_SILU, None, _lib.ptr(bias), 1.0, 0.0, None, 0)
        n = L.fmoe_fused_experts_workspace_bytes(ctypes.byref(a))
        ws = torch.empty(max(n, 1), dtype=torch.uint8, device=DEV)
        a.workspace, a.workspace_bytes = ws.data_ptr(), n
        _lib.check(L.fmoe_fused_experts(ctypes.byref(a), st), "fused_experts")
        torch.cuda.synchronize()
        return out

    tiled = run(_lib.W_INT4_TILED, t1, t2, b2)
    rowm = run(_lib.W_INT4, q1, q2, b2)
    assert torch.equal(tiled, rowm)  # same two-launch kernels, addresses only
    plain = run(_lib.W_INT4_TILED, t1, t2, None)
    # each slot adds its expert's bias row times its gate weight
    want = plain.float() + sum(float(tw[0, j]) * b2[int(ti[0, j])] for j in range(k))
    _rel_below(tiled, want, 1e-2)


@pytest.mark.gpu
def test_one_launch_regression_bits():
    """The single-token tiled-int4 route against its stored output, bit for
    bit (tests/golden/make_int4_regression.py): pins the plane order and the
    rounding points that the tolerance checks above would let drift."""
    import os
    import sys
    here = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    sys.path.insert(0, here)
    import make_int4_regression as R
    ref = np.load(os.path.join(here, R.NAME), allow_pickle=False)
    sha, bits = R.run_case()
    assert sha == str(ref["input_sha256"]), "seeded inputs drifted"
    assert np.array_equal(bits, ref["out"])
