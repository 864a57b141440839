"""GPU parity of the fused-MoE path against the CPU oracle, through the C ABI.

Mirrors the reference's accuracy tests (tests/test_fused_moe.py:84-113: every
FUSED_MOE_SHAPES entry, plus apply_router_weight_on_input on the small
shapes; inputs per its _make_inputs, seed M+K+N+E+topk) and adds the
BASELINE configurations (bf16, skewed routing, fp8 block-scale, int4) at
sizes the oracle finishes in seconds.  Tolerances: bf16 atol=rtol=2e-2;
fp8 / int4 5e-2 against the dequantize-then-compute oracle -- with the
absolute term scaled by the output RMS (_close), and on the BASELINE input
recipes also exactly as written (_close_literal).
"""

import numpy as np
import pytest
import torch

import flaggems_sglang
from flaggems_sglang import quant as Q
from flaggems_sglang.ops import fused_moe as F
from oracle import fused_moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"

# tests/accuracy_utils.py:100-118
FUSED_MOE_SHAPES_SMALL = [(1, 128, 256, 8, 2), (7, 128, 256, 8, 2), (33, 256, 512, 16, 4)]
FUSED_MOE_SHAPES_LARGE = [(m, 1280, 3072, 64, 8) for m in (1, 4, 17, 64, 1024, 2048, 4096)]


def _ref_inputs(M, K, N, E, topk):
    """The reference's _make_inputs (tests/test_fused_moe.py:50-58), on CPU:
    x ~ N(0,1) bf16, w1 [E,K,2N] and w2 [E,N,K] ~ N(0,1)*0.1 bf16, logits."""
    torch.manual_seed(M + K + N + E + topk)
    x = torch.randn(M, K, dtype=torch.bfloat16)
    w1 = torch.randn(E, K, N * 2, dtype=torch.bfloat16) * 0.1
    w2 = torch.randn(E, N, K, dtype=torch.bfloat16) * 0.1
    logits = torch.randn(M, E, dtype=torch.float32)
    tw, ti = O.softmax_topk(logits, topk)
    return x, w1, w2, tw, ti


def _close(out, ref, tol):
    """Elementwise |out - ref| <= tol * rms(ref) + tol * |ref|, and the global
    relative error ||out - ref|| / ||ref|| below tol / 4.

    The absolute part scales with the output's RMS: both sides round the
    GEMM1 output and the activation to bf16, so a one-ulp flip there (from a
    different fp32 summation order) moves an output by about
    ulp(act) * |w2| * sqrt(#flips) -- proportional to the output scale, not
    to the value itself (the reference's own shapes, weights N(0,1)*0.1, give
    outputs of RMS ~10 where a cancelling element can sit near 0)."""
    out = out.float().cpu()
    ref = ref.float()
    rms = float(ref.pow(2).mean().sqrt()) if ref.numel() else 1.0
    scale = max(rms, 1e-3)
    torch.testing.assert_close(out, ref, atol=tol * scale, rtol=tol)
    if ref.numel():
        rel = float((out - ref).norm() / ref.norm().clamp_min(1e-30))
        assert rel < tol / 4, f"global relative error {rel:.3e}"


def _close_literal(out, ref, tol):
    """north_star's tolerance as written: |out - ref| <= tol + tol * |ref|
    elementwise (torch.testing.assert_close(atol=rtol=tol)).  Used on the
    BASELINE input recipes (weights N(0, 0.02), outputs of RMS ~1), where
    one bf16 ulp of the output is well inside tol; the reference's own test
    shapes (weights N(0,1)*0.1, output RMS ~10, where an output ulp alone is
    0.06) take _close."""
    torch.testing.assert_close(out.float().cpu(), ref.float(), atol=tol, rtol=tol)


@pytest.mark.parametrize("shape", FUSED_MOE_SHAPES_SMALL + FUSED_MOE_SHAPES_LARGE,
                         ids=lambda s: "M{}_K{}_N{}_E{}_topk{}".format(*s))
def test_fused_moe(shape):
    M, K, N, E, topk = shape
    x, w1, w2, tw, ti = _ref_inputs(M, K, N, E, topk)
    rd, gi, si = F._standard_topk_to_triton_kernels(tw.to(DEV), ti.to(DEV), E)
    res = flaggems_sglang.triton_kernel_fused_experts(x.to(DEV), w1.to(DEV), w2.to(DEV), rd, gi, si)
    ref = O.fused_experts(x, w1.transpose(1, 2), w2.transpose(1, 2), tw, ti)
    _close(res, ref, 2e-2)


@pytest.mark.parametrize("shape", FUSED_MOE_SHAPES_SMALL, ids=lambda s: "M{}_K{}_N{}_E{}_topk{}".format(*s))
def test_fused_moe_input_gate(shape):
    M, K, N, E, topk = shape
    x, w1, w2, tw, ti = _ref_inputs(M, K, N, E, topk)
    rd, gi, si = F._standard_topk_to_triton_kernels(tw.to(DEV), ti.to(DEV), E)
    res = flaggems_sglang.triton_kernel_fused_experts(x.to(DEV), w1.to(DEV), w2.to(DEV), rd, gi, si,
                                                      apply_router_weight_on_input=True)
    ref = O.fused_experts(x, w1.transpose(1, 2), w2.transpose(1, 2), tw, ti,
                          apply_router_weight_on_input=True)
    _close(res, ref, 2e-2)


@pytest.mark.parametrize("topk", [1, 6, 12])
@pytest.mark.parametrize("M", [1, 3, 300])
def test_topk_counts(M, topk):
    """Top-k counts outside the BASELINE set: 1 (switch routing), 6 and 12
    (the top-k sum's 8-term batches end part-full), one token (GEMM2 and the
    top-k sum in one launch), decode and prefill; bit-identical reruns."""
    K, N, E = 256, 384, 32
    x, w1, w2, tw, ti = _ref_inputs(M, K, N, E, topk)
    w13, w2t = w1.transpose(1, 2).contiguous(), w2.transpose(1, 2).contiguous()
    args = (x.to(DEV), w13.to(DEV), w2t.to(DEV), tw.to(DEV), ti.to(DEV))
    out = flaggems_sglang.fused_experts(*args)
    _close(out, O.fused_experts(x, w13, w2t, tw, ti), 2e-2)
    assert torch.equal(out, flaggems_sglang.fused_experts(*args))


@pytest.mark.parametrize("path", [1, 2])
@pytest.mark.parametrize("M", [1, 16, 64, 300])
def test_fused_experts_both_paths(M, path):
    """Prefill (LDS-tiled) and decode (streaming) kernels on the same inputs."""
    K, N, E, k = 512, 384, 16, 4
    d = O.make_inputs(M, K, N, E, k, wscale=0.05)
    out = flaggems_sglang.fused_experts(d["x"].to(DEV), d["w13"].to(DEV), d["w2"].to(DEV),
                                        d["topk_weights"].to(DEV), d["topk_ids"].to(DEV), path=path)
    ref = O.fused_experts(d["x"], d["w13"], d["w2"], d["topk_weights"], d["topk_ids"])
    _close(out, ref, 2e-2)


def test_tiny_config():
    """M=64, K=128, N=256, E=8, top-2 (fp32 oracle; the
    GPU computes in bf16 with fp32 accumulation)."""
    d = O.make_inputs(64, 128, 256, 8, 2, wscale=0.02)
    out = flaggems_sglang.fused_experts(d["x"].to(DEV), d["w13"].to(DEV), d["w2"].to(DEV),
                                        d["topk_weights"].to(DEV), d["topk_ids"].to(DEV))
    ref = O.fused_experts(d["x"], d["w13"], d["w2"], d["topk_weights"], d["topk_ids"])
    _close(out, ref, 2e-2)


def test_routed_scaling_and_no_combine():
    d = O.make_inputs(40, 256, 256, 8, 2, wscale=0.05)
    args = [d[n].to(DEV) for n in ("x", "w13", "w2", "topk_weights", "topk_ids")]
    out = flaggems_sglang.fused_experts(*args, routed_scaling_factor=2.5)
    ref = O.fused_experts(d["x"], d["w13"], d["w2"], d["topk_weights"], d["topk_ids"],
                          routed_scaling_factor=2.5)
    _close(out, ref, 2e-2)
    per = flaggems_sglang.fused_experts(*args, no_combine=True)
    assert per.shape == (40, 2, 256)
    base = flaggems_sglang.fused_experts(*args)
    _close(per.float().sum(1), base.float().cpu(), 2e-2)


# ------------------------------------------------------------ BASELINE configs
def _bf16_case(M, K, N, E, k, bias=0.0, seed=None):
    d = O.make_inputs(M, K, N, E, k, wscale=0.02, expert_bias_std=bias, seed=seed)
    out = flaggems_sglang.fused_experts(d["x"].to(DEV), d["w13"].to(DEV), d["w2"].to(DEV),
                                        d["topk_weights"].to(DEV), d["topk_ids"].to(DEV))
    ref = O.fused_experts(d["x"], d["w13"], d["w2"], d["topk_weights"], d["topk_ids"])
    _close(out, ref, 2e-2)
    _close_literal(out, ref, 2e-2)


@pytest.mark.parametrize("M", [1, 16, 64, 256, 1024])
def test_qwen3_skewed_bf16(M):
    # E=128 top-8 K=2048 N=768, per-expert bias N(0, 0.5) skews the routing
    _bf16_case(M, 2048, 768, 128, 8, bias=0.5)


def test_mixtral_shape_bf16_small_experts():
    # Mixtral K/N at M=16 with all 8 experts (weights 2.8 GB bf16)
    _bf16_case(16, 4096, 14336, 8, 2)


@pytest.mark.parametrize("M", [1, 128, 512])
def test_dsv3_fp8(M):
    """DeepSeek-V3 shape fp8 W8A8 with 128x128 weight blocks, grouped top-k
    routing; E reduced to 32 to keep the CPU oracle within seconds (the
    kernels see the full K=7168, N=2048)."""
    K, N, E, k = 7168, 2048, 32, 8
    d = O.make_inputs(M, K, N, E, k, wscale=0.02, routing="grouped", n_group=8, topk_group=4)
    w13 = d["w13"].to(DEV)
    w2 = d["w2"].to(DEV)
    q1, s1 = Q.quantize_fp8_block(w13)
    q2, s2 = Q.quantize_fp8_block(w2)
    out = flaggems_sglang.fused_experts(d["x"].to(DEV), q1, q2, d["topk_weights"].to(DEV),
                                        d["topk_ids"].to(DEV), use_fp8_w8a8=True, w1_scale=s1,
                                        w2_scale=s2, block_shape=[128, 128])
    ref = O.fused_experts_fp8(d["x"], q1.cpu(), s1.cpu(), q2.cpu(), s2.cpu(), d["topk_weights"],
                              d["topk_ids"])
    _close(out, ref, 5e-2)
    _close_literal(out, ref, 5e-2)


@pytest.mark.parametrize("K,N", [(7168, 256), (8448, 256), (256, 8448)])
def test_fp8_tile_height_choice(K, N):
    """fp8 prefill at ~128 slots per expert picks 160-row tiles (one M-tile
    for experts of up to 160 slots); with K or N above 8192 the fused path
    and the stage path (triton_kernel_fused_experts) fall back to 128-row
    tiles.  Both against the oracle; uneven expert loads from the routing."""
    M, E, k = 256, 8, 4
    from flaggems_sglang import _lib as LB
    assert LB.lib().fmoe_choose_block_m(LB.W_FP8, M, k, E, 0) == 160
    assert F._block_m(LB.W_FP8, M, k, E, 0, K, N) == (160 if max(K, N) <= 8192 else 128)
    d = O.make_inputs(M, K, N, E, k, wscale=0.02)
    q1, s1 = Q.quantize_fp8_block(d["w13"].to(DEV))
    q2, s2 = Q.quantize_fp8_block(d["w2"].to(DEV))
    tw, ti = d["topk_weights"].to(DEV), d["topk_ids"].to(DEV)
    ref = O.fused_experts_fp8(d["x"], q1.cpu(), s1.cpu(), q2.cpu(), s2.cpu(), d["topk_weights"],
                              d["topk_ids"])
    out = flaggems_sglang.fused_experts(d["x"].to(DEV), q1, q2, tw, ti, use_fp8_w8a8=True, w1_scale=s1,
                                        w2_scale=s2, block_shape=[128, 128])
    _close(out, ref, 5e-2)
    rd, gi, si = F._standard_topk_to_triton_kernels(tw, ti, E)
    out2 = flaggems_sglang.triton_kernel_fused_experts(
        d["x"].to(DEV), q1.transpose(1, 2), q2.transpose(1, 2), rd, gi, si, use_fp8_w8a8=True,
        w1_scale=s1.transpose(1, 2), w2_scale=s2.transpose(1, 2), block_shape=[128, 128])
    _close(out2, ref, 5e-2)


def test_bf16_160_row_tiles_skewed():
    """bf16 prefill at 128 slots per expert on average takes 160-row tiles;
    skewed routing gives experts that need two of them and nearly empty
    ones, and K = 384 is not a multiple of the 256-wide output tile.  Fused
    and stage paths against the oracle."""
    M, K, N, E, k = 512, 384, 640, 8, 2
    from flaggems_sglang import _lib as LB
    assert LB.lib().fmoe_choose_block_m(LB.W_BF16, M, k, E, 0) == 160
    d = O.make_inputs(M, K, N, E, k, wscale=0.05, expert_bias_std=0.7)
    counts = torch.bincount(d["topk_ids"].flatten().long(), minlength=E)
    assert int(counts.max()) > 160 and int(counts.min()) < 128
    tw, ti = d["topk_weights"].to(DEV), d["topk_ids"].to(DEV)
    ref = O.fused_experts(d["x"], d["w13"], d["w2"], d["topk_weights"], d["topk_ids"])
    out = flaggems_sglang.fused_experts(d["x"].to(DEV), d["w13"].to(DEV), d["w2"].to(DEV), tw, ti)
    _close(out, ref, 2e-2)
    rd, gi, si = F._standard_topk_to_triton_kernels(tw, ti, E)
    out2 = flaggems_sglang.triton_kernel_fused_experts(
        d["x"].to(DEV), d["w13"].transpose(1, 2).to(DEV), d["w2"].transpose(1, 2).to(DEV), rd, gi, si)
    _close(out2, ref, 2e-2)


@pytest.mark.parametrize("M", [1, 4, 16, 64, 256])  # 256: ~64 slots per expert, paired row-split tiles
def test_mixtral_w4a16(M):
    K, N, E, k = 4096, 14336, 8, 2
    d = O.make_inputs(M, K, N, E, k, wscale=0.02)
    q1, sc1, z1 = Q.quantize_int4_group(d["w13"].to(DEV))
    q2, sc2, z2 = Q.quantize_int4_group(d["w2"].to(DEV))
    out = flaggems_sglang.fused_experts(d["x"].to(DEV), q1, q2, d["topk_weights"].to(DEV),
                                        d["topk_ids"].to(DEV), use_int4_w4a16=True, w1_scale=sc1,
                                        w2_scale=sc2, w1_zp=z1, w2_zp=z2)
    ref = O.fused_experts_w4a16(d["x"], q1.cpu(), sc1.cpu(), z1.cpu(), q2.cpu(), sc2.cpu(),
                                z2.cpu(), d["topk_weights"], d["topk_ids"])
    _close(out, ref, 5e-2)
    _close_literal(out, ref, 5e-2)
    # the tiled layout (the one serving loads by default) at the same full shape
    outt = flaggems_sglang.fused_experts(d["x"].to(DEV), Q.tile_int4(q1), Q.tile_int4(q2),
                                         d["topk_weights"].to(DEV), d["topk_ids"].to(DEV),
                                         use_int4_w4a16=True, w1_scale=sc1, w2_scale=sc2, w1_zp=z1,
                                         w2_zp=z2)
    _close(outt, ref, 5e-2)
    _close_literal(outt, ref, 5e-2)


def test_product_quantizers_match_oracle():
    g = torch.Generator().manual_seed(11)
    w = (torch.randn(2, 256, 384, generator=g) * 0.02).to(torch.bfloat16)
    q, s = Q.quantize_fp8_block(w.to(DEV))
    qo, so = O.block_quant_fp8(w)
    assert torch.equal(q.cpu().view(torch.uint8), qo.view(torch.uint8)) and torch.equal(s.cpu(), so)
    a, b, c = Q.quantize_int4_group(w.to(DEV))
    ao, bo, co = O.quant_int4(w)
    assert torch.equal(a.cpu(), ao) and torch.equal(b.cpu(), bo) and torch.equal(c.cpu(), co)


# --------------------------------------------- full-size, size-independent checks
def test_mixtral_prefill_permutation_and_determinism():
    """Mixtral bf16 at M=4096 (the bench workload): outputs are bit-identical
    across runs, and permuting the tokens permutes the output rows -- exactly
    except for rows that land in a GEMM2 tail-split tile in one of the two
    runs (each XCD's last partial round of tiles is reduced in split parts,
    and which tiles those are follows the token order), which agree to bf16
    rounding.  The whole output against the oracle."""
    M, K, N, E, k = 4096, 4096, 14336, 8, 2
    gen = torch.Generator(device=DEV).manual_seed(7)
    x = torch.randn(M, K, device=DEV, generator=gen).to(torch.bfloat16)
    w13 = (torch.randn(E, 2 * N, K, device=DEV, generator=gen) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(E, K, N, device=DEV, generator=gen) * 0.02).to(torch.bfloat16)
    logits = torch.randn(M, E, device=DEV, generator=gen)
    tw, ti = flaggems_sglang.topk_softmax(logits, k)
    a = flaggems_sglang.fused_experts(x, w13, w2, tw, ti)
    b = flaggems_sglang.fused_experts(x, w13, w2, tw, ti)
    assert torch.equal(a, b)
    perm = torch.randperm(M, device=DEV, generator=gen)
    c = flaggems_sglang.fused_experts(x[perm], w13, w2, tw[perm], ti[perm])
    differ = (c != a[perm]).any(dim=1).float().mean().item()
    assert differ < 0.5, f"{differ:.2%} of the rows differ under the permutation"
    # a slot row's bf16 rounding can flip by one ulp, and the top-k sum can
    # cancel it to a small output: the absolute part scales with the RMS
    rms = float(a.float().pow(2).mean().sqrt())
    torch.testing.assert_close(c.float(), a[perm].float(), rtol=2 ** -7, atol=2 ** -7 * rms)
    ref = O.fused_experts(x.cpu(), w13.cpu(), w2.cpu(), tw.cpu(), ti.cpu())
    _close(a, ref, 2e-2)
    _close_literal(a, ref, 2e-2)


# ------------------------------------------------------------ activations / bias path
@pytest.mark.parametrize("path", [1, 2])
@pytest.mark.parametrize("M", [1, 64, 300])
def test_gelu_activation(M, path):
    """activation="gelu" (ops/fused_moe.py:203-204) on both kernel families."""
    K, N, E, k = 512, 384, 16, 4
    d = O.make_inputs(M, K, N, E, k, wscale=0.05)
    out = flaggems_sglang.fused_experts(d["x"].to(DEV), d["w13"].to(DEV), d["w2"].to(DEV),
                                        d["topk_weights"].to(DEV), d["topk_ids"].to(DEV), path=path,
                                        activation="gelu")
    ref = O.fused_experts(d["x"], d["w13"], d["w2"], d["topk_weights"], d["topk_ids"],
                          activation="gelu")
    _close(out, ref, 2e-2)


@pytest.mark.parametrize("shape", FUSED_MOE_SHAPES_SMALL, ids=lambda s: "M{}_K{}_N{}_E{}_topk{}".format(*s))
def test_gelu_reference_api(shape):
    M, K, N, E, topk = shape
    x, w1, w2, tw, ti = _ref_inputs(M, K, N, E, topk)
    rd, gi, si = F._standard_topk_to_triton_kernels(tw.to(DEV), ti.to(DEV), E)
    res = flaggems_sglang.triton_kernel_fused_experts(x.to(DEV), w1.to(DEV), w2.to(DEV), rd, gi, si,
                                                      activation="gelu")
    ref = O.fused_experts(x, w1.transpose(1, 2), w2.transpose(1, 2), tw, ti, activation="gelu")
    _close(res, ref, 2e-2)


@pytest.mark.parametrize("on_input", [False, True])
@pytest.mark.parametrize("alpha,limit", [(None, None), (1.702, 7.0), (1.0, 0.05)])
@pytest.mark.parametrize("M", [1, 16, 200])
def test_bias_swiglu(M, alpha, limit, on_input):
    """triton_kernel_fused_experts_with_bias (ops/fused_moe.py:219-309): biases,
    interleaved swiglu with alpha / clamp limit, both routing-weight placements,
    decode (M <= 16) and prefill kernels."""
    K, N, E, k = 256, 384, 8, 2
    d = O.make_inputs(M, K, N, E, k, wscale=0.05)
    gen = torch.Generator().manual_seed(M + 3)
    b13 = torch.randn(E, 2 * N, generator=gen) * 0.1
    b2 = torch.randn(E, K, generator=gen) * 0.1
    rd, gi, si = F._standard_topk_to_triton_kernels(d["topk_weights"].to(DEV), d["topk_ids"].to(DEV), E)
    w1 = d["w13"].transpose(1, 2).to(DEV)          # matmul_ogs layout [E, K, 2N], interleaved columns
    w2 = d["w2"].transpose(1, 2).to(DEV)           # [E, N, K]
    out = flaggems_sglang.triton_kernel_fused_experts_with_bias(
        d["x"].to(DEV), w1, None, b13.to(DEV), w2, None, b2.to(DEV), rd, gi, si,
        apply_router_weight_on_input=on_input, gemm1_alpha=alpha, gemm1_clamp_limit=limit)
    ref = O.fused_experts_bias(d["x"], d["w13"], b13, d["w2"], b2, d["topk_weights"], d["topk_ids"],
                               apply_router_weight_on_input=on_input,
                               alpha=1.0 if alpha is None else alpha, limit=limit)
    _close(out, ref, 2e-2)


# ------------------------------------------------------------ expert parallel
@pytest.mark.parametrize("M", [3, 200, 700])  # 700: several 256-token routing chunks
def test_expert_map(M):
    """expert_map / global_num_experts (ops/fused_moe.py:145-146,160): identity
    map equals no map bit for bit; a two-rank split matches the oracle per rank
    and the partials sum to the single-rank output."""
    K, N, E, k = 256, 384, 16, 4
    d = O.make_inputs(M, K, N, E, k, wscale=0.05)
    x, w13, w2 = d["x"].to(DEV), d["w13"].to(DEV), d["w2"].to(DEV)
    tw, ti = d["topk_weights"].to(DEV), d["topk_ids"].to(DEV)
    full = flaggems_sglang.fused_experts(x, w13, w2, tw, ti)
    ident = flaggems_sglang.fused_experts(x, w13, w2, tw, ti, expert_map=torch.arange(E, device=DEV),
                                          global_num_experts=E)
    assert torch.equal(full, ident)
    parts = []
    for r in range(2):
        emap = torch.full((E,), -1, dtype=torch.int32)
        emap[r::2] = torch.arange(E // 2, dtype=torch.int32)      # rank r owns experts r, r+2, ...
        lw13, lw2 = d["w13"][r::2].contiguous(), d["w2"][r::2].contiguous()
        out = flaggems_sglang.fused_experts(x, lw13.to(DEV), lw2.to(DEV), tw, ti,
                                            expert_map=emap.to(DEV), global_num_experts=E)
        ltw, lti = O.ep_localize(d["topk_weights"], d["topk_ids"], emap)
        _close(out, O.fused_experts(d["x"], lw13, lw2, ltw, lti), 2e-2)
        parts.append(out.float())
    _close(parts[0] + parts[1], O.fused_experts(d["x"], d["w13"], d["w2"], d["topk_weights"],
                                                d["topk_ids"]).float(), 2e-2)


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("M", [1, 5, 16])
def test_tiny_decode_path_equals_aligned_path(M, fp8):
    """fused_experts at M <= 16 (bf16 / fp8) computes each tile's routing
    inside the GEMM workgroups instead of launching the align kernels; the
    tiles, their row order and every sum are the same, so the output equals
    the aligned path (triton_kernel_fused_experts) bit for bit."""
    K, N, E, k = 512, 384, 16, 4
    d = O.make_inputs(M, K, N, E, k, wscale=0.05)
    x, w13, w2 = d["x"].to(DEV), d["w13"].to(DEV), d["w2"].to(DEV)
    tw, ti = d["topk_weights"].to(DEV), d["topk_ids"].to(DEV)
    kw, tkw = {}, {}
    if fp8:
        w13, s13 = Q.quantize_fp8_block(w13)
        w2, s2 = Q.quantize_fp8_block(w2)
        kw = dict(use_fp8_w8a8=True, w1_scale=s13, w2_scale=s2, block_shape=[128, 128])
        tkw = dict(use_fp8_w8a8=True, w1_scale=s13.transpose(1, 2), w2_scale=s2.transpose(1, 2),
                   block_shape=[128, 128])
    out = flaggems_sglang.fused_experts(x, w13, w2, tw, ti, **kw)
    rd, gi, si = F._standard_topk_to_triton_kernels(tw, ti, E)
    ref = flaggems_sglang.triton_kernel_fused_experts(x, w13.transpose(1, 2), w2.transpose(1, 2),
                                                      rd, gi, si, **tkw)
    assert torch.equal(out, ref)


# ------------------------------------------------------------ fused-path internals
@pytest.mark.parametrize("M,on_input", [(256, False), (200, True), (1024, False)])
def test_fp8_fused_act_quant_matches_stage_path(M, on_input):
    """The fused fp8 prefill path quantizes the GEMM1 activation in the GEMM1
    epilogue; the stage path (triton_kernel_fused_experts) runs the separate
    fmoe_quant_fp8_group pass on the bf16 activation.  At N = 16384 the
    stage path splits GEMM2 into fp32 planes while the fused path keeps whole
    tiles as bf16 slot rows and splits only each XCD's tail tiles, so the two
    differ by GEMM2 summation order and the slot rows' bf16 rounding (about
    one bf16 ulp of an output): far inside the fp8 tolerance, and a wrong
    activation code would be a much larger error only where it matters."""
    K, N, E, k = 512, 16384, 8, 2
    d = O.make_inputs(M, K, N, E, k, wscale=0.02)
    q1, s1 = Q.quantize_fp8_block(d["w13"].to(DEV))
    q2, s2 = Q.quantize_fp8_block(d["w2"].to(DEV))
    tw, ti = d["topk_weights"].to(DEV), d["topk_ids"].to(DEV)
    x = d["x"].to(DEV)
    fused = flaggems_sglang.fused_experts(x, q1, q2, tw, ti, use_fp8_w8a8=True, w1_scale=s1, w2_scale=s2,
                                          block_shape=[128, 128], apply_router_weight_on_input=on_input)
    rd, gi, si = F._standard_topk_to_triton_kernels(tw, ti, E)
    staged = flaggems_sglang.triton_kernel_fused_experts(
        x, q1.transpose(1, 2), q2.transpose(1, 2), rd, gi, si, use_fp8_w8a8=True,
        w1_scale=s1.transpose(1, 2), w2_scale=s2.transpose(1, 2), block_shape=[128, 128],
        apply_router_weight_on_input=on_input)
    f, g = fused.float(), staged.float()
    rms = float(g.pow(2).mean().sqrt())
    torch.testing.assert_close(f, g, rtol=2 ** -6, atol=2 ** -6 * rms)
    rel = float((f - g).norm() / g.norm())
    assert rel < 4e-3, f"relative difference {rel:.3e}"


@pytest.mark.parametrize("on_input", [False, True])
def test_fp8_fused_act_quant_bit_exact_identity_w2(on_input):
    """Pins the fused fp8 path's in-epilogue activation quantization bit for
    bit against the stage path's separate fmoe_quant_fp8_group pass.  With
    K = N, w2 = the identity (fp8, 128x128 block scales) and top-1 routing,
    each GEMM2 output element has exactly one nonzero term, so every GEMM2
    summation order (whole tiles, tail split, split-K planes) gives the same
    bits, and the two outputs can differ only through the activation codes
    and scales."""
    M, K, E, k = 512, 512, 4, 1
    N = K
    d = O.make_inputs(M, K, N, E, k, wscale=0.02)
    eye = torch.eye(K, dtype=torch.bfloat16).expand(E, K, K).contiguous()
    q1, s1 = Q.quantize_fp8_block(d["w13"].to(DEV))
    q2, s2 = Q.quantize_fp8_block(eye.to(DEV))
    tw, ti = d["topk_weights"].to(DEV), d["topk_ids"].to(DEV)
    x = d["x"].to(DEV)
    fused = flaggems_sglang.fused_experts(x, q1, q2, tw, ti, use_fp8_w8a8=True, w1_scale=s1, w2_scale=s2,
                                          block_shape=[128, 128], apply_router_weight_on_input=on_input)
    rd, gi, si = F._standard_topk_to_triton_kernels(tw, ti, E)
    staged = flaggems_sglang.triton_kernel_fused_experts(
        x, q1.transpose(1, 2), q2.transpose(1, 2), rd, gi, si, use_fp8_w8a8=True,
        w1_scale=s1.transpose(1, 2), w2_scale=s2.transpose(1, 2), block_shape=[128, 128],
        apply_router_weight_on_input=on_input)
    assert torch.count_nonzero(fused) > fused.numel() // 2  # a real activation, not zeros
    assert torch.equal(fused, staged)


@pytest.mark.parametrize("M", [1, 5, 16])
def test_int4_identity_expert_map_bit_exact(M):
    """int4 decode with an identity expert map (the expert-parallel routing
    path of fmoe_align_ex) equals the call without a map, bit for bit."""
    K, N, E, k = 512, 384, 16, 4
    d = O.make_inputs(M, K, N, E, k, wscale=0.05)
    q1, s1, z1 = Q.quantize_int4_group(d["w13"].to(DEV))
    q2, s2, z2 = Q.quantize_int4_group(d["w2"].to(DEV))
    args = (d["x"].to(DEV), q1, q2, d["topk_weights"].to(DEV), d["topk_ids"].to(DEV))
    kw = dict(use_int4_w4a16=True, w1_scale=s1, w2_scale=s2, w1_zp=z1, w2_zp=z2)
    plain = flaggems_sglang.fused_experts(*args, **kw)
    emap = torch.arange(E, dtype=torch.int32, device=DEV)
    mapped = flaggems_sglang.fused_experts(*args, expert_map=emap, global_num_experts=E, **kw)
    assert torch.equal(plain, mapped)
