"""Seeded random shapes through the fused op, every weight format (GPU).

A fixed list of shapes drawn once from a seeded generator: M from 1 to 600,
K and N multiples of 128 up to 1024 / 2048, E from 1 to 16, top-k up to 8,
routing softmax or skewed.  The draws land on the decode kernels (one-token
and tiny-batch routes included), the prefill kernels at every tile height
and, for 4-bit weights, the row-split and one-launch decode kernels.  Each
output against the oracle at north_star's tolerance (bf16 2e-2, fp8 / int4 /
MXFP4 5e-2, the absolute part scaled by the output RMS where that exceeds
1), and bit identity across two runs.
"""

import random

import pytest
import torch

import flaggems_sglang
from flaggems_sglang import quant as Q
from oracle import fused_moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
FORMATS = ["bf16", "fp8", "int4", "int4t", "mxfp4", "mxfp4t"]


def _shapes(n=30, seed=20261202):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        fmt = FORMATS[i % len(FORMATS)]
        E = rng.randint(1, 16)
        k = rng.randint(1, min(8, E))
        M = rng.choice([1, 1, 2, 5, 16, 33, 64, 128, 300, 600])
        K = 128 * rng.randint(1, 8)
        N = 128 * rng.randint(1, 16)
        out.append((fmt, M, K, N, E, k, rng.random() < 0.3, rng.randint(0, 10 ** 6)))
    return out


def _close(out, ref, tol):
    """north_star's tolerance (atol = rtol = tol) with the absolute part
    scaled up by the output RMS where that exceeds 1 (a one-ulp flip of an
    fp8 / bf16 intermediate moves an output in proportion to the output
    scale), and the global relative error below tol / 4."""
    out, ref = out.float().cpu(), ref.float()
    rms = float(ref.pow(2).mean().sqrt())
    torch.testing.assert_close(out, ref, atol=tol * max(rms, 1.0), rtol=tol)
    rel = float((out - ref).norm() / ref.norm().clamp_min(1e-30))
    assert rel < tol / 4, f"relative error {rel:.3e}"


@pytest.mark.parametrize("fmt,M,K,N,E,k,skew,seed", _shapes(),
                         ids=lambda v: str(v))
def test_random_shape(fmt, M, K, N, E, k, skew, seed):
    d = O.make_inputs(M, K, N, E, k, wscale=0.03, seed=seed, expert_bias_std=1.0 if skew else 0.0)
    x, tw, ti = d["x"].to(DEV), d["topk_weights"].to(DEV), d["topk_ids"].to(DEV)
    w13, w2 = d["w13"].to(DEV), d["w2"].to(DEV)
    args = (d["topk_weights"], d["topk_ids"])
    if fmt == "bf16":
        kw, tol = {}, 2e-2
        a1, a2 = w13, w2
        ref = O.fused_experts(d["x"], d["w13"], d["w2"], *args)
    elif fmt == "fp8":
        a1, s1 = Q.quantize_fp8_block(w13)
        a2, s2 = Q.quantize_fp8_block(w2)
        kw, tol = dict(use_fp8_w8a8=True, w1_scale=s1, w2_scale=s2, block_shape=[128, 128]), 5e-2
        ref = O.fused_experts_fp8(d["x"], a1.cpu(), s1.cpu(), a2.cpu(), s2.cpu(), *args)
    elif fmt in ("int4", "int4t"):
        q1, s1, z1 = Q.quantize_int4_group(w13)
        q2, s2, z2 = Q.quantize_int4_group(w2)
        kw, tol = dict(use_int4_w4a16=True, w1_scale=s1, w2_scale=s2, w1_zp=z1, w2_zp=z2), 5e-2
        a1, a2 = (Q.tile_int4(q1), Q.tile_int4(q2)) if fmt == "int4t" else (q1, q2)
        ref = O.fused_experts_w4a16(d["x"], q1.cpu(), s1.cpu(), z1.cpu(), q2.cpu(), s2.cpu(), z2.cpu(), *args)
    else:
        q1, s1 = Q.quantize_mxfp4(w13)
        q2, s2 = Q.quantize_mxfp4(w2)
        kw, tol = dict(use_mxfp4_w4a16=True, w1_scale=s1, w2_scale=s2), 5e-2
        a1, a2 = (Q.tile_mxfp4(q1), Q.tile_mxfp4(q2)) if fmt == "mxfp4t" else (q1, q2)
        ref = O.fused_experts_mxfp4(d["x"], q1.cpu(), s1.cpu(), q2.cpu(), s2.cpu(), *args)
    out = flaggems_sglang.fused_experts(x, a1, a2, tw, ti, **kw)
    again = flaggems_sglang.fused_experts(x, a1, a2, tw, ti, **kw)
    assert torch.equal(out, again), "not bit-identical across runs"
    _close(out, ref, tol)


def _option_draws(n=18, seed=1202):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        fp8 = i % 3 == 2
        E = rng.randint(2, 16)
        on_input = (not fp8) and rng.random() < 0.25
        k = 1 if on_input else rng.randint(1, min(6, E))
        out.append(dict(fp8=fp8, M=rng.choice([1, 3, 16, 40, 300]), K=128 * rng.randint(1, 6),
                        N=128 * rng.randint(1, 12), E=E, k=k, on_input=on_input,
                        gelu=(not fp8) and rng.random() < 0.4, rsf=rng.choice([None, 2.5]),
                        drop=rng.random() < 0.35, seed=rng.randint(0, 10 ** 6)))
    return out


@pytest.mark.parametrize("o", _option_draws(), ids=lambda o: "-".join(f"{k}{v}" for k, v in o.items() if k != "seed"))
def test_random_options(o):
    """Seeded draws of the call options: GELU, the routing weight on the input
    (top-1), routed_scaling_factor, and an expert map that drops experts (a
    dropped choice contributes nothing, as in expert parallelism); bf16 and
    fp8 against the oracle on the localized routing."""
    M, K, N, E, k = o["M"], o["K"], o["N"], o["E"], o["k"]
    d = O.make_inputs(M, K, N, E, k, wscale=0.03, seed=o["seed"])
    x, tw, ti = d["x"].to(DEV), d["topk_weights"].to(DEV), d["topk_ids"].to(DEV)
    ltw, lti = d["topk_weights"], d["topk_ids"]
    kw = dict(apply_router_weight_on_input=o["on_input"], routed_scaling_factor=o["rsf"])
    if o["drop"]:
        emap = torch.arange(E, dtype=torch.int32)
        emap[torch.randperm(E, generator=torch.Generator().manual_seed(o["seed"]))[: max(1, E // 3)]] = -1
        kw.update(expert_map=emap.to(DEV), global_num_experts=E)
        ltw, lti = O.ep_localize(ltw, lti, emap)
    if o["fp8"]:
        a1, s1 = Q.quantize_fp8_block(d["w13"].to(DEV))
        a2, s2 = Q.quantize_fp8_block(d["w2"].to(DEV))
        kw.update(use_fp8_w8a8=True, w1_scale=s1, w2_scale=s2, block_shape=[128, 128])
        ref = O.fused_experts_fp8(d["x"], a1.cpu(), s1.cpu(), a2.cpu(), s2.cpu(), ltw, lti,
                                  routed_scaling_factor=o["rsf"])
        tol = 5e-2
    else:
        a1, a2 = d["w13"].to(DEV), d["w2"].to(DEV)
        act = "gelu" if o["gelu"] else "silu"
        kw.update(activation=act)
        ref = O.fused_experts(d["x"], d["w13"], d["w2"], ltw, lti, apply_router_weight_on_input=o["on_input"],
                              routed_scaling_factor=o["rsf"], activation=act)
        tol = 2e-2
    out = flaggems_sglang.fused_experts(x, a1, a2, tw, ti, **kw)
    assert torch.equal(out, flaggems_sglang.fused_experts(x, a1, a2, tw, ti, **kw))
    _close(out, ref, tol)
