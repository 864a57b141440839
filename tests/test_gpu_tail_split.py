"""Prefill GEMM2 tail split on the GPU (fused path).

Calls whose GEMM2 the split rule would cut into fp32 planes (few output tiles,
a long reduction) run whole tiles as bf16 slot rows and split only each XCD's
last partial round; ``tail_fold_kernel`` adds the parts.  These shapes take
that route (asserted through the C ABI's own split rule), with K = 640 so the
last output tile is partial (640 = 2 x 256 + 128), across the bf16 tile
heights 64 / 160 / 256, the fp8 128-row tiles and SwiGLU with both biases.  Whole output against the
oracle, and bit identity across runs.
"""

import ctypes

import pytest
import torch

import flaggems_sglang
from flaggems_sglang import _lib
from flaggems_sglang import quant as Q
from oracle import fused_moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _takes_tail_split(wt, M, K, N, E, k):
    L = _lib.lib()
    bm = L.fmoe_fused_block_m(wt, M, k, E, 0, K, N)
    r = _lib.Routing(None, None, None, None, None, None, None, M, k, E, bm, L.fmoe_max_tiles(M * k, E))
    return bm, bm > 16 and L.fmoe_gemm2_splits(wt, K, N, ctypes.byref(r), 0) > 1


def _close(out, ref, tol):
    out, ref = out.float().cpu(), ref.float()
    rms = float(ref.pow(2).mean().sqrt())
    torch.testing.assert_close(out, ref, atol=tol * rms, rtol=tol)
    rel = float((out - ref).norm() / ref.norm())
    assert rel < tol / 4, f"relative error {rel:.3e}"


@pytest.mark.parametrize("M,N,bm", [(64, 8192, 64), (256, 16384, 160), (512, 16384, 256)])
def test_bf16_tail_split(M, N, bm):
    K, E, k = 640, 4, 2
    got_bm, tail = _takes_tail_split(_lib.W_BF16, M, K, N, E, k)
    assert got_bm == bm and tail
    d = O.make_inputs(M, K, N, E, k, wscale=0.02)
    args = (d["x"].to(DEV), d["w13"].to(DEV), d["w2"].to(DEV), d["topk_weights"].to(DEV), d["topk_ids"].to(DEV))
    a = flaggems_sglang.fused_experts(*args)
    b = flaggems_sglang.fused_experts(*args)
    assert torch.equal(a, b)
    _close(a, O.fused_experts(d["x"], d["w13"], d["w2"], d["topk_weights"], d["topk_ids"]), 2e-2)


def test_fp8_tail_split():
    M, K, N, E, k = 256, 640, 16384, 4, 2
    got_bm, tail = _takes_tail_split(_lib.W_FP8, M, K, N, E, k)
    assert got_bm == 128 and tail
    d = O.make_inputs(M, K, N, E, k, wscale=0.02)
    q1, s1 = Q.quantize_fp8_block(d["w13"].to(DEV))
    q2, s2 = Q.quantize_fp8_block(d["w2"].to(DEV))
    kw = dict(use_fp8_w8a8=True, w1_scale=s1, w2_scale=s2, block_shape=[128, 128])
    args = (d["x"].to(DEV), q1, q2, d["topk_weights"].to(DEV), d["topk_ids"].to(DEV))
    a = flaggems_sglang.fused_experts(*args, **kw)
    b = flaggems_sglang.fused_experts(*args, **kw)
    assert torch.equal(a, b)
    ref = O.fused_experts_fp8(d["x"], q1.cpu(), s1.cpu(), q2.cpu(), s2.cpu(), d["topk_weights"], d["topk_ids"])
    _close(a, ref, 5e-2)


@pytest.mark.parametrize("M", [64, 256])
def test_bf16_swiglu_bias_tail_split(M):
    """SwiGLU with both biases (alpha, clamp) through the C ABI's fused path at
    tail-split shapes: GEMM2's bias enters the split-0 part only, so every
    output adds it once.  Against the bias path's oracle."""
    K, N, E, k = 640, 8192, 4, 2
    got_bm, tail = _takes_tail_split(_lib.W_BF16, M, K, N, E, k)
    assert got_bm > 16 and tail
    d = O.make_inputs(M, K, N, E, k, wscale=0.02)
    g = torch.Generator().manual_seed(M)
    b13 = torch.randn(E, 2 * N, generator=g) * 0.1
    b2 = torch.randn(E, K, generator=g) * 0.1
    alpha, limit = 1.702, 7.0
    x, tw, ti = d["x"].to(DEV), d["topk_weights"].to(DEV), d["topk_ids"].to(DEV)
    w13, w2 = d["w13"].to(DEV), d["w2"].to(DEV)
    b13d, b2d = b13.to(DEV), b2.to(DEV)
    L = _lib.lib()
    st = torch.cuda.current_stream().cuda_stream

    def run():
        out = torch.empty(M, K, dtype=torch.bfloat16, device=DEV)
        a = _lib.FusedArgs(_lib.W_BF16, x.data_ptr(), M, K, N, E, k, w13.data_ptr(), w2.data_ptr(),
                           None, None, None, None, 128, tw.data_ptr(), ti.data_ptr(), 0, 1.0, 0,
                           out.data_ptr(), None, 0, _lib.ACT_SWIGLU, b13d.data_ptr(), b2d.data_ptr(),
                           alpha, limit, None, 0)
        n = L.fmoe_fused_experts_workspace_bytes(ctypes.byref(a))
        ws = torch.empty(max(n, 1), dtype=torch.uint8, device=DEV)
        a.workspace, a.workspace_bytes = ws.data_ptr(), n
        _lib.check(L.fmoe_fused_experts(ctypes.byref(a), st), "fused_experts")
        torch.cuda.synchronize()
        return out

    a = run()
    assert torch.equal(a, run())
    ref = O.fused_experts_bias(d["x"], d["w13"], b13, d["w2"], b2, d["topk_weights"], d["topk_ids"],
                               alpha=alpha, limit=limit)
    _close(a, ref, 2e-2)
