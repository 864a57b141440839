"""MXFP4 weights (OCP e2m1 + e8m0 block scales, bf16 activations).

CPU: the oracle's E2M1 coding against the OCP table and its tie / saturation
known answers, its quantizer against torch's reference MX quantizer
(``to_mxfp``) bit for bit, the product quantizer against the oracle, and the
scale semantics.  GPU (``gpu``): the HIP streaming kernels through the C ABI
against the oracle (bf16 tolerance: the dequantized weights are exact, so
only the bf16 rounding points differ), plain and bias/swiglu paths, and the
SGLang hook on an MXFP4 layer.
"""

import sys
import types

import numpy as np
import pytest
import torch

from oracle import fused_moe_oracle as O

OCP_E2M1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]


def test_e2m1_table_and_known_answers():
    codes = np.arange(16, dtype=np.uint8)
    assert O.e2m1_decode(codes).tolist() == OCP_E2M1
    # every representable value encodes to its own code
    assert np.array_equal(O.e2m1_encode(np.array(OCP_E2M1[:8], np.float32)), codes[:8])
    # ties go to the even code, beyond 6 saturates
    v = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 7.0, 100.0, 0.26, -0.75, -5.5], np.float32)
    want = [0, 2, 2, 4, 4, 6, 6, 7, 7, 1, 10, 15]
    assert O.e2m1_encode(v).tolist() == want


def test_e8m0_scale_values():
    s = np.array([127, 128, 120, 0, 254], np.uint8)
    assert O.e8m0_value(s).tolist() == [1.0, 2.0, 2.0 ** -7, 2.0 ** -127, 2.0 ** 127]
    assert np.isnan(O.e8m0_value(np.array([255], np.uint8))[0])


def _torch_reference_mx():
    """torch's reference MX quantizer; its module imports a test-only package
    that this image lacks, stood in for by an empty module."""
    sys.modules.setdefault("expecttest", types.ModuleType("expecttest"))
    if not hasattr(sys.modules["expecttest"], "TestCase"):
        sys.modules["expecttest"].TestCase = object
    try:
        from torch.testing._internal.common_quantized import to_mxfp
    except Exception as exc:  # pragma: no cover
        pytest.skip(f"torch reference MX quantizer not importable: {exc}")
    return to_mxfp


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_oracle_quantizer_matches_torch_reference(seed):
    to_mxfp = _torch_reference_mx()
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(3, 16, 256, generator=g) * (0.02 if seed else 3.0)).to(torch.bfloat16)
    w[0, 0, :32] = 0  # an all-zero block
    scale_t, data_t = to_mxfp(w.reshape(-1, 256).contiguous(), 32, "mxfp4")
    q, s = O.mxfp4_quant(w)
    assert torch.equal(s.reshape(-1), scale_t.view(torch.uint8).reshape(-1))
    assert torch.equal(q.reshape(-1), data_t.view(torch.uint8).reshape(-1))


def test_product_quantizer_matches_oracle_and_round_trip():
    from flaggems_sglang import quant as Q

    g = torch.Generator().manual_seed(5)
    w = (torch.randn(2, 32, 512, generator=g) * 0.02).to(torch.bfloat16)
    q, s = Q.quantize_mxfp4(w)
    qo, so = O.mxfp4_quant(w)
    assert torch.equal(q, qo) and torch.equal(s, so)
    # values already on the MXFP4 grid survive quantize -> dequantize
    d = O.mxfp4_dequant(qo, so).to(torch.bfloat16)
    q2, s2 = O.mxfp4_quant(d)
    assert torch.equal(O.mxfp4_dequant(q2, s2), d.float())


# ------------------------------------------------------------------ GPU
DEV = "cuda"


def _close(out, ref, tol=2e-2):
    out = out.float().cpu()
    ref = ref.float()
    scale = max(float(ref.pow(2).mean().sqrt()), 1e-3)
    torch.testing.assert_close(out, ref, atol=tol * scale, rtol=tol)
    rel = float((out - ref).norm() / ref.norm().clamp_min(1e-30))
    assert rel < tol / 4, f"global relative error {rel:.3e}"


def _mx_case(M, K, N, E, k, seed=None):
    from flaggems_sglang import quant as Q

    d = O.make_inputs(M, K, N, E, k, wscale=0.05, seed=seed)
    q13, s13 = Q.quantize_mxfp4(d["w13"])
    q2, s2 = Q.quantize_mxfp4(d["w2"])
    return d, q13, s13, q2, s2


@pytest.mark.gpu
@pytest.mark.parametrize("on_input", [False, True])
@pytest.mark.parametrize("M", [1, 16, 200])
def test_gpu_mxfp4_fused_experts(M, on_input):
    import flaggems_sglang

    K, N, E, k = 512, 384, 8, 2
    d, q13, s13, q2, s2 = _mx_case(M, K, N, E, k)
    out = flaggems_sglang.fused_experts(
        d["x"].to(DEV), q13.to(DEV), q2.to(DEV), d["topk_weights"].to(DEV), d["topk_ids"].to(DEV),
        use_mxfp4_w4a16=True, w1_scale=s13.to(DEV), w2_scale=s2.to(DEV),
        apply_router_weight_on_input=on_input)
    ref = O.fused_experts_mxfp4(d["x"], q13, s13, q2, s2, d["topk_weights"], d["topk_ids"],
                                apply_router_weight_on_input=on_input)
    _close(out, ref)


@pytest.mark.gpu
def test_gpu_mxfp4_mixtral_shape_gelu_and_e8m0_dtype():
    import flaggems_sglang

    M, K, N, E, k = 4, 4096, 14336, 8, 2
    d, q13, s13, q2, s2 = _mx_case(M, K, N, E, k)
    args = (d["x"].to(DEV), q13.to(DEV), q2.to(DEV), d["topk_weights"].to(DEV), d["topk_ids"].to(DEV))
    out = flaggems_sglang.fused_experts(*args, use_mxfp4_w4a16=True, activation="gelu",
                                        w1_scale=s13.to(DEV).view(torch.float8_e8m0fnu),
                                        w2_scale=s2.to(DEV).view(torch.float8_e8m0fnu))
    ref = O.fused_experts_mxfp4(d["x"], q13, s13, q2, s2, d["topk_weights"], d["topk_ids"],
                                activation="gelu")
    _close(out, ref)


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 64])
def test_gpu_mxfp4_bias_swiglu_precision_config(M):
    """triton_kernel_fused_experts_with_bias with MXFP4 weights passed as
    matmul_ogs-layout uint8 tensors plus precision configs holding the scales."""
    import flaggems_sglang
    from flaggems_sglang.ops import fused_moe as F

    K, N, E, k = 256, 384, 8, 2
    d, q13, s13, q2, s2 = _mx_case(M, K, N, E, k, seed=M + 11)
    gen = torch.Generator().manual_seed(M)
    b13 = torch.randn(E, 2 * N, generator=gen) * 0.1
    b2 = torch.randn(E, K, generator=gen) * 0.1
    tw, ti = d["topk_weights"].to(DEV), d["topk_ids"].to(DEV)
    rd, gi, si = F._standard_topk_to_triton_kernels(tw, ti, E)
    pcg1 = types.SimpleNamespace(weight_scale=s13.to(DEV).transpose(1, 2).contiguous())
    pcg2 = types.SimpleNamespace(weight_scale=s2.to(DEV).transpose(1, 2).contiguous())
    out = flaggems_sglang.triton_kernel_fused_experts_with_bias(
        d["x"].to(DEV), q13.to(DEV).transpose(1, 2).contiguous(), pcg1, b13.to(DEV),
        q2.to(DEV).transpose(1, 2).contiguous(), pcg2, b2.to(DEV), rd, gi, si,
        gemm1_alpha=1.702, gemm1_clamp_limit=7.0)
    w13d = O.mxfp4_dequant(q13, s13)
    w2d = O.mxfp4_dequant(q2, s2)
    ref = O.fused_experts_bias(d["x"], w13d, b13, w2d, b2, d["topk_weights"], d["topk_ids"],
                               alpha=1.702, limit=7.0)
    _close(out, ref)


@pytest.mark.gpu
def test_gpu_flagos_hook_mxfp4_layer_with_bias():
    from flaggems_sglang.ops.fused_moe import fused_moe_flagos

    M, K, N, E, k = 5, 256, 256, 4, 2
    d, q13, s13, q2, s2 = _mx_case(M, K, N, E, k, seed=3)
    gen = torch.Generator().manual_seed(9)
    b13 = torch.randn(E, 2 * N, generator=gen) * 0.1
    b2 = torch.randn(E, K, generator=gen) * 0.1
    layer = torch.nn.Module()
    for name, t in (("w13_weight", q13), ("w13_weight_scale", s13), ("w2_weight", q2),
                    ("w2_weight_scale", s2), ("w13_weight_bias", b13), ("w2_weight_bias", b2)):
        layer.register_parameter(name, torch.nn.Parameter(t.to(DEV), requires_grad=False))
    cfg = types.SimpleNamespace(num_experts=E, no_combine=False, activation="silu",
                                apply_router_weight_on_input=False, routed_scaling_factor=None,
                                gemm1_alpha=1.702, gemm1_clamp_limit=7.0)
    obj = types.SimpleNamespace(runner=types.SimpleNamespace(config=cfg))
    disp = types.SimpleNamespace(hidden_states=d["x"].to(DEV),
                                 topk_output=types.SimpleNamespace(topk_weights=d["topk_weights"].to(DEV),
                                                                   topk_ids=d["topk_ids"].to(DEV)))
    out = fused_moe_flagos(obj, layer, disp).hidden_states
    ref = O.fused_experts_bias(d["x"], O.mxfp4_dequant(q13, s13), b13, O.mxfp4_dequant(q2, s2), b2,
                               d["topk_weights"], d["topk_ids"], alpha=1.702, limit=7.0)
    _close(out, ref)
