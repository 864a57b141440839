"""CPU checks of the host mirror: the reference's argument contract
(ops/fused_moe.py:154-179, :206) is enforced before any device work."""

import pytest
import torch

import flaggems_sglang
from flaggems_sglang.ops import fused_moe as F


def _rd():
    z = torch.zeros(4, dtype=torch.int32)
    return F.RoutingData(torch.zeros(4), z, 8, 2), F.GatherIndx(z, z), F.ScatterIndx(z, z)


@pytest.mark.parametrize("kw,msg", [
    (dict(expert_map=torch.zeros(1)), "expert_map is not supported"),
    (dict(a1_scale=torch.zeros(1)), "a1_scale is not supported"),
    (dict(w1_scale=torch.zeros(1)), "w1_scale is not supported"),
    (dict(block_shape=[128, 128]), "block_shape is not supported"),
    (dict(per_channel_quant=True), "per_channel_quant is not supported"),
    (dict(inplace=True), "Inplace is not supported"),
])
def test_unsupported_features_assert(kw, msg):
    x = torch.zeros(2, 128, dtype=torch.bfloat16)
    w1 = torch.zeros(8, 128, 512, dtype=torch.bfloat16)
    w2 = torch.zeros(8, 256, 128, dtype=torch.bfloat16)
    with pytest.raises(AssertionError, match=msg):
        flaggems_sglang.triton_kernel_fused_experts(x, w1, w2, *_rd(), **kw)


def test_dtype_and_shape_asserts():
    x = torch.zeros(2, 128, dtype=torch.float32)
    w1 = torch.zeros(8, 128, 512, dtype=torch.bfloat16)
    w2 = torch.zeros(8, 256, 128, dtype=torch.bfloat16)
    with pytest.raises(AssertionError, match="hidden_states must be bfloat16"):
        flaggems_sglang.triton_kernel_fused_experts(x, w1, w2, *_rd())
    with pytest.raises(AssertionError, match="hidden size mismatch"):
        flaggems_sglang.triton_kernel_fused_experts(
            torch.zeros(2, 64, dtype=torch.bfloat16), w1, w2, *_rd())


def test_unknown_activation_raises_value_error():
    x = torch.zeros(2, 128, dtype=torch.bfloat16)
    w1 = torch.zeros(8, 128, 512, dtype=torch.bfloat16)
    w2 = torch.zeros(8, 256, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="Unsupported FusedMoe activation: gelu_tanh"):
        flaggems_sglang.triton_kernel_fused_experts(x, w1, w2, *_rd(), activation="gelu_tanh")


def test_cpu_tensors_are_rejected_not_computed():
    """No CPU fallback: host tensors raise instead of being computed in torch."""
    x = torch.zeros(2, 128, dtype=torch.bfloat16)
    w1 = torch.zeros(8, 512, 128, dtype=torch.bfloat16)
    w2 = torch.zeros(8, 128, 256, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        flaggems_sglang.fused_experts(x, w1, w2, torch.ones(2, 2), torch.zeros(2, 2, dtype=torch.int32))


def test_bias_path_argument_checks():
    """triton_kernel_fused_experts_with_bias (ops/fused_moe.py:219-309): the
    reference's asserts and its ValueError for other activations, raised
    before any device work (host tensors are enough)."""
    E, K, N, M = 4, 128, 128, 3
    x = torch.zeros(M, K, dtype=torch.bfloat16)
    w1 = torch.zeros(E, K, 2 * N, dtype=torch.bfloat16)
    w2 = torch.zeros(E, N, K, dtype=torch.bfloat16)
    b1 = torch.zeros(E, 2 * N)
    b2 = torch.zeros(E, K)
    rd = F.RoutingData(torch.ones(M * 2), torch.zeros(E, dtype=torch.int32), E, 2, None)
    f = flaggems_sglang.triton_kernel_fused_experts_with_bias
    with pytest.raises(AssertionError, match="Inplace is not supported"):
        f(x, w1, None, b1, w2, None, b2, rd, None, None, inplace=True)
    with pytest.raises(ValueError, match="Unsupported FusedMoe activation: gelu"):
        f(x, w1, None, b1, w2, None, b2, rd, None, None, activation="gelu")
    with pytest.raises(AssertionError, match="go together"):
        f(x, w1, object(), b1, w2, None, b2, rd, None, None)
    # precision configs must carry plain MXFP4 block scales
    with pytest.raises(AssertionError, match="w1_pcg without a plain weight_scale tensor is not supported"):
        f(x, w1, object(), b1, w2, object(), b2, rd, None, None)
    with pytest.raises(AssertionError, match="requires both"):
        f(x, w1, None, b1, w2, None, None, rd, None, None)
    with pytest.raises(ValueError, match="GPU"):
        f(x, w1, None, b1, w2, None, b2, rd, None, None)


def test_activation_names():
    """silu and gelu are accepted (ops/fused_moe.py:198-206); anything else is
    the reference's ValueError."""
    x = torch.zeros(2, 128, dtype=torch.bfloat16)
    w1 = torch.zeros(8, 512, 128, dtype=torch.bfloat16)
    w2 = torch.zeros(8, 128, 256, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="Unsupported FusedMoe activation: relu"):
        flaggems_sglang.fused_experts(x, w1, w2, torch.ones(2, 2), torch.zeros(2, 2, dtype=torch.int32),
                                      activation="relu")
    with pytest.raises(ValueError, match="GPU"):
        flaggems_sglang.fused_experts(x, w1, w2, torch.ones(2, 2), torch.zeros(2, 2, dtype=torch.int32),
                                      activation="gelu")
