from flaggems_sglang.ops.fused_moe import (  # noqa: F401
    fused_experts,
    fused_moe_flagos,
    triton_kernel_fused_experts,
    triton_kernel_fused_experts_with_bias,
)

__all__ = [
    "fused_experts",
    "fused_moe_flagos",
    "triton_kernel_fused_experts",
    "triton_kernel_fused_experts_with_bias",
]
