"""flaggems_sglang for MI355X: FlagGems-sglang's fused-MoE path on gfx950 HIP kernels.

Keeps the reference's package name and fused-MoE entry points
(``src/flaggems_sglang/__init__.py:7-10``): ``triton_kernel_fused_experts``,
``triton_kernel_fused_experts_with_bias`` and, in ``ops.fused_moe``, the SGLang
hook ``fused_moe_flagos``.  The compute runs in ``libfmoe.so`` (C ABI in
``include/fmoe.h``), loaded on first use; a missing library raises.
"""

from flaggems_sglang.ops.fused_moe import (  # noqa: F401
    fused_experts,
    fused_moe_flagos,
    grouped_topk,
    moe_align_block_size,
    per_token_group_quant_fp8,
    topk_softmax,
    triton_kernel_fused_experts,
    triton_kernel_fused_experts_with_bias,
)
from flaggems_sglang import formats, quant  # noqa: F401

device = "cuda"  # torch's device string for HIP devices on ROCm
vendor_name = "amd"

__version__ = "0.1.0"
