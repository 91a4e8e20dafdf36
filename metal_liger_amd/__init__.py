"""metal_liger_amd — MetalLiger's fused-op training hot path, MI355X-native.

Same public API as the reference package (__init__.py:24-59 of
krrish-v/metal_liger); every fused op runs hand-written HIP kernels for
gfx950 from libmetal_liger_amd.so (C ABI in include/metal_liger_amd.h).

    from metal_liger_amd import apply_metal_liger_to_qwen3vl
    model = apply_metal_liger_to_qwen3vl(model)
"""

__version__ = "0.3.0"

from metal_liger_amd.ops.fused_rms_norm import MetalLigerRMSNorm  # noqa: E402
from metal_liger_amd.ops.fused_swiglu import MetalLigerSwiGLU  # noqa: E402
from metal_liger_amd.ops.fused_rope import MetalLigerRoPE  # noqa: E402
from metal_liger_amd.ops.fused_linear_cross_entropy import MetalLigerFusedLinearCrossEntropy  # noqa: E402
from metal_liger_amd.ops.fused_lora import (  # noqa: E402
    apply_fused_lora_mlp,
    apply_fused_lora_qkv,
    patch_fused_lora,
)
from metal_liger_amd.patch import apply_metal_liger_to_qwen3vl  # noqa: E402
from metal_liger_amd._compile import apply_compile  # noqa: E402
from metal_liger_amd._torch_library import register_metal_liger_ops  # noqa: E402

register_metal_liger_ops()

__all__ = [
    "MetalLigerRMSNorm",
    "MetalLigerSwiGLU",
    "MetalLigerRoPE",
    "MetalLigerFusedLinearCrossEntropy",
    "apply_metal_liger_to_qwen3vl",
    "apply_fused_lora_qkv",
    "apply_fused_lora_mlp",
    "patch_fused_lora",
    "apply_compile",
    "register_metal_liger_ops",
]
