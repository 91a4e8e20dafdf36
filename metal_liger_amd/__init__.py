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

__all__ = [
    "MetalLigerRMSNorm",
    "MetalLigerSwiGLU",
    "MetalLigerRoPE",
]
