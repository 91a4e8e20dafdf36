"""Fused ops (drop-in for the reference's ops/ package, ops/__init__.py:2-5)."""
from metal_liger_amd.ops.fused_rms_norm import MetalLigerRMSNorm  # noqa: F401
from metal_liger_amd.ops.fused_swiglu import MetalLigerSwiGLU  # noqa: F401
from metal_liger_amd.ops.fused_rope import MetalLigerRoPE  # noqa: F401
from metal_liger_amd.ops.fused_linear_cross_entropy import MetalLigerFusedLinearCrossEntropy  # noqa: F401
