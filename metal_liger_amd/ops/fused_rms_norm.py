"""Fused RMSNorm on MI355X (drop-in for the reference's ops/fused_rms_norm.py).

Forward and backward are one HIP launch each (plus a small fixed-order dW
reduction): x is read once and y written once in the forward; x and dy are
read once and dx written once in the backward. Only x, weight and the fp32
per-row rrms are saved for backward, as in the reference
(ops/fused_rms_norm.py:38-40).
"""

import torch
import torch.nn as nn

from metal_liger_amd import _custom_ops as cops


class _FusedRMSNormFunction(torch.autograd.Function):
    """y = (x * rrms) * w, rrms = rsqrt(mean(x^2) + eps); closed-form VJP.

    Mirrors ops/fused_rms_norm.py:22-60: same saved tensors (x, weight,
    rrms[..., 1] fp32), same outputs and dtypes (y and dx in x's dtype, dw in
    weight's dtype, None for eps).
    """

    @staticmethod
    def forward(ctx, x: torch.Tensor, weight: torch.Tensor, eps: float):
        output, rrms = cops.rms_norm_fwd(x, weight, eps)
        ctx.save_for_backward(x, weight, rrms.unsqueeze(-1))
        ctx.eps = eps
        return output

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        x, weight, rrms = ctx.saved_tensors
        grad_x, grad_weight = cops.rms_norm_bwd(x, weight, grad_output, rrms, ctx.eps)
        return grad_x, grad_weight, None


class MetalLigerRMSNorm(nn.Module):
    """Drop-in replacement for nn.RMSNorm / HF RMSNorm (ops/fused_rms_norm.py:63-82).

    ``weight`` wraps the given tensor (sharing its storage) so state_dict keys
    and tied storage are unchanged by patching.
    """

    def __init__(self, hidden_size: int, eps: float = 1e-6, weight: torch.Tensor = None):
        super().__init__()
        self.eps = eps
        self.hidden_size = hidden_size
        if weight is not None:
            self.weight = nn.Parameter(weight)
        else:
            self.weight = nn.Parameter(torch.ones(hidden_size))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return _FusedRMSNormFunction.apply(x, self.weight, self.eps)

    def extra_repr(self) -> str:
        return f"hidden_size={self.hidden_size}, eps={self.eps}, fused=MetalLiger-Phase3"
