"""Fused SwiGLU on MI355X (drop-in for the reference's ops/fused_swiglu.py).

One streaming HIP kernel each way. Unlike the reference, which kept
sigmoid(gate) as an extra fp32 tensor for backward (ops/fused_swiglu.py:34),
sigmoid is recomputed in the backward kernel: it costs no HBM traffic there,
while the saved tensor cost 4 bytes per element of memory and traffic.
"""

import torch
import torch.nn as nn

from metal_liger_amd import _custom_ops as cops


class _FusedSwiGLUFunction(torch.autograd.Function):
    """silu(gate) * up, computed in fp32 and rounded to gate's dtype
    (ops/fused_swiglu.py:18-50); grads in gate's / up's dtype."""

    @staticmethod
    def forward(ctx, gate: torch.Tensor, up: torch.Tensor):
        output = cops.swiglu_fwd(gate, up)
        ctx.save_for_backward(gate, up)
        return output

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        gate, up = ctx.saved_tensors
        grad_gate, grad_up = cops.swiglu_bwd(gate, up, grad_output)
        return grad_gate, grad_up


def fused_swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """Functional: SiLU(gate) * up in a single fused op (ops/fused_swiglu.py:54-56)."""
    return _FusedSwiGLUFunction.apply(gate, up)


class MetalLigerSwiGLU(nn.Module):
    """Drop-in for a SwiGLU MLP block; fuses the activation step only
    (ops/fused_swiglu.py:59-75). Keeps gate_proj / up_proj / down_proj under
    their original names so state_dict keys are unchanged."""

    def __init__(self, original_mlp: nn.Module):
        super().__init__()
        self.gate_proj = original_mlp.gate_proj
        self.up_proj = original_mlp.up_proj
        self.down_proj = original_mlp.down_proj

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        gate = self.gate_proj(x)
        up = self.up_proj(x)
        activated = _FusedSwiGLUFunction.apply(gate, up)
        return self.down_proj(activated)

    def extra_repr(self) -> str:
        return "fused=MetalLiger-Phase3"
