"""Fused rotate-half RoPE on MI355X (drop-in for the reference's ops/fused_rope.py).

Two entry styles:

* table mode, the reference's signature: ``_FusedRoPEFunction.apply(x, cos,
  sin)`` and ``apply_fused_rotary(q, k, cos, sin)``. cos/sin are broadcast
  in-kernel (stride-0 dims), never materialised; q and k go through one launch.
* position mode, what the reference's docstring promises
  (``FusedRoPE(q, positions, theta)``, ops/fused_rope.py:10-13):
  ``apply_fused_rotary_inline(q, k, position_ids, theta)`` computes cos/sin in
  the kernel from the positions and the fp32 inverse frequencies, so no table
  is built or read.

The backward is the reference's: the same rotation with -sin
(ops/fused_rope.py:48-57), which is the exact VJP when cos/sin have
duplicated halves (HF's layout).
"""

import torch
import torch.nn as nn

from metal_liger_amd import _custom_ops as cops
from metal_liger_amd import hip_ops


class _FusedRoPEFunction(torch.autograd.Function):
    """x * cos + rotate_half(x) * sin for one tensor (ops/fused_rope.py:22-57)."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
        output, _ = cops.rope_table(x, None, cos, sin, 1.0)
        ctx.save_for_backward(cos, sin)
        ctx.x_dtype = x.dtype
        return output

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        cos, sin = ctx.saved_tensors
        grad_x, _ = cops.rope_table(grad_output, None, cos, sin, -1.0)
        return grad_x, None, None


class _FusedRoPEQKFunction(torch.autograd.Function):
    """q and k rotated by the same tables in one launch each way."""

    @staticmethod
    def forward(ctx, q, k, cos, sin):
        q_out, k_out = cops.rope_table(q, k, cos, sin, 1.0)
        ctx.save_for_backward(cos, sin)
        return q_out, k_out

    @staticmethod
    def backward(ctx, dq, dk):
        cos, sin = ctx.saved_tensors
        if dq is None and dk is None:
            return None, None, None, None
        if dq is None:
            return None, cops.rope_table(dk, None, cos, sin, -1.0)[0], None, None
        if dk is None:
            return cops.rope_table(dq, None, cos, sin, -1.0)[0], None, None, None
        gq, gk = cops.rope_table(dq, dk, cos, sin, -1.0)
        return gq, gk, None, None


class _FusedRoPEPositionsFunction(torch.autograd.Function):
    """q and k rotated with cos/sin computed in-kernel from positions."""

    @staticmethod
    def forward(ctx, q, k, positions, inv_freq):
        q_out, k_out = cops.rope_pos(q, k, positions, inv_freq, 1.0)
        ctx.save_for_backward(positions, inv_freq)
        ctx.has_k = k is not None
        return q_out, cops.maybe(k_out)

    @staticmethod
    def backward(ctx, dq, dk):
        positions, inv_freq = ctx.saved_tensors
        if dq is None and dk is None:
            return None, None, None, None
        if dq is None:
            return None, cops.rope_pos(dk, None, positions, inv_freq, -1.0)[0], None, None
        if dk is None:
            return cops.rope_pos(dq, None, positions, inv_freq, -1.0)[0], None, None, None
        gq, gk = cops.rope_pos(dq, dk, positions, inv_freq, -1.0)
        return gq, gk, None, None


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    """Rotate half of the hidden dims: [x1, x2] -> [-x2, x1] (ops/fused_rope.py:60-64).

    Plain torch, kept for API compatibility (the reference's tests import it);
    the fused path never calls it.
    """
    x1 = x[..., : x.shape[-1] // 2]
    x2 = x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def _apply_rotary_fused(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x * cos + rotate_half(x) * sin in one HIP launch (ops/fused_rope.py:67-75)."""
    return cops.rope_table(x, None, cos, sin, 1.0)[0]


class MetalLigerRoPE(nn.Module):
    """Pass-through wrapper around a HF rotary module (ops/fused_rope.py:78-107):
    returns the wrapped module's (cos, sin); rotation happens in attention."""

    def __init__(self, original_rope: nn.Module):
        super().__init__()
        self._original = original_rope
        if hasattr(original_rope, 'dim'):
            self.dim = original_rope.dim
        if hasattr(original_rope, 'max_position_embeddings'):
            self.max_position_embeddings = original_rope.max_position_embeddings
        if hasattr(original_rope, 'base'):
            self.base = original_rope.base
        if hasattr(original_rope, 'inv_freq'):
            self.register_buffer('inv_freq', original_rope.inv_freq, persistent=False)

    def forward(self, x, position_ids=None, **kwargs):
        result = self._original(x, position_ids=position_ids, **kwargs)
        if isinstance(result, tuple) and len(result) == 2:
            cos, sin = result
            return cos, sin
        return result


def apply_fused_rotary(q: torch.Tensor, k: torch.Tensor,
                       cos: torch.Tensor, sin: torch.Tensor):
    """Rotates q and k with the given cos/sin tables (ops/fused_rope.py:110-127).

    Same results as applying _FusedRoPEFunction to q and to k; one launch for
    both in each direction.
    """
    return _FusedRoPEQKFunction.apply(q, k, cos, sin)


def apply_fused_rotary_inline(q: torch.Tensor, k: torch.Tensor, position_ids: torch.Tensor,
                              theta: float = 10000.0, inv_freq: torch.Tensor = None):
    """Rotates q, k ([batch, heads, seq, head_dim]) with cos/sin computed in-kernel.

    angle = float(position) * inv_freq[i], inv_freq = 1 / theta^(2i/D) in fp32
    (the HF rotary module's default rope, which duplicates the angle across
    the two halves). Pass ``inv_freq`` (e.g. the rotary module's buffer) to
    use other frequencies; ``theta`` is then ignored.
    """
    if inv_freq is None:
        inv_freq = hip_ops.rope_inv_freq(q.shape[-1], theta, q.device)
    return _FusedRoPEPositionsFunction.apply(q, k, position_ids, inv_freq)


def fused_rope(x: torch.Tensor, position_ids: torch.Tensor, theta: float = 10000.0,
               inv_freq: torch.Tensor = None) -> torch.Tensor:
    """Single-tensor form of apply_fused_rotary_inline."""
    if inv_freq is None:
        inv_freq = hip_ops.rope_inv_freq(x.shape[-1], theta, x.device)
    return _FusedRoPEPositionsFunction.apply(x, None, position_ids, inv_freq)[0]
