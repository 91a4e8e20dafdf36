"""Fused lm_head + cross-entropy on MI355X (drop-in for the reference's
ops/fused_linear_cross_entropy.py).

The [tokens, vocab] logits never exist, in the forward or the backward:

* forward: one bf16 MFMA GEMM over the whole vocabulary whose epilogue keeps
  each logits tile in registers and reduces it to per-row (max, sum-exp)
  partials (an online logsumexp across tiles); a row pass merges them into
  lse and the masked mean loss. Same result as the reference's chunked
  online-softmax loop (:39-55, :93-157).
* backward, per vocabulary chunk of ``chunk_size`` columns: the logits tile
  is recomputed and its epilogue writes dlogits = (softmax - one_hot) * mask *
  grad / #valid in bf16; dH and dW come from MFMA GEMMs on that chunk
  (:57-80, :159-185). dW is skipped when the lm_head weight is frozen.

Semantics kept from the reference: labels are not shifted; ignore_index
tokens contribute nothing; the mean divides by max(#valid, 1) (all-ignored
batches give loss 0); the loss is fp32; no bias gradient is returned.
"""

import torch
import torch.nn as nn

from metal_liger_amd import hip_ops


class _FusedLinearCrossEntropyFunction(torch.autograd.Function):
    """Chunked linear + cross-entropy that never materialises full logits
    (ops/fused_linear_cross_entropy.py:82-185)."""

    @staticmethod
    def forward(ctx, hidden: torch.Tensor, weight: torch.Tensor,
                labels: torch.Tensor, bias: torch.Tensor = None,
                ignore_index: int = -100, chunk_size: int = 8192):
        loss, lse, n_valid = hip_ops.flce_fwd(hidden, weight, labels, bias, ignore_index)
        ctx.save_for_backward(hidden, weight, labels, lse, n_valid)
        ctx.bias = bias
        ctx.ignore_index = ignore_index
        ctx.chunk_size = chunk_size
        return loss

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        hidden, weight, labels, lse, n_valid = ctx.saved_tensors
        need_h, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        grad_hidden, grad_weight = hip_ops.flce_bwd(
            hidden, weight, labels, ctx.bias, ctx.ignore_index, lse, n_valid, grad_output,
            ctx.chunk_size, need_dhidden=need_h, need_dweight=need_w)
        if grad_hidden is not None and grad_hidden.dtype != hidden.dtype:
            grad_hidden = grad_hidden.to(hidden.dtype)
        if grad_weight is not None and grad_weight.dtype != weight.dtype:
            grad_weight = grad_weight.to(weight.dtype)
        return grad_hidden, grad_weight, None, None, None, None


class MetalLigerFusedLinearCrossEntropy(nn.Module):
    """Fused lm_head + cross-entropy loss (ops/fused_linear_cross_entropy.py:188-230).

    Args:
        lm_head: The language model head linear layer
        ignore_index: Label ID to ignore (default: -100)
        chunk_size: Vocab chunk held at once in the backward (default: 8192)
    """

    def __init__(self, lm_head: nn.Linear, ignore_index: int = -100,
                 chunk_size: int = 8192):
        super().__init__()
        self.weight = lm_head.weight
        self.bias = lm_head.bias
        self.ignore_index = ignore_index
        self.chunk_size = chunk_size

    def forward(self, hidden_states: torch.Tensor,
                labels: torch.Tensor) -> torch.Tensor:
        batch_seq = (hidden_states.shape[0] * hidden_states.shape[1]
                     if hidden_states.ndim == 3 else hidden_states.shape[0])
        hidden_flat = hidden_states.reshape(batch_seq, -1)
        labels_flat = labels.reshape(-1)
        return _FusedLinearCrossEntropyFunction.apply(
            hidden_flat, self.weight, labels_flat,
            self.bias, self.ignore_index, self.chunk_size
        )
