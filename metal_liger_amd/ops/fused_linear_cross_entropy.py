"""Fused lm_head + cross-entropy on MI355X (drop-in for the reference's
ops/fused_linear_cross_entropy.py).

The [tokens, vocab] logits never exist. When gradients are needed, the
forward computes the loss and both gradients in one pass over token chunks,
with every logit computed once (three MFMA GEMMs in all):

* per chunk, the logits GEMM's epilogue reduces each 128-column slice to
  per-row (max, sum-exp) partials (the reference's online logsumexp,
  :39-55) and stores exp(z - max) in bf16; a row pass forms lse and the
  masked loss; an elementwise pass turns the stored values into dlogits =
  (softmax - one_hot) * mask / #valid; dH and dW come from MFMA GEMMs on
  them (:57-80, :159-185);
* the backward multiplies those gradients by grad_output.

The reference instead recomputes every logits chunk in its backward (four
GEMMs). ``chunk_size`` keeps its meaning for the vocabulary-chunked backward
that runs when the same graph is backpropagated a second time
(retain_graph): that path starts from the saved lse and recomputes.
Without gradients (no_grad, or nothing requires grad) only the loss is
computed. dW is skipped when the lm_head weight is frozen.

Semantics kept from the reference: labels are not shifted; ignore_index
tokens contribute nothing; the mean divides by max(#valid, 1) (all-ignored
batches give loss 0); the loss is fp32; no bias gradient is returned.
"""

import torch
import torch.nn as nn

from metal_liger_amd import hip_ops


class _FusedLinearCrossEntropyFunction(torch.autograd.Function):
    """Linear + cross-entropy that never materialises full logits
    (ops/fused_linear_cross_entropy.py:82-185)."""

    @staticmethod
    def forward(ctx, hidden: torch.Tensor, weight: torch.Tensor,
                labels: torch.Tensor, bias: torch.Tensor = None,
                ignore_index: int = -100, chunk_size: int = 8192):
        need_h, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        loss, lse, n_valid, dh, dw = hip_ops.flce_fwd_grad(
            hidden, weight, labels, bias, ignore_index, need_dhidden=need_h, need_dweight=need_w)
        ctx.save_for_backward(hidden, weight, labels, lse, n_valid, dh, dw)
        ctx.bias = bias
        ctx.ignore_index = ignore_index
        ctx.chunk_size = chunk_size
        ctx.grads_used = False
        return loss

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        hidden, weight, labels, lse, n_valid, dh, dw = ctx.saved_tensors
        need_h, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        if not ctx.grads_used:
            # gradients from the forward, scaled in place and handed over once
            ctx.grads_used = True
            grad_hidden = dh if need_h else None
            grad_weight = dw if need_w else None
            hip_ops.flce_scale_grads(grad_output, grad_hidden, grad_weight)
        else:
            # a second backward through the same graph: fresh tensors from the
            # vocabulary-chunked recomputation
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
        chunk_size: Vocab chunk of a repeated (retain_graph) backward (default: 8192)
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
