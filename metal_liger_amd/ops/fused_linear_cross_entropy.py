"""Fused lm_head + cross-entropy on MI355X (drop-in for the reference's
ops/fused_linear_cross_entropy.py).

The [tokens, vocab] logits never exist. When gradients are needed, the
forward computes the loss and both gradients in one pass over token chunks,
with every logit computed once (three MFMA GEMMs in all):

* per chunk of 2048 tokens, each row gets a shift (its label logit + 30)
  before the logits GEMM, whose epilogue stores exp(z - shift) in bf16 and
  reduces each 64-column slice to per-row partials; a row pass forms lse
  (the reference's logsumexp, :39-55), the masked loss and a row factor
  such that dlogits = (softmax - one_hot) * mask / #valid = row factor x
  the stored values (label entry rewritten); dH and dW come from MFMA GEMMs
  on them with the row factor folded in (:57-80, :159-185). Rows whose
  stored values would leave a safe range (a token loss above ~78 nats) are
  recomputed with their exact max;
* the backward multiplies those gradients by grad_output.

The reference instead recomputes every logits chunk in its backward (four
GEMMs). ``chunk_size`` keeps its meaning for the vocabulary-chunked backward
that runs when the same graph is backpropagated a second time
(retain_graph): that path starts from the saved lse and recomputes.
The module and the causal-LM loss compute the loss alone (one logits GEMM,
no gradient buffers) when grad mode is off (``torch.no_grad()``,
``torch.inference_mode()``), whatever requires grad; inside the
autograd.Function, which cannot see grad mode, gradients are formed for the
inputs that require them. dW is skipped when the lm_head weight is frozen.

Semantics kept from the reference: labels are not shifted; ignore_index
tokens contribute nothing; the mean divides by max(#valid, 1) (all-ignored
batches give loss 0); the loss is fp32; no bias gradient is returned.
fp32 inputs run the reference's own vocabulary-chunked schedule on fp32
matrix-core GEMMs (logits tile [tokens, chunk_size] fp32); other float
dtypes are upcast to fp32 first, as the reference upcasts, and their
gradients cast back.

``patch_causal_lm_loss(model)`` (``apply_metal_liger_to_qwen3vl(...,
fuse_lm_loss=True)``) goes one step further than the reference, whose
patcher only logs for ``fuse_cross_entropy`` (patch.py:230-232): a
causal LM called with ``labels`` while training gets its loss from the fused
op, with transformers' label shift and ``num_items_in_batch`` handling, and
never forms the logits.
"""

import contextvars
import inspect

import torch
import torch.nn as nn
import torch.nn.functional as F

from metal_liger_amd import _custom_ops as cops
from metal_liger_amd._model_walk import shadowed


def _compute_dtype(hidden, weight, bias):
    """hidden, weight (and bias) in the dtype the kernels compute in: bf16
    stays bf16; fp32 stays fp32; any other float dtype (or a mix) is upcast
    to fp32, as the reference upcasts both (:108-109)."""
    if hidden.dtype == weight.dtype and hidden.dtype in (torch.bfloat16, torch.float32):
        return hidden, weight, bias
    return hidden.float(), weight.float(), bias.float() if bias is not None else None


class _FusedLinearCrossEntropyFunction(torch.autograd.Function):
    """Linear + cross-entropy that never materialises full logits
    (ops/fused_linear_cross_entropy.py:82-185)."""

    @staticmethod
    def forward(ctx, hidden: torch.Tensor, weight: torch.Tensor,
                labels: torch.Tensor, bias: torch.Tensor = None,
                ignore_index: int = -100, chunk_size: int = 8192):
        need_h, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        hidden_c, weight_c, bias_c = _compute_dtype(hidden, weight, bias)
        loss, lse, n_valid, dh, dw = cops.flce_fwd_grad(
            hidden_c, weight_c, labels, bias_c, ignore_index, need_h, need_w, chunk_size)
        ctx.save_for_backward(hidden, weight, labels, lse, n_valid)
        # The gradients are handed over (scaled in place) by the first
        # backward, so they are kept out of the saved tensors, whose versions
        # a later backward through the same graph checks.
        ctx.grads = (cops.maybe(dh), cops.maybe(dw))
        ctx.bias = bias
        ctx.ignore_index = ignore_index
        ctx.chunk_size = chunk_size
        return loss

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        hidden, weight, labels, lse, n_valid = ctx.saved_tensors
        need_h, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        if ctx.grads is not None:
            # gradients from the forward, scaled in place and handed over once
            dh, dw = ctx.grads
            ctx.grads = None
            grad_hidden = dh if need_h else None
            grad_weight = dw if need_w else None
            cops.flce_scale_grads(grad_output, grad_hidden, grad_weight)
        else:
            # a second backward through the same graph: fresh tensors from the
            # vocabulary-chunked recomputation
            hidden_c, weight_c, bias_c = _compute_dtype(hidden, weight, ctx.bias)
            grad_hidden, grad_weight = cops.flce_bwd(
                hidden_c, weight_c, labels, bias_c, ctx.ignore_index, lse, n_valid, grad_output,
                ctx.chunk_size, need_h, need_w)
            grad_hidden, grad_weight = cops.maybe(grad_hidden), cops.maybe(grad_weight)
        if grad_hidden is not None and grad_hidden.dtype != hidden.dtype:
            grad_hidden = grad_hidden.to(hidden.dtype)
        if grad_weight is not None and grad_weight.dtype != weight.dtype:
            grad_weight = grad_weight.to(weight.dtype)
        return grad_hidden, grad_weight, None, None, None, None


def _fused_loss(hidden, weight, labels, bias, ignore_index, chunk_size):
    """The fused loss through the autograd Function, or, with grad mode off
    (where no graph is recorded and no backward can follow), by the
    loss-only path: the Function's forward cannot tell grad mode (autograd
    runs it with grad disabled) and would form the gradients of every input
    that requires grad."""
    if torch.is_grad_enabled():
        return _FusedLinearCrossEntropyFunction.apply(hidden, weight, labels, bias, ignore_index,
                                                      chunk_size)
    hidden_c, weight_c, bias_c = _compute_dtype(hidden, weight, bias)
    return cops.flce_fwd(hidden_c, weight_c, labels, bias_c, ignore_index, chunk_size)[0]


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
        hidden_flat = hidden_states.reshape(batch_seq, hidden_states.shape[-1])
        labels_flat = labels.reshape(-1)
        return _fused_loss(hidden_flat, self.weight, labels_flat, self.bias, self.ignore_index,
                           self.chunk_size)


# ------------------------------------------------------ causal-LM loss hook --

_LOSS_STATE: contextvars.ContextVar = contextvars.ContextVar("metal_liger_flce_loss", default=None)


def _identity(x):
    return x


def causal_lm_loss(hidden_states: torch.Tensor, lm_head: nn.Linear, labels: torch.Tensor,
                   num_items_in_batch=None, ignore_index: int = -100,
                   shift_labels: torch.Tensor = None, chunk_size: int = 8192) -> torch.Tensor:
    """transformers' ForCausalLMLoss over lm_head(hidden_states) without the
    logits: labels shifted left (the last position ignored) unless
    shift_labels is given; mean over the valid tokens, or their sum divided
    by num_items_in_batch when that is given. All-ignored batches give 0 (the
    reference's clamp) where torch's mean would give NaN."""
    if shift_labels is None:
        labels = F.pad(labels, (0, 1), value=ignore_index)
        shift_labels = labels[..., 1:]
    h = hidden_states.reshape(-1, hidden_states.shape[-1])
    y = shift_labels.reshape(-1).to(h.device)
    if y.shape[0] != h.shape[0]:
        raise ValueError(f"fused causal-LM loss: {y.shape[0]} labels for {h.shape[0]} positions")
    loss = _fused_loss(h, lm_head.weight, y, lm_head.bias, ignore_index, chunk_size)
    if num_items_in_batch is not None:
        n_valid = (y != ignore_index).sum().to(loss.dtype)
        if torch.is_tensor(num_items_in_batch):
            num_items_in_batch = num_items_in_batch.to(loss.device)
        loss = loss * n_valid / num_items_in_batch
    return loss


def _eligible_lm(mod: nn.Module) -> bool:
    head = getattr(mod, "lm_head", None)
    cfg = getattr(mod, "config", None)
    return (isinstance(head, nn.Linear) and hasattr(mod, "loss_function") and
            getattr(cfg, "final_logit_softcapping", None) is None)


def _make_lm_forward(lm: nn.Module, orig_fwd, chunk_size: int):
    try:
        sig = inspect.signature(orig_fwd)
    except (TypeError, ValueError):
        sig = None

    def labels_of(args, kwargs):
        if "labels" in kwargs or sig is None:
            return kwargs.get("labels")
        try:
            return sig.bind_partial(*args, **kwargs).arguments.get("labels")
        except TypeError:
            return None

    def forward(*args, **kwargs):
        if not lm.training or labels_of(args, kwargs) is None:
            return orig_fwd(*args, **kwargs)
        head = lm.lm_head
        state = {"used": False}

        def loss_fn(logits, labels, vocab_size=None, **kw):
            # logits are the final hidden states here (lm_head is shadowed)
            state["used"] = True
            return causal_lm_loss(logits, head, labels, kw.get("num_items_in_batch"),
                                  kw.get("ignore_index", -100), kw.get("shift_labels"), chunk_size)

        token = _LOSS_STATE.set(state)
        try:
            with shadowed(lm, lm_head=_identity, _loss_function=loss_fn):
                out = orig_fwd(*args, **kwargs)
        finally:
            _LOSS_STATE.reset(token)
        if not state["used"]:
            raise RuntimeError(f"fused causal-LM loss: {type(lm).__name__}.forward did not call "
                               "loss_function with the labels")
        if hasattr(out, "logits"):
            out.logits = None  # the field held the hidden states
        return out

    return forward


def patch_causal_lm_loss(model: nn.Module, chunk_size: int = 8192) -> int:
    """Routes the training loss of every causal LM in `model` (a module with
    an nn.Linear ``lm_head``, transformers' ``loss_function`` and no final
    logit soft-capping) through the fused linear cross-entropy: in training
    mode with ``labels``, its forward returns the loss with ``logits=None``;
    otherwise it is unchanged. Modules are not replaced. Returns the number
    of patched modules."""
    count = 0
    for mod in model.modules():
        if getattr(mod, "_metal_liger_flce_loss", False) or not _eligible_lm(mod):
            continue
        mod.forward = _make_lm_forward(mod, mod.forward, chunk_size)
        mod._metal_liger_flce_loss = True
        count += 1
    return count
