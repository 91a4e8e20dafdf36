"""Residual add fused into the RMSNorm that follows it.

In a Qwen3 decoder layer (transformers' modeling_qwen3.py,
Qwen3DecoderLayer.forward; Qwen3-VL's text layer is the same) the attention
output, after o_proj (the reference's unimplemented "LoRA_W",
ops/fused_lora.py:26), is added to the residual stream and the sum goes
through post_attention_layernorm:

    hidden = residual + attn_out
    residual = hidden
    hidden = post_attention_layernorm(hidden)

``_FusedAddRMSNormFunction`` does both in one HIP pass (x and the residual
read once, the sum and the normalised sum written once) and its backward
adds the gradient the sum gets from the residual branch into the norm's dx
in the same pass. The sum is rounded to the input dtype exactly as torch's
add rounds it, and the norm is MetalLigerRMSNorm's, so the forward is
bit-identical to the unfused pair; the backward rounds once where autograd
rounds the norm's dx and the sum of the two gradients separately.

``patch_residual_add_norm(model)`` swaps the forward of each decoder layer
whose forward has exactly that structure (checked on its bytecode: the four
submodules in order and two additions) and whose post_attention_layernorm is
a MetalLigerRMSNorm (so the numerics are the reference's fused norm's).
Modules and state_dict keys are unchanged.
"""

from __future__ import annotations

import dis
import inspect
import logging

import torch
import torch.nn as nn

from metal_liger_amd import _custom_ops as cops
from metal_liger_amd.ops.fused_rms_norm import MetalLigerRMSNorm

logger = logging.getLogger(__name__)


class _FusedAddRMSNormFunction(torch.autograd.Function):
    """(x, residual) -> (norm(x + residual), x + residual)."""

    @staticmethod
    def forward(ctx, x, residual, weight, eps: float):
        y, total, rrms = cops.rms_norm_add_fwd(x, residual, weight, eps)
        ctx.save_for_backward(total, weight, rrms)
        ctx.eps = eps
        return y, total

    @staticmethod
    def backward(ctx, dy, dtotal):
        total, weight, rrms = ctx.saved_tensors
        if dy is None:
            dy = torch.zeros_like(total)
        if dtotal is None:
            dtotal = torch.zeros_like(total)
        dx, dw = cops.rms_norm_add_bwd(total, weight, dy, dtotal, rrms, ctx.eps)
        return (dx if ctx.needs_input_grad[0] else None, dx if ctx.needs_input_grad[1] else None,
                dw if ctx.needs_input_grad[2] else None, None)


def fused_add_rms_norm(x: torch.Tensor, residual: torch.Tensor, norm: nn.Module):
    """Returns (norm(x + residual), x + residual) from one fused launch.

    norm: an RMSNorm module over the last dim (``weight``, ``eps`` or
    ``variance_epsilon``); x and residual share shape and dtype.
    """
    eps = float(getattr(norm, "eps", getattr(norm, "variance_epsilon", 1e-6)))
    return _FusedAddRMSNormFunction.apply(x, residual, norm.weight, eps)


# ------------------------------------------------------------------ patching --

_LAYER_PARTS = ("input_layernorm", "self_attn", "post_attention_layernorm", "mlp")


_CONTAINER_OPS = ("BUILD_TUPLE", "BUILD_LIST", "LIST_APPEND", "LIST_EXTEND", "LIST_TO_TUPLE")


def _structure(fn) -> tuple:
    """(attribute loads of the layer parts in order, number of additions
    (in-place ones included), whether every return hands back one local
    variable and no tuple or list is built) of a forward's bytecode. The
    fused forward returns one tensor, so a layer that returns an outputs
    tuple (older transformers: ``outputs = (hidden_states,)`` with attention
    weights appended by ``+=``) does not match."""
    parts, adds, single = [], 0, True
    prev = None
    for ins in dis.get_instructions(fn):
        if ins.opname in ("LOAD_ATTR", "LOAD_METHOD") and ins.argval in _LAYER_PARTS:
            parts.append(ins.argval)
        elif ins.opname in ("BINARY_ADD", "INPLACE_ADD") or (
                ins.opname == "BINARY_OP" and ins.argrepr in ("+", "+=")):
            adds += 1
        elif ins.opname in _CONTAINER_OPS:
            single = False
        elif ins.opname == "RETURN_VALUE" and (prev is None or prev.opname != "LOAD_FAST"):
            single = False
        prev = ins
    return tuple(parts), adds, single


def _eligible(layer: nn.Module) -> bool:
    if not all(hasattr(layer, p) for p in _LAYER_PARTS):
        return False
    if not isinstance(layer.post_attention_layernorm, MetalLigerRMSNorm):
        return False
    fwd = getattr(type(layer).forward, "__func__", type(layer).forward)
    try:
        params = inspect.signature(fwd).parameters
    except (TypeError, ValueError):
        return False
    return "hidden_states" in params and _structure(fwd) == (_LAYER_PARTS, 2, True)


def _make_forward(layer: nn.Module, orig_fwd):
    """The decoder layer's forward with the post-attention add + norm fused.
    Every argument but hidden_states goes to self_attn, as the replaced
    forward passes them."""
    sig = inspect.signature(orig_fwd)
    var_kw = next((p.name for p in sig.parameters.values() if p.kind is p.VAR_KEYWORD), None)

    def forward(*args, **kwargs):
        bound = sig.bind(*args, **kwargs)
        bound.apply_defaults()
        attn_kwargs = dict(bound.arguments)
        extra = attn_kwargs.pop(var_kw, {}) if var_kw else {}
        residual = attn_kwargs.pop("hidden_states")
        hidden = layer.input_layernorm(residual)
        hidden, _ = layer.self_attn(hidden_states=hidden, **attn_kwargs, **extra)
        if hidden.shape == residual.shape and hidden.dtype == residual.dtype:
            hidden, residual = fused_add_rms_norm(hidden, residual, layer.post_attention_layernorm)
        else:  # promotion or broadcasting: the unfused pair
            residual = residual + hidden
            hidden = layer.post_attention_layernorm(residual)
        hidden = layer.mlp(hidden)
        return residual + hidden

    return forward


def patch_residual_add_norm(model: nn.Module) -> int:
    """Fuses the post-attention residual add into post_attention_layernorm in
    every eligible decoder layer (see the module docstring). Returns the
    number of patched layers."""
    count = 0
    for mod in model.modules():
        if getattr(mod, "_metal_liger_add_norm", False) or not _eligible(mod):
            continue
        mod.forward = _make_forward(mod, mod.forward)
        mod._metal_liger_add_norm = True
        count += 1
    logger.info(f"MetalLiger residual add + RMSNorm: activated on {count} decoder layers.")
    return count
