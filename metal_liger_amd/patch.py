"""Model patcher: swaps a HuggingFace Qwen3 / Qwen3-VL model's RMSNorms, SwiGLU
MLPs and (with LoRA) attention / MLP projections onto the fused ops.

Same entry point and behaviour as the reference's patch.py:181-240
(``apply_metal_liger_to_qwen3vl``): decoder layers and the final norm are
located through the same wrapping layouts (bare HF, PEFT, Qwen3-VL's nested
language_model, accelerate), RMSNorm modules are replaced by
MetalLigerRMSNorm sharing the original weight storage (state_dict keys
unchanged), MLPs by MetalLigerSwiGLU, and LoRA projections are routed through
the fused LoRA functions without replacing modules.
"""

import logging

import torch.nn as nn

from metal_liger_amd._model_walk import find_final_norm, find_layers
from metal_liger_amd.ops.fused_add_rms_norm import patch_residual_add_norm
from metal_liger_amd.ops.fused_linear_cross_entropy import patch_causal_lm_loss
from metal_liger_amd.ops.fused_lora import patch_fused_lora
from metal_liger_amd.ops.fused_qk_norm_rope import patch_qk_norm_rope
from metal_liger_amd.ops.fused_rms_norm import MetalLigerRMSNorm
from metal_liger_amd.ops.fused_swiglu import MetalLigerSwiGLU
from metal_liger_amd.ops.gqa_attention import patch_efficient_attention

logger = logging.getLogger(__name__)

# The decoder layers and the final norm are found along the wrapping layouts
# the reference's patch.py:27-89 walks (bare HF, PEFT, Qwen3-VL's nested
# language_model, accelerate); the path tables live in _model_walk.
_find_layers = find_layers
_find_final_norm = find_final_norm


def _fused_norm_like(old: nn.Module) -> MetalLigerRMSNorm:
    eps = getattr(old, "variance_epsilon", getattr(old, "eps", 1e-6))
    return MetalLigerRMSNorm(hidden_size=old.weight.shape[0], eps=eps, weight=old.weight.data)


def _replace_rms_norms(model: nn.Module) -> int:
    """Replaces each layer's input / post-attention norm and the final norm;
    returns the number replaced (patch.py:92-159)."""
    layers = _find_layers(model)
    if layers is None:
        logger.warning("MetalLiger: could not find transformer layers for RMSNorm patching")
        return 0
    count = 0
    for layer in layers:
        for name in ("input_layernorm", "post_attention_layernorm"):
            if hasattr(layer, name):
                setattr(layer, name, _fused_norm_like(getattr(layer, name)))
                count += 1
    old, parent = _find_final_norm(model)
    if old is not None:
        parent.norm = _fused_norm_like(old)
        count += 1
    return count


def _replace_mlps(model: nn.Module) -> int:
    """Wraps every layer MLP that has gate_proj in MetalLigerSwiGLU (patch.py:162-178)."""
    layers = _find_layers(model)
    if layers is None:
        return 0
    count = 0
    for layer in layers:
        if hasattr(layer, "mlp") and hasattr(layer.mlp, "gate_proj"):
            layer.mlp = MetalLigerSwiGLU(layer.mlp)
            count += 1
    return count


def apply_metal_liger_to_qwen3vl(
    model: nn.Module,
    fuse_rms_norm: bool = True,
    fuse_swiglu: bool = True,
    fuse_rope: bool = False,
    fuse_cross_entropy: bool = False,
    fuse_lora: bool = True,
    use_optimized_generator: bool = False,
    fuse_residual_norm: bool = False,
    fuse_qk_norm_rope: bool = False,
    fuse_lm_loss: bool = False,
    efficient_attention: bool = False,
) -> nn.Module:
    """Apply the fused operations to a Qwen3 / Qwen3-VL model in place and
    return it (patch.py:181-240).

    The reference's flags keep their meaning: fuse_rms_norm, fuse_swiglu
    and fuse_lora patch the model; fuse_rope and fuse_cross_entropy only
    record that the ops are available (RoPE is applied by the caller with
    apply_fused_rotary / apply_fused_rotary_inline, the fused cross-entropy
    through MetalLigerFusedLinearCrossEntropy in the training loop).

    Fusions the reference does not have, off by default:
    fuse_residual_norm: each decoder layer's post-attention residual add runs
    in the same launch as its post_attention_layernorm
    (ops/fused_add_rms_norm.py); needs fuse_rms_norm, whose norm it extends.
    fuse_qk_norm_rope: attention modules with q_norm / k_norm (Qwen3) get
    their head-dim norms and RoPE in one launch (ops/fused_qk_norm_rope.py).
    fuse_lm_loss: the causal LM's training loss (forward with labels in
    training mode) comes from the fused linear cross-entropy with
    transformers' label shift, and the output's logits are None
    (ops/fused_linear_cross_entropy.py, patch_causal_lm_loss).
    efficient_attention: grouped-query attention modules on transformers'
    "sdpa" implementation run SDPA's memory-efficient kernel over repeated
    key / value heads instead of the flash kernel with GQA
    (ops/gqa_attention.py).
    use_optimized_generator is not part of metal_liger_amd (inference path).
    """
    stats = {}
    if fuse_rms_norm:
        n = _replace_rms_norms(model)
        stats["rms_norm"] = n
        logger.info(f"MetalLiger: replaced {n} RMSNorm layers with fused versions")
    if fuse_swiglu:
        n = _replace_mlps(model)
        stats["swiglu"] = n
        logger.info(f"MetalLiger: replaced {n} MLP layers with fused SwiGLU")
    if fuse_residual_norm:
        n = patch_residual_add_norm(model)
        stats["residual_add_norm"] = n
        logger.info(f"MetalLiger: fused residual add + RMSNorm in {n} decoder layers")
    if fuse_qk_norm_rope:
        # before the LoRA patch, which wraps whatever attention forward it finds
        n = patch_qk_norm_rope(model)
        stats["qk_norm_rope"] = n
        logger.info(f"MetalLiger: fused q/k norm + RoPE on {n} attention modules")
    if fuse_lora:
        n = patch_fused_lora(model)
        stats["fused_lora"] = n
        logger.info(f"MetalLiger: fused LoRA QKV+MLP marked {n} modules")
    if fuse_lm_loss:
        n = patch_causal_lm_loss(model)
        stats["lm_loss"] = n
        logger.info(f"MetalLiger: fused linear cross-entropy loss on {n} causal LM heads")
    if efficient_attention:
        n = patch_efficient_attention(model)
        stats["efficient_attention"] = n
        logger.info(f"MetalLiger: {n} attention modules on SDPA's memory-efficient kernel")
    if use_optimized_generator:
        logger.warning("MetalLiger: the optimized generator is not part of metal_liger_amd; skipped")
        stats["generator"] = "unavailable"
    if fuse_rope:
        logger.info("MetalLiger: fused RoPE available — use apply_fused_rotary() / "
                    "apply_fused_rotary_inline()")
        stats["rope"] = "available"
    if fuse_cross_entropy:
        logger.info("MetalLiger: fused CE available — use MetalLigerFusedLinearCrossEntropy in the "
                    "training loop")
        stats["cross_entropy"] = "available"
    total = sum(v for v in stats.values() if isinstance(v, int))
    logger.info(f"MetalLiger: {total} total layers patched. Details: {stats}")
    return model
