"""Grouped-query attention through SDPA's memory-efficient kernel (opt-in).

transformers' "sdpa" attention hands grouped-query attention (fewer key /
value heads than query heads) to torch's scaled_dot_product_attention with
enable_gqa=True whenever no mask tensor is given
(transformers/integrations/sdpa_attention.py, use_gqa_in_sdpa), and on ROCm
that selects the flash kernel. For a Qwen3 layer of 16 query / 8 key-value
heads, head_dim 128, 4 x 2048 tokens, bf16, on MI355X, the memory-efficient
kernel over key / value heads repeated to 16 takes 0.85 ms forward +
backward against 1.38-1.43 ms for the flash kernel with GQA.

The reference has no attention code (its models run transformers' attention
unchanged), so this is an option of the patcher, off by default:
apply_metal_liger_to_qwen3vl(model, efficient_attention=True) switches every
grouped-query attention module whose config asks for "sdpa" to the function
registered here under ATTN_KEY. Masks are built as for "sdpa" (the same mask
function is registered under the key). On GPU tensors SDPA may pick only its
memory-efficient kernel, else flash; a shape neither takes raises instead of
falling back to the batched-matmul path. On CPU tensors the math path stays
allowed.
"""

import torch
from torch.nn.attention import SDPBackend, sdpa_kernel

ATTN_KEY = "metal_liger_sdpa"

_GPU_BACKENDS = [SDPBackend.EFFICIENT_ATTENTION, SDPBackend.FLASH_ATTENTION]
_CPU_BACKENDS = _GPU_BACKENDS + [SDPBackend.MATH]


def _repeat_heads(x: torch.Tensor, groups: int) -> torch.Tensor:
    """[B, Hkv, S, D] -> [B, Hkv * groups, S, D], each key / value head
    repeated for the `groups` query heads that share it (query head h reads
    key / value head h // groups)."""
    b, h, s, d = x.shape
    return x[:, :, None].expand(b, h, groups, s, d).reshape(b, h * groups, s, d)


def expanded_kv_attention_forward(module, query, key, value, attention_mask, dropout=0.0,
                                  scaling=None, is_causal=None, **kwargs):
    """AttentionInterface function: query [B, Hq, S, D], key / value
    [B, Hkv, Skv, D]; returns (output [B, S, Hq, D] contiguous, None).

    Causality follows transformers' sdpa path: SDPA's is_causal flag is set
    when the module is causal, there is more than one query and no mask tensor
    was built; keys beyond the query length are then dropped (an empty static
    cache's slots). Calls with a position bias go to transformers' own sdpa
    function unchanged."""
    if kwargs.get("position_bias") is not None:
        from transformers.integrations.sdpa_attention import sdpa_attention_forward
        return sdpa_attention_forward(module, query, key, value, attention_mask, dropout=dropout,
                                      scaling=scaling, is_causal=is_causal, **kwargs)
    groups = getattr(module, "num_key_value_groups", 1)
    if groups > 1:
        key = _repeat_heads(key, groups)
        value = _repeat_heads(value, groups)
    q_len, kv_len = query.shape[2], key.shape[2]
    if attention_mask is not None and attention_mask.ndim == 4:
        attention_mask = attention_mask[:, :, :, :kv_len]  # as transformers' sdpa path
    causal = getattr(module, "is_causal", True) if is_causal is None else is_causal
    causal = bool(causal) and q_len > 1 and attention_mask is None
    if causal and kv_len > q_len:
        key = key[:, :, :q_len]
        value = value[:, :, :q_len]
    with sdpa_kernel(_GPU_BACKENDS if query.is_cuda else _CPU_BACKENDS, set_priority=True):
        out = torch.nn.functional.scaled_dot_product_attention(
            query, key, value, attn_mask=attention_mask, dropout_p=dropout, scale=scaling,
            is_causal=causal)
    return out.transpose(1, 2).contiguous(), None


def register_efficient_attention() -> str:
    """Registers the attention function and the "sdpa" mask builder under
    ATTN_KEY (idempotent); returns the key."""
    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface, sdpa_mask
    AttentionInterface.register(ATTN_KEY, expanded_kv_attention_forward)
    AttentionMaskInterface.register(ATTN_KEY, sdpa_mask)
    return ATTN_KEY


def patch_efficient_attention(model: torch.nn.Module) -> int:
    """Points the config of every grouped-query attention module (one with
    num_key_value_groups > 1) that uses "sdpa" at ATTN_KEY; returns the
    number of attention modules that run through it afterwards. Modules on
    another implementation (eager, flash_attention_2, a custom one) and
    attention without head groups (a vision tower's) keep theirs."""
    register_efficient_attention()
    configs = {}
    for m in model.modules():
        cfg = getattr(m, "config", None)
        if getattr(m, "num_key_value_groups", 1) > 1 and cfg is not None:
            configs.setdefault(id(cfg), (cfg, []))[1].append(m)
    n = 0
    for cfg, mods in configs.values():
        if cfg._attn_implementation == "sdpa":
            cfg._attn_implementation = ATTN_KEY
        if cfg._attn_implementation == ATTN_KEY:
            n += len(mods)
    return n
