"""Qwen3 causal LMs (HF transformers) with PEFT-layout LoRA adapters, for
patcher and end-to-end tests: a tiny one, and the 4-layer Qwen3-style model
of the LoRA train-step workload (also built by bench.py)."""

import torch
import torch.nn as nn

from tests.peft_shim import LoraLinear, init_lora, wrap_lora


def tiny_config(**kw):
    from transformers import Qwen3Config
    cfg = dict(vocab_size=512, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
               num_attention_heads=4, num_key_value_heads=2, head_dim=32, rms_norm_eps=1e-6,
               rope_theta=1e6, max_position_embeddings=256, tie_word_embeddings=False)
    cfg.update(kw)
    return Qwen3Config(**cfg)


class PeftLike(nn.Module):
    """PeftModel -> LoraModel -> causal LM nesting (base_model.model)."""

    def __init__(self, lm: nn.Module):
        super().__init__()
        self.base_model = nn.Module()
        self.base_model.model = lm

    def forward(self, *a, **k):
        return self.base_model.model(*a, **k)


def build(seed=0, lora=True, peft_wrap=True, attn="eager", dtype=torch.float32):
    from transformers import Qwen3ForCausalLM
    torch.manual_seed(seed)
    cfg = tiny_config()
    cfg._attn_implementation = attn
    lm = Qwen3ForCausalLM(cfg).to(dtype)
    if lora:
        for i, layer in enumerate(lm.model.layers):
            wrap_lora(layer.self_attn, ["q_proj", "k_proj", "v_proj", "o_proj"], r=16, alpha=32)
            wrap_lora(layer.mlp, ["gate_proj", "up_proj", "down_proj"], r=16, alpha=32)
            for j, m in enumerate(list(layer.self_attn.children()) + list(layer.mlp.children())):
                if isinstance(m, LoraLinear):
                    init_lora(m, 1000 * seed + 10 * i + j)
        lm.to(dtype)
    return PeftLike(lm) if peft_wrap else lm


def register_fp32_attention(name="ml_fp32_eager"):
    """Eager attention evaluated in fp32 with contiguous operands (the bf16
    batched products with transposed right operands are avoided on ROCm)."""
    from transformers import AttentionInterface
    from transformers.models.qwen3.modeling_qwen3 import repeat_kv

    def attn(module, query, key, value, attention_mask, scaling, dropout=0.0, **kwargs):
        k = repeat_kv(key, module.num_key_value_groups).float()
        v = repeat_kv(value, module.num_key_value_groups).float().contiguous()
        w = torch.matmul(query.float().contiguous(), k.transpose(2, 3).contiguous()) * scaling
        if attention_mask is not None:
            w = w + attention_mask.float()
        w = torch.softmax(w, dim=-1)
        out = torch.matmul(w, v).to(query.dtype)
        return out.transpose(1, 2).contiguous(), None

    AttentionInterface.register(name, attn)
    return name


def build_vl(seed=0, attn="eager", dtype=torch.float32):
    """A tiny Qwen3-VL (text stack as tiny_config, interleaved M-RoPE; a
    one-block vision tower), norm weights 1 + 0.1 N(0, 1)."""
    from transformers import Qwen3VLConfig, Qwen3VLForConditionalGeneration
    cfg = Qwen3VLConfig(
        text_config=dict(vocab_size=512, hidden_size=128, intermediate_size=256,
                         num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                         head_dim=32, rms_norm_eps=1e-6, rope_theta=1e6,
                         max_position_embeddings=256,
                         rope_scaling={"rope_type": "default", "mrope_section": [8, 4, 4],
                                       "mrope_interleaved": True}),
        vision_config=dict(depth=1, hidden_size=64, intermediate_size=128, num_heads=2,
                           out_hidden_size=128, deepstack_visual_indexes=[]))
    cfg._attn_implementation = attn
    cfg.text_config._attn_implementation = attn
    torch.manual_seed(seed)
    model = Qwen3VLForConditionalGeneration(cfg)
    with torch.no_grad():
        for n, p in model.named_parameters():
            if n.endswith("norm.weight"):
                p.normal_(1.0, 0.1)
    return model.to(dtype)


# The 4-layer Qwen3-style LoRA train-step workload: hidden 2048, 16 q / 8 kv
# heads, head_dim 128, MLP 6144, eps 1e-6, theta 1e6, vocab 151936, tied
# embeddings, rank-16 alpha-32 LoRA on q, k, v, o, gate, up, down; token ids
# [4, 2048] uniform in [0, vocab).
TRAIN_LAYERS, TRAIN_B, TRAIN_S, TRAIN_V = 4, 4, 2048, 151936
TRAIN_H, TRAIN_I, TRAIN_R = 2048, 6144, 16


def build_train_config(dev, layers=TRAIN_LAYERS, attn="sdpa", seed=0):
    """The train-step model, unpatched, bf16 on `dev`, HF's random init with
    seeded adapters (A ~ N(0, 0.25^2), B ~ N(0, 0.02^2)), wrapped as PEFT
    nests it; only the adapters require grad."""
    from transformers import Qwen3Config, Qwen3ForCausalLM
    cfg = Qwen3Config(vocab_size=TRAIN_V, hidden_size=TRAIN_H, intermediate_size=TRAIN_I,
                      num_hidden_layers=layers, num_attention_heads=16, num_key_value_heads=8,
                      head_dim=128, rms_norm_eps=1e-6, rope_theta=1e6,
                      max_position_embeddings=TRAIN_S, tie_word_embeddings=True)
    cfg._attn_implementation = attn
    torch.manual_seed(seed)
    with torch.device(dev):
        lm = Qwen3ForCausalLM(cfg)
    for i, layer in enumerate(lm.model.layers):
        wrap_lora(layer.self_attn, ["q_proj", "k_proj", "v_proj", "o_proj"], r=TRAIN_R, alpha=32)
        wrap_lora(layer.mlp, ["gate_proj", "up_proj", "down_proj"], r=TRAIN_R, alpha=32)
        for j, m in enumerate(list(layer.self_attn.children()) + list(layer.mlp.children())):
            if isinstance(m, LoraLinear):
                init_lora(m, 10 * i + j)
    lm.to(device=dev, dtype=torch.bfloat16)
    model = PeftLike(lm)
    freeze_all_but_lora(model)
    return model


def freeze_all_but_lora(model):
    """Only LoRA adapters train (the patcher wraps norm weights in new
    Parameters, as the reference's MetalLigerRMSNorm does: call it again
    after patching)."""
    for n, p in model.named_parameters():
        p.requires_grad_("lora_" in n)


def train_ids(dev, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, TRAIN_V, (TRAIN_B, TRAIN_S), generator=g).to(dev)
