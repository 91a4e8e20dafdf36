"""The opt-in grouped-query attention path (patcher flag efficient_attention:
key / value heads repeated, SDPA's memory-efficient kernel) on the GPU.

At the train-step layer's attention shape (query [4, 16, 2048, 128], key /
value [4, 8, 2048, 128], bf16, causal) its output and input gradients are
compared with an fp32 evaluation of the same attention (SDPA's math path on
fp32 copies) and must be no less accurate than transformers' default path
(SDPA with enable_gqa, the flash kernel): relative Frobenius error at most
1.5 x the default path's plus 2e-3. On the tiny GQA model the patched
forward + backward matches the default "sdpa" model's (loss within 1e-3
relative, LoRA gradients within relative Frobenius 2e-2), both with every fused op
patched in."""

import copy

import pytest
import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from tests import qwen_tiny
from tests.parity import rel_fro

pytestmark = pytest.mark.gpu


class _Attn(torch.nn.Module):
    num_key_value_groups = 2
    is_causal = True


def test_expanded_kv_attention_train_shape(dev):
    from metal_liger_amd.ops.gqa_attention import expanded_kv_attention_forward
    g = torch.Generator(device=dev).manual_seed(11)
    B, HQ, HK, S, D = 4, 16, 8, 2048, 128
    q0 = torch.randn(B, HQ, S, D, device=dev, generator=g).to(torch.bfloat16)
    k0 = torch.randn(B, HK, S, D, device=dev, generator=g).to(torch.bfloat16)
    v0 = torch.randn(B, HK, S, D, device=dev, generator=g).to(torch.bfloat16)
    dout = torch.randn(B, S, HQ, D, device=dev, generator=g).to(torch.bfloat16)
    scale = D ** -0.5
    print("attention: train-step shape, seed 11", flush=True)

    def run(fn, dtype):
        q, k, v = (t.detach().to(dtype).requires_grad_() for t in (q0, k0, v0))
        out = fn(q, k, v)
        out.backward(dout.to(dtype))
        return [t.float() for t in (out.detach(), q.grad, k.grad, v.grad)]

    def exact(q, k, v):
        k = k.repeat_interleave(2, dim=1)
        v = v.repeat_interleave(2, dim=1)
        with sdpa_kernel([SDPBackend.MATH]):
            o = F.scaled_dot_product_attention(q, k, v, scale=scale, is_causal=True)
        return o.transpose(1, 2)

    def default(q, k, v):
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            o = F.scaled_dot_product_attention(q, k, v, scale=scale, is_causal=True,
                                               enable_gqa=True)
        return o.transpose(1, 2)

    def ours(q, k, v):
        return expanded_kv_attention_forward(_Attn(), q, k, v, None, scaling=scale)[0]

    ref = run(exact, torch.float32)
    base = run(default, torch.bfloat16)
    got = run(ours, torch.bfloat16)
    assert got[0].shape == (B, S, HQ, D) and got[2].shape == (B, HK, S, D)
    for name, r, b, o in zip(("out", "dq", "dk", "dv"), ref, base, got):
        e_b, e_o = rel_fro(b, r), rel_fro(o, r)
        print(f"attention {name}: ours {e_o:.3e}, default {e_b:.3e}", flush=True)
        assert e_o <= 1.5 * e_b + 2e-3, (name, e_o, e_b)


def test_efficient_attention_tiny_model(dev):
    from metal_liger_amd import apply_metal_liger_to_qwen3vl
    from metal_liger_amd.ops.gqa_attention import ATTN_KEY
    model = qwen_tiny.build(attn="sdpa", dtype=torch.bfloat16).to(dev)
    kw = dict(fuse_qk_norm_rope=True, fuse_residual_norm=True, fuse_lm_loss=True)
    base = apply_metal_liger_to_qwen3vl(copy.deepcopy(model), **kw)
    patched = apply_metal_liger_to_qwen3vl(model, efficient_attention=True, **kw)
    assert base.base_model.model.config._attn_implementation == "sdpa"
    assert patched.base_model.model.config._attn_implementation == ATTN_KEY
    qwen_tiny.freeze_all_but_lora(base)
    qwen_tiny.freeze_all_but_lora(patched)
    ids = torch.randint(0, 512, (2, 64), device=dev,
                        generator=torch.Generator(device=dev).manual_seed(3))
    res = []
    for m in (base, patched):
        m.train()
        out = m(input_ids=ids, labels=ids, use_cache=False)
        out.loss.backward()
        res.append((out.loss.float().item(),
                    {n: p.grad.float() for n, p in m.named_parameters() if p.grad is not None}))
    (l_b, g_b), (l_p, g_p) = res
    assert abs(l_p - l_b) <= 1e-3 * abs(l_b), (l_p, l_b)
    assert set(g_b) == set(g_p) and len(g_b) == 2 * 7 * 2
    for n in g_b:
        assert rel_fro(g_p[n], g_b[n]) <= 2e-2, n
