"""The 4-layer Qwen3-style LoRA train step at its full size on the GPU:
hidden 2048, 16 q / 8 kv heads, head_dim 128, MLP 6144, vocab 151936, tied
embeddings, rank-16 LoRA on q, k, v, o, gate, up, down, token ids [4, 2048]
(reference patch.py:181-240, ops/fused_lora.py:323-421).

The model patched with every flag (fused RMSNorm, SwiGLU, LoRA QKV / MLP /
o_proj, q/k norm + RoPE, residual add + norm, the causal-LM loss through the
chunked fused linear cross-entropy) takes one forward + backward against the
same bf16 model unpatched and against that model evaluated in fp32 from the
same weights ("exact"). All three run the same fp32 eager attention, so the
comparison isolates the fused ops.

Bar: the patched loss within 1e-3 relative of the unpatched bf16 loss; every
LoRA gradient within relative Frobenius 5e-2 of the unpatched bf16
model's, and, against the fp32 evaluation, no less accurate than the
unpatched bf16 model's (factor 1.5 plus 2e-3, the criterion of
test_gpu_model.py: the two bf16 evaluations round at different points)."""

import copy

import pytest
import torch

from tests import qwen_tiny
from tests.parity import rel_fro

pytestmark = pytest.mark.gpu


def _step(model, ids):
    model.train()
    model.zero_grad(set_to_none=True)
    out = model(input_ids=ids, labels=ids, use_cache=False)
    out.loss.backward()
    grads = {n: p.grad.detach().float().clone() for n, p in model.named_parameters()
             if "lora_" in n and p.grad is not None}
    return out.loss.detach().float().item(), grads, out.logits


def test_train_step_full_config(dev):
    from metal_liger_amd import apply_metal_liger_to_qwen3vl
    attn = qwen_tiny.register_fp32_attention()
    print("train step: building the 4-layer model", flush=True)
    base = qwen_tiny.build_train_config(dev, attn=attn)
    ids = qwen_tiny.train_ids(dev)

    l_bf, g_bf, _ = _step(base, ids)
    print(f"train step: unpatched bf16 loss {l_bf:.6f}", flush=True)
    patched = apply_metal_liger_to_qwen3vl(copy.deepcopy(base), fuse_qk_norm_rope=True,
                                           fuse_lm_loss=True, fuse_residual_norm=True)
    qwen_tiny.freeze_all_but_lora(patched)
    layers = patched.base_model.model.model.layers
    assert all(getattr(l.self_attn, "_metal_liger_fused_lora", False) for l in layers)
    assert all(getattr(l.mlp, "_metal_liger_fused_lora", False) for l in layers)
    assert all(getattr(l.self_attn, "_metal_liger_qk_norm_rope", False) for l in layers)
    assert all(getattr(l, "_metal_liger_add_norm", False) for l in layers)
    l_pt, g_pt, logits = _step(patched, ids)
    print(f"train step: patched loss {l_pt:.6f}", flush=True)
    assert logits is None                                   # no [tokens, vocab] logits
    del patched
    exact = copy.deepcopy(base).float()
    del base
    torch.cuda.empty_cache()
    l_ex, g_ex, _ = _step(exact, ids)
    print(f"train step: fp32 loss {l_ex:.6f}", flush=True)

    assert abs(l_pt - l_bf) <= 1e-3 * abs(l_bf), (l_pt, l_bf)
    err_bf, err_pt = abs(l_bf - l_ex), abs(l_pt - l_ex)
    assert err_pt <= 1.5 * err_bf + 2e-3 * abs(l_ex), (err_pt, err_bf)
    assert set(g_pt) == set(g_bf) == set(g_ex) and len(g_ex) == 4 * 7 * 2
    worst = 0.0
    for n in g_ex:
        e_bf = rel_fro(g_bf[n], g_ex[n])
        e_pt = rel_fro(g_pt[n], g_ex[n])
        d = rel_fro(g_pt[n], g_bf[n])
        worst = max(worst, d)
        assert e_pt <= 1.5 * e_bf + 2e-3, f"{n}: patched {e_pt:.3e} vs bf16 {e_bf:.3e}"
        assert d <= 5e-2, f"{n}: patched vs unpatched bf16 {d:.3e}"
    print(f"train step: worst LoRA grad difference (rel. Frobenius) {worst:.3e}", flush=True)
