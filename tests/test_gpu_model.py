"""End to end on the GPU: a tiny Qwen3 causal LM with LoRA adapters on every
projection (PEFT layout), patched by apply_metal_liger_to_qwen3vl, trained
one step against the same model unpatched.

Criterion (bf16 model): against the unpatched model evaluated in fp32 from the
same bf16 weights ("exact"), the patched model's loss and LoRA gradients are
no less accurate than the unpatched bf16 model's, within a factor 1.5 plus a
floor of 2e-3 relative (the two bf16 evaluations round at different points),
and the patched and unpatched bf16 results agree within relative Frobenius
5e-2 (12 bf16 layers of rounding on each side)."""

import copy

import pytest
import torch
import torch.nn.functional as F

from tests import qwen_tiny
from tests.parity import rel_fro

pytestmark = pytest.mark.gpu


def lora_grads(model):
    return {n: p.grad.detach().float().clone() for n, p in model.named_parameters()
            if "lora_" in n and p.grad is not None}


def train_step(model, ids):
    model.zero_grad(set_to_none=True)
    out = model(input_ids=ids, labels=ids)
    out.loss.backward()
    return out.loss.detach().float(), lora_grads(model)


@pytest.mark.parametrize("fuse_qkn,fuse_ce,fuse_res", [(False, False, False), (True, False, False),
                                                        (False, False, True), (True, True, True)])
def test_patched_qwen3_lora_train_step(dev, fuse_qkn, fuse_ce, fuse_res):
    """fuse_qk_norm_rope=True routes q_norm / k_norm + RoPE through the fused
    kernel; fuse_lm_loss=True computes the model's training loss (from
    labels) with the fused linear cross-entropy instead of logits;
    fuse_residual_norm=True fuses each layer's post-attention residual add
    into its norm."""
    from metal_liger_amd import apply_metal_liger_to_qwen3vl
    attn = qwen_tiny.register_fp32_attention()
    base = qwen_tiny.build(seed=3, attn=attn, dtype=torch.bfloat16).to(dev)
    for n, p in base.named_parameters():
        p.requires_grad_("lora_" in n)
    exact = copy.deepcopy(base).float()
    patched = apply_metal_liger_to_qwen3vl(copy.deepcopy(base), fuse_qk_norm_rope=fuse_qkn,
                                           fuse_lm_loss=fuse_ce, fuse_residual_norm=fuse_res)
    lm = patched.base_model.model
    qkn = [getattr(l.self_attn, "_metal_liger_qk_norm_rope", False) for l in lm.model.layers]
    assert qkn == [fuse_qkn] * 2
    assert getattr(lm, "_metal_liger_flce_loss", False) == fuse_ce
    assert [getattr(l, "_metal_liger_add_norm", False) for l in lm.model.layers] == [fuse_res] * 2
    g = torch.Generator().manual_seed(7)
    ids = torch.randint(0, 512, (2, 96), generator=g).to(dev)

    l_ex, g_ex = train_step(exact, ids)
    l_bf, g_bf = train_step(base, ids)
    l_pt, g_pt = train_step(patched, ids)
    assert torch.isfinite(l_pt)
    assert set(g_pt) == set(g_ex) and len(g_pt) == 2 * 7 * 2
    err_bf = abs(l_bf - l_ex).item()
    err_pt = abs(l_pt - l_ex).item()
    assert err_pt <= 1.5 * err_bf + 2e-3 * abs(l_ex.item()), (err_pt, err_bf)
    for n in g_ex:
        e_bf = rel_fro(g_bf[n], g_ex[n])
        e_pt = rel_fro(g_pt[n], g_ex[n])
        assert e_pt <= 1.5 * e_bf + 2e-3, f"{n}: patched {e_pt:.3e} vs bf16 {e_bf:.3e}"
        assert rel_fro(g_pt[n], g_bf[n]) <= 5e-2, n


def test_patched_model_fused_loss(dev):
    """The patched decoder's hidden states through MetalLigerFusedLinearCrossEntropy
    equal cross_entropy over the fp32 logits (1e-3 relative)."""
    from metal_liger_amd import MetalLigerFusedLinearCrossEntropy, apply_metal_liger_to_qwen3vl
    attn = qwen_tiny.register_fp32_attention()
    model = apply_metal_liger_to_qwen3vl(qwen_tiny.build(seed=4, attn=attn, dtype=torch.bfloat16).to(dev))
    lm = model.base_model.model
    ids = torch.randint(0, 512, (2, 80), generator=torch.Generator().manual_seed(1)).to(dev)
    hidden = lm.model(input_ids=ids).last_hidden_state
    h = hidden[:, :-1]
    lab = ids[:, 1:]
    loss = MetalLigerFusedLinearCrossEntropy(lm.lm_head, chunk_size=128)(h, lab)
    ref = F.cross_entropy((h.float().reshape(-1, 128) @ lm.lm_head.weight.float().t()), lab.reshape(-1))
    assert abs(loss.item() - ref.item()) <= 1e-3 * abs(ref.item())
    loss.backward()
    assert all(torch.isfinite(p.grad).all() for n, p in lm.named_parameters()
               if "lora_" in n and p.grad is not None)


def test_patched_qwen3_vl_train_step(dev):
    """The Qwen3-VL text stack (its interleaved M-RoPE tables feed the fused
    q/k norm + RoPE), patched with every flag, trained one step in bf16
    (all text-stack parameters trainable) against the same model unpatched:
    against the fp32 evaluation, the loss and every gradient are no less
    accurate than the unpatched bf16 model's (criterion as above)."""
    from metal_liger_amd import apply_metal_liger_to_qwen3vl
    attn = qwen_tiny.register_fp32_attention()
    base = qwen_tiny.build_vl(seed=9, attn=attn, dtype=torch.bfloat16).to(dev)
    exact = copy.deepcopy(base).float()
    patched = apply_metal_liger_to_qwen3vl(copy.deepcopy(base), fuse_qk_norm_rope=True,
                                           fuse_lm_loss=True, fuse_residual_norm=True)
    layers = patched.model.language_model.layers
    assert all(getattr(l.self_attn, "_metal_liger_qk_norm_rope", False) for l in layers)
    assert all(getattr(l, "_metal_liger_add_norm", False) for l in layers)
    ids = torch.randint(0, 512, (2, 96), generator=torch.Generator().manual_seed(10)).to(dev)

    def step(model):
        model.train()
        model.zero_grad(set_to_none=True)
        out = model(input_ids=ids, labels=ids)
        out.loss.backward()
        return out.loss.detach().float(), {n: p.grad.detach().float().clone()
                                           for n, p in model.named_parameters() if p.grad is not None}

    l_ex, g_ex = step(exact)
    l_bf, g_bf = step(base)
    l_pt, g_pt = step(patched)
    assert torch.isfinite(l_pt) and set(g_pt) == set(g_ex) == set(g_bf) and len(g_ex) > 20
    err_bf = abs(l_bf - l_ex).item()
    err_pt = abs(l_pt - l_ex).item()
    assert err_pt <= 1.5 * err_bf + 2e-3 * abs(l_ex.item()), (err_pt, err_bf)
    for n in g_ex:
        e_bf = rel_fro(g_bf[n], g_ex[n])
        e_pt = rel_fro(g_pt[n], g_ex[n])
        assert e_pt <= 1.5 * e_bf + 2e-3, f"{n}: patched {e_pt:.3e} vs bf16 {e_bf:.3e}"


def test_patched_qwen3_lora_train_step_fp32(dev):
    """An fp32 model (the reference's own test dtype) patched with every
    flag: the fused LoRA Functions run fp32 matrix-core products, the norms
    and SwiGLU their fp32 kernels, the loss the fp32 chunked cross-entropy;
    loss and LoRA gradients match the unpatched fp32 model (relative 1e-4:
    fp32 sums in another order through two layers)."""
    from metal_liger_amd import apply_metal_liger_to_qwen3vl
    attn = qwen_tiny.register_fp32_attention()
    base = qwen_tiny.build(seed=11, attn=attn, dtype=torch.float32).to(dev)
    for n, p in base.named_parameters():
        p.requires_grad_("lora_" in n)
    patched = apply_metal_liger_to_qwen3vl(copy.deepcopy(base), fuse_qk_norm_rope=True,
                                           fuse_lm_loss=True, fuse_residual_norm=True)
    for n, p in patched.named_parameters():
        p.requires_grad_("lora_" in n)
    ids = torch.randint(0, 512, (2, 64), generator=torch.Generator().manual_seed(12)).to(dev)
    l_ref, g_ref = train_step(base, ids)
    l_pt, g_pt = train_step(patched, ids)
    assert abs(l_pt - l_ref).item() <= 1e-5 * abs(l_ref.item())
    assert set(g_pt) == set(g_ref) and len(g_ref) == 2 * 7 * 2
    for n in g_ref:
        assert rel_fro(g_pt[n], g_ref[n]) <= 1e-4, (n, rel_fro(g_pt[n], g_ref[n]))
