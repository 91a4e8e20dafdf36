"""Empty batches through the drop-in autograd Functions on the GPU (torch's
own ops, which the reference's Functions are made of, accept them): outputs
of the right empty shapes, input gradients empty, parameter gradients zero
(empty sums). FLCE's empty case is in test_gpu_flce.py."""

import pytest
import torch

from tests.parity import seeded

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def _bf(shape, seed, dev, scale=1.0):
    return seeded(shape, seed, BF, scale=scale).to(dev)


def _adapter(out_f, in_f, seed, dev, r=16):
    return (_bf((out_f, in_f), seed, dev, 0.05), _bf((r, in_f), seed + 1, dev, 0.25).requires_grad_(True),
            _bf((out_f, r), seed + 2, dev, 0.05).requires_grad_(True), 2.0)


def _check_zero_grads(ts):
    for t in ts:
        assert t.grad is not None and torch.count_nonzero(t.grad) == 0


def test_lora_functions_empty_batch(dev):
    from metal_liger_amd.ops.fused_lora import _LoRA_MLP, _LoRA_QKV, _LoRA_W
    H, I = 128, 256
    X = torch.empty(0, H, dtype=BF, device=dev, requires_grad=True)
    qkv = [_adapter(o, H, 10 + 5 * i, dev) for i, o in enumerate((H, 64, 64))]
    Q, K, V = _LoRA_QKV.apply(X, *[t for a in qkv for t in a])
    assert Q.shape == (0, H) and K.shape == (0, 64) and V.shape == (0, 64)
    (Q.float().sum() + K.float().sum() + V.float().sum()).backward()
    assert X.grad.shape == (0, H)
    _check_zero_grads([t for a in qkv for t in a[1:3]])

    X.grad = None
    mlp = [_adapter(I, H, 30, dev), _adapter(I, H, 35, dev), _adapter(H, I, 40, dev)]
    out = _LoRA_MLP.apply(X, *[t for a in mlp for t in a])
    assert out.shape == (0, H)
    out.float().sum().backward()
    assert X.grad.shape == (0, H)
    _check_zero_grads([t for a in mlp for t in a[1:3]])

    X.grad = None
    o = _adapter(H, H, 50, dev)
    y = _LoRA_W.apply(X, *o)
    assert y.shape == (0, H)
    y.float().sum().backward()
    assert X.grad.shape == (0, H)
    _check_zero_grads(o[1:3])


def test_rope_and_qk_norm_empty_sequence(dev):
    from metal_liger_amd.ops.fused_qk_norm_rope import _FusedQKNormRoPEFunction
    from metal_liger_amd.ops.fused_rope import apply_fused_rotary, apply_fused_rotary_inline
    q = torch.empty(2, 4, 0, 64, dtype=BF, device=dev, requires_grad=True)
    k = torch.empty(2, 2, 0, 64, dtype=BF, device=dev, requires_grad=True)
    cos = torch.empty(0, 64, dtype=BF, device=dev)
    qa, ka = apply_fused_rotary(q, k, cos, cos)
    qb, kb = apply_fused_rotary_inline(qa, ka, torch.empty(0, dtype=torch.int64, device=dev), theta=1e4)
    wq = seeded((64,), 1, BF, 0.1, 1.0).to(dev).requires_grad_(True)
    wk = seeded((64,), 2, BF, 0.1, 1.0).to(dev).requires_grad_(True)
    c4 = torch.empty(2, 1, 0, 64, dtype=BF, device=dev)
    qc, kc = _FusedQKNormRoPEFunction.apply(qb, kb, wq, wk, c4, c4, 1e-6)
    assert qc.shape == q.shape and kc.shape == k.shape
    (qc.float().sum() + kc.float().sum()).backward()
    assert q.grad.shape == q.shape and k.grad.shape == k.shape
    _check_zero_grads([wq, wk])


def test_norms_empty_rows_through_modules(dev):
    from metal_liger_amd import MetalLigerRMSNorm
    from metal_liger_amd.ops.fused_add_rms_norm import fused_add_rms_norm
    norm = MetalLigerRMSNorm(256, weight=seeded((256,), 3, BF, 0.1, 1.0)).to(dev)
    x = torch.empty(0, 7, 256, dtype=BF, device=dev, requires_grad=True)
    r = torch.empty(0, 7, 256, dtype=BF, device=dev, requires_grad=True)
    y, total = fused_add_rms_norm(norm(x), r, norm)
    assert y.shape == total.shape == (0, 7, 256)
    (y.float().sum() + total.float().sum()).backward()
    assert x.grad.shape == r.grad.shape == (0, 7, 256)
    _check_zero_grads([norm.weight])


def test_flce_module_empty_batch(dev):
    """The module flattens [B, S, H] itself: B = 0 gives the reference's loss
    for no valid token (0) and zero / empty gradients."""
    from metal_liger_amd import MetalLigerFusedLinearCrossEntropy
    lm_head = torch.nn.Linear(128, 512, bias=False).to(dev, BF)
    h = torch.empty(0, 5, 128, dtype=BF, device=dev, requires_grad=True)
    loss = MetalLigerFusedLinearCrossEntropy(lm_head)(h, torch.empty(0, 5, dtype=torch.int64, device=dev))
    assert loss.item() == 0.0
    loss.backward()
    assert h.grad.shape == h.shape
    _check_zero_grads([lm_head.weight])
