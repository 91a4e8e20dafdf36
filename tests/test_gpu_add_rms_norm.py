"""Residual add fused into RMSNorm on the GPU against the oracle.

Forward: the stored sum must equal torch's own add on the same device bit for
bit (the kernel rounds the exact sum once to the input dtype, as torch does),
the normalised output must equal the plain fused RMSNorm of that sum bit for
bit (the same arithmetic), and both are checked against the oracle
(oracle/reference_ops.py add_rms_norm_forward): bf16 / fp16 rtol 2e-2 / atol
1e-2 plus relative Frobenius 2e-2, fp32 rtol 1e-5.
Backward: dx (the gradient of both x and the residual) against the oracle's
fp32 closed form plus the residual branch's gradient, rounded once; dw
against the oracle and bit-equal to the plain norm's backward (the residual
gradient does not enter it). In fp32 dx is also bit-equal to the unfused
pair (the plain norm's dx, then torch's add).
"""

import pytest
import torch

from oracle import reference_ops as ref
from tests.parity import assert_close, seeded

pytestmark = pytest.mark.gpu

BF16, F16, F32 = torch.bfloat16, torch.float16, torch.float32

CASES = [
    # shape, x dtype, weight dtype, layout
    ((8192, 2048), BF16, BF16, "contig"),     # the decoder layer's hidden states
    ((37, 2048), F32, F32, "contig"),
    ((5, 3, 1000), F16, F32, "contig"),        # tail chunk masked on the fast path
    ((17, 1001), BF16, BF16, "contig"),        # generic path (cols % 8 != 0)
    ((64, 4096), BF16, F32, "contig"),         # register forward, generic backward
    ((300, 2048), BF16, BF16, "strided"),      # row stride > cols (a column slice)
    ((33, 512), F32, F32, "misaligned"),       # base not 16-byte aligned: generic path
]


def make(shape, dtype, seed, layout, dev="cpu"):
    """A seeded tensor in the given layout, the view taken on `dev` (so a
    device copy keeps the strides / misalignment)."""
    if layout == "strided":
        wide = seeded(shape[:-1] + (shape[-1] + 64,), seed, dtype).to(dev)
        return wide[..., 32:32 + shape[-1]]
    if layout == "misaligned":
        n = 1
        for d in shape:
            n *= d
        return seeded((n + 1,), seed, dtype).to(dev)[1:].view(shape)
    return seeded(shape, seed, dtype).to(dev)


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{'x'.join(map(str, c[0]))}-{c[1]}-{c[2]}-{c[3]}")
def test_add_rms_norm_fwd_bwd(dev, case):
    from metal_liger_amd import hip_ops
    shape, dtype, wdtype, layout = case
    eps = 1e-6
    x, gx = make(shape, dtype, 1, layout), make(shape, dtype, 1, layout, dev)
    res = make(shape, dtype, 2, "contig")
    ds, gds = make(shape, dtype, 5, layout), make(shape, dtype, 5, layout, dev)
    w = seeded((shape[-1],), 3, wdtype, 0.1, 1.0)
    dy = seeded(shape, 4, dtype)
    gr, gw, gdy = (t.to(dev) for t in (res, w, dy))
    assert gx.is_contiguous() == (layout != "strided")
    assert (gx.data_ptr() % 16 != 0) == (layout == "misaligned")

    y, total, rrms = hip_ops.rms_norm_add_fwd(gx, gr, gw, eps)
    assert y.dtype == total.dtype == dtype and rrms.dtype == F32
    assert torch.equal(total, gx + gr)
    if layout != "misaligned":
        # (a misaligned x takes the generic path, whose sum of squares is
        # reduced in another order than the aligned sum's register path)
        assert torch.equal(y, hip_ops.rms_norm_fwd(total, gw, eps)[0])
    ry, rtotal, rr = ref.add_rms_norm_forward(x, res, w, eps)
    assert torch.equal(total.cpu(), rtotal)
    assert_close(y, ry, "y", dtype)
    assert_close(rrms, rr.squeeze(-1), "rrms", F32)

    dx, dw = hip_ops.rms_norm_bwd(total, gw, gdy, rrms, eps, dsum=gds)
    assert dx.dtype == dtype and dw.dtype == wdtype
    rdx, rdw = ref.add_rms_norm_backward(rtotal, w, rr, dy, ds)
    assert_close(dx, rdx, "dx", dtype)
    assert_close(dw, rdw, "dw", wdtype)
    plain_dx, plain_dw = hip_ops.rms_norm_bwd(total, gw, gdy, rrms, eps)
    if layout != "misaligned":   # (the same path: see above)
        assert torch.equal(dw, plain_dw)
        if dtype == F32:
            assert torch.equal(dx, plain_dx + gds)


def test_add_rms_norm_empty_rows(dev):
    from metal_liger_amd import hip_ops
    x = torch.empty(0, 2048, dtype=BF16, device=dev)
    w = torch.ones(2048, dtype=BF16, device=dev)
    y, total, rrms = hip_ops.rms_norm_add_fwd(x, x, w, 1e-6)
    assert y.shape == total.shape == (0, 2048) and rrms.shape == (0,)
    dx, dw = hip_ops.rms_norm_bwd(total, w, y, rrms, 1e-6, dsum=y)
    assert dx.shape == (0, 2048) and torch.equal(dw, torch.zeros_like(dw))


def test_add_rms_norm_rejects_mismatched_residual(dev):
    from metal_liger_amd import hip_ops
    x = torch.zeros(4, 256, dtype=BF16, device=dev)
    w = torch.ones(256, dtype=BF16, device=dev)
    with pytest.raises(ValueError, match="residual"):
        hip_ops.rms_norm_add_fwd(x, x.float(), w, 1e-6)
    with pytest.raises(ValueError, match="residual"):
        hip_ops.rms_norm_add_fwd(x, x[:2], w, 1e-6)


def test_add_rms_norm_autograd_function(dev):
    """fused_add_rms_norm through autograd: x and the residual receive the
    same gradient, the norm weight its dw; against fp32 autograd of the
    oracle's norm from the sum rounded to bf16 (as torch's add rounds it,
    and as the kernel normalises it)."""
    from metal_liger_amd.ops.fused_add_rms_norm import fused_add_rms_norm
    from metal_liger_amd.ops.fused_rms_norm import MetalLigerRMSNorm
    shape = (4, 96, 2048)
    x, r = seeded(shape, 10, BF16), seeded(shape, 11, BF16)
    norm = MetalLigerRMSNorm(2048, eps=1e-6, weight=seeded((2048,), 12, BF16, 0.1, 1.0)).to(dev)
    gy, gs = seeded(shape, 13, BF16), seeded(shape, 14, BF16)
    gx = x.to(dev).requires_grad_(True)
    gr = r.to(dev).requires_grad_(True)
    y, total = fused_add_rms_norm(gx, gr, norm)
    ((y.float() * gy.to(dev).float()).sum() + (total.float() * gs.to(dev).float()).sum()).backward()
    assert torch.equal(gx.grad, gr.grad)

    tf = (x + r).float().requires_grad_(True)
    assert torch.equal(total.cpu().float(), tf.detach())
    wf = norm.weight.detach().cpu().float().requires_grad_(True)
    yf, _ = ref.rms_norm_forward(tf, wf, 1e-6)
    ((yf * gy.float()).sum() + (tf * gs.float()).sum()).backward()
    assert_close(y, yf, "y", BF16)
    assert_close(gx.grad, tf.grad, "dx", BF16)
    assert_close(norm.weight.grad, wf.grad, "dw", BF16)
