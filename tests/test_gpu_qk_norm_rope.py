"""Fused q/k head-dim RMSNorm + RoPE on the GPU against the oracle
(transformers' Qwen3RMSNorm + apply_rotary_pos_emb, restated; exact fp32 VJP).

Forward: the kernel computes in fp32 and rounds once. It is checked against
the oracle evaluated in fp32 from the same inputs (bf16 / fp16: rtol 2e-2 /
atol 1e-2 plus relative Frobenius 2e-2; fp32: rtol 1e-5), and must be no less
accurate than transformers' own rounding sequence in the input dtype (the
oracle run in that dtype), whose separately rounded products n * cos and
rotate_half(n) * sin can cancel to errors beyond the bf16 bar.
Backward: the oracle's fp32 closed form (pinned against fp64 autograd) from
the same inputs, to the same bars. Weight gradients of bf16 weights are
rounded to bf16 once.
"""

import pytest
import torch

from oracle import reference_ops as ref
from tests.parity import assert_close, rel_fro, seeded

pytestmark = pytest.mark.gpu

BF16, F16, F32 = torch.bfloat16, torch.float16, torch.float32


def make_inputs(B, Hq, Hk, S, D, dtype, wdtype, layout, table_b, seed):
    """q, k as [B, H, S, D]: 'hf' = transposed views of [B, S, H, D] memory
    (what the Qwen3 attention passes), 'contig' = contiguous. Tables [table_b,
    S, D] with generic (not duplicated-half) values."""
    def x(H, s):
        if layout == "hf":
            return seeded((B, S, H, D), s, dtype).transpose(1, 2)
        return seeded((B, H, S, D), s, dtype)
    q, k = x(Hq, seed), x(Hk, seed + 1)
    wq = seeded((D,), seed + 2, wdtype, 0.1, 1.0)
    wk = seeded((D,), seed + 3, wdtype, 0.1, 1.0)
    cos = seeded((table_b, S, D), seed + 4, dtype, 0.7)
    sin = seeded((table_b, S, D), seed + 5, dtype, 0.7)
    return q, k, wq, wk, cos, sin


CASES = [
    # B, Hq, Hk, S, D, dtype, weight dtype, layout, table batch
    (2, 4, 2, 33, 128, BF16, BF16, "hf", 2),
    (1, 3, 3, 7, 64, F32, F32, "contig", 1),
    (2, 2, 1, 50, 256, BF16, F32, "hf", 1),
    (3, 4, 2, 5, 32, F16, F16, "contig", 3),
    (2, 16, 8, 129, 128, BF16, BF16, "hf", 2),
    (1, 1, 1, 1, 128, F32, F32, "hf", 1),
]


def dev_all(dev, *ts):
    return [t.to(dev) for t in ts]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"B{c[0]}H{c[1]}/{c[2]}S{c[3]}D{c[4]}-{c[5]}-{c[7]}")
def test_qk_norm_rope_fwd_bwd(dev, case):
    from metal_liger_amd import hip_ops
    B, Hq, Hk, S, D, dtype, wdtype, layout, tb = case
    eps = 1e-6
    q, k, wq, wk, cos, sin = make_inputs(B, Hq, Hk, S, D, dtype, wdtype, layout, tb, 300 + D)
    c4, s4 = cos.unsqueeze(1), sin.unsqueeze(1)
    gq, gk, gwq, gwk, gc, gs = dev_all(dev, q, k, wq, wk, c4, s4)
    oq, ok = hip_ops.qk_norm_rope_fwd(gq, gk, gwq, gwk, gc, gs, eps)
    assert oq.dtype == dtype and oq.shape == q.shape
    assert oq.transpose(1, 2).is_contiguous()                     # [B, S, H, D] memory
    for out, x, w, name in ((oq, q, wq, "q out"), (ok, k, wk, "k out")):
        exact = ref.qk_norm_rope_forward(x.float(), w.float(), eps, c4.float(), s4.float())
        assert_close(out, exact, name, dtype)
        if wdtype == dtype:
            # transformers' sequence (with an fp32 weight it would promote the
            # output to fp32; the fused op keeps x's dtype)
            hf = ref.qk_norm_rope_forward(x, w, eps, c4, s4)
            assert hf.dtype == dtype
            assert rel_fro(out, exact) <= rel_fro(hf, exact) + 1e-6, name

    # upstream grads in the other layout than the inputs
    other = "contig" if layout == "hf" else "hf"
    dyq = make_inputs(B, Hq, Hk, S, D, dtype, wdtype, other, tb, 400 + D)[0]
    dyk = make_inputs(B, Hq, Hk, S, D, dtype, wdtype, other, tb, 500 + D)[1]
    dq, dk, dwq, dwk = hip_ops.qk_norm_rope_bwd(gq, gk, gwq, gwk, gc, gs, eps, *dev_all(dev, dyq, dyk))
    rq, rwq = ref.qk_norm_rope_backward(q, wq, eps, c4, s4, dyq)
    rk, rwk = ref.qk_norm_rope_backward(k, wk, eps, c4, s4, dyk)
    assert dq.dtype == dtype and dwq.dtype == wdtype
    assert_close(dq, rq, "dq", dtype)
    assert_close(dk, rk, "dk", dtype)
    assert_close(dwq, rwq, "dwq", wdtype)
    assert_close(dwk, rwk, "dwk", wdtype)

    # without weight gradients, dx is unchanged
    dq2, dk2, n1, n2 = hip_ops.qk_norm_rope_bwd(gq, gk, gwq, gwk, gc, gs, eps,
                                                *dev_all(dev, dyq, dyk), need_dq_weight=False,
                                                need_dk_weight=False)
    assert n1 is None and n2 is None
    assert torch.equal(dq2, dq) and torch.equal(dk2, dk)


def test_qk_norm_rope_dw_deterministic(dev):
    from metal_liger_amd import hip_ops
    q, k, wq, wk, cos, sin = make_inputs(2, 8, 4, 300, 128, BF16, F32, "hf", 2, 77)
    args = dev_all(dev, q, k, wq, wk, cos.unsqueeze(1), sin.unsqueeze(1))
    dys = dev_all(dev, seeded((2, 8, 300, 128), 78, BF16), seeded((2, 4, 300, 128), 79, BF16))
    first = hip_ops.qk_norm_rope_bwd(*args, 1e-6, *dys)
    for _ in range(3):
        again = hip_ops.qk_norm_rope_bwd(*args, 1e-6, *dys)
        assert all(torch.equal(a, b) for a, b in zip(first, again))


def test_qk_norm_rope_autograd_function(dev):
    """The autograd Function through apply_fused_qk_norm_rope (HF-shaped
    tables [B, S, D], norm modules) against fp32 autograd of the oracle."""
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm

    from metal_liger_amd.ops.fused_qk_norm_rope import apply_fused_qk_norm_rope
    B, Hq, Hk, S, D = 2, 4, 2, 40, 64
    q, k, wq, wk, cos, sin = make_inputs(B, Hq, Hk, S, D, BF16, BF16, "hf", 2, 90)
    qn, kn = Qwen3RMSNorm(D, eps=1e-6).to(BF16), Qwen3RMSNorm(D, eps=1e-6).to(BF16)
    with torch.no_grad():
        qn.weight.copy_(wq)
        kn.weight.copy_(wk)
    qn, kn = qn.to(dev), kn.to(dev)
    gq = q.to(dev).requires_grad_(True)
    gk = k.to(dev).requires_grad_(True)
    oq, ok = apply_fused_qk_norm_rope(gq, gk, qn, kn, cos.to(dev), sin.to(dev))
    dyq, dyk = seeded(oq.shape, 91, BF16), seeded(ok.shape, 92, BF16)
    (oq.float() * dyq.to(dev).float()).sum().add((ok.float() * dyk.to(dev).float()).sum()).backward()

    xs = [t.float().requires_grad_(True) for t in (q, k)]
    ws = [t.float().requires_grad_(True) for t in (wq, wk)]
    c4, s4 = cos.float().unsqueeze(1), sin.float().unsqueeze(1)
    for x, w, dy in zip(xs, ws, (dyq, dyk)):
        ref.qk_norm_rope_forward(x, w, 1e-6, c4, s4).backward(dy.float())
    assert_close(gq.grad, xs[0].grad, "dq", BF16)
    assert_close(gk.grad, xs[1].grad, "dk", BF16)
    assert_close(qn.weight.grad, ws[0].grad, "dwq", BF16)
    assert_close(kn.weight.grad, ws[1].grad, "dwk", BF16)


def test_qk_norm_rope_config_shape(dev):
    """Qwen3 attention at the RoPE config: q [4, 16, 2048, 128], k [4, 8, 2048,
    128] bf16 as HF's transposed views, theta 1e6 tables (bf16, duplicated
    halves), against the oracle evaluated in fp32 on the GPU; the backward's
    dx is checked the same way and the rotation's norm-preservation holds."""
    from metal_liger_amd import hip_ops
    B, Hq, Hk, S, D = 4, 16, 8, 2048, 128
    q = seeded((B, S, Hq, D), 11, BF16).to(dev).transpose(1, 2)
    k = seeded((B, S, Hk, D), 12, BF16).to(dev).transpose(1, 2)
    wq = seeded((D,), 13, BF16, 0.1, 1.0).to(dev)
    wk = seeded((D,), 14, BF16, 0.1, 1.0).to(dev)
    pos = torch.arange(S).unsqueeze(0).expand(B, S)
    cos, sin = ref.rope_tables(pos, D, 1e6)
    c4, s4 = cos.to(BF16).unsqueeze(1).to(dev), sin.to(BF16).unsqueeze(1).to(dev)
    oq, ok = hip_ops.qk_norm_rope_fwd(q, k, wq, wk, c4, s4, 1e-6)
    for out, x, w in ((oq, q, wq), (ok, k, wk)):
        want = ref.qk_norm_rope_forward(x.float(), w.float(), 1e-6, c4.float(), s4.float())
        assert_close(out.float(), want, "config fwd", BF16)
    dyq = seeded((B, Hq, S, D), 15, BF16).to(dev)
    dyk = seeded((B, Hk, S, D), 16, BF16).to(dev)
    dq, dk, dwq, dwk = hip_ops.qk_norm_rope_bwd(q, k, wq, wk, c4, s4, 1e-6, dyq, dyk)
    for got, x, w, dy, gw in ((dq, q, wq, dyq, dwq), (dk, k, wk, dyk, dwk)):
        rdx, rdw = ref.qk_norm_rope_backward(x, w, 1e-6, c4, s4, dy)
        assert_close(got.float(), rdx, "config dx", BF16)
        assert_close(gw.float(), rdw, "config dw", BF16)
