"""torch.compile compatibility of the fused ops (the intent of the reference's
_torch_library.py:1-13, carried to every fused op).

* torch.library.opcheck on every metal_liger_amd:: custom op with real
  inputs: the schema (declared mutation only), the fake kernel against the
  real kernel's output metadata (shapes, dtypes, strides), and AOT dispatch.
* torch.compile(fullgraph=True, backend="aot_eager") of forward + backward
  through each fused autograd Function: no graph break, and the same values
  and gradients as eager (the same kernels run: equal up to a last bit).
"""

import pytest
import torch

from tests.parity import seeded

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
CHECKS = ("test_schema", "test_faketensor", "test_aot_dispatch_dynamic")


def _ops():
    import metal_liger_amd._custom_ops  # noqa: F401  (registers the ops)
    return torch.ops.metal_liger_amd


def _bf(shape, seed, dev, scale=1.0):
    return seeded(shape, seed, BF, scale=scale).to(dev)


def test_opcheck_elementwise_ops(dev):
    ops = _ops()
    x = seeded((64, 256), 1).to(dev)
    w = seeded((256,), 2, scale=0.1, shift=1.0).to(dev)
    y, rrms = ops.rms_norm_fwd(x, w, 1e-6)
    torch.library.opcheck(ops.rms_norm_fwd.default, (x, w, 1e-6), test_utils=CHECKS)
    torch.library.opcheck(ops.rms_norm_bwd.default, (x, w, x.clone(), rrms, 1e-6), test_utils=CHECKS)
    r = seeded((64, 256), 5).to(dev)
    torch.library.opcheck(ops.rms_norm_add_fwd.default, (x, r, w, 1e-6), test_utils=CHECKS)
    _, total, rrms2 = ops.rms_norm_add_fwd(x, r, w, 1e-6)
    torch.library.opcheck(ops.rms_norm_add_bwd.default, (total, w, x.clone(), r.clone(), rrms2, 1e-6),
                          test_utils=CHECKS)
    g, u = _bf((32, 512), 3, dev), _bf((32, 512), 4, dev)
    torch.library.opcheck(ops.swiglu_fwd.default, (g, u), test_utils=CHECKS)
    torch.library.opcheck(ops.swiglu_bwd.default, (g, u, g.clone()), test_utils=CHECKS)


def test_opcheck_rope_ops(dev):
    ops = _ops()
    # HF's transposed views and contiguous tensors, with and without k
    q = _bf((2, 33, 4, 64), 5, dev).transpose(1, 2)
    k = _bf((2, 4, 33, 64), 6, dev)
    cos = _bf((33, 64), 7, dev)
    sin = _bf((33, 64), 8, dev)
    pos = torch.arange(33, device=dev)
    inv = torch.rand(32, device=dev)
    for args in ((q, k, cos, sin, 1.0), (q, None, cos.float(), sin.float(), -1.0)):
        torch.library.opcheck(ops.rope_table.default, args, test_utils=CHECKS)
    for args in ((q, k, pos, inv, 1.0), (k, None, pos, inv, -1.0)):
        torch.library.opcheck(ops.rope_pos.default, args, test_utils=CHECKS)
    qh = _bf((2, 17, 4, 128), 9, dev).transpose(1, 2)
    kh = _bf((2, 17, 2, 128), 10, dev).transpose(1, 2)
    wq = seeded((128,), 11, BF, 0.1, 1.0).to(dev)
    wk = seeded((128,), 12, BF, 0.1, 1.0).to(dev)
    c4 = _bf((2, 1, 17, 128), 13, dev)
    s4 = _bf((2, 1, 17, 128), 14, dev)
    torch.library.opcheck(ops.qk_norm_rope_fwd.default, (qh, kh, wq, wk, c4, s4, 1e-6),
                          test_utils=CHECKS)
    dq, dk = _bf((2, 4, 17, 128), 15, dev), _bf((2, 2, 17, 128), 16, dev)
    for need in (True, False):
        torch.library.opcheck(ops.qk_norm_rope_bwd.default,
                              (qh, kh, wq, wk, c4, s4, 1e-6, dq, dk, need, need), test_utils=CHECKS)


def test_opcheck_flce_ops(dev):
    ops = _ops()
    N, H, V = 64, 128, 1000
    h = _bf((N, H), 20, dev)
    w = _bf((V, H), 21, dev, 0.05)
    lab = torch.randint(0, V, (N,), generator=torch.Generator().manual_seed(22)).to(dev)
    lab[::7] = -100
    for need_h, need_w in ((True, True), (True, False)):
        torch.library.opcheck(ops.flce_fwd_grad.default, (h, w, lab, None, -100, need_h, need_w),
                              test_utils=CHECKS)
    loss, lse, n_valid, dh, dw = ops.flce_fwd_grad(h, w, lab, None, -100, True, True)
    g = torch.full((), 0.5, device=dev)
    torch.library.opcheck(ops.flce_scale_grads.default, (g, dh.clone(), dw.clone()),
                          test_utils=CHECKS)
    torch.library.opcheck(ops.flce_bwd.default, (h, w, lab, None, -100, lse, n_valid, g, 256,
                                                 True, True), test_utils=CHECKS)


def test_opcheck_lora_ops(dev):
    ops = _ops()
    N, IN, r = 96, 128, 16
    x = _bf((N, IN), 30, dev)
    W = [_bf((o, IN), 31 + i, dev, 0.05) for i, o in enumerate((128, 64, 64))]
    A = _bf((3 * r, IN), 35, dev, 0.25)
    B = [_bf((o, r), 36 + i, dev, 0.05) for i, o in enumerate((128, 64, 64))]
    xa = ops.lora_xa(x, A)
    torch.library.opcheck(ops.linear_bf16.default, (x, W[0]), test_utils=CHECKS)
    torch.library.opcheck(ops.lora_xa.default, (x, A), test_utils=CHECKS)
    torch.library.opcheck(ops.lora_linear_out.default, (x, W[0], xa[:, :r].contiguous(), B[0]),
                          test_utils=CHECKS)
    dys = [_bf((N, o), 40 + i, dev) for i, o in enumerate((128, 64, 64))]
    torch.library.opcheck(ops.lora_qkv_bwd.default, (x, dys, W, A, B, [2.0, 2.0, 2.0], xa, r),
                          test_utils=CHECKS)
    torch.library.opcheck(ops.lora_linear_bwd.default,
                          (x, dys[0], W[0], A[:r].contiguous(), B[0], 2.0, xa[:, :r].contiguous(), r),
                          test_utils=CHECKS)
    I = 256  # noqa: E741
    wg, wu = _bf((I, IN), 50, dev, 0.05), _bf((I, IN), 51, dev, 0.05)
    wd = _bf((IN, I), 52, dev, 0.05)
    a_gu, a_d = _bf((2 * r, IN), 53, dev, 0.25), _bf((r, I), 54, dev, 0.25)
    bg, bu, bd = _bf((I, r), 55, dev, 0.05), _bf((I, r), 56, dev, 0.05), _bf((IN, r), 57, dev, 0.05)
    xa_gu = ops.lora_xa(x, a_gu)
    gate = ops.lora_linear_out(x, wg, xa_gu[:, :r].contiguous(), bg)
    up = ops.lora_linear_out(x, wu, xa_gu[:, r:].contiguous(), bu)
    h = ops.swiglu_fwd(gate, up)
    ha_d = ops.lora_xa(h, a_d)
    torch.library.opcheck(ops.lora_mlp_bwd.default,
                          (x, gate, up, h, _bf((N, IN), 58, dev), wg, wu, wd, a_gu, a_d, bg, bu, bd,
                           [2.0, 2.0, 2.0], xa_gu, ha_d, r), test_utils=CHECKS)


def _compiled_matches_eager(fn, leaves):
    """fullgraph compile (aot_eager) of fn(*leaves).backward(); returns after
    comparing outputs and leaf gradients with eager, bit for bit."""
    import torch._dynamo
    torch._dynamo.reset()

    def run(f):
        for t in leaves:
            t.grad = None
        out = f(*leaves)
        out.backward()
        return out.detach().clone(), [t.grad.clone() for t in leaves]

    want, want_g = run(fn)
    got, got_g = run(torch.compile(fn, fullgraph=True, backend="aot_eager"))

    def same(a, b):  # the same kernels run; allow a last-bit difference from layouts
        return torch.equal(a, b) or (a - b).abs().max() <= 1e-3 * b.abs().max()

    assert same(got, want), (got.item(), want.item())
    for i, (a, b) in enumerate(zip(got_g, want_g)):
        assert same(a.float(), b.float()), f"grad of leaf {i}"


def test_compile_elementwise_and_rope(dev):
    from metal_liger_amd import MetalLigerRMSNorm
    from metal_liger_amd.ops.fused_add_rms_norm import fused_add_rms_norm
    from metal_liger_amd.ops.fused_qk_norm_rope import _FusedQKNormRoPEFunction
    from metal_liger_amd.ops.fused_rope import apply_fused_rotary, apply_fused_rotary_inline
    from metal_liger_amd.ops.fused_swiglu import fused_swiglu
    norm = MetalLigerRMSNorm(256).to(dev)
    x = _bf((4, 16, 256), 60, dev).requires_grad_(True)
    g = _bf((4, 16, 256), 61, dev).requires_grad_(True)
    q = _bf((2, 4, 32, 64), 62, dev).requires_grad_(True)
    k = _bf((2, 2, 32, 64), 63, dev).requires_grad_(True)
    cos, sin = _bf((32, 64), 64, dev), _bf((32, 64), 65, dev)
    pos = torch.arange(32, device=dev)
    wq = seeded((64,), 66, BF, 0.1, 1.0).to(dev).requires_grad_(True)
    wk = seeded((64,), 67, BF, 0.1, 1.0).to(dev).requires_grad_(True)

    def f(x, g, q, k, wq, wk):
        y, total = fused_add_rms_norm(norm(x), g, norm)
        y = fused_swiglu(y, total)
        qa, ka = apply_fused_rotary(q, k, cos, sin)
        qb, kb = apply_fused_rotary_inline(qa, ka, pos, theta=1e4)
        qc, kc = _FusedQKNormRoPEFunction.apply(qb, kb, wq, wk, cos, sin, 1e-6)
        return y.float().square().mean() + qc.float().square().mean() + kc.float().mean()

    _compiled_matches_eager(f, [x, g, q, k, wq, wk])


def test_compile_flce_and_lora(dev):
    from metal_liger_amd.ops.fused_linear_cross_entropy import _FusedLinearCrossEntropyFunction
    from metal_liger_amd.ops.fused_lora import _LoRA_MLP, _LoRA_QKV, _LoRA_W
    N, H, V, r = 128, 128, 512, 16
    X = _bf((N, H), 70, dev).requires_grad_(True)
    lab = torch.randint(0, V, (N,), generator=torch.Generator().manual_seed(71)).to(dev)
    Wlm = _bf((V, H), 72, dev, 0.05).requires_grad_(True)

    def adapter(out_f, in_f, seed):
        return (_bf((out_f, in_f), seed, dev, 0.05), _bf((r, in_f), seed + 1, dev, 0.25).requires_grad_(True),
                _bf((out_f, r), seed + 2, dev, 0.05).requires_grad_(True), 2.0)

    qkv = [adapter(o, H, 80 + 5 * i) for i, o in enumerate((H, 64, 64))]
    mlp = [adapter(256, H, 100), adapter(256, H, 105), adapter(H, 256, 110)]
    o = adapter(H, H, 120)
    leaves = [X, Wlm] + [t for a in qkv + mlp + [o] for t in a[1:3]]

    def f(X, Wlm, *ab):
        qa = [(W, ab[2 * i], ab[2 * i + 1], s) for i, (W, _, _, s) in enumerate(qkv)]
        ma = [(W, ab[6 + 2 * i], ab[7 + 2 * i], s) for i, (W, _, _, s) in enumerate(mlp)]
        Q, K, V_ = _LoRA_QKV.apply(X, *[t for a in qa for t in a])
        m = _LoRA_MLP.apply(X, *[t for a in ma for t in a])
        hid = _LoRA_W.apply(Q + m, o[0], ab[12], ab[13], o[3])
        loss = _FusedLinearCrossEntropyFunction.apply(hid, Wlm, lab, None, -100, 8192)
        return loss + K.float().mean() + V_.float().mean()

    _compiled_matches_eager(f, leaves)
