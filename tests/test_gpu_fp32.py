"""GPU parity of the fp32 paths against the oracle at the fp32 bar (rtol
1e-5 relative to the tensor's scale, tests/parity.py): the fp32
matrix-core GEMM (v_mfma_f32_32x32x2_f32), the LoRA Functions with fp32
activations (the reference's own test runs them in fp32,
tests/test_fused_ops.py:21, :198-242) and the fused linear cross-entropy
with fp32 hidden / weight (its vocabulary-chunked schedule,
ops/fused_linear_cross_entropy.py:39-185), including sizes that are not
multiples of 8; fp16 activations go through the same fp32 products."""

import pytest
import torch

from oracle import reference_ops as ref
from tests.parity import assert_close, seeded

pytestmark = pytest.mark.gpu
F32 = torch.float32


@pytest.mark.parametrize("a_t,b_t", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("M,N,K", [(64, 96, 40), (300, 130, 257), (1, 7, 3), (517, 257, 1031)])
def test_gemm_f32_layouts(dev, a_t, b_t, M, N, K):
    from metal_liger_amd import hip_ops
    a = seeded((K, M) if a_t else (M, K), 1)
    b = seeded((N, K) if b_t else (K, N), 2)
    out = hip_ops.gemm_f32([a.to(dev)], [b.to(dev)], a_t, b_t, 0.5)
    want = 0.5 * ((a.t() if a_t else a).double() @ (b.t() if b_t else b).double())
    assert_close(out, want.float(), f"gemm_f32 {M}x{N}x{K} a_t={a_t} b_t={b_t}")


def test_gemm_f32_segments_and_strides(dev):
    """K-concatenated segments of different lengths (one empty), a
    column-sliced operand and an odd leading dimension."""
    from metal_liger_amd import hip_ops
    big = seeded((200, 91), 3)
    a0, a1, a2 = big[:, :37], seeded((200, 0), 4), seeded((200, 19), 5)
    b0, b1, b2 = seeded((37, 66), 6), seeded((0, 66), 7), seeded((19, 66), 8)
    out = hip_ops.gemm_f32([t.to(dev) for t in (a0, a1, a2)], [t.to(dev) for t in (b0, b1, b2)])
    want = a0.double() @ b0.double() + a2.double() @ b2.double()
    assert_close(out, want.float(), "gemm_f32 segments")


def test_lora_qkv_reference_test_case_fp32(dev):
    """The reference's own case (tests/test_fused_ops.py:198-242) as written:
    fp32 X [2, 16, 128], W/A/B ~N(0, 1), r 8, s 2, loss sum(Q)+sum(K)+sum(V),
    at its tolerances (atol 1e-4, rtol 1e-3) and at the fp32 bar against
    fp64 autograd; W gets no gradient."""
    from metal_liger_amd.ops.fused_lora import _LoRA_QKV
    g = torch.Generator().manual_seed(42)
    X = torch.randn(2, 16, 128, generator=g)
    P = [(torch.randn(128, 128, generator=g), torch.randn(8, 128, generator=g),
          torch.randn(128, 8, generator=g), 2.0) for _ in range(3)]
    Xd = X.to(dev).requires_grad_(True)
    args, leaves = [], []
    for W, A, B, s in P:
        Wd, Ad, Bd = (t.to(dev).requires_grad_(True) for t in (W, A, B))
        leaves.append((Wd, Ad, Bd))
        args += [Wd, Ad, Bd, s]
    Q, K, V = _LoRA_QKV.apply(Xd, *args)
    (Q.sum() + K.sum() + V.sum()).backward()
    Xr = X.double().requires_grad_(True)
    refs = []
    for W, A, B, s in P:
        Ar, Br = A.double().requires_grad_(True), B.double().requires_grad_(True)
        refs.append((Ar, Br, Xr @ W.double().t() + (Xr @ Ar.t()) @ Br.t() * s))
    sum(o.sum() for _, _, o in refs).backward()
    for o, (_, _, ro) in zip((Q, K, V), refs):
        assert torch.allclose(o.cpu().double(), ro, atol=1e-4, rtol=1e-3)
        assert_close(o, ro.float(), "QKV fwd fp32")
    assert torch.allclose(Xd.grad.cpu().double(), Xr.grad, atol=1e-4, rtol=1e-3)
    assert_close(Xd.grad, Xr.grad.float(), "dX fp32")
    for (Wd, Ad, Bd), (Ar, Br, _) in zip(leaves, refs):
        assert Wd.grad is None and Ad.grad.dtype == F32 and Bd.grad.dtype == F32
        assert_close(Ad.grad, Ar.grad.float(), "dA fp32")
        assert_close(Bd.grad, Br.grad.float(), "dB fp32")


def _adapter(out_f, in_f, r, seed, w_std=0.05, a_std=0.25, b_std=0.05):
    return (seeded((out_f, in_f), seed, scale=w_std), seeded((r, in_f), seed + 1, scale=a_std),
            seeded((out_f, r), seed + 2, scale=b_std))


def _run(dev, fn, X, params, dys):
    Xd = X.to(dev).requires_grad_(True)
    args, leaves = [], []
    for W, A, B, s in params:
        Ad, Bd = A.to(dev).requires_grad_(True), B.to(dev).requires_grad_(True)
        leaves.append((Ad, Bd))
        args += [W.to(dev), Ad, Bd, s]
    outs = fn(Xd, *args)
    outs = outs if isinstance(outs, tuple) else (outs,)
    torch.autograd.backward(outs, [d.to(dev) for d in dys])
    return outs, Xd.grad, leaves


@pytest.mark.parametrize("N,IN,OUTS,r", [(77, 100, (96, 40, 40), 7), (300, 256, (256, 128, 128), 16)])
def test_lora_qkv_fp32(dev, N, IN, OUTS, r):
    from metal_liger_amd.ops.fused_lora import _LoRA_QKV
    X = seeded((N, IN), 1)
    params = [(*_adapter(o, IN, r, 10 * i + 2), 2.0) for i, o in enumerate(OUTS)]
    dys = [seeded((N, o), 50 + i) for i, o in enumerate(OUTS)]
    outs, dX, leaves = _run(dev, _LoRA_QKV.apply, X, params, dys)
    flat = [t for p in params for t in p]
    for o, ro in zip(outs, ref.lora_qkv_forward(X, *flat)):
        assert_close(o, ro, "qkv fwd")
    rdX, *rdAB = ref.lora_qkv_backward(X, *dys, *flat)
    assert_close(dX, rdX, "qkv dX")
    for i, (Ad, Bd) in enumerate(leaves):
        assert_close(Ad.grad, rdAB[2 * i], f"qkv dA[{i}]")
        assert_close(Bd.grad, rdAB[2 * i + 1], f"qkv dB[{i}]")


@pytest.mark.parametrize("N,H,I,r", [(48, 100, 260, 8), (200, 256, 768, 16)])
def test_lora_mlp_fp32(dev, N, H, I, r):
    from metal_liger_amd.ops.fused_lora import _LoRA_MLP
    X = seeded((N, H), 5)
    params = [(*_adapter(I, H, r, 80, w_std=0.1), 2.0), (*_adapter(I, H, r, 83, w_std=0.1), 2.0),
              (*_adapter(H, I, r, 86, w_std=0.1), 2.0)]
    dY = seeded((N, H), 90)
    (out,), dX, leaves = _run(dev, _LoRA_MLP.apply, X, params, [dY])
    flat = [t for p in params for t in p]
    rout, gate, up, h = ref.lora_mlp_forward(X, *flat)
    assert_close(out, rout, "mlp out")
    rdX, *rdAB = ref.lora_mlp_backward(X, gate, up, h, dY, *flat)
    assert_close(dX, rdX, "mlp dX")
    for i, (Ad, Bd) in enumerate(leaves):
        assert_close(Ad.grad, rdAB[2 * i], f"mlp dA[{i}]")
        assert_close(Bd.grad, rdAB[2 * i + 1], f"mlp dB[{i}]")


@pytest.mark.parametrize("dtype", [F32, torch.float16])
def test_lora_linear_fp32_and_fp16(dev, dtype):
    """_LoRA_W and _lora_linear with fp32 activations at the fp32 bar; fp16
    activations (products in fp32, outputs rounded to fp16) at the fp16 bar
    against the oracle in fp32."""
    from metal_liger_amd.ops.fused_lora import _LoRA_W, _lora_linear
    N, IN, OUT, r = 130, 72, 200, 12
    X = seeded((N, IN), 3)
    W, A, B = _adapter(OUT, IN, r, 20)
    dY = seeded((N, OUT), 21)
    Xt, Wt, At, Bt, dYt = (t.to(dtype) for t in (X, W, A, B, dY))
    (out,), dX, ((Ad, Bd),) = _run(dev, _LoRA_W.apply, Xt, [(Wt, At, Bt, 2.0)], [dYt])
    assert out.dtype == dtype and dX.dtype == dtype
    Xr, Wr, Ar, Br, dYr = (t.float() for t in (Xt, Wt, At, Bt, dYt))
    rout = ref.lora_linear(Xr, Wr, Ar, Br, 2.0)
    rdX, rdA, rdB = ref.lora_linear_backward(Xr, dYr, Wr, Ar, Br, 2.0)
    assert_close(out, rout.to(dtype), "LoRA_W out", dtype=dtype)
    assert_close(dX, rdX.to(dtype), "LoRA_W dX", dtype=dtype)
    assert_close(Ad.grad.float(), rdA, "LoRA_W dA", dtype=dtype)
    assert_close(Bd.grad.float(), rdB, "LoRA_W dB", dtype=dtype)
    lin = _lora_linear(Xt.to(dev), Wt.to(dev), At.to(dev), Bt.to(dev), 2.0)
    assert lin.dtype == dtype
    assert_close(lin, rout.to(dtype), "_lora_linear", dtype=dtype)


@pytest.mark.parametrize("N,H,V,chunk,bias", [(200, 64, 1000, 256, False), (77, 100, 1001, 300, True),
                                              (64, 128, 4104, 8192, False)])
def test_flce_fp32(dev, N, H, V, chunk, bias):
    """fp32 hidden / weight through the autograd Function (vocabulary chunks
    of `chunk`, a ragged last one; H and V not multiples of 8 in the second
    case), loss at 1e-3 relative, lse and both gradients at the fp32 bar,
    grad_output 0.7."""
    from metal_liger_amd.ops.fused_linear_cross_entropy import _FusedLinearCrossEntropyFunction
    h = seeded((N, H), N)
    w = seeded((V, H), N + 1, scale=0.3)
    b = seeded((V,), N + 2, scale=0.5) if bias else None
    g = torch.Generator().manual_seed(N + 3)
    lab = torch.randint(0, V, (N,), generator=g)
    lab[torch.rand(N, generator=g) < 0.2] = -100
    hd, wd = h.to(dev).requires_grad_(True), w.to(dev).requires_grad_(True)
    loss = _FusedLinearCrossEntropyFunction.apply(hd, wd, lab.to(dev), b.to(dev) if bias else None,
                                                  -100, chunk)
    (loss * 0.7).backward()
    rl, lse, mask = ref.flce_forward(h, w, lab, b, -100, chunk)
    rdh, rdw = ref.flce_backward(h, w, lab, lse, mask, torch.tensor(0.7), b, chunk)
    assert loss.dtype == F32 and hd.grad.dtype == F32 and wd.grad.dtype == F32
    assert abs(loss.item() - rl.item()) <= 1e-5 * abs(rl.item())
    assert_close(hd.grad, rdh, "flce fp32 dH")
    assert_close(wd.grad, rdw, "flce fp32 dW")


def test_flce_fp32_second_backward_and_fp16(dev):
    """retain_graph: the second backward of an fp32 loss recomputes (1.5 +
    2.0 times the unit gradient in .grad); fp16 inputs are upcast to fp32 as
    the reference upcasts, gradients come back in fp16."""
    from metal_liger_amd.ops.fused_linear_cross_entropy import _FusedLinearCrossEntropyFunction
    N, H, V = 96, 64, 904
    h = seeded((N, H), 17)
    w = seeded((V, H), 18, scale=0.3)
    lab = torch.randint(0, V, (N,), generator=torch.Generator().manual_seed(19))
    hd, wd = h.to(dev).requires_grad_(True), w.to(dev).requires_grad_(True)
    loss = _FusedLinearCrossEntropyFunction.apply(hd, wd, lab.to(dev), None, -100, 256)
    loss.backward(torch.tensor(1.5, device=dev), retain_graph=True)
    loss.backward(torch.tensor(2.0, device=dev))
    rl, lse, mask = ref.flce_forward(h, w, lab, None, -100, 256)
    rdh, rdw = ref.flce_backward(h, w, lab, lse, mask, torch.tensor(3.5), None, 256)
    assert_close(hd.grad, rdh, "retain_graph dH")
    assert_close(wd.grad, rdw, "retain_graph dW")
    h16, w16 = h.half(), w.half()
    hd, wd = h16.to(dev).requires_grad_(True), w16.to(dev).requires_grad_(True)
    loss = _FusedLinearCrossEntropyFunction.apply(hd, wd, lab.to(dev), None, -100, 256)
    loss.backward()
    rl, lse, mask = ref.flce_forward(h16.float(), w16.float(), lab, None, -100, 256)
    rdh, rdw = ref.flce_backward(h16.float(), w16.float(), lab, lse, mask, torch.tensor(1.0), None,
                                 256)
    assert hd.grad.dtype == torch.float16
    assert abs(loss.item() - rl.item()) <= 1e-5 * abs(rl.item())
    assert_close(hd.grad, rdh.half(), "fp16 dH", dtype=torch.float16)
    assert_close(wd.grad, rdw.half(), "fp16 dW", dtype=torch.float16)


def test_custom_ops_fp32_opcheck(dev):
    """torch.library.opcheck of the fp32 GEMM and of the fp32 FLCE op (fake
    kernels match the real outputs' shapes and dtypes)."""
    from metal_liger_amd import _custom_ops as ops
    a = seeded((40, 24), 1).to(dev)
    b = seeded((24, 33), 2).to(dev)
    torch.library.opcheck(ops.gemm_f32, ([a], [b], False, False, 1.0))
    h = seeded((32, 24), 3).to(dev)
    w = seeded((100, 24), 4, scale=0.3).to(dev)
    lab = torch.randint(0, 100, (32,), generator=torch.Generator().manual_seed(5)).to(dev)
    torch.library.opcheck(ops.flce_fwd_grad, (h, w, lab, None, -100, True, True, 64))
