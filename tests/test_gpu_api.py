"""GPU coverage of the thin pieces of the drop-in API against the oracle:
the torch.library ops registered under the reference's schemas
(_torch_library.py:44-76), MetalLigerSwiGLU.forward (ops/fused_swiglu.py:59-75)
with plain projections, MetalLigerRoPE (ops/fused_rope.py:78-107) feeding
apply_fused_rotary, _lora_linear (ops/fused_lora.py:69-82), and the LoRA
Functions on strided inputs (column slices, a row-broadcast gradient)."""

import pytest
import torch
import torch.nn.functional as F

from oracle import reference_ops as ref
from tests.parity import assert_close, rel_fro, seeded

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


@pytest.mark.parametrize("dtype", [torch.float32, BF])
def test_torch_library_ops_on_gpu(dev, dtype):
    """torch.ops.metal_liger.{rms_norm,swiglu}_{forward,backward} run the HIP
    kernels on ROCm tensors and match the oracle (rms_cache is fp32
    [tokens], the shape the reference's native op returns)."""
    import metal_liger_amd  # noqa: F401  (registers on import)
    ops = torch.ops.metal_liger
    x = seeded((3, 50, 512), 1, dtype)
    w = seeded((512,), 2, dtype, scale=0.1, shift=1.0)
    g = seeded((3, 50, 512), 3, dtype)
    y, cache = ops.rms_norm_forward(x.to(dev), w.to(dev), 1e-6, "")
    ry, rr = ref.rms_norm_forward(x, w, 1e-6)
    assert y.is_cuda and cache.shape == (150,) and cache.dtype == torch.float32
    assert_close(y, ry, "rms_norm_forward y")
    assert_close(cache, rr.reshape(-1), "rms_norm_forward cache")
    dx, dw = ops.rms_norm_backward(x.to(dev), w.to(dev), g.to(dev), 1e-6, "")
    rdx, rdw = ref.rms_norm_backward(x, w, rr, g)
    assert_close(dx, rdx, "rms_norm_backward dx")
    assert_close(dw, rdw, "rms_norm_backward dw")

    gate = seeded((64, 384), 4, dtype)
    up = seeded((64, 384), 5, dtype)
    dy = seeded((64, 384), 6, dtype)
    out = ops.swiglu_forward(gate.to(dev), up.to(dev), "")
    ro, sig = ref.swiglu_forward(gate, up)
    assert_close(out, ro, "swiglu_forward")
    dg, du = ops.swiglu_backward(gate.to(dev), up.to(dev), dy.to(dev), "")
    rdg, rdu = ref.swiglu_backward(gate, up, sig, dy)
    assert_close(dg, rdg, "swiglu_backward dgate")
    assert_close(du, rdu, "swiglu_backward dup")


class _MLP(torch.nn.Module):
    def __init__(self, h, i):
        super().__init__()
        self.gate_proj = torch.nn.Linear(h, i, bias=False)
        self.up_proj = torch.nn.Linear(h, i, bias=False)
        self.down_proj = torch.nn.Linear(i, h, bias=False)


def test_swiglu_module_forward_and_backward(dev):
    """MetalLigerSwiGLU over plain bf16 projections: down(silu(gate x) * up x)
    with the activation fused, against the oracle's SwiGLU between the same
    projections evaluated in fp32 from the same bf16 weights (bf16 bar, the
    projections being hipBLAS bf16 products on the GPU side)."""
    from metal_liger_amd import MetalLigerSwiGLU
    torch.manual_seed(0)
    mlp = _MLP(256, 768).to(BF)
    mod = MetalLigerSwiGLU(mlp).to(dev)
    assert mod.gate_proj is mlp.gate_proj and "fused=MetalLiger" in repr(mod)
    x = seeded((4, 40, 256), 7, BF)
    dy = seeded((4, 40, 256), 8, BF)
    xd = x.to(dev).requires_grad_(True)
    out = mod(xd)
    out.backward(dy.to(dev))

    wg, wu, wd = (p.detach().float().cpu().requires_grad_(True)
                  for p in (mlp.gate_proj.weight, mlp.up_proj.weight, mlp.down_proj.weight))
    xr = x.float().requires_grad_(True)
    gate, up = F.linear(xr, wg), F.linear(xr, wu)
    act = F.silu(gate) * up
    rout = F.linear(act, wd)
    rout.backward(dy.float())
    assert out.dtype == BF
    assert_close(out, rout.to(BF), "module out", dtype=BF)
    assert_close(xd.grad, xr.grad.to(BF), "module dx", dtype=BF)
    for p, r in zip((mod.gate_proj.weight, mod.up_proj.weight, mod.down_proj.weight), (wg, wu, wd)):
        assert rel_fro(p.grad, r.grad) <= 2e-2


def test_rope_module_feeds_fused_rotary(dev):
    """MetalLigerRoPE passes HF's rotary module through (same cos/sin, same
    inv_freq buffer); its tables drive apply_fused_rotary, which matches the
    oracle's rotation forward and backward."""
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding

    from metal_liger_amd import MetalLigerRoPE
    from metal_liger_amd.ops.fused_rope import apply_fused_rotary
    cfg = Qwen3Config(hidden_size=512, num_attention_heads=4, head_dim=128, rope_theta=1e6,
                      max_position_embeddings=256)
    hf = Qwen3RotaryEmbedding(cfg).to(dev)
    mod = MetalLigerRoPE(hf)
    assert torch.equal(mod.inv_freq, hf.inv_freq)
    q = seeded((2, 4, 96, 128), 9, BF)
    k = seeded((2, 2, 96, 128), 10, BF)
    pos = torch.arange(96).unsqueeze(0).expand(2, -1).to(dev)
    cos, sin = mod(q.to(dev), pos)
    hcos, hsin = hf(q.to(dev), pos)
    assert torch.equal(cos, hcos) and torch.equal(sin, hsin)
    qd = q.to(dev).requires_grad_(True)
    kd = k.to(dev).requires_grad_(True)
    c4, s4 = cos.unsqueeze(1), sin.unsqueeze(1)
    qo, ko = apply_fused_rotary(qd, kd, c4, s4)
    gq, gk = seeded(q.shape, 11, BF), seeded(k.shape, 12, BF)
    torch.autograd.backward([qo, ko], [gq.to(dev), gk.to(dev)])
    c4c, s4c = c4.cpu(), s4.cpu()
    assert_close(qo, ref.rope_forward(q, c4c, s4c), "rope q")
    assert_close(ko, ref.rope_forward(k, c4c, s4c), "rope k")
    assert_close(qd.grad, ref.rope_backward(gq, c4c, s4c, q.dtype), "rope dq")
    assert_close(kd.grad, ref.rope_backward(gk, c4c, s4c, k.dtype), "rope dk")


@pytest.mark.parametrize("with_lora", [True, False])
def test_lora_linear_helper(dev, with_lora):
    """_lora_linear: X W^T + s (X A^T) B^T on the MFMA engine (X W^T alone
    when A or B is None) against the oracle."""
    from metal_liger_amd.ops.fused_lora import _lora_linear
    X = seeded((3, 70, 256), 13, BF)
    W = seeded((384, 256), 14, BF, scale=0.05)
    A = seeded((16, 256), 15, BF, scale=0.25) if with_lora else None
    B = seeded((384, 16), 16, BF, scale=0.05) if with_lora else None
    dev_args = [t.to(dev) if t is not None else None for t in (X, W, A, B)]
    out = _lora_linear(*dev_args, 2.0)
    assert out.shape == (3, 70, 384) and out.dtype == BF
    want = ref.lora_linear(X.float(), W.float(), A.float() if with_lora else None,
                           B.float() if with_lora else None, 2.0)
    assert_close(out, want.to(BF), "_lora_linear", dtype=BF)


def test_lora_functions_strided_inputs(dev):
    """The LoRA backward kernels take dense rows: a column-sliced X (row
    stride wider than its width) and a row-broadcast upstream gradient
    (stride 0) give the same results as their dense copies."""
    from metal_liger_amd.ops.fused_lora import _LoRA_QKV, _LoRA_W
    N, IN, OUT, r = 96, 128, 64, 16
    big = seeded((N, IN + 64), 17, BF).to(dev)
    Xs = big[:, :IN]
    assert Xs.stride(0) == IN + 64
    params = [(seeded((OUT, IN), 20 + i, BF, 0.05).to(dev), seeded((r, IN), 30 + i, BF, 0.25).to(dev),
               seeded((OUT, r), 40 + i, BF, 0.05).to(dev), 2.0) for i in range(3)]
    row = seeded((1, OUT), 18, BF).to(dev)
    dy_b = row.expand(N, OUT)
    assert dy_b.stride(0) == 0

    def run(X, dy, fn, ps):
        Xd = X.detach().requires_grad_(True)
        leaves, args = [], []
        for W, A, B, s in ps:
            Ad, Bd = A.clone().requires_grad_(True), B.clone().requires_grad_(True)
            leaves += [Ad, Bd]
            args += [W, Ad, Bd, s]
        outs = fn(Xd, *args)
        outs = outs if isinstance(outs, tuple) else (outs,)
        torch.autograd.backward(outs, [dy] * len(outs))
        return [o.detach() for o in outs] + [Xd.grad] + [t.grad for t in leaves]

    for fn, ps in ((_LoRA_QKV.apply, params), (_LoRA_W.apply, params[:1])):
        got = run(Xs, dy_b, fn, ps)
        want = run(Xs.contiguous(), dy_b.contiguous(), fn, ps)
        for a, b in zip(got, want):
            assert torch.equal(a, b)
