"""Pins the CPU oracle (oracle/reference_ops.py) — runs without a GPU.

Each oracle function is checked against something that does not restate its
own formula: fp64 torch autograd of the plain forward expression, a brute
force F.cross_entropy, HF's own rotary module, closed forms and invariants,
and the reference's own test formulas and tolerances
(tests/test_fused_ops.py:31-242 of the reference). The last section plants
plausible mistakes in copies of oracle functions and shows that the pins
catch each one.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import reference_ops as ref

torch.set_num_threads(min(8, torch.get_num_threads()))


def gen(seed):
    return torch.Generator().manual_seed(seed)


def close_scaled(a, b, rel):
    """max |a - b| <= rel * max |b| (fp32 bar with a scale-aware atol)."""
    return (a.double() - b.double()).abs().max() <= rel * b.double().abs().max()


def randn(*shape, seed=0, dtype=torch.float32, scale=1.0):
    return (torch.randn(*shape, generator=gen(seed), dtype=torch.float32) * scale).to(dtype)


# ------------------------------------------------------------------ RMSNorm --


def rms64(x, w, eps):
    x = x.double()
    return x * w.double() / torch.sqrt(x.pow(2).mean(-1, keepdim=True) + eps)


def test_rmsnorm_forward_reference_test_case():
    # reference tests/test_fused_ops.py:37-54 (shapes, formula, tolerances)
    x = randn(2, 128, 2048, seed=1)
    w = randn(2048, seed=2)
    y, _ = ref.rms_norm_forward(x, w, 1e-6)
    var = x.float().pow(2).mean(dim=-1, keepdim=True)
    expect = ((x.float() * torch.rsqrt(var + 1e-6)) * w.float()).to(x.dtype)
    assert torch.allclose(expect, y, atol=1e-5, rtol=1e-4)


def test_rmsnorm_forward_fp64_closed_form():
    x = randn(64, 2048, seed=3)
    w = 1.0 + 0.1 * randn(2048, seed=4)
    y, rrms = ref.rms_norm_forward(x, w, 1e-6)
    y64 = rms64(x, w, 1e-6)
    assert torch.allclose(y.double(), y64, rtol=1e-5, atol=1e-6)
    r64 = 1.0 / torch.sqrt(x.double().pow(2).mean(-1, keepdim=True) + 1e-6)
    assert torch.allclose(rrms.double(), r64, rtol=1e-6)
    assert rrms.dtype == torch.float32 and rrms.shape == (64, 1)


@pytest.mark.parametrize("shape", [(2, 16, 256), (33, 200)])
def test_rmsnorm_backward_vs_fp64_autograd(shape):
    x = randn(*shape, seed=5)
    w = randn(shape[-1], seed=6)
    g = randn(*shape, seed=7)
    eps = 1e-6
    _, rrms = ref.rms_norm_forward(x, w, eps)
    dx, dw = ref.rms_norm_backward(x, w, rrms, g)
    x64 = x.double().requires_grad_(True)
    w64 = w.double().requires_grad_(True)
    rms64(x64, w64, eps).backward(g.double())
    # reference tolerances (tests/test_fused_ops.py:80-83) ...
    assert torch.allclose(dx.double(), x64.grad, atol=1e-4, rtol=1e-3)
    assert torch.allclose(dw.double(), w64.grad, atol=1e-4, rtol=1e-3)
    # ... and the fp32 bar with a scale-aware atol
    assert (dx.double() - x64.grad).abs().max() <= 1e-5 * x64.grad.abs().max()
    assert (dw.double() - w64.grad).abs().max() <= 1e-5 * w64.grad.abs().max()


def test_rmsnorm_backward_invariant():
    # sum_c x_c dx_c = eps * r^3 * sum_c (g w x)_c  (closed form of the VJP)
    eps = 1e-2
    x = randn(16, 96, seed=8).double()
    w = randn(96, seed=9).double()
    g = randn(16, 96, seed=10).double()
    _, r = ref.rms_norm_forward(x, w, eps)
    dx, _ = ref.rms_norm_backward(x, w, r.double(), g)
    lhs = (x * dx.double()).sum(-1)
    rhs = eps * r.double().squeeze(-1) ** 3 * (g * w * x).sum(-1)
    assert torch.allclose(lhs, rhs, rtol=1e-4, atol=1e-10)


def test_rmsnorm_backward_special_case_unit_weight_constant_grad():
    # w = 1, g = c: dx = c*r*(1 - r^2 * x * mean(x)) elementwise, dw = c * sum_rows x*r
    x = randn(8, 32, seed=11).double()
    w = torch.ones(32, dtype=torch.float64)
    g = torch.full((8, 32), 0.5, dtype=torch.float64)
    _, r = ref.rms_norm_forward(x, w, 1e-6)
    r = r.double()
    dx, dw = ref.rms_norm_backward(x, w, r, g)
    # the oracle computes in fp32 (as the reference does): fp32 bar
    assert torch.allclose(dx, 0.5 * r * (1 - r * r * x * x.mean(-1, keepdim=True)), rtol=1e-5)
    assert torch.allclose(dw, 0.5 * (x * r).sum(0), rtol=1e-5)


def test_rmsnorm_bf16_dtypes():
    x = randn(4, 64, seed=12, dtype=torch.bfloat16)
    w = randn(64, seed=13, dtype=torch.bfloat16)
    y, r = ref.rms_norm_forward(x, w, 1e-6)
    dx, dw = ref.rms_norm_backward(x, w, r, randn(4, 64, seed=14, dtype=torch.bfloat16))
    assert y.dtype == dx.dtype == dw.dtype == torch.bfloat16 and r.dtype == torch.float32


# ---------------------------------------------------- residual add + RMSNorm --


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_add_rms_norm_forward_vs_library_routines(dtype):
    # the sum is the exact sum rounded once to the input dtype (torch's add);
    # the norm of that sum is F.rms_norm evaluated in fp64
    x = randn(6, 96, seed=15, dtype=dtype)
    r = randn(6, 96, seed=16, dtype=dtype)
    w = 1.0 + 0.1 * randn(96, seed=17)
    y, s, rrms = ref.add_rms_norm_forward(x, r, w, 1e-6)
    assert s.dtype == y.dtype == dtype and rrms.dtype == torch.float32
    assert torch.equal(s, (x.double() + r.double()).to(dtype))
    want = F.rms_norm(s.double(), (96,), w.double(), 1e-6)
    assert close_scaled(y, want, 1e-5 if dtype == torch.float32 else 8e-3)


def test_add_rms_norm_backward_vs_fp64_autograd():
    """Both outputs receive a gradient (the norm's and the residual
    branch's); x and residual get the same total. A dropped residual-branch
    gradient fails the check."""
    eps = 1e-6
    x, r = randn(5, 64, seed=18), randn(5, 64, seed=19)
    w = 1.0 + 0.1 * randn(64, seed=20)
    gy, gs = randn(5, 64, seed=21), randn(5, 64, seed=22)
    x64, r64, w64 = (t.double().requires_grad_(True) for t in (x, r, w))
    s64 = x64 + r64
    ((rms64(s64, w64, eps) * gy.double()).sum() + (s64 * gs.double()).sum()).backward()
    _, s, rrms = ref.add_rms_norm_forward(x, r, w, eps)
    dx, dw = ref.add_rms_norm_backward(s, w, rrms, gy, gs)
    assert close_scaled(dx, x64.grad, 1e-5) and close_scaled(dx, r64.grad, 1e-5)
    assert close_scaled(dw, w64.grad, 1e-5)
    dropped = ref.rms_norm_backward(s, w, rrms, gy)[0]       # planted: grad_sum left out
    assert not close_scaled(dropped, x64.grad, 1e-2)


# ------------------------------------------------------------------- SwiGLU --


def test_swiglu_forward_reference_test_case():
    # reference tests/test_fused_ops.py:94-109
    g = randn(4, 128, 5120, seed=20)
    u = randn(4, 128, 5120, seed=21)
    out, _ = ref.swiglu_forward(g, u)
    assert torch.allclose(F.silu(g) * u, out, atol=1e-5, rtol=1e-4)


def test_swiglu_backward_vs_fp64_autograd():
    # reference tests/test_fused_ops.py:111-136 shapes, plus the fp32 bar
    g = randn(2, 16, 512, seed=22)
    u = randn(2, 16, 512, seed=23)
    dy = randn(2, 16, 512, seed=24)
    _, sig = ref.swiglu_forward(g, u)
    dg, du = ref.swiglu_backward(g, u, sig, dy)
    g64 = g.double().requires_grad_(True)
    u64 = u.double().requires_grad_(True)
    (F.silu(g64) * u64).backward(dy.double())
    assert torch.allclose(dg.double(), g64.grad, atol=1e-6, rtol=1e-5)
    assert torch.allclose(du.double(), u64.grad, atol=1e-6, rtol=1e-5)


def test_swiglu_special_values():
    g = torch.tensor([0.0, 0.0, 40.0, -40.0])
    u = torch.tensor([1.0, -3.0, 2.0, 2.0])
    dy = torch.tensor([2.0, 1.0, 1.0, 1.0])
    out, sig = ref.swiglu_forward(g, u)
    dg, du = ref.swiglu_backward(g, u, sig, dy)
    assert out[0] == 0 and out[1] == 0
    assert dg[0] == 2.0 * 1.0 / 2 and dg[1] == -3.0 / 2      # dy * u / 2 at g = 0
    assert du[0] == 0 and du[1] == 0
    assert torch.isclose(out[2], torch.tensor(80.0)) and abs(out[3]) < 1e-12  # saturation
    assert torch.isclose(dg[2], torch.tensor(2.0)) and abs(dg[3]) < 1e-12


# --------------------------------------------------------------------- RoPE --


def rope_complex64(x, theta_angles):
    """Rotation as complex multiplication (independent of rotate_half)."""
    h = x.shape[-1] // 2
    z = torch.complex(x[..., :h].double(), x[..., h:].double())
    z = z * torch.polar(torch.ones_like(theta_angles.double()), theta_angles.double())
    return torch.cat((z.real, z.imag), dim=-1)


def test_rope_forward_vs_complex_rotation():
    S, D = 128, 64
    x = randn(2, 8, S, D, seed=30)
    pos = torch.arange(S)
    cos, sin = ref.rope_tables(pos, D, 1e4)
    y = ref.rope_forward(x, cos, sin)
    ang = pos.double().unsqueeze(-1) * ref.rope_inv_freq(D, 1e4).double()
    assert torch.allclose(y.double(), rope_complex64(x, ang), atol=2e-5)
    # reference tests/test_fused_ops.py:156-172 formula
    assert torch.allclose(x * cos + ref.rotate_half(x) * sin, y, atol=1e-6)


def test_rope_tables_match_reference_helper_and_hf():
    # reference helper tests/test_fused_ops.py:146-154 (theta 1e4, repeat(1, 2))
    S, D = 64, 32
    freqs = 1.0 / (10000.0 ** (torch.arange(0, D, 2).float() / D))
    ang = torch.arange(S).float().unsqueeze(1) * freqs.unsqueeze(0)
    c, s = ref.rope_tables(torch.arange(S), D, 1e4)
    assert torch.allclose(c, torch.cos(ang).repeat(1, 2), atol=1e-6)
    assert torch.allclose(s, torch.sin(ang).repeat(1, 2), atol=1e-6)
    # HF's Qwen3 rotary module (independent implementation), theta 1e6
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding
    cfg = Qwen3Config(hidden_size=256, num_attention_heads=2, head_dim=128,
                      rope_theta=1e6, max_position_embeddings=4096)
    rot = Qwen3RotaryEmbedding(cfg)
    pos = torch.arange(2048).unsqueeze(0)
    hc, hs = rot(torch.zeros(1, dtype=torch.float32), pos)
    oc, os_ = ref.rope_tables(pos, 128, 1e6)
    assert torch.equal(hc, oc) and torch.equal(hs, os_)


def test_rope_invariants():
    S, D = 40, 16
    x = randn(1, 3, S, D, seed=31).double()
    # fp64 tables (the fp32 tables are pinned against HF above)
    ang = torch.arange(S).double().unsqueeze(-1) * ref.rope_inv_freq(D, 1e6).double()
    emb = torch.cat((ang, ang), -1)
    cos, sin = emb.cos(), emb.sin()
    y = ref.rope_forward(x, cos, sin)
    h = D // 2
    pair_norm = lambda t: t[..., :h] ** 2 + t[..., h:] ** 2  # noqa: E731
    assert torch.allclose(pair_norm(y), pair_norm(x), rtol=1e-12)
    back = ref.rope_backward(y, cos, sin, torch.float64)       # inverse rotation
    assert torch.allclose(back, x, atol=1e-12)
    assert torch.allclose(y[:, :, 0], x[:, :, 0])              # position 0 = identity


def test_rope_backward_vs_fp64_autograd():
    S, D = 32, 64
    x = randn(1, 4, S, D, seed=32)
    g = randn(1, 4, S, D, seed=33)
    cos, sin = ref.rope_tables(torch.arange(S), D, 1e4)
    dx = ref.rope_backward(g, cos, sin, torch.float32)
    x64 = x.double().requires_grad_(True)
    (x64 * cos.double() + ref.rotate_half(x64) * sin.double()).backward(g.double())
    assert torch.allclose(dx.double(), x64.grad, atol=1e-5)


def test_rope_dtype_promotion():
    x = randn(1, 2, 8, 16, seed=34, dtype=torch.bfloat16)
    cos, sin = ref.rope_tables(torch.arange(8), 16, 1e4)
    assert ref.rope_forward(x, cos, sin).dtype == torch.float32
    assert ref.rope_forward(x, cos.bfloat16(), sin.bfloat16()).dtype == torch.bfloat16


# ------------------------------------------------ q/k head-dim norm + RoPE --


def _hf_qk_norm_rope(x, weight, eps, cos, sin):
    """transformers' own modules: Qwen3RMSNorm, then apply_rotary_pos_emb."""
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm, apply_rotary_pos_emb
    norm = Qwen3RMSNorm(x.shape[-1], eps=eps).to(weight.dtype)
    with torch.no_grad():
        norm.weight.copy_(weight)
    n = norm(x)
    y, _ = apply_rotary_pos_emb(n, n, cos, sin, unsqueeze_dim=1)
    return y


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_qk_norm_rope_forward_matches_transformers(dtype):
    B, H, S, D = 2, 3, 17, 64
    x = randn(B, S, H, D, seed=150, dtype=dtype).transpose(1, 2)     # HF's transposed view
    w = (1.0 + 0.1 * randn(D, seed=151)).to(dtype)
    cos, sin = ref.rope_tables(torch.arange(S).unsqueeze(0).expand(B, S), D, 1e6)
    cos, sin = cos.to(dtype), sin.to(dtype)                           # the rotary module's cast
    y = ref.qk_norm_rope_forward(x, w, 1e-6, cos.unsqueeze(1), sin.unsqueeze(1))
    assert y.dtype == dtype
    assert torch.equal(y, _hf_qk_norm_rope(x, w, 1e-6, cos, sin))


def test_qk_norm_rope_backward_vs_fp64_autograd():
    B, H, S, D = 2, 2, 9, 32
    x = randn(B, H, S, D, seed=152)
    w = 1.0 + 0.1 * randn(D, seed=153)
    # generic tables (halves not duplicated), so both sin halves matter
    cos, sin = randn(B, 1, S, D, seed=154), randn(B, 1, S, D, seed=155)
    g = randn(B, H, S, D, seed=156)
    dx, dw = ref.qk_norm_rope_backward(x, w, 1e-6, cos, sin, g)
    x64 = x.double().requires_grad_(True)
    w64 = w.double().requires_grad_(True)
    ref.qk_norm_rope_forward(x64, w64, 1e-6, cos.double(), sin.double()).backward(g.double())
    assert close_scaled(dx, x64.grad, 1e-5)
    assert close_scaled(dw, w64.grad, 1e-5)


def test_qk_norm_rope_invariants():
    S, D = 12, 16
    x = randn(1, 2, S, D, seed=157).double()
    w = torch.ones(D, dtype=torch.float64)
    # identity rotation: y is x / rms(x)
    y = ref.qk_norm_rope_forward(x, w, 0.0, torch.ones(S, D, dtype=torch.float64),
                                 torch.zeros(S, D, dtype=torch.float64))
    assert torch.allclose(y.pow(2).mean(-1), torch.ones(1, 2, S, dtype=torch.float64))
    # a rotation (duplicated-half tables) keeps each pair's norm
    ang = torch.arange(S).double().unsqueeze(-1) * ref.rope_inv_freq(D, 1e4).double()
    emb = torch.cat((ang, ang), -1)
    y2 = ref.qk_norm_rope_forward(x, w, 0.0, emb.cos(), emb.sin())
    h = D // 2
    assert torch.allclose(y2[..., :h] ** 2 + y2[..., h:] ** 2, y[..., :h] ** 2 + y[..., h:] ** 2)
    # the backward of a pure rotation at unit weight is the inverse rotation
    # followed by the norm's backward: dx is orthogonal to x
    dx, _ = ref.qk_norm_rope_backward(x, w, 0.0, emb.cos(), emb.sin(), randn(1, 2, S, D, seed=158))
    assert torch.allclose((dx.double() * x).sum(-1), torch.zeros(1, 2, S, dtype=torch.float64),
                          atol=1e-5)


# ----------------------------------------------- fused linear cross-entropy --


def flce_inputs(N=48, H=24, V=1000, seed=40, ignore_frac=0.25):
    h = randn(N, H, seed=seed)
    w = randn(V, H, seed=seed + 1, scale=0.3)
    lab = torch.randint(0, V, (N,), generator=gen(seed + 2))
    drop = torch.rand(N, generator=gen(seed + 3)) < ignore_frac
    lab[drop] = -100
    return h, w, lab


@pytest.mark.parametrize("chunk", [256, 1000, 4096, 333])
def test_flce_vs_cross_entropy_fp64(chunk):
    h, w, lab = flce_inputs()
    loss, lse, mask = ref.flce_forward(h, w, lab, None, -100, chunk)
    h64 = h.double().requires_grad_(True)
    w64 = w.double().requires_grad_(True)
    ce = F.cross_entropy(h64 @ w64.t(), lab, ignore_index=-100, reduction="mean")
    ce.backward()
    assert loss.dtype == torch.float32
    assert abs(loss.item() - ce.item()) <= 1e-6 * abs(ce.item())
    assert torch.allclose(lse.double(), torch.logsumexp(h.double() @ w.double().t(), -1), rtol=1e-6)
    dh, dw = ref.flce_backward(h, w, lab, lse, mask, torch.tensor(1.0), None, chunk)
    assert torch.allclose(dh.double(), h64.grad, rtol=1e-4, atol=1e-7)
    assert torch.allclose(dw.double(), w64.grad, rtol=1e-4, atol=1e-7)


def test_flce_bias_and_grad_scale():
    h, w, lab = flce_inputs(seed=50)
    b = randn(w.shape[0], seed=54)
    loss, lse, mask = ref.flce_forward(h, w, lab, b, -100, 300)
    h64 = h.double().requires_grad_(True)
    w64 = w.double().requires_grad_(True)
    ce = F.cross_entropy(F.linear(h64, w64, b.double()), lab, ignore_index=-100)
    (2.5 * ce).backward()
    assert abs(loss.item() - ce.item()) <= 1e-6 * abs(ce.item())
    dh, dw = ref.flce_backward(h, w, lab, lse, mask, torch.tensor(2.5), b, 300)
    assert torch.allclose(dh.double(), h64.grad, rtol=1e-4, atol=1e-7)
    assert torch.allclose(dw.double(), w64.grad, rtol=1e-4, atol=1e-7)


def test_flce_invariants_and_all_ignored():
    h, w, lab = flce_inputs(seed=60)
    loss, lse, mask = ref.flce_forward(h, w, lab, None, -100, 128)
    _, dw = ref.flce_backward(h, w, lab, lse, mask, torch.tensor(1.0), None, 128)
    # softmax - one_hot sums to zero over the vocabulary (fp32 rounding aside)
    assert dw.sum(0).abs().max() < 1e-5 * dw.abs().sum(0).max()
    ign = torch.full_like(lab, -100)
    loss0, lse0, mask0 = ref.flce_forward(h, w, ign, None, -100, 128)
    assert loss0.item() == 0.0                       # clamp(#valid, 1): loss 0, not NaN
    dh0, dw0 = ref.flce_backward(h, w, ign, lse0, mask0, torch.tensor(1.0), None, 128)
    assert dh0.abs().max() == 0 and dw0.abs().max() == 0


# --------------------------------------------------------------------- LoRA --


def lora_params(out_f, in_f, r, seed, scale_b=0.02):
    W = randn(out_f, in_f, seed=seed, scale=0.02)
    A = randn(r, in_f, seed=seed + 1, scale=0.25)
    B = randn(out_f, r, seed=seed + 2, scale=scale_b)
    return W, A, B


def test_lora_qkv_vs_fp64_autograd():
    # reference tests/test_fused_ops.py:198-242 (shapes, s=2.0) with the fp64 bar
    X = randn(2, 16, 128, seed=70)
    P = [lora_params(128, 128, 8, 71 + 3 * i, scale_b=0.5) for i in range(3)]
    s = 2.0
    args = []
    for (W, A, B) in P:
        args += [W, A, B, s]
    Q, K, V = ref.lora_qkv_forward(X, *args)
    dQ, dK, dV = (randn(2, 16, 128, seed=80 + i) for i in range(3))
    dX, *dAB = ref.lora_qkv_backward(X, dQ, dK, dV, *args)

    X64 = X.double().requires_grad_(True)
    leaves = [(W.double(), A.double().requires_grad_(True), B.double().requires_grad_(True))
              for (W, A, B) in P]
    outs = [X64 @ W.t() + (X64 @ A.t()) @ B.t() * s for (W, A, B) in leaves]
    for o, o32 in zip(outs, (Q, K, V)):
        assert torch.allclose(o32.double(), o, atol=1e-4, rtol=1e-3)
    torch.autograd.backward(outs, [dQ.double(), dK.double(), dV.double()])
    assert torch.allclose(dX.double(), X64.grad, atol=1e-4, rtol=1e-3)
    for i, (_, A, B) in enumerate(leaves):
        assert dAB[2 * i].dtype == torch.float32
        assert torch.allclose(dAB[2 * i].double(), A.grad, atol=1e-4, rtol=1e-3)
        assert torch.allclose(dAB[2 * i + 1].double(), B.grad, atol=1e-4, rtol=1e-3)


def test_lora_linear_backward_vs_fp64_autograd():
    X = randn(40, 96, seed=90)
    W, A, B = lora_params(64, 96, 8, 91, scale_b=0.5)
    dY = randn(40, 64, seed=92)
    dX, dA, dB = ref.lora_linear_backward(X, dY, W, A, B, 2.0)
    X64 = X.double().requires_grad_(True)
    A64 = A.double().requires_grad_(True)
    B64 = B.double().requires_grad_(True)
    out = X64 @ W.double().t() + (X64 @ A64.t()) @ B64.t() * 2.0
    assert torch.allclose(ref.lora_linear(X, W, A, B, 2.0).double(), out, atol=1e-4, rtol=1e-3)
    out.backward(dY.double())
    assert torch.allclose(dX.double(), X64.grad, atol=1e-4, rtol=1e-3)
    assert torch.allclose(dA.double(), A64.grad, atol=1e-4, rtol=1e-3)
    assert torch.allclose(dB.double(), B64.grad, atol=1e-4, rtol=1e-3)


def test_lora_special_cases():
    X = randn(3, 5, 32, seed=90)
    W, A, B = lora_params(24, 32, 4, 91)
    dY = randn(3, 5, 24, seed=95)
    zero_B = torch.zeros_like(B)
    zero_A = torch.zeros_like(A)
    _, dA, _, *_ = ref.lora_qkv_backward(X, dY, dY, dY, W, A, zero_B, 2.0, W, A, zero_B, 2.0,
                                         W, A, zero_B, 2.0)
    assert dA.abs().max() == 0                                   # B = 0 -> dA = 0
    _, _, dB, *_ = ref.lora_qkv_backward(X, dY, dY, dY, W, zero_A, B, 2.0, W, zero_A, B, 2.0,
                                         W, zero_A, B, 2.0)
    assert dB.abs().max() == 0                                   # A = 0 -> dB = 0
    dX, *_ = ref.lora_qkv_backward(X, dY, dY, dY, W, A, B, 0.0, W, A, B, 0.0, W, A, B, 0.0)
    assert torch.allclose(dX.reshape(-1, 32), 3 * dY.reshape(-1, 24) @ W, atol=1e-6)


def test_lora_mlp_vs_fp64_autograd():
    X = randn(2, 8, 64, seed=100)
    G = lora_params(96, 64, 4, 101, scale_b=0.3)
    U = lora_params(96, 64, 4, 104, scale_b=0.3)
    Dn = lora_params(64, 96, 4, 107, scale_b=0.3)
    s = 2.0
    args = [*G, s, *U, s, *Dn, s]
    out, gate, up, h = ref.lora_mlp_forward(X, *args)
    dY = randn(2, 8, 64, seed=110)
    dX, *dAB = ref.lora_mlp_backward(X, gate, up, h, dY, *args)

    X64 = X.double().requires_grad_(True)
    L = [(W.double(), A.double().requires_grad_(True), B.double().requires_grad_(True))
         for (W, A, B) in (G, U, Dn)]
    lin = lambda t, W, A, B: t @ W.t() + (t @ A.t()) @ B.t() * s  # noqa: E731
    g64 = lin(X64, *L[0])
    u64 = lin(X64, *L[1])
    o64 = lin(F.silu(g64) * u64, *L[2])
    assert close_scaled(out, o64, 1e-5)
    o64.backward(dY.double())
    assert close_scaled(dX, X64.grad, 1e-5)
    names = ["GA", "GB", "UA", "UB", "DA", "DB"]
    for i, (_, A, B) in enumerate(L):
        assert close_scaled(dAB[2 * i], A.grad, 1e-5), names[2 * i]
        assert close_scaled(dAB[2 * i + 1], B.grad, 1e-5), names[2 * i + 1]


# ------------------------------------------------- planted mistakes are caught --


def test_planted_mistakes_fail_the_pins():
    """Copies of oracle functions with one plausible slip each must fail the
    checks above (so the checks are not tautologies)."""
    x = randn(6, 40, seed=120)
    w = randn(40, seed=121)
    g = randn(6, 40, seed=122)
    x64 = x.double().requires_grad_(True)
    w64 = w.double().requires_grad_(True)
    rms64(x64, w64, 1e-6).backward(g.double())
    _, r = ref.rms_norm_forward(x, w, 1e-6)

    def close(a, b):
        return torch.allclose(a.double(), b, atol=1e-4, rtol=1e-3)

    gw = g * w
    m = (gw * x).mean(-1, keepdim=True)
    assert close(gw * r - x * m * r ** 3, x64.grad)            # the correct VJP passes
    assert not close(gw * r, x64.grad)                          # dropped term
    assert not close(gw * r + x * m * r ** 3, x64.grad)         # wrong sign
    assert not close(gw * r - x * m * r ** 2, x64.grad)         # wrong power
    assert close((g * (x * r)).sum(0), w64.grad)                # the correct dW passes
    assert not close((g * x).sum(0), w64.grad)                  # rrms factor dropped in dW

    # RoPE: rotate_half with the halves swapped / sign on the wrong half
    S, D = 16, 8
    xr = randn(1, 1, S, D, seed=123)
    cos, sin = ref.rope_tables(torch.arange(S), D, 1e4)
    ang = torch.arange(S).double().unsqueeze(-1) * ref.rope_inv_freq(D, 1e4).double()
    good = rope_complex64(xr, ang)
    h = D // 2
    bad1 = xr * cos + torch.cat((xr[..., h:], -xr[..., :h]), -1) * sin
    bad2 = xr * cos + torch.cat((-xr[..., :h], xr[..., h:]), -1) * sin
    assert torch.allclose(ref.rope_forward(xr, cos, sin).double(), good, atol=1e-5)
    assert not torch.allclose(bad1.double(), good, atol=1e-3)
    assert not torch.allclose(bad2.double(), good, atol=1e-3)

    # q/k norm + RoPE backward: the rotation transposed with the wrong sign
    xq = randn(1, 2, 5, 8, seed=124)
    wq = 1.0 + 0.1 * randn(8, seed=125)
    cq, sq = randn(1, 1, 5, 8, seed=126), randn(1, 1, 5, 8, seed=127)
    gq = randn(1, 2, 5, 8, seed=128)
    x64q = xq.double().requires_grad_(True)
    ref.qk_norm_rope_forward(x64q, wq.double(), 1e-6, cq.double(), sq.double()).backward(gq.double())
    gs = gq * sq
    rq = torch.rsqrt(xq.pow(2).mean(-1, keepdim=True) + 1e-6)
    nq = xq * rq
    for dn, ok in ((gq * cq + torch.cat((gs[..., 4:], -gs[..., :4]), -1), True),
                   (gq * cq + torch.cat((-gs[..., 4:], gs[..., :4]), -1), False)):
        gw = dn * wq
        dxq = rq * (gw - nq * (gw * nq).mean(-1, keepdim=True))
        assert close_scaled(dxq, x64q.grad, 1e-5) == ok

    # FLCE: forgetting the mask in the mean, or the one-hot subtraction
    hh, ww, lab = flce_inputs(seed=130)
    ce = F.cross_entropy(hh.double() @ ww.double().t(), lab, ignore_index=-100).item()
    loss, lse, mask = ref.flce_forward(hh, ww, lab, None, -100, 256)
    zy = (hh * ww[torch.where(mask, lab, 0)]).sum(-1)
    unmasked_mean = ((lse - zy) * mask.float()).sum() / len(lab)
    assert abs(loss.item() - ce) <= 1e-6 * abs(ce)
    assert abs(unmasked_mean.item() - ce) > 1e-3 * abs(ce)
    p = (hh @ ww.t() - lse.unsqueeze(-1)).exp() * mask.float().unsqueeze(-1) / mask.sum()
    h64 = hh.double().requires_grad_(True)
    F.cross_entropy(h64 @ ww.double().t(), lab, ignore_index=-100).backward()
    assert not torch.allclose((p @ ww).double(), h64.grad, rtol=1e-3, atol=1e-6)

    # LoRA: transposed operand in dB
    X = randn(4, 32, seed=140)
    W, A, B = lora_params(16, 32, 4, 141, scale_b=0.5)
    dY = randn(4, 16, seed=145)
    A64 = A.double().requires_grad_(True)
    B64 = B.double().requires_grad_(True)
    (X.double() @ W.double().t() + (X.double() @ A64.t()) @ B64.t() * 2.0).backward(dY.double())
    dB_wrong = (torch.mm((X @ A.t()).t(), dY) * 2.0).t()   # (XA^T)^T dY transposed back
    dB_wrong_scale = torch.mm(dY.t(), X @ A.t())           # scale dropped
    assert not torch.allclose(dB_wrong_scale.double(), B64.grad, rtol=1e-3)
    assert torch.allclose(dB_wrong.double(), B64.grad, rtol=1e-4, atol=1e-6)  # same thing, fine
    assert math.isfinite(loss.item())
