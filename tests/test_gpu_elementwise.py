"""GPU parity: RMSNorm, SwiGLU, RoPE (HIP path) against the CPU oracle.

Inputs are drawn on the CPU from seeded generators and copied to the GPU, so
the oracle and the kernels see identical values. Full config sizes are
covered (the oracle finishes them in seconds), plus the reference's own test
shapes and edge cases: empty inputs, ragged widths, strided views,
broadcast grads, mixed dtypes.
"""

import pytest
import torch

from oracle import reference_ops as ref
from tests.parity import assert_close, seeded

pytestmark = pytest.mark.gpu

LOW = (torch.bfloat16, torch.float16)


def to(dev, *ts):
    return [t.to(dev) for t in ts]


# ------------------------------------------------------------------ RMSNorm --


def run_rms(dev, x, w, g, eps=1e-6):
    from metal_liger_amd.ops.fused_rms_norm import MetalLigerRMSNorm
    xd = x.to(dev).requires_grad_(True)
    norm = MetalLigerRMSNorm(x.shape[-1], eps=eps, weight=w.to(dev).clone())
    y = norm(xd)
    y.backward(g.to(dev))
    return y, xd.grad, norm.weight.grad


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(8192, 2048), (2, 128, 2048), (2, 16, 256), (3, 7),
                                   (5, 1000), (4, 3000), (3, 5000), (64, 4096), (1, 64)])
def test_rmsnorm_parity(dev, dtype, shape):
    x = seeded(shape, 0, dtype)
    w = seeded(shape[-1:], 1, dtype, scale=0.1, shift=1.0)
    g = seeded(shape, 2, dtype)
    y, dx, dw = run_rms(dev, x, w, g)
    ry, rr = ref.rms_norm_forward(x, w, 1e-6)
    rdx, rdw = ref.rms_norm_backward(x, w, rr, g)
    assert y.dtype == dtype and dx.dtype == dtype and dw.dtype == dtype
    assert_close(y, ry, f"y {shape}")
    assert_close(dx, rdx, f"dx {shape}")
    assert_close(dw, rdw, f"dw {shape}")


def test_rmsnorm_config_fp32_saved_rrms(dev):
    """The fp32 RMSNorm workload: x [8192, 2048] fp32, weight 1 + 0.1 N(0,1),
    eps 1e-6, the rrms the forward saves."""
    from metal_liger_amd import hip_ops
    x = seeded((8192, 2048), 0)
    w = seeded((2048,), 1, scale=0.1, shift=1.0)
    y, r = hip_ops.rms_norm_fwd(x.to(dev), w.to(dev), 1e-6)
    ry, rr = ref.rms_norm_forward(x, w, 1e-6)
    assert r.shape == (8192,) and r.dtype == torch.float32
    assert_close(r, rr.squeeze(-1), "rrms")
    assert_close(y, ry, "y")


def test_rmsnorm_fp32_weight_with_bf16_input(dev):
    x = seeded((64, 512), 3, torch.bfloat16)
    w = seeded((512,), 4, torch.float32, scale=0.1, shift=1.0)
    g = seeded((64, 512), 5, torch.bfloat16)
    y, dx, dw = run_rms(dev, x, w, g)
    ry, rr = ref.rms_norm_forward(x, w, 1e-6)
    rdx, rdw = ref.rms_norm_backward(x, w, rr, g)
    assert dw.dtype == torch.float32
    assert_close(y, ry, "y")
    assert_close(dx, rdx, "dx")
    assert_close(dw, rdw, "dw")


def test_rmsnorm_strided_rows_and_broadcast_grad(dev):
    big = seeded((32, 3072), 6)
    x = big.to(dev)[:, 512:2560]            # row stride 3072, 16-byte aligned
    w = seeded((2048,), 7, scale=0.1, shift=1.0)
    from metal_liger_amd.ops.fused_rms_norm import MetalLigerRMSNorm
    xd = x.clone().requires_grad_(True)
    xs = big[:, 512:2560]
    norm = MetalLigerRMSNorm(2048, weight=w.to(dev).clone())
    y = norm(x)                              # strided input, no grad
    ry, rr = ref.rms_norm_forward(xs, w, 1e-6)
    assert_close(y, ry, "strided y")
    out = norm(xd)
    out.sum().backward()                     # grad_output is an expanded (stride-0) tensor
    rdx, rdw = ref.rms_norm_backward(xs, w, rr, torch.ones_like(xs))
    assert_close(xd.grad, rdx, "dx (expanded grad)")
    assert_close(norm.weight.grad, rdw, "dw (expanded grad)")
    # misaligned start (offset by one element): generic path
    xm = big.to(dev)[:, 1:2049]
    ym = norm(xm)
    assert_close(ym, ref.rms_norm_forward(big[:, 1:2049], w, 1e-6)[0], "misaligned y")


def test_rmsnorm_empty_rows(dev):
    from metal_liger_amd import hip_ops
    x = torch.empty(0, 64, device=dev)
    w = torch.ones(64, device=dev)
    y, r = hip_ops.rms_norm_fwd(x, w, 1e-6)
    assert y.shape == (0, 64) and r.shape == (0,)
    dx, dw = hip_ops.rms_norm_bwd(x, w, torch.empty(0, 64, device=dev), r, 1e-6)
    assert dx.shape == (0, 64)
    assert torch.equal(dw.cpu(), torch.zeros(64))


def test_rmsnorm_ext_surface(dev):
    from metal_liger_amd import metal_liger_ext as ext
    x = seeded((4, 100, 2048), 8, torch.bfloat16)
    w = seeded((2048,), 9, torch.bfloat16, scale=0.1, shift=1.0)
    g = seeded((4, 100, 2048), 10, torch.bfloat16)
    out, cache = ext.rms_norm_forward(x.to(dev), w.to(dev), 1e-6, "unused")
    ry, rr = ref.rms_norm_forward(x, w, 1e-6)
    assert cache.shape == (400,) and cache.dtype == torch.float32
    assert_close(out, ry, "ext y")
    assert_close(cache, rr.reshape(-1), "ext rms_cache")
    gx, gw = ext.rms_norm_backward(x.to(dev), w.to(dev), g.to(dev), 1e-6, "unused")
    rdx, rdw = ref.rms_norm_backward(x, w, rr, g)
    assert_close(gx, rdx, "ext dx (recomputed rrms)")
    assert_close(gw, rdw, "ext dw")


def test_rmsnorm_deterministic(dev):
    from metal_liger_amd import hip_ops
    x = seeded((4096, 2048), 11).to(dev)
    w = seeded((2048,), 12).to(dev)
    g = seeded((4096, 2048), 13).to(dev)
    _, r = hip_ops.rms_norm_fwd(x, w, 1e-6)
    a = hip_ops.rms_norm_bwd(x, w, g, r, 1e-6)[1]
    b = hip_ops.rms_norm_bwd(x, w, g, r, 1e-6)[1]
    assert torch.equal(a, b)


# ------------------------------------------------------------------- SwiGLU --


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(8192, 6144), (4, 128, 5120), (2, 16, 512), (1, 1), (3, 37),
                                   (1000003,)])
def test_swiglu_parity(dev, dtype, shape):
    from metal_liger_amd.ops.fused_swiglu import fused_swiglu
    if dtype == torch.float32 and shape == (8192, 6144):
        pytest.skip("fp32 at the bf16 config size adds nothing over (4, 128, 5120)")
    gate = seeded(shape, 20, dtype)
    up = seeded(shape, 21, dtype)
    dy = seeded(shape, 22, dtype)
    gd = gate.to(dev).requires_grad_(True)
    ud = up.to(dev).requires_grad_(True)
    out = fused_swiglu(gd, ud)
    out.backward(dy.to(dev))
    ro, sig = ref.swiglu_forward(gate, up)
    rdg, rdu = ref.swiglu_backward(gate, up, sig, dy)
    assert out.dtype == dtype
    assert_close(out, ro, f"out {shape}")
    assert_close(gd.grad, rdg, f"dgate {shape}")
    assert_close(ud.grad, rdu, f"dup {shape}")


def test_swiglu_misaligned_and_special_values(dev):
    from metal_liger_amd import hip_ops
    base = seeded((4099,), 23)
    baseu = seeded((4099,), 24)
    g = base.to(dev)[3:]
    u = baseu.to(dev)[3:]
    out = hip_ops.swiglu_fwd(g, u)
    assert_close(out, ref.swiglu_forward(base[3:], baseu[3:])[0], "misaligned")
    gs = torch.tensor([0.0, 0.0, 40.0, -40.0, 100.0, -100.0], device=dev)
    us = torch.tensor([1.0, -3.0, 2.0, 2.0, 1.0, 1.0], device=dev)
    dys = torch.tensor([2.0, 1.0, 1.0, 1.0, 1.0, 1.0], device=dev)
    o = hip_ops.swiglu_fwd(gs, us).cpu()
    dg, du = [t.cpu() for t in hip_ops.swiglu_bwd(gs, us, dys)]
    assert o[0] == 0 and o[1] == 0 and du[0] == 0
    assert dg[0] == 1.0 and dg[1] == -1.5
    assert torch.isclose(o[2], torch.tensor(80.0)) and abs(o[3]) < 1e-12
    assert o[4] == 100.0 and o[5] == 0.0 and torch.isfinite(dg).all()


def test_swiglu_module_and_ext(dev):
    from metal_liger_amd import metal_liger_ext as ext
    g = seeded((3, 64, 256), 25, torch.bfloat16)
    u = seeded((3, 64, 256), 26, torch.bfloat16)
    dy = seeded((3, 64, 256), 27, torch.bfloat16)
    o = ext.swiglu_forward(g.to(dev), u.to(dev), "")
    dg, du = ext.swiglu_backward(g.to(dev), u.to(dev), dy.to(dev), "")
    ro, sig = ref.swiglu_forward(g, u)
    rdg, rdu = ref.swiglu_backward(g, u, sig, dy)
    assert_close(o, ro, "ext out")
    assert_close(dg, rdg, "ext dgate")
    assert_close(du, rdu, "ext dup")
    with pytest.raises(RuntimeError):
        ext.swiglu_forward(g.to(dev), u[:, :32].to(dev))


def test_swiglu_empty(dev):
    from metal_liger_amd import hip_ops
    e = torch.empty(0, 8, device=dev, dtype=torch.bfloat16)
    assert hip_ops.swiglu_fwd(e, e).shape == (0, 8)


@pytest.mark.parametrize("n", [8192 * 48 + 5, 4096])
def test_swiglu_bwd_in_place(dev, n):
    """ml_swiglu_bwd with dy and dgate the same buffer (the LoRA MLP backward
    runs it that way) gives the out-of-place result bit for bit, vector path
    and scalar tail included."""
    from metal_liger_amd import hip_ops
    from metal_liger_amd._hip import call
    g = seeded((n,), 31, torch.bfloat16).to(dev)
    u = seeded((n,), 32, torch.bfloat16).to(dev)
    dy = seeded((n,), 33, torch.bfloat16).to(dev)
    rdg, rdu = hip_ops.swiglu_bwd(g, u, dy)
    buf = dy.clone()
    du = torch.empty_like(buf)
    stream = torch.cuda.current_stream(dev).cuda_stream
    call("ml_swiglu_bwd", g.data_ptr(), u.data_ptr(), buf.data_ptr(), buf.data_ptr(),
         du.data_ptr(), n, 1, stream)
    assert torch.equal(buf, rdg)
    assert torch.equal(du, rdu)


# --------------------------------------------------------------------- RoPE --


def test_rope_reference_test_case(dev):
    """reference tests/test_fused_ops.py:156-188: [2, 8, 128, 64] fp32, theta 1e4."""
    from metal_liger_amd.ops.fused_rope import _FusedRoPEFunction, _apply_rotary_fused
    x = seeded((2, 8, 128, 64), 30)
    cos, sin = ref.rope_tables(torch.arange(128), 64, 1e4)
    y = _apply_rotary_fused(x.to(dev), cos.to(dev), sin.to(dev))
    assert_close(y, ref.rope_forward(x, cos, sin), "rope fwd")
    assert (y.cpu() - ref.rope_forward(x, cos, sin)).abs().max() <= 1e-6
    xd = seeded((1, 4, 32, 64), 31).to(dev).requires_grad_(True)
    c2, s2 = ref.rope_tables(torch.arange(32), 64, 1e4)
    g = seeded((1, 4, 32, 64), 32)
    _FusedRoPEFunction.apply(xd, c2.to(dev), s2.to(dev)).backward(g.to(dev))
    assert_close(xd.grad, ref.rope_backward(g, c2, s2, torch.float32), "rope bwd")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rope_qk_tables_hf_layout(dev, dtype):
    """HF passes transpose(1, 2) views and [B, 1, S, D] tables (HF modeling_qwen3)."""
    from metal_liger_amd.ops.fused_rope import apply_fused_rotary
    B, S, Hq, Hk, D = 2, 64, 4, 2, 128
    qraw = seeded((B, S, Hq, D), 33, dtype)
    kraw = seeded((B, S, Hk, D), 34, dtype)
    pos = torch.arange(S).unsqueeze(0).expand(B, S)
    cos, sin = ref.rope_tables(pos, D, 1e6)
    cos, sin = cos.to(dtype).unsqueeze(1), sin.to(dtype).unsqueeze(1)
    q = qraw.to(dev).transpose(1, 2).requires_grad_(True)
    k = kraw.to(dev).transpose(1, 2).requires_grad_(True)
    qo, ko = apply_fused_rotary(q, k, cos.to(dev), sin.to(dev))
    rq = ref.rope_forward(qraw.transpose(1, 2), cos, sin)
    rk = ref.rope_forward(kraw.transpose(1, 2), cos, sin)
    assert qo.shape == q.shape and qo.dtype == dtype
    assert_close(qo, rq, "q")
    assert_close(ko, rk, "k")
    gq = seeded(q.shape, 35, dtype)
    gk = seeded(k.shape, 36, dtype)
    torch.autograd.backward([qo, ko], [gq.to(dev), gk.to(dev)])
    assert_close(q.grad, ref.rope_backward(gq, cos, sin, dtype), "dq")
    assert_close(k.grad, ref.rope_backward(gk, cos, sin, dtype), "dk")


def test_rope_mixed_dtype_promotes(dev):
    from metal_liger_amd.ops.fused_rope import _FusedRoPEFunction
    x = seeded((1, 2, 16, 32), 37, torch.bfloat16)
    cos, sin = ref.rope_tables(torch.arange(16), 32, 1e4)
    xd = x.to(dev).requires_grad_(True)
    y = _FusedRoPEFunction.apply(xd, cos.to(dev), sin.to(dev))
    assert y.dtype == torch.float32
    assert_close(y, ref.rope_forward(x, cos, sin), "promoted fwd")
    g = seeded((1, 2, 16, 32), 38)
    y.backward(g.to(dev))
    assert xd.grad.dtype == torch.bfloat16
    assert_close(xd.grad, ref.rope_backward(g, cos, sin, torch.bfloat16), "promoted bwd")


def test_rope_positions_config(dev):
    """The bf16 RoPE workload: q [4,16,2048,128], k [4,8,2048,128] bf16, positions 0..2047,
    theta 1e6, cos/sin computed in-kernel. Compared with the oracle's rotation
    using the HF-style fp32 tables (the kernel rounds once, to bf16)."""
    from metal_liger_amd.ops.fused_rope import apply_fused_rotary_inline
    B, S, D = 4, 2048, 128
    q = seeded((B, 16, S, D), 40, torch.bfloat16)
    k = seeded((B, 8, S, D), 41, torch.bfloat16)
    pos = torch.arange(S)
    cos, sin = ref.rope_tables(pos, D, 1e6)
    qd = q.to(dev).requires_grad_(True)
    kd = k.to(dev).requires_grad_(True)
    qo, ko = apply_fused_rotary_inline(qd, kd, pos.to(dev), theta=1e6)
    rq = ref.rope_forward(q.float(), cos, sin).to(torch.bfloat16)
    rk = ref.rope_forward(k.float(), cos, sin).to(torch.bfloat16)
    assert_close(qo, rq, "q (positions)")
    assert_close(ko, rk, "k (positions)")
    # HF's own bf16 evaluation casts the tables to bf16 and rounds each product
    # and the sum to bf16 (three roundings, ~2^-8 each, on terms that can
    # cancel), so elementwise it can sit 3e-2 from the exact value; it stays
    # within the Frobenius bar of the single-rounded result.
    from tests.parity import rel_fro
    hf = ref.rope_forward(q, cos.to(torch.bfloat16), sin.to(torch.bfloat16))
    assert rel_fro(qo, hf) <= 2e-2
    gq = seeded(q.shape, 42, torch.bfloat16)
    gk = seeded(k.shape, 43, torch.bfloat16)
    torch.autograd.backward([qo, ko], [gq.to(dev), gk.to(dev)])
    assert_close(qd.grad, ref.rope_backward(gq.float(), cos, sin, torch.bfloat16), "dq (positions)")
    assert_close(kd.grad, ref.rope_backward(gk.float(), cos, sin, torch.bfloat16), "dk (positions)")


def test_rope_positions_properties_fp32(dev):
    """Size-independent properties: fwd then bwd is the identity; per-pair
    norms are preserved; position 0 is the identity."""
    from metal_liger_amd import hip_ops
    q = seeded((2, 6, 512, 64), 44).to(dev)
    pos = torch.arange(512, device=dev)
    inv = hip_ops.rope_inv_freq(64, 1e6, dev)
    y, _ = hip_ops.rope_pos(q, None, pos, inv, 1.0)
    back, _ = hip_ops.rope_pos(y, None, pos, inv, -1.0)
    assert (back - q).abs().max().item() < 1e-5
    pn = lambda t: t[..., :32] ** 2 + t[..., 32:] ** 2  # noqa: E731
    assert torch.allclose(pn(y), pn(q), rtol=1e-5, atol=1e-5)
    assert torch.equal(y[:, :, 0], q[:, :, 0])


def test_rope_positions_large_angles_fp32(dev):
    """In-kernel cos/sin at positions up to 200,000 (angles up to 2e5 rad)
    against the rotation by the exact (fp64) cos/sin of the same fp32 angles
    the HF rotary module forms (fp32 position times fp32 inv_freq), at the
    fp32 bar."""
    from metal_liger_amd import hip_ops
    B, H, S, D = 2, 3, 64, 64
    x = seeded((B, H, S, D), 47)
    pos = torch.randint(0, 200_000, (B, S), generator=torch.Generator().manual_seed(48))
    inv = hip_ops.rope_inv_freq(D, 1e4, dev)
    y, _ = hip_ops.rope_pos(x.to(dev), None, pos.to(dev), inv, 1.0)
    ang = (pos.float().unsqueeze(-1) * inv.cpu()).double()          # fp32 angles, exact trig
    emb = torch.cat((ang, ang), -1).unsqueeze(1)
    want = ref.rope_forward(x.double(), emb.cos(), emb.sin())
    assert_close(y, want.float(), "large-angle positions", torch.float32)


def test_rope_positions_batched_and_odd_head_dim(dev):
    from metal_liger_amd import hip_ops
    B, H, S, D = 3, 2, 10, 12            # D/2 = 6: scalar path
    x = seeded((B, H, S, D), 45)
    pos = torch.randint(0, 5000, (B, S), generator=torch.Generator().manual_seed(46))
    y, _ = hip_ops.rope_pos(x.to(dev), None, pos.to(dev), hip_ops.rope_inv_freq(D, 1e4, dev), 1.0)
    cos, sin = ref.rope_tables(pos, D, 1e4)
    assert_close(y, ref.rope_forward(x, cos.unsqueeze(1), sin.unsqueeze(1)), "batched positions")
