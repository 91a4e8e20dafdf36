"""The metal_liger_amd:: custom ops' fake kernels (no GPU needed): under
FakeTensorMode, on fake ROCm-device tensors, each op returns outputs of the
documented shapes, dtypes and layouts (the GPU suite's opcheck compares the
same fakes with the real kernels)."""

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

BF, F32 = torch.bfloat16, torch.float32


@pytest.fixture
def ops():
    import metal_liger_amd._custom_ops  # noqa: F401
    return torch.ops.metal_liger_amd


def e(*shape, dtype=BF):
    return torch.empty(*shape, dtype=dtype, device="cuda")


def test_fake_kernels_elementwise_rope_qkn(ops):
    with FakeTensorMode():
        y, r = ops.rms_norm_fwd(e(4, 8, 256, dtype=F32), e(256, dtype=F32), 1e-6)
        assert y.shape == (4, 8, 256) and r.shape == (4, 8) and r.dtype == F32
        dx, dw = ops.rms_norm_bwd(e(32, 64), e(64, dtype=F32), e(32, 64), None, 1e-6)
        assert dx.dtype == BF and dw.shape == (64,) and dw.dtype == F32
        y, total, r = ops.rms_norm_add_fwd(e(2, 5, 64), e(2, 5, 64), e(64, dtype=F32), 1e-6)
        assert y.shape == total.shape == (2, 5, 64) and total.dtype == BF and r.shape == (2, 5)
        dx, dw = ops.rms_norm_add_bwd(total, e(64, dtype=F32), y, y, r, 1e-6)
        assert dx.shape == (2, 5, 64) and dx.dtype == BF and dw.dtype == F32
        assert ops.swiglu_fwd(e(8, 96), e(8, 96)).shape == (8, 96)
        q = e(2, 33, 4, 64).transpose(1, 2)                  # HF's transposed view
        qo, ko = ops.rope_table(q, None, e(33, 64, dtype=F32), e(33, 64, dtype=F32), 1.0)
        assert qo.shape == q.shape and qo.stride() == q.stride() and qo.dtype == F32
        assert ko.shape == (0,)
        qo, ko = ops.rope_pos(q, e(2, 2, 33, 64), torch.empty(33, dtype=torch.int64, device="cuda"),
                              e(32, dtype=F32), 1.0)
        assert qo.dtype == BF and qo.stride() == q.stride() and ko.shape == (2, 2, 33, 64)
        q4, k4 = e(2, 4, 17, 128), e(2, 2, 17, 128)
        o1, o2 = ops.qk_norm_rope_fwd(q4, k4, e(128), e(128), e(2, 1, 17, 128), e(2, 1, 17, 128), 1e-6)
        assert o1.shape == q4.shape and o1.transpose(1, 2).is_contiguous()
        dq, dk, dwq, dwk = ops.qk_norm_rope_bwd(q4, k4, e(128), e(128, dtype=F32), e(17, 128),
                                                 e(17, 128), 1e-6, q4, k4, True, False)
        assert dk.shape == k4.shape and dwq.shape == (128,) and dwk.shape == (0,)


def test_fake_kernels_flce_lora(ops):
    with FakeTensorMode():
        h, w = e(64, 128), e(1000, 128)
        lab = torch.empty(64, dtype=torch.int64, device="cuda")
        loss, lse, nv, dh, dw = ops.flce_fwd_grad(h, w, lab, None, -100, True, False)
        assert loss.shape == () and lse.shape == (64,) and nv.shape == (1,)
        assert dh.shape == (64, 128) and dh.dtype == BF and dw.shape == (0,)
        dh2, dw2 = ops.flce_bwd(h, w, lab, None, -100, lse, nv, loss, 256, False, True)
        assert dh2.shape == (0,) and dw2.shape == (1000, 128)
        x = e(96, 128)
        assert ops.linear_bf16(x, e(64, 128)).shape == (96, 64)
        assert ops.lora_xa(x, e(48, 128)).shape == (96, 48)
        qo, ko, vo = ops.lora_qkv_out(x, [e(128, 128), e(64, 128), e(64, 128)], e(96, 48),
                                      [e(128, 16), e(64, 16), e(64, 16)])
        assert qo.shape == (96, 128) and ko.shape == (96, 64) and vo.shape == (96, 64)
        assert qo.dtype == BF
        # LoRA backwards: dX and one fp32 buffer of the adapter gradients,
        # each starting on a 64-element boundary (hip_ops.grad_layout)
        dX, g = ops.lora_qkv_bwd(x, [e(96, 128), e(96, 64), e(96, 64)],
                                 [e(128, 128), e(64, 128), e(64, 128)], e(48, 128),
                                 [e(128, 16), e(64, 16), e(64, 16)], [2.0] * 3, e(96, 48), 16)
        assert dX.shape == (96, 128) and g.dtype == F32
        assert g.shape == (48 * 128 + 128 * 16 + 64 * 16 + 64 * 16,)
        dX, g = ops.lora_linear_bwd(x, e(96, 64), e(64, 128), e(16, 128), e(64, 16), 2.0,
                                    e(96, 16), 16)
        assert dX.shape == (96, 128) and g.shape == (16 * 128 + 64 * 16,)
        dX, g = ops.lora_mlp_bwd(x, e(96, 256), e(96, 256), e(96, 256), e(96, 128), e(256, 128),
                                 e(256, 128), e(128, 256), e(32, 128), e(16, 256), e(256, 16),
                                 e(256, 16), e(128, 16), [2.0] * 3, e(96, 32), e(96, 16), 16)
        assert dX.shape == (96, 128) and g.shape == (32 * 128 + 16 * 256 + 2 * 256 * 16 + 128 * 16,)


def test_grad_layout_offsets():
    from metal_liger_amd import hip_ops
    offs, total = hip_ops.grad_layout([(3, 5), (2, 32), (7,)])
    assert offs == [0, 64, 128] and total == 192          # 15 -> 64, 64 -> 64, 7 -> 64
    flat = torch.arange(192, dtype=torch.float32)
    a, b, c = hip_ops.grad_views(flat, [(3, 5), (2, 32), (7,)])
    assert a.shape == (3, 5) and a[2, 4].item() == 14
    assert b.shape == (2, 32) and b[0, 0].item() == 64 and b.is_contiguous()
    assert c.shape == (7,) and c[0].item() == 128
