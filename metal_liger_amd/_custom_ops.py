"""The HIP entry points as torch.library custom ops (namespace metal_liger_amd).

The reference registers its native ops with torch.library so that
torch.compile can trace through them (_torch_library.py:1-13); it does so for
RMSNorm and SwiGLU only (reproduced in _torch_library.py here, under the
reference's schemas). This module gives every launch the fused autograd
Functions make the same standing: an opaque operator with a fake kernel that
produces outputs of the real kernel's shapes, dtypes and strides, so
torch.compile (dynamo / AOTAutograd) traces the Functions without graph
breaks and torch.library.opcheck can check each one.

Absent outputs (a gradient that was not requested, k in the q-only RoPE
forms) come back as empty tensors ([0]) and the Functions map them to None.
The real kernels are the hip_ops wrappers; they run on the ROCm device
("cuda" in PyTorch-ROCm) and raise for tensors elsewhere.
"""

from __future__ import annotations

from typing import List, Optional

import torch
from torch import Tensor

from metal_liger_amd import hip_ops

NS = "metal_liger_amd"
# Registered for every device: the implementations raise ValueError for
# tensors that are not on a ROCm GPU (the library's contract), rather than
# the dispatcher's NotImplementedError.
_DEV = None


def _none(t: Tensor) -> Tensor:
    """The [0] placeholder for an absent output."""
    return t.new_empty((0,))


def maybe(t: Tensor) -> Optional[Tensor]:
    """An op output, or None for the [0] placeholder."""
    return None if t.dim() == 1 and t.shape[0] == 0 else t


# ------------------------------------------------------------------ RMSNorm --

@torch.library.custom_op(f"{NS}::rms_norm_fwd", mutates_args=(), device_types=_DEV)
def rms_norm_fwd(x: Tensor, weight: Tensor, eps: float) -> tuple[Tensor, Tensor]:
    return hip_ops.rms_norm_fwd(x, weight, eps)


@rms_norm_fwd.register_fake
def _(x, weight, eps):
    return x.new_empty(x.shape), x.new_empty(x.shape[:-1], dtype=torch.float32)


@torch.library.custom_op(f"{NS}::rms_norm_bwd", mutates_args=(), device_types=_DEV)
def rms_norm_bwd(x: Tensor, weight: Tensor, dy: Tensor, rrms: Optional[Tensor],
                 eps: float) -> tuple[Tensor, Tensor]:
    return hip_ops.rms_norm_bwd(x, weight, dy, rrms, eps)


@rms_norm_bwd.register_fake
def _(x, weight, dy, rrms, eps):
    return x.new_empty(x.shape), weight.new_empty((x.shape[-1],))


@torch.library.custom_op(f"{NS}::rms_norm_add_fwd", mutates_args=(), device_types=_DEV)
def rms_norm_add_fwd(x: Tensor, residual: Tensor, weight: Tensor,
                     eps: float) -> tuple[Tensor, Tensor, Tensor]:
    return hip_ops.rms_norm_add_fwd(x, residual, weight, eps)


@rms_norm_add_fwd.register_fake
def _(x, residual, weight, eps):
    return (x.new_empty(x.shape), x.new_empty(x.shape),
            x.new_empty(x.shape[:-1], dtype=torch.float32))


@torch.library.custom_op(f"{NS}::rms_norm_add_bwd", mutates_args=(), device_types=_DEV)
def rms_norm_add_bwd(total: Tensor, weight: Tensor, dy: Tensor, dsum: Tensor, rrms: Tensor,
                     eps: float) -> tuple[Tensor, Tensor]:
    return hip_ops.rms_norm_bwd(total, weight, dy, rrms, eps, dsum=dsum)


@rms_norm_add_bwd.register_fake
def _(total, weight, dy, dsum, rrms, eps):
    return total.new_empty(total.shape), weight.new_empty((total.shape[-1],))


# ------------------------------------------------------------------- SwiGLU --

@torch.library.custom_op(f"{NS}::swiglu_fwd", mutates_args=(), device_types=_DEV)
def swiglu_fwd(gate: Tensor, up: Tensor) -> Tensor:
    return hip_ops.swiglu_fwd(gate, up)


@swiglu_fwd.register_fake
def _(gate, up):
    return gate.new_empty(gate.shape)


@torch.library.custom_op(f"{NS}::swiglu_bwd", mutates_args=(), device_types=_DEV)
def swiglu_bwd(gate: Tensor, up: Tensor, dy: Tensor) -> tuple[Tensor, Tensor]:
    return hip_ops.swiglu_bwd(gate, up, dy)


@swiglu_bwd.register_fake
def _(gate, up, dy):
    return gate.new_empty(gate.shape), up.new_empty(up.shape)


# --------------------------------------------------------------------- RoPE --

def _rope_fake(xs, out_dtypes):
    return tuple(hip_ops.rope_out(x, dt)[2] for x, dt in zip(xs, out_dtypes))


@torch.library.custom_op(f"{NS}::rope_table", mutates_args=(), device_types=_DEV)
def rope_table(q: Tensor, k: Optional[Tensor], cos: Tensor, sin: Tensor,
               sgn: float) -> tuple[Tensor, Tensor]:
    qo, ko = hip_ops.rope_table(q, k, cos, sin, sgn)
    return qo, (ko if ko is not None else _none(qo))


@rope_table.register_fake
def _(q, k, cos, sin, sgn):
    dt = lambda x: hip_ops.rope_out_dtype(x.dtype, cos.dtype, sin.dtype)  # noqa: E731
    if k is None:
        qo, = _rope_fake([q], [dt(q)])
        return qo, _none(qo)
    return _rope_fake([q, k], [dt(q), dt(k)])


@torch.library.custom_op(f"{NS}::rope_pos", mutates_args=(), device_types=_DEV)
def rope_pos(q: Tensor, k: Optional[Tensor], positions: Tensor, inv_freq: Tensor,
             sgn: float) -> tuple[Tensor, Tensor]:
    qo, ko = hip_ops.rope_pos(q, k, positions, inv_freq, sgn)
    return qo, (ko if ko is not None else _none(qo))


@rope_pos.register_fake
def _(q, k, positions, inv_freq, sgn):
    if k is None:
        qo, = _rope_fake([q], [q.dtype])
        return qo, _none(qo)
    return _rope_fake([q, k], [q.dtype, k.dtype])


# ------------------------------------------------------ q/k norm + RoPE --

def _qkn_fake_out(x: Tensor) -> Tensor:
    B, H, S, D = x.shape
    return x.new_empty((B, S, H, D)).transpose(1, 2)


@torch.library.custom_op(f"{NS}::qk_norm_rope_fwd", mutates_args=(), device_types=_DEV)
def qk_norm_rope_fwd(q: Tensor, k: Tensor, q_weight: Tensor, k_weight: Tensor, cos: Tensor,
                     sin: Tensor, eps: float) -> tuple[Tensor, Tensor]:
    return hip_ops.qk_norm_rope_fwd(q, k, q_weight, k_weight, cos, sin, eps)


@qk_norm_rope_fwd.register_fake
def _(q, k, q_weight, k_weight, cos, sin, eps):
    return _qkn_fake_out(q), _qkn_fake_out(k)


@torch.library.custom_op(f"{NS}::qk_norm_rope_bwd", mutates_args=(), device_types=_DEV)
def qk_norm_rope_bwd(q: Tensor, k: Tensor, q_weight: Tensor, k_weight: Tensor, cos: Tensor,
                     sin: Tensor, eps: float, dq_out: Tensor, dk_out: Tensor, need_dq_weight: bool,
                     need_dk_weight: bool) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    dq, dk, dwq, dwk = hip_ops.qk_norm_rope_bwd(q, k, q_weight, k_weight, cos, sin, eps, dq_out,
                                                 dk_out, need_dq_weight, need_dk_weight)
    return (dq, dk, dwq if dwq is not None else _none(dq), dwk if dwk is not None else _none(dq))


@qk_norm_rope_bwd.register_fake
def _(q, k, q_weight, k_weight, cos, sin, eps, dq_out, dk_out, need_dq_weight, need_dk_weight):
    dq, dk = _qkn_fake_out(q), _qkn_fake_out(k)
    return (dq, dk, q_weight.new_empty(q_weight.shape) if need_dq_weight else _none(dq),
            k_weight.new_empty(k_weight.shape) if need_dk_weight else _none(dq))


# ------------------------------------------------------------------- FLCE --

@torch.library.custom_op(f"{NS}::flce_fwd", mutates_args=(), device_types=_DEV)
def flce_fwd(hidden: Tensor, weight: Tensor, labels: Tensor, bias: Optional[Tensor],
             ignore_index: int, chunk_size: int = 8192) -> tuple[Tensor, Tensor, Tensor]:
    return hip_ops.flce_fwd(hidden, weight, labels, bias, ignore_index, vocab_chunk=chunk_size)


@flce_fwd.register_fake
def _(hidden, weight, labels, bias, ignore_index, chunk_size=8192):
    f32 = torch.float32
    return (hidden.new_empty((), dtype=f32), hidden.new_empty((hidden.shape[0],), dtype=f32),
            hidden.new_empty((1,), dtype=f32))


@torch.library.custom_op(f"{NS}::flce_fwd_grad", mutates_args=(), device_types=_DEV)
def flce_fwd_grad(hidden: Tensor, weight: Tensor, labels: Tensor, bias: Optional[Tensor],
                  ignore_index: int, need_dhidden: bool, need_dweight: bool,
                  chunk_size: int = 8192) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    loss, lse, n_valid, dh, dw = hip_ops.flce_fwd_grad(hidden, weight, labels, bias, ignore_index,
                                                       need_dhidden, need_dweight,
                                                       vocab_chunk=chunk_size)
    return (loss, lse, n_valid, dh if dh is not None else _none(lse),
            dw if dw is not None else _none(lse))


@flce_fwd_grad.register_fake
def _(hidden, weight, labels, bias, ignore_index, need_dhidden, need_dweight, chunk_size=8192):
    N, H = hidden.shape
    V = weight.shape[0]
    f32 = torch.float32
    lse = hidden.new_empty((N,), dtype=f32)
    return (hidden.new_empty((), dtype=f32), lse, hidden.new_empty((1,), dtype=f32),
            hidden.new_empty((N, H), dtype=hidden.dtype) if need_dhidden else _none(lse),
            hidden.new_empty((V, H), dtype=hidden.dtype) if need_dweight else _none(lse))


@torch.library.custom_op(f"{NS}::flce_scale_grads", mutates_args=("d_hidden", "d_weight"),
                         device_types=_DEV)
def flce_scale_grads(grad_loss: Tensor, d_hidden: Optional[Tensor],
                     d_weight: Optional[Tensor]) -> None:
    hip_ops.flce_scale_grads(grad_loss, d_hidden, d_weight)


@flce_scale_grads.register_fake
def _(grad_loss, d_hidden, d_weight):
    return None


@torch.library.custom_op(f"{NS}::flce_bwd", mutates_args=(), device_types=_DEV)
def flce_bwd(hidden: Tensor, weight: Tensor, labels: Tensor, bias: Optional[Tensor],
             ignore_index: int, lse: Tensor, n_valid: Tensor, grad_loss: Tensor, chunk_size: int,
             need_dhidden: bool, need_dweight: bool) -> tuple[Tensor, Tensor]:
    dh, dw = hip_ops.flce_bwd(hidden, weight, labels, bias, ignore_index, lse, n_valid, grad_loss,
                              chunk_size, need_dhidden, need_dweight)
    return (dh if dh is not None else _none(lse), dw if dw is not None else _none(lse))


@flce_bwd.register_fake
def _(hidden, weight, labels, bias, ignore_index, lse, n_valid, grad_loss, chunk_size,
      need_dhidden, need_dweight):
    N, H = hidden.shape
    V = weight.shape[0]
    return (hidden.new_empty((N, H), dtype=hidden.dtype) if need_dhidden else _none(lse),
            hidden.new_empty((V, H), dtype=hidden.dtype) if need_dweight else _none(lse))


# ------------------------------------------------------------------- LoRA --

@torch.library.custom_op(f"{NS}::gemm_f32", mutates_args=(), device_types=_DEV)
def gemm_f32(a_list: List[Tensor], b_list: List[Tensor], a_t: bool, b_t: bool,
             alpha: float) -> Tensor:
    """alpha * sum_s op(a_s) op(b_s), fp32 matrix cores (the fp32 LoRA path)."""
    return hip_ops.gemm_f32(a_list, b_list, a_t, b_t, alpha)


@gemm_f32.register_fake
def _(a_list, b_list, a_t, b_t, alpha):
    M = a_list[0].shape[1] if a_t else a_list[0].shape[0]
    N = b_list[0].shape[0] if b_t else b_list[0].shape[1]
    return a_list[0].new_empty((M, N), dtype=torch.float32)


@torch.library.custom_op(f"{NS}::linear_bf16", mutates_args=(), device_types=_DEV)
def linear_bf16(x2: Tensor, w: Tensor) -> Tensor:
    """x2 w^T on the MFMA engine ([N, in] x [out, in]^T -> [N, out] bf16)."""
    return hip_ops.matmul(x2, w, b_t=True, out_dtype=torch.bfloat16)


@linear_bf16.register_fake
def _(x2, w):
    return x2.new_empty((x2.shape[0], w.shape[0]), dtype=torch.bfloat16)


@torch.library.custom_op(f"{NS}::lora_xa", mutates_args=(), device_types=_DEV)
def lora_xa(x2: Tensor, a_stack: Tensor) -> Tensor:
    return hip_ops.lora_xa(x2, a_stack)


@lora_xa.register_fake
def _(x2, a_stack):
    return x2.new_empty((x2.shape[0], a_stack.shape[0]), dtype=torch.bfloat16)


@torch.library.custom_op(f"{NS}::lora_linear_out", mutates_args=(), device_types=_DEV)
def lora_linear_out(x2: Tensor, w: Tensor, xa: Tensor, sb: Tensor) -> Tensor:
    return hip_ops.lora_linear_out(x2, w, xa, sb)


@lora_linear_out.register_fake
def _(x2, w, xa, sb):
    return x2.new_empty((x2.shape[0], w.shape[0]), dtype=torch.bfloat16)


@torch.library.custom_op(f"{NS}::lora_qkv_out", mutates_args=(), device_types=_DEV)
def lora_qkv_out(x2: Tensor, ws: List[Tensor], xa: Tensor, sbs: List[Tensor]) -> List[Tensor]:
    return hip_ops.lora_qkv_out(x2, ws, xa, sbs)


@lora_qkv_out.register_fake
def _(x2, ws, xa, sbs):
    return [x2.new_empty((x2.shape[0], w.shape[0]), dtype=torch.bfloat16) for w in ws]


# The LoRA backwards return (dX, grads): grads is one fp32 buffer holding the
# adapter gradients as laid out by hip_ops.grad_layout (hip_ops.grad_views
# splits it), so that the caller can cast them to the parameters' dtype in
# one launch.
def _grads_fake(x2, shapes):
    return x2.new_empty((max(hip_ops.grad_layout(shapes)[1], 1),), dtype=torch.float32)


@torch.library.custom_op(f"{NS}::lora_qkv_bwd", mutates_args=(), device_types=_DEV)
def lora_qkv_bwd(x2: Tensor, dys: List[Tensor], ws: List[Tensor], a_stack: Tensor,
                 bs: List[Tensor], scales: List[float], xa: Tensor,
                 rank: int) -> tuple[Tensor, Tensor]:
    return hip_ops.lora_qkv_bwd(x2, dys, ws, a_stack, bs, scales, xa, rank)


@lora_qkv_bwd.register_fake
def _(x2, dys, ws, a_stack, bs, scales, xa, rank):
    N, IN = x2.shape
    shapes = hip_ops.lora_qkv_grad_shapes(IN, [d.shape[1] for d in dys], rank)
    return x2.new_empty((N, IN), dtype=torch.bfloat16), _grads_fake(x2, shapes)


@torch.library.custom_op(f"{NS}::lora_linear_bwd", mutates_args=(), device_types=_DEV)
def lora_linear_bwd(x2: Tensor, dy: Tensor, w: Tensor, a: Tensor, b: Tensor, scale: float,
                    xa: Tensor, rank: int) -> tuple[Tensor, Tensor]:
    return hip_ops.lora_linear_bwd(x2, dy, w, a, b, scale, xa, rank)


@lora_linear_bwd.register_fake
def _(x2, dy, w, a, b, scale, xa, rank):
    N, IN = x2.shape
    shapes = hip_ops.lora_linear_grad_shapes(IN, dy.shape[1], rank)
    return x2.new_empty((N, IN), dtype=torch.bfloat16), _grads_fake(x2, shapes)


@torch.library.custom_op(f"{NS}::lora_mlp_bwd", mutates_args=(), device_types=_DEV)
def lora_mlp_bwd(x2: Tensor, gate: Tensor, up: Tensor, h: Optional[Tensor], dy: Tensor,
                 wg: Tensor, wu: Tensor, wd: Tensor, a_gu: Tensor, a_d: Tensor, bg: Tensor,
                 bu: Tensor, bd: Tensor, scales: List[float], xa_gu: Tensor, ha_d: Tensor,
                 rank: int) -> tuple[Tensor, Tensor]:
    # h None: silu(gate) * up is recomputed by the kernels
    return hip_ops.lora_mlp_bwd(x2, gate, up, h, dy, wg, wu, wd, a_gu, a_d, bg, bu, bd, scales,
                                xa_gu, ha_d, rank)


@lora_mlp_bwd.register_fake
def _(x2, gate, up, h, dy, wg, wu, wd, a_gu, a_d, bg, bu, bd, scales, xa_gu, ha_d, rank):
    N, H = x2.shape
    shapes = hip_ops.lora_mlp_grad_shapes(H, gate.shape[1], rank)
    return x2.new_empty((N, H), dtype=torch.bfloat16), _grads_fake(x2, shapes)
