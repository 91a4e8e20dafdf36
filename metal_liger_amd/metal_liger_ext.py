"""The reference's native-extension surface, backed by the HIP library.

Same functions, argument names and return structure as the pybind module
``metal_liger_ext`` (csrc/bindings.mm:10-33, csrc/metal_liger_ops.h:13-36).
``kernel_dir`` is accepted for signature compatibility and ignored: the
kernels are compiled ahead of time into libmetal_liger_amd.so.
"""

from __future__ import annotations

from typing import List

import torch

from metal_liger_amd import hip_ops


def rms_norm_forward(x: torch.Tensor, weight: torch.Tensor, eps: float,
                     kernel_dir: str = "") -> List[torch.Tensor]:
    """[output (x's shape and dtype), rms_cache (fp32, [tokens])]
    (csrc/rms_norm_metal.mm:110-160)."""
    if x.dim() < 2:
        raise RuntimeError("metal_liger_amd RMSNorm: input must be >=2D")
    out, rrms = hip_ops.rms_norm_fwd(x, weight, eps)
    return [out, rrms.reshape(-1)]


def rms_norm_backward(x: torch.Tensor, weight: torch.Tensor, grad_out: torch.Tensor, eps: float,
                      kernel_dir: str = "") -> List[torch.Tensor]:
    """[grad_x, grad_weight]; rrms is recomputed from x and eps, as the
    reference's native backward does (csrc/rms_norm_metal.mm:164-214)."""
    gx, gw = hip_ops.rms_norm_bwd(x, weight, grad_out, None, eps)
    return [gx, gw]


def swiglu_forward(gate: torch.Tensor, up: torch.Tensor, kernel_dir: str = "") -> torch.Tensor:
    """SiLU(gate) * up (csrc/swiglu_metal.mm:66-100)."""
    if gate.shape != up.shape:
        raise RuntimeError("metal_liger_amd SwiGLU: gate and up must match")
    return hip_ops.swiglu_fwd(gate, up)


def swiglu_backward(gate: torch.Tensor, up: torch.Tensor, grad_out: torch.Tensor,
                    kernel_dir: str = "") -> List[torch.Tensor]:
    """[grad_gate, grad_up] with sigmoid recomputed (csrc/swiglu_metal.mm:106-144)."""
    dg, du = hip_ops.swiglu_bwd(gate, up, grad_out)
    return [dg, du]
