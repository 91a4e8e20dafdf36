"""torch.library registration of the native ops (replaces _torch_library.py).

Registers the reference's two operators with the same schemas
(_torch_library.py:44-76 of the reference) plus their backward counterparts,
with implementations for PyTorch-ROCm's GPU dispatch key ("CUDA") and fake
(meta) kernels for tracing:

    metal_liger::rms_norm_forward(Tensor x, Tensor weight, float eps, str kernel_dir) -> (Tensor, Tensor)
    metal_liger::swiglu_forward(Tensor gate, Tensor up, str kernel_dir) -> Tensor
    metal_liger::rms_norm_backward(Tensor x, Tensor weight, Tensor grad_out, float eps, str kernel_dir) -> (Tensor, Tensor)
    metal_liger::swiglu_backward(Tensor gate, Tensor up, Tensor grad_out, str kernel_dir) -> (Tensor, Tensor)

The Library object is kept at module level: a definition made through a
temporary Library disappears when that object is collected.
"""

import logging

import torch
from torch import Tensor

logger = logging.getLogger(__name__)

_REGISTERED = False
_LIB = None


def register_metal_liger_ops():
    """Registers the ops once; no-op when the HIP library is not built."""
    global _REGISTERED, _LIB
    if _REGISTERED:
        return
    try:
        from metal_liger_amd import _hip
        if not _hip.LIB_PATH.exists():
            raise ImportError(str(_hip.LIB_PATH))
        from metal_liger_amd import metal_liger_ext as ext
    except ImportError:
        logger.debug("metal_liger: HIP library not built; skipping torch.library registration")
        return
    try:
        lib = torch.library.Library("metal_liger", "DEF")
        lib.define("rms_norm_forward(Tensor x, Tensor weight, float eps, str kernel_dir) -> (Tensor, Tensor)")
        lib.define("swiglu_forward(Tensor gate, Tensor up, str kernel_dir) -> Tensor")
        lib.define("rms_norm_backward(Tensor x, Tensor weight, Tensor grad_out, float eps, "
                   "str kernel_dir) -> (Tensor, Tensor)")
        lib.define("swiglu_backward(Tensor gate, Tensor up, Tensor grad_out, str kernel_dir) "
                   "-> (Tensor, Tensor)")

        def _rms_fwd(x: Tensor, weight: Tensor, eps: float, kernel_dir: str):
            out, cache = ext.rms_norm_forward(x, weight, eps, kernel_dir)
            return out, cache

        def _rms_bwd(x: Tensor, weight: Tensor, grad_out: Tensor, eps: float, kernel_dir: str):
            gx, gw = ext.rms_norm_backward(x, weight, grad_out, eps, kernel_dir)
            return gx, gw

        def _swiglu_fwd(gate: Tensor, up: Tensor, kernel_dir: str):
            return ext.swiglu_forward(gate, up, kernel_dir)

        def _swiglu_bwd(gate: Tensor, up: Tensor, grad_out: Tensor, kernel_dir: str):
            dg, du = ext.swiglu_backward(gate, up, grad_out, kernel_dir)
            return dg, du

        lib.impl("rms_norm_forward", _rms_fwd, "CUDA")
        lib.impl("rms_norm_backward", _rms_bwd, "CUDA")
        lib.impl("swiglu_forward", _swiglu_fwd, "CUDA")
        lib.impl("swiglu_backward", _swiglu_bwd, "CUDA")

        @torch.library.register_fake("metal_liger::rms_norm_forward", lib=lib)
        def _rms_fwd_fake(x, weight, eps, kernel_dir):
            rows = 1
            for d in x.shape[:-1]:
                rows *= d
            return torch.empty_like(x), x.new_empty((rows,), dtype=torch.float32)

        @torch.library.register_fake("metal_liger::rms_norm_backward", lib=lib)
        def _rms_bwd_fake(x, weight, grad_out, eps, kernel_dir):
            return torch.empty_like(x), torch.empty_like(weight)

        @torch.library.register_fake("metal_liger::swiglu_forward", lib=lib)
        def _swiglu_fwd_fake(gate, up, kernel_dir):
            return torch.empty_like(gate)

        @torch.library.register_fake("metal_liger::swiglu_backward", lib=lib)
        def _swiglu_bwd_fake(gate, up, grad_out, kernel_dir):
            return torch.empty_like(gate), torch.empty_like(up)

        _LIB = lib
        _REGISTERED = True
        logger.info("metal_liger: registered metal_liger::{rms_norm,swiglu}_{forward,backward}")
    except Exception as e:  # same contract as the reference: log and continue
        logger.warning(f"metal_liger: torch.library registration failed — {e}")
