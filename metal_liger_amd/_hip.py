"""ctypes binding of libmetal_liger_amd.so and the device/layout guards.

Replaces _metal_dispatch.py (load_metal_source / MetalKernelRegistry,
_metal_dispatch.py:33-85, and the ensure_mps_device / check_contiguous guards,
:88-105). There is exactly one compute path: the HIP library. If it is not
built or the tensors are not on a ROCm GPU, calls raise; nothing falls back to
torch or the CPU.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

LIB_NAME = "libmetal_liger_amd.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME

F32, BF16, F16 = 0, 1, 2
DTYPE_TAG = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_sz = ctypes.c_size_t
_i64p = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes); mirrors include/metal_liger_amd.h
SIGNATURES: dict[str, tuple] = {
    "ml_abi_version": (_i32, []),
    "ml_last_error": (ctypes.c_char_p, []),
    "ml_rmsnorm_fwd": (_i32, [_p, _i64, _p, _p, _i64, _p, _i64, _i64, _f32, _i32, _i32, _p]),
    "ml_rmsnorm_bwd_workspace_bytes": (_sz, [_i64, _i64]),
    "ml_rmsnorm_bwd": (
        _i32,
        [_p, _i64, _p, _p, _i64, _p, _f32, _p, _i64, _p, _p, _sz, _i64, _i64, _i32, _i32, _p],
    ),
    "ml_rmsnorm_bwd_noalloc": (
        _i32, [_p, _i64, _p, _p, _i64, _p, _f32, _p, _i64, _p, _i64, _i64, _i32, _i32, _p],
    ),
    "ml_rmsnorm_add_fwd": (
        _i32, [_p, _i64, _p, _i64, _p, _p, _i64, _p, _i64, _p, _i64, _i64, _f32, _i32, _i32, _p],
    ),
    "ml_rmsnorm_add_bwd": (
        _i32,
        [_p, _i64, _p, _p, _i64, _p, _i64, _p, _f32, _p, _i64, _p, _p, _sz, _i64, _i64, _i32, _i32,
         _p],
    ),
    "ml_swiglu_fwd": (_i32, [_p, _p, _p, _i64, _i32, _p]),
    "ml_swiglu_bwd": (_i32, [_p, _p, _p, _p, _p, _i64, _i32, _p]),
    "ml_rope_table": (
        _i32,
        [_p, _p, _i64p, _p, _p, _i64p, _i64, _p, _p, _i64p, _f32, _i32, _i32, _i32, _p],
    ),
    "ml_rope_pos": (
        _i32,
        [_p, _p, _i64p, _p, _p, _i64p, _i64, _p, _i64, _i64, _p, _f32, _i32, _p],
    ),
    "ml_qk_norm_rope_fwd": (
        _i32,
        [_p, _p, _i64p, _p, _p, _p, _i64p, _p, _i64, _f32, _p, _p, _i64p, _i32, _i32, _p],
    ),
    "ml_qk_norm_rope_bwd_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _i64]),
    "ml_qk_norm_rope_bwd": (
        _i32,
        [_p, _p, _p, _i64p, _p, _p, _p, _p, _p, _i64p, _p, _p, _i64, _f32, _p, _p, _i64p, _i32,
         _i32, _p, _sz, _p],
    ),
    "ml_gemm_bf16": (
        _i32,
        [_i64, _i64, _i64, _p, _i64, _i32, _p, _i64, _i32, _p, _i64, _i32, _f32, _f32, _p],
    ),
    "ml_gemm_bf16_segments": (
        _i32,
        [_i64, _i64, _i32, _i64p, ctypes.POINTER(_p), _i64p, ctypes.POINTER(_p), _i64p, _i32, _i32,
         _p, _i64, _i32, _f32, _f32, _p],
    ),
    "ml_lora_xa": (_i32, [_p, _i64, _i64, _i64, _p, _i64, _p, _i64, _p]),
    "ml_gemm_bf16_segments_group": (
        _i32,
        [_i32, _i64p, _i64p, ctypes.POINTER(_i32), _i64p, ctypes.POINTER(_p), _i64p,
         ctypes.POINTER(_p), _i64p, _i32, ctypes.POINTER(_p), _i64p, _i32, _f32, _f32, _p],
    ),
    "ml_flce_fwd_workspace_bytes": (_sz, [_i64, _i64]),
    "ml_flce_fwd": (
        _i32,
        [_p, _i64, _p, _i64, _p, _i32, _p, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _sz, _p],
    ),
    "ml_flce_bwd_workspace_bytes": (_sz, [_i64, _i64, _i64, _i32]),
    "ml_flce_bwd": (
        _i32,
        [_p, _i64, _p, _i64, _p, _i32, _p, _i64, _i64, _i64, _i64, _p, _p, _p, _i64, _p, _p, _p,
         _sz, _p],
    ),
    "ml_flce_fwd_grad_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _i32]),
    "ml_flce_fwd_grad": (
        _i32,
        [_p, _i64, _p, _i64, _p, _i32, _p, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p,
         _sz, _p],
    ),
    "ml_flce_scale_grads": (_i32, [_p, _p, _i64, _p, _i64, _p]),
    "ml_gemm_f32_segments": (
        _i32,
        [_i64, _i64, _i32, _i64p, ctypes.POINTER(_p), _i64p, ctypes.POINTER(_p), _i64p, _i32, _i32,
         _p, _i64, _f32, _f32, _p],
    ),
    "ml_flce_fwd_grad_f32_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "ml_flce_fwd_grad_f32": (
        _i32,
        [_p, _i64, _p, _i64, _p, _p, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p, _sz, _p],
    ),
    "ml_flce_scale_grads_f32": (_i32, [_p, _p, _i64, _p, _i64, _p]),
    "ml_gemm_splitk_workspace_bytes": (_sz, [_i64, _i64, _i64, _i32]),
    "ml_gemm_bf16_splitk": (
        _i32,
        [_i64, _i64, _i64, _p, _i64, _i32, _p, _i64, _i32, _p, _i64, _i32, _f32, _f32, _i32, _i32,
         _p, _sz, _p],
    ),
    "ml_lora_qkv_bwd_workspace_bytes": (_sz, [_i64, _i64, _i64p, _i64]),
    "ml_lora_qkv_bwd": (
        _i32,
        [_p, _i64, _i64, ctypes.POINTER(_p), _i64p, ctypes.POINTER(_p), _p, ctypes.POINTER(_p),
         ctypes.POINTER(_f32), _p, _i64, _p, _p, ctypes.POINTER(_p), _p, _sz, _p],
    ),
    "ml_lora_linear_bwd_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64]),
    "ml_lora_linear_bwd": (
        _i32,
        [_p, _i64, _i64, _p, _i64, _p, _p, _p, _f32, _p, _i64, _p, _p, _p, _p, _sz, _p],
    ),
    "ml_lora_mlp_bwd_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64]),
    "ml_lora_mlp_bwd": (
        _i32,
        [_p, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p,
         ctypes.POINTER(_f32), _p, _p, _i64, _p, _p, _p, _p, _p, _p, _p, _sz, _p],
    ),
}

ABI_VERSION = 6

_lib = None
_lock = threading.Lock()


class HipLibraryMissing(RuntimeError):
    """The HIP library has not been built (run metal_liger_amd.build)."""


def lib() -> ctypes.CDLL:
    """Loads the HIP library once and declares every C-ABI signature."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise HipLibraryMissing(
                f"metal_liger_amd: {LIB_PATH} is not built; run "
                "`python -m metal_liger_amd.build` (hipcc, gfx950) first"
            )
        handle = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_LOCAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        ver = handle.ml_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(
                f"metal_liger_amd: library ABI {ver} does not match the bindings ({ABI_VERSION})"
            )
        _lib = handle
        return _lib


def call(name: str, *args) -> None:
    """Calls a status-returning entry point; raises RuntimeError on failure."""
    fn = getattr(lib(), name)
    rc = fn(*args)
    if rc != 0:
        msg = lib().ml_last_error()
        raise RuntimeError(f"{name}: {msg.decode(errors='replace') if msg else 'error'} (status {rc})")


def query(name: str, *args):
    return getattr(lib(), name)(*args)


# ------------------------------------------------------------------ helpers --

def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def geom(vals) -> ctypes.Array:
    return (ctypes.c_int64 * len(vals))(*vals)


def ptrs(vals) -> ctypes.Array:
    return (ctypes.c_void_p * len(vals))(*[v for v in vals])


def ints(vals) -> ctypes.Array:
    return (ctypes.c_int * len(vals))(*[int(v) for v in vals])


def floats(vals) -> ctypes.Array:
    return (ctypes.c_float * len(vals))(*[float(v) for v in vals])


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def dtype_tag(t: torch.Tensor, what: str) -> int:
    try:
        return DTYPE_TAG[t.dtype]
    except KeyError:
        raise TypeError(f"metal_liger_amd: {what} has unsupported dtype {t.dtype}") from None


def ensure_rocm_device(*tensors: torch.Tensor | None) -> torch.device:
    """Every tensor must live on the same ROCm GPU (replaces ensure_mps_device)."""
    dev = None
    for i, t in enumerate(tensors):
        if t is None:
            continue
        if t.device.type != "cuda" or torch.version.hip is None:
            raise ValueError(
                f"metal_liger_amd requires ROCm GPU tensors, got {t.device} for tensor {i}. "
                "Move the model to the GPU: model.to('cuda')"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"metal_liger_amd: tensors on different devices ({dev} vs {t.device})")
    return dev


def check_contiguous(*tensors: torch.Tensor) -> None:
    """Same contract as the reference guard (_metal_dispatch.py:98-105)."""
    for i, t in enumerate(tensors):
        if not t.is_contiguous():
            raise ValueError(
                f"metal_liger_amd: tensor {i} is not contiguous. "
                "Call .contiguous() before passing to fused ops."
            )


def rows_view(t: torch.Tensor) -> torch.Tensor:
    """[..., C] -> [R, C] with unit column stride and row stride >= C."""
    c = t.shape[-1]
    t2 = t.reshape(-1, c)
    if t2.shape[0] > 1 and (t2.stride(1) != 1 or t2.stride(0) < c):
        t2 = t2.contiguous()
    elif t2.shape[0] <= 1 and t2.stride(1) != 1:
        t2 = t2.contiguous()
    return t2


def row_stride(t2: torch.Tensor) -> int:
    return t2.stride(0) if t2.shape[0] > 1 else t2.shape[1]
