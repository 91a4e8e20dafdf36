"""Import alias: ``import metal_liger`` resolves to metal_liger_amd.

Code written against the reference package (``from metal_liger import
apply_metal_liger_to_qwen3vl``, ``from metal_liger.ops.fused_lora import
apply_fused_lora_qkv``, ``import metal_liger_ext``) runs unchanged on the
MI355X build: every module path of the reference that exists here maps to
the corresponding metal_liger_amd module.
"""

import importlib
import sys

import metal_liger_amd as _impl

_SUBMODULES = (
    "ops",
    "ops.fused_rms_norm",
    "ops.fused_swiglu",
    "ops.fused_rope",
    "ops.fused_linear_cross_entropy",
    "ops.fused_lora",
    "patch",
    "_torch_library",
    "_compile",
    "metal_liger_ext",
)

for _name in _SUBMODULES:
    sys.modules[f"{__name__}.{_name}"] = importlib.import_module(f"metal_liger_amd.{_name}")
sys.modules.setdefault("metal_liger_ext", sys.modules[f"{__name__}.metal_liger_ext"])

from metal_liger_amd import *  # noqa: E402,F401,F403
from metal_liger_amd import __all__, __version__  # noqa: E402,F401

ops = sys.modules[f"{__name__}.ops"]
patch = sys.modules[f"{__name__}.patch"]
