"""Locating decoder layers in wrapped HuggingFace models, and temporarily
shadowing submodules of one module instance.

Shared by the model patcher (patch.py) and the per-block patchers
(ops/fused_lora.py, ops/fused_qk_norm_rope.py,
ops/fused_linear_cross_entropy.py).

Layer search: the wrapping layouts the reference's patcher walks
(patch.py:27-64 and ops/fused_lora.py:347-363: bare HF decoder, causal LM,
PEFT's ``base_model.model``, Qwen3-VL's ``language_model``, an accelerate
``module`` wrapper) as a table of attribute paths, most specific first; a
model none of them fits is searched for the first non-empty ModuleList
called ``layers`` in module order.

Shadowing: ``shadowed(module, q_proj=f, ...)`` makes ``module.q_proj``
resolve to ``f`` inside a ``with`` block without touching ``_modules``
(instance ``__dict__`` entries take precedence over nn.Module's attribute
lookup), so state_dict keys, hooks on the real submodules and parameter
registration are unchanged, and restores whatever the instance dict held
before on exit, also when the block raises.
"""

from __future__ import annotations

import contextlib

import torch.nn as nn

# Attribute paths to the decoder-layer list, most specific first.
LAYER_PATHS = (
    ("base_model", "model", "model", "language_model", "layers"),  # PEFT + Qwen3-VL
    ("base_model", "model", "model", "layers"),                    # PEFT + causal LM
    ("model", "language_model", "layers"),                         # Qwen3-VL
    ("model", "layers"),                                           # HF causal LM
    ("layers",),                                                   # bare decoder
    ("module", "model", "layers"),                                 # accelerate wrapper
)

# Attribute paths to the final norm's parent (patch.py:67-89 of the reference).
NORM_PARENT_PATHS = (
    ("base_model", "model", "model", "language_model"),
    ("model", "language_model"),
    ("base_model", "model", "model"),
    ("model",),
)


def resolve(obj, path):
    """obj.path[0].path[1]... or None where an attribute is missing."""
    for name in path:
        obj = getattr(obj, name, None)
        if obj is None:
            return None
    return obj


def find_layers(model: nn.Module):
    """The model's decoder-layer list: the first non-empty one along
    LAYER_PATHS, else the first non-empty ModuleList named ``layers`` in
    module order, else None."""
    for path in LAYER_PATHS:
        try:
            layers = resolve(model, path)
            if layers is not None and len(layers) > 0:
                return layers
        except (AttributeError, TypeError):
            continue
    for name, mod in model.named_modules():
        if name.rsplit(".", 1)[-1] == "layers" and isinstance(mod, nn.ModuleList) and len(mod):
            return mod
    return None


def find_final_norm(model: nn.Module):
    """(norm module, parent) of the final norm, or (None, None)."""
    for path in NORM_PARENT_PATHS:
        parent = resolve(model, path)
        norm = getattr(parent, "norm", None) if parent is not None else None
        if norm is not None and hasattr(norm, "weight"):
            return norm, parent
    return None, None


_MISSING = object()


@contextlib.contextmanager
def shadowed(module: nn.Module, **replacements):
    """Within the block, ``module.<name>`` is ``replacements[name]``; the
    instance dict is restored on exit (see the module docstring)."""
    d = module.__dict__
    saved = {name: d.get(name, _MISSING) for name in replacements}
    d.update(replacements)
    try:
        yield module
    finally:
        for name, old in saved.items():
            if old is _MISSING:
                d.pop(name, None)
            else:
                d[name] = old
