"""Minimal stand-in for PEFT's LoRA Linear layout (peft is not installed).

Only the attributes the fused LoRA path reads are modelled
(ops/fused_lora.py:53-65 of the reference): base_layer, lora_A / lora_B as
ModuleDicts keyed by adapter name, and scaling[adapter] = lora_alpha / r.
forward() is PEFT's unfused formula, used as the unpatched baseline.
"""

import torch
import torch.nn as nn


class LoraLinear(nn.Module):
    def __init__(self, base: nn.Linear, r: int = 16, alpha: float = 32.0, adapter: str = "default"):
        super().__init__()
        self.base_layer = base
        self.lora_A = nn.ModuleDict({adapter: nn.Linear(base.in_features, r, bias=False)})
        self.lora_B = nn.ModuleDict({adapter: nn.Linear(r, base.out_features, bias=False)})
        self.scaling = {adapter: alpha / r}
        self._adapter = adapter

    @property
    def weight(self):
        return self.base_layer.weight

    def forward(self, x):
        a = self._adapter
        return self.base_layer(x) + self.lora_B[a](self.lora_A[a](x)) * self.scaling[a]


def wrap_lora(module: nn.Module, names, r=16, alpha=32.0):
    """Replaces the named nn.Linear children of module with LoraLinear."""
    for n in names:
        lin = getattr(module, n)
        setattr(module, n, LoraLinear(lin, r=r, alpha=alpha))


def init_lora(lin: "LoraLinear", seed: int, a_std=0.25, b_std=0.02):
    g = torch.Generator().manual_seed(seed)
    A = lin.lora_A[lin._adapter].weight
    B = lin.lora_B[lin._adapter].weight
    with torch.no_grad():
        A.copy_(torch.randn(A.shape, generator=g) * a_std)
        B.copy_(torch.randn(B.shape, generator=g) * b_std)
