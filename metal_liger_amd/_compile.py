"""torch.compile helper — kept for API compatibility only.

The reference's apply_compile (_compile.py:369-379) is a deprecated no-op
that logs and returns the model; the rest of that module is an MPS
graph-capture helper that metal_liger_amd does not include (the fused ops are
ahead-of-time HIP kernels and need no tracing compiler).
"""

import logging

import torch.nn as nn

logger = logging.getLogger(__name__)


def apply_compile(model: nn.Module, **kwargs) -> nn.Module:
    """Deprecated no-op: logs and returns the model unchanged."""
    logger.warning("MetalLiger: apply_compile() is deprecated; skipping compile.")
    return model
