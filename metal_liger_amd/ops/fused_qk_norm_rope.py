"""Qwen3 attention's q_norm / k_norm fused with rotate-half RoPE.

In a Qwen3 attention forward (transformers' modeling_qwen3.py) the q and k
projections go through a head-dim RMSNorm (Qwen3RMSNorm: fp32 upcast, mean of
squares, rsqrt, scale, cast, weight) and then apply_rotary_pos_emb. The
reference's patcher leaves both steps to torch (patch.py:104-131 replaces only
the layer norms). Here one HIP launch normalises and rotates q and k, and one
launch computes the backward (dx exact for any tables, and the weight
gradients when the norms train).

``patch_qk_norm_rope(model)`` routes every attention that has q_norm /
k_norm through it without replacing modules (state_dict keys unchanged): for
the duration of the attention forward, the two norm modules are shadowed by
identity functions in the instance ``__dict__`` and the forward module's
``apply_rotary_pos_emb`` applies the deferred norms together with the
rotation. A forward that does not call ``apply_rotary_pos_emb`` after the
norms raises instead of silently skipping them.
"""

from __future__ import annotations

import contextvars
import inspect
import logging

import torch
import torch.nn as nn

from metal_liger_amd import _custom_ops as cops
from metal_liger_amd._model_walk import shadowed

logger = logging.getLogger(__name__)

SUPPORTED_HEAD_DIMS = (32, 64, 128, 256)


class _FusedQKNormRoPEFunction(torch.autograd.Function):
    """(q, k) -> (rope(norm_q(q)), rope(norm_k(k))) on [B, H, S, D] inputs."""

    @staticmethod
    def forward(ctx, q, k, q_weight, k_weight, cos, sin, eps: float):
        q_out, k_out = cops.qk_norm_rope_fwd(q, k, q_weight, k_weight, cos, sin, eps)
        ctx.save_for_backward(q, k, q_weight, k_weight, cos, sin)
        ctx.eps = eps
        return q_out, k_out

    @staticmethod
    def backward(ctx, dq_out, dk_out):
        q, k, q_weight, k_weight, cos, sin = ctx.saved_tensors
        if dq_out is None:
            dq_out = torch.zeros_like(q)
        if dk_out is None:
            dk_out = torch.zeros_like(k)
        dq, dk, dwq, dwk = cops.qk_norm_rope_bwd(
            q, k, q_weight, k_weight, cos, sin, ctx.eps, dq_out, dk_out,
            ctx.needs_input_grad[2], ctx.needs_input_grad[3])
        return (dq if ctx.needs_input_grad[0] else None, dk if ctx.needs_input_grad[1] else None,
                cops.maybe(dwq), cops.maybe(dwk), None, None, None)


def _norm_eps(norm: nn.Module) -> float:
    return float(getattr(norm, "variance_epsilon", getattr(norm, "eps", 1e-6)))


def apply_fused_qk_norm_rope(q: torch.Tensor, k: torch.Tensor, q_norm: nn.Module,
                             k_norm: nn.Module, cos: torch.Tensor, sin: torch.Tensor,
                             unsqueeze_dim: int = 1):
    """rope(q_norm(q)), rope(k_norm(k)) as Qwen3's attention computes them.

    q, k: the projections as [B, H, S, D] (HF's transposed views); q_norm /
    k_norm: RMSNorm modules over D (``weight``, ``variance_epsilon``); cos /
    sin as the rotary module returns them ([B, S, D]), unsqueezed at
    ``unsqueeze_dim`` to broadcast against q, as apply_rotary_pos_emb does.
    """
    eps = _norm_eps(q_norm)
    if _norm_eps(k_norm) != eps:
        raise ValueError("fused q/k norm: q_norm and k_norm must share eps")
    return _FusedQKNormRoPEFunction.apply(q, k, q_norm.weight, k_norm.weight,
                                          cos.unsqueeze(unsqueeze_dim), sin.unsqueeze(unsqueeze_dim),
                                          eps)


# ------------------------------------------------------------------ patching --

class _Deferred:
    """The norms an attention forward has deferred to its rotary step."""

    __slots__ = ("q_norm", "k_norm", "used")

    def __init__(self, q_norm, k_norm):
        self.q_norm = q_norm
        self.k_norm = k_norm
        self.used = False


_ACTIVE: contextvars.ContextVar = contextvars.ContextVar("metal_liger_qk_norm", default=None)


def _identity(x):
    return x


def _rotary_dispatch(original):
    """apply_rotary_pos_emb that applies the deferred norms with the rotation
    inside a patched attention forward, and is ``original`` everywhere else."""
    sig = inspect.signature(original)

    def apply_rotary_pos_emb(q, k, cos, sin, *args, **kwargs):
        st = _ACTIVE.get()
        if st is None or st.used:
            return original(q, k, cos, sin, *args, **kwargs)
        bound = sig.bind(q, k, cos, sin, *args, **kwargs)
        bound.apply_defaults()
        if bound.arguments.get("position_ids") is not None:
            raise ValueError("fused q/k norm: position_ids in apply_rotary_pos_emb is not supported")
        st.used = True
        return apply_fused_qk_norm_rope(q, k, st.q_norm, st.k_norm, cos, sin,
                                        int(bound.arguments.get("unsqueeze_dim", 1)))

    apply_rotary_pos_emb._metal_liger_original = original
    return apply_rotary_pos_emb


def _install_dispatch(forward_fn) -> bool:
    """Replaces apply_rotary_pos_emb in the globals of the module defining
    forward_fn (once); False when that module has none."""
    g = getattr(forward_fn, "__globals__", None)
    if g is None or "apply_rotary_pos_emb" not in g:
        return False
    cur = g["apply_rotary_pos_emb"]
    if not hasattr(cur, "_metal_liger_original"):
        g["apply_rotary_pos_emb"] = _rotary_dispatch(cur)
    return True


def _eligible(attn: nn.Module) -> bool:
    qn, kn = getattr(attn, "q_norm", None), getattr(attn, "k_norm", None)
    if qn is None or kn is None or getattr(qn, "weight", None) is None or \
            getattr(kn, "weight", None) is None:
        return False
    d = qn.weight.shape[0]
    return (qn.weight.dim() == 1 and kn.weight.shape == qn.weight.shape and
            d in SUPPORTED_HEAD_DIMS and getattr(attn, "head_dim", d) == d and
            _norm_eps(qn) == _norm_eps(kn))


def _make_forward(attn: nn.Module, orig_fwd):
    def forward(hidden_states, *args, **kwargs):
        st = _Deferred(attn.q_norm, attn.k_norm)
        token = _ACTIVE.set(st)
        try:
            with shadowed(attn, q_norm=_identity, k_norm=_identity):
                out = orig_fwd(hidden_states, *args, **kwargs)
        finally:
            _ACTIVE.reset(token)
        if not st.used:
            raise RuntimeError(
                f"fused q/k norm: {type(attn).__name__}.forward did not call apply_rotary_pos_emb "
                "after q_norm / k_norm; the norms would be skipped")
        return out

    return forward


def patch_qk_norm_rope(model: nn.Module) -> int:
    """Routes every attention module with q_norm / k_norm (head dim 32, 64,
    128 or 256, shared eps) whose forward calls apply_rotary_pos_emb through the
    fused norm + RoPE. Returns the number of patched modules."""
    count = 0
    for mod in model.modules():
        if not hasattr(mod, "q_proj") or getattr(mod, "_metal_liger_qk_norm_rope", False):
            continue
        if not _eligible(mod):
            continue
        fwd_fn = getattr(type(mod).forward, "__func__", type(mod).forward)
        if not _install_dispatch(fwd_fn):
            continue
        mod.forward = _make_forward(mod, mod.forward)
        mod._metal_liger_qk_norm_rope = True
        count += 1
    logger.info(f"MetalLiger fused q/k norm + RoPE: activated on {count} attention modules.")
    return count
