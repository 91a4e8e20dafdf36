"""Fused LoRA QKV + MLP on MI355X (drop-in for the reference's ops/fused_lora.py).

X is saved once per fused block (as in the reference), and the backward of
each block is a single call into the HIP library:

* QKV (`_LoRA_QKV`): P_i = s_i dY_i B_i and dB_i = s_i dY_i^T (X A_i^T)
  come from one streaming pass over each dY_i, dA = P^T X from one pass
  over X (rank 16; other ranks use split-K products on narrow MFMA tiles);
  the shared dX is ONE MFMA GEMM over the K-concatenation
  [dQ | dK | dV | P] x [Wq; Wk; Wv; A_q; A_k; A_v].
* MLP (`_LoRA_MLP`): dH = dY W_D + s (dY B_D) A_D in one MFMA GEMM, the
  SwiGLU backward over it in place (sigmoid recomputed), writing d_gate /
  d_up; then the gate / up adapters as above, and dX as one GEMM over
  [d_gate | d_up | P] x [W_G; W_U; A_G; A_U].
* One projection (`_LoRA_W`, o_proj): the same backward with one adapter;
  the patcher routes an attention's o_proj through it when it has LoRA.

The forward passes also run on the MFMA engine: X A^T for the stacked A
matrices (saved for the backward, where the reference recomputed it) and
each output as one GEMM over [X | X A^T] x [W; s B]^T.

Semantics kept from the reference (ops/fused_lora.py:43-421): PEFT parameter
layout (first adapter only, dropout ignored), A/B cast to the activation
dtype, dA/dB returned in fp32, no gradient for the frozen base weights, and
the patcher shadows q/k/v_proj without replacing modules (state_dict keys
unchanged). bf16 activations run the bf16 MFMA kernels above; fp32 (and,
upcast, fp16) activations run fp32 matrix-core products of the same
formulas (gemm_f32: forward [X | X A^T] x [W; s B]^T, backward P = s dY B,
dA = P^T X, dB = s dY^T (X A^T), dX one K-concatenated product).
"""

import logging

import torch
import torch.nn as nn

from metal_liger_amd import _custom_ops as cops
from metal_liger_amd import hip_ops
from metal_liger_amd._model_walk import find_layers, shadowed

logger = logging.getLogger(__name__)


def _get_lora_params(linear):
    """(W, A, B, scaling) of a PEFT LoRA Linear, else (None,)*4
    (ops/fused_lora.py:43-66): first adapter, base weight from base_layer."""
    if not hasattr(linear, 'lora_A'):
        return None, None, None, None
    adapters = list(linear.lora_A.keys())
    if not adapters:
        return None, None, None, None
    adapter = adapters[0]
    W = linear.base_layer.weight if hasattr(linear, 'base_layer') else linear.weight
    A = linear.lora_A[adapter].weight   # [r, in_features]
    B = linear.lora_B[adapter].weight   # [out_features, r]
    scaling = linear.scaling[adapter]
    return W, A, B, scaling


def _fp32_path(X: torch.Tensor, *features: int) -> bool:
    """Whether a LoRA Function runs on the fp32 kernels: activations that are
    not bf16 (fp16 is upcast), and bf16 activations whose feature sizes are
    not all multiples of 8 (the bf16 MFMA kernels move 8 elements per access;
    the fp32 ones take any size, and the result is cast back to bf16)."""
    return X.dtype != torch.bfloat16 or any(int(f) % 8 for f in features)


def _check_float(X: torch.Tensor, what: str):
    if not X.is_floating_point():
        raise TypeError(f"metal_liger_amd {what}: activations must be floating point (got {X.dtype})")


# ---------------------------------------------------------- fp32 building blocks --
# Activations other than bf16 run in fp32 on the fp32 matrix cores (fp16 is
# upcast, as the reference's fp32 upcasts elsewhere; outputs and dX are cast
# back to the activation dtype, dA / dB are fp32 as in the reference).

def _f32(t: torch.Tensor) -> torch.Tensor:
    return t.detach().float()


def _lora_out_f32(X2, W, A, B, s):
    """(X W^T + (X A^T) (s B)^T, X A^T) in fp32 (ops/fused_lora.py:69-82)."""
    xa = cops.gemm_f32([X2], [_f32(A)], False, True, 1.0)
    out = cops.gemm_f32([X2, xa], [_f32(W), _f32(B) * float(s)], False, True, 1.0)
    return out, xa


def _adapter_grads_f32(dY, X2, xa, B, s):
    """P = s dY B, dA = P^T X, dB = s dY^T (X A^T) in fp32
    (ops/fused_lora.py:121-171)."""
    P = cops.gemm_f32([dY], [B], False, False, float(s))
    dA = cops.gemm_f32([P], [X2], True, False, 1.0)
    dB = cops.gemm_f32([dY], [xa], True, False, float(s))
    return P, dA, dB


def _rows_f32(t: torch.Tensor) -> torch.Tensor:
    return t.reshape(-1, t.shape[-1]).float()


def _pad_rank(r: int) -> int:
    return (r + 7) // 8 * 8


def _stack_a(As, rp: int) -> torch.Tensor:
    """[A_1; A_2; ...] in bf16, each padded with zero rows to rp."""
    parts = []
    for A in As:
        a = A.detach().to(torch.bfloat16)
        if a.shape[0] != rp:
            a = torch.cat([a, a.new_zeros(rp - a.shape[0], a.shape[1])], 0)
        parts.append(a)
    return torch.cat(parts, 0).contiguous()


def _pad_b(B: torch.Tensor, rp: int, scale: float = 1.0) -> torch.Tensor:
    """B (optionally times the LoRA scale) in bf16, padded with zero columns to rp."""
    b = B.detach().to(torch.bfloat16)
    if scale != 1.0:
        b = b * scale
    if b.shape[1] != rp:
        b = torch.cat([b, b.new_zeros(b.shape[0], rp - b.shape[1])], 1)
    return b.contiguous()


def _adapter_grads(flat, shapes, dtypes):
    """The adapter gradients of one fused backward call, from the fp32
    buffer it returns (hip_ops.grad_layout): cast once to the adapters' dtype
    when they share one, instead of autograd casting each gradient in a
    launch of its own."""
    if len(set(dtypes)) == 1 and dtypes[0] != flat.dtype:
        flat = flat.to(dtypes[0])
    return hip_ops.grad_views(flat, shapes)


def _lora_linear(X: torch.Tensor, W: torch.Tensor,
                 A: torch.Tensor, B: torch.Tensor, scaling: float) -> torch.Tensor:
    """X W^T + s (X A^T) B^T (ops/fused_lora.py:69-82) on the MFMA engine
    (bf16 activations: bf16 products; other float dtypes, and feature sizes
    that are not multiples of 8: fp32 products)."""
    _check_float(X, "_lora_linear")
    shape = X.shape
    if _fp32_path(X, X.shape[-1], W.shape[0]):
        X2 = _rows_f32(X)
        if A is None or B is None:
            out = cops.gemm_f32([X2], [_f32(W)], False, True, 1.0)
        else:
            out, _ = _lora_out_f32(X2, W, A, B, scaling)
        return out.to(X.dtype).view(*shape[:-1], out.shape[-1])
    X2 = hip_ops._bf16_rows(X.reshape(-1, shape[-1]))
    W2 = hip_ops._bf16_rows(W.detach())
    if A is None or B is None:
        out = cops.linear_bf16(X2, W2)
    else:
        rp = _pad_rank(A.shape[0])
        xa = cops.lora_xa(X2, _stack_a([A], rp))
        out = cops.lora_linear_out(X2, W2, xa, _pad_b(B, rp, float(scaling)))
    return out.view(*shape[:-1], out.shape[-1])


class _LoRA_QKV(torch.autograd.Function):
    """Fused Q+K+V LoRA projections — X saved once for all three backward
    passes (ops/fused_lora.py:85-171)."""

    @staticmethod
    def forward(ctx,
                X,
                QW, QA, QB, QS,
                KW, KA, KB, KS,
                VW, VA, VB, VS):
        _check_float(X, "LoRA QKV")
        shape = X.shape
        ctx.fp32 = _fp32_path(X, X.shape[-1], QW.shape[0], KW.shape[0], VW.shape[0])
        if ctx.fp32:
            X2 = _rows_f32(X)
            outs, xas = [], []
            for W, A, B, S in ((QW, QA, QB, QS), (KW, KA, KB, KS), (VW, VA, VB, VS)):
                o, xa = _lora_out_f32(X2, W, A, B, S)
                outs.append(o.to(X.dtype).view(*shape[:-1], o.shape[-1]))
                xas.append(xa)
            # the parameters as given (upcast per use in the backward): an fp32
            # copy of every frozen base weight would live until the backward
            ctx.save_for_backward(X2, *xas, *(W.detach() for W in (QW, KW, VW)),
                                  *(A.detach() for A in (QA, KA, VA)),
                                  *(B.detach() for B in (QB, KB, VB)))
            ctx.scales = [float(QS), float(KS), float(VS)]
            ctx.orig_shape, ctx.x_dtype = shape, X.dtype
            return tuple(outs)
        Xf = hip_ops._bf16_rows(X.reshape(-1, shape[-1]))
        # adapters of different ranks (PEFT rank_pattern) are padded to the
        # largest: zero A rows and B columns add nothing to the output and get
        # zero gradients, which the backward slices off
        ranks = [A.shape[0] for A in (QA, KA, VA)]
        rp = _pad_rank(max(ranks))
        a_stack = _stack_a([QA, KA, VA], rp)
        xa = cops.lora_xa(Xf, a_stack)                         # [N, 3 rp], saved
        Ws = [hip_ops._bf16_rows(W.detach()) for W in (QW, KW, VW)]
        Bs = [_pad_b(B, rp) for B in (QB, KB, VB)]
        scales = [float(QS), float(KS), float(VS)]
        sbs = [Bs[i] * scales[i] if scales[i] != 1.0 else Bs[i] for i in range(3)]
        # the three projections in one launch: k and v alone would each leave
        # half of the GPU idle for a round of tiles
        outs = cops.lora_qkv_out(Xf, Ws, xa, sbs)
        ctx.save_for_backward(Xf, xa, a_stack, *Ws, *Bs)
        ctx.scales = scales
        ctx.ranks, ctx.rank_p = ranks, rp
        ctx.orig_shape = shape
        ctx.param_dtypes = [(A.dtype, B.dtype) for A, B in ((QA, QB), (KA, KB), (VA, VB))]
        return tuple(o.view(*shape[:-1], o.shape[-1]) for o in outs)

    @staticmethod
    def backward(ctx, dQ, dK, dV):
        if ctx.fp32:
            X2, *rest = ctx.saved_tensors
            xas, Ws, As, Bs = rest[0:3], rest[3:6], rest[6:9], rest[9:12]
            dys = [_rows_f32(d) for d in (dQ, dK, dV)]
            grads, a_ops, b_ops = [], [], []
            for dy, xa, W, A, B, s in zip(dys, xas, Ws, As, Bs, ctx.scales):
                P, dA, dB = _adapter_grads_f32(dy, X2, xa, _f32(B), s)
                grads.append((dA, dB))
                a_ops += [dy, P]
                b_ops += [_f32(W), _f32(A)]
            dX = cops.gemm_f32(a_ops, b_ops, False, False, 1.0)
            dX = dX.to(ctx.x_dtype).view(*ctx.orig_shape)
            return (dX,
                    None, grads[0][0], grads[0][1], None,
                    None, grads[1][0], grads[1][1], None,
                    None, grads[2][0], grads[2][1], None)
        Xf, xa, a_stack, QW, KW, VW, QB, KB, VB = ctx.saved_tensors
        ranks, rp = ctx.ranks, ctx.rank_p
        shape = ctx.orig_shape
        dys = [hip_ops._bf16_rows(d.reshape(-1, d.shape[-1])) for d in (dQ, dK, dV)]
        dX, flat = cops.lora_qkv_bwd(Xf, dys, [QW, KW, VW], a_stack, [QB, KB, VB],
                                     ctx.scales, xa, rp)
        shapes = hip_ops.lora_qkv_grad_shapes(Xf.shape[1], [d.shape[1] for d in dys], rp)
        dA, *dBs = _adapter_grads(flat, shapes, [t for pair in ctx.param_dtypes for t in pair])
        grads = []
        for i in range(3):
            dAi = dA[i * rp:i * rp + ranks[i]]
            dBi = dBs[i][:, :ranks[i]]
            grads.append((dAi, dBi))
        dX = dX.view(*shape)
        return (dX,
                None, grads[0][0], grads[0][1], None,   # QW, QA, QB, QS
                None, grads[1][0], grads[1][1], None,   # KW, KA, KB, KS
                None, grads[2][0], grads[2][1], None)   # VW, VA, VB, VS


class _LoRA_MLP(torch.autograd.Function):
    """Fused gate+up+down LoRA MLP with SwiGLU (ops/fused_lora.py:174-266)."""

    @staticmethod
    def forward(ctx,
                X,
                GW, GA, GB, GS,   # gate projection
                UW, UA, UB, US,   # up projection
                DW, DA, DB, DS):  # down projection
        _check_float(X, "LoRA MLP")
        shape = X.shape
        ctx.fp32 = _fp32_path(X, X.shape[-1], GW.shape[0])
        if ctx.fp32:
            X2 = _rows_f32(X)
            gate, xa_g = _lora_out_f32(X2, GW, GA, GB, GS)
            up, xa_u = _lora_out_f32(X2, UW, UA, UB, US)
            h = cops.swiglu_fwd(gate, up)                          # silu(gate) * up, fp32
            out, ha = _lora_out_f32(h, DW, DA, DB, DS)
            ctx.save_for_backward(X2, gate, up, h, xa_g, xa_u, ha,
                                  *(t.detach() for t in (GW, UW, DW, GA, UA, DA, GB, UB, DB)))
            ctx.scales = [float(GS), float(US), float(DS)]
            ctx.orig_shape, ctx.x_dtype = shape, X.dtype
            return out.to(X.dtype).view(*shape[:-1], out.shape[-1])
        Xf = hip_ops._bf16_rows(X.reshape(-1, shape[-1]))
        ranks = [A.shape[0] for A in (GA, UA, DA)]  # padded to the largest, as in _LoRA_QKV
        rp = _pad_rank(max(ranks))
        scales = [float(GS), float(US), float(DS)]
        a_gu = _stack_a([GA, UA], rp)                            # [2 rp, hidden]
        a_d = _stack_a([DA], rp)                                 # [rp, inter]
        GWc, UWc, DWc = (hip_ops._bf16_rows(W.detach()) for W in (GW, UW, DW))
        BG, BU, BD = (_pad_b(B, rp) for B in (GB, UB, DB))
        xa_gu = cops.lora_xa(Xf, a_gu)                            # [N, 2 rp]
        gate = cops.lora_linear_out(Xf, GWc, xa_gu[:, :rp], BG * scales[0])
        up = cops.lora_linear_out(Xf, UWc, xa_gu[:, rp:], BU * scales[1])
        h = cops.swiglu_fwd(gate, up)                             # silu(gate) * up, bf16
        ha_d = cops.lora_xa(h, a_d)                               # [N, rp]
        out = cops.lora_linear_out(h, DWc, ha_d, BD * scales[2])
        # h is not saved: the backward recomputes it from gate and up (the
        # same kernel math, so the same bits), one [N, inter] tensor less
        ctx.save_for_backward(Xf, gate, up, xa_gu, ha_d, a_gu, a_d, GWc, UWc, DWc, BG, BU, BD)
        ctx.scales = scales
        ctx.param_dtypes = [t.dtype for t in (GA, UA, DA, GB, UB, DB)]
        ctx.ranks, ctx.rank_p = ranks, rp
        ctx.orig_shape = shape
        return out.view(*shape)

    @staticmethod
    def backward(ctx, dY):
        if ctx.fp32:
            (X2, gate, up, h, xa_g, xa_u, ha, *params) = ctx.saved_tensors
            GW, UW, DW, GA, UA, DA, GB, UB, DB = (_f32(t) for t in params)
            sg, su, sd = ctx.scales
            dy = _rows_f32(dY)
            PD, dA_D, dB_D = _adapter_grads_f32(dy, h, ha, DB, sd)
            dH = cops.gemm_f32([dy, PD], [DW, DA], False, False, 1.0)
            d_gate, d_up = cops.swiglu_bwd(gate, up, dH)
            PG, dA_G, dB_G = _adapter_grads_f32(d_gate, X2, xa_g, GB, sg)
            PU, dA_U, dB_U = _adapter_grads_f32(d_up, X2, xa_u, UB, su)
            dX = cops.gemm_f32([d_gate, PG, d_up, PU], [GW, GA, UW, UA], False, False, 1.0)
            dX = dX.to(ctx.x_dtype).view(*ctx.orig_shape)
            return (dX,
                    None, dA_G, dB_G, None,
                    None, dA_U, dB_U, None,
                    None, dA_D, dB_D, None)
        (Xf, gate, up, xa_gu, ha_d, a_gu, a_d, GW, UW, DW, BG, BU, BD) = ctx.saved_tensors
        (rg, ru, rd), rp = ctx.ranks, ctx.rank_p
        shape = ctx.orig_shape
        dy = hip_ops._bf16_rows(dY.reshape(-1, dY.shape[-1]))
        dX, flat = cops.lora_mlp_bwd(
            Xf, gate, up, None, dy, GW, UW, DW, a_gu, a_d, BG, BU, BD, ctx.scales, xa_gu, ha_d, rp)
        shapes = hip_ops.lora_mlp_grad_shapes(Xf.shape[1], gate.shape[1], rp)
        dA_GU, dA_D, dB_G, dB_U, dB_D = _adapter_grads(flat, shapes, ctx.param_dtypes)
        dX = dX.view(*shape)
        return (dX,
                None, dA_GU[:rg], dB_G[:, :rg], None,        # GW, GA, GB, GS
                None, dA_GU[rp:rp + ru], dB_U[:, :ru], None,  # UW, UA, UB, US
                None, dA_D[:rd], dB_D[:, :rd], None)          # DW, DA, DB, DS


class _LoRA_W(torch.autograd.Function):
    """One projection with LoRA, X W^T + s (X A^T) B^T: the "LoRA_W" block
    (output / o_proj) the reference announces but does not implement
    (ops/fused_lora.py:26), with _lora_linear's forward (:69-82) and the
    per-adapter backward of _LoRA_QKV (:121-171). X A^T is saved from the
    forward; the backward is one library call (rank-r products and one
    K-concatenated dX GEMM [dY | P] x [W; A])."""

    @staticmethod
    def forward(ctx, X, W, A, B, S):
        _check_float(X, "LoRA projection")
        shape = X.shape
        ctx.fp32 = _fp32_path(X, X.shape[-1], W.shape[0])
        if ctx.fp32:
            X2 = _rows_f32(X)
            out, xa = _lora_out_f32(X2, W, A, B, S)
            ctx.save_for_backward(X2, xa, W.detach(), A.detach(), B.detach())
            ctx.scale, ctx.orig_shape, ctx.x_dtype = float(S), shape, X.dtype
            return out.to(X.dtype).view(*shape[:-1], out.shape[-1])
        Xf = hip_ops._bf16_rows(X.reshape(-1, shape[-1]))
        r = A.shape[0]
        rp = _pad_rank(r)
        a = _stack_a([A], rp)
        xa = cops.lora_xa(Xf, a)                                 # [N, rp], saved
        Wc = hip_ops._bf16_rows(W.detach())
        Bp = _pad_b(B, rp)
        scale = float(S)
        out = cops.lora_linear_out(Xf, Wc, xa, Bp * scale if scale != 1.0 else Bp)
        ctx.save_for_backward(Xf, xa, a, Wc, Bp)
        ctx.scale = scale
        ctx.param_dtypes = [A.dtype, B.dtype]
        ctx.rank, ctx.rank_p = r, rp
        ctx.orig_shape = shape
        return out.view(*shape[:-1], out.shape[-1])

    @staticmethod
    def backward(ctx, dY):
        if ctx.fp32:
            X2, xa, *params = ctx.saved_tensors
            W, A, B = (_f32(t) for t in params)
            dy = _rows_f32(dY)
            P, dA, dB = _adapter_grads_f32(dy, X2, xa, B, ctx.scale)
            dX = cops.gemm_f32([dy, P], [W, A], False, False, 1.0)
            return dX.to(ctx.x_dtype).view(*ctx.orig_shape), None, dA, dB, None
        Xf, xa, a, Wc, Bp = ctx.saved_tensors
        r, rp = ctx.rank, ctx.rank_p
        dy = hip_ops._bf16_rows(dY.reshape(-1, dY.shape[-1]))
        dX, flat = cops.lora_linear_bwd(Xf, dy, Wc, a, Bp, ctx.scale, xa, rp)
        shapes = hip_ops.lora_linear_grad_shapes(Xf.shape[1], dy.shape[1], rp)
        dA, dB = _adapter_grads(flat, shapes, ctx.param_dtypes)
        return dX.view(*ctx.orig_shape), None, dA[:r], dB[:, :r], None


def apply_fused_lora_linear(linear, X: torch.Tensor) -> torch.Tensor:
    """One LoRA projection (e.g. o_proj) through _LoRA_W; the module's own
    forward when it has no LoRA adapter."""
    W, A, B, S = _get_lora_params(linear)
    if A is None:
        return linear(X)
    return _LoRA_W.apply(X, W, A, B, S)


def apply_fused_lora_qkv(attn_module, X: torch.Tensor):
    """Fused Q+K+V LoRA projections of an attention module
    (ops/fused_lora.py:269-295); plain module calls when any projection has
    no LoRA adapter."""
    QW, QA, QB, QS = _get_lora_params(attn_module.q_proj)
    KW, KA, KB, KS = _get_lora_params(attn_module.k_proj)
    VW, VA, VB, VS = _get_lora_params(attn_module.v_proj)

    if QA is None or KA is None or VA is None:
        Q = attn_module.q_proj(X)
        K = attn_module.k_proj(X)
        V = attn_module.v_proj(X)
        return Q, K, V

    return _LoRA_QKV.apply(
        X,
        QW, QA, QB, QS,
        KW, KA, KB, KS,
        VW, VA, VB, VS,
    )


def apply_fused_lora_mlp(mlp_module, X: torch.Tensor) -> torch.Tensor:
    """Fused gate+up+down LoRA MLP (ops/fused_lora.py:298-320); the module's
    own forward when any projection has no LoRA adapter."""
    GW, GA, GB, GS = _get_lora_params(mlp_module.gate_proj)
    UW, UA, UB, US = _get_lora_params(mlp_module.up_proj)
    DW, DA, DB, DS = _get_lora_params(mlp_module.down_proj)

    if GA is None or UA is None or DA is None:
        return mlp_module(X)

    return _LoRA_MLP.apply(
        X,
        GW, GA, GB, GS,
        UW, UA, UB, US,
        DW, DA, DB, DS,
    )


_QKV_PROJ = ("q_proj", "k_proj", "v_proj")
_MLP_PROJ = ("gate_proj", "up_proj", "down_proj")


def _all_lora(module: nn.Module, names) -> bool:
    """Every projection in `names` exists on module and carries a LoRA adapter."""
    return all(_get_lora_params(getattr(module, n, None))[1] is not None for n in names)


class _Returns:
    """Stands in for a projection whose output is already computed."""

    __slots__ = ("value",)

    def __init__(self, value):
        self.value = value

    def __call__(self, *_args, **_kwargs):
        return self.value


class _FusedAttentionForward:
    """Forward of an attention module whose q/k/v projections all carry
    LoRA: q, k and v come from one _LoRA_QKV call on the hidden states, and
    the module's own forward then runs with q/k/v_proj shadowed by those
    results (o_proj by _LoRA_W when it carries LoRA too, which the
    reference's patcher leaves to PEFT)."""

    def __init__(self, attn: nn.Module, original):
        self.attn = attn
        self.original = original
        o_proj = getattr(attn, "o_proj", None)
        self.o_proj = o_proj if _all_lora(attn, ("o_proj",)) else None

    def __call__(self, hidden_states, *args, **kwargs):
        q, k, v = apply_fused_lora_qkv(self.attn, hidden_states)
        subs = dict(zip(_QKV_PROJ, (_Returns(q), _Returns(k), _Returns(v))))
        if self.o_proj is not None:
            o_proj = self.o_proj
            subs["o_proj"] = lambda x: apply_fused_lora_linear(o_proj, x)
        with shadowed(self.attn, **subs):
            return self.original(hidden_states, *args, **kwargs)


class _FusedMLPForward:
    """Forward of an MLP whose gate/up/down projections all carry LoRA: the
    whole block is one _LoRA_MLP call."""

    def __init__(self, mlp: nn.Module):
        self.mlp = mlp

    def __call__(self, x):
        return apply_fused_lora_mlp(self.mlp, x)


def patch_fused_lora(model: nn.Module) -> int:
    """Routes every decoder layer's attention and MLP whose three
    projections all carry LoRA through _LoRA_QKV / _LoRA_MLP and returns how
    many modules were routed (ops/fused_lora.py:323-421).

    Only the instances' ``forward`` attributes change (no module is replaced
    and q/k/v_proj are shadowed only while an attention forward runs), so
    state_dict keys and checkpoints are unaffected. The decoder layers are
    found as the model patcher finds them (PEFT's base_model.model, a bare
    HF model or decoder, Qwen3-VL's language_model); modules already routed
    are left as they are, so a second call returns 0."""
    layers = find_layers(model)
    if layers is None:
        logger.warning("MetalLiger fused LoRA: could not find transformer layers")
        return 0
    routed = 0
    for layer in layers:
        for attr, names, make in (("self_attn", _QKV_PROJ, lambda m: _FusedAttentionForward(m, m.forward)),
                                  ("mlp", _MLP_PROJ, _FusedMLPForward)):
            mod = getattr(layer, attr, None)
            if mod is None or getattr(mod, "_metal_liger_fused_lora", False):
                continue
            if not _all_lora(mod, names):
                continue
            mod.forward = make(mod)
            mod._metal_liger_fused_lora = True
            routed += 1
    logger.info(f"MetalLiger fused LoRA: activated on {routed} modules.")
    return routed
