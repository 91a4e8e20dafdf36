"""CPU oracle for the fused-op hot path — TEST INFRASTRUCTURE ONLY.

A restatement, in plain torch on the CPU, of the reference's pure-torch fused
ops (krrish-v/metal_liger, ops/*.py). Each function follows the cited lines
op for op, including where the reference casts between dtypes, so that it
reproduces the reference's rounding sequence on the same inputs. The HIP
path is tested against it: only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg use it, and never as a product code path.

Pinning (what checks this oracle independently of its own formulas) lives in
tests/test_oracle.py: fp64 autograd of the plain forward expressions (so a
dropped term or wrong sign in a hand-written VJP fails), F.cross_entropy as a
brute-force CE, closed forms and invariants (norm preservation and inverse of
the rotation, sum-to-zero of softmax gradients, LoRA special cases), and the
reference's own test formulas and tolerances (tests/test_fused_ops.py).
Every function below has at least one such check; none is "parity unpinned".
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

# ------------------------------------------------------------------ RMSNorm --


def rms_norm_forward(x: torch.Tensor, weight: torch.Tensor, eps: float):
    """ops/fused_rms_norm.py:31-41. Returns (y, rrms[..., 1] fp32)."""
    xf = x.float()
    var = xf.pow(2).mean(dim=-1, keepdim=True)
    rrms = torch.rsqrt(var + eps)
    y = ((xf * rrms) * weight.float()).to(x.dtype)
    return y, rrms


def rms_norm_backward(x: torch.Tensor, weight: torch.Tensor, rrms: torch.Tensor,
                      grad_out: torch.Tensor):
    """ops/fused_rms_norm.py:43-60. Returns (dx in x dtype, dw in weight dtype)."""
    g = grad_out.float()
    xf = x.float()
    wf = weight.float()
    gw = g * wf
    m = (gw * xf).mean(dim=-1, keepdim=True)
    dx = (gw * rrms - xf * m * rrms.pow(3)).to(x.dtype)
    dw = (g * (xf * rrms)).sum(dim=list(range(grad_out.ndim - 1))).to(weight.dtype)
    return dx, dw


# ---------------------------------------------------- residual add + RMSNorm --
# Not a reference op: torch's add in a Qwen3 decoder layer (transformers'
# modeling_qwen3.py, Qwen3DecoderLayer.forward: `residual + hidden_states`,
# then post_attention_layernorm) followed by the reference's fused norm.


def add_rms_norm_forward(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                         eps: float):
    """(y, sum, rrms): sum = x + residual in x's dtype (torch's add rounds
    the exact sum once), then rms_norm_forward of that sum."""
    total = x + residual
    y, rrms = rms_norm_forward(total, weight, eps)
    return y, total, rrms


def add_rms_norm_backward(total: torch.Tensor, weight: torch.Tensor, rrms: torch.Tensor,
                          grad_out: torch.Tensor, grad_sum: torch.Tensor):
    """Gradient of x (equal to that of residual): the norm's dx at the sum in
    fp32 plus grad_sum, rounded once to the sum's dtype; dw as
    rms_norm_backward."""
    dxf, dw = rms_norm_backward(total.float(), weight.float(), rrms, grad_out.float())
    dx = (dxf + grad_sum.float()).to(total.dtype)
    return dx, dw.to(weight.dtype)


# ------------------------------------------------------------------- SwiGLU --


def swiglu_forward(gate: torch.Tensor, up: torch.Tensor):
    """ops/fused_swiglu.py:26-35. Returns (out in gate dtype, sigmoid fp32)."""
    gf = gate.float()
    sig = torch.sigmoid(gf)
    out = ((gf * sig) * up.float()).to(gate.dtype)
    return out, sig


def swiglu_backward(gate: torch.Tensor, up: torch.Tensor, sig: torch.Tensor,
                    grad_out: torch.Tensor):
    """ops/fused_swiglu.py:37-50. Returns (dgate, dup)."""
    gf = gate.float()
    uf = up.float()
    g = grad_out.float()
    silu = gf * sig
    dup = (g * silu).to(up.dtype)
    dgate = (g * uf * sig * (1.0 + gf * (1.0 - sig))).to(gate.dtype)
    return dgate, dup


# --------------------------------------------------------------------- RoPE --


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """ops/fused_rope.py:60-64: [x1, x2] -> [-x2, x1] over the last dim."""
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def rope_forward(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """ops/fused_rope.py:67-75 (the forward of _FusedRoPEFunction, :30-41)."""
    return x * cos + rotate_half(x) * sin


def rope_backward(grad_out: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                  x_dtype: torch.dtype) -> torch.Tensor:
    """ops/fused_rope.py:43-57: the same rotation with -sin; autograd then
    casts the gradient to the input's dtype."""
    return rope_forward(grad_out, cos, -sin).to(x_dtype)


def rope_inv_freq(head_dim: int, theta: float) -> torch.Tensor:
    """Default-rope inverse frequencies as the HF rotary module builds them
    (HF modeling_qwen3 compute_default_rope_parameters): fp32."""
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))


def rope_tables(positions: torch.Tensor, head_dim: int, theta: float):
    """cos/sin [B, S, D] (or [S, D] for 1-D positions) with duplicated halves,
    angle = fp32(position) * inv_freq in fp32 (HF rotary forward; also the
    reference test helper tests/test_fused_ops.py:146-154 for theta=1e4)."""
    inv = rope_inv_freq(head_dim, theta)
    p = positions.float()
    ang = p.unsqueeze(-1) * inv
    emb = torch.cat((ang, ang), dim=-1)
    return emb.cos(), emb.sin()


# ------------------------------------------------ q/k head-dim norm + RoPE --
# Not among the reference's ops: its patcher leaves Qwen3's q_norm / k_norm to
# transformers (patch.py:104-131 replaces only the layer norms). Restated from
# transformers' models/qwen3/modeling_qwen3.py as installed here
# (Qwen3RMSNorm.forward; apply_rotary_pos_emb with rotate_half), the
# library the reference's model boundary depends on.


def qk_norm_rope_forward(x: torch.Tensor, weight: torch.Tensor, eps: float,
                         cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """rope(norm(x)) with HF's rounding sequence: the norm in fp32, cast to
    x's dtype, times the weight; then x * cos + rotate_half(x) * sin with the
    tables broadcast against x."""
    xf = x.to(torch.float32)
    var = xf.pow(2).mean(-1, keepdim=True)
    n = weight * (xf * torch.rsqrt(var + eps)).to(x.dtype)
    return n * cos + rotate_half(n) * sin


def qk_norm_rope_backward(x: torch.Tensor, weight: torch.Tensor, eps: float,
                          cos: torch.Tensor, sin: torch.Tensor, grad_out: torch.Tensor):
    """Exact VJP of qk_norm_rope_forward in fp32 (no intermediate roundings):
    (dx [..., D], dweight [D]), both fp32. The rotation's transpose maps
    g * sin = [a, b] to [b, -a]; the norm's is RMSNorm's."""
    xf, w = x.float(), weight.float()
    g = grad_out.float()
    c, s = cos.float(), sin.float()
    h = x.shape[-1] // 2
    r = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    nh = xf * r
    gs = g * s
    dn = g * c + torch.cat((gs[..., h:], -gs[..., :h]), dim=-1)
    gw = dn * w
    dx = r * (gw - nh * (gw * nh).mean(-1, keepdim=True))
    dw = (dn * nh).reshape(-1, x.shape[-1]).sum(0)
    return dx, dw


# ----------------------------------------------- fused linear cross-entropy --


def flce_forward(hidden: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor,
                 bias: torch.Tensor | None = None, ignore_index: int = -100,
                 chunk_size: int = 8192):
    """ops/fused_linear_cross_entropy.py:39-55 and :93-157 (eager path).

    Returns (loss fp32 scalar, lse fp32 [N], mask bool [N]).
    """
    V = weight.shape[0]
    N = hidden.shape[0]
    hf = hidden.float()
    wf = weight.float()
    run_max = torch.full((N,), float("-inf"), dtype=torch.float32, device=hidden.device)
    run_sum = torch.zeros(N, dtype=torch.float32, device=hidden.device)
    for lo in range(0, V, chunk_size):
        hi = min(lo + chunk_size, V)
        bc = bias[lo:hi].float() if bias is not None else None
        z = F.linear(hf, wf[lo:hi], bc)
        new_max = torch.maximum(run_max, z.max(dim=-1).values)
        run_sum = run_sum * torch.exp(run_max - new_max) + torch.exp(z - new_max.unsqueeze(-1)).sum(-1)
        run_max = new_max
    lse = run_max + run_sum.log()
    mask = labels != ignore_index
    safe = torch.where(mask, labels, 0)
    zy = (hf * wf[safe]).sum(dim=-1)
    if bias is not None:
        zy = zy + bias[safe].float()
    per_tok = (lse - zy) * mask.float()
    loss = per_tok.sum() / torch.clamp(mask.float().sum(), min=1.0)
    return loss.squeeze(), lse, mask


def flce_backward(hidden: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor,
                  lse: torch.Tensor, mask: torch.Tensor, grad_out: torch.Tensor,
                  bias: torch.Tensor | None = None, chunk_size: int = 8192):
    """ops/fused_linear_cross_entropy.py:57-80 and :159-185.

    Returns (dhidden in hidden dtype, dweight in weight dtype). No bias grad,
    as in the reference.
    """
    V = weight.shape[0]
    hf = hidden.float()
    wf = weight.float()
    n_valid = torch.clamp(mask.sum().float(), min=1.0)
    dh = torch.zeros_like(hf)
    dw = torch.zeros_like(wf)
    scale = grad_out.float().to(hidden.device) / n_valid
    m2 = mask.float().unsqueeze(-1)
    for lo in range(0, V, chunk_size):
        hi = min(lo + chunk_size, V)
        wc = wf[lo:hi]
        bc = bias[lo:hi].float() if bias is not None else None
        p = (F.linear(hf, wc, bc) - lse.unsqueeze(-1)).exp()
        cls = torch.arange(lo, hi, dtype=labels.dtype, device=labels.device).unsqueeze(0)
        p = torch.where(labels.unsqueeze(1) == cls, p - 1.0, p)
        p = p * m2 * scale
        dh.addmm_(p, wc)
        dw[lo:hi] += p.t() @ hf
    return dh.to(hidden.dtype), dw.to(weight.dtype)


# --------------------------------------------------------------------- LoRA --


def lora_linear(X: torch.Tensor, W: torch.Tensor, A: torch.Tensor | None,
                B: torch.Tensor | None, s: float) -> torch.Tensor:
    """ops/fused_lora.py:69-82: X W^T + ((X A^T) B^T) * s, A/B cast to X's dtype."""
    dt = X.dtype
    out = F.linear(X, W)
    if A is not None and B is not None:
        out = out + F.linear(F.linear(X, A.to(dt)), B.to(dt)) * s
    return out


def lora_qkv_forward(X, QW, QA, QB, QS, KW, KA, KB, KS, VW, VA, VB, VS):
    """ops/fused_lora.py:97-119. Returns (Q, K, V) shaped like X[..., out]."""
    shp = X.shape
    Xf = X.reshape(-1, shp[-1])
    outs = [lora_linear(Xf, W, A, B, s) for (W, A, B, s) in
            ((QW, QA, QB, QS), (KW, KA, KB, KS), (VW, VA, VB, VS))]
    return tuple(o.view(*shp[:-1], -1) for o in outs)


def _lora_grads(dY, Xin, A_c, B_c, s):
    """dA, dB of one adapter: ops/fused_lora.py:142-149 (and :228-252)."""
    dA = (torch.mm(torch.mm(dY, B_c).t(), Xin) * s).float()
    dB = (torch.mm(dY.t(), F.linear(Xin, A_c)) * s).float()
    return dA, dB


def lora_qkv_backward(X, dQ, dK, dV, QW, QA, QB, QS, KW, KA, KB, KS, VW, VA, VB, VS):
    """ops/fused_lora.py:121-171. Returns (dX, dQA, dQB, dKA, dKB, dVA, dVB)."""
    shp = X.shape
    Xf = X.reshape(-1, shp[-1])
    dQ = dQ.reshape(-1, dQ.shape[-1])
    dK = dK.reshape(-1, dK.shape[-1])
    dV = dV.reshape(-1, dV.shape[-1])
    dt = dQ.dtype
    cast = lambda t: t.to(dt)  # noqa: E731
    dQA, dQB = _lora_grads(dQ, Xf, cast(QA), cast(QB), QS)
    dKA, dKB = _lora_grads(dK, Xf, cast(KA), cast(KB), KS)
    dVA, dVB = _lora_grads(dV, Xf, cast(VA), cast(VB), VS)
    q = torch.mm(dQ, QW) + torch.mm(torch.mm(dQ, cast(QB)), cast(QA)) * QS
    k = torch.mm(dK, KW) + torch.mm(torch.mm(dK, cast(KB)), cast(KA)) * KS
    v = torch.mm(dV, VW) + torch.mm(torch.mm(dV, cast(VB)), cast(VA)) * VS
    dX = (q + k + v).view(*shp)
    return dX, dQA, dQB, dKA, dKB, dVA, dVB


def lora_linear_backward(X, dY, W, A, B, s):
    """One LoRA projection (the "LoRA_W" block of ops/fused_lora.py:26, which
    the reference does not implement): the per-adapter terms of
    _LoRA_QKV.backward (ops/fused_lora.py:121-171) for a single adapter.
    Returns (dX, dA, dB)."""
    shp = X.shape
    Xf = X.reshape(-1, shp[-1])
    dY = dY.reshape(-1, dY.shape[-1])
    dt = dY.dtype
    A_c, B_c = A.to(dt), B.to(dt)
    dA, dB = _lora_grads(dY, Xf, A_c, B_c, s)
    dX = torch.mm(dY, W) + torch.mm(torch.mm(dY, B_c), A_c) * s
    return dX.view(*shp), dA, dB


def lora_mlp_forward(X, GW, GA, GB, GS, UW, UA, UB, US, DW, DA, DB, DS):
    """ops/fused_lora.py:183-207. Returns (out, gate, up, h)."""
    shp = X.shape
    Xf = X.reshape(-1, shp[-1])
    gate = lora_linear(Xf, GW, GA, GB, GS)
    up = lora_linear(Xf, UW, UA, UB, US)
    gf = gate.float()
    h = (gf * torch.sigmoid(gf) * up.float()).to(X.dtype)
    out = lora_linear(h, DW, DA, DB, DS)
    return out.view(*shp), gate, up, h


def lora_mlp_backward(X, gate, up, h, dY, GW, GA, GB, GS, UW, UA, UB, US, DW, DA, DB, DS):
    """ops/fused_lora.py:209-266.

    Returns (dX, dGA, dGB, dUA, dUB, dDA, dDB).
    """
    shp = X.shape
    Xf = X.reshape(-1, shp[-1])
    dY = dY.reshape(-1, dY.shape[-1])
    dt = dY.dtype
    cast = lambda t: t.to(dt)  # noqa: E731
    dDA, dDB = _lora_grads(dY, h, cast(DA), cast(DB), DS)
    dH = torch.mm(dY, DW) + torch.mm(torch.mm(dY, cast(DB)), cast(DA)) * DS
    gf = gate.float()
    uf = up.float()
    sg = torch.sigmoid(gf)
    dHf = dH.float()
    d_gate = (dHf * uf * sg * (1.0 + gf * (1.0 - sg))).to(dt)
    d_up = (dHf * (gf * sg)).to(dt)
    dGA, dGB = _lora_grads(d_gate, Xf, cast(GA), cast(GB), GS)
    dUA, dUB = _lora_grads(d_up, Xf, cast(UA), cast(UB), US)
    g_part = torch.mm(d_gate, GW) + torch.mm(torch.mm(d_gate, cast(GB)), cast(GA)) * GS
    u_part = torch.mm(d_up, UW) + torch.mm(torch.mm(d_up, cast(UB)), cast(UA)) * US
    dX = (g_part + u_part).view(*shp)
    return dX, dGA, dGB, dUA, dUB, dDA, dDB
