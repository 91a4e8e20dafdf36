"""Tensor-level wrappers over the C ABI: validate, normalise layout, allocate
outputs with torch's caching allocator, enqueue on the current stream.

These are the only callers of the HIP library; the autograd functions in
``metal_liger_amd.ops`` and the ``metal_liger_ext`` surface are built on them.
"""

from __future__ import annotations

import torch

from . import _hip
from ._hip import call, dtype_tag, ensure_rocm_device, geom, ptr, row_stride, rows_view, stream_of

# ----------------------------------------------------------------- RMSNorm --


def _norm_weight(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """Weight as the kernel reads it: x's dtype or fp32 (exact upcast otherwise)."""
    if weight.dim() != 1 or weight.shape[0] != x.shape[-1]:
        raise ValueError(
            f"rms_norm: weight shape {tuple(weight.shape)} does not match hidden size {x.shape[-1]}"
        )
    w = weight if weight.dtype in (x.dtype, torch.float32) else weight.float()
    return w.contiguous()


def rms_norm_fwd(x: torch.Tensor, weight: torch.Tensor, eps: float):
    """Returns (y, rrms) with y like x (contiguous) and rrms fp32 of shape x.shape[:-1]."""
    ensure_rocm_device(x, weight)
    if x.dim() < 1:
        raise ValueError("rms_norm: input must have at least one dimension")
    cols = x.shape[-1]
    x2 = rows_view(x)
    w = _norm_weight(x, weight)
    y = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    rrms = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device)
    rows = x2.shape[0]
    if rows > 0:
        call(
            "ml_rmsnorm_fwd", ptr(x2), row_stride(x2), ptr(w), ptr(y), cols, ptr(rrms), rows, cols,
            float(eps), dtype_tag(x, "x"), dtype_tag(w, "weight"), stream_of(x),
        )
    return y, rrms


def rms_norm_bwd(x: torch.Tensor, weight: torch.Tensor, dy: torch.Tensor,
                 rrms: torch.Tensor | None, eps: float):
    """Returns (dx, dweight); rrms may be None (recomputed from x and eps)."""
    ensure_rocm_device(x, weight, dy, rrms)
    if dy.shape != x.shape:
        raise ValueError(f"rms_norm backward: grad shape {tuple(dy.shape)} != input {tuple(x.shape)}")
    cols = x.shape[-1]
    if dy.dtype != x.dtype:
        dy = dy.to(x.dtype)
    x2 = rows_view(x)
    g2 = rows_view(dy)
    w = _norm_weight(x, weight)
    rows = x2.shape[0]
    dx = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    dw = torch.empty(cols, dtype=w.dtype, device=x.device)
    r = None
    if rrms is not None:
        r = rrms.reshape(-1)
        if r.dtype != torch.float32:
            r = r.float()
        r = r.contiguous()
    ws_bytes = _hip.query("ml_rmsnorm_bwd_workspace_bytes", rows, cols)
    ws = torch.empty(max(1, (ws_bytes + 3) // 4), dtype=torch.float32, device=x.device)
    call(
        "ml_rmsnorm_bwd", ptr(x2), row_stride(x2), ptr(w), ptr(g2), row_stride(g2), ptr(r),
        float(eps), ptr(dx), cols, ptr(dw), ptr(ws), ws.numel() * 4, rows, cols,
        dtype_tag(x, "x"), dtype_tag(w, "weight"), stream_of(x),
    )
    if dw.dtype != weight.dtype:
        dw = dw.to(weight.dtype)
    return dx, dw


# ------------------------------------------------------------------ SwiGLU --


def _swiglu_operands(gate: torch.Tensor, up: torch.Tensor, *more: torch.Tensor):
    if gate.shape != up.shape:
        raise ValueError(
            f"swiglu: gate {tuple(gate.shape)} and up {tuple(up.shape)} must have the same shape"
        )
    ct = gate.dtype if all(t.dtype == gate.dtype for t in (up, *more)) else torch.float32
    return ct, [t.to(ct).contiguous() for t in (gate, up, *more)]


def swiglu_fwd(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up in fp32, rounded to gate's dtype (ops/fused_swiglu.py:26-35)."""
    ensure_rocm_device(gate, up)
    ct, (g, u) = _swiglu_operands(gate, up)
    out = torch.empty(g.shape, dtype=ct, device=g.device)
    call("ml_swiglu_fwd", ptr(g), ptr(u), ptr(out), g.numel(), dtype_tag(g, "gate"), stream_of(g))
    return out if out.dtype == gate.dtype else out.to(gate.dtype)


def swiglu_bwd(gate: torch.Tensor, up: torch.Tensor, dy: torch.Tensor):
    """(dgate, dup) in gate's / up's dtype (ops/fused_swiglu.py:37-50)."""
    ensure_rocm_device(gate, up, dy)
    if dy.shape != gate.shape:
        raise ValueError("swiglu backward: grad shape does not match gate")
    ct, (g, u, y) = _swiglu_operands(gate, up, dy)
    dg = torch.empty(g.shape, dtype=ct, device=g.device)
    du = torch.empty(g.shape, dtype=ct, device=g.device)
    call(
        "ml_swiglu_bwd", ptr(g), ptr(u), ptr(y), ptr(dg), ptr(du), g.numel(), dtype_tag(g, "gate"),
        stream_of(g),
    )
    if dg.dtype != gate.dtype:
        dg = dg.to(gate.dtype)
    if du.dtype != up.dtype:
        du = du.to(up.dtype)
    return dg, du


# -------------------------------------------------------------------- RoPE --


def _as4d(x: torch.Tensor) -> torch.Tensor:
    if x.dim() < 1:
        raise ValueError("rope: input must have a head dimension")
    if x.dim() <= 4:
        return x.reshape((1,) * (4 - x.dim()) + tuple(x.shape))
    return x.reshape(-1, *x.shape[-3:])


def _unit_last(t: torch.Tensor) -> torch.Tensor:
    return t if t.shape[-1] <= 1 or t.stride(-1) == 1 else t.contiguous()


def _tensor_geom(x4: torch.Tensor, o4: torch.Tensor):
    return geom([x4.shape[0], x4.shape[1], x4.shape[2], x4.stride(0), x4.stride(1), x4.stride(2),
                 o4.stride(0), o4.stride(1), o4.stride(2)])


def _table4(t: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """cos/sin broadcast to x's shape, as a 4-D view (stride 0 on broadcast dims)."""
    if torch.broadcast_shapes(x.shape, t.shape) != x.shape:
        raise ValueError(f"rope: table shape {tuple(t.shape)} does not broadcast to {tuple(x.shape)}")
    t4 = _as4d(t.expand(x.shape))
    if t4.stride(-1) != 1:
        t4 = t4.contiguous()
    return t4


def rope_table(q: torch.Tensor, k: torch.Tensor | None, cos: torch.Tensor, sin: torch.Tensor,
               sgn: float):
    """x*cos + rotate_half(x)*(sgn*sin) for q (and k); returns (q_out, k_out).

    Output dtype is torch's promotion of (x, cos, sin), as the reference's
    eager expression produces (ops/fused_rope.py:67-75).
    """
    ensure_rocm_device(q, k, cos, sin)
    if cos.dtype != sin.dtype:
        cos, sin = cos.float(), sin.float()
    outs = []
    xs = [q] if k is None else [q, k]
    x_dtype = q.dtype
    if k is not None and k.dtype != q.dtype:
        # different input dtypes: rotate each on its own
        return (rope_table(q, None, cos, sin, sgn)[0], rope_table(k, None, cos, sin, sgn)[0])
    out_dtype = torch.promote_types(x_dtype, cos.dtype)
    D = q.shape[-1]
    if D % 2 != 0:
        raise ValueError(f"rope: head dim must be even (got {D})")
    x4s, o4s, outs = [], [], []
    for x in xs:
        if x.shape[-1] != D:
            raise ValueError("rope: q and k must share the head dimension")
        x4 = _unit_last(_as4d(x))
        o4 = torch.empty_like(x4, dtype=out_dtype)
        if o4.stride(-1) != 1:
            o4 = torch.empty(x4.shape, dtype=out_dtype, device=x4.device)
        x4s.append(x4)
        o4s.append(o4)
        outs.append(o4.view(x.shape) if o4.is_contiguous() else o4.reshape(x.shape))
    c4 = _table4(cos, xs[0])
    s4 = _table4(sin, xs[0])
    joint = k is not None and x4s[0].shape[0] == x4s[1].shape[0] and x4s[0].shape[2] == x4s[1].shape[2]
    if joint:
        c4k, s4k = _table4(cos, xs[1]), _table4(sin, xs[1])
        joint = c4k.stride()[:3] == c4.stride()[:3] and s4k.stride()[:3] == s4.stride()[:3] and \
            c4k.data_ptr() == c4.data_ptr() and s4k.data_ptr() == s4.data_ptr()
    if k is not None and not joint:
        return (rope_table(q, None, cos, sin, sgn)[0], rope_table(k, None, cos, sin, sgn)[0])
    cs = geom([c4.stride(0), c4.stride(1), c4.stride(2), s4.stride(0), s4.stride(1), s4.stride(2)])
    gq = _tensor_geom(x4s[0], o4s[0])
    gk = _tensor_geom(x4s[1], o4s[1]) if k is not None else None
    call(
        "ml_rope_table", ptr(x4s[0]), ptr(o4s[0]), gq,
        ptr(x4s[1]) if k is not None else None, ptr(o4s[1]) if k is not None else None, gk,
        D, ptr(c4), ptr(s4), cs, float(sgn), dtype_tag(q, "x"), dtype_tag(c4, "cos"),
        dtype_tag(o4s[0], "out"), stream_of(q),
    )
    # keep the expanded tables alive until the launch is enqueued (it is, by now)
    return outs[0], (outs[1] if k is not None else None)


_INV_FREQ_CACHE: dict = {}


def rope_inv_freq(head_dim: int, theta: float, device: torch.device) -> torch.Tensor:
    """1 / theta^(2i/D) in fp32, computed as the HF rotary module does."""
    key = (int(head_dim), float(theta), str(device))
    t = _INV_FREQ_CACHE.get(key)
    if t is None:
        inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
        t = inv.to(torch.float32).to(device)
        _INV_FREQ_CACHE[key] = t
    return t


def _positions2d(positions: torch.Tensor, B: int, S: int, device) -> torch.Tensor:
    p = positions
    if p.device != device:
        p = p.to(device)
    if p.dtype != torch.int64:
        p = p.to(torch.int64)
    if p.dim() == 1:
        p = p.unsqueeze(0)
    if p.dim() != 2 or p.shape[-1] != S or p.shape[0] not in (1, B):
        raise ValueError(f"rope: positions shape {tuple(positions.shape)} does not match [B={B}, S={S}]")
    return p


def rope_pos(q: torch.Tensor, k: torch.Tensor | None, positions: torch.Tensor,
             inv_freq: torch.Tensor, sgn: float):
    """Rotation with cos/sin computed in-kernel from positions (4-D [B, H, S, D] inputs)."""
    ensure_rocm_device(q, k)
    xs = [q] if k is None else [q, k]
    for x in xs:
        if x.dim() != 4:
            raise ValueError("rope (positions): q/k must be [batch, heads, seq, head_dim]")
    if k is not None and (k.dtype != q.dtype or k.shape[0] != q.shape[0] or k.shape[2] != q.shape[2]
                          or k.shape[3] != q.shape[3]):
        return (rope_pos(q, None, positions, inv_freq, sgn)[0],
                rope_pos(k, None, positions, inv_freq, sgn)[0])
    B, _, S, D = q.shape
    if D % 2 != 0:
        raise ValueError(f"rope: head dim must be even (got {D})")
    inv = inv_freq.to(device=q.device, dtype=torch.float32).contiguous()
    if inv.numel() != D // 2:
        raise ValueError(f"rope: inv_freq has {inv.numel()} entries, expected {D // 2}")
    p = _positions2d(positions, B, S, q.device)
    x4s, o4s = [], []
    for x in xs:
        x4 = _unit_last(x)
        o4 = torch.empty_like(x4)
        if o4.stride(-1) != 1:
            o4 = torch.empty(x4.shape, dtype=x4.dtype, device=x4.device)
        x4s.append(x4)
        o4s.append(o4)
    gq = _tensor_geom(x4s[0], o4s[0])
    gk = _tensor_geom(x4s[1], o4s[1]) if k is not None else None
    call(
        "ml_rope_pos", ptr(x4s[0]), ptr(o4s[0]), gq,
        ptr(x4s[1]) if k is not None else None, ptr(o4s[1]) if k is not None else None, gk,
        D, ptr(p), p.stride(0) if p.shape[0] > 1 else 0, p.stride(1), ptr(inv), float(sgn),
        dtype_tag(q, "q"), stream_of(q),
    )
    return o4s[0], (o4s[1] if k is not None else None)
