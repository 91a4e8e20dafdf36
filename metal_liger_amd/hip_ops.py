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


def rms_norm_add_fwd(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float):
    """Residual add fused with the norm after it: returns (y, sum, rrms) with
    sum = x + residual (x's dtype, contiguous) and y, rrms the norm of sum."""
    ensure_rocm_device(x, residual, weight)
    if x.dim() < 1:
        raise ValueError("rms_norm add: input must have at least one dimension")
    if residual.shape != x.shape or residual.dtype != x.dtype:
        raise ValueError(f"rms_norm add: residual {tuple(residual.shape)} {residual.dtype} does not "
                         f"match x {tuple(x.shape)} {x.dtype}")
    cols = x.shape[-1]
    x2 = rows_view(x)
    r2 = rows_view(residual)
    w = _norm_weight(x, weight)
    y = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    total = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    rrms = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device)
    rows = x2.shape[0]
    if rows > 0:
        call(
            "ml_rmsnorm_add_fwd", ptr(x2), row_stride(x2), ptr(r2), row_stride(r2), ptr(w),
            ptr(total), cols, ptr(y), cols, ptr(rrms), rows, cols, float(eps), dtype_tag(x, "x"),
            dtype_tag(w, "weight"), stream_of(x),
        )
    return y, total, rrms


def rms_norm_bwd(x: torch.Tensor, weight: torch.Tensor, dy: torch.Tensor,
                 rrms: torch.Tensor | None, eps: float, dsum: torch.Tensor | None = None):
    """Returns (dx, dweight); rrms may be None (recomputed from x and eps).
    dsum (the residual form): a second gradient of x added into dx."""
    ensure_rocm_device(x, weight, dy, rrms, dsum)
    if dy.shape != x.shape:
        raise ValueError(f"rms_norm backward: grad shape {tuple(dy.shape)} != input {tuple(x.shape)}")
    if dsum is not None and dsum.shape != x.shape:
        raise ValueError(f"rms_norm backward: sum grad shape {tuple(dsum.shape)} != input "
                         f"{tuple(x.shape)}")
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
    tail = (float(eps), ptr(dx), cols, ptr(dw), ptr(ws), ws.numel() * 4, rows, cols,
            dtype_tag(x, "x"), dtype_tag(w, "weight"), stream_of(x))
    if dsum is None:
        call("ml_rmsnorm_bwd", ptr(x2), row_stride(x2), ptr(w), ptr(g2), row_stride(g2), ptr(r),
             *tail)
    else:
        d2 = rows_view(dsum if dsum.dtype == x.dtype else dsum.to(x.dtype))
        call("ml_rmsnorm_add_bwd", ptr(x2), row_stride(x2), ptr(w), ptr(g2), row_stride(g2),
             ptr(d2), row_stride(d2), ptr(r), *tail)
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
    return geom([*x4.shape[:3], *x4.stride()[:3], *o4.stride()[:3]])


def rope_out(x: torch.Tensor, out_dtype) -> tuple:
    """(x4, o4, out) for a RoPE input x: x as a 4-D view with a unit last
    stride, its output buffer (x's layout where it has one) and the output
    in x's shape. Shared by the launch and by the fake kernels."""
    x4 = _unit_last(_as4d(x))
    o4 = torch.empty_like(x4, dtype=out_dtype)
    if o4.stride(-1) != 1:
        o4 = torch.empty(x4.shape, dtype=out_dtype, device=x4.device)
    return x4, o4, (o4.view(x.shape) if o4.is_contiguous() else o4.reshape(x.shape))


def rope_out_dtype(x_dtype, cos_dtype, sin_dtype):
    """Output dtype of the table-mode rotation: torch's promotion of x and
    the tables (tables of different dtypes are read as fp32)."""
    return torch.promote_types(x_dtype, cos_dtype if cos_dtype == sin_dtype else torch.float32)


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
        x4, o4, out = rope_out(x, out_dtype)
        x4s.append(x4)
        o4s.append(o4)
        outs.append(out)
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
    inv = inv_freq
    if inv.device != q.device or inv.dtype != torch.float32 or not inv.is_contiguous():
        inv = inv.to(device=q.device, dtype=torch.float32).contiguous()
    if inv.numel() != D // 2:
        raise ValueError(f"rope: inv_freq has {inv.numel()} entries, expected {D // 2}")
    p = _positions2d(positions, B, S, q.device)
    x4s, o4s = [], []
    for x in xs:
        x4, o4, _ = rope_out(x, x.dtype)
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


# --------------------------------------------------- q/k norm + RoPE --

_QKN_HEAD_DIMS = (32, 64, 128, 256)


def _qkn_aligned(t: torch.Tensor, dims: int) -> bool:
    """16-byte aligned base and the first `dims` strides in multiples of 16
    bytes, with a contiguous last dimension."""
    es = t.element_size()
    return t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and \
        all((st * es) % 16 == 0 for st in t.stride()[:dims])


def _qkn_rows(x: torch.Tensor, what: str) -> torch.Tensor:
    """x as [B, H, S, D] with D contiguous, 16-byte aligned rows."""
    if x.dim() != 4:
        raise ValueError(f"qk_norm_rope: {what} must be [batch, heads, seq, head_dim]")
    if not _qkn_aligned(x, 3):
        x = x.clone(memory_format=torch.contiguous_format)
    return x


def _qkn_out(B: int, H: int, S: int, D: int, dtype, device) -> torch.Tensor:
    """[B, H, S, D] view of fresh [B, S, H, D] memory (the layout of HF's
    transposed projections)."""
    return torch.empty(B, S, H, D, dtype=dtype, device=device).transpose(1, 2)


def _qkn_weight(w: torch.Tensor, x_dtype, D: int, what: str) -> torch.Tensor:
    if w.dim() != 1 or w.shape[0] != D:
        raise ValueError(f"qk_norm_rope: {what} weight must be [{D}] (got {tuple(w.shape)})")
    if w.dtype not in (x_dtype, torch.float32):
        w = w.float()
    if not _qkn_aligned(w, 0):
        w = w.clone(memory_format=torch.contiguous_format)
    return w


def _qkn_table_strides(t: torch.Tensor, shape) -> list | None:
    """Strides of t broadcast to the 4-D `shape` (0 on broadcast dims), or
    None when t does not broadcast to it."""
    ts = tuple(t.shape)
    if len(ts) > 4:
        return None
    pad = 4 - len(ts)
    st = t.stride()
    out = []
    for d in range(4):
        if d < pad:
            out.append(0)
            continue
        n = ts[d - pad]
        if n == shape[d]:
            out.append(st[d - pad] if n > 1 else 0)
        elif n == 1:
            out.append(0)
        else:
            return None
    return out


def _qkn_tables(cos: torch.Tensor, sin: torch.Tensor, x: torch.Tensor):
    """cos/sin in x's dtype with their strides broadcast to x's [B, H, S, D]
    shape (0 on broadcast dims): (cos, sin, 6-entry stride list)."""
    shape = tuple(x.shape)
    out, strides = [], []
    for t in (cos, sin):
        if t.dtype != x.dtype:
            t = t.to(x.dtype)
        st = _qkn_table_strides(t, shape)
        if st is None:
            raise ValueError(f"qk_norm_rope: table shape {tuple(t.shape)} does not broadcast to "
                             f"{shape}")
        if st[3] != 1 or t.data_ptr() % 16 or any((v * t.element_size()) % 16 for v in st[:3]):
            t = t.clone(memory_format=torch.contiguous_format)
            st = _qkn_table_strides(t, shape)
        out.append(t)
        strides.append(st)
    cs = geom(strides[0][:3] + strides[1][:3])
    return out[0], out[1], cs


def _qkn_common(q, k, q_weight, k_weight, cos, sin):
    ensure_rocm_device(q, k, q_weight, k_weight, cos, sin)
    if q.dim() != 4 or k.dim() != 4:
        raise ValueError("qk_norm_rope: q and k must be [batch, heads, seq, head_dim]")
    B, _, S, D = q.shape
    if k.shape[0] != B or k.shape[2] != S or k.shape[3] != D:
        raise ValueError("qk_norm_rope: q and k must share batch, sequence and head_dim")
    if k.dtype != q.dtype:
        raise TypeError("qk_norm_rope: q and k must share a dtype")
    if D not in _QKN_HEAD_DIMS:
        raise ValueError(f"qk_norm_rope: head_dim must be one of {_QKN_HEAD_DIMS} (got {D})")
    wq = _qkn_weight(q_weight, q.dtype, D, "q")
    wk = _qkn_weight(k_weight, q.dtype, D, "k")
    if wk.dtype != wq.dtype:
        wq, wk = wq.float(), wk.float()
    c4, s4, cs = _qkn_tables(cos, sin, q)
    if k.shape[1] != q.shape[1] and (cs[1] != 0 or cs[4] != 0):
        # the tables must not vary across heads when q and k head counts differ
        raise ValueError("qk_norm_rope: per-head tables need equal q and k head counts")
    return B, S, D, wq, wk, c4, s4, cs


def qk_norm_rope_fwd(q: torch.Tensor, k: torch.Tensor, q_weight: torch.Tensor,
                     k_weight: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, eps: float):
    """Head-dim RMSNorm with weight (q_norm / k_norm), then rotate-half RoPE.

    q, k: [B, H, S, D] in one dtype (any strides with D contiguous), D in
    {32, 64, 128, 256}; weights [D] (x's dtype or fp32); cos/sin broadcastable to
    q's shape (HF's [B, S, D] tables unsqueezed at dim 1), cast to x's dtype.
    Returns (q_out, k_out) in x's dtype, [B, H, S, D] views of [B, S, H, D]
    memory (with fp32 weights and bf16 / fp16 x, transformers' expression
    would promote to fp32; the fused op keeps x's dtype).
    """
    B, S, D, wq, wk, c4, s4, cs = _qkn_common(q, k, q_weight, k_weight, cos, sin)
    xq, xk = _qkn_rows(q, "q"), _qkn_rows(k, "k")
    oq = _qkn_out(B, q.shape[1], S, D, q.dtype, q.device)
    ok = _qkn_out(B, k.shape[1], S, D, q.dtype, q.device)
    gq = geom([B, xq.shape[1], S, *xq.stride()[:3], *oq.stride()[:3]])
    gk = geom([B, xk.shape[1], S, *xk.stride()[:3], *ok.stride()[:3]])
    call(
        "ml_qk_norm_rope_fwd", ptr(xq), ptr(oq), gq, ptr(wq), ptr(xk), ptr(ok), gk, ptr(wk), D,
        float(eps), ptr(c4), ptr(s4), cs, dtype_tag(q, "q"), dtype_tag(wq, "weight"), stream_of(q),
    )
    return oq, ok


def qk_norm_rope_bwd(q: torch.Tensor, k: torch.Tensor, q_weight: torch.Tensor,
                     k_weight: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, eps: float,
                     dq_out: torch.Tensor, dk_out: torch.Tensor, need_dq_weight: bool = True,
                     need_dk_weight: bool = True):
    """Returns (dq, dk, dq_weight or None, dk_weight or None): dq / dk in x's
    dtype as [B, H, S, D] views of [B, S, H, D] memory, weight gradients in
    the weights' dtype (summed in a fixed order)."""
    B, S, D, wq, wk, c4, s4, cs = _qkn_common(q, k, q_weight, k_weight, cos, sin)
    xq, xk = _qkn_rows(q, "q"), _qkn_rows(k, "k")
    ensure_rocm_device(dq_out, dk_out)
    if dq_out.shape != q.shape or dk_out.shape != k.shape:
        raise ValueError("qk_norm_rope: gradient shapes must match q and k")
    yq = _qkn_rows(dq_out.to(q.dtype), "dq")
    yk = _qkn_rows(dk_out.to(q.dtype), "dk")
    dq = _qkn_out(B, q.shape[1], S, D, q.dtype, q.device)
    dk = _qkn_out(B, k.shape[1], S, D, q.dtype, q.device)
    dwq = torch.empty(D, dtype=wq.dtype, device=q.device) if need_dq_weight else None
    dwk = torch.empty(D, dtype=wk.dtype, device=q.device) if need_dk_weight else None
    ws = None
    if dwq is not None or dwk is not None:
        wsb = _hip.query("ml_qk_norm_rope_bwd_workspace_bytes", B, S, q.shape[1], k.shape[1], D)
        ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=q.device)
    gq = geom([B, xq.shape[1], S, *xq.stride()[:3], *yq.stride()[:3], *dq.stride()[:3]])
    gk = geom([B, xk.shape[1], S, *xk.stride()[:3], *yk.stride()[:3], *dk.stride()[:3]])
    call(
        "ml_qk_norm_rope_bwd", ptr(xq), ptr(yq), ptr(dq), gq, ptr(wq), ptr(dwq), ptr(xk), ptr(yk),
        ptr(dk), gk, ptr(wk), ptr(dwk), D, float(eps), ptr(c4), ptr(s4), cs, dtype_tag(q, "q"),
        dtype_tag(wq, "weight"), ptr(ws), ws.numel() if ws is not None else 0, stream_of(q),
    )
    if dwq is not None and dwq.dtype != q_weight.dtype:
        dwq = dwq.to(q_weight.dtype)
    if dwk is not None and dwk.dtype != k_weight.dtype:
        dwk = dwk.to(k_weight.dtype)
    return dq, dk, dwq, dwk


# -------------------------------------------------------------------- GEMM --


def _gemm_operand(t: torch.Tensor, what: str) -> torch.Tensor:
    if t.dtype != torch.bfloat16:
        raise TypeError(f"gemm: {what} must be bfloat16 (got {t.dtype})")
    if t.dim() != 2:
        raise ValueError(f"gemm: {what} must be 2-D")
    if t.stride(1) != 1 or t.stride(0) % 8 != 0 or t.data_ptr() % 16 != 0:
        t = t.contiguous()
    return t


def matmul(a: torch.Tensor, b: torch.Tensor, *, a_t: bool = False, b_t: bool = False,
           out: torch.Tensor | None = None, out_dtype: torch.dtype = torch.float32,
           alpha: float = 1.0, beta: float = 0.0, tile_cfg: int = 0,
           ksplit: int = 1) -> torch.Tensor:
    """op(a) @ op(b) on the MFMA engine, op(x) = x.T when the flag is set.

    a: [M, K] (or [K, M] with a_t); b: [K, N] (or [N, K] with b_t, an
    nn.Linear weight). bf16 inputs, fp32 accumulation; out fp32 or bf16.
    With out given, computes out = alpha * op(a) op(b) + beta * out.
    """
    ensure_rocm_device(a, b, out)
    a = _gemm_operand(a, "a")
    b = _gemm_operand(b, "b")
    M, K = (a.shape[1], a.shape[0]) if a_t else (a.shape[0], a.shape[1])
    Kb, N = (b.shape[1], b.shape[0]) if b_t else (b.shape[0], b.shape[1])
    if K != Kb:
        raise ValueError(f"gemm: inner dimensions differ ({K} vs {Kb})")
    if out is None:
        if out_dtype == torch.bfloat16 and N % 8 != 0 and tile_cfg == 0 and ksplit == 1:
            # the engines store bf16 rows as 16-byte vectors (row stride a
            # multiple of 8): compute in fp32 and round once
            return matmul(a, b, a_t=a_t, b_t=b_t, out_dtype=torch.float32, alpha=alpha).to(out_dtype)
        out = torch.empty(M, N, dtype=out_dtype, device=a.device)
        beta = 0.0
    elif out.shape != (M, N) or out.stride(1) != 1:
        raise ValueError("gemm: out must be a row-major [M, N] tensor")
    if M == 0 or N == 0:
        return out
    if K == 0:   # an empty sum: alpha * 0 + beta * out
        return out.mul_(beta) if beta != 0.0 else out.zero_()
    if tile_cfg == 0 and ksplit == 1:
        call(
            "ml_gemm_bf16", M, N, K, ptr(a), a.stride(0), 1 if a_t else 0, ptr(b), b.stride(0),
            0 if b_t else 1, ptr(out), out.stride(0), dtype_tag(out, "out"), float(alpha),
            float(beta), stream_of(a),
        )
    else:
        wsb = _hip.query("ml_gemm_splitk_workspace_bytes", M, N, K, ksplit)
        ws = torch.empty(max(wsb // 4, 1), dtype=torch.float32, device=a.device)
        call(
            "ml_gemm_bf16_splitk", M, N, K, ptr(a), a.stride(0), 1 if a_t else 0, ptr(b),
            b.stride(0), 0 if b_t else 1, ptr(out), out.stride(0), dtype_tag(out, "out"),
            float(alpha), float(beta), int(tile_cfg), int(ksplit), ptr(ws), ws.numel() * 4,
            stream_of(a),
        )
    return out


def _f32_2d(t: torch.Tensor) -> torch.Tensor:
    if t.dtype != torch.float32:
        t = t.float()
    if t.dim() != 2 or t.stride(1) != 1 or t.stride(0) < t.shape[1]:
        t = t.contiguous()
    return t


def gemm_f32(a_list, b_list, a_t: bool = False, b_t: bool = False, alpha: float = 1.0):
    """alpha * sum_s op(a_s) @ op(b_s) in fp32 on the matrix cores (op(x) =
    x.T when the flag is set): a_s [M, K_s] (or [K_s, M]), b_s [K_s, N] (or
    [N, K_s]). Returns a new [M, N] fp32 tensor."""
    ensure_rocm_device(*a_list, *b_list)
    if len(a_list) != len(b_list) or not a_list:
        raise ValueError("gemm_f32: one b operand per a operand")
    a_list = [_f32_2d(a) for a in a_list]
    b_list = [_f32_2d(b) for b in b_list]
    M = a_list[0].shape[1] if a_t else a_list[0].shape[0]
    N = b_list[0].shape[0] if b_t else b_list[0].shape[1]
    ks = []
    for a, b in zip(a_list, b_list):
        ma, ka = (a.shape[1], a.shape[0]) if a_t else (a.shape[0], a.shape[1])
        kb, nb = (b.shape[1], b.shape[0]) if b_t else (b.shape[0], b.shape[1])
        if ma != M or nb != N or ka != kb:
            raise ValueError(f"gemm_f32: segment shapes {tuple(a.shape)} x {tuple(b.shape)} do "
                             f"not fit [{M}, K] x [K, {N}]")
        ks.append(int(ka))
    out = torch.empty(M, N, dtype=torch.float32, device=a_list[0].device)
    if M == 0 or N == 0:
        return out
    if sum(ks) == 0:
        return out.zero_()
    call(
        "ml_gemm_f32_segments", M, N, len(ks), geom(ks), _hip.ptrs([a.data_ptr() for a in a_list]),
        geom([a.stride(0) for a in a_list]), _hip.ptrs([b.data_ptr() for b in b_list]),
        geom([b.stride(0) for b in b_list]), 1 if a_t else 0, 0 if b_t else 1, ptr(out),
        out.stride(0), float(alpha), 0.0, stream_of(a_list[0]),
    )
    return out


# -------------------------------------------------------------------- FLCE --


def _flce_operands(hidden, weight, labels, bias):
    ensure_rocm_device(hidden, weight, labels, bias)
    if hidden.dtype != weight.dtype or hidden.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(
            "fused linear cross-entropy: hidden and weight must share a dtype, bfloat16 (bf16 "
            f"MFMA GEMMs) or float32 (fp32 MFMA GEMMs) (got {hidden.dtype}, {weight.dtype})"
        )
    if hidden.dim() != 2 or weight.dim() != 2 or hidden.shape[1] != weight.shape[1]:
        raise ValueError(f"flce: hidden {tuple(hidden.shape)} / weight {tuple(weight.shape)} mismatch")
    if labels.shape != (hidden.shape[0],):
        raise ValueError(f"flce: labels shape {tuple(labels.shape)} != ({hidden.shape[0]},)")

    def rowmajor(t):
        ok = t.stride(1) == 1 and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0
        return t if ok and t.shape[0] > 0 else t.contiguous()

    hidden = rowmajor(hidden)
    weight = rowmajor(weight)
    labels = labels.to(torch.int64).contiguous()
    if bias is not None:
        if bias.shape != (weight.shape[0],):
            raise ValueError("flce: bias must be [vocab]")
        ok = (torch.float32, torch.bfloat16) if hidden.dtype == torch.bfloat16 else (torch.float32,)
        bias = bias if bias.dtype in ok else bias.float()
        bias = bias.contiguous()
    return hidden, weight, labels, bias


def _flce_pad8(hidden, weight, bias):
    """bf16 operands whose vocab or hidden size is not a multiple of 8 (the
    MFMA GEMMs move 8 bf16 per 16-byte access): hidden and weight get zero
    columns up to a multiple of 8 (no logit changes), weight zero rows whose
    bias is -inf (exp(-inf) = 0: no share of the softmax, zero gradient).
    Returns (hidden, weight, bias, V, H) with V, H the original sizes."""
    N, H = hidden.shape
    V = weight.shape[0]
    if V % 8 == 0 and H % 8 == 0:
        return hidden, weight, bias, V, H
    V8, H8 = -(-V // 8) * 8, -(-H // 8) * 8
    if H8 != H:
        hp = hidden.new_zeros(N, H8)
        hp[:, :H] = hidden
        hidden = hp
    wp = weight.new_zeros(V8, H8)
    wp[:V, :H] = weight
    bp = torch.full((V8,), float("-inf"), dtype=bias.dtype if bias is not None else torch.float32,
                    device=weight.device)
    bp[:V] = bias if bias is not None else 0.0
    return hidden, wp, bp, V, H


def _flce_unpad(t, rows, cols):
    """The [rows, cols] block of a gradient computed on padded operands."""
    if t is None or (t.shape[0] == rows and t.shape[1] == cols):
        return t
    return t[:rows, :cols].contiguous()


def _flce_f32(hidden, weight, labels, bias, ignore_index, need_dhidden, need_dweight, chunk):
    """fp32 loss, lse, n_valid and (unit grad_output) gradients by the
    vocabulary-chunked schedule (ml_flce_fwd_grad_f32)."""
    N, H = hidden.shape
    V = weight.shape[0]
    dev = hidden.device
    f32 = torch.float32
    loss = torch.empty((), dtype=f32, device=dev)
    lse = torch.empty(N, dtype=f32, device=dev)
    n_valid = torch.empty(1, dtype=f32, device=dev)
    dh = torch.empty(N, H, dtype=f32, device=dev) if need_dhidden else None
    dw = torch.empty(V, H, dtype=f32, device=dev) if need_dweight else None
    c = max(1, min(int(chunk), V))
    wsb = _hip.query("ml_flce_fwd_grad_f32_workspace_bytes", N, V, c)
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=dev)
    call(
        "ml_flce_fwd_grad_f32", ptr(hidden), hidden.stride(0) if N > 0 else H, ptr(weight),
        weight.stride(0), ptr(bias), ptr(labels), N, V, H, int(ignore_index), c, ptr(loss),
        ptr(lse), ptr(n_valid), ptr(dh), ptr(dw), ptr(ws), ws.numel(), stream_of(weight),
    )
    return loss, lse, n_valid, dh, dw


def flce_fwd(hidden, weight, labels, bias=None, ignore_index: int = -100,
             vocab_chunk: int = 8192):
    """The loss alone. Returns (loss 0-d fp32, lse [N] fp32, n_valid [1]
    fp32). bf16: one logits GEMM over the whole vocabulary whose epilogue
    keeps per-row (max, sum-exp) partials and stores nothing
    (ml_flce_fwd); fp32: the vocabulary-chunked schedule's first pass
    (ml_flce_fwd_grad_f32 with no gradient outputs, vocab_chunk columns per
    chunk)."""
    hidden, weight, labels, bias = _flce_operands(hidden, weight, labels, bias)
    if hidden.dtype == torch.float32:
        loss, lse, n_valid, _, _ = _flce_f32(hidden, weight, labels, bias, ignore_index, False,
                                             False, vocab_chunk)
        return loss, lse, n_valid
    hidden, weight, bias, _, _ = _flce_pad8(hidden, weight, bias)
    N, H = hidden.shape
    V = weight.shape[0]
    dev = hidden.device
    loss = torch.empty((), dtype=torch.float32, device=dev)
    lse = torch.empty(N, dtype=torch.float32, device=dev)
    n_valid = torch.empty(1, dtype=torch.float32, device=dev)
    wsb = _hip.query("ml_flce_fwd_workspace_bytes", N, V)
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=dev)
    call(
        "ml_flce_fwd", ptr(hidden), hidden.stride(0) if N > 0 else H, ptr(weight), weight.stride(0),
        ptr(bias), dtype_tag(bias, "bias") if bias is not None else 0, ptr(labels), N, V, H,
        int(ignore_index), ptr(loss), ptr(lse), ptr(n_valid), ptr(ws), ws.numel(), stream_of(weight),
    )
    return loss, lse, n_valid


# Bytes of the [token_chunk, vocab] bf16 buffer the one-pass schedule holds:
# a quarter of a [8192, 151936] bf16 logits tensor (2048-token chunks). The
# whole forward + backward then holds 1.39 GB of extra memory at that shape
# (the buffer, partials, the dH / dW outputs), a third of what the
# reference's fp32 schedule allocates; two chunks of 4096 tokens ran 2% faster
# (13.50 against 13.76 ms) for 0.67 GB more.
FLCE_CHUNK_BYTES = 640 << 20


def flce_token_chunk(n_tokens: int, vocab: int) -> int:
    """Tokens per chunk of ml_flce_fwd_grad: all of them when the [tokens,
    vocab] bf16 buffer fits FLCE_CHUNK_BYTES, else the tokens split into the
    fewest chunks that fit, of equal size rounded up to a multiple of 256
    (at least 256)."""
    if n_tokens * vocab * 2 <= FLCE_CHUNK_BYTES:
        return max(n_tokens, 1)
    cap = max(256, (FLCE_CHUNK_BYTES // (vocab * 2)) // 256 * 256)
    n_chunks = -(-n_tokens // cap)
    per = -(-n_tokens // n_chunks)
    return min(cap, -(-per // 256) * 256)


def flce_fwd_grad(hidden, weight, labels, bias=None, ignore_index: int = -100,
                  need_dhidden: bool = True, need_dweight: bool = True,
                  token_chunk: int | None = None, vocab_chunk: int = 8192):
    """Loss and gradients for d(loss) = 1.

    bf16: one pass over token chunks (logits computed once); fp32: the
    reference's vocabulary-chunked schedule with vocab_chunk columns per
    chunk. Returns (loss 0-d fp32, lse [N] fp32, n_valid [1] fp32, d_hidden
    or None, d_weight or None), gradients in the input dtype.
    """
    hidden, weight, labels, bias = _flce_operands(hidden, weight, labels, bias)
    if hidden.dtype == torch.float32:
        return _flce_f32(hidden, weight, labels, bias, ignore_index, need_dhidden, need_dweight,
                         vocab_chunk)
    hidden, weight, bias, V0, H0 = _flce_pad8(hidden, weight, bias)
    N, H = hidden.shape
    V = weight.shape[0]
    dev = hidden.device
    loss = torch.empty((), dtype=torch.float32, device=dev)
    lse = torch.empty(N, dtype=torch.float32, device=dev)
    n_valid = torch.empty(1, dtype=torch.float32, device=dev)
    dh = torch.empty(N, H, dtype=torch.bfloat16, device=dev) if need_dhidden else None
    dw = torch.empty(V, H, dtype=torch.bfloat16, device=dev) if need_dweight else None
    T = int(token_chunk) if token_chunk else flce_token_chunk(N, V)
    wsb = _hip.query("ml_flce_fwd_grad_workspace_bytes", N, V, H, T, 1 if need_dhidden else 0)
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=dev)
    call(
        "ml_flce_fwd_grad", ptr(hidden), hidden.stride(0) if N > 0 else H, ptr(weight),
        weight.stride(0), ptr(bias), dtype_tag(bias, "bias") if bias is not None else 0, ptr(labels),
        N, V, H, int(ignore_index), T, ptr(loss), ptr(lse), ptr(n_valid), ptr(dh), ptr(dw), ptr(ws),
        ws.numel(), stream_of(weight),
    )
    return loss, lse, n_valid, _flce_unpad(dh, N, H0), _flce_unpad(dw, V0, H0)


def flce_scale_grads(grad_loss, d_hidden, d_weight):
    """d_hidden *= grad_loss, d_weight *= grad_loss in place (bf16 or fp32,
    as flce_fwd_grad returned them; no-op on the device when grad_loss == 1)."""
    t = d_hidden if d_hidden is not None else d_weight
    if t is None:
        return
    g = grad_loss.detach().to(device=t.device, dtype=torch.float32).reshape(1).contiguous()
    fn = "ml_flce_scale_grads_f32" if t.dtype == torch.float32 else "ml_flce_scale_grads"
    call(
        fn, ptr(g), ptr(d_hidden), d_hidden.numel() if d_hidden is not None else 0,
        ptr(d_weight), d_weight.numel() if d_weight is not None else 0, stream_of(t),
    )


def flce_bwd(hidden, weight, labels, bias, ignore_index, lse, n_valid, grad_loss, chunk_size,
             need_dhidden=True, need_dweight=True):
    """Returns (d_hidden or None, d_weight or None) in the input dtype."""
    hidden, weight, labels, bias = _flce_operands(hidden, weight, labels, bias)
    if hidden.dtype == torch.float32:
        # the fp32 schedule recomputes everything from the inputs
        _, _, _, dh, dw = _flce_f32(hidden, weight, labels, bias, ignore_index, need_dhidden,
                                    need_dweight, chunk_size)
        flce_scale_grads(grad_loss, dh, dw)
        return dh, dw
    hidden, weight, bias, V0, H0 = _flce_pad8(hidden, weight, bias)
    N, H = hidden.shape
    V = weight.shape[0]
    dev = hidden.device
    g = grad_loss.detach().to(device=dev, dtype=torch.float32).reshape(1).contiguous()
    dh = torch.empty(N, H, dtype=torch.bfloat16, device=dev) if need_dhidden else None
    dw = torch.empty(V, H, dtype=torch.bfloat16, device=dev) if need_dweight else None
    if dh is None and dw is None:
        return None, None
    chunk = int(chunk_size)
    chunk = max(8, (min(chunk, V) + 7) // 8 * 8)
    wsb = _hip.query("ml_flce_bwd_workspace_bytes", N, H, chunk, 1 if need_dhidden else 0)
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=dev)
    call(
        "ml_flce_bwd", ptr(hidden), hidden.stride(0) if N > 0 else H, ptr(weight), weight.stride(0),
        ptr(bias), dtype_tag(bias, "bias") if bias is not None else 0, ptr(labels), N, V, H,
        int(ignore_index), ptr(lse), ptr(n_valid), ptr(g), chunk, ptr(dh), ptr(dw), ptr(ws),
        ws.numel(), stream_of(weight),
    )
    return _flce_unpad(dh, N, H0), _flce_unpad(dw, V0, H0)


# -------------------------------------------------------------------- LoRA --


def _bf16_rows(t: torch.Tensor) -> torch.Tensor:
    """bf16, row-major with row strides in multiples of 8 (a copy only when
    needed). Shape and stride metadata only, so torch.compile can trace it
    inside the fused Functions; base-pointer alignment is fixed by the
    launching wrappers (_al16)."""
    if t.dtype != torch.bfloat16:
        t = t.to(torch.bfloat16)
    if t.dim() != 2 or t.stride(1) != 1 or t.stride(0) % 8 != 0 or t.stride(0) < t.shape[1]:
        t = t.contiguous()
    return t


def _al16(*ts):
    """The tensors with 16-byte aligned base pointers (an aligned copy of any
    that is not); None passes through."""
    out = []
    for t in ts:
        if t is not None and t.data_ptr() % 16 != 0:
            t = t.clone(memory_format=torch.contiguous_format)
        out.append(t)
    return out if len(out) > 1 else out[0]


def _dense16(*ts):
    """The tensors as dense row-major 2-D blocks (row stride == width) with
    16-byte aligned bases, copying any that is not: the LoRA backward entry
    points take no leading dimensions. None passes through."""
    out = []
    for t in ts:
        if t is not None and (t.stride(-1) != 1 or t.stride(0) != t.shape[-1]
                              or t.data_ptr() % 16 != 0):
            t = t.clone(memory_format=torch.contiguous_format)
        out.append(t)
    return out if len(out) > 1 else out[0]


def _ksplit_for(tiles: int, k: int) -> int:
    ktiles = (k + 63) // 64
    return max(1, min(ktiles, (512 + tiles - 1) // max(tiles, 1)))


def lora_xa(x2: torch.Tensor, a_stack: torch.Tensor) -> torch.Tensor:
    """X A^T for stacked LoRA A matrices: [N, in] x [R, in]^T -> [N, R] bf16.
    Up to 64 stacked rows: one pass over X (ml_lora_xa); more: 256x32
    tiles, split-K over in."""
    N, K = x2.shape
    R = a_stack.shape[0]
    if R <= 64 and K % 8 == 0 and x2.stride(-1) == 1 and x2.stride(0) % 8 == 0:
        out = torch.empty(N, R, dtype=torch.bfloat16, device=x2.device)
        if N == 0:
            return out
        x2, a_stack = _al16(x2, a_stack.contiguous())
        call("ml_lora_xa", ptr(x2), N, K, x2.stride(0), ptr(a_stack), R, ptr(out), out.stride(0),
             stream_of(x2))
        return out
    tiles = ((N + 255) // 256) * ((R + 31) // 32)
    return matmul(x2, a_stack, b_t=True, out_dtype=torch.bfloat16, tile_cfg=1,
                  ksplit=_ksplit_for(tiles, K))


def lora_linear_out(x2: torch.Tensor, w: torch.Tensor, xa: torch.Tensor,
                    sb: torch.Tensor) -> torch.Tensor:
    """X W^T + XA (s B)^T as ONE K-concatenated GEMM -> [N, out] bf16."""
    x2, w, xa, sb = _al16(x2, w, xa, sb)
    N, K = x2.shape
    out_f = w.shape[0]
    r = xa.shape[1]
    out = torch.empty(N, out_f, dtype=torch.bfloat16, device=x2.device)
    if N == 0:
        return out
    call(
        "ml_gemm_bf16_segments", N, out_f, 2, geom([K, r]), _hip.ptrs([x2.data_ptr(), xa.data_ptr()]),
        geom([x2.stride(0), xa.stride(0)]), _hip.ptrs([w.data_ptr(), sb.data_ptr()]),
        geom([w.stride(0), sb.stride(0)]), 0, 0, ptr(out), out.stride(0), dtype_tag(out, "out"),
        1.0, 0.0, stream_of(x2),
    )
    return out


def lora_qkv_out(x2: torch.Tensor, ws, xa: torch.Tensor, sbs) -> list:
    """The q, k, v LoRA projections X W_i^T + XA_i (s_i B_i)^T (XA_i the i-th
    block of rank columns of xa) as three K-concatenated products in ONE
    grouped launch -> three [N, out_i] bf16 tensors."""
    x2, xa = _al16(x2, xa)
    ws = [_al16(w) for w in ws]
    sbs = [_al16(sb) for sb in sbs]
    N, K = x2.shape
    rp = sbs[0].shape[1]
    outs = [torch.empty(N, w.shape[0], dtype=torch.bfloat16, device=x2.device) for w in ws]
    if N == 0:
        return outs
    k_lens, a_p, ldas, b_p, ldbs = [], [], [], [], []
    for i, (w, sb) in enumerate(zip(ws, sbs)):
        k_lens += [K, rp]
        a_p += [x2.data_ptr(), xa.data_ptr() + i * rp * xa.element_size()]
        ldas += [x2.stride(0), xa.stride(0)]
        b_p += [w.data_ptr(), sb.data_ptr()]
        ldbs += [w.stride(0), sb.stride(0)]
    call(
        "ml_gemm_bf16_segments_group", len(ws), geom([N] * len(ws)), geom([w.shape[0] for w in ws]),
        _hip.ints([2] * len(ws)), geom(k_lens), _hip.ptrs(a_p), geom(ldas), _hip.ptrs(b_p),
        geom(ldbs), 0, _hip.ptrs([o.data_ptr() for o in outs]), geom([o.stride(0) for o in outs]),
        _hip.BF16, 1.0, 0.0, stream_of(x2),
    )
    return outs


# The adapter gradients of one LoRA backward call live in one fp32 buffer:
# each gradient starts on a 256-byte boundary, in the order the call lists
# them. A caller that wants them in the parameters' dtype converts the buffer
# with one cast instead of one per gradient.
def grad_layout(shapes):
    """(offsets, total elements) of gradients of the given shapes in one buffer."""
    offs, total = [], 0
    for s in shapes:
        offs.append(total)
        n = 1
        for d in s:
            n *= int(d)
        total += -(-n // 64) * 64
    return offs, total


def grad_views(flat, shapes):
    """The gradients (views) in a buffer laid out by grad_layout."""
    offs, _ = grad_layout(shapes)
    out = []
    for o, s in zip(offs, shapes):
        n = 1
        for d in s:
            n *= int(d)
        out.append(flat[o:o + n].view(*s))
    return out


def _grad_buffer(shapes, dev):
    _, total = grad_layout(shapes)
    flat = torch.empty(max(total, 1), dtype=torch.float32, device=dev)
    return flat, grad_views(flat, shapes)


def lora_qkv_grad_shapes(IN, outs, rank):
    return [(3 * rank, IN), *((int(o), rank) for o in outs)]


def lora_qkv_bwd(x2, dys, ws_, a_stack, bs, scales, xa, rank):
    """Returns (dX bf16 [N, in], grads fp32): grads holds dA [3r, in] and
    dB_i [out_i, r] as laid out by grad_layout(lora_qkv_grad_shapes(...))."""
    ensure_rocm_device(x2, *dys, *ws_, a_stack, *bs, xa)
    x2, a_stack, xa = _dense16(x2, a_stack, xa)
    dys, ws_, bs = [list(_dense16(*t, None))[:-1] for t in (dys, ws_, bs)]
    N, IN = x2.shape
    outs = [int(d.shape[1]) for d in dys]
    dev = x2.device
    dX = torch.empty(N, IN, dtype=torch.bfloat16, device=dev)
    flat, (dA, *dBs) = _grad_buffer(lora_qkv_grad_shapes(IN, outs, rank), dev)
    if N == 0:   # no tokens: the adapter gradients are empty sums
        return dX, flat.zero_()
    wsb = _hip.query("ml_lora_qkv_bwd_workspace_bytes", N, IN, geom(outs), rank)
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=dev)
    call(
        "ml_lora_qkv_bwd", ptr(x2), N, IN, _hip.ptrs([d.data_ptr() for d in dys]), geom(outs),
        _hip.ptrs([w.data_ptr() for w in ws_]), ptr(a_stack), _hip.ptrs([b.data_ptr() for b in bs]),
        _hip.floats(scales), ptr(xa), rank, ptr(dX), ptr(dA),
        _hip.ptrs([b.data_ptr() for b in dBs]), ptr(ws), ws.numel(), stream_of(x2),
    )
    return dX, flat


def lora_linear_grad_shapes(IN, OUT, rank):
    return [(rank, IN), (int(OUT), rank)]


def lora_linear_bwd(x2, dy, w, a, b, scale, xa, rank):
    """One LoRA projection's backward: (dX bf16 [N, in], grads fp32 holding
    dA [r, in] and dB [out, r] as laid out by grad_layout)."""
    ensure_rocm_device(x2, dy, w, a, b, xa)
    x2, dy, w, a, b, xa = _dense16(x2, dy, w, a, b, xa)
    N, IN = x2.shape
    OUT = int(dy.shape[1])
    dev = x2.device
    dX = torch.empty(N, IN, dtype=torch.bfloat16, device=dev)
    flat, (dA, dB) = _grad_buffer(lora_linear_grad_shapes(IN, OUT, rank), dev)
    if N == 0:
        return dX, flat.zero_()
    wsb = _hip.query("ml_lora_linear_bwd_workspace_bytes", N, IN, OUT, rank)
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=dev)
    call(
        "ml_lora_linear_bwd", ptr(x2), N, IN, ptr(dy), OUT, ptr(w), ptr(a), ptr(b), float(scale),
        ptr(xa), rank, ptr(dX), ptr(dA), ptr(dB), ptr(ws), ws.numel(), stream_of(x2),
    )
    return dX, flat


def lora_mlp_grad_shapes(H, I, rank):
    return [(2 * rank, H), (rank, int(I)), (int(I), rank), (int(I), rank), (H, rank)]


def lora_mlp_bwd(x2, gate, up, h, dy, wg, wu, wd, a_gu, a_d, bg, bu, bd, scales, xa_gu, ha_d, rank):
    """Returns (dX, grads fp32) with grads holding dA_GU [2r, H], dA_D [r, I],
    dB_G [I, r], dB_U [I, r], dB_D [H, r] as laid out by grad_layout. h None:
    silu(gate) * up (bf16, as swiglu_fwd rounds it) is recomputed from gate
    and up instead of read."""
    ensure_rocm_device(x2, gate, up, h, dy, wg, wu, wd, a_gu, a_d, bg, bu, bd, xa_gu, ha_d)
    (x2, gate, up, h, dy, wg, wu, wd, a_gu, a_d, bg, bu, bd, xa_gu, ha_d) = _dense16(
        x2, gate, up, h, dy, wg, wu, wd, a_gu, a_d, bg, bu, bd, xa_gu, ha_d)
    N, H = x2.shape
    I = gate.shape[1]
    dev = x2.device
    dX = torch.empty(N, H, dtype=torch.bfloat16, device=dev)
    flat, (dA_GU, dA_D, dB_G, dB_U, dB_D) = _grad_buffer(lora_mlp_grad_shapes(H, I, rank), dev)
    if N == 0:
        return dX, flat.zero_()
    wsb = _hip.query("ml_lora_mlp_bwd_workspace_bytes", N, H, I, rank)
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=dev)
    call(
        "ml_lora_mlp_bwd", ptr(x2), N, H, I, ptr(gate), ptr(up), ptr(h), ptr(dy), ptr(wg), ptr(wu),
        ptr(wd), ptr(a_gu), ptr(a_d), ptr(bg), ptr(bu), ptr(bd), _hip.floats(scales), ptr(xa_gu),
        ptr(ha_d), rank, ptr(dX), ptr(dA_GU), ptr(dA_D), ptr(dB_G), ptr(dB_U), ptr(dB_D), ptr(ws),
        ws.numel(), stream_of(x2),
    )
    return dX, flat
