"""Comparison helpers with the tolerances of the parity bar.

fp32: rtol 1e-5 with a scale-aware atol (1e-5 * max |ref|), because summation
order differs between the GPU and torch's CPU kernels and near-zero entries
of cancelling sums have no meaningful relative error.
bf16 / fp16: rtol 2e-2, atol 1e-2, plus relative Frobenius error <= 2e-2
(atol alone is vacuous for tiny gradients).
"""

import torch

FP32_RTOL = 1e-5
LOW_RTOL, LOW_ATOL, LOW_FRO = 2e-2, 1e-2, 2e-2


def rel_fro(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    den = b.norm().item()
    return (a - b).norm().item() / den if den > 0 else (a - b).norm().item()


def assert_close(out: torch.Tensor, ref: torch.Tensor, what: str = "", dtype=None):
    dtype = dtype or ref.dtype
    out = out.detach().cpu()
    ref = ref.detach().cpu()
    assert out.shape == ref.shape, f"{what}: shape {tuple(out.shape)} != {tuple(ref.shape)}"
    o = out.double()
    r = ref.double()
    if not torch.isfinite(r).all():
        same_nonfinite = torch.equal(torch.isfinite(o), torch.isfinite(r))
        assert same_nonfinite, f"{what}: non-finite pattern differs"
        mask = torch.isfinite(r)
        o, r = o[mask], r[mask]
    if o.numel() == 0:
        return
    scale = r.abs().max().item()
    if dtype in (torch.float32, torch.float64):
        tol = FP32_RTOL * r.abs() + FP32_RTOL * scale
        err = (o - r).abs()
        bad = err > tol
        assert not bad.any(), (
            f"{what}: {int(bad.sum())} of {o.numel()} elements beyond fp32 bar; "
            f"max err {err.max().item():.3e} (scale {scale:.3e})"
        )
    else:
        ok = torch.allclose(o, r, rtol=LOW_RTOL, atol=LOW_ATOL)
        fro = rel_fro(o, r)
        assert ok, f"{what}: max err {(o - r).abs().max().item():.3e} beyond rtol 2e-2/atol 1e-2"
        assert fro <= LOW_FRO, f"{what}: relative Frobenius error {fro:.3e} > 2e-2"


def seeded(shape, seed, dtype=torch.float32, scale=1.0, shift=0.0):
    """N(shift, scale^2) drawn on the CPU from a seeded generator, then cast."""
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g, dtype=torch.float32) * scale + shift).to(dtype)
