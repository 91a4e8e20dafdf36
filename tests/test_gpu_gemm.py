"""GPU: the bf16 MFMA GEMM engine against torch (fp32 products of the same
bf16 inputs), for every operand layout, ragged M/N/K, K segments, and
alpha/beta accumulation."""

import ctypes

import pytest
import torch

from tests.parity import assert_close, seeded

pytestmark = pytest.mark.gpu


def ref_mm(a, b, a_t, b_t):
    A = a.float().t() if a_t else a.float()
    B = b.float().t() if b_t else b.float()
    return A @ B


@pytest.mark.parametrize("a_t", [False, True])
@pytest.mark.parametrize("b_t", [False, True])
@pytest.mark.parametrize("mnk", [(256, 256, 64), (512, 768, 1024), (136, 264, 200), (8, 8, 8),
                                 (1000, 520, 48), (296, 40, 2048)])
def test_gemm_layouts(dev, a_t, b_t, mnk):
    from metal_liger_amd import hip_ops
    M, N, K = mnk
    a = seeded((K, M) if a_t else (M, K), 1, torch.bfloat16)
    b = seeded((N, K) if b_t else (K, N), 2, torch.bfloat16)
    out = hip_ops.matmul(a.to(dev), b.to(dev), a_t=a_t, b_t=b_t)
    ref = ref_mm(a, b, a_t, b_t)
    # fp32 bar, scale-aware (different summation order)
    assert_close(out, ref, f"gemm {mnk} a_t={a_t} b_t={b_t}")
    outb = hip_ops.matmul(a.to(dev), b.to(dev), a_t=a_t, b_t=b_t, out_dtype=torch.bfloat16)
    assert_close(outb, ref.to(torch.bfloat16), "gemm bf16 out")


@pytest.mark.parametrize("K", [128, 136, 192, 320, 384, 448, 520])
@pytest.mark.parametrize("b_t", [True, False])
def test_gemm_r4_k_tile_counts(dev, K, b_t):
    """A K-major A runs the r4 engine, whose five 32 KB LDS slots hold two
    k-tiles and a free slot and rotate every k-tile (a period of 5): 2, 3,
    3, 5, 6, 7 and 9 k-tiles of 64 cover every count modulo 5, with ragged
    K (136, 520); both B layouts; bf16 and fp32 outputs and a beta pass."""
    from metal_liger_amd import hip_ops
    M, N = 520, 776
    a = seeded((M, K), 40, torch.bfloat16)
    b = seeded((N, K) if b_t else (K, N), 41, torch.bfloat16)
    ref = ref_mm(a, b, False, b_t)
    out = hip_ops.matmul(a.to(dev), b.to(dev), b_t=b_t)
    assert_close(out, ref, f"r4 K={K} b_t={b_t}")
    outb = hip_ops.matmul(a.to(dev), b.to(dev), b_t=b_t, out_dtype=torch.bfloat16)
    assert_close(outb, ref.to(torch.bfloat16), f"r4 K={K} b_t={b_t} bf16 out")
    c0 = seeded((M, N), 42, torch.bfloat16)
    c = c0.to(dev).clone()
    hip_ops.matmul(a.to(dev), b.to(dev), b_t=b_t, out=c, alpha=0.5, beta=1.0)
    assert_close(c, (0.5 * ref.to(torch.bfloat16).float() + c0.float()).to(torch.bfloat16),
                 f"r4 K={K} b_t={b_t} beta")


def test_gemm_alpha_beta_and_strides(dev):
    from metal_liger_amd import hip_ops
    big = seeded((600, 1040), 3, torch.bfloat16).to(dev)
    a = big[:, 16:528]                         # row stride 1040, K = 512
    b = seeded((512, 384), 4, torch.bfloat16).to(dev)
    c0 = seeded((600, 384), 5).to(dev)
    c = c0.clone()
    hip_ops.matmul(a, b, out=c, alpha=0.5, beta=2.0)
    ref = 0.5 * (a.float() @ b.float()) + 2.0 * c0
    assert_close(c, ref, "alpha/beta")


def test_gemm_segments(dev):
    """K-concatenated operands: [A1 | A2 | A3] @ [B1; B2; B3], incl. a 48-long segment."""
    from metal_liger_amd import _hip
    M, N = 520, 272
    ks = [256, 128, 48]
    As = [seeded((M, k), 10 + i, torch.bfloat16).to(dev) for i, k in enumerate(ks)]
    Bs = [seeded((k, N), 20 + i, torch.bfloat16).to(dev) for i, k in enumerate(ks)]
    C = torch.empty(M, N, device=dev)
    _hip.call("ml_gemm_bf16_segments", M, N, len(ks), _hip.geom(ks), _hip.ptrs([t.data_ptr() for t in As]),
              _hip.geom([t.stride(0) for t in As]), _hip.ptrs([t.data_ptr() for t in Bs]),
              _hip.geom([t.stride(0) for t in Bs]), 0, 1, C.data_ptr(), C.stride(0), 0, 1.0, 0.0,
              torch.cuda.current_stream().cuda_stream)
    ref = sum(a.float() @ b.float() for a, b in zip(As, Bs))
    assert_close(C, ref, "segments")


def test_gemm_bf16_output_row_stride(dev):
    """A bf16 C is stored as 16-byte rows of 8 columns: the C ABI refuses a
    row stride that is not a multiple of 8, and matmul with an odd N and no
    `out` computes in fp32 and rounds once."""
    from metal_liger_amd import hip_ops
    a = seeded((300, 264), 50, torch.bfloat16)
    b = seeded((1003, 264), 51, torch.bfloat16)
    out = hip_ops.matmul(a.to(dev), b.to(dev), b_t=True, out_dtype=torch.bfloat16)
    assert out.shape == (300, 1003) and out.dtype == torch.bfloat16
    assert_close(out, ref_mm(a, b, False, True).to(torch.bfloat16), "bf16 out, N = 1003")
    c = torch.empty(300, 1003, dtype=torch.bfloat16, device=dev)
    with pytest.raises(RuntimeError, match="bf16 C"):
        hip_ops.matmul(a.to(dev), b.to(dev), b_t=True, out=c)


def test_gemm_rejects_bad_shapes(dev):
    from metal_liger_amd import hip_ops
    a = torch.zeros(64, 12, dtype=torch.bfloat16, device=dev)   # K = 12 not a multiple of 8
    b = torch.zeros(12, 64, dtype=torch.bfloat16, device=dev)
    with pytest.raises(RuntimeError, match="multiple of 8"):
        hip_ops.matmul(a, b)


@pytest.mark.parametrize("cfg", [0, 1, 2])
@pytest.mark.parametrize("ksplit", [1, 3, 8])
@pytest.mark.parametrize("a_t,b_t,mnk", [(False, True, (520, 48, 2048)), (True, False, (48, 264, 1000)),
                                         (True, False, (2048, 16, 777)), (False, False, (300, 32, 512))])
def test_gemm_splitk_shapes(dev, cfg, ksplit, a_t, b_t, mnk):
    """Tile shapes 256x256 / 256x32 / 64x256 with split-K (fixed-order partial sums)."""
    from metal_liger_amd import hip_ops
    M, N, K = mnk
    a_kmajor, b_kmajor = not a_t, b_t
    if (a_kmajor or b_kmajor) and K % 8:
        pytest.skip("K-major operands need K % 8 == 0")
    a = seeded((K, M) if a_t else (M, K), 31, torch.bfloat16)
    b = seeded((N, K) if b_t else (K, N), 32, torch.bfloat16)
    out = hip_ops.matmul(a.to(dev), b.to(dev), a_t=a_t, b_t=b_t, tile_cfg=cfg, ksplit=ksplit)
    assert_close(out, ref_mm(a, b, a_t, b_t), f"splitk cfg={cfg} ks={ksplit} {mnk}")
    c0 = seeded((M, N), 33).to(dev)
    c = c0.clone()
    hip_ops.matmul(a.to(dev), b.to(dev), a_t=a_t, b_t=b_t, out=c, alpha=2.0, beta=0.5,
                   tile_cfg=cfg, ksplit=ksplit)
    assert_close(c, 2.0 * ref_mm(a, b, a_t, b_t) + 0.5 * c0.cpu(), "splitk alpha/beta")


@pytest.mark.parametrize("b_t", [True, False])
def test_gemm_segments_group_matches_single_launches(dev, b_t):
    """ml_gemm_bf16_segments_group: each product of one grouped launch equals
    the same product launched alone (same engine, segments and tile order:
    bit for bit), for the LoRA QKV forward's shapes scaled down (q twice as
    wide as k and v, a rank-16 segment beside each) plus ragged sizes."""
    from metal_liger_amd import _hip
    M, K, r = 600, 264, 16
    outs_n = [512, 256, 136]
    X = seeded((M, K), 30, torch.bfloat16).to(dev)
    XA = seeded((M, 3 * r), 31, torch.bfloat16).to(dev)
    Ws = [seeded((n, K) if b_t else (K, n), 32 + i, torch.bfloat16).to(dev) for i, n in enumerate(outs_n)]
    SBs = [seeded((n, r) if b_t else (r, n), 40 + i, torch.bfloat16).to(dev) for i, n in enumerate(outs_n)]
    b_layout = 0 if b_t else 1
    a_p, ldas, b_p, ldbs, k_lens = [], [], [], [], []
    for i in range(3):
        k_lens += [K, r]
        a_p += [X.data_ptr(), XA.data_ptr() + 2 * r * i]
        ldas += [X.stride(0), XA.stride(0)]
        b_p += [Ws[i].data_ptr(), SBs[i].data_ptr()]
        ldbs += [Ws[i].stride(0), SBs[i].stride(0)]
    for dtype, tag in ((torch.bfloat16, 1), (torch.float32, 0)):
        Cg = [torch.full((M, n), float("nan"), dtype=dtype, device=dev) for n in outs_n]
        _hip.call("ml_gemm_bf16_segments_group", 3, _hip.geom([M] * 3), _hip.geom(outs_n),
                  _hip.ints([2, 2, 2]), _hip.geom(k_lens), _hip.ptrs(a_p), _hip.geom(ldas),
                  _hip.ptrs(b_p), _hip.geom(ldbs), b_layout, _hip.ptrs([c.data_ptr() for c in Cg]),
                  _hip.geom([c.stride(0) for c in Cg]), tag, 1.0, 0.0,
                  torch.cuda.current_stream().cuda_stream)
        for i, n in enumerate(outs_n):
            C1 = torch.full((M, n), float("nan"), dtype=dtype, device=dev)
            _hip.call("ml_gemm_bf16_segments", M, n, 2, _hip.geom(k_lens[2 * i:2 * i + 2]),
                      _hip.ptrs(a_p[2 * i:2 * i + 2]), _hip.geom(ldas[2 * i:2 * i + 2]),
                      _hip.ptrs(b_p[2 * i:2 * i + 2]), _hip.geom(ldbs[2 * i:2 * i + 2]), 0,
                      b_layout, C1.data_ptr(), C1.stride(0), tag, 1.0, 0.0,
                      torch.cuda.current_stream().cuda_stream)
            torch.cuda.synchronize()
            assert torch.equal(Cg[i], C1), (i, dtype)
            Wf = Ws[i].float() if not b_t else Ws[i].float().t()
            Sf = SBs[i].float() if not b_t else SBs[i].float().t()
            ref = X.float() @ Wf + XA[:, r * i:r * (i + 1)].float() @ Sf
            assert_close(Cg[i], ref.to(dtype), f"group product {i}")


def test_gemm_segments_group_rejects_bad_counts(dev):
    from metal_liger_amd import _hip
    with pytest.raises(RuntimeError, match="grouped|products"):
        _hip.call("ml_gemm_bf16_segments_group", 4, _hip.geom([8] * 4), _hip.geom([8] * 4),
                  _hip.ints([1] * 4), _hip.geom([8] * 4), _hip.ptrs([0] * 4), _hip.geom([8] * 4),
                  _hip.ptrs([0] * 4), _hip.geom([8] * 4), 0, _hip.ptrs([0] * 4),
                  _hip.geom([8] * 4), 1, 1.0, 0.0, torch.cuda.current_stream().cuda_stream)
