"""ml_rmsnorm_bwd_noalloc (the RMSNorm backward whose dW partials live in
the library's own device array instead of a caller workspace) against
ml_rmsnorm_bwd, both called through the C ABI: bit-identical dx and dw on
two calls in a row, the second with a smaller input, and an input whose
partials exceed the array is refused before any launch."""

import pytest
import torch

from tests.parity import seeded

pytestmark = pytest.mark.gpu


def _bwd(x, w, dy, rrms, noalloc):
    from metal_liger_amd import _hip
    rows, cols = x.shape
    dx = torch.empty_like(x)
    dw = torch.empty(cols, dtype=w.dtype, device=x.device)
    head = (_hip.ptr(x), x.stride(0), _hip.ptr(w), _hip.ptr(dy), dy.stride(0), _hip.ptr(rrms), 1e-6,
            _hip.ptr(dx), dx.stride(0), _hip.ptr(dw))
    tail = (rows, cols, _hip.dtype_tag(x, "x"), _hip.dtype_tag(w, "w"), _hip.stream_of(x))
    if noalloc:
        _hip.call("ml_rmsnorm_bwd_noalloc", *head, *tail)
    else:
        wsb = _hip.query("ml_rmsnorm_bwd_workspace_bytes", rows, cols)
        ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=x.device)
        _hip.call("ml_rmsnorm_bwd", *head, _hip.ptr(ws), ws.numel(), *tail)
    return dx, dw


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rmsnorm_bwd_noalloc_matches_workspace_entry(dev, dtype):
    from metal_liger_amd import hip_ops
    for rows, cols, seed in ((8192, 2048, 0), (300, 1536, 10)):  # second call: smaller input
        x = seeded((rows, cols), seed, dtype).to(dev)
        w = seeded((cols,), seed + 1, dtype, scale=0.1, shift=1.0).to(dev)
        dy = seeded((rows, cols), seed + 2, dtype).to(dev)
        _, rrms = hip_ops.rms_norm_fwd(x, w, 1e-6)
        want = _bwd(x, w, dy, rrms, noalloc=False)
        got = _bwd(x, w, dy, rrms, noalloc=True)
        torch.cuda.synchronize()
        assert torch.equal(got[0], want[0]), (rows, cols, "dx")
        assert torch.equal(got[1], want[1]), (rows, cols, "dw")


def test_rmsnorm_bwd_noalloc_refuses_oversized_partials(dev):
    from metal_liger_amd import _hip
    L = _hip.lib()
    # 256 partial rows x 8200 columns x 4 bytes > 8 MiB: refused on the host
    rc = L.ml_rmsnorm_bwd_noalloc(None, 8200, None, None, 8200, None, 1e-6, None, 8200, None,
                                  4096, 8200, 0, 0, None)
    assert rc != 0 and b"scratch" in L.ml_last_error()
