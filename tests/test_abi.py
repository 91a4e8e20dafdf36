"""The C-ABI library: loads, exports every symbol include/*.h declares, and
rejects bad arguments on the host (no GPU work is issued by these calls)."""

import ctypes
import re
from pathlib import Path

import pytest

from metal_liger_amd import _hip

ROOT = Path(__file__).resolve().parents[1]


def header_functions():
    names = []
    for h in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(ml_[a-z_0-9]+)\s*\(", text, flags=re.M)
    return names


def lib():
    if not _hip.LIB_PATH.exists():
        pytest.fail(f"{_hip.LIB_PATH} not built (run __graft_entry__.build())")
    return _hip.lib()


def test_header_declares_entry_points():
    names = header_functions()
    assert len(names) >= 9, names
    assert "ml_last_error" in names and "ml_abi_version" in names


def test_library_exports_every_declared_symbol():
    L = lib()
    missing = [n for n in header_functions() if not hasattr(L, n)]
    assert not missing, f"not exported: {missing}"


def test_python_bindings_cover_the_header():
    assert set(header_functions()) == set(_hip.SIGNATURES)


def test_abi_version():
    assert lib().ml_abi_version() == _hip.ABI_VERSION


def test_host_side_argument_errors():
    L = lib()
    # cols = 0 is rejected before any HIP call
    rc = L.ml_rmsnorm_fwd(None, 0, None, None, 0, None, 4, 0, 1e-6, 0, 0, None)
    assert rc == 1 and b"bad shape" in L.ml_last_error()
    rc = L.ml_swiglu_fwd(None, None, None, 16, 0, None)
    assert rc == 1 and b"null pointer" in L.ml_last_error()
    rc = L.ml_swiglu_fwd(None, None, None, 16, 7, None)  # still null pointers first
    assert rc == 1
    g = _hip.geom([1, 1, 1, 0, 0, 0, 0, 0, 0])
    rc = L.ml_rope_pos(None, None, g, None, None, None, 3, None, 0, 0, None, 1.0, 1, None)
    assert rc == 1 and b"even" in L.ml_last_error()
    with pytest.raises(RuntimeError, match="ml_swiglu_fwd"):
        _hip.call("ml_swiglu_fwd", None, None, None, 16, 0, None)
    # a bf16 C must have a row stride that is a multiple of 8 (16-byte row
    # vectors); refused before any HIP call (the pointers are never read)
    rc = L.ml_gemm_bf16(8, 1003, 64, 4096, 64, 0, 8192, 64, 0, 16384, 1003, 1, 1.0, 0.0, None)
    assert rc == 1 and b"bf16 C" in L.ml_last_error()
    # the one-pass FLCE writes dW as 16-byte vectors: a misaligned dW is refused
    rc = L.ml_flce_fwd_grad(4096, 64, 8192, 64, None, 0, 12288, 8, 64, 64, -100, 8, 16384, 20480,
                            24576, None, 28674, None, 0, None)
    assert rc == 1 and b"16-byte aligned" in L.ml_last_error()
    assert L.ml_rmsnorm_bwd_workspace_bytes(8192, 2048) >= 8192 // 8 * 2048 * 4 // 8


def test_unsupported_dtype_is_an_error():
    L = lib()
    buf = ctypes.create_string_buffer(64)
    p = ctypes.cast(buf, ctypes.c_void_p)
    # host pointers are fine here: the dtype check fails before any launch
    rc = L.ml_swiglu_fwd(p, p, p, 4, 9, None)
    assert rc == 1 and b"dtype" in L.ml_last_error()


def test_flce_dh_split_count_fills_its_rounds():
    """The FLCE dH product splits K (the vocabulary) into work items of
    256 x 256 tiles, one workgroup per CU (256 CUs). Its split count shows in
    the workspace query (the fp32 partials: splits x T x H x 4 bytes, the
    only dH-dependent buffer): at the Qwen3 head (H = 2048, V = 151936) the
    items of the last round of a launch fill at least 3/4 of the CUs (a fixed
    item target had left 264 items at 2736-token chunks: a second round of 8
    items as long as the first); 2048-token chunks (the default at the
    config) take four splits and 4096-token chunks two."""
    L = lib()
    H, V = 2048, 151936
    al = lambda b: (b + 255) // 256 * 256
    for T, want in ((4096, 2), (8192, 1), (256, 32), (2736, None), (3072, None), (2048, 4)):
        part = (L.ml_flce_fwd_grad_workspace_bytes(T, V, H, T, 1)
                - L.ml_flce_fwd_grad_workspace_bytes(T, V, H, T, 0))
        splits, rem = divmod(part, al(T * H * 4))
        assert rem == 0 and splits >= 1, (T, part)
        if want is not None:
            assert splits == want, (T, splits)
        items = -(-T // 256) * (H // 256) * splits
        rounds = -(-items // 256)
        assert rounds == 1 or items - (rounds - 1) * 256 >= 192, (T, splits, items)
