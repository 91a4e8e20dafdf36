"""Build recipe for libmetal_liger_amd.so (the C-ABI HIP library, gfx950).

Replaces the reference's setup_ext.py (a CppExtension over Objective-C++ and
the macOS Metal SDK, setup_ext.py:32-87): every ``csrc/*.hip`` file is
compiled by ``hipcc --offload-arch=gfx950`` into an object under ``_build/``
(in parallel) and the objects are linked into one shared library next to this
file. The library has no torch dependency; Python binds it with ctypes.

Usage: ``python -m metal_liger_amd.build`` (or ``build()`` from Python).
"""

from __future__ import annotations

import concurrent.futures as _cf
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC_DIR = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_NAME = "libmetal_liger_amd.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
ARCH = "gfx950"

# -packed-fp32-ops: hipcc must not form v_pk_{add,mul,fma}_f32 from scalar or
# float2 code (some forms have produced silently wrong results on these GPUs).
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP library cannot be built")


def _sources() -> list[str]:
    return sorted(
        os.path.join(CSRC_DIR, f) for f in os.listdir(CSRC_DIR) if f.endswith(".hip")
    )


def _compile(hipcc: str, src: str, extra: list[str]) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src)[:-4] + ".o")
    cmd = [hipcc, *HIP_FLAGS, *extra, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass does not know the packed-fp32 feature and says so; that
    # warning is expected and harmless.
    noise = "is not a recognized feature for this target"
    msgs = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {os.path.basename(src)}:\n{msgs}")
    if msgs.strip():
        print(msgs, file=sys.stderr)
    return obj


def build(verbose: bool = True, jobs: int | None = None, extra_flags: list[str] | None = None) -> str:
    """Compiles every csrc/*.hip for gfx950 and links the shared library.

    Always rebuilds (the build is the "does it compile" check). Returns the
    path of the library.
    """
    hipcc = _hipcc()
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = _sources()
    extra = list(extra_flags or [])
    jobs = jobs or min(len(srcs), max(1, min(16, os.cpu_count() or 1)))
    with _cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(hipcc, s, extra), srcs))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)  # atomic: a loaded old copy stays valid
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} sources", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build()
