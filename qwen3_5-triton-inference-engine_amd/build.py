"""Build libwy_attn.so (the gfx950 HIP kernels + C ABI) in-tree with hipcc.

Run as ``python build.py`` from anywhere, or call :func:`build`.  The library
lands next to this file in ``lib/libwy_attn.so``; nothing is installed.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_DIR = PKG_DIR / "lib"
LIB_PATH = LIB_DIR / "libwy_attn.so"
OBJ_DIR = PKG_DIR / "_build"
ARCH = os.environ.get("WY_OFFLOAD_ARCH", "gfx950")

SOURCES = ["capi.hip", "kv_cache.hip", "rope_gate.hip", "rmsnorm.hip", "decode.hip", "prefill.hip",
           "prefill_direct.hip", "prefill_short.hip", "gemm.hip", "gdn.hip", "gdn_block.hip", "gdn_chunk.hip",
           "model_ops.hip"]

# Per-source extra flags.  The direct-launch prefill variants keep their MFMA
# accumulators in VGPRs (faster there; the queue variants in prefill.hip are
# slower with it).
EXTRA_FLAGS = {"prefill_direct.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
               "prefill_short.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}

# Packed fp32 VALU ops are disabled: their occasional silent miscompares on
# this hardware pool are not worth the few percent they might buy.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain (ROCm) is required to build")


def _compile(hipcc: str, src: str) -> Path:
    obj = OBJ_DIR / (Path(src).stem + ".o")
    cmd = [hipcc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(src, []), "-c", str(CSRC / src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every kernel source for gfx950 and link ``lib/libwy_attn.so``."""
    hipcc = _hipcc()
    OBJ_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(4, os.cpu_count() or 1)) as ex:
        objs = list(ex.map(lambda s: _compile(hipcc, s), SOURCES))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
