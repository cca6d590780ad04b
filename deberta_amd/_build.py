"""Builds ``libdsa.so`` (the HIP kernels and their C ABI) in-tree with hipcc for gfx950."""

from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC_DIR = PKG_DIR / "csrc"
LIB_PATH = PKG_DIR / "libdsa.so"
SOURCES = ("dsa_capi.hip",)
ARCH = "gfx950"

# Packed fp32 VALU ops are kept out of the generated code: hipcc otherwise
# forms v_pk_{add,mul,fma}_f32 from plain float arithmetic.
HIPCC_FLAGS = (
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
)


def hipcc_path() -> str:
    """Locate hipcc (PATH first, then the ROCm install)."""
    found = shutil.which("hipcc")
    if found:
        return found
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    raise RuntimeError("hipcc not found: libdsa.so cannot be built without the ROCm toolchain")


def build(verbose: bool = False) -> Path:
    """Compile every HIP source into ``deberta_amd/libdsa.so``.

    Always recompiles.  The library is written to a temporary name first and
    renamed into place, so a process that already loaded the old file keeps a
    consistent image.
    """
    srcs = [str(CSRC_DIR / s) for s in SOURCES]
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc_path(), *HIPCC_FLAGS, *srcs, "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    if verbose:
        print(" ".join(cmd))
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
