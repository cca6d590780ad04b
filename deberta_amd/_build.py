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
# bench.py's MFMA throughput probe (include/dsa_probe.h), a library of its own
PROBE_PATH = PKG_DIR / "libdsa_probe.so"
PROBE_SOURCES = ("dsa_probe.hip",)
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


def _compile(sources, out: Path, verbose: bool) -> Path:
    srcs = [str(CSRC_DIR / s) for s in sources]
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc_path(), *HIPCC_FLAGS, *srcs, "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    if verbose:
        print(" ".join(cmd))
    os.replace(tmp, out)
    return out


def build(verbose: bool = False) -> Path:
    """Compile every HIP source: ``deberta_amd/libdsa.so`` (the kernels and
    their C ABI) and ``deberta_amd/libdsa_probe.so`` (the MFMA probe).

    Always recompiles.  Each library is written to a temporary name first and
    renamed into place, so a process that already loaded the old file keeps a
    consistent image.
    """
    _compile(PROBE_SOURCES, PROBE_PATH, verbose)
    return _compile(SOURCES, LIB_PATH, verbose)


if __name__ == "__main__":
    print(build(verbose=True))
