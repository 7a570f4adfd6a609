"""Ahead-of-time build of the gfx950 HIP library ``libreskv_hip.so``.

The library is built in-tree (next to this file) so it travels with the source
tree; there is no JIT build at import time.  ``python -m reskv_amd.build``
rebuilds it.  Environment: ``RESKV_HIPCC`` (compiler path, default
``/opt/rocm/bin/hipcc``), ``RESKV_OFFLOAD_ARCH`` (default ``gfx950``),
``RESKV_VERBOSE_BUILD=1`` (echo the command).
"""

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB_NAME = "libreskv_hip.so"
SOURCES = ("capi.hip", "encode.hip", "kmeans.hip", "decode.hip", "llama_ops.hip")


def library_path() -> Path:
    return HERE / LIB_NAME


def build_command(out: Path):
    hipcc = os.environ.get("RESKV_HIPCC", "/opt/rocm/bin/hipcc")
    arch = os.environ.get("RESKV_OFFLOAD_ARCH", "gfx950")
    flags = [
        hipcc,
        f"--offload-arch={arch}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-Wall",
        "-Wno-unused-function",
        # packed fp32 VALU forms are kept out of every kernel
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # matrix-core accumulators in ordinary VGPRs: accumulators that the VALU
        # rescales are then not copied between the two register files
        "-mllvm", "-amdgpu-mfma-vgpr-form",
        f"-I{HERE.parent / 'include'}",
        "-o", str(out),
    ]
    return flags + [str(CSRC / s) for s in SOURCES]


def build(verbose: bool = False) -> Path:
    out = library_path()
    tmp = out.with_suffix(".so.tmp")
    cmd = build_command(tmp)
    if verbose or os.environ.get("RESKV_VERBOSE_BUILD") == "1":
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed building {LIB_NAME} (exit {proc.returncode})")
    warnings = [ln for ln in proc.stderr.splitlines() if "warning" in ln and "packed-fp32-ops" not in ln]
    if warnings and verbose:
        sys.stderr.write("\n".join(warnings) + "\n")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
