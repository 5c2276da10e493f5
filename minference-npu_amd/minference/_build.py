"""Build libmsa.so (the HIP kernels + C ABI) in-tree for gfx950.

    python -m minference._build          (from minference-npu_amd/)

hipcc cross-compiles without a GPU.  The library lands next to this file as
``_lib/libmsa.so`` so that it travels with the source tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC_DIR = os.path.join(os.path.dirname(PKG_DIR), "csrc")
LIB_DIR = os.path.join(PKG_DIR, "_lib")
LIB_PATH = os.path.join(LIB_DIR, "libmsa.so")

SOURCES = ("msa_abi.hip", "msa_estimator.hip", "msa_attention.hip", "msa_decode.hip", "msa_vs.hip",
           "msa_rope.hip")

HIPCC_FLAGS = (
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-shared",
    "-fPIC",
    # packed fp32 VALU ops are kept out of the generated code
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
)


def hipcc_path() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = os.path.join(rocm, "bin", "hipcc")
    if os.path.exists(cand):
        return cand
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (set ROCM_PATH)")
    return found


def build(verbose: bool = False, extra_flags: tuple[str, ...] = ()) -> str:
    """Compile every HIP source into libmsa.so; returns the library path."""
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc_path(), *HIPCC_FLAGS, *extra_flags, "-o", tmp]
    cmd += [os.path.join(CSRC_DIR, s) for s in SOURCES]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(
            "hipcc failed (%d):\n%s\n%s" % (proc.returncode, " ".join(cmd), proc.stderr)
        )
    if verbose:
        err = "\n".join(
            ln for ln in proc.stderr.splitlines() if "packed-fp32-ops" not in ln
        )
        if err.strip():
            print(err, file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
