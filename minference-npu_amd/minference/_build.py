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
import tempfile
from concurrent.futures import ThreadPoolExecutor

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


def _run(cmd: list) -> subprocess.CompletedProcess:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(
            "hipcc failed (%d):\n%s\n%s" % (proc.returncode, " ".join(cmd), proc.stderr)
        )
    return proc


def build(verbose: bool = False, extra_flags: tuple[str, ...] = (), csrc_dir: str = CSRC_DIR,
          out_path: str = LIB_PATH, jobs: int = 0) -> str:
    """Compile every HIP source into libmsa.so; returns the library path.

    Each source is compiled to an object of its own (in parallel, ``jobs``
    processes, default one per source up to the CPU count), then the objects
    are linked into the shared library."""
    out_dir = os.path.dirname(os.path.abspath(out_path))
    os.makedirs(out_dir, exist_ok=True)
    hipcc = hipcc_path()
    jobs = jobs or max(1, min(len(SOURCES), os.cpu_count() or 1))
    with tempfile.TemporaryDirectory(prefix="msa_obj_", dir=out_dir) as obj_dir:
        objs = [os.path.join(obj_dir, os.path.splitext(s)[0] + ".o") for s in SOURCES]
        cmds = [[hipcc, *HIPCC_FLAGS, *extra_flags, "-c", "-o", o, os.path.join(csrc_dir, s)]
                for s, o in zip(SOURCES, objs)]
        with ThreadPoolExecutor(max_workers=jobs) as pool:
            procs = list(pool.map(_run, cmds))
        tmp = out_path + ".tmp"
        procs.append(_run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]))
    if verbose:
        err = "\n".join(
            ln for p in procs for ln in p.stderr.splitlines() if "packed-fp32-ops" not in ln
        )
        if err.strip():
            print(err, file=sys.stderr)
    os.replace(tmp, out_path)
    return out_path


if __name__ == "__main__":
    print(build(verbose=True))
