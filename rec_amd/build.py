"""Build recipe for the gfx950 C-ABI library ``rec_amd/librec_amd.so``.

Run ``python -m rec_amd.build`` (or ``__graft_entry__.build()``).  The
library is compiled in-tree with ``hipcc --offload-arch=gfx950``; nothing is
JIT-compiled at import time.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "librec_amd.so")
SOURCES = ["abi.hip", "append.hip", "decode.hip", "decode_bf16.hip", "gemv.hip", "prefill.hip", "prefill_few.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # keep the compiler from emitting packed-fp32 instructions
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    # MFMA accumulators in ordinary VGPRs: the decode loop rescales them on the
    # VALU, and AGPR accumulators cost a copy out and back per chunk
    "-mllvm",
    "-amdgpu-mfma-vgpr-form",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the ROCm toolchain is required to build rec_amd")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{proc.stderr[-8000:]}")


def build(verbose: bool = False, jobs: int = 0) -> str:
    """Compile every HIP source into ``librec_amd.so`` (always rebuilds).

    Each source compiles to its own object (its own device code object) in a
    temporary directory, ``jobs`` at a time (default: one per source, at most
    the CPUs this process may use), then one link makes the library."""
    srcs = [os.path.join(CSRC, s) for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    jobs = jobs or max(1, min(len(srcs), len(os.sched_getaffinity(0))))
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    with tempfile.TemporaryDirectory(dir=HERE, prefix=".build.") as tmpdir:
        objs = [os.path.join(tmpdir, os.path.basename(s) + ".o") for s in srcs]
        with ThreadPoolExecutor(jobs) as ex:
            list(ex.map(lambda so: _run([hipcc(), *compile_flags, "-c", so[0], "-o", so[1]], verbose), zip(srcs, objs)))
        tmp = os.path.join(tmpdir, "librec_amd.so")
        _run([hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp], verbose)
        os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
