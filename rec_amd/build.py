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


def build(verbose: bool = False) -> str:
    """Compile every HIP source into ``librec_amd.so`` (always rebuilds)."""
    srcs = [os.path.join(CSRC, s) for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    fd, tmp = tempfile.mkstemp(suffix=".so", dir=HERE, prefix=".librec_amd.")
    os.close(fd)
    cmd = [hipcc(), *HIPCC_FLAGS, *srcs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        os.unlink(tmp)
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{proc.stderr[-8000:]}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
