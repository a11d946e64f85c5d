"""Builds libspikeinfer_amd.so (gfx950) in-tree with hipcc.

Usage: ``python -m spikeinfer_amd.build`` (or ``build()`` from Python).  The
library is a plain C-ABI shared object (see include/spikeinfer_amd.h); it is
loaded with ctypes by ``spikeinfer_amd._lib``.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_NAME = "libspikeinfer_amd.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
ARCH = "gfx950"

# -ffp-contract=off: the LIF recurrence must round mul and add separately.
# -packed-fp32-ops off: no v_pk_*_f32 in generated code.
HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "-shared",
    f"--offload-arch={ARCH}",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def sources() -> list[str]:
    return sorted(
        os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip")
    )


def build(verbose: bool = False) -> str:
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc, *HIPCC_FLAGS, "-o", tmp, *sources()]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
