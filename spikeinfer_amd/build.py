"""Builds libspikeinfer_amd.so (gfx950) in-tree with hipcc.

Usage: ``python -m spikeinfer_amd.build`` (or ``build()`` from Python).  The
library is a plain C-ABI shared object (see include/spikeinfer_amd.h); it is
loaded with ctypes by ``spikeinfer_amd._lib``.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_NAME = "libspikeinfer_amd.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
ARCH = "gfx950"

# -ffp-contract=off: the LIF recurrence must round mul and add separately.
# -packed-fp32-ops off: no v_pk_*_f32 in generated code.
HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC",
    f"--offload-arch={ARCH}",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def sources() -> list[str]:
    return sorted(
        os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip")
    )


OBJ_DIR = os.path.join(HERE, "_build")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr}")


def build(verbose: bool = False) -> str:
    """Compiles every csrc/*.hip to an object (in parallel, one hipcc per
    file) and links them into the shared library.  Always recompiles."""
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sources()
    objs = [os.path.join(OBJ_DIR, os.path.basename(s)[:-4] + ".o") for s in srcs]
    jobs = max(1, min(len(srcs), os.cpu_count() or 1, 16))
    with ThreadPoolExecutor(jobs) as ex:
        list(ex.map(lambda so: _run([hipcc, *HIPCC_FLAGS, "-c", "-o", so[1], so[0]], verbose),
                    zip(srcs, objs)))
    tmp = LIB_PATH + ".tmp"
    _run([hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", tmp, *objs], verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
