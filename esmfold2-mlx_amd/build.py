"""Build libesmfold2_amd.so (gfx950) in-tree with hipcc.

    python -m esmfold2_mlx_amd.build      (or __graft_entry__.build())

The library is compiled for gfx950 only. Every HIP source is compiled with the
packed-fp32 target feature disabled (-Xclang -target-feature -Xclang
-packed-fp32-ops): the kernels are written without packed fp32 arithmetic and
the compiler must not introduce it.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_NAME = "libesmfold2_amd.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
SOURCES = ["project.hip", "contract.hip", "epilogue.hip", "q8.hip", "transition.hip", "esmc.hip", "recycle.hip", "capi.cpp"]
HEADERS = ["common.h", "kernels.h", os.path.join("..", "..", "include", "esmfold2_amd.h")]
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP library cannot be built")


def command(out: str = LIB_PATH) -> list[str]:
    return [hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared", "-Wall",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            *[os.path.join(CSRC, s) for s in SOURCES], "-o", out]


def up_to_date() -> bool:
    if not os.path.exists(LIB_PATH):
        return False
    t = os.path.getmtime(LIB_PATH)
    deps = [os.path.join(CSRC, s) for s in SOURCES + HEADERS]
    return all(os.path.getmtime(d) <= t for d in deps if os.path.exists(d))


def build(force: bool = True, verbose: bool = False) -> str:
    """Compile the library (always when ``force``); returns its path."""
    if not force and up_to_date():
        return LIB_PATH
    tmp = LIB_PATH + ".tmp"
    cmd = command(tmp)
    if verbose:
        print("[build]", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"  # host pass of the fp32 feature flag
    msgs = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{msgs}")
    if verbose and msgs.strip():
        print(msgs, flush=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(force=True, verbose=True))
    sys.exit(0)
