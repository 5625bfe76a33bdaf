"""Build libesmfold2_amd.so (gfx950) in-tree with hipcc.

    python -m esmfold2_mlx_amd.build      (or __graft_entry__.build())

The library is compiled for gfx950 only. Every HIP source is compiled with the
packed-fp32 target feature disabled (-Xclang -target-feature -Xclang
-packed-fp32-ops): the kernels are written without packed fp32 arithmetic and
the compiler must not introduce it.
"""

from __future__ import annotations

import hashlib
import os
import re
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_NAME = "libesmfold2_amd.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
SOURCES = ["project.hip", "contract.hip", "epilogue.hip", "q8.hip", "transition.hip", "esmc.hip",
           "recycle.hip", "wide.hip", "capi.cpp"]
HEADERS = ["common.h", "kernels.h", os.path.join("..", "..", "include", "esmfold2_amd.h")]
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP library cannot be built")


def source_hash() -> str:
    """sha256 over the names and contents of every source and header the library is built from."""
    h = hashlib.sha256()
    for name in SOURCES + HEADERS:
        h.update(name.encode() + b"\0")
        with open(os.path.join(CSRC, name), "rb") as f:
            h.update(f.read())
    return h.hexdigest()


_TAG = re.compile(rb"ESMSRC:([0-9a-f]{64})")


def library_hash(path: str = LIB_PATH) -> str | None:
    """The source hash a built library was compiled from (the ESMSRC tag capi.cpp embeds), or None."""
    try:
        with open(path, "rb") as f:
            m = _TAG.search(f.read())
    except OSError:
        return None
    return m.group(1).decode() if m else None


FLAGS = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def compile_command(src: str, obj: str, src_hash: str) -> list[str]:
    """hipcc -c of one source (every HIP source with packed fp32 disabled)."""
    return [hipcc(), *FLAGS, f"-DESM_SOURCE_HASH=\"{src_hash}\"", "-c", os.path.join(CSRC, src), "-o", obj]


def link_command(objs: list[str], out: str) -> list[str]:
    return [hipcc(), f"--offload-arch={ARCH}", "-shared", *objs, "-o", out]


def up_to_date() -> bool:
    """True when the built library exists and was compiled from the current sources (by content)."""
    return library_hash() == source_hash()


_NOISE = "is not a recognized feature for this target"  # host pass of the fp32 feature flag


def _run(procs) -> str:
    msgs, failed = [], []
    for cmd, p in procs:
        out, _ = p.communicate()
        text = "\n".join(l for l in out.splitlines() if _NOISE not in l)
        if p.returncode != 0:
            failed.append(f"{' '.join(cmd)}\n{text}")
        elif text.strip():
            msgs.append(text)
    if failed:
        raise RuntimeError("hipcc failed:\n" + "\n".join(failed))
    return "\n".join(msgs)


def build(force: bool = True, verbose: bool = False, jobs: int | None = None) -> str:
    """Compile the library (always when ``force``): one hipcc -c per source, up to ``jobs`` at a
    time, then one link into the in-tree .so. Returns its path."""
    if not force and up_to_date():
        return LIB_PATH
    import tempfile
    h = source_hash()
    jobs = jobs or max(1, min(len(SOURCES), os.cpu_count() or 1, 16))
    with tempfile.TemporaryDirectory(prefix="esm_build_") as tmpdir:
        objs, pending = [], []
        for src in SOURCES:
            obj = os.path.join(tmpdir, src.replace(".", "_") + ".o")
            objs.append(obj)
            pending.append(compile_command(src, obj, h))
        msgs = []
        while pending:
            batch, pending = pending[:jobs], pending[jobs:]
            if verbose:
                for cmd in batch:
                    print("[build]", " ".join(cmd), flush=True)
            msgs.append(_run([(cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                                                     text=True)) for cmd in batch]))
        tmp = LIB_PATH + ".tmp"
        cmd = link_command(objs, tmp)
        if verbose:
            print("[build]", " ".join(cmd), flush=True)
        msgs.append(_run([(cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                                                 text=True))]))
    if verbose and any(m.strip() for m in msgs):
        print("\n".join(m for m in msgs if m.strip()), flush=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(force=True, verbose=True))
    sys.exit(0)
