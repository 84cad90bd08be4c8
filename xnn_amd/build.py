"""Compile the HIP sources of xnn_amd into ``xnn_amd/libxnn_amd.so`` (gfx950).

One ``hipcc`` invocation per source object, then a shared link. The library
is built in-tree so that it travels with the repository snapshot to the GPU
box. Usage: ``python -m xnn_amd.build`` or :func:`build`.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIBRARY = os.path.join(HERE, "libxnn_amd.so")
SOURCES = ("edge.hip", "segment.hip", "basis_message.hip", "graph.hip", "d4.hip", "readout.hip",
           "atm.hip", "eeq.hip", "radial_mlp.hip", "uvu_conv.hip", "pair.hip", "d4_tiles.hip")
ARCH = os.environ.get("XNN_AMD_ARCH", "gfx950")

# packed FP32 instructions stay off (the compiler must not form v_pk_* f32 ops)
FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result", "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the xnn_amd HIP library cannot be built")


def build(verbose: bool = False, jobs: int = 4) -> str:
    """Compile every source and link ``libxnn_amd.so``; returns its path."""
    hipcc = _hipcc()
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    sources = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]

    def compile_one(name: str) -> str:
        obj = os.path.join(objdir, name.replace(".hip", ".o"))
        cmd = [hipcc, *FLAGS, "-I", INCLUDE, "-I", CSRC, "-c", os.path.join(CSRC, name), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed on {name}:\n{res.stderr[-6000:]}")
        return obj

    with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        objs = list(pool.map(compile_one, sources))
    tmp = LIBRARY + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr[-6000:]}")
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
