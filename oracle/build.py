"""Build recipe of the C oracle: ``oracle/liboracle.so`` from ``oracle/neighbor.c``.

TEST INFRASTRUCTURE ONLY. ``gcc -O2 -fopenmp -shared``; built by
``__graft_entry__.build()`` and before the CPU tests.
"""
from __future__ import annotations

import os
import shutil
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(HERE, "liboracle.so")
SOURCES = ["neighbor.c"]


def build() -> str:
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        raise RuntimeError("no C compiler for the oracle")
    tmp = LIBRARY + ".tmp"
    cmd = [cc, "-O2", "-fopenmp", "-fPIC", "-shared", "-std=c11", "-o", tmp,
           *[os.path.join(HERE, s) for s in SOURCES], "-lm"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stderr}")
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build())
