"""Build the oracle's C restatement (``rotation_seq.c``) into
``oracle/_build/liboracle_rot.so`` with gcc.  Test infrastructure only: the
product never loads it."""

from __future__ import annotations

import os
import shutil
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(BUILD, "liboracle_rot.so")
SRC = os.path.join(HERE, "rotation_seq.c")

# explicit fmaf() calls are the fused operation; nothing else may be contracted
CFLAGS = ["-O3", "-march=x86-64-v3", "-ffp-contract=off", "-fopenmp", "-fPIC", "-shared"]


def build() -> str:
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        raise RuntimeError("no C compiler to build the oracle")
    os.makedirs(BUILD, exist_ok=True)
    tmp = LIB + ".tmp"
    r = subprocess.run([cc, *CFLAGS, SRC, "-o", tmp, "-lm"], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
