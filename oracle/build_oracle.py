"""Build the C restatement oracle/fa2_blockwise.c into oracle/build/libfa2_oracle.so.

Test infrastructure only (tests/ load it as a checker).  The reference itself
(Dell710000/ascend-rsfa) is Python + TritonAscend with no C/C++ sources, so
there is nothing under /root/reference to compile into oracle/_ref.
"""
import os
import shutil
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "fa2_blockwise.c")
OUT_DIR = os.path.join(HERE, "build")
LIB = os.path.join(OUT_DIR, "libfa2_oracle.so")


def build():
    os.makedirs(OUT_DIR, exist_ok=True)
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        raise RuntimeError("no C compiler found for the oracle")
    tmp = LIB + ".tmp"
    subprocess.run([cc, "-O2", "-std=c99", "-fPIC", "-shared", "-Wall", "-Werror", "-o", tmp, SRC, "-lm"],
                   check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
