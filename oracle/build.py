"""Builds the oracle's C restatement: oracle/layout.c -> oracle/_build/liboracle.so.

Test infrastructure only (see oracle/__init__.py)."""

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(OUT_DIR, "liboracle.so")


def build() -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    tmp = LIB + ".tmp"
    subprocess.run(["gcc", "-O2", "-fPIC", "-shared", "-std=c11",
                    os.path.join(HERE, "layout.c"), "-o", tmp], check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print("built", build())
    sys.exit(0)
