"""Build recipe for the C part of the oracle (test infrastructure only).

Compiles permute_oracle.c with gcc into oracle/_build/liboracle_uttt.so.
-ffp-contract=off keeps every multiply and add separately rounded unless the
source asks for fmaf() explicitly, so the restatement's rounding points are
exactly the ones written in the source.
"""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "permute_oracle.c")
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(OUT_DIR, "liboracle_uttt.so")


def build(force: bool = True) -> str:
    if not force and os.path.exists(LIB) and os.path.getmtime(LIB) >= os.path.getmtime(SRC):
        return LIB
    os.makedirs(OUT_DIR, exist_ok=True)
    tmp = LIB + ".tmp"
    subprocess.run(
        ["gcc", "-O2", "-std=c99", "-ffp-contract=off", "-fPIC", "-shared", SRC, "-o", tmp, "-lm"],
        check=True,
    )
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
