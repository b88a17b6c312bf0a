"""Build the CPU oracle (test infrastructure): gcc + OpenMP -> oracle/_build/libsk_oracle.so.

Compiled for x86-64-v3 (AVX2/FMA) rather than -march=native: the library is
built in the development container and also runs on the GPU box's host CPU.
"""

from __future__ import annotations

import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "sk_oracle.c"
OUT = HERE / "_build" / "libsk_oracle.so"

# No -ffast-math: the fixed summation order and IEEE division/sqrt are part of
# the restatement.  -ffp-contract=off keeps a*b + c as two roundings.
CFLAGS = ["-O3", "-march=x86-64-v3", "-ffp-contract=off", "-fopenmp", "-fPIC", "-shared", "-std=c11"]


def build() -> Path:
    OUT.parent.mkdir(parents=True, exist_ok=True)
    tmp = OUT.with_name(OUT.name + f".{os.getpid()}.tmp")
    r = subprocess.run(["gcc", *CFLAGS, str(SRC), "-o", str(tmp), "-lm"], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stderr}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build())
