"""Build the CPU oracle (test infrastructure): oracle/libppk_oracle.so.

gcc -O2 with -fno-fast-math -ffp-contract=off keeps every float operation a
single IEEE-754 binary32 operation, which the bit-exact quantize rule needs.

The reference's own implementations of this path cannot be built here
(Rust/Candle needs cargo and crates.io, the CUDA kernels need NVRTC, the AMD
variant needs libtorch + Windows HIPRTC), so there is no oracle/_ref.
"""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libppk_oracle.so")


def build(verbose: bool = True) -> str:
    tmp = LIB + f".tmp{os.getpid()}"
    cmd = [
        os.environ.get("CC", "gcc"), "-O2", "-std=c11", "-fPIC", "-shared", "-Wall",
        "-fno-fast-math", "-ffp-contract=off", "-pthread",
        os.path.join(HERE, "ppk_oracle.c"), "-o", tmp, "-lm",
    ]
    if verbose:
        print("+", " ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
