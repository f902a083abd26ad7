"""Build the CPU oracle and the CPU baseline (test infrastructure):
oracle/libppk_oracle.so and oracle/libppk_cpu_baseline.so.

The oracle: gcc -O2 with -fno-fast-math -ffp-contract=off keeps every float
operation a single IEEE-754 binary32 operation, which the bit-exact quantize
rule needs. The baseline (oracle/cpu_baseline.c, the Candle CPU path timed by
bench.py): gcc -O3 with fused multiply-adds allowed, its hot loops compiled
for AVX2 + FMA beside plain x86-64 and picked at run time, as Candle's gemm
crate does.

The reference's own implementations of the int8 path cannot be built here
(Rust/Candle needs cargo and crates.io, the CUDA kernels need NVRTC, the AMD
variant needs libtorch + Windows HIPRTC); oracle/build_ref.py builds the
reference's two HIP kernels of the float path and the sampler.
"""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libppk_oracle.so")


BASELINE_LIB = os.path.join(HERE, "libppk_cpu_baseline.so")


def _compile(src: str, out: str, flags: list[str], verbose: bool) -> None:
    tmp = out + f".tmp{os.getpid()}"
    cmd = [os.environ.get("CC", "gcc"), *flags, "-std=c11", "-fPIC", "-shared", "-Wall", "-pthread",
           os.path.join(HERE, src), "-o", tmp, "-lm"]
    if verbose:
        print("+", " ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"{src} build failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)


def build(verbose: bool = True) -> str:
    _compile("ppk_oracle.c", LIB, ["-O2", "-fno-fast-math", "-ffp-contract=off"], verbose)
    _compile("cpu_baseline.c", BASELINE_LIB, ["-O3", "-fno-fast-math", "-ffp-contract=fast"], verbose)
    return LIB


if __name__ == "__main__":
    print(build())
