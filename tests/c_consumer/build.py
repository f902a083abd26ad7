"""Build tests/c_consumer/ppk_c_consumer: a plain C host of the C-ABI (test infrastructure).

It links the product library (pop2-bezier_amd/ppk/libppk.so), the HIP runtime for device memory, and the
CPU oracle (oracle/libppk_oracle.so) as its checker; run-time paths are relative to the binary, so the tree
can move (the GPU box runs it from a copy of the repository).
"""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
EXE = os.path.join(HERE, "ppk_c_consumer")


def build(verbose: bool = True) -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    tmp = EXE + f".tmp{os.getpid()}"
    cmd = [os.environ.get("CC", "gcc"), "-std=c11", "-O2", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__",
           "-I", os.path.join(ROOT, "include"), "-I", os.path.join(rocm, "include"),
           os.path.join(HERE, "ppk_c_consumer.c"), "-o", tmp,
           "-L", os.path.join(ROOT, "pop2-bezier_amd", "ppk"), "-lppk",
           "-L", os.path.join(ROOT, "oracle"), "-lppk_oracle",
           "-L", os.path.join(rocm, "lib"), "-lamdhip64", "-lm",
           "-Wl,-rpath,$ORIGIN/../../pop2-bezier_amd/ppk:$ORIGIN/../../oracle:" + os.path.join(rocm, "lib")]
    if verbose:
        print("+", " ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"ppk_c_consumer build failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, EXE)
    return EXE


if __name__ == "__main__":
    print(build())
