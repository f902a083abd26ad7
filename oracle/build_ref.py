"""Build oracle/_ref: the reference's own HIP kernels for the float-KV decode
attention (app/src/model/decode_attention.hip) and the CFG + Renyi sampler
(app/src/inference/renyi_sample.hip), compiled unchanged from where they lie
under /root/reference, plus the launcher oracle/ref_launch.cpp.

TEST INFRASTRUCTURE ONLY: tests/ use these as a second checker beside the C
oracle. Nothing is copied from the reference into the repository; outputs go
to oracle/_ref/ (git-ignored, carried to the GPU box with the tree). Both
sources include only <hip/hip_runtime.h> and <math.h>; they are built with
the reference's own compile flags (FLAGS of app/src/model/hip_kernel.rs:46:
--genco -O3 -std=c++17 -ffp-contract=off), plus the flag that keeps packed
fp32 VALU forms out of every code object run on this pool.

  python oracle/build_ref.py [--reference /root/reference]
"""
from __future__ import annotations

import argparse
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "_ref")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
# The reference's FLAGS (hip_kernel.rs:46); --genco and the target are added below.
REFERENCE_FLAGS = ["-O3", "-std=c++17", "-ffp-contract=off"]
DEVICE_FLAGS = [*REFERENCE_FLAGS, "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
SOURCES = {
    "decode_attention.hsaco": "app/src/model/decode_attention.hip",
    "renyi_sample.hsaco": "app/src/inference/renyi_sample.hip",
}


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in res.stderr.splitlines() if "is not a recognized feature for this target" not in l
                    and "argument unused during compilation" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"{' '.join(cmd)} failed:\n{err}")


def build(reference: str = "/root/reference") -> bool:
    """Returns False (and builds nothing) when the reference tree is absent."""
    if not all(os.path.exists(os.path.join(reference, s)) for s in SOURCES.values()):
        return False
    os.makedirs(OUT, exist_ok=True)
    for out, src in SOURCES.items():
        tmp = os.path.join(OUT, out + f".tmp{os.getpid()}")
        _run([f"{ROCM}/bin/hipcc", "--genco", "--offload-arch=gfx950", *DEVICE_FLAGS,
              os.path.join(reference, src), "-o", tmp])
        os.replace(tmp, os.path.join(OUT, out))
    tmp = os.path.join(OUT, f"libppk_ref.so.tmp{os.getpid()}")
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include",
          os.path.join(HERE, "ref_launch.cpp"), "-o", tmp, f"-L{ROCM}/lib", f"-Wl,-rpath,{ROCM}/lib", "-lamdhip64"])
    os.replace(tmp, os.path.join(OUT, "libppk_ref.so"))
    return True


if __name__ == "__main__":
    p = argparse.ArgumentParser()
    p.add_argument("--reference", default="/root/reference")
    ok = build(p.parse_args().reference)
    print("built oracle/_ref" if ok else "reference tree absent: oracle/_ref not built")
    sys.exit(0)
