"""Build the MI355X int8 KV decode library in-tree.

Outputs (next to the Python package, git-ignored, shipped with the tree):
  ppk/ppk_kernels.hsaco  gfx950 code object with every kernel (hipcc --genco)
  ppk/ppk_kernels_clock.hsaco  the same kernels with the wave-clock diagnostics (-DPPK_WAVE_CLOCK)
  ppk/libppk.so          C-ABI shim + int8_kv_ops host mirror (include/ppk_int8_kv.h), with
                         the no-alloc entry point's device scratch array (csrc/ppk_scratch.hip,
                         compiled by hipcc for gfx950 and linked in)

Usage: python pop2-bezier_amd/build.py
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "ppk")
ROOT = os.path.dirname(HERE)

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.environ.get("HIPCC", f"{ROCM}/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
ARCH = "gfx950"
# Packed-fp32 VALU forms stay off: hipcc would otherwise emit them from plain
# float code, and some of their forms have produced wrong results on this pool.
DEVICE_FLAGS = ["-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print("+", " ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(
        line for line in (res.stderr or "").splitlines() if "is not a recognized feature for this target" not in line
    )
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{res.stdout}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = True) -> dict:
    os.makedirs(OUT, exist_ok=True)
    hsaco = os.path.join(OUT, "ppk_kernels.hsaco")
    clock = os.path.join(OUT, "ppk_kernels_clock.hsaco")
    lib = os.path.join(OUT, "libppk.so")
    probe = os.path.join(OUT, "libppk_probe.so")
    tmp_probe = probe + f".tmp{os.getpid()}"
    tmp_hsaco = hsaco + f".tmp{os.getpid()}"
    tmp_clock = clock + f".tmp{os.getpid()}"
    tmp_lib = lib + f".tmp{os.getpid()}"
    tmp_obj = os.path.join(OUT, f"ppk_scratch.o.tmp{os.getpid()}")
    try:
        _run(
            [HIPCC, "--genco", f"--offload-arch={ARCH}", *DEVICE_FLAGS, os.path.join(CSRC, "ppk_kernels.hip"), "-o",
             tmp_hsaco],
            verbose,
        )
        # The same kernels with the wave-clock diagnostics compiled in, for a
        # context created with this code object (bench.py --wave-clock).
        _run(
            [HIPCC, "--genco", f"--offload-arch={ARCH}", *DEVICE_FLAGS, "-DPPK_WAVE_CLOCK",
             os.path.join(CSRC, "ppk_kernels.hip"), "-o", tmp_clock],
            verbose,
        )
        # The device scratch array of the no-alloc entry point lives in the
        # library itself (a __device__ variable in a HIP translation unit).
        _run(
            [HIPCC, "-c", "-fPIC", f"--offload-arch={ARCH}", *DEVICE_FLAGS, "-fvisibility=hidden",
             f"-I{os.path.join(ROOT, 'include')}", os.path.join(CSRC, "ppk_scratch.hip"), "-o", tmp_obj],
            verbose,
        )
        # The shim is host-only code over the HIP runtime API: plain g++.
        _run(
            [
                CXX, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-fvisibility=hidden", "-D__HIP_PLATFORM_AMD__",
                f"-I{os.path.join(ROOT, 'include')}", f"-I{ROCM}/include",
                os.path.join(CSRC, "ppk_abi.cpp"), os.path.join(CSRC, "int8_kv_ops.cpp"),
                os.path.join(CSRC, "fused_attention.cpp"), os.path.join(CSRC, "kv_arena.cpp"), tmp_obj,
                "-o", tmp_lib, f"-L{ROCM}/lib", f"-Wl,-rpath,{ROCM}/lib", "-lamdhip64", "-ldl",
            ],
            verbose,
        )
        # The streaming-read probe bench.py --probe compares the decode with: a
        # library of its own, not part of the decode library's C-ABI.
        _run(
            [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *DEVICE_FLAGS,
             os.path.join(CSRC, "ppk_read_probe.hip"), "-o", tmp_probe],
            verbose,
        )
        # The outputs replace the previous build together, only once all compiled.
        os.replace(tmp_hsaco, hsaco)
        os.replace(tmp_clock, clock)
        os.replace(tmp_lib, lib)
        os.replace(tmp_probe, probe)
    finally:
        for t in (tmp_hsaco, tmp_clock, tmp_lib, tmp_obj, tmp_probe):
            if os.path.exists(t):
                os.remove(t)
    return {"hsaco": hsaco, "clock_hsaco": clock, "lib": lib, "probe_lib": probe}


if __name__ == "__main__":
    print(build())
