"""Times this repository's kernels beside the reference's own HIP kernels
(built unchanged from their sources into oracle/_ref) on identical device
buffers, at the reference's shapes. Prints one JSON line per workload.

TEST-SIDE TOOL (not collected by pytest): it runs the oracle/_ref checker
kernels, which bench.py may not. Also the command the committed rocprofv3
summary profiles/reference_kernels_vs_ppk_trace.md was made with.

  python tests/compare_reference_kernels.py [--iters 200]
"""
from __future__ import annotations

import argparse
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
for sub in ("pop2-bezier_amd", "oracle", "tests"):
    sys.path.insert(0, os.path.join(ROOT, sub))

import numpy as np  # noqa: E402
import torch  # noqa: E402

import ppk  # noqa: E402
import refkernels  # noqa: E402

SEED = 20261011


def timed(fn, iters: int) -> float:
    for _ in range(20):
        fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(iters):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / iters * 1e3


def float_attention(iters: int, kv: torch.dtype, split: int) -> dict:
    """The reference's largest float-KV decode: 32 x 16 rows of a 1024-token D = 64 store."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(SEED)
    rows, size, heads = 512, 1024, 16
    k = torch.randn((rows, size, 64), generator=g, device=dev).to(kv)
    v = torch.randn((rows, size, 64), generator=g, device=dev).to(kv)
    q = torch.randn((rows, 1, 64), generator=g, device=dev)
    lengths = torch.full((rows // heads,), size, dtype=torch.int32, device=dev)
    ours = ppk.FloatDecodeAttention(q, k, v, lengths, heads, split)
    ours_us = timed(ours, iters)
    ref_us = timed(lambda: refkernels.decode_attention(q, k, v, lengths, heads, split), iters)
    diff = (ours.out.reshape(rows, 64) - refkernels.decode_attention(q, k, v, lengths, heads, split)).abs().max()
    kv_bytes = rows * size * 64 * 2 * (2 if kv == torch.bfloat16 else 4)
    return {"workload": f"float-KV decode attention rows=512 length=1024 D=64 {str(kv)[6:]} split={split}",
            "ppk_us": round(ours_us, 2), "reference_us": round(ref_us, 2),
            "ppk_gbps": round(kv_bytes / ours_us / 1e3, 1), "reference_gbps": round(kv_bytes / ref_us / 1e3, 1),
            "speedup": round(ref_us / ours_us, 2), "max_abs_diff": float(diff)}


def sampler(iters: int, batch: int, guidance: int, choices: int) -> dict:
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(SEED)
    raw = torch.from_numpy((rng.standard_normal((batch * guidance, choices)) * 3).astype(np.float32)).to(dev)
    u = torch.from_numpy(rng.uniform(0, 1, (batch, 1)).astype(np.float32)).to(dev)
    b = torch.from_numpy(np.tile(np.array([0, choices], np.int32), (batch, 1))).to(dev)
    cfg = 2.0 if guidance == 2 else 1.0
    ours = ppk.RenyiSampler(raw, u, b, 4.0, cfg, guidance, 0)
    ours_us = timed(ours, iters)
    ref_us = timed(lambda: refkernels.renyi_sample(raw, u, b, 4.0, cfg, guidance, 0), iters)
    same = bool(torch.equal(ours(), refkernels.renyi_sample(raw, u, b, 4.0, cfg, guidance, 0)))
    return {"workload": f"CFG + Renyi sampler batch={batch} guidance={guidance} choices={choices} alpha=4",
            "ppk_us": round(ours_us, 2), "reference_us": round(ref_us, 2), "speedup": round(ref_us / ours_us, 2),
            "bit_identical": same}


def main() -> int:
    p = argparse.ArgumentParser()
    p.add_argument("--iters", type=int, default=200)
    args = p.parse_args()
    for kv in (torch.bfloat16, torch.float32):
        for split in (0, 128):
            print(json.dumps(float_attention(args.iters, kv, split)), flush=True)
    for batch, guidance, choices in ((32, 2, 2048), (32, 1, 2048), (8, 2, 512)):
        print(json.dumps(sampler(args.iters, batch, guidance, choices)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
