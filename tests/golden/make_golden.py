"""Generate the golden fixtures of the int8 KV path (tests/golden/*.npz).

The reference (Rust/Candle + CUDA) cannot be built or imported here, and it
stores no golden files for this path; its known-answer checks are procedural
(app/src/model/int8_kv_ops.rs:56-103). This script restates, independently of
oracle/ppk_oracle.c, in plain numpy:

  * the quantize rule of int8_kv_ops.rs:17-18 (numpy float32 division, np.rint
    is round-half-to-even, clip, two's-complement byte);
  * Candle's dequantize (.., BF16) rounding (int8_kv_ops.rs:35): float32
    product rounded to bfloat16 by torch (round-to-nearest-even);
  * the reference's host attention formula (int8_kv_ops.rs:69-73 and 94-98):
    f32 products summed left to right (Rust `.sum::<f32>()`), times 0.125,
    exp(s - max), weighted sum / z, all in float32;

and records the reference's own procedural inputs (sin/cos sequences) and the
BASELINE config-2 append case with their expected outputs.

  python tests/golden/make_golden.py   # rewrites the .npz files in place
"""
from __future__ import annotations

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
SEED = 20261011


def np_quantize(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """int8_kv_ops.rs:17-18 on the last axis: (uint8 codes, float32 scales)."""
    x = np.asarray(x, np.float32)
    with np.errstate(invalid="ignore", divide="ignore"):
        amax = np.max(np.abs(x), axis=-1)
        s = np.maximum(amax / np.float32(127.0), np.float32(1e-12)).astype(np.float32)
        q = np.rint(x / s[..., None])
        q = np.where(np.isnan(q), 0, np.clip(q, -127, 127))
    return q.astype(np.int8).view(np.uint8), s


def np_dequantize(codes: np.ndarray, scales: np.ndarray, bf16: bool) -> np.ndarray:
    y = codes.view(np.int8).astype(np.float32) * scales[..., None].astype(np.float32)
    if bf16:
        y = torch.from_numpy(y).to(torch.bfloat16).to(torch.float32).numpy()
    return y.astype(np.float32)


def _fsum(terms) -> np.float32:
    acc = np.float32(0.0)
    for t in terms:
        acc = np.float32(acc + np.float32(t))
    return acc


def host_attention(q, khist, kcur, vhist, vcur, lens) -> np.ndarray:
    """The reference's host formula, row by row, in float32 (D = 64, scale 0.125)."""
    rows, d = q.shape
    out = np.zeros((rows, d), np.float32)
    for r in range(rows):
        n = int(lens[r])
        keys = [khist[r, t] for t in range(n)] + [kcur[r]]
        vals = [vhist[r, t] for t in range(n)] + [vcur[r]]
        scores = [np.float32(_fsum(np.float32(q[r, i]) * np.float32(k[i]) for i in range(d)) * np.float32(0.125))
                  for k in keys]
        mx = max(scores)
        p = [np.float32(np.exp(np.float32(s - mx))) for s in scores]
        z = _fsum(p)
        for i in range(d):
            out[r, i] = np.float32(_fsum(np.float32(p[t] * np.float32(vals[t][i])) for t in range(n + 1)) / z)
    return out


def kat_quantize() -> dict:
    """int8_kv_ops.rs:59-62: sin(0.17 i) * 2, shape (2, 3, 64)."""
    x = (np.sin(np.arange(384, dtype=np.float32) * np.float32(0.17)) * np.float32(2.0)).astype(np.float32)
    x = x.reshape(2, 3, 64)
    codes, scales = np_quantize(x)
    return {"x": x, "codes": codes, "scales": scales}


def kat_attention_ii(kq: dict) -> dict:
    """int8_kv_ops.rs:63-74: rows 2, capacity 3, heads 1, past [2, 1], K = V = the KAT (i) codes."""
    q = np.cos(np.arange(128, dtype=np.float32) * np.float32(0.07)).astype(np.float32).reshape(2, 64)
    scratch = np.sin(np.arange(128, dtype=np.float32) * np.float32(0.09)).astype(np.float32).reshape(2, 64)
    past = np.array([2, 1], np.uint32)
    rounded = np_dequantize(kq["codes"], kq["scales"], bf16=True)  # (2, 3, 64)
    expected = host_attention(q, rounded, scratch, rounded, scratch, past)
    return {"q": q, "scratch": scratch, "past": past, "codes": kq["codes"], "scales": kq["scales"],
            "heads": np.array(1), "expected_bf16_history": expected}


def kat_attention_iii() -> dict:
    """int8_kv_ops.rs:75-101: rows 4, capacity 67, heads 2, one-row-offset views, past [0, 66]."""
    rows, cap, heads = 4, 67, 2
    n = (rows + 1) * cap * 64
    i = np.arange(n, dtype=np.float32)
    history = (np.sin(i * np.float32(0.013)) * np.float32(1.7)).astype(np.float32).reshape(rows + 1, cap, 64)[1:]
    values = (np.cos(i * np.float32(0.019)) * np.float32(0.8)).astype(np.float32).reshape(rows + 1, cap, 64)[1:]
    kc, ks = np_quantize(history)
    vc, vs = np_quantize(values)

    def vector(factor, phase):
        j = np.arange((rows + 1) * 64, dtype=np.float32)
        return np.sin(j * np.float32(factor) + np.float32(phase)).astype(np.float32).reshape(rows + 1, 64)[1:]

    q, sk, sv = vector(0.027, 0.4), vector(0.031, 1.1), vector(0.047, -0.8)
    past = np.array([0, 66], np.uint32)
    lens = np.array([past[r // heads] for r in range(rows)])
    kb = np_dequantize(kc, ks, bf16=True)
    vb = np_dequantize(vc, vs, bf16=True)
    expected = host_attention(q, kb, sk, vb, sv, lens)
    return {"k_codes": kc, "k_scales": ks, "v_codes": vc, "v_scales": vs,
            "q": q, "sk": sk, "sv": sv, "past": past, "heads": np.array(heads), "expected_bf16_history": expected}


def config2_append() -> dict:
    """one fp16 K/V token per head (H=16, D=128) with 2% heavy 10*t3 channels."""
    rng = np.random.default_rng(SEED)
    h, d = 16, 128
    out = {}
    for name in ("k", "v"):
        x = rng.standard_normal((h, d)).astype(np.float32)
        heavy = rng.permutation(h * d)[: int(round(0.02 * h * d))]
        x.reshape(-1)[heavy] = (10.0 * rng.standard_t(3, size=heavy.size)).astype(np.float32)
        x16 = x.astype(np.float16)
        codes, scales = np_quantize(x16.astype(np.float32))
        out[f"{name}_new_f16"] = x16.reshape(1, h, 1, d)
        out[f"{name}_codes"] = codes.reshape(h, 1, d)
        out[f"{name}_scales"] = scales.reshape(h, 1)
    out["past"] = np.array([1000], np.uint32)
    out["capacity"] = np.array(4096)
    return out


def main() -> None:
    kq = kat_quantize()
    np.savez(os.path.join(HERE, "kat_quantize_sin017.npz"), **kq)
    np.savez(os.path.join(HERE, "kat_attention_ii.npz"), **kat_attention_ii(kq))
    np.savez(os.path.join(HERE, "kat_attention_iii.npz"), **kat_attention_iii())
    np.savez(os.path.join(HERE, "config2_append.npz"), **config2_append())
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
