"""Seeded synthetic inputs and comparison helpers shared by the tests."""
from __future__ import annotations

import numpy as np

SEED = 20261011  # the reference acceptance tool's default seed (app/src/bin/kv_int8_acceptance.rs:93)
ATOL, RTOL = 2e-3, 1e-2  # attention tolerance vs the fp32-dequantised oracle


def heavy_channels(rng: np.random.Generator, heads: int, d: int, frac: float = 0.02) -> np.ndarray:
    """round(frac*H*D) (head, channel) pairs chosen by a seeded permutation (flat indices h*d + c)."""
    n = int(round(frac * heads * d))
    return np.sort(rng.permutation(heads * d)[:n])


def kv_values(rng: np.random.Generator, b: int, h: int, t: int, d: int, heavy: bool = True) -> np.ndarray:
    """float32 [b, h, t, d] ~ N(0,1); with heavy=True, 2% of (head, channel) pairs are 10 * Student-t(3)
    for every token (the heavy-tail rule of the benchmark configs)."""
    x = rng.standard_normal((b, h, t, d), dtype=np.float32)
    if heavy:
        for flat in heavy_channels(rng, h, d):
            hh, cc = divmod(int(flat), d)
            x[:, hh, :, cc] = (10.0 * rng.standard_t(3, size=(b, t))).astype(np.float32)
    return x


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bits, round-to-nearest-even (NaN kept quiet)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    r[nan] = 0x7FC0
    return r


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def assert_close(got: np.ndarray, ref: np.ndarray, atol: float = ATOL, rtol: float = RTOL, what: str = "") -> float:
    """|got - ref| <= atol + rtol*|ref| elementwise, NaN where the reference is NaN. Returns max abs error."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan), f"{what}: NaN pattern differs"
    g, r = got[~nan], ref[~nan]
    if g.size == 0:
        return 0.0
    err = np.abs(g - r)
    bad = err > atol + rtol * np.abs(r)
    assert not bad.any(), f"{what}: {int(bad.sum())} elements out of tolerance, max abs err {err.max():.3e}"
    return float(err.max())
