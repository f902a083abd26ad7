"""Seeded synthetic inputs and comparison helpers shared by the tests."""
from __future__ import annotations

import json
import os

import numpy as np

SEED = 20261011  # the reference acceptance tool's default seed (app/src/bin/kv_int8_acceptance.rs:93)
ATOL, RTOL = 2e-3, 1e-2  # attention bar vs the fp32-dequantised oracle: max abs 2e-3 and max relative 1e-2


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


# Relative errors are taken where |oracle| >= REL_FLOOR (elements nearer zero are held by the absolute bar).
REL_FLOOR = 1e-3
# Set PPK_PARITY_LOG=path to append one JSON line per comparison (what, max abs, max rel, elements).
_PARITY_LOG = os.environ.get("PPK_PARITY_LOG")


def narrow_half_ulp(ref: np.ndarray, dtype: str | None) -> np.ndarray | float:
    """Half a unit in the last place of |ref| in a 16-bit output type ("bf16" / "f16"), 0 for f32 outputs:
    the rounding the output conversion itself adds, which is the type's and not the kernel's."""
    if dtype is None or dtype == "f32":
        return 0.0
    mant, min_exp = (7, -126) if dtype == "bf16" else (10, -14)
    e = np.floor(np.log2(np.maximum(np.abs(ref), np.finfo(np.float64).tiny)))
    return 0.5 * np.exp2(np.maximum(e, min_exp) - mant)


def assert_close(got: np.ndarray, ref: np.ndarray, atol: float = ATOL, rtol: float = RTOL, what: str = "",
                 rel_floor: float = REL_FLOOR, out_dtype: str | None = None) -> tuple[float, float]:
    """The parity bar as two separate maxima: max |got - ref| <= atol, and max |got - ref| / |ref| <= rtol
    over the elements with |ref| >= rel_floor (rtol <= 0: no relative bar). Non-finite references must be
    matched exactly: NaN where the reference is NaN, the same infinity (sign included). For a 16-bit output
    (out_dtype "bf16" / "f16") the output type's own rounding, half an ulp at |ref|, is taken off each
    error first. Prints and returns (max abs error, max relative error)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    finite = np.isfinite(ref)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan), f"{what}: NaN pattern differs"
    inf = ~finite & ~nan
    assert np.array_equal(got[inf], ref[inf]), f"{what}: infinities differ"
    assert np.isfinite(got[finite]).all(), f"{what}: non-finite output where the reference is finite"
    g, r = got[finite], ref[finite]
    if g.size == 0:
        return 0.0, 0.0
    err = np.maximum(np.abs(g - r) - narrow_half_ulp(r, out_dtype), 0.0)
    max_abs = float(err.max())
    big = np.abs(r) >= rel_floor
    max_rel = float((err[big] / np.abs(r[big])).max()) if big.any() else 0.0
    print(f"parity {what}: max abs {max_abs:.3e}, max rel {max_rel:.3e} over {g.size} elements")
    if _PARITY_LOG:
        with open(_PARITY_LOG, "a") as f:
            f.write(json.dumps({"what": what, "max_abs": max_abs, "max_rel": max_rel, "n": int(g.size),
                                "atol": atol, "rtol": rtol}) + "\n")
    assert max_abs <= atol, f"{what}: max abs error {max_abs:.3e} > {atol:g}"
    if rtol > 0:
        assert max_rel <= rtol, f"{what}: max relative error {max_rel:.3e} > {rtol:g} (|ref| >= {rel_floor:g})"
    return max_abs, max_rel
