"""numpy front end of the CPU oracle (oracle/ppk_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or (cpu_baseline*, from
oracle/cpu_baseline.c) the timed CPU baseline. The product path
(pop2-bezier_amd/ppk) never imports it.

Array conventions match the C-ABI (include/ppk_int8_kv.h):
  codes  uint8 [rows, capacity, d] (two's-complement int8 bytes)
  scales float32 [rows, capacity]
  q/sk/sv float32 [rows, d]; past uint32 [rows // heads]
bf16/f16 inputs are widened to float32 exactly before they reach the oracle.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libppk_oracle.so")

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle not built: {LIB_PATH} (run python oracle/build.py)")
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        Z = ctypes.c_size_t
        L.oracle_quantize.argtypes = [P, Z, Z, P, P]
        L.oracle_quantize.restype = Z
        L.oracle_dequantize.argtypes = [P, P, Z, Z, ctypes.c_int, P]
        L.oracle_dequantize.restype = None
        L.oracle_append.argtypes = [P, Z, Z, Z, Z, P, Z, P, P]
        L.oracle_append.restype = Z
        L.oracle_attention.argtypes = [P, P, P, P, P, P, P, P, Z, Z, Z, Z, ctypes.c_float, ctypes.c_int, P]
        L.oracle_attention.restype = None
        L.oracle_attention_mt.argtypes = [P, P, P, P, P, P, P, P, Z, Z, Z, Z, ctypes.c_float, ctypes.c_int, Z, P]
        L.oracle_attention_mt.restype = ctypes.c_int
        L.oracle_attention_splitk_reference.argtypes = [P, P, P, P, P, P, P, P, Z, Z, Z, Z, ctypes.c_float, Z, P]
        L.oracle_attention_splitk_reference.restype = None
        L.oracle_attention_float.argtypes = [P, P, P, ctypes.c_int, Z, Z, P, Z, Z, Z, Z, ctypes.c_float, P]
        L.oracle_attention_float.restype = None
        L.oracle_renyi_sample.argtypes = [P, Z, Z, P, P, ctypes.c_float, ctypes.c_float, Z, ctypes.c_uint32,
                                          ctypes.c_int, P, P, P, P]
        L.oracle_renyi_sample.restype = ctypes.c_int
        _lib = L
    return _lib


BASELINE_PATH = os.path.join(HERE, "libppk_cpu_baseline.so")
_baseline = None


def baseline_lib() -> ctypes.CDLL:
    """oracle/libppk_cpu_baseline.so: the Candle CPU path timed by bench.py (oracle/cpu_baseline.c)."""
    global _baseline
    if _baseline is None:
        if not os.path.exists(BASELINE_PATH):
            raise RuntimeError(f"CPU baseline not built: {BASELINE_PATH} (run python oracle/build.py)")
        L = ctypes.CDLL(BASELINE_PATH)
        P = ctypes.c_void_p
        Z = ctypes.c_size_t
        L.cpu_baseline_float_decode.argtypes = [P, P, P, ctypes.c_int, Z, Z, Z, ctypes.c_float, Z, P]
        L.cpu_baseline_float_decode.restype = ctypes.c_int
        L.cpu_baseline_decode.argtypes = [P, P, P, P, P, P, P, P, Z, Z, Z, Z, ctypes.c_float, Z, P]
        L.cpu_baseline_decode.restype = ctypes.c_int
        L.cpu_baseline_uses_avx2.argtypes = []
        L.cpu_baseline_uses_avx2.restype = ctypes.c_int
        _baseline = L
    return _baseline


def cpu_baseline_isa() -> str:
    return "AVX2+FMA" if baseline_lib().cpu_baseline_uses_avx2() else "x86-64 (SSE2)"


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def quantize(x: np.ndarray) -> tuple[np.ndarray, np.ndarray, int]:
    """int8_kv_ops::quantize on [..., d] float32 -> (codes uint8 [..., d], scales f32 [...], nonfinite rows)."""
    x = _c(x, np.float32)
    d = x.shape[-1]
    rows = x.size // d
    codes = np.empty(x.shape, np.uint8)
    scales = np.empty(x.shape[:-1], np.float32)
    bad = lib().oracle_quantize(_p(x), rows, d, _p(codes), _p(scales))
    return codes, scales, int(bad)


def dequantize(codes: np.ndarray, scales: np.ndarray, round_bf16: bool = False) -> np.ndarray:
    codes = _c(codes, np.uint8)
    scales = _c(scales, np.float32)
    d = codes.shape[-1]
    rows = codes.size // d
    assert scales.size == rows
    out = np.empty(codes.shape, np.float32)
    lib().oracle_dequantize(_p(codes), _p(scales), rows, d, int(bool(round_bf16)), _p(out))
    return out


def append(src: np.ndarray, past: np.ndarray, codes: np.ndarray, scales: np.ndarray) -> int:
    """In-place append of src [B, H, T, d] into arenas codes [B*H, cap, d], scales [B*H, cap]."""
    src = _c(src, np.float32)
    past = _c(past, np.uint32)
    assert codes.flags.c_contiguous and scales.flags.c_contiguous
    assert codes.dtype == np.uint8 and scales.dtype == np.float32
    b, h, t, d = src.shape
    cap = codes.shape[1]
    return int(lib().oracle_append(_p(src), b, h, t, d, _p(past), cap, _p(codes), _p(scales)))


def attention(q, k, v, ks, vs, sk, sv, past, heads: int, scale: float | None = None,
              history_bf16: bool = False, threads: int | None = None) -> np.ndarray:
    """f64 decode attention (see oracle_attention); returns float64 [rows, d]. Rows are shared out over
    `threads` POSIX threads (default: the usable cores, at most 16); the result does not depend on it."""
    k = _c(k, np.uint8)
    v = _c(v, np.uint8)
    rows, cap, d = k.shape
    q = _c(q, np.float32).reshape(rows, d)
    sk = _c(sk, np.float32).reshape(rows, d)
    sv = _c(sv, np.float32).reshape(rows, d)
    ks = _c(ks, np.float32).reshape(rows, cap)
    vs = _c(vs, np.float32).reshape(rows, cap)
    past = _c(past, np.uint32)
    assert past.size == rows // heads and rows % heads == 0
    if scale is None:
        scale = 1.0 / np.sqrt(d)
    if threads is None:
        threads = max(1, min(len(os.sched_getaffinity(0)), 16))
    out = np.empty((rows, d), np.float64)
    lib().oracle_attention_mt(_p(q), _p(k), _p(v), _p(ks), _p(vs), _p(sk), _p(sv), _p(past), rows, heads, cap, d,
                              float(scale), int(bool(history_bf16)), int(threads), _p(out))
    return out


def attention_splitk_reference(q, k, v, ks, vs, sk, sv, past, heads: int, split: int,
                               scale: float | None = None) -> np.ndarray:
    """The reference kernel's f32 split-K arithmetic (bf16 history); float32 [rows, d]."""
    k = _c(k, np.uint8)
    v = _c(v, np.uint8)
    rows, cap, d = k.shape
    q = _c(q, np.float32).reshape(rows, d)
    sk = _c(sk, np.float32).reshape(rows, d)
    sv = _c(sv, np.float32).reshape(rows, d)
    ks = _c(ks, np.float32).reshape(rows, cap)
    vs = _c(vs, np.float32).reshape(rows, cap)
    past = _c(past, np.uint32)
    assert past.size == rows // heads and rows % heads == 0
    if scale is None:
        scale = 1.0 / np.sqrt(d)
    out = np.empty((rows, d), np.float32)
    lib().oracle_attention_splitk_reference(_p(q), _p(k), _p(v), _p(ks), _p(vs), _p(sk), _p(sv), _p(past), rows,
                                            heads, cap, d, float(scale), int(split), _p(out))
    return out


def cpu_baseline(q, k, v, ks, vs, sk, sv, past, heads: int, threads: int, scale: float | None = None) -> np.ndarray:
    """Candle CPU decode restated op for op (oracle/cpu_baseline.c cpu_baseline_decode); float32 [rows, d]."""
    k = _c(k, np.uint8)
    v = _c(v, np.uint8)
    rows, cap, d = k.shape
    q = _c(q, np.float32).reshape(rows, d)
    sk = _c(sk, np.float32).reshape(rows, d)
    sv = _c(sv, np.float32).reshape(rows, d)
    ks = _c(ks, np.float32).reshape(rows, cap)
    vs = _c(vs, np.float32).reshape(rows, cap)
    past = _c(past, np.uint32)
    assert past.size == rows // heads and rows % heads == 0
    if scale is None:
        scale = 1.0 / np.sqrt(d)
    out = np.empty((rows, d), np.float32)
    rc = baseline_lib().cpu_baseline_decode(_p(q), _p(k), _p(v), _p(ks), _p(vs), _p(sk), _p(sv), _p(past), rows,
                                            heads, cap, d, float(scale), int(threads), _p(out))
    if rc != 0:
        raise RuntimeError("cpu_baseline_decode: a worker thread failed to start (ran inline)")
    return out


def attention_float(q, k, v, lengths, heads: int, scale: float | None = None) -> np.ndarray:
    """Float-KV decode attention (see oracle_attention_float). k/v: float32 or bfloat16 bits (uint16)
    arrays [rows, size, d] (row-strided views allowed); lengths: uint32 [rows // heads] or None."""
    kv_bf16 = k.dtype == np.uint16
    assert v.dtype == k.dtype and k.shape == v.shape
    rows, size, d = k.shape
    elem = 2 if kv_bf16 else 4
    for a in (k, v):
        assert a.strides[2] == elem and a.strides[1] == d * elem, "tokens must be dense"
    q = _c(q, np.float32).reshape(rows, d)
    if lengths is not None:
        lengths = _c(lengths, np.uint32)
        assert lengths.size == rows // heads
    if scale is None:
        scale = 1.0 / np.sqrt(d)
    out = np.empty((rows, d), np.float64)
    lib().oracle_attention_float(_p(q), k.ctypes.data, v.ctypes.data, int(kv_bf16), k.strides[0] // elem,
                                 v.strides[0] // elem, _p(lengths) if lengths is not None else None, rows, heads,
                                 size, d, float(scale), _p(out))
    return out


def renyi_sample(raw, uniforms, bounds, alpha: float, cfg: float, guidance: int, offset: int,
                 cfg_fma: bool = False) -> dict:
    """CFG + Renyi sampler (see oracle_renyi_sample). raw float32 [batch*guidance, choices];
    uniforms float32 [batch]; bounds uint32 [batch, 2] = (start, count). Returns a dict of
    token / valid / support (uint32 [batch]) and margin (float32 [batch]); raises ValueError
    for metadata the reference rejects. cfg_fma=False is the reference's separately rounded CFG value;
    True (a fused multiply-add) exists only for tests that show a case separates the two forms."""
    raw = _c(raw, np.float32)
    physical, choices = raw.shape
    uniforms = _c(uniforms, np.float32).reshape(-1)
    bounds = _c(bounds, np.uint32).reshape(-1, 2)
    if physical % guidance or uniforms.size != physical // guidance or bounds.shape[0] != physical // guidance:
        raise ValueError("renyi_sample input lengths differ")
    batch = physical // guidance
    token = np.empty(batch, np.uint32)
    valid = np.empty(batch, np.uint32)
    support = np.empty(batch, np.uint32)
    margin = np.empty(batch, np.float32)
    rc = lib().oracle_renyi_sample(_p(raw), physical, choices, _p(uniforms), _p(bounds), float(alpha), float(cfg),
                                   guidance, int(offset), int(bool(cfg_fma)), _p(token), _p(valid), _p(support),
                                   _p(margin))
    if rc != 0:
        raise ValueError("invalid reference metadata")
    return {"token": token, "valid": valid, "support": support, "margin": margin}


def cpu_baseline_float(q, k, v, threads: int, scale: float | None = None) -> np.ndarray:
    """Candle's ordinary CPU attention over a dense bf16 (uint16 bits) or f32 store [rows, size, d], f32,
    parallel over rows (see cpu_baseline_float_decode); float32 [rows, d]."""
    kv_bf16 = k.dtype == np.uint16
    k = np.ascontiguousarray(k)
    v = np.ascontiguousarray(v, dtype=k.dtype)
    rows, size, d = k.shape
    q = _c(q, np.float32).reshape(rows, d)
    if scale is None:
        scale = 1.0 / np.sqrt(d)
    out = np.empty((rows, d), np.float32)
    rc = baseline_lib().cpu_baseline_float_decode(_p(q), k.ctypes.data, v.ctypes.data, int(kv_bf16), rows, size, d,
                                         float(scale), int(threads), _p(out))
    if rc != 0:
        raise RuntimeError("cpu_baseline_float_decode: a worker thread failed to start (ran inline)")
    return out
