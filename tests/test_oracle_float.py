"""Pins of the oracle's float-KV decode attention (oracle_attention_float), CPU only.

The oracle restates pp_attention_part / pp_attention_merge
(app/src/model/decode_attention.hip:9-66) in f64. It is pinned here by a
library routine (torch's scaled_dot_product_attention in float64 on the CPU),
by closed forms (uniform keys give the mean of V, one token gives V[0],
zero inputs give zero: the check of prepare_optional_kernels,
app/src/model/mod.rs:440-451), by the validity rule (length 0 or beyond the
store gives NaN), by the per-sequence length mapping and the row strides of a
narrowed store, and by the reference's own split-K validation inputs
(hip_attention.rs:18-45). Planted mistakes in a numpy copy show that the
pins catch a wrong length index and a dropped scale.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from helpers import SEED, bf16_bits_to_f32, to_bf16_bits


def sdpa_reference(q, k, v, lengths, heads, scale=None):
    """torch's scaled_dot_product_attention in float64 with a length mask; [rows, d]. The scale defaults to
    fp32(1/sqrt(d)), the value the ABI's fp32 softmax_scale carries."""
    rows, size, d = k.shape
    if scale is None:
        scale = float(np.float32(1.0 / np.sqrt(d)))
    qt = torch.from_numpy(np.asarray(q, np.float64)).reshape(rows, 1, 1, d)
    kt = torch.from_numpy(np.asarray(k, np.float64)).reshape(rows, 1, size, d)
    vt = torch.from_numpy(np.asarray(v, np.float64)).reshape(rows, 1, size, d)
    n = np.full(rows, size) if lengths is None else np.repeat(np.asarray(lengths, np.int64), heads)
    mask = torch.from_numpy(np.arange(size)[None, :] < n[:, None]).reshape(rows, 1, 1, size)
    out = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask, scale=scale)
    return out.reshape(rows, d).numpy()


def _inputs(rng, rows, size, d, bf16):
    q = rng.standard_normal((rows, d), dtype=np.float32)
    k = rng.standard_normal((rows, size, d), dtype=np.float32)
    v = rng.standard_normal((rows, size, d), dtype=np.float32)
    if bf16:
        return q, to_bf16_bits(k), to_bf16_bits(v), bf16_bits_to_f32(to_bf16_bits(k)), bf16_bits_to_f32(to_bf16_bits(v))
    return q, k, v, k, v


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("d", [64, 128])
def test_float_attention_matches_torch_sdpa(bf16, d):
    rng = np.random.default_rng(SEED + d + bf16)
    heads, batch, size = 4, 3, 300
    rows = heads * batch
    q, k, v, kf, vf = _inputs(rng, rows, size, d, bf16)
    lengths = np.array([1, 157, 300], np.uint32)
    got = oracle.attention_float(q, k, v, lengths, heads)
    ref = sdpa_reference(q, kf, vf, lengths, heads)
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)
    # No lengths: every row attends the whole store. The oracle takes the scale as fp32 (the ABI's type).
    got = oracle.attention_float(q, k, v, None, heads, scale=0.3)
    ref = sdpa_reference(q, kf, vf, None, heads, scale=float(np.float32(0.3)))
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)


def test_float_attention_closed_forms():
    rng = np.random.default_rng(SEED)
    rows, size, d = 4, 37, 64
    v = rng.standard_normal((rows, size, d), dtype=np.float32)
    q = rng.standard_normal((rows, d), dtype=np.float32)
    # Every key identical: uniform weights over the n live tokens.
    k = np.broadcast_to(rng.standard_normal((rows, 1, d), dtype=np.float32), (rows, size, d)).copy()
    lengths = np.array([5, 37], np.uint32)
    got = oracle.attention_float(q, k, v, lengths, heads=2)
    for r in range(rows):
        n = int(lengths[r // 2])
        np.testing.assert_allclose(got[r], v[r, :n].astype(np.float64).mean(0), rtol=1e-12, atol=1e-13)
    # One live token: its value, exactly.
    got = oracle.attention_float(q, rng.standard_normal((rows, size, d), dtype=np.float32), v,
                                 np.array([1, 1], np.uint32), heads=2)
    np.testing.assert_array_equal(got, v[:, 0].astype(np.float64))
    # prepare_optional_kernels: all-zero q/K/V of 257 tokens give zero.
    z = np.zeros((1, 257, 64), np.float32)
    assert np.all(oracle.attention_float(np.zeros((1, 64), np.float32), z, z, None, 1) == 0.0)


def test_float_attention_invalid_lengths_give_nan():
    rng = np.random.default_rng(SEED + 1)
    q, k, v, _, _ = _inputs(rng, 6, 16, 64, False)
    out = oracle.attention_float(q, k, v, np.array([0, 16, 17], np.uint32), heads=2)
    assert np.isnan(out[0:2]).all() and np.isnan(out[4:6]).all()
    assert np.isfinite(out[2:4]).all()


def test_float_attention_row_strides_of_a_narrowed_store():
    rng = np.random.default_rng(SEED + 2)
    cap, size = 64, 40
    q, k, v, _, _ = _inputs(rng, 4, cap, 128, True)
    lengths = np.array([40, 23], np.uint32)
    view = oracle.attention_float(q, k[:, :size], v[:, :size], lengths, heads=2)
    dense = oracle.attention_float(q, np.ascontiguousarray(k[:, :size]), np.ascontiguousarray(v[:, :size]),
                                   lengths, heads=2)
    np.testing.assert_array_equal(view, dense)


def reference_kat_inputs(dtype_bf16: bool):
    """hip_attention::validate_split_k inputs: values(count, salt, scale) = ((i*37+salt)%107 - 53) * scale."""
    def values(count, salt, scale):
        i = np.arange(count, dtype=np.int64)
        return (((i * 37 + salt) % 107).astype(np.float32) - np.float32(53.0)) * np.float32(scale)
    q = values(64, 17, 0.013).reshape(1, 64)
    k = values(257 * 64, 23, 0.011).reshape(1, 257, 64)
    v = values(257 * 64, 31, 0.017).reshape(1, 257, 64)
    if dtype_bf16:
        return q, to_bf16_bits(k), to_bf16_bits(v)
    return q, k, v


@pytest.mark.parametrize("bf16", [False, True])
def test_reference_split_k_validation_inputs(bf16):
    q, k, v = reference_kat_inputs(bf16)
    kf = bf16_bits_to_f32(k) if bf16 else k
    vf = bf16_bits_to_f32(v) if bf16 else v
    got = oracle.attention_float(q, k, v, None, 1)
    # The reference's own comparison: softmax(q K^T / 8) V in f32, max abs error 1e-4.
    scores = (q.astype(np.float32) @ kf[0].T.astype(np.float32)) / np.float32(8.0)
    p = np.exp(scores - scores.max())
    ref32 = (p / p.sum()) @ vf[0]
    assert np.max(np.abs(got - ref32)) <= 1e-4
    np.testing.assert_allclose(got, sdpa_reference(q, kf, vf, None, 1), rtol=1e-12, atol=1e-12)


def _planted_row_lengths(q, k, v, lengths, heads):
    """Wrong: indexes lengths by row instead of by sequence (row // heads)."""
    rows, size, d = k.shape
    out = np.empty((rows, d))
    for r in range(rows):
        n = int(lengths[min(r, len(lengths) - 1)])
        s = (k[r, :n].astype(np.float64) @ q[r].astype(np.float64)) / np.sqrt(d)
        p = np.exp(s - s.max())
        out[r] = p @ v[r, :n] / p.sum()
    return out


def _planted_no_scale(q, k, v, lengths, heads):
    """Wrong: drops the 1/sqrt(d) softmax scale."""
    rows, size, d = k.shape
    out = np.empty((rows, d))
    for r in range(rows):
        n = int(lengths[r // heads])
        s = k[r, :n].astype(np.float64) @ q[r].astype(np.float64)
        p = np.exp(s - s.max())
        out[r] = p @ v[r, :n] / p.sum()
    return out


def test_pins_catch_planted_float_attention_mistakes():
    rng = np.random.default_rng(SEED + 3)
    q, k, v, _, _ = _inputs(rng, 6, 50, 64, False)
    lengths = np.array([10, 50, 31], np.uint32)
    ref = sdpa_reference(q, k, v, lengths, 2)
    np.testing.assert_allclose(oracle.attention_float(q, k, v, lengths, 2), ref, rtol=1e-12, atol=1e-12)
    for planted in (_planted_row_lengths, _planted_no_scale):
        assert np.max(np.abs(planted(q, k, v, lengths, 2) - ref)) > 1e-3, planted.__name__


@pytest.mark.parametrize("bf16", [False, True])
def test_cpu_baseline_float_matches_oracle(bf16):
    """The float path's CPU baseline (Candle's ordinary attention restated) agrees with the f64 oracle."""
    rng = np.random.default_rng(SEED + 21)
    q, k, v, _, _ = _inputs(rng, 12, 333, 64, bf16)
    got = oracle.cpu_baseline_float(q, k, v, threads=3)
    np.testing.assert_allclose(got, oracle.attention_float(q, k, v, None, 1), rtol=1e-4, atol=1e-5)
