"""GPU parity of the float-KV balanced plan (ppk_fdecode_flat_* + ppk_fmerge_flat_*).

The plan is taken when the caller passes its host copy of the lengths
(PpkFloatAttentionArgs.lengths_host) for a ragged batch whose longest row
holds more than 512 KiB of K and V and whose per-row plan's waves are uneven
(large batches of short rows beside long ones); every test below asserts
that its shape takes it. Bars as for the per-row plan
(tests/test_gpu_float_attention.py): against the f64 oracle, max abs error
<= 1e-4 and max relative error <= 1e-2 (|oracle| >= 1e-3); rows whose length
is 0, beyond the store or max_length, or whose device length differs from
the host copy, give NaN.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import ppk
from helpers import SEED, assert_close
from test_gpu_float_attention import ATOL, RTOL, FloatCase

pytestmark = pytest.mark.gpu


def _plan(c: FloatCase, lengths_host, **kw):
    a, _ = ppk.fused_attention.decode_attention_args(c.q, c.k, c.v, c.lengths_t, c.H, lengths_host=lengths_host,
                                                     **kw)
    return ppk.fused_attention.plan(a, ppk.context(c.q.device))


def _balanced(c: FloatCase, lengths_host, **kw) -> int:
    """Asserts the host lengths change the plan (the balanced one) and returns its record slots per row."""
    plan = _plan(c, lengths_host, **kw)
    assert plan != _plan(c, None, **kw), "the balanced plan is taken"
    return plan[1]


@pytest.mark.parametrize("kv", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("d", [64, 128, 256])
def test_ragged_batch_balanced(device, kv, d):
    size = 262144 // d  # rows of 1 MiB (bf16) or 2 MiB (f32) of K and V
    lengths = [size, 1, 700, 64, size // 2, 3, 65, 3 * size // 8] + [30] * 24
    c = FloatCase(device, 32, 8, d, size, kv, lengths=lengths, seed=SEED + d)
    assert _balanced(c, lengths) > 1
    ref = c.reference()
    got = c.run(lengths_host=lengths)
    assert_close(got, ref, atol=ATOL, rtol=RTOL, what=f"balanced d{d} {kv}")
    # The per-row plan over the same inputs agrees within the same bar.
    assert_close(c.run(), ref, atol=ATOL, rtol=RTOL, what=f"per-row d{d} {kv}")


@pytest.mark.parametrize("kv", [torch.bfloat16, torch.float32])
def test_skewed_long_rows(device, kv):
    """The shape the balanced plan is for: a few long sequences beside many short ones."""
    lengths = [4096, 256, 256, 4096] + [256] * 26 + [150, 4000]
    c = FloatCase(device, len(lengths), 8, 128, 4096, kv, lengths=lengths, seed=SEED + 11)
    assert _balanced(c, lengths) > 1
    assert_close(c.run(lengths_host=lengths), c.reference(), atol=ATOL, rtol=RTOL, what=f"skewed {kv}")


@pytest.mark.parametrize("d", [64, 128, 256])
def test_edge_lengths_balanced(device, d):
    """Empty rows, one-token rows, rows at the store's size, rows past it (NaN), single-unit rows beside
    rows of many units."""
    lengths = [0, 1, 700, 2000, 2049, 3, 2048, 5000] + [2000] * 2 + [10] * 22
    c = FloatCase(device, 32, 8, d, 2048, torch.float32, lengths=lengths, seed=SEED + 12 + d)
    assert _balanced(c, lengths) > 1
    got = c.run(lengths_host=lengths)
    ref = c.reference()
    bad = np.repeat((np.array(lengths) == 0) | (np.array(lengths) > 2048), 8)
    assert np.isnan(got[bad]).all() and np.isnan(ref[bad]).all()
    assert not np.isnan(got[~bad]).any()
    assert_close(got[~bad], ref[~bad], atol=ATOL, rtol=RTOL, what=f"edge lengths d{d}")


def test_rows_beyond_max_length_give_nan(device):
    lengths = [300, 2800, 2400, 2600, 2400] + [40] * 27
    c = FloatCase(device, 32, 8, 128, 3000, torch.float32, lengths=lengths, seed=SEED + 13)
    _balanced(c, lengths, max_length=2500)
    ref = c.reference()
    bad = np.repeat(np.array(lengths) > 2500, 8)
    for host in (lengths, None):  # balanced and per-row plans
        got = c.run(lengths_host=host, max_length=2500)
        assert np.isnan(got[bad]).all() and not np.isnan(got[~bad]).any()
        assert_close(got[~bad], ref[~bad], atol=ATOL, rtol=RTOL, what=f"rows within max_length ({host})")


def test_per_row_plan_nans_rows_beyond_max_length_inside_its_cover(device):
    """max_length = 50 plans one wave per row; with an explicit 64-token split a 60-token row fits the wave
    but exceeds max_length, and gives NaN as documented rather than its value (so does the automatic plan,
    whose wave covers 52 tokens)."""
    c = FloatCase(device, 2, 4, 64, 100, torch.float32, lengths=[60, 40], seed=SEED + 14)
    assert _plan(c, None, max_length=50)[1] == 1
    a, _ = ppk.fused_attention.decode_attention_args(c.q, c.k, c.v, c.lengths_t, c.H, 64, max_length=50)
    assert ppk.fused_attention.plan(a, ppk.context(device))[:2] == (64, 1)
    got = c.run(64, max_length=50)
    assert np.isnan(got[:4]).all()
    assert_close(got[4:], c.reference()[4:], atol=ATOL, rtol=RTOL, what="row within max_length, split 64")
    got = c.run(max_length=50)
    assert np.isnan(got[:4]).all()
    assert_close(got[4:], c.reference()[4:], atol=ATOL, rtol=RTOL, what="row within max_length")


def test_stale_device_lengths_give_nan(device):
    """A sequence whose device length differs from the host copy the plan was made from gives NaN rows;
    the others are computed."""
    lengths = [2000, 64, 700, 5] + [30] * 28
    c = FloatCase(device, 32, 8, 128, 2048, torch.bfloat16, lengths=lengths, seed=SEED + 15)
    stale = [2000, 64, 701, 5] + lengths[4:]
    assert _balanced(c, stale) > 1
    got = c.run(lengths_host=stale)
    bad = np.repeat(np.array(stale) != np.array(lengths), 8)
    assert np.isnan(got[bad]).all() and not np.isnan(got[~bad]).any()
    assert_close(got[~bad], c.reference()[~bad], atol=ATOL, rtol=RTOL, what="fresh rows")


def test_short_ragged_rows_keep_the_per_row_plan(device):
    """Longest row within 512 KiB of K and V: the host lengths change nothing (the per-row plan, bit for
    bit the same outputs). Even per-row waves (few rows, short splits) keep it as well."""
    lengths = [10, 0, 60, 1024]
    c = FloatCase(device, 4, 16, 64, 1024, torch.bfloat16, lengths=lengths, seed=SEED + 16)
    assert _plan(c, lengths) == _plan(c, None)
    got = c.run(lengths_host=lengths)
    np.testing.assert_array_equal(got, c.run())
    ref = c.reference()
    assert np.isnan(got[16:32]).all() and np.isnan(ref[16:32]).all()
    ok = np.r_[0:16, 32:64]
    assert_close(got[ok], ref[ok], atol=ATOL, rtol=RTOL, what="short ragged rows")
    few = FloatCase(device, 4, 4, 128, 4096, torch.bfloat16, lengths=[4096, 1, 700, 64], seed=SEED + 18)
    assert _plan(few, [4096, 1, 700, 64]) == _plan(few, None)


def test_dtypes_and_prepared_call(device):
    """bf16/f16 outputs are the f32 result rounded once; a bf16 query computes what the f32 query of the same
    values computes; the prepared call (argument block built once) gives the functional call's bits."""
    lengths = [3000, 30, 900, 64] + [20] * 28
    c = FloatCase(device, 32, 8, 128, 3072, torch.bfloat16, lengths=lengths, seed=SEED + 17)
    assert _balanced(c, lengths) == 47, "balanced: 47 units of 64 tokens"
    f32 = c.run(lengths_host=lengths)
    for dt in (torch.bfloat16, torch.float16):
        out = ppk.fused_attention.decode_attention(c.q, c.k, c.v, c.lengths_t, c.H, out_dtype=dt,
                                                   lengths_host=lengths)
        torch.cuda.synchronize()
        expect = torch.from_numpy(f32).to(dt).float().numpy()
        np.testing.assert_array_equal(out.float().reshape(c.rows, c.D).cpu().numpy(), expect)
    qb = c.q.to(torch.bfloat16)
    np.testing.assert_array_equal(c.run(q=qb, lengths_host=lengths), c.run(q=qb.float(), lengths_host=lengths))
    prepared = ppk.fused_attention.FloatDecodeAttention(c.q, c.k, c.v, c.lengths_t, c.H, lengths_host=lengths)
    assert prepared.ngroups > 1
    for _ in range(2):
        out = prepared()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.reshape(c.rows, c.D).cpu().numpy(), f32)
