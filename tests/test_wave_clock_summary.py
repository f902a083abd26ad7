"""Host logic of the wave-clock breakdown (bench.py summarize_wave_clock) on hand-built records.

Record layout (pop2-bezier_amd/csrc/ppk_kernel_args.h): [0] kind << 56 | launch sequence << 32 | block << 8 | wave,
[1] XCC id << 32 | HW_ID, [2 + i] the wave's 100 MHz clock at point i. Decode points: 0 entry, 1 loads issued,
2 past here, 3 first K data here, 4 stream done, 5 block joined, 6 output / record stored. Merge points: 0 entry,
1 records combined, 2 output stored.
"""
from __future__ import annotations

import importlib.util
import os

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _record(kind, seq, block, wave, xcc, ticks):
    r = np.zeros(16, dtype=np.uint64)
    r[0] = (kind << 56) | (seq << 32) | (block << 8) | wave
    r[1] = xcc << 32
    r[2:2 + len(ticks)] = ticks
    return r


def _decode(seq, block, wave, xcc, t0, stream):
    # entry, +1 loads, +2 past, +3 first data, +3+stream done, +1 joined, +2 stored (10 ns ticks)
    first = t0 + 3
    done = first + stream
    return _record(1, seq, block, wave, xcc, [t0, t0 + 1, t0 + 2, first, done, done + 1, done + 3, 0])


def test_summary_of_two_layers_with_merges(bench):
    recs = []
    base = 1_000_000
    for seq in range(2):
        t = base + seq * 10_000
        # block 0 on XCC 0 (streams 100 ticks), block 1 on XCC 1 (streams 150 ticks); two waves each
        for w in range(2):
            recs.append(_decode(seq, 0, w, 0, t, 100))
            recs.append(_decode(seq, 1, w, 1, t + 2, 150))
        last_store = t + 2 + 3 + 150 + 3          # wave 0 of block 1 stores last
        m0 = last_store + 50                       # merge enters 50 ticks later
        recs.append(_record(2, seq, 0, 0, 0, [m0, m0 + 20, m0 + 25]))
    rec = np.stack(recs)
    summary, md = bench.summarize_wave_clock(rec)
    us = 1e6 / bench.WAVE_CLOCK_HZ  # 0.01 us per tick
    assert summary["launches"] == 2 and summary["records"] == len(recs)
    med = summary["decode_wave_intervals_us_median"]
    assert med["entry -> loads issued"] == pytest.approx(1 * us)
    assert med["entry -> first K data here"] == pytest.approx(3 * us)
    assert med["first K data -> stream done"] == pytest.approx(125 * us)  # median of 100, 100, 150, 150
    assert summary["decode_dispatch_spread_us"] == pytest.approx(2 * us)
    assert summary["decode_span_us"] == pytest.approx((2 + 3 + 150 + 3) * us)
    assert summary["gap_decode_end_to_merge_start_us"] == pytest.approx(50 * us)
    assert summary["merge_entry_to_combined_us"] == pytest.approx(20 * us)
    assert summary["merge_span_us"] == pytest.approx(25 * us)
    assert summary["layer_first_entry_to_last_store_us"] == pytest.approx((158 + 50 + 25) * us)
    # next layer's first entry (t + 10_000) minus this layer's last merge store
    assert summary["gap_merge_end_to_next_decode_start_us"] == pytest.approx((10_000 - 233) * us)
    x = summary["decode_by_xcd"]
    assert set(x) == {"0", "1"}
    assert x["0"]["waves"] == 4 and x["1"]["waves"] == 4
    assert x["0"]["stream_us_median"] == pytest.approx(100 * us)
    assert x["1"]["stream_us_median"] == pytest.approx(150 * us)
    # XCC 1's waves: wave 0 ends at its store (+2 +3 +150 +3), wave 1 at its join (+2 +3 +150 +1)
    assert x["1"]["last_end_us_median"] == pytest.approx(158 * us)
    assert x["0"]["last_end_us_median"] == pytest.approx((3 + 100 + 3) * us)
    assert "| 1 | 4 |" in md


def test_summary_without_merge_launches(bench):
    recs = [_decode(0, 0, 0, 3, 500, 40), _decode(0, 0, 1, 3, 501, 60), _decode(1, 0, 0, 3, 900, 40),
            _decode(1, 0, 1, 3, 901, 60)]
    summary, _ = bench.summarize_wave_clock(np.stack(recs))
    assert summary["merge_span_us"] is None and summary["gap_decode_end_to_merge_start_us"] is None
    # one-launch steps: the gap runs from the decode's last end to the next decode's first entry
    last_end = max(500 + 3 + 40 + 3, 501 + 3 + 60 + 1)
    assert summary["gap_merge_end_to_next_decode_start_us"] == pytest.approx((900 - last_end) * 0.01)
