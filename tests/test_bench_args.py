"""bench.py's --lengths syntax (host logic only): lists, NxL repeats and seeded uniform draws."""
from __future__ import annotations

import importlib.util
import os

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_args_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_lists_and_repeats(bench):
    assert bench.parse_lengths("7,2x300, 5") == [7, 300, 300, 5]
    assert bench.parse_lengths("3x4096,1x1") == [4096, 4096, 4096, 1]


def test_uniform_draw_is_numpys_seeded_integers(bench):
    got = bench.parse_lengths("uniform:6:256:4096:107")
    assert got == [int(x) for x in np.random.default_rng(107).integers(256, 4097, size=6)]
    assert len(got) == 6 and all(256 <= x <= 4096 for x in got)
    # config 4's own draw, default_rng(SEED).integers(256, 4097, 8)
    assert bench.parse_lengths(f"uniform:8:256:4096:{bench.SEED}") == [2850, 1888, 2139, 344, 2921, 1487, 1740, 3043]
