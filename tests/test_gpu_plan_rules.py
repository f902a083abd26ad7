"""Parity of the per-row plan's sizing rules against the f64 oracle, one seeded ragged batch per rule.

The plan (ppk_attention_plan_info) decides how a row's waves are cut into blocks; these shapes land in each
rule: few long rows cut into blocks that cover the CUs (larger where they land evenly, smaller where the
chosen ones do not), rows beyond the CU count spread over small blocks or given a power-of-two wave count, and
two-round grids turned into one block per row. Lengths are ragged within the span (some rows empty or one
token) so every rule also runs with waves past a row's end. Bar as the other attention tests: max abs
<= 2e-3, max rel <= 1e-2.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import ppk
from helpers import SEED, assert_close
from test_gpu_attention import Case

pytestmark = pytest.mark.gpu

# (sequences B of 16 heads, head_dim, span, expected (tokens per wave, blocks per row, waves per block))
CASES = [
    (17, 64, 1800, (272, 7, 1)),   # 272 rows: seven 1-wave blocks a row (two-round grid avoided)
    (25, 128, 3000, (600, 5, 1)),  # 400 rows: five 1-wave blocks a row
    (41, 64, 900, (464, 1, 2)),    # 656 rows: two waves in one block a row
    (5, 128, 1024, (64, 16, 1)),   # 80 rows: sixteen 1-wave blocks, five a CU (the even split)
    (3, 64, 4096, (128, 16, 2)),   # 48 rows: 2-wave blocks, three a CU
    (8, 128, 4000, (256, 2, 8)),   # 128 rows: two 8-wave blocks a row, one a CU
    (11, 64, 3000, (384, 1, 8)),   # 176 rows: one 8-wave block a row (two-round grid avoided)
]


@pytest.mark.parametrize("B,D,span,want", CASES, ids=[f"rows{16 * c[0]}-d{c[1]}-span{c[2]}" for c in CASES])
def test_plan_rule_parity(device, B, D, span, want):
    rng = np.random.default_rng(SEED + 51 + B)
    lengths = [int(x) for x in rng.integers(span // 3, span + 1, size=B)]
    lengths[0] = span
    if B > 2:
        lengths[1], lengths[2] = 0, 1
    c = Case(device, B, 16, D, lengths, span + 1, q_dtype=torch.bfloat16, scratch_dtype=torch.bfloat16,
             seed=SEED + 61 + B)
    a, _ = ppk.int8_kv_ops.attention_args(c.q, c.kc, c.vc, c.ks, c.vs, c.sk, c.sv, c.past_t, c.H, max_past=span)
    info = ppk.int8_kv_ops.plan_info(a, ppk.context(device))
    assert (info["split_tokens"], info["nsplits"], info["waves_per_block"]) == want
    assert info["blocks"] <= 256 * (8 // info["waves_per_block"]), "one round of resident blocks"
    print(f"plan rows={c.rows} D={D} span={span}: {info}", flush=True)
    assert_close(c.run(max_past=span), c.reference(), what=f"{c.rows} rows x {span} at D = {D}")
