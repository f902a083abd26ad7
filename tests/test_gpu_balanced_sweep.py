"""Seeded sweep of the balanced-plan kernels over small shapes, forced with PPK_ATTN_PLAN_BALANCED (the
library's own choice takes them only for large ragged batches): int8 attention and decode step
(ppk_decode_flat*, ppk_attn_merge_flat*) and float-KV attention (ppk_fdecode_flat_*, ppk_fmerge_flat_*)
against the f64 oracle, with empty, one-token, full, beyond-capacity and beyond-max rows mixed in.

Bars as the per-row tests: int8 max abs <= 2e-3 and max rel <= 1e-2 (|oracle| >= 1e-3), the bf16-history
mode within 2e-5 absolute (on N(0, 1) history, as the reference's own check); float max abs <= 1e-4 and max
rel <= 1e-2; appended codes and scales bit-exact.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import ppk
from helpers import SEED, assert_close
from test_gpu_attention import Case
from test_gpu_float_attention import ATOL as F_ATOL, RTOL as F_RTOL, FloatCase

pytestmark = pytest.mark.gpu


def _lengths(rng, batch: int, cap: int) -> list[int]:
    """Ragged lengths with the edge values mixed in: 0, 1, cap, cap + 1 (invalid) and random ones."""
    pool = [0, 1, cap, cap + 1, int(rng.integers(2, 64)), int(rng.integers(1, cap + 1))]
    return [int(pool[rng.integers(len(pool))]) if rng.random() < 0.4 else int(rng.integers(0, cap + 1))
            for _ in range(batch)]


@pytest.mark.parametrize("case", range(24))
def test_int8_balanced_sweep(device, case):
    rng = np.random.default_rng(SEED + 1000 + case)
    D = int(rng.choice([64, 128, 256]))
    H = int(rng.choice([1, 2, 4, 8]))
    B = int(rng.integers(1, 13))
    cap = int(rng.integers(32, 1500))
    lengths = _lengths(rng, B, cap)
    dt = [torch.float32, torch.bfloat16, torch.float16][int(rng.integers(3))]
    bf16h = bool(rng.random() < 0.3)
    max_past = 0 if rng.random() < 0.5 else int(rng.integers(1, cap + 1))
    # The bf16-history bar (the reference's 2e-5 absolute, set on its smooth known-answer data) is checked on
    # N(0, 1) history; with the heavy-tailed channels (values in the hundreds) fp32 summation alone exceeds it.
    c = Case(device, B, H, D, lengths, cap, q_dtype=dt, scratch_dtype=dt, seed=SEED + 2000 + case, heavy=not bf16h)
    print(f"case {case}: B={B} H={H} D={D} cap={cap} lengths={lengths} max_past={max_past} {dt} bf16h={bf16h}",
          flush=True)
    ref = c.reference(history_bf16=bf16h)
    span = max_past or cap
    beyond = np.repeat(np.array(lengths) > span, H)
    ref[beyond] = np.nan  # rows past max_past give NaN (past the capacity the oracle gives it already)
    atol, rtol = (2e-5, 0) if bf16h else (2e-3, 1e-2)
    got = c.run(past_host=lengths, max_past=max_past, bf16_history=bf16h, plan="balanced")
    assert_close(got, ref, atol=atol, rtol=rtol, what=f"int8 balanced case {case}")
    if case % 3 == 0:
        # The fused step through the same plan: append at slot past[b], then attend.
        flags = torch.zeros(1, dtype=torch.int32, device=device)
        out = ppk.decode_step(c.q, c.kc, c.vc, c.ks, c.vs, c.sk, c.sv, c.past_t, H, flags=flags, past_host=lengths,
                              max_past=max_past, bf16_history=bf16h, plan="balanced")
        torch.cuda.synchronize()
        assert_close(out.float().reshape(c.rows, D).cpu().numpy(), ref, atol=atol, rtol=rtol,
                     what=f"int8 balanced step case {case}")
        codes, scales, _ = oracle.quantize(c.sk32.reshape(c.rows, 1, D))
        kc, ks = c.kc.cpu().numpy(), c.ks.cpu().numpy()
        for b, p in enumerate(lengths):
            if p < cap:
                rows = slice(b * H, (b + 1) * H)
                assert np.array_equal(kc[rows, p], codes[rows, 0])
                assert np.array_equal(ks[rows, p].view(np.uint32), scales[rows, 0].view(np.uint32))


def test_int8_balanced_all_rows_one_unit_is_one_launch(device):
    """Every row within one unit: the decode launch writes every output, no records and no merge launch."""
    lengths = [10, 0, 60, 64]
    c = Case(device, 4, 16, 64, lengths, 1024)
    a, _ = ppk.int8_kv_ops.attention_args(c.q, c.kc, c.vc, c.ks, c.vs, c.sk, c.sv, c.past_t, c.H, max_past=900,
                                          past_host=lengths, plan="balanced")
    assert ppk.int8_kv_ops.plan(a, ppk.context(device)) == (64, 1, 0)
    ppk.kernel_stats(ppk.PPK_KERNEL_ATTN_MERGE, reset=True)
    ppk.set_profiling(True)
    got = c.run(past_host=lengths, max_past=900, plan="balanced")
    ppk.set_profiling(False)
    assert ppk.kernel_stats(ppk.PPK_KERNEL_ATTN_MERGE, reset=True)[0] == 0
    assert_close(got, c.reference(), what="one-unit rows")


@pytest.mark.parametrize("case", range(18))
def test_float_balanced_sweep(device, case):
    rng = np.random.default_rng(SEED + 3000 + case)
    D = int(rng.choice([64, 128, 256]))
    H = int(rng.choice([1, 2, 4, 8]))
    B = int(rng.integers(1, 13))
    size = int(rng.integers(16, 1200))
    kv = [torch.bfloat16, torch.float32][int(rng.integers(2))]
    lengths = _lengths(rng, B, size)
    max_length = 0 if rng.random() < 0.5 else int(rng.integers(1, size + 1))
    c = FloatCase(device, B, H, D, size, kv, lengths=lengths, seed=SEED + 4000 + case)
    print(f"case {case}: B={B} H={H} D={D} size={size} lengths={lengths} max_length={max_length} {kv}", flush=True)
    ref = c.reference()
    beyond = np.repeat(np.array(lengths) > (max_length or size), H)
    ref[beyond] = np.nan
    got = c.run(lengths_host=lengths, max_length=max_length, plan="balanced")
    assert_close(got, ref, atol=F_ATOL, rtol=F_RTOL, what=f"float balanced case {case}")


def test_float_balanced_all_rows_one_unit_is_one_launch(device):
    lengths = [10, 0, 60, 64]
    c = FloatCase(device, 4, 16, 64, 1024, torch.bfloat16, lengths=lengths, seed=SEED + 5000)
    a, _ = ppk.fused_attention.decode_attention_args(c.q, c.k, c.v, c.lengths_t, c.H, lengths_host=lengths,
                                                     plan="balanced")
    assert ppk.fused_attention.plan(a, ppk.context(device)) == (64, 1, 0)
    ppk.kernel_stats(ppk.PPK_KERNEL_FLOAT_MERGE, reset=True)
    ppk.set_profiling(True)
    got = c.run(lengths_host=lengths, plan="balanced")
    ppk.set_profiling(False)
    assert ppk.kernel_stats(ppk.PPK_KERNEL_FLOAT_MERGE, reset=True)[0] == 0
    assert_close(got, c.reference(), atol=F_ATOL, rtol=F_RTOL, what="float one-unit rows")


@pytest.mark.parametrize("d", [64, 128, 256])
def test_forced_per_row_ignores_host_lengths_for_planning(device, d):
    """PPK_ATTN_PLAN_PER_ROW with the host lengths of a batch the library would balance: the per-row plan's
    outputs, bit for bit. With the host lengths most of the per-row waves are known to hold no history, so the
    kernel does not request their first K batches before past[] arrives; without them it does: both paths
    give the same bits, for attention and for the fused step (same appended codes and scales)."""
    lengths = [1500, 333, 2900]
    c = Case(device, 3, 8, d, lengths, 3000)
    np.testing.assert_array_equal(c.run(past_host=lengths, plan="per-row"), c.run())
    outs, arenas = [], []
    for host in (lengths, None):
        kc, vc, ks, vs = (t.clone() for t in (c.kc, c.vc, c.ks, c.vs))
        out = ppk.decode_step(c.q, kc, vc, ks, vs, c.sk, c.sv, c.past_t, c.H, past_host=host, plan="per-row")
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
        arenas.append([t.cpu().numpy() for t in (kc, vc, ks, vs)])
    np.testing.assert_array_equal(outs[0], outs[1])
    for x, y in zip(*arenas):
        np.testing.assert_array_equal(x.view(np.uint8), y.view(np.uint8))
