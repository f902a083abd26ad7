"""GPU parity of the per-row plan sized from the host lengths: with past_host / lengths_host (and no plan bit)
the per-row plan covers the longest live host length instead of the whole span (max_past / max_length, or the
capacity), so a caller that passes only the arena's capacity gets the plan of its actual lengths.

A device length the plan still covers gives its exact rows whatever the host copy said; one beyond the
coverage (a stale host copy) gives NaN rows and PPK_FLAG_STALE_LENGTHS in a decode step's flags. Bars as the
per-row tests: int8 max abs <= 2e-3 and max rel <= 1e-2 against the f64 oracle, float max abs <= 1e-4 and
max rel <= 1e-2.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import ppk
from helpers import SEED, assert_close
from test_gpu_attention import Case
from test_gpu_float_attention import ATOL as F_ATOL, RTOL as F_RTOL, FloatCase
from test_gpu_float_step import StepCase

pytestmark = pytest.mark.gpu

# Near-uniform lengths (no balanced plan) far below the arena's 4096 slots.
HOST = [1000, 950, 980]


def _int8_plan(c: Case, host, **kw):
    """(split, groups, waves per block, blocks, launches): two spans can share split and groups and differ
    only in how many waves each block holds."""
    a, _ = ppk.int8_kv_ops.attention_args(c.q, c.kc, c.vc, c.ks, c.vs, c.sk, c.sv, c.past_t, c.H, past_host=host,
                                          **kw)
    i = ppk.int8_kv_ops.plan_info(a, ppk.context(c.q.device))
    return i["split_tokens"], i["nsplits"], i["waves_per_block"], i["blocks"], i["launches"]


@pytest.mark.parametrize("d", [64, 128])
def test_int8_per_row_plan_covers_the_longest_host_length(device, d):
    c = Case(device, 3, 8, d, HOST, 4096, q_dtype=torch.bfloat16, scratch_dtype=torch.bfloat16, seed=SEED + d)
    sized = _int8_plan(c, HOST)
    assert sized == _int8_plan(c, None, max_past=max(HOST)) != _int8_plan(c, None)
    assert _int8_plan(c, HOST, plan="per-row") == _int8_plan(c, None)
    ref = c.reference()
    assert_close(c.run(past_host=HOST), ref, what=f"host-sized per-row d={d}")
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    out = ppk.decode_step(c.q, c.kc, c.vc, c.ks, c.vs, c.sk, c.sv, c.past_t, c.H, flags=flags, past_host=HOST)
    torch.cuda.synchronize()
    assert int(flags.item()) == 0
    assert_close(out.reshape(c.rows, d).cpu().numpy(), ref, what=f"host-sized per-row step d={d}")


def test_int8_stale_host_lengths_beyond_the_coverage(device):
    """Device lengths 1000 / 1500 / 500 against host 1000 / 950 / 980: sequence 1 lies past the plan's
    coverage (NaN, flagged), sequence 2 is shorter than its host copy and still exact."""
    device_lengths = [1000, 1500, 500]
    c = Case(device, 3, 8, 128, device_lengths, 4096, q_dtype=torch.bfloat16, scratch_dtype=torch.bfloat16,
             seed=SEED + 3)
    ref = c.reference()
    bad = np.repeat(np.array([False, True, False]), c.H)
    got = c.run(past_host=HOST)
    assert np.isnan(got[bad]).all()
    assert_close(got[~bad], ref[~bad], what="rows the plan covers")
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    out = ppk.decode_step(c.q, c.kc, c.vc, c.ks, c.vs, c.sk, c.sv, c.past_t, c.H, flags=flags, past_host=HOST)
    torch.cuda.synchronize()
    step = out.reshape(c.rows, c.D).cpu().numpy()
    assert int(flags.item()) == ppk.PPK_FLAG_STALE_LENGTHS
    assert np.isnan(step[bad]).all()
    assert_close(step[~bad], ref[~bad], what="step rows the plan covers")


def _float_plan(c: FloatCase, host, **kw):
    a, _ = ppk.fused_attention.decode_attention_args(c.q, c.k, c.v, c.lengths_t, c.H, lengths_host=host, **kw)
    return ppk.fused_attention.plan(a, ppk.context(c.q.device))


@pytest.mark.parametrize("kv", [torch.bfloat16, torch.float32])
def test_float_per_row_plan_covers_the_longest_host_length(device, kv):
    c = FloatCase(device, 3, 8, 128, 4096, kv, lengths=HOST, seed=SEED + 4)
    # The plan of the same call with max_length = the longest host length (the (split, blocks, workspace)
    # triple need not differ from the capacity's plan: the waves per block may be what changes).
    assert _float_plan(c, HOST) == _float_plan(c, None, max_length=max(HOST))
    assert_close(c.run(lengths_host=HOST), c.reference(), atol=F_ATOL, rtol=F_RTOL, what=f"host-sized {kv}")


@pytest.mark.parametrize("kv", [torch.bfloat16, torch.float32])
def test_float_step_stale_host_lengths_beyond_the_coverage(device, kv):
    """The fused float step with stored lengths 999 / 1500 / 400 against host 999 / 949 / 979."""
    host = [n - 1 for n in HOST]
    c = StepCase(device, 3, 8, 128, 4096, kv, [999, 1500, 400], seed=SEED + 5)
    got, flags = c.step(lengths_host=host)
    bad = np.repeat(np.array([False, True, False]), c.H)
    ref = c.expected()
    assert flags == ppk.PPK_FLAG_STALE_LENGTHS
    assert np.isnan(got[bad]).all()
    assert_close(got[~bad], ref[~bad], atol=F_ATOL, rtol=F_RTOL, what=f"float step rows the plan covers {kv}")
    c.check_store()  # every row's token is written, stale or not
    c2 = StepCase(device, 3, 8, 128, 4096, kv, host, seed=SEED + 6)
    got2, flags2 = c2.step(lengths_host=host)
    assert flags2 == 0
    assert_close(got2, c2.expected(), atol=F_ATOL, rtol=F_RTOL, what=f"float step host-sized {kv}")


def test_prepared_int8_call_follows_new_host_lengths(device):
    """A prepared balanced call built with one host copy of past[] and run after the device lengths moved:
    the stale sequences give NaN; set_past_host() with the new copy re-plans and every row is exact."""
    old = [1000, 300, 300, 900, 120, 700, 40, 1000]
    new = [1000, 301, 305, 950, 121, 700, 41, 999]
    c = Case(device, 8, 4, 128, new, 1001, q_dtype=torch.bfloat16, scratch_dtype=torch.bfloat16, seed=SEED + 7)
    call = ppk.DecodeAttention(c.q, c.kc, c.vc, c.ks, c.vs, c.sk, c.sv, c.past_t, c.H, past_host=old,
                               plan="balanced")
    got = call().float().reshape(c.rows, c.D).cpu().numpy()
    bad = np.repeat(np.array(old) != np.array(new), c.H)
    ref = c.reference()
    assert np.isnan(got[bad]).all()
    assert_close(got[~bad], ref[~bad], what="prepared call, unchanged sequences")
    call.set_past_host(new)
    got = call().float().reshape(c.rows, c.D).cpu().numpy()
    assert_close(got, ref, what="prepared call after set_past_host")


@pytest.mark.parametrize("kv", [torch.bfloat16, torch.float32])
def test_prepared_float_call_follows_new_host_lengths(device, kv):
    old = [1000, 300, 300, 900, 120, 700, 40, 1000]
    new = [1000, 301, 305, 950, 121, 700, 41, 999]
    c = FloatCase(device, 8, 4, 128, 1024, kv, lengths=new, seed=SEED + 8)
    call = ppk.fused_attention.FloatDecodeAttention(c.q, c.k, c.v, c.lengths_t, c.H, lengths_host=old,
                                                    plan="balanced")
    got = call().float().reshape(c.rows, c.D).cpu().numpy()
    bad = np.repeat(np.array(old) != np.array(new), c.H)
    ref = c.reference()
    assert np.isnan(got[bad]).all()
    assert_close(got[~bad], ref[~bad], atol=F_ATOL, rtol=F_RTOL, what=f"prepared float call, unchanged {kv}")
    call.set_lengths_host(new)
    got = call().float().reshape(c.rows, c.D).cpu().numpy()
    assert_close(got, ref, atol=F_ATOL, rtol=F_RTOL, what=f"prepared float call after set_lengths_host {kv}")
