"""The wave-clock diagnostics build (ppk_kernels_clock.hsaco, ppk_context_set_wave_clock).

The same kernels built with per-wave real-time clock points must compute bit-identical outputs, write one
record per wave (and per merge row) with ordered clock points, and never write past the record capacity the
host derived from the buffer's size, whatever the buffer's own capacity word says.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest
import torch

import ppk
from ppk import _abi

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLOCK_HSACO = os.path.join(ROOT, "pop2-bezier_amd", "ppk", "ppk_kernels_clock.hsaco")
WORDS = 16  # u64 words per record (kWaveClockWords)


def _problem(device, B, H, D, lengths, cap, seed):
    g = torch.Generator(device=device).manual_seed(seed)
    rows = B * H
    kc = torch.zeros((rows, cap, D), dtype=torch.uint8, device=device)
    vc = torch.zeros_like(kc)
    ks = torch.zeros((rows, cap), dtype=torch.float32, device=device)
    vs = torch.zeros_like(ks)
    lmax = max(lengths)
    c, s = ppk.quantize(torch.randn((rows, lmax, D), generator=g, device=device))
    kc[:, :lmax], ks[:, :lmax] = c, s
    c, s = ppk.quantize(torch.randn((rows, lmax, D), generator=g, device=device))
    vc[:, :lmax], vs[:, :lmax] = c, s
    q = torch.randn((rows, 1, D), generator=g, device=device).to(torch.bfloat16)
    sk = torch.randn((rows, 1, D), generator=g, device=device).to(torch.bfloat16)
    sv = torch.randn((rows, 1, D), generator=g, device=device).to(torch.bfloat16)
    past = torch.tensor(lengths, dtype=torch.int32, device=device)
    return q, kc, vc, ks, vs, sk, sv, past


def _clock_context(device):
    lib = _abi.lib()
    ctx = ctypes.c_void_p()
    _abi.check(lib.ppk_context_create(device.index or 0, CLOCK_HSACO.encode(), ctypes.byref(ctx)),
               "ppk_context_create")
    return lib, ctx


@pytest.mark.parametrize("split", [0, 64, 256])
def test_clock_build_same_output_ordered_records(device, split):
    B, H, D, cap = 2, 8, 128, 700
    lengths = [600, 431]
    print(f"wave clock split={split} B={B} H={H} D={D} lengths={lengths}", flush=True)
    call = ppk.DecodeAttention(*_problem(device, B, H, D, lengths, cap, 5), H, split_tokens=split)
    info = call.plan_info
    want = call().clone()
    torch.cuda.synchronize()
    lib, ctx = _clock_context(device)
    rows = B * H
    per = max(info["blocks"] * info["waves_per_block"], rows)
    nrec = 2 * per
    buf = torch.zeros(WORDS * (nrec + 1), dtype=torch.int64, device=device)
    buf[0], buf[1] = per, nrec
    prod = call.ctx
    try:
        _abi.check(lib.ppk_context_set_wave_clock(ctx, ctypes.c_void_p(buf.data_ptr()), buf.numel() * 8),
                   "ppk_context_set_wave_clock")
        call.ctx = ctx
        got = call().clone()
        torch.cuda.synchronize()
        _abi.check(lib.ppk_context_set_wave_clock(ctx, None, 0), "ppk_context_set_wave_clock")
    finally:
        call.ctx = prod
        torch.cuda.synchronize()
        lib.ppk_context_release(ctx)
    assert torch.equal(got, want), "the clock build must compute the same bits"
    rec = buf[WORDS:].view(-1, WORDS).cpu().numpy().view(np.uint64)
    rec = rec[rec[:, 0] != 0]
    kind = (rec[:, 0] >> np.uint64(56)).astype(int)
    seq = ((rec[:, 0] >> np.uint64(32)) & np.uint64(0xFFFFFF)).astype(int)
    assert set(seq.tolist()) == {0}
    n_decode = int((kind == 1).sum())
    n_merge = int((kind == 2).sum())
    assert n_decode == info["blocks"] * info["waves_per_block"]
    assert n_merge == (rows if info["launches"] == 2 else 0)
    t = rec[:, 2:10].astype(np.int64)
    d = t[kind == 1]
    wave = (rec[kind == 1, 0] & np.uint64(0xFF)).astype(int)
    # entry <= loads issued <= past here <= stream done <= block joined; wave 0 stores after joining
    for a, b in ((0, 1), (1, 2), (2, 4), (4, 5)):
        assert (d[:, a] <= d[:, b]).all(), (a, b)
    assert (d[wave == 0, 5] <= d[wave == 0, 6]).all()
    streamed = d[:, 3] != 0  # waves with history saw their first K data between issue and the stream's end
    assert (d[streamed, 1] <= d[streamed, 3]).all() and (d[streamed, 3] <= d[streamed, 4]).all()
    if n_merge:
        m = t[kind == 2]
        assert (m[:, 0] <= m[:, 1]).all() and (m[:, 1] <= m[:, 2]).all()
        assert m[:, 0].min() >= d[:, 0].min()


def test_clock_records_stop_at_the_buffer_size(device):
    """The capacity word of the buffer claims far more records than the buffer holds: only the records that
    fit the size given to ppk_context_set_wave_clock are written, and the memory after them stays untouched."""
    B, H, D, cap = 2, 8, 64, 300
    call = ppk.DecodeAttention(*_problem(device, B, H, D, [250, 250], cap, 9), H)
    lib, ctx = _clock_context(device)
    fit, guard = 3, 64
    buf = torch.zeros(WORDS * (1 + fit + guard), dtype=torch.int64, device=device)
    per = max(call.plan_info["blocks"] * call.plan_info["waves_per_block"], B * H)
    assert per > fit
    buf[0], buf[1] = per, 1 << 40
    prod = call.ctx
    try:
        _abi.check(lib.ppk_context_set_wave_clock(ctx, ctypes.c_void_p(buf.data_ptr()), WORDS * (1 + fit) * 8),
                   "ppk_context_set_wave_clock")
        call.ctx = ctx
        call()
        torch.cuda.synchronize()
        _abi.check(lib.ppk_context_set_wave_clock(ctx, None, 0), "ppk_context_set_wave_clock")
    finally:
        call.ctx = prod
        torch.cuda.synchronize()
        lib.ppk_context_release(ctx)
    rec = buf.view(-1, WORDS).cpu().numpy()
    assert (rec[1:1 + fit, 0] != 0).all()
    assert (rec[1 + fit:] == 0).all()


def test_set_wave_clock_refuses_a_buffer_without_room_for_a_record(device):
    lib, ctx = _clock_context(device)
    try:
        buf = torch.zeros(WORDS * 2, dtype=torch.int64, device=device)
        assert lib.ppk_context_set_wave_clock(ctx, ctypes.c_void_p(buf.data_ptr()), WORDS * 8 * 2 - 8) == 1
        assert lib.ppk_context_set_wave_clock(ctx, ctypes.c_void_p(buf.data_ptr() + 8), WORDS * 8 * 2) == 1
        assert lib.ppk_context_set_wave_clock(ctx, ctypes.c_void_p(buf.data_ptr()), WORDS * 8 * 2) == 0
        assert lib.ppk_context_set_wave_clock(ctx, None, 0) == 0
    finally:
        lib.ppk_context_release(ctx)
