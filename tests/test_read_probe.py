"""The streaming-read probe bench.py --probe times beside the decode (pop2-bezier_amd/csrc/ppk_read_probe.hip).

It is a measurement tool, not part of the decode library: these tests pin that it reads exactly the ranges it is
given (every lane's checksum equals the xor of the 16-byte words that lane is meant to load, at every ring depth,
at arena-like strides) and that it refuses arguments out of range before launching anything.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "pop2-bezier_amd", "ppk", "libppk_probe.so")


def _lib():
    # torch first, as in bench.py: the probe library and torch share one HIP runtime by soname, and the one
    # loaded first is the one every later library binds to (torch's own, which it was built against).
    import torch  # noqa: F401

    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(LIB)
    lib.ppk_read_probe.restype = ctypes.c_int
    lib.ppk_read_probe.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
                                   ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                   ctypes.c_uint64, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_void_p]
    return lib


def test_probe_refuses_arguments_out_of_range():
    lib = _lib()
    buf = ctypes.create_string_buffer(64)
    p = ctypes.cast(buf, ctypes.c_void_p)
    ok = dict(k=p, v=p, tiles=8, waves=8, wpb=2, bpc=2, ring=3, wpr=2, row_stride=2 * 8 * 64 + 16,
              wave_stride=8 * 64, out=p)

    def call(**kw):
        a = dict(ok, **kw)
        return lib.ppk_read_probe(a["k"], a["v"], a["tiles"], a["waves"], a["wpb"], a["bpc"], a["ring"], a["wpr"],
                                  a["row_stride"], a["wave_stride"], a["out"], None)

    # Each of these is refused by the host checks, before any HIP call.
    assert call(k=None) == -1
    assert call(tiles=0) == -1
    assert call(tiles=6) == -1             # not a whole number of 4-tile batches
    assert call(waves=7) == -1             # not whole blocks
    assert call(wpb=9) == -1
    assert call(bpc=1) == -1               # one block per CU would need more than 64 KiB of LDS
    assert call(ring=5) == -1
    assert call(wpr=3) == -1               # not whole rows
    assert call(wave_stride=8 * 64 - 1) == -1   # ranges of one row would overlap
    assert call(row_stride=8 * 64) == -1        # rows would overlap


def _expected(k: np.ndarray, v: np.ndarray, waves: int, wpr: int, row_stride: int, wave_stride: int,
              tiles: int) -> np.ndarray:
    """Per (wave, lane): xor of the four dwords of every 16-byte word the lane loads from both ranges."""
    k4 = k.view(np.uint32).reshape(-1, 4)
    v4 = v.view(np.uint32).reshape(-1, 4)
    out = np.zeros((waves, 64), dtype=np.uint32)
    lanes = np.arange(64)
    for w in range(waves):
        base = (w // wpr) * row_stride + (w % wpr) * wave_stride
        idx = base + np.arange(tiles)[:, None] * 64 + lanes[None, :]  # [tiles, 64]
        words = np.concatenate([k4[idx], v4[idx]], axis=0)             # [2 tiles, 64, 4]
        out[w] = np.bitwise_xor.reduce(np.bitwise_xor.reduce(words, axis=2), axis=0)
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("ring", [2, 3, 4, 6])
def test_probe_reads_exactly_its_ranges(device, ring):
    import torch

    from ppk.int8_kv_ops import current_stream_handle

    lib = _lib()
    rows, wpr, split, D = 6, 2, 64, 128
    cap = wpr * split + 1                     # odd capacity: rows start off the 1 KiB grid, as in the arenas
    tiles = split * D // 1024
    waves = rows * wpr
    g = torch.Generator().manual_seed(11)
    kc = torch.randint(0, 256, (rows, cap, D), dtype=torch.uint8, generator=g)
    vc = torch.randint(0, 256, (rows, cap, D), dtype=torch.uint8, generator=g)
    kd, vd = kc.to(device), vc.to(device)
    out = torch.full((waves * 64,), -1, dtype=torch.int32, device=device)
    row_stride, wave_stride = cap * D // 16, split * D // 16
    print(f"probe ring={ring} rows={rows} wpr={wpr} split={split} D={D}", flush=True)
    rc = lib.ppk_read_probe(kd.data_ptr(), vd.data_ptr(), tiles, waves, wpr, 2, ring, wpr, row_stride, wave_stride,
                            out.data_ptr(), current_stream_handle(device))
    assert rc == 0
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint32).reshape(waves, 64)
    want = _expected(kc.numpy().reshape(-1), vc.numpy().reshape(-1), waves, wpr, row_stride, wave_stride, tiles)
    np.testing.assert_array_equal(got, want)
