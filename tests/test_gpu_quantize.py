"""GPU parity of kernel 1 (quantize / quantize-and-append) and dequantize.

Codes and scales must be bit-exact with the oracle (oracle/ppk_oracle.c,
restating app/src/model/int8_kv_ops.rs:11-21). Everything runs through the
C-ABI (libppk.so) via the ppk package.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import ppk
from helpers import SEED, bf16_bits_to_f32, kv_values, to_bf16_bits

pytestmark = pytest.mark.gpu

DTYPES = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def _to_device(x32: np.ndarray, dtype: torch.dtype, device) -> tuple[torch.Tensor, np.ndarray]:
    """Device tensor of dtype plus the exact float32 values it holds (the oracle's input)."""
    if dtype == torch.float32:
        return torch.from_numpy(np.ascontiguousarray(x32)).to(device), x32
    if dtype == torch.float16:
        # Special rows hold values past f16's range: they become ±inf, a
        # non-finite f16 input, which the oracle sees as well.
        with np.errstate(over="ignore"):
            h = x32.astype(np.float16)
        return torch.from_numpy(h).to(device), h.astype(np.float32)
    bits = to_bf16_bits(x32)
    t = torch.from_numpy(bits.view(np.int16)).to(device).view(torch.bfloat16)
    return t, bf16_bits_to_f32(bits)


def test_prepare_known_answer_checks(device):
    """int8_kv_ops::prepare's three checks (int8_kv_ops.rs:56-103), run on the device."""
    ppk.prepare(device)


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_quantize_bit_exact(device, d, dt):
    rng = np.random.default_rng(SEED + d)
    x = kv_values(rng, 1, 16, 257, d).reshape(16, 257, d)
    xt, x32 = _to_device(x, DTYPES[dt], device)
    codes, scales = ppk.quantize(xt)
    ref_codes, ref_scales, _ = oracle.quantize(x32)
    assert np.array_equal(codes.cpu().numpy(), ref_codes)
    assert np.array_equal(scales.cpu().numpy().view(np.uint32), ref_scales.view(np.uint32))


def _special_rows(d: int) -> np.ndarray:
    rows = []
    rows.append(np.zeros(d, np.float32))                                       # zero row -> scale 1e-12
    r = np.zeros(d, np.float32); r[:5] = [0.5, 1.5, 2.5, -2.5, 127.0]; rows.append(r)   # ties at scale 1
    r = np.full(d, -3.0, np.float32); r[7] = -11.0; rows.append(r)              # all negative
    rows.append(np.full(d, 1e-40, np.float32))                                  # subnormal inputs
    r = np.zeros(d, np.float32); r[3] = 3e38; r[4] = -1e38; rows.append(r)     # near-max magnitudes
    r = np.zeros(d, np.float32); r[0] = 1e-10; rows.append(r)                   # absmax/127 below the floor
    r = np.arange(d, dtype=np.float32) - d / 2; rows.append(r)                  # ramp
    r = np.linspace(-254.0, 254.0, d, dtype=np.float32); rows.append(r)        # many exact half-steps
    return np.stack(rows)[None]


@pytest.mark.parametrize("d", [64, 128, 256])
def test_quantize_special_rows(device, d):
    x = _special_rows(d)
    codes, scales = ppk.quantize(torch.from_numpy(x).to(device))
    ref_codes, ref_scales, _ = oracle.quantize(x)
    assert np.array_equal(codes.cpu().numpy(), ref_codes)
    assert np.array_equal(scales.cpu().numpy().view(np.uint32), ref_scales.view(np.uint32))
    assert scales[0, 0].item() == np.float32(1e-12)
    assert scales[0, 1].item() == 1.0


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_quantize_streaming_kernel_special_rows(device, d, dt):
    """The special rows, tiled past the size where ppk_quantize takes the streaming kernel (one block of
    work per CU), bit-exact against the oracle; random rows in between, so rows of every kind share waves."""
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    per_lane = 4 if dt == "f32" else 8
    need_rows = cus * 1024 * per_lane // d + 64
    special = _special_rows(d)[0]
    rng = np.random.default_rng(SEED + 61 + d)
    filler = kv_values(rng, 1, 1, need_rows, d).reshape(need_rows, d)
    x = filler.copy()
    x[::3] = np.resize(special, (len(x[::3]), d))
    xt, x32 = _to_device(x[None], DTYPES[dt], device)
    codes, scales = ppk.quantize(xt)
    ref_codes, ref_scales, _ = oracle.quantize(x32)
    assert np.array_equal(codes.cpu().numpy(), ref_codes)
    assert np.array_equal(scales.cpu().numpy().view(np.uint32), ref_scales.view(np.uint32))


def test_streaming_quantize_quotients_next_to_half_integers(device):
    """f32 rows whose quotients x / s lie within 0-3 ulps of a half-integer on either side (and exactly on
    one), at the streaming kernel's size: the codes decided near a tie equal the oracle's bit for bit."""
    d = 128
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    rows = cus * 1024 * 4 // d + 64
    rng = np.random.default_rng(SEED + 81)
    amax = (np.float32(127.0) * np.float32(2.0) ** rng.integers(-20, 20, rows).astype(np.float32)
            * (1 + rng.random(rows, dtype=np.float32))).astype(np.float32)
    s = np.maximum(amax / np.float32(127.0), np.float32(1e-12)).astype(np.float32)
    half = rng.integers(-127, 127, (rows, d)).astype(np.float32) + np.float32(0.5)
    x = (half * s[:, None]).astype(np.float32)
    steps = rng.integers(-3, 4, (rows, d))
    toward = np.where(steps > 0, np.float32(np.inf), np.float32(-np.inf))
    for k in range(1, 4):
        x = np.where(np.abs(steps) >= k, np.nextafter(x, toward).astype(np.float32), x)
    x[:, 0] = amax
    x[:, 1] = -amax * np.float32(0.5)                       # a quotient next to -63.5
    xt = torch.from_numpy(x).to(device)
    codes, scales = ppk.quantize(xt.reshape(1, rows, d))
    ref_codes, ref_scales, _ = oracle.quantize(x.reshape(1, rows, d))
    assert np.array_equal(scales.cpu().numpy().view(np.uint32), ref_scales.view(np.uint32))
    got = codes.cpu().numpy()
    assert np.array_equal(got, ref_codes), f"{int((got != ref_codes).sum())} codes differ"
    q = x / s[:, None]                                      # share of values that sit within the band
    assert np.mean(np.abs(np.abs(q - np.rint(q)) - 0.5) < 2.0 ** -14) > 0.5


@pytest.mark.parametrize("kernel", ["row", "streaming"])
@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_quantize_signalling_nan_skipped_by_absmax(device, dt, kernel):
    """Signalling NaNs (either sign) next to the row's largest value: the absmax skips them as Rust's
    f32::max fold does (int8_kv_ops.rs:17), so the other values keep their codes and NaNs code to 0."""
    d = 128
    if kernel == "row":
        rows = 96
    else:
        cus = torch.cuda.get_device_properties(device).multi_processor_count
        rows = cus * 1024 * (4 if dt == "f32" else 8) // d + 64
    rng = np.random.default_rng(SEED + 71)
    x = rng.standard_normal((rows, d)).astype(np.float32)
    x[:, 1] = 40.0 * np.sign(x[:, 1] + 0.5)               # the row max, in the first lane's 16 bytes
    if dt == "bf16":
        bits = to_bf16_bits(x)
        snan = (np.uint16(0x7F81), np.uint16(0xFF81))
    elif dt == "f16":
        bits = x.astype(np.float16).view(np.uint16)
        snan = (np.uint16(0x7C01), np.uint16(0xFC01))
    else:
        bits = x.view(np.uint32).copy()
        snan = (np.uint32(0x7F800001), np.uint32(0xFF800001))
    bits[0::3, 0] = snan[0]                                # same lane as the max
    bits[1::3, 2] = snan[1]
    bits[2::5, d - 1] = snan[0]                            # another lane
    bits[7::11, :] = snan[1]                               # whole rows
    if dt == "bf16":
        xt = torch.from_numpy(bits.view(np.int16)).to(device).view(torch.bfloat16)
        x32 = (bits.astype(np.uint32) << 16).view(np.float32)
    elif dt == "f16":
        xt = torch.from_numpy(bits.view(np.float16)).to(device)
        x32 = bits.view(np.float16).astype(np.float32)
    else:
        xt = torch.from_numpy(bits.view(np.float32)).to(device)
        x32 = bits.view(np.float32)
    codes, scales = ppk.quantize(xt.reshape(1, rows, d))
    ref_codes, ref_scales, _ = oracle.quantize(x32.reshape(1, rows, d))
    assert np.array_equal(codes.cpu().numpy(), ref_codes)
    assert np.array_equal(scales.cpu().numpy().view(np.uint32), ref_scales.view(np.uint32))
    assert float(ref_scales[0, 0]) == np.float32(40.0) / np.float32(127.0)  # the NaN did not hide the max


def test_quantize_nonfinite_rows_flagged(device):
    d = 128
    x = np.random.default_rng(SEED).standard_normal((1, 4, d)).astype(np.float32)
    x[0, 1, 5] = np.nan
    x[0, 2, 9] = np.inf
    x[0, 3, :] = np.nan
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    xt = torch.from_numpy(x).to(device)
    codes = torch.empty((1, 4, d), dtype=torch.uint8, device=device)
    scales = torch.empty((1, 4), dtype=torch.float32, device=device)
    import ctypes
    a = ppk._abi.PpkQuantizeArgs(struct_size=ctypes.sizeof(ppk._abi.PpkQuantizeArgs), src_dtype=0,
                                 src=xt.data_ptr(), codes=codes.data_ptr(), scales=scales.data_ptr(), rows=4,
                                 head_dim=d, flags=flags.data_ptr())
    ppk._abi.check(ppk._abi.lib().ppk_quantize(ppk.context(device), None, ctypes.byref(a)), "ppk_quantize")
    torch.cuda.synchronize()
    assert flags.item() & ppk.PPK_FLAG_NONFINITE
    ref_codes, ref_scales, bad = oracle.quantize(x)
    assert bad == 3
    assert np.array_equal(codes.cpu().numpy(), ref_codes)
    assert np.array_equal(scales.cpu().numpy().view(np.uint32), ref_scales.view(np.uint32))


def _quantize_raw(device, src_ptr, src_dtype, codes, scales, rows, d):
    import ctypes
    a = ppk._abi.PpkQuantizeArgs(struct_size=ctypes.sizeof(ppk._abi.PpkQuantizeArgs), src_dtype=src_dtype,
                                 src=src_ptr, codes=codes.data_ptr(), scales=scales.data_ptr(), rows=rows,
                                 head_dim=d, flags=None)
    ppk._abi.check(ppk._abi.lib().ppk_quantize(ppk.context(device), None, ctypes.byref(a)), "ppk_quantize")


@pytest.mark.parametrize("dt,d", [("bf16", 64), ("f32", 128), ("f16", 256)])
def test_quantize_misaligned_source_matches_oracle(device, dt, d):
    """A source that is not 16-byte aligned takes the one-wave-per-row kernel; it stays bit-exact."""
    rng = np.random.default_rng(SEED + 31 + d)
    x = np.concatenate([kv_values(rng, 1, 8, 65, d).reshape(520, d), _special_rows(d)[0]])
    rows = x.shape[0]
    xt, x32 = _to_device(x, DTYPES[dt], device)
    eb = xt.element_size()
    big = torch.empty(rows * d + 16 // eb, dtype=xt.dtype, device=device)
    view = big[4 // eb:4 // eb + rows * d]           # 4 bytes past a 16-byte boundary
    view.copy_(xt.reshape(-1))
    codes = torch.empty((rows, d), dtype=torch.uint8, device=device)
    scales = torch.empty(rows, dtype=torch.float32, device=device)
    _quantize_raw(device, view.data_ptr(), ppk._abi.PPK_F32 if dt == "f32" else
                  (ppk._abi.PPK_BF16 if dt == "bf16" else ppk._abi.PPK_F16), codes, scales, rows, d)
    torch.cuda.synchronize()
    ref_codes, ref_scales, _ = oracle.quantize(x32)
    assert np.array_equal(codes.cpu().numpy(), ref_codes.reshape(rows, d))
    assert np.array_equal(scales.cpu().numpy().view(np.uint32), ref_scales.reshape(rows).view(np.uint32))


@pytest.mark.parametrize("dt,d", [("bf16", 128), ("f32", 64), ("f16", 256)])
def test_quantize_streaming_kernel_large_equals_row_kernel(device, dt, d):
    """Past the largest grid (two grid-stride passes plus a ragged tail, ~1 GB of input, special rows
    mixed in): the streaming kernel's codes and scales equal the one-wave-per-row kernel's bit for bit."""
    out_dt = DTYPES[dt]
    per_lane = 4 if out_dt == torch.float32 else 8
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    units = 2 * cus * 128 * 256 * 4 + 777                  # 128 blocks/CU x 256 lanes x 4-unit batches
    rows = -(-units * per_lane // d)
    g = torch.Generator(device=device).manual_seed(SEED + 41)
    x32 = torch.randn((rows, d), generator=g, device=device) * 3.0
    x32[::1009] *= 1e30                                    # huge rows
    x32[3::1013] = 0.0                                     # zero rows
    x32[5::2003, 7] = float("nan")                         # non-finite rows
    x32[11::4001] = torch.round(x32[11::4001] * 4) / 4     # quarter steps: exact half-step quotients
    x = x32.to(out_dt)
    del x32
    eb = x.element_size()
    code = ppk._abi.PPK_F32 if dt == "f32" else (ppk._abi.PPK_BF16 if dt == "bf16" else ppk._abi.PPK_F16)
    codes, scales = ppk.quantize(x.reshape(1, rows, d))
    big = torch.empty(rows * d + 16 // eb, dtype=x.dtype, device=device)
    view = big[4 // eb:4 // eb + rows * d]
    view.copy_(x.reshape(-1))
    del x
    codes_r = torch.empty((rows, d), dtype=torch.uint8, device=device)
    scales_r = torch.empty(rows, dtype=torch.float32, device=device)
    _quantize_raw(device, view.data_ptr(), code, codes_r, scales_r, rows, d)
    torch.cuda.synchronize()
    assert torch.equal(codes.reshape(rows, d), codes_r)
    assert torch.equal(scales.reshape(rows).view(torch.int32), scales_r.view(torch.int32))


@pytest.mark.parametrize("dt,d", [("bf16", 128), ("f32", 256), ("f16", 64)])
def test_append_streaming_kernel_equals_row_kernel(device, dt, d):
    """A ragged multi-token append (several thousand tokens per row, the last sequence running past the
    capacity) through the streaming kernel writes the same arenas and flags as the one-wave-per-row
    kernel, which a source 4 bytes off a 16-byte boundary selects."""
    import ctypes
    B, H, T, cap = 5, 16, 3000, 9000
    out_dt = DTYPES[dt]
    g = torch.Generator(device=device).manual_seed(SEED + 51)
    src = (torch.randn((2, B, H, T, d), generator=g, device=device) * 2).to(out_dt)
    past = torch.tensor([0, 17, 3000, 5999, 7500], dtype=torch.int32, device=device)  # last: 1500 overflow
    eb = src.element_size()
    results = []
    for misaligned in (False, True):
        kc = torch.full((B * H, cap, d), 0xAB, dtype=torch.uint8, device=device)
        vc = torch.full_like(kc, 0xCD)
        ks = torch.full((B * H, cap), -7.0, device=device)
        vs = torch.full_like(ks, -9.0)
        flags = torch.zeros(1, dtype=torch.int32, device=device)
        if misaligned:
            big = torch.empty(2 * src[0].numel() + 32 // eb, dtype=out_dt, device=device)
            n = src[0].numel()
            k_src = big[4 // eb:4 // eb + n]
            v_src = big[4 // eb + n + 16 // eb:4 // eb + 2 * n + 16 // eb]
            k_src.copy_(src[0].reshape(-1))
            v_src.copy_(src[1].reshape(-1))
            kp, vp = k_src.data_ptr(), v_src.data_ptr()
        else:
            kp, vp = src[0].data_ptr(), src[1].data_ptr()
        a = ppk._abi.PpkAppendArgs(struct_size=ctypes.sizeof(ppk._abi.PpkAppendArgs),
                                   src_dtype=ppk.int8_kv_ops._DTYPES[out_dt], k_src=kp, v_src=vp,
                                   past=past.data_ptr(), k_codes=kc.data_ptr(), v_codes=vc.data_ptr(),
                                   k_scales=ks.data_ptr(), v_scales=vs.data_ptr(), batch=B, heads=H, tokens=T,
                                   head_dim=d, capacity=cap, flags=flags.data_ptr())
        ppk._abi.check(ppk._abi.lib().ppk_quantize_append(ppk.context(device), None, ctypes.byref(a)),
                       "ppk_quantize_append")
        torch.cuda.synchronize()
        results.append((kc, vc, ks, vs, flags.item()))
    (a_k, a_v, a_ks, a_vs, a_f), (b_k, b_v, b_ks, b_vs, b_f) = results
    assert a_f == b_f and a_f & ppk.PPK_FLAG_OVERFLOW
    assert torch.equal(a_k, b_k) and torch.equal(a_v, b_v)
    assert torch.equal(a_ks.view(torch.int32), b_ks.view(torch.int32))
    assert torch.equal(a_vs.view(torch.int32), b_vs.view(torch.int32))


def _arenas(rng, rows, cap, d, filled):
    codes = rng.integers(-127, 128, size=(rows, cap, d)).astype(np.int8).view(np.uint8)
    scales = rng.random((rows, cap), dtype=np.float32) * 0.1
    codes[:, filled:] = 0xAB  # sentinel bytes beyond the committed history
    scales[:, filled:] = -7.0
    return codes, scales


def test_append_config2_bit_exact(device):
    """B=1, H=16, D=128, one fp16 token into capacity 4096 holding 1000 tokens."""
    rng = np.random.default_rng(SEED)
    B, H, D, cap, filled = 1, 16, 128, 4096, 1000
    kc, ks = _arenas(rng, B * H, cap, D, filled)
    vc, vs = _arenas(rng, B * H, cap, D, filled)
    k_new = kv_values(rng, B, H, 1, D)
    v_new = kv_values(rng, B, H, 1, D)
    kt, k32 = _to_device(k_new, torch.float16, device)
    vt, v32 = _to_device(v_new, torch.float16, device)
    past_np = np.array([filled], np.uint32)
    dk, dv = torch.from_numpy(kc.copy()).to(device), torch.from_numpy(vc.copy()).to(device)
    dks, dvs = torch.from_numpy(ks.copy()).to(device), torch.from_numpy(vs.copy()).to(device)
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    ppk.append(kt, vt, torch.from_numpy(past_np.view(np.int32)).to(device), dk, dv, dks, dvs, flags)
    torch.cuda.synchronize()
    assert flags.item() == 0
    for codes, scales, src, got_c, got_s in ((kc, ks, k32, dk, dks), (vc, vs, v32, dv, dvs)):
        exp_c, exp_s = codes.copy(), scales.copy()
        assert oracle.append(src, past_np, exp_c, exp_s) == 0
        assert np.array_equal(got_c.cpu().numpy(), exp_c)
        assert np.array_equal(got_s.cpu().numpy().view(np.uint32), exp_s.view(np.uint32))


@pytest.mark.parametrize("d", [64, 256])
def test_append_ragged_multi_token_with_overflow(device, d):
    rng = np.random.default_rng(SEED + 7)
    B, H, T, cap = 3, 2, 3, 40
    past_np = np.array([0, 17, cap - 2], np.uint32)  # last sequence: token 2 would land past capacity
    kc, ks = _arenas(rng, B * H, cap, d, 0)
    vc, vs = _arenas(rng, B * H, cap, d, 0)
    k_new = kv_values(rng, B, H, T, d, heavy=False)
    v_new = kv_values(rng, B, H, T, d, heavy=False)
    kt, k32 = _to_device(k_new, torch.bfloat16, device)
    vt, v32 = _to_device(v_new, torch.bfloat16, device)
    dk, dv = torch.from_numpy(kc.copy()).to(device), torch.from_numpy(vc.copy()).to(device)
    dks, dvs = torch.from_numpy(ks.copy()).to(device), torch.from_numpy(vs.copy()).to(device)
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    ppk.append(kt, vt, torch.from_numpy(past_np.view(np.int32)).to(device), dk, dv, dks, dvs, flags)
    torch.cuda.synchronize()
    assert flags.item() & ppk.PPK_FLAG_OVERFLOW
    for codes, scales, src, got_c, got_s in ((kc, ks, k32, dk, dks), (vc, vs, v32, dv, dvs)):
        exp_c, exp_s = codes.copy(), scales.copy()
        assert oracle.append(src, past_np, exp_c, exp_s) == H  # one token of each head of sequence 2
        assert np.array_equal(got_c.cpu().numpy(), exp_c)
        assert np.array_equal(got_s.cpu().numpy().view(np.uint32), exp_s.view(np.uint32))


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_dequantize_matches_oracle(device, d, dt):
    rng = np.random.default_rng(SEED + 3)
    x = kv_values(rng, 1, 8, 33, d).reshape(8, 33, d)
    codes, scales = ppk.quantize(torch.from_numpy(x).to(device))
    out = ppk.dequantize(codes, scales, DTYPES[dt]).cpu()
    ref = oracle.dequantize(codes.cpu().numpy(), scales.cpu().numpy())
    if dt == "f32":
        assert np.array_equal(out.numpy().view(np.uint32), ref.view(np.uint32))
    elif dt == "bf16":
        assert np.array_equal(out.view(torch.int16).numpy().view(np.uint16), to_bf16_bits(ref))
    else:
        assert np.array_equal(out.numpy().view(np.uint16), ref.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("dt,round_bf16,d", [("f32", 0, 128), ("f32", 1, 256), ("bf16", 0, 64), ("f16", 0, 128),
                                            ("f16", 1, 256)])
def test_dequantize_grid_stride_sizes(device, dt, round_bf16, d):
    """Inputs past one batch per lane of the largest grid (two grid-stride passes plus a ragged tail), every
    output type and the bf16 pre-rounding flag. Reference on the device: int8 code * f32 scale is one exact
    IEEE product, then torch's round-to-nearest-even conversions (bf16 first when the flag is set)."""
    import ctypes

    from ppk import _abi
    from ppk import int8_kv_ops as ops

    out_dt = DTYPES[dt]
    per_unit = 4 if out_dt == torch.float32 else 8          # codes per 16-byte output chunk
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    units = 2 * cus * 128 * 256 * 8 + 12345                  # 128 blocks/CU x 256 lanes x 8-chunk batches
    rows = -(-units * per_unit // d)
    g = torch.Generator(device=device).manual_seed(SEED + 11)
    codes = torch.randint(0, 256, (rows, d), dtype=torch.uint8, device=device, generator=g)
    scales = torch.rand((rows,), generator=g, device=device) * 10.0 ** torch.randint(
        -30, 30, (rows,), generator=g, device=device).float()
    out = torch.empty((rows, d), dtype=out_dt, device=device)
    a = _abi.PpkDequantizeArgs(struct_size=ctypes.sizeof(_abi.PpkDequantizeArgs), out_dtype=ops._DTYPES[out_dt],
                               codes=codes.data_ptr(), scales=scales.data_ptr(), out=out.data_ptr(), rows=rows,
                               head_dim=d, round_bf16=round_bf16)
    _abi.check(_abi.lib().ppk_dequantize(ops.context(device), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream),
                                         ctypes.byref(a)), "ppk_dequantize")
    ref = codes.view(torch.int8).float() * scales[:, None]
    if round_bf16:
        ref = ref.to(torch.bfloat16).float()
    ref = ref.to(out_dt)
    bits = torch.int32 if out_dt == torch.float32 else torch.int16
    mismatch = (out.view(bits) != ref.view(bits)).sum().item()
    assert mismatch == 0, f"{mismatch} of {out.numel()} outputs differ ({dt}, round_bf16={round_bf16}, d={d})"


def test_int8_capability_gate(device):
    """prepare_int8_kv (int8_policy.rs:26-55): not requested, unavailable head width, then ready + enabled."""
    off = ppk.prepare_int8_kv(False, 64, device)
    assert not off["enabled"] and off["format"] == "BF16/F32" and off["requested"] is False
    odd = ppk.prepare_int8_kv(True, 96, device)
    assert odd["requested"] and not odd["available"] and not odd["enabled"]
    on = ppk.prepare_int8_kv(True, 64, device)
    assert on["available"] and on["ready"] and on["enabled"] and on["format"].startswith("INT8")
    assert (on["packed_bytes_per_token_head"], on["scale_bytes_per_token_head"]) == (128, 8)
    again = ppk.prepare_int8_kv(True, 128, device)
    assert again["enabled"] and again["packed_bytes_per_token_head"] == 256
