"""Seeded randomized parity sweep over the whole C-ABI surface (GPU).

Each case draws its geometry, dtypes, lengths, splits and value ranges from a
seeded generator (the case id is the seed offset, printed on failure) and
checks the device result against the oracle at the bar of the row it
belongs to: quantize and dequantize bit-exact; int8 attention within max abs 2e-3 and max relative 1e-2 (|ref| >= 1e-3);
float-KV attention within 1e-4 + 1e-4 |ref|; the sampler bit-identical to
the reference's own kernel (oracle/_ref). Sizes are bounded so the whole
sweep runs in seconds.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import ppk
import refkernels
from helpers import SEED, assert_close, bf16_bits_to_f32, to_bf16_bits

pytestmark = pytest.mark.gpu
DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def as_device(x32: np.ndarray, dtype, device):
    """float32 host values -> device tensor of `dtype` plus the float32 values it holds exactly."""
    if dtype == torch.float32:
        return torch.from_numpy(x32).to(device), x32
    if dtype == torch.float16:
        h = x32.astype(np.float16)
        return torch.from_numpy(h).to(device), h.astype(np.float32)
    bits = to_bf16_bits(x32)
    return torch.from_numpy(bits.view(np.int16)).to(device).view(torch.bfloat16), bf16_bits_to_f32(bits)


@pytest.mark.parametrize("case", range(24))
def test_quantize_random(device, case):
    rng = np.random.default_rng(SEED + 1000 + case)
    d = int(rng.choice([64, 128, 256]))
    heads, tokens = int(rng.integers(1, 9)), int(rng.integers(1, 700))
    dtype = DTYPES[case % 3]
    top = {torch.float32: 6, torch.bfloat16: 3, torch.float16: 2}[dtype]  # 127 * mag stays finite in f16
    mag = 10.0 ** rng.uniform(-6, top)
    x = (rng.standard_normal((heads, tokens, d)) * mag).astype(np.float32)
    x[:, ::17] = 0.0                                   # zero rows
    x[:, 3::29, 5] = np.float32(mag * 127)             # large entries fix the scale exactly
    xt, x32 = as_device(x, dtype, device)
    codes, scales = ppk.quantize(xt)
    ref_c, ref_s, _ = oracle.quantize(x32)
    assert np.array_equal(codes.cpu().numpy(), ref_c), f"case {case}"
    assert np.array_equal(scales.cpu().numpy(), ref_s), f"case {case}"


@pytest.mark.parametrize("case", range(12))
def test_dequantize_random(device, case):
    import ctypes

    from ppk import _abi
    from ppk import int8_kv_ops as ops

    rng = np.random.default_rng(SEED + 1500 + case)
    d = int(rng.choice([64, 128, 256]))
    rows = int(rng.integers(1, 5000))
    out_dt = DTYPES[case % 3]
    round_bf16 = int(rng.integers(0, 2))
    codes = rng.integers(0, 256, (rows, d), dtype=np.uint8)
    scales = (rng.random(rows) * 10.0 ** rng.uniform(-20, 20, rows)).astype(np.float32)
    c_t, s_t = torch.from_numpy(codes).to(device), torch.from_numpy(scales).to(device)
    out = torch.empty((rows, d), dtype=out_dt, device=device)
    a = _abi.PpkDequantizeArgs(struct_size=ctypes.sizeof(_abi.PpkDequantizeArgs), out_dtype=ops._DTYPES[out_dt],
                               codes=c_t.data_ptr(), scales=s_t.data_ptr(), out=out.data_ptr(), rows=rows,
                               head_dim=d, round_bf16=round_bf16)
    _abi.check(_abi.lib().ppk_dequantize(ops.context(device), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream),
                                         ctypes.byref(a)), "ppk_dequantize")
    ref = oracle.dequantize(codes, scales, round_bf16=bool(round_bf16))
    what = f"case {case}: rows {rows} d {d} {out_dt} round {round_bf16}"
    if out_dt == torch.float32:
        assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32)), what
    elif out_dt == torch.bfloat16:
        assert np.array_equal(out.cpu().view(torch.int16).numpy().view(np.uint16), to_bf16_bits(ref)), what
    else:
        # Scales up to 1e20 put values past f16's range: the expected result is
        # the round-to-nearest cast, ±inf there, as the kernel's conversion gives.
        with np.errstate(over="ignore"):
            want = ref.astype(np.float16)
        assert np.array_equal(out.cpu().numpy().view(np.uint16), want.view(np.uint16)), what


@pytest.mark.parametrize("case", range(16))
def test_int8_attention_random(device, case):
    rng = np.random.default_rng(SEED + 2000 + case)
    d = int(rng.choice([64, 128, 256]))
    B, H = int(rng.integers(1, 5)), int(rng.integers(1, 9))
    rows = B * H
    past = rng.integers(0, 2500, B).astype(np.uint32)
    past[0] = int(rng.choice([0, int(past[0])]))
    cap = int(past.max()) + 1 + int(rng.integers(0, 40))
    hist = rng.standard_normal((rows, cap, d)).astype(np.float32) * np.float32(rng.uniform(0.1, 5))
    vhist = rng.standard_normal((rows, cap, d)).astype(np.float32)
    kc, ks, _ = oracle.quantize(hist)
    vc, vs, _ = oracle.quantize(vhist)
    q_dt, s_dt, o_dt = DTYPES[case % 3], DTYPES[(case // 3) % 3], DTYPES[(case // 2) % 3]
    qt, q32 = as_device(rng.standard_normal((rows, 1, d)).astype(np.float32), q_dt, device)
    skt, sk32 = as_device(rng.standard_normal((rows, 1, d)).astype(np.float32), s_dt, device)
    svt, sv32 = as_device(rng.standard_normal((rows, 1, d)).astype(np.float32), s_dt, device)
    split = int(rng.choice([0, 0, int(rng.integers(1, 3000))]))
    t = lambda a: torch.from_numpy(a).to(device)
    out = ppk.attention(qt, t(kc), t(vc), t(ks), t(vs), skt, svt, t(past.view(np.int32)), H, split, out_dtype=o_dt)
    torch.cuda.synchronize()
    ref = oracle.attention(q32, kc, vc, ks, vs, sk32, sv32, past, H)
    got = out.float().reshape(rows, d).cpu().numpy()
    narrow = {torch.float32: None, torch.bfloat16: "bf16", torch.float16: "f16"}[o_dt]
    assert_close(got, ref, what=f"case {case} d{d} B{B} H{H} split {split}", out_dtype=narrow)


@pytest.mark.parametrize("case", range(16))
def test_float_attention_random(device, case):
    rng = np.random.default_rng(SEED + 3000 + case)
    d = int(rng.choice([64, 128, 256]))
    B, H = int(rng.integers(1, 5)), int(rng.integers(1, 9))
    rows = B * H
    size = int(rng.integers(1, 2000))
    cap = size + int(rng.integers(0, 3)) * 8
    kv = torch.bfloat16 if case % 2 else torch.float32
    k32 = rng.standard_normal((rows, cap, d)).astype(np.float32)
    v32 = rng.standard_normal((rows, cap, d)).astype(np.float32)
    if kv == torch.bfloat16:
        kh, vh = to_bf16_bits(k32), to_bf16_bits(v32)
        k = torch.from_numpy(kh.view(np.int16)).to(device).view(torch.bfloat16)[:, :size]
        v = torch.from_numpy(vh.view(np.int16)).to(device).view(torch.bfloat16)[:, :size]
    else:
        kh, vh = k32, v32
        k, v = torch.from_numpy(k32).to(device)[:, :size], torch.from_numpy(v32).to(device)[:, :size]
    lengths = None
    if rng.random() < 0.7:
        lengths = rng.integers(0, size + 2, B).astype(np.uint32)
    lt = None if lengths is None else torch.from_numpy(lengths.view(np.int32)).to(device)
    q = rng.standard_normal((rows, 1, d)).astype(np.float32)
    split = int(rng.choice([0, 0, int(rng.integers(1, 2048))]))
    out = ppk.fused_attention.decode_attention(torch.from_numpy(q).to(device), k, v, lt, H, split)
    torch.cuda.synchronize()
    ref = oracle.attention_float(q, kh[:, :size], vh[:, :size], lengths, H)
    assert_close(out.reshape(rows, d).cpu().numpy(), ref, atol=1e-4, rtol=1e-2,
                 what=f"case {case} d{d} B{B} H{H} size {size} split {split}")


@pytest.mark.parametrize("case", range(12))
def test_sampler_random_vs_reference_kernel(device, case):
    rng = np.random.default_rng(SEED + 4000 + case)
    guidance = 1 + case % 2
    batch, choices = int(rng.integers(1, 70)), int(rng.integers(1, 2049))
    scale = 10.0 ** rng.uniform(-2, 1.5)
    raw = (rng.standard_normal((batch * guidance, choices)) * scale).astype(np.float32)
    if case % 3 == 0:
        raw = np.round(raw)  # heavy ties
    u = rng.uniform(0, 1, batch).astype(np.float32)
    starts = rng.integers(0, choices, batch)
    counts = rng.integers(1, choices - starts + 1)
    bounds = np.stack([starts, counts], 1).astype(np.uint32)
    alpha = float(rng.uniform(1.01, 20))
    cfg = float(rng.uniform(0, 5)) if guidance == 2 else 1.0
    offset = int(rng.integers(0, 1 << 20))
    raw_t = torch.from_numpy(raw).to(device)
    u_t = torch.from_numpy(u.reshape(-1, 1)).to(device)
    b_t = torch.from_numpy(bounds.view(np.int32)).to(device)
    tok, val, sup = ppk.sampling.sample(raw_t, u_t, b_t, alpha, cfg, guidance, offset)
    ref = refkernels.renyi_sample(raw_t, u_t, b_t, alpha, cfg, guidance, offset)
    torch.cuda.synchronize()
    got = torch.stack([tok.reshape(-1), val.reshape(-1), sup.reshape(-1)])
    assert torch.equal(got, ref), f"case {case}: batch {batch} choices {choices} guidance {guidance}"


@pytest.mark.parametrize("case", range(32))
def test_decode_step_random(device, case):
    """ppk_decode_step (append of the current token + attention in one call) at random geometry, lengths
    (empty rows, short windows, full rows), splits, dtypes and max_past: output against the oracle at the
    attention bar, slot past[b] holding the oracle's codes of the current token (nothing at a full row,
    which is flagged), every other arena byte untouched."""
    from test_gpu_attention import Case

    rng = np.random.default_rng(SEED + 5000 + case)
    d = int(rng.choice([64, 128, 256]))
    B, H = int(rng.integers(1, 6)), int(rng.integers(1, 9))
    cap = int(rng.choice([int(rng.integers(1, 80)), int(rng.integers(80, 3000))]))
    lengths = [int(rng.choice([0, cap, int(rng.integers(0, cap + 1)), int(rng.integers(0, min(cap, 40) + 1))]))
               for _ in range(B)]
    q_dt, s_dt = DTYPES[case % 3], DTYPES[(case // 3) % 3]
    c = Case(device, B, H, d, lengths, cap, q_dtype=q_dt, scratch_dtype=s_dt, seed=SEED + 5100 + case)
    bf16h = case % 4 == 3  # the reference-exact mode (history rounded through bf16, int8_kv.cu:26)
    ref = c.reference(history_bf16=bf16h)
    before = [t.clone() for t in (c.kc, c.vc, c.ks, c.vs)]
    split = int(rng.choice([0, 0, int(rng.integers(1, 3000))]))
    max_past = int(rng.choice([0, max(lengths)]))
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    out = ppk.decode_step(c.q, c.kc, c.vc, c.ks, c.vs, c.sk, c.sv, c.past_t, H, split_tokens=split, flags=flags,
                          max_past=max_past, bf16_history=bf16h)
    torch.cuda.synchronize()
    what = f"case {case}: d{d} B{B} H{H} cap {cap} lengths {lengths} split {split} max_past {max_past} bf16h {bf16h}"
    assert_close(out.reshape(c.rows, d).cpu().numpy(), ref, atol=2e-3, rtol=1e-2, what=what)
    codes, scales, _ = oracle.quantize(c.sk32.reshape(c.rows, 1, d))
    vcodes, vscales, _ = oracle.quantize(c.sv32.reshape(c.rows, 1, d))
    exp = [t.cpu().numpy() for t in before]
    for r in range(c.rows):
        p = lengths[r // H]
        if p < cap:
            exp[0][r, p], exp[2][r, p] = codes[r, 0], scales[r, 0]
            exp[1][r, p], exp[3][r, p] = vcodes[r, 0], vscales[r, 0]
    for got, want, name in zip((c.kc, c.vc, c.ks, c.vs), exp, ("k", "v", "ks", "vs")):
        np.testing.assert_array_equal(got.cpu().numpy(), want, err_msg=f"{name} arena, {what}")
    assert bool(flags.item() & ppk.PPK_FLAG_OVERFLOW) == (cap in lengths), what
    assert not flags.item() & ppk.PPK_FLAG_NONFINITE, what


@pytest.mark.parametrize("case", range(16))
def test_append_random(device, case):
    """ppk_quantize_append: ragged multi-token appends of K and V [B, H, T, D] at random pasts (some running
    past the capacity) into pre-filled arenas, bit-exact against the oracle's append (slots written,
    slots past the capacity skipped and flagged, everything else untouched). Sizes cover the
    one-wave-per-row kernel and the streaming kernel."""
    rng = np.random.default_rng(SEED + 6000 + case)
    d = int(rng.choice([64, 128, 256]))
    B, H = int(rng.integers(1, 5)), int(rng.integers(1, 9))
    T = int(rng.choice([1, int(rng.integers(2, 40)), int(rng.integers(200, 3000))]))
    cap = int(rng.integers(T, 2 * T + 64))
    past = rng.integers(0, cap + 1, B).astype(np.uint32)
    past[0] = min(int(past[0]), cap - T)                      # one sequence that fits
    dt = DTYPES[case % 3]
    top = {torch.float32: 4, torch.bfloat16: 3, torch.float16: 2}[dt]
    x32 = (rng.standard_normal((2, B, H, T, d)) * 10.0 ** rng.uniform(-3, top)).astype(np.float32)
    kt, k32 = as_device(x32[0], dt, device)
    vt, v32 = as_device(x32[1], dt, device)
    rows = B * H
    kc0 = rng.integers(0, 256, (rows, cap, d), dtype=np.uint8)
    vc0 = rng.integers(0, 256, (rows, cap, d), dtype=np.uint8)
    ks0 = rng.standard_normal((rows, cap)).astype(np.float32)
    vs0 = rng.standard_normal((rows, cap)).astype(np.float32)
    t = lambda a: torch.from_numpy(a.copy()).to(device)  # noqa: E731
    kc, vc, ks, vs = t(kc0), t(vc0), t(ks0), t(vs0)
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    ppk.int8_kv_ops.append(kt.contiguous(), vt.contiguous(), t(past.view(np.int32)), kc, vc, ks, vs, flags=flags)
    torch.cuda.synchronize()
    ek, eks, ev, evs = kc0.copy(), ks0.copy(), vc0.copy(), vs0.copy()
    oracle.append(k32, past, ek, eks)
    oracle.append(v32, past, ev, evs)
    what = f"case {case}: d{d} B{B} H{H} T{T} cap {cap} past {past.tolist()} {dt}"
    assert np.array_equal(kc.cpu().numpy(), ek) and np.array_equal(vc.cpu().numpy(), ev), what
    assert np.array_equal(ks.cpu().numpy().view(np.uint32), eks.view(np.uint32)), what
    assert np.array_equal(vs.cpu().numpy().view(np.uint32), evs.view(np.uint32)), what
    overflow = bool((past.astype(np.int64) + T > cap).any())
    assert bool(flags.item() & ppk.PPK_FLAG_OVERFLOW) == overflow, what
