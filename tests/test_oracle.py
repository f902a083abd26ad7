"""Pins of the CPU oracle (oracle/ppk_oracle.c) that need no GPU.

Each function of the oracle is checked against something it does not share
code with: the golden fixtures of the reference's own procedural
known-answer checks (tests/golden/, restated in plain numpy from
app/src/model/int8_kv_ops.rs:56-103), an independent numpy restatement,
closed forms, and brute force on tiny inputs. Where useful, a plausible
mistake is planted in a numpy copy of the rule to show that the pin catches it.
"""
from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch

import oracle
from golden.make_golden import host_attention, np_dequantize, np_quantize
from helpers import SEED, kv_values, to_bf16_bits, bf16_bits_to_f32

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def golden(name: str) -> dict:
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _bits(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


# --------------------------------------------------------------------------- quantize

def _stress_rows(rng: np.random.Generator, d: int) -> np.ndarray:
    rows = [kv_values(rng, 1, 8, 64, d).reshape(-1, d)]                     # N(0,1) + heavy 10*t3 channels
    rows.append(rng.standard_normal((64, d)).astype(np.float32) * np.float32(1e-39))  # subnormal rows
    rows.append(rng.standard_normal((64, d)).astype(np.float32) * np.float32(3e37))   # near the top of f32
    ties = np.zeros((64, d), np.float32)
    ties[:, 0] = 127.0                                                        # scale exactly 1
    ties[:, 1:] = rng.integers(-254, 255, size=(64, d - 1)) / np.float32(2.0)  # many exact .5 quotients
    rows.append(ties)
    rows.append(np.zeros((2, d), np.float32))
    return np.concatenate(rows).astype(np.float32)


@pytest.mark.parametrize("d", [64, 128, 256])
def test_quantize_matches_independent_numpy_restatement(d):
    x = _stress_rows(np.random.default_rng(SEED + d), d)
    codes, scales, bad = oracle.quantize(x)
    ref_codes, ref_scales = np_quantize(x)
    assert bad == 0
    assert np.array_equal(codes, ref_codes)
    assert np.array_equal(_bits(scales), _bits(ref_scales))


def test_quantize_golden_fixtures():
    """Reference KAT (i) inputs (int8_kv_ops.rs:59) and the config-2 fp16 append rows."""
    g = golden("kat_quantize_sin017.npz")
    codes, scales, _ = oracle.quantize(g["x"])
    assert np.array_equal(codes, g["codes"]) and np.array_equal(_bits(scales), _bits(g["scales"]))
    # The reference's own acceptance bound for the round trip (int8_kv_ops.rs:62).
    restored = oracle.dequantize(codes, scales)
    assert np.all(np.abs(restored - g["x"]) < 0.009)
    c2 = golden("config2_append.npz")
    for name in ("k", "v"):
        x = c2[f"{name}_new_f16"].astype(np.float32).reshape(16, 1, 128)  # fp16 -> f32 is exact
        codes, scales, _ = oracle.quantize(x)
        assert np.array_equal(codes, c2[f"{name}_codes"])
        assert np.array_equal(_bits(scales), _bits(c2[f"{name}_scales"]))


def test_quantize_closed_forms():
    # absmax 127 -> scale exactly 1, codes are textbook round-half-to-even.
    x = np.zeros((1, 64), np.float32)
    x[0, :9] = [127.0, 0.5, 1.5, 2.5, -2.5, -0.5, 3.5, -126.5, 126.5]
    codes, scales, _ = oracle.quantize(x)
    assert scales[0] == 1.0
    assert codes[0, :9].view(np.int8).tolist() == [127, 0, 2, 2, -2, 0, 4, -126, 126]
    # A zero row takes the 1e-12 floor and all-zero codes.
    codes, scales, _ = oracle.quantize(np.zeros((1, 128), np.float32))
    assert scales[0] == np.float32(1e-12) and not codes.any()
    # The absmax element always maps to +-127; every element is within half a step.
    x = kv_values(np.random.default_rng(SEED), 1, 16, 33, 128).reshape(-1, 128)
    codes, scales, _ = oracle.quantize(x)
    c = codes.view(np.int8).astype(np.int64)
    idx = np.argmax(np.abs(x), axis=1)
    assert np.all(np.abs(c[np.arange(len(x)), idx]) == 127)
    err = np.abs(x.astype(np.float64) - c * scales[:, None].astype(np.float64))
    assert np.all(err <= scales[:, None] * (0.5 + 1e-5))
    # Odd symmetry and power-of-two scaling are exact.
    n_codes, n_scales, _ = oracle.quantize(-x)
    assert np.array_equal(n_codes.view(np.int8), -codes.view(np.int8)) and np.array_equal(n_scales, scales)
    s_codes, s_scales, _ = oracle.quantize(x * np.float32(8.0))
    assert np.array_equal(s_codes, codes) and np.array_equal(s_scales, scales * np.float32(8.0))


def test_quantize_nonfinite_rows_are_counted():
    x = np.ones((3, 64), np.float32)
    x[1, 3] = np.nan
    x[2, 0] = np.inf
    codes, scales, bad = oracle.quantize(x)
    assert bad == 2
    assert codes[1, 3] == 0  # NaN quotient -> 0, like Rust `as i8` and CUDA __float2int_rn
    assert scales[2] == np.inf and not codes[2].any()


def test_quantize_absmax_skips_nans_of_both_kinds():
    """int8_kv_ops.rs:17 folds |x| with f32::max, which returns the other argument whenever one is NaN,
    quiet or signalling: the scale is max(nanmax|x| / 127, 1e-12) and the NaNs code to 0."""
    x = np.random.default_rng(SEED).standard_normal((6, 64)).astype(np.float32)
    x[:, 5] = 40.0
    bits = x.view(np.uint32)
    bits[0, 0] = 0x7F800001   # signalling NaN before the max
    bits[1, 9] = 0xFF800001   # negative signalling NaN after it
    bits[2, 63] = 0x7FA00000  # signalling NaN last
    bits[3, 7] = 0x7FC00000   # quiet NaN
    bits[4, :] = 0xFF800001   # all NaN -> scale 1e-12
    codes, scales, bad = oracle.quantize(x)
    assert bad == 5
    amax = np.fmax.reduce(np.abs(x), axis=1, initial=np.float32(0))  # fmax skips NaN
    want = np.maximum(amax / np.float32(127.0), np.float32(1e-12))
    assert np.array_equal(scales, want.astype(np.float32))
    assert scales[0] == np.float32(40.0) / np.float32(127.0) and scales[4] == np.float32(1e-12)
    assert codes[0, 0] == 0 and codes[1, 9] == 0 and not codes[4].any()
    assert codes[0, 5] == 127


def _planted_reciprocal(x):
    """The AMD variant's rule (kv_int8.cpp:51): absmax * (1/127) instead of absmax / 127."""
    amax = np.max(np.abs(x), axis=-1)
    s = np.maximum(amax * np.float32(1.0 / 127.0), np.float32(1e-12)).astype(np.float32)
    return np.clip(np.rint(x / s[..., None]), -127, 127).astype(np.int8).view(np.uint8), s


def _planted_half_away(x):
    amax = np.max(np.abs(x), axis=-1)
    s = np.maximum(amax / np.float32(127.0), np.float32(1e-12)).astype(np.float32)
    q = np.trunc(x / s[..., None] + np.copysign(np.float32(0.5), x))
    return np.clip(q, -127, 127).astype(np.int8).view(np.uint8), s


def test_pins_catch_planted_quantize_mistakes():
    """The checks above distinguish the division rule from the reciprocal rule and ties-to-even
    from round-half-away: the planted variants disagree with the oracle on the same inputs."""
    x = _stress_rows(np.random.default_rng(SEED + 128), 128)
    codes, scales, _ = oracle.quantize(x)
    _, recip_scales = _planted_reciprocal(x)
    assert not np.array_equal(_bits(recip_scales), _bits(scales))
    ties = np.zeros((1, 64), np.float32)
    ties[0, :3] = [127.0, 0.5, 2.5]
    away_codes, _ = _planted_half_away(ties)
    assert away_codes[0, 1:3].view(np.int8).tolist() == [1, 3]  # the closed-form test expects [0, 2]


# --------------------------------------------------------------------------- dequantize / append

def test_dequantize_matches_numpy_and_torch_bf16():
    x = kv_values(np.random.default_rng(SEED + 1), 1, 4, 40, 128).reshape(4, 40, 128)
    codes, scales, _ = oracle.quantize(x)
    assert np.array_equal(_bits(oracle.dequantize(codes, scales)), _bits(np_dequantize(codes, scales, False)))
    got = oracle.dequantize(codes, scales, round_bf16=True)
    ref = np_dequantize(codes, scales, True)  # torch's float32 -> bfloat16 conversion
    assert np.array_equal(_bits(got), _bits(ref))
    assert np.array_equal(to_bf16_bits(oracle.dequantize(codes, scales)), to_bf16_bits(ref))


def test_append_places_rows_at_past_and_skips_overflow():
    rng = np.random.default_rng(SEED + 2)
    B, H, T, cap, d = 3, 2, 3, 12, 64
    past = np.array([0, 5, cap - 2], np.uint32)
    src = kv_values(rng, B, H, T, d)
    codes = rng.integers(0, 256, size=(B * H, cap, d)).astype(np.uint8)
    scales = rng.random((B * H, cap)).astype(np.float32)
    before_c, before_s = codes.copy(), scales.copy()
    skipped = oracle.append(src, past, codes, scales)
    assert skipped == H  # token 2 of sequence 2 lands at slot cap
    exp_c, exp_s = before_c.copy(), before_s.copy()
    for b in range(B):
        for h in range(H):
            for t in range(T):
                slot = int(past[b]) + t
                if slot < cap:
                    qc, qs = np_quantize(src[b, h, t][None])
                    exp_c[b * H + h, slot], exp_s[b * H + h, slot] = qc[0], qs[0]
    assert np.array_equal(codes, exp_c) and np.array_equal(scales, exp_s)


# --------------------------------------------------------------------------- attention

def _problem(rng, rows, heads, cap, d, lengths, heavy=True):
    hist = kv_values(rng, 1, rows, cap, d, heavy=heavy).reshape(rows, cap, d)
    vals = kv_values(rng, 1, rows, cap, d, heavy=heavy).reshape(rows, cap, d)
    kc, ks, _ = oracle.quantize(hist)
    vc, vs, _ = oracle.quantize(vals)
    q = rng.standard_normal((rows, d)).astype(np.float32)
    sk = rng.standard_normal((rows, d)).astype(np.float32)
    sv = rng.standard_normal((rows, d)).astype(np.float32)
    return q, kc, vc, ks, vs, sk, sv, np.asarray(lengths, np.uint32)


def _numpy_attention(q, kc, vc, ks, vs, sk, sv, past, heads, scale, bf16=False):
    """Independent vectorised f64 restatement."""
    rows, cap, d = kc.shape
    kd = np_dequantize(kc, ks, bf16).astype(np.float64)
    vd = np_dequantize(vc, vs, bf16).astype(np.float64)
    out = np.empty((rows, d))
    for r in range(rows):
        p = int(past[r // heads])
        if p > cap:
            out[r] = np.nan
            continue
        keys = np.concatenate([kd[r, :p], sk[r][None].astype(np.float64)])
        vals = np.concatenate([vd[r, :p], sv[r][None].astype(np.float64)])
        s = keys @ q[r].astype(np.float64) * scale
        w = np.exp(s - s.max())
        out[r] = w @ vals / w.sum()
    return out


@pytest.mark.parametrize("bf16", [False, True])
def test_attention_matches_independent_numpy(bf16):
    rng = np.random.default_rng(SEED + 3)
    rows, heads, cap, d = 8, 2, 90, 128
    args = _problem(rng, rows, heads, cap, d, [0, 1, 89, 90])
    got = oracle.attention(*args, heads, history_bf16=bf16)
    ref = _numpy_attention(*args, heads, float(np.float32(1 / math.sqrt(d))), bf16)  # the oracle takes an f32 scale
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)


def test_threaded_attention_is_the_single_thread_result():
    """oracle_attention_mt shares rows over threads; each row is computed exactly as by one thread."""
    rng = np.random.default_rng(SEED + 31)
    rows, heads, cap, d = 24, 4, 70, 64
    args = _problem(rng, rows, heads, cap, d, [0, 3, 69, 71, 40, 12])
    one = oracle.attention(*args, heads, threads=1)
    for threads in (2, 5, 24, 64):
        many = oracle.attention(*args, heads, threads=threads)
        assert np.array_equal(np.isnan(one), np.isnan(many))
        assert np.array_equal(one[~np.isnan(one)].view(np.uint64), many[~np.isnan(many)].view(np.uint64))


def test_attention_brute_force_tiny():
    """Plain Python loops with math.exp on a 2-row, 3-token, 64-channel problem."""
    rng = np.random.default_rng(SEED + 4)
    q, kc, vc, ks, vs, sk, sv, past = _problem(rng, 2, 1, 3, 64, [2, 3], heavy=False)
    got = oracle.attention(q, kc, vc, ks, vs, sk, sv, past, 1)
    for r in range(2):
        p = int(past[r])
        keys = [[float(np.int8(kc[r, t, i].astype(np.int8))) * float(ks[r, t]) for i in range(64)] for t in range(p)]
        keys.append([float(x) for x in sk[r]])
        vals = [[float(np.int8(vc[r, t, i].astype(np.int8))) * float(vs[r, t]) for i in range(64)] for t in range(p)]
        vals.append([float(x) for x in sv[r]])
        s = [sum(float(q[r, i]) * k[i] for i in range(64)) / 8.0 for k in keys]
        mx = max(s)
        w = [math.exp(x - mx) for x in s]
        z = sum(w)
        ref = [sum(w[t] * vals[t][i] for t in range(p + 1)) / z for i in range(64)]
        # f32 products of code * scale: the loops above use exact doubles of the same f32 values.
        np.testing.assert_allclose(got[r], ref, rtol=1e-6, atol=1e-7)


def test_attention_closed_forms():
    rng = np.random.default_rng(SEED + 5)
    rows, heads, cap, d = 4, 1, 50, 64
    q, kc, vc, ks, vs, sk, sv, past = _problem(rng, rows, heads, cap, d, [0, 50, 50, 51], heavy=False)
    out = oracle.attention(q, kc, vc, ks, vs, sk, sv, past, heads)
    # Empty history: the softmax has one term, the output is sv exactly.
    assert np.array_equal(out[0], sv[0].astype(np.float64))
    # Past beyond capacity: NaN (int8_kv.cu:33,51).
    assert np.isnan(out[3]).all()
    # Identical keys (history and current): uniform weights, the output is the mean of the values.
    kc2, ks2 = kc.copy(), ks.copy()
    kc2[1, :] = kc2[1, 0]
    ks2[1, :] = ks2[1, 0]
    sk2 = sk.copy()
    sk2[1] = kc2[1, 0].view(np.int8).astype(np.float32) * ks2[1, 0]
    out2 = oracle.attention(q, kc2, vc, ks2, vs, sk2, sv, past, heads)
    hist_v = (vc[1, :50].view(np.int8).astype(np.float32) * vs[1, :50, None]).astype(np.float64)  # f32 products
    vals = np.concatenate([hist_v, sv[1][None].astype(np.float64)])
    np.testing.assert_allclose(out2[1], vals.mean(0), rtol=1e-12, atol=1e-12)
    # One dominant score: the output is that token's value.
    q3 = q.copy()
    q3[2] = sk[2] * 1e4
    out3 = oracle.attention(q3, kc, vc, ks, vs, sk, sv, past, heads)
    np.testing.assert_allclose(out3[2], sv[2], rtol=1e-9, atol=1e-9)
    # Permuting the history tokens changes nothing; scaling all values scales the output.
    perm = rng.permutation(50)
    out4 = oracle.attention(q, kc[:, perm], vc[:, perm], ks[:, perm], vs[:, perm], sk, sv, past, heads)
    np.testing.assert_allclose(out4[:3], out[:3], rtol=1e-12, atol=1e-12)
    out5 = oracle.attention(q, kc, vc, ks, vs * 2, sk, sv * 2, past, heads)
    np.testing.assert_allclose(out5[:3], 2 * out[:3], rtol=1e-12, atol=1e-12)


def _planted_drop_current(q, kc, vc, ks, vs, sk, sv, past, heads):
    """A plausible mistake: attend over the history only (forget the current token)."""
    rows, cap, d = kc.shape
    out = _numpy_attention(q, kc, vc, ks, vs, sk, sv, past, heads, 1 / math.sqrt(d))
    for r in range(rows):
        p = int(past[r // heads])
        if 0 < p <= cap:
            kd = kc[r, :p].view(np.int8).astype(np.float64) * ks[r, :p, None]
            vd = vc[r, :p].view(np.int8).astype(np.float64) * vs[r, :p, None]
            s = kd @ q[r] / math.sqrt(d)
            w = np.exp(s - s.max())
            out[r] = w @ vd / w.sum()
    return out


def test_pins_catch_planted_attention_mistakes():
    rng = np.random.default_rng(SEED + 6)
    args = _problem(rng, 4, 1, 50, 64, [0, 50, 20, 7], heavy=False)
    good = oracle.attention(*args, 1)
    bad = _planted_drop_current(*args, 1)
    assert np.abs(bad[1:] - good[1:]).max() > 1e-3
    # A transposed scale convention (1/sqrt(d) applied twice) is visible too.
    twice = oracle.attention(*args, 1, scale=1 / 64)
    assert np.abs(twice - good)[1:].max() > 1e-3


def test_reference_known_answer_ii():
    """int8_kv_ops.rs:63-74, bf16-rounded history, the reference's own 2e-5 tolerance."""
    g = golden("kat_attention_ii.npz")
    got = oracle.attention(g["q"], g["codes"], g["codes"], g["scales"], g["scales"], g["scratch"], g["scratch"],
                           g["past"], int(g["heads"]), scale=0.125, history_bf16=True)
    assert np.abs(got - g["expected_bf16_history"]).max() < 2e-5


def test_reference_known_answer_iii_and_splits():
    """int8_kv_ops.rs:75-101: two heads per sequence, an empty history, unequal lengths; the reference
    kernel's own f32 split-K arithmetic at splits 32 and 128 agrees with the oracle at 2e-5."""
    g = golden("kat_attention_iii.npz")
    args = (g["q"], g["k_codes"], g["v_codes"], g["k_scales"], g["v_scales"], g["sk"], g["sv"], g["past"])
    heads = int(g["heads"])
    got = oracle.attention(*args, heads, scale=0.125, history_bf16=True)
    assert np.abs(got - g["expected_bf16_history"]).max() < 2e-5
    for split in (32, 128):
        sk_out = oracle.attention_splitk_reference(*args, heads, split, scale=0.125)
        assert np.abs(sk_out - got).max() < 2e-5


def test_cpu_baseline_matches_oracle():
    rng = np.random.default_rng(SEED + 7)
    args = _problem(rng, 8, 4, 300, 128, [0, 299])
    ref = oracle.attention(*args, 4)
    for threads in (1, 3):
        got = oracle.cpu_baseline(*args, 4, threads)
        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6)


def test_cpu_baseline_thread_pool_reuse():
    """The baseline's worker threads persist between calls: calls that ask for more threads than before, fewer,
    more than there are rows, and one, give the same rows bit for bit (each row is computed by one thread)."""
    rng = np.random.default_rng(SEED + 8)
    args = _problem(rng, 8, 2, 200, 64, [0, 199, 57, 200])
    first = oracle.cpu_baseline(*args, 2, 1)
    assert np.isfinite(first).all()
    for threads in (5, 2, 16, 3, 40, 1, 8):
        assert np.array_equal(oracle.cpu_baseline(*args, 2, threads), first), threads
    k = rng.standard_normal((8, 70, 64)).astype(np.float32)
    v = rng.standard_normal((8, 70, 64)).astype(np.float32)
    fgot = [oracle.cpu_baseline_float(args[0], k, v, threads=t) for t in (1, 6, 2, 9)]
    assert all(np.array_equal(fgot[0], x) for x in fgot[1:])


def test_bf16_helpers_match_torch():
    x = np.random.default_rng(SEED).standard_normal(10000).astype(np.float32) * 100
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(to_bf16_bits(x), ref)
    assert np.array_equal(bf16_bits_to_f32(ref), torch.from_numpy(x).to(torch.bfloat16).float().numpy())
