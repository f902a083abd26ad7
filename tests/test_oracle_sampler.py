"""Pins of the oracle's CFG + Renyi sampler (oracle_renyi_sample), CPU only.

The oracle restates the reference's host validation oracle
(app/src/inference/hip_sampling_reference.rs:12-141) of pp_hip_renyi_sample
(app/src/inference/renyi_sample.hip:23-204). Pinned here by the reference's
own known answers (hip_sampling_reference.rs:143-205), by the definition of
the Renyi entropy of order alpha computed in float64
(H_a = log(sum p^a) / (1 - a)), by numpy's lexsort for the candidate order,
and by closed forms (a uniform head has support = count; k equal leaders
far above the rest have support k for every alpha). Planted mistakes in a
numpy copy (Shannon entropy, descending index ties, swapped CFG operands)
disagree with the oracle on the same inputs.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from helpers import SEED

F32_MAX = np.finfo(np.float32).max


def test_reference_known_answer_uniform_support_and_index_ties():
    """hip_sampling_reference.rs:147-168."""
    for count in [1, 2, 127, 128, 255, 256, 270, 1024, 2048]:
        for alpha in [1.25, 3.5, 4.0, 7.0, 32.0]:
            raw = np.zeros((4, count), np.float32)
            u = np.array([0.0, 0.25, 0.75, np.float32(0.99999994)], np.float32)
            bounds = np.tile(np.array([0, count], np.uint32), (4, 1))
            r = oracle.renyi_sample(raw, u, bounds, alpha, 1.0, 1, 100)
            for row in range(4):
                expect = 100 + min(int(np.float32(u[row]) * np.float32(count)), count - 1)
                assert (r["token"][row], r["valid"][row], r["support"][row]) == (expect, 1, count)


def test_reference_known_answer_guided_rows_and_legal_ranges():
    """hip_sampling_reference.rs:169-180: c0/u0/c1/u1 rows with restricted legal ranges."""
    raw = np.array([0, 1, 2, 3, 1, 1, 1, 1, 9, 8, 7, 6, 1, 1, 1, 1], np.float32).reshape(4, 4)
    for fma in (False, True):
        r = oracle.renyi_sample(raw, np.zeros(2, np.float32), np.array([[1, 2], [2, 2]], np.uint32), 4.0, 2.5, 2,
                                2048, cfg_fma=fma)
        assert list(r["token"]) == [2050, 2050] and list(r["valid"]) == [1, 1]


def test_cfg_value_is_a_rounded_product_then_a_rounded_sum():
    """hip_sampling_reference.rs:73 (Rust never contracts) and renyi_sample.hip:85 built with
    -ffp-contract=off (hip_kernel.rs:46): numpy's float32 u + cfg * (c - u) rounds after each operation.
    Column 0 holds that value exactly; column 1 computes it from (c, u). A fused multiply-add makes
    column 1 one ulp larger, so the two forms pick different tokens."""
    cfg = np.float32(2.5)
    u1, c1 = np.float32(0.8192756772041321), np.float32(1.6597106456756592)
    tie = np.float32(u1 + np.float32(cfg * np.float32(c1 - u1)))
    assert tie == np.float32(2.920362949371338)
    cond = np.array([tie, c1, -30.0, -30.0], np.float32)
    uncond = np.array([tie, u1, -30.0, -30.0], np.float32)
    raw = np.stack([cond, uncond, cond, uncond])
    uniforms = np.array([0.0, 0.75], np.float32)
    bounds = np.array([[0, 4], [0, 4]], np.uint32)
    r = oracle.renyi_sample(raw, uniforms, bounds, 4.0, float(cfg), 2, 0)
    assert list(r["token"]) == [0, 1] and list(r["support"]) == [2, 2]  # tie broken by index
    f = oracle.renyi_sample(raw, uniforms, bounds, 4.0, float(cfg), 2, 0, cfg_fma=True)
    assert list(f["token"]) == [1, 0]


def test_reference_known_answer_invalid_inputs():
    """hip_sampling_reference.rs:181-204: every raw logit is checked, bad uniforms, CFG overflow, bad bounds."""
    for value in [np.nan, np.inf, -np.inf]:
        r = oracle.renyi_sample(np.array([[1, 2, value]], np.float32), np.zeros(1, np.float32),
                                np.array([[0, 2]], np.uint32), 4.0, 1.0, 1, 0)
        assert (r["token"][0], r["valid"][0], r["support"][0]) == (0, 0, 1)
    for u in [1.0, -0.1, np.nan, np.inf]:
        r = oracle.renyi_sample(np.array([[1, 2]], np.float32), np.array([u], np.float32),
                                np.array([[0, 2]], np.uint32), 4.0, 1.0, 1, 0)
        assert r["valid"][0] == 0
    r = oracle.renyi_sample(np.array([[F32_MAX], [-F32_MAX]], np.float32), np.zeros(1, np.float32),
                            np.array([[0, 1]], np.uint32), 4.0, 2.0, 2, 0)
    assert r["valid"][0] == 0
    r = oracle.renyi_sample(np.zeros((1, 2), np.float32), np.zeros(1, np.float32), np.array([[2, 1]], np.uint32),
                            4.0, 1.0, 1, 0)
    assert (r["token"][0], r["valid"][0], r["support"][0]) == (0, 0, 1)


@pytest.mark.parametrize("bad", [dict(guidance=3), dict(alpha=1.0), dict(alpha=np.nan), dict(cfg=-1.0),
                                 dict(cfg=2.0, guidance=1), dict(offset=2**32 - 1)])
def test_reference_metadata_rules(bad):
    kw = dict(alpha=4.0, cfg=1.0, guidance=1, offset=0)
    kw.update(bad)
    g = kw["guidance"]
    with pytest.raises(ValueError):
        oracle.renyi_sample(np.zeros((2 * g if g in (1, 2) else 3, 16), np.float32), np.zeros(2, np.float32),
                            np.tile(np.array([0, 16], np.uint32), (2, 1)), **kw)


def renyi_support_f64(v: np.ndarray, alpha: float) -> tuple[int, float]:
    """support = clamp(floor(exp(H_alpha) + 0.5), 1, n) from the definition, and exp(H)+0.5's distance to
    the nearest integer."""
    v = v.astype(np.float64)
    p = np.exp(v - v.max())
    p /= p.sum()
    h = np.log(np.sum(p ** alpha)) / (1.0 - alpha)
    h = min(max(h, 0.0), np.log(len(v)))
    x = np.exp(h) + 0.5
    return int(min(max(np.floor(x), 1), len(v))), abs(x - np.round(x))


def lexsort_token(v: np.ndarray, start: int, rank: int) -> int:
    """rank-th candidate by (value descending, index ascending), by numpy's lexsort."""
    idx = np.arange(len(v))
    order = np.lexsort((idx, -v.astype(np.float64)))
    return start + int(order[rank])


@pytest.mark.parametrize("guidance", [1, 2])
def test_support_and_token_match_the_definition(guidance):
    rng = np.random.default_rng(SEED + guidance)
    batch, choices = 64, 700
    raw = (rng.standard_normal((batch * guidance, choices)) * rng.uniform(0.2, 6.0, (batch * guidance, 1)))
    raw = raw.astype(np.float32)
    raw[:, 5] = raw[:, 9]  # exact ties exercise the index order
    uniforms = rng.uniform(0, 1, batch).astype(np.float32)
    starts = rng.integers(0, 300, batch)
    counts = rng.integers(1, choices - starts + 1)
    bounds = np.stack([starts, counts], 1).astype(np.uint32)
    alpha, cfg = 3.5, (2.5 if guidance == 2 else 1.0)
    r = oracle.renyi_sample(raw, uniforms, bounds, alpha, cfg, guidance, 7, cfg_fma=False)
    checked = 0
    for b in range(batch):
        s, n = int(starts[b]), int(counts[b])
        c = raw[b * guidance]
        v = c if guidance == 1 else raw[b * guidance + 1] + np.float32(cfg) * (c - raw[b * guidance + 1])
        v = v.astype(np.float32)[s:s + n]
        support, dist = renyi_support_f64(v, alpha)
        assert r["valid"][b] == 1
        if dist < 1e-3:
            continue  # an f32 rounding boundary: float32 sums may round either way
        checked += 1
        assert r["support"][b] == support, b
        rank = min(int(np.float32(uniforms[b]) * np.float32(support)), support - 1)
        assert r["token"][b] == 7 + lexsort_token(v, s, rank), b
    assert checked > batch * 0.9


def test_closed_form_supports():
    # k equal leaders 80 nats above the rest: p is uniform over the leaders for every alpha.
    for k in (1, 3, 17, 200):
        for alpha in (1.5, 4.0, 30.0):
            v = np.full(1600, -80.0, np.float32)
            lead = np.arange(10, 10 + 7 * k, 7)
            v[lead] = 0.0
            r = oracle.renyi_sample(v[None], np.array([0.999], np.float32), np.array([[0, 1600]], np.uint32),
                                    alpha, 1.0, 1, 0)
            assert r["support"][0] == k
            assert r["token"][0] == lead[min(int(np.float32(0.999) * np.float32(k)), k - 1)]
    # -0.0 and +0.0 are equal logits: their order is by index.
    v = np.array([[-0.0, 0.0, -0.0, 0.0]], np.float32)
    r = oracle.renyi_sample(v, np.array([0.8], np.float32), np.array([[0, 4]], np.uint32), 4.0, 1.0, 1, 0)
    assert (r["support"][0], r["token"][0]) == (4, 3)


def _planted(v, alpha, uniform, *, shannon=False, index_desc=False):
    p = np.exp(v.astype(np.float64) - v.max())
    p /= p.sum()
    h = -np.sum(p * np.log(np.maximum(p, 1e-300))) if shannon else np.log(np.sum(p ** alpha)) / (1.0 - alpha)
    support = int(min(max(np.floor(np.exp(min(max(h, 0), np.log(len(v)))) + 0.5), 1), len(v)))
    rank = min(int(np.float32(uniform) * np.float32(support)), support - 1)
    idx = np.arange(len(v))
    order = np.lexsort(((-idx) if index_desc else idx, -v.astype(np.float64)))
    return support, int(order[rank])


def test_pins_catch_planted_sampler_mistakes():
    rng = np.random.default_rng(SEED + 11)
    v = (rng.standard_normal(300) * 2).astype(np.float32)
    v[100:140] = v[100]  # a tied block
    r = oracle.renyi_sample(v[None], np.array([0.6], np.float32), np.array([[0, 300]], np.uint32), 4.0, 1.0, 1, 0)
    good = _planted(v, 4.0, 0.6)
    assert (r["support"][0], r["token"][0]) == good
    assert _planted(v, 4.0, 0.6, shannon=True)[0] != good[0]
    tied = np.full(64, 1.0, np.float32)
    r = oracle.renyi_sample(tied[None], np.array([0.3], np.float32), np.array([[0, 64]], np.uint32), 4.0, 1.0, 1, 0)
    assert r["token"][0] == _planted(tied, 4.0, 0.3)[1] != _planted(tied, 4.0, 0.3, index_desc=True)[1]
    # Swapped CFG operands (c + cfg * (u - c)) pick another token on guided rows.
    c = rng.standard_normal(200).astype(np.float32)
    u = rng.standard_normal(200).astype(np.float32)
    r = oracle.renyi_sample(np.stack([c, u]), np.array([0.0], np.float32), np.array([[0, 200]], np.uint32), 4.0,
                            3.0, 2, 0)
    assert r["token"][0] == int(np.argmax(u + np.float32(3.0) * (c - u)))
    assert r["token"][0] != int(np.argmax(c + np.float32(3.0) * (u - c)))
