"""GPU parity of the balanced plan for ragged batches (ppk_decode_flat + ppk_attn_merge_flat).

The library takes the plan by itself when the caller passes its host copy of the lengths
(PpkAttentionArgs.past_host) for a ragged batch where its timing model of both plans favours it
(test_library_balances_a_skewed_batch; the rule itself is checked on the CPU in test_abi.py); the other
tests force it with PPK_ATTN_PLAN_BALANCED (plan="balanced") so that their small shapes exercise its
kernels whatever the model picks, and assert that the forced plan differs from the per-row one.
Bars as for the per-row plan (tests/test_gpu_attention.py): against the f64
oracle, max abs error <= 2e-3 and max relative error <= 1e-2 (|oracle| >=
1e-3); the bf16-history mode within 2e-5 absolute; appended codes and scales
bit-exact; rows whose device length is invalid, or differs from the host
copy, give NaN.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import ppk
from helpers import SEED, assert_close
from test_gpu_attention import Case

pytestmark = pytest.mark.gpu


def _plan(c: Case, past_host, max_past=0, **kw):
    a, _ = ppk.int8_kv_ops.attention_args(c.q, c.kc, c.vc, c.ks, c.vs, c.sk, c.sv, c.past_t, c.H,
                                          max_past=max_past, past_host=past_host, **kw)
    return ppk.int8_kv_ops.plan(a, ppk.context(c.q.device))


BAL = "balanced"


def _balanced(c: Case, past_host, max_past=0) -> int:
    """Asserts the forced balanced plan differs from the per-row one and returns its record slots per row."""
    plan = _plan(c, past_host, max_past, plan=BAL)
    assert plan != _plan(c, None, max_past), "the balanced plan is a plan of its own"
    return plan[1]


def test_config4_ragged_balanced(device):
    """BASELINE config 4 (B=8, H=16, D=128, lengths U[256, 4096], bf16 q) through the balanced plan (the
    library itself keeps the per-row plan here: a step of under 20 us where the balanced plan's merge launch
    and short units cost more than its balance saves)."""
    lengths = [int(x) for x in np.random.default_rng(SEED).integers(256, 4097, size=8)]
    c = Case(device, 8, 16, 128, lengths, max(lengths) + 1, q_dtype=torch.bfloat16, scratch_dtype=torch.bfloat16)
    assert _balanced(c, lengths, max_past=max(lengths)) > 1, "config 4 rows span several units"
    ref = c.reference()
    assert_close(c.run(past_host=lengths, max_past=max(lengths), plan=BAL), ref, what="config 4 balanced")
    assert_close(c.run(past_host=lengths, plan=BAL), ref, what="config 4 balanced, span = capacity")
    a, _ = ppk.int8_kv_ops.attention_args(c.q, c.kc, c.vc, c.ks, c.vs, c.sk, c.sv, c.past_t, c.H,
                                          max_past=max(lengths), past_host=lengths)
    assert ppk.int8_kv_ops.plan_info(a, ppk.context(device))["kind"] == "per-row"


def test_library_balances_a_skewed_batch(device):
    """Two sequences of 8192 tokens beside 30 of 256 (H = 8, D = 64): with the host lengths the library
    itself takes the balanced plan (at H = 16 measured 19.3 against 40.2 us per-row), its results within the
    bars."""
    lengths = [8192] * 2 + [256] * 30
    c = Case(device, 32, 8, 64, lengths, 8193, q_dtype=torch.bfloat16, scratch_dtype=torch.bfloat16)
    auto = _plan(c, lengths)
    assert auto == _plan(c, lengths, plan=BAL) != _plan(c, None)
    assert_close(c.run(past_host=lengths), c.reference(), what="library-chosen balanced plan")


@pytest.mark.parametrize("d", [64, 128, 256])
def test_edge_lengths_balanced(device, d):
    """Empty rows, one-token rows, rows at the capacity, rows past it (NaN), single-unit rows beside rows
    of many units."""
    lengths = [0, 1, 700, 2000, 2049, 3, 2048, 5000] + [2000] * 4 + [10] * 20
    c = Case(device, 32, 8, d, lengths, 2048)
    assert _balanced(c, lengths) > 1
    got = c.run(past_host=lengths, plan=BAL)
    ref = c.reference()
    bad = np.repeat(np.array(lengths) > 2048, 8)
    assert np.isnan(got[bad]).all() and not np.isnan(got[~bad]).any()
    assert_close(got, ref, what=f"edge lengths d={d}")


def test_rows_beyond_max_past_give_nan(device):
    lengths = [900, 1200, 40, 1100, 30, 950, 20, 10] * 4
    c = Case(device, 32, 8, 128, lengths, 1500)
    _balanced(c, lengths, max_past=1000)
    got = c.run(past_host=lengths, max_past=1000, plan=BAL)
    ref = c.reference()
    bad = np.repeat(np.array(lengths) > 1000, 8)
    assert np.isnan(got[bad]).all() and not np.isnan(got[~bad]).any()
    assert_close(got[~bad], ref[~bad], what="rows within max_past")


def test_short_rows_keep_the_per_row_plan(device):
    """Short ragged rows: one block per row puts every row on a CU of its own, so the host lengths keep the
    per-row plan (one launch, no merge), sized for the longest live row (64 tokens: one wave) instead of the
    span (900: eight 128-token waves, an int8 block's most)."""
    lengths = [10, 0, 60, 64]
    c = Case(device, 4, 16, 64, lengths, 1024)
    assert _plan(c, lengths, max_past=900) == (64, 1, 0)
    assert _plan(c, None, max_past=900) == (128, 1, 0)
    ppk.kernel_stats(ppk.PPK_KERNEL_ATTN_MERGE, reset=True)
    ppk.set_profiling(True)
    got = c.run(past_host=lengths, max_past=900)
    ppk.set_profiling(False)
    assert ppk.kernel_stats(ppk.PPK_KERNEL_ATTN_MERGE, reset=True)[0] == 0
    assert_close(got, c.reference(), what="one-unit rows")


def test_bf16_history_balanced(device):
    """The reference-exact mode (history rounded through bf16, int8_kv.cu:23-27) at the reference's 2e-5."""
    lengths = [900, 30, 2500, 1700]
    c = Case(device, 4, 8, 64, lengths, 2600)
    _balanced(c, lengths)
    got = c.run(past_host=lengths, bf16_history=True, plan=BAL)
    assert_close(got, c.reference(history_bf16=True), atol=2e-5, rtol=0, what="balanced bf16 history")


@pytest.mark.parametrize("q_dtype,out_dtype", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                                (torch.float16, torch.float16)])
def test_balanced_dtypes(device, q_dtype, out_dtype):
    lengths = [1500, 333, 2900]
    c = Case(device, 3, 8, 128, lengths, 3000, q_dtype=q_dtype, scratch_dtype=q_dtype)
    _balanced(c, lengths)
    got = c.run(past_host=lengths, out_dtype=out_dtype, plan=BAL)
    narrow = {torch.float32: None, torch.bfloat16: "bf16", torch.float16: "f16"}[out_dtype]
    assert_close(got, c.reference(), what=f"balanced {q_dtype} -> {out_dtype}", out_dtype=narrow)


def test_decode_step_balanced_appends_and_attends(device):
    """The fused step over the balanced plan: each row's new token quantised into slot past[b] (bit-exact
    against the oracle), attention over the pre-append history plus the current token."""
    lengths = [2047, 0, 610, 1300, 2048]
    B, H, D, cap = 5, 8, 128, 2048
    c = Case(device, B, H, D, lengths, cap, q_dtype=torch.bfloat16, scratch_dtype=torch.bfloat16)
    _balanced(c, lengths)
    ref = c.reference()
    before = [t.clone() for t in (c.kc, c.vc, c.ks, c.vs)]
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    out = ppk.decode_step(c.q, c.kc, c.vc, c.ks, c.vs, c.sk, c.sv, c.past_t, H, flags=flags, past_host=lengths,
                          plan=BAL)
    torch.cuda.synchronize()
    assert_close(out.reshape(c.rows, D).cpu().numpy(), ref, what="balanced decode step")
    assert int(flags.item()) & ppk.PPK_FLAG_OVERFLOW  # the row at the capacity could not append
    for src, codes, scales, old in ((c.sk32, c.kc, c.ks, before[0]), (c.sv32, c.vc, c.vs, before[1])):
        exp_c, exp_s, _ = oracle.quantize(src.reshape(c.rows, 1, D))
        got_c, got_s = codes.cpu().numpy(), scales.cpu().numpy()
        for b, p in enumerate(lengths):
            rows = slice(b * H, (b + 1) * H)
            if p < cap:
                assert np.array_equal(got_c[rows, p], exp_c[rows, 0])
                assert np.array_equal(got_s[rows, p].view(np.uint32), exp_s[rows, 0].view(np.uint32))
    # Nothing else in the arenas moved.
    for got, old in zip((c.kc, c.vc), before[:2]):
        g, o = got.cpu().numpy(), old.cpu().numpy()
        for b, p in enumerate(lengths):
            if p < cap:
                g[b * H:(b + 1) * H, p] = o[b * H:(b + 1) * H, p]
        assert np.array_equal(g, o)


def test_stale_host_lengths_give_nan_and_a_flag(device):
    """A host copy that no longer matches the device's lengths never yields a wrong row: the sequences whose
    device value differs give NaN and the step's flags carry PPK_FLAG_STALE_LENGTHS; the others stay right."""
    lengths = [1500, 700, 2000, 20] + [1900] * 2 + [30] * 26
    c = Case(device, 32, 8, 128, lengths, 2100)
    stale = [1500, 650, 2000, 21] + lengths[4:]  # sequences 1 and 3 differ
    _balanced(c, stale)
    ref = c.reference()
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    out = ppk.decode_step(c.q, c.kc, c.vc, c.ks, c.vs, c.sk, c.sv, c.past_t, c.H, flags=flags, past_host=stale,
                          plan=BAL)
    torch.cuda.synchronize()
    got = out.reshape(c.rows, c.D).cpu().numpy()
    bad = np.repeat(np.array(lengths) != np.array(stale), 8)
    assert np.isnan(got[bad]).all()
    assert_close(got[~bad], ref[~bad], what="fresh sequences beside stale ones")
    assert int(flags.item()) & ppk.PPK_FLAG_STALE_LENGTHS


def test_balanced_plan_through_the_noalloc_entry_point(device):
    """ppk_decode_step_noalloc takes the same balanced plan (host lengths in the argument block)."""
    import ctypes

    from ppk import _abi

    lengths = [3000, 120, 1800] + [50] * 29
    c = Case(device, 32, 8, 128, lengths, 3001, q_dtype=torch.bfloat16, scratch_dtype=torch.bfloat16)
    _balanced(c, lengths)
    ref = c.reference()
    a, out = ppk.int8_kv_ops.attention_args(c.q, c.kc, c.vc, c.ks, c.vs, c.sk, c.sv, c.past_t, c.H,
                                            past_host=lengths, plan=BAL)
    step = ppk.int8_kv_ops._step_args(a, c.sk, c.sv, None, c.D)
    stream = ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
    assert _abi.lib().ppk_decode_step_noalloc(ppk.context(device), stream, ctypes.byref(step)) == 0, _abi.last_error()
    torch.cuda.synchronize()
    assert_close(out.reshape(c.rows, c.D).cpu().numpy(), ref, what="balanced no-alloc")


def test_balanced_step_captured_in_a_hip_graph(device):
    """A prepared balanced step replays in a HIP graph bit for bit (the table travels in the kernel
    arguments; no memset)."""
    lengths = [2500, 64, 900, 1700]
    c = Case(device, 4, 16, 128, lengths, 2600, q_dtype=torch.bfloat16, scratch_dtype=torch.bfloat16)
    _balanced(c, lengths)
    st = ppk.DecodeAttention(c.q, c.kc, c.vc, c.ks, c.vs, c.sk, c.sv, c.past_t, c.H, past_host=lengths, plan=BAL)
    eager = st().clone()
    torch.cuda.synchronize()
    assert_close(eager.reshape(c.rows, c.D).cpu().numpy(), c.reference(), what="balanced eager")
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        st(side)
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        st()
    for _ in range(3):
        st.out.fill_(float("nan"))
        junk = torch.randn(1 << 20, device=device).sin_().sum()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(junk)
        assert torch.equal(st.out, eager)
