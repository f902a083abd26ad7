"""GPU parity of the float path's fused decode step (ppk_float_decode_step): the current token written at
slot lengths[b] of the bf16 / f32 store, then attention over the stored tokens plus it.

Expected values: the store as the reference's caller leaves it after its scatter_set of the current token
(app/src/model/graph_decode.rs:290-292: the new K/V rounded to the store's dtype at slot lengths[b]), and
the f64 oracle of the float attention over lengths + 1 tokens (graph_decode.rs:253,298-305). Bars as the
float path's: max abs <= 1e-4 and max rel <= 1e-2 (|oracle| >= 1e-3); the written slot bit-exact, every
other byte of the store untouched; rows whose slot is past the store (not written, PPK_FLAG_OVERFLOW) or
past max_length give NaN.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import ppk
from helpers import SEED, assert_close, bf16_bits_to_f32, to_bf16_bits
from test_gpu_float_attention import ATOL, RTOL, FloatCase

pytestmark = pytest.mark.gpu

_NP = {torch.float32: np.float32, torch.float16: np.float16}


class StepCase(FloatCase):
    """A seeded store of `size` tokens per row, `lengths` of them live, and the current token per row."""

    def __init__(self, device, B, H, D, size, kv, lengths, new_dtype=torch.float32, seed=SEED):
        super().__init__(device, B, H, D, size, kv, lengths=lengths, seed=seed)
        rng = np.random.default_rng(seed + 77)
        k32 = rng.standard_normal((self.rows, D), dtype=np.float32)
        v32 = rng.standard_normal((self.rows, D), dtype=np.float32)
        if new_dtype == torch.bfloat16:
            kb, vb = to_bf16_bits(k32), to_bf16_bits(v32)
            self.k_new = torch.from_numpy(kb.view(np.int16)).to(device).view(torch.bfloat16)
            self.v_new = torch.from_numpy(vb.view(np.int16)).to(device).view(torch.bfloat16)
            k32, v32 = bf16_bits_to_f32(kb), bf16_bits_to_f32(vb)
        else:
            k32 = k32.astype(_NP[new_dtype]).astype(np.float32)
            v32 = v32.astype(_NP[new_dtype]).astype(np.float32)
            self.k_new = torch.from_numpy(k32.astype(_NP[new_dtype])).to(device)
            self.v_new = torch.from_numpy(v32.astype(_NP[new_dtype])).to(device)
        # The values the store holds once the token is written (its dtype's rounding).
        self.k_cur = to_bf16_bits(k32) if kv == torch.bfloat16 else k32
        self.v_cur = to_bf16_bits(v32) if kv == torch.bfloat16 else v32
        self.before = (self.k.cpu().clone(), self.v.cpu().clone())

    def expected_store(self):
        k, v = self.k_host.copy(), self.v_host.copy()
        for r in range(self.rows):
            p = int(self.lengths[r // self.H])
            if p < self.size:
                k[r, p], v[r, p] = self.k_cur[r], self.v_cur[r]
        return k, v

    def expected(self, max_length=0):
        k, v = self.expected_store()
        n = self.lengths.astype(np.uint64) + 1
        ref = oracle.attention_float(self.q32, k, v, np.minimum(n, 2 ** 32 - 1).astype(np.uint32), self.H)
        span = max_length or self.size
        ref[np.repeat((self.lengths >= self.size) | (n > span), self.H)] = np.nan
        return ref

    def step(self, **kw):
        flags = torch.zeros(1, dtype=torch.int32, device=self.q.device)
        out = ppk.fused_attention.decode_step(self.q, self.k, self.v, self.lengths_t, self.H, self.k_new, self.v_new,
                                              flags=flags, **kw)
        torch.cuda.synchronize()
        return out.float().reshape(self.rows, self.D).cpu().numpy(), int(flags.item())

    def check_store(self):
        """The written slots hold the expected values bit for bit and nothing else moved."""
        k, v = self.expected_store()
        for got, exp in ((self.k, k), (self.v, v)):
            g = got.cpu()
            g = g.view(torch.int16).numpy().view(np.uint16) if g.dtype == torch.bfloat16 else g.numpy()
            np.testing.assert_array_equal(g.view(np.uint8), np.ascontiguousarray(exp).view(np.uint8))


@pytest.mark.parametrize("kv", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("d", [64, 128, 256])
def test_step_per_row_plan(device, kv, d):
    """Ragged lengths with an empty row, a row one short of the store and a full row (its slot is past the
    store: not written, flagged, NaN)."""
    lengths = [0, 511, 300, 512, 7, 130]
    c = StepCase(device, 6, 4, d, 512, kv, lengths, seed=SEED + d)
    got, flags = c.step()
    assert flags & ppk.PPK_FLAG_OVERFLOW
    assert_close(got, c.expected(), atol=ATOL, rtol=RTOL, what=f"step d{d} {kv}")
    c.check_store()


@pytest.mark.parametrize("kv", [torch.bfloat16, torch.float32])
def test_step_rows_across_blocks(device, kv):
    """Few long rows: the per-row plan splits each over many blocks and the merge kernel folds the current
    token."""
    c = StepCase(device, 1, 2, 128, 4096, kv, [3000], seed=SEED + 11)
    a, _ = ppk.fused_attention.decode_attention_args(c.q, c.k, c.v, c.lengths_t, c.H)
    assert ppk.fused_attention.plan(a, ppk.context(device))[1] > 1, "rows span several blocks"
    got, flags = c.step()
    assert flags == 0
    assert_close(got, c.expected(), atol=ATOL, rtol=RTOL, what=f"step across blocks {kv}")
    c.check_store()


@pytest.mark.parametrize("kv", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("d", [64, 256])
def test_step_balanced_plan(device, kv, d):
    """The balanced plan (forced): one-unit rows folding the token in the decode launch beside multi-unit
    rows folding it in the merge; empty and full rows."""
    lengths = [0, 1500, 3, 64, 1000, 1536, 65, 900]
    c = StepCase(device, 8, 4, d, 1536, kv, lengths, seed=SEED + 12 + d)
    a, _ = ppk.fused_attention.decode_attention_args(c.q, c.k, c.v, c.lengths_t, c.H, lengths_host=lengths,
                                                     plan="balanced")
    assert ppk.fused_attention.plan(a, ppk.context(device))[1] > 1
    got, flags = c.step(lengths_host=lengths, plan="balanced")
    assert flags & ppk.PPK_FLAG_OVERFLOW
    assert_close(got, c.expected(), atol=ATOL, rtol=RTOL, what=f"balanced step d{d} {kv}")
    c.check_store()


@pytest.mark.parametrize("kv", [torch.bfloat16, torch.float32])
def test_step_balanced_plan_stale_host_lengths(device, kv):
    """The balanced step with host lengths that differ from the stored ones for two sequences (one longer,
    one shorter than the host copy): those rows give NaN and the step's flags carry PPK_FLAG_STALE_LENGTHS;
    every other row is exact, and every row's token is still written at its device length."""
    lengths = [0, 1500, 3, 64, 1000, 1400, 65, 900]
    host = [0, 1500, 3, 64, 1100, 1400, 65, 700]
    c = StepCase(device, 8, 4, 128, 1536, kv, lengths, seed=SEED + 14)
    got, flags = c.step(lengths_host=host, plan="balanced")
    bad = np.repeat(np.array(host) != np.array(lengths), c.H)
    assert flags & ppk.PPK_FLAG_STALE_LENGTHS
    assert np.isnan(got[bad]).all()
    assert_close(got[~bad], c.expected()[~bad], atol=ATOL, rtol=RTOL, what=f"balanced step fresh rows {kv}")
    c.check_store()
    # The same store with the right host copy: no flag.
    c2 = StepCase(device, 8, 4, 128, 1536, kv, lengths, seed=SEED + 15)
    got2, flags2 = c2.step(lengths_host=lengths, plan="balanced")
    assert not flags2 & ppk.PPK_FLAG_STALE_LENGTHS
    assert_close(got2, c2.expected(), atol=ATOL, rtol=RTOL, what=f"balanced step {kv}")


def test_step_balanced_plan_taken_by_the_library(device):
    """A ragged batch the library balances by itself (host lengths, auto plan)."""
    lengths = [4000, 200, 200, 3900] + [100] * 28
    c = StepCase(device, 32, 8, 64, 4096, torch.bfloat16, lengths, seed=SEED + 13)
    auto, _ = ppk.fused_attention.decode_attention_args(c.q, c.k, c.v, c.lengths_t, c.H, lengths_host=lengths)
    per_row, _ = ppk.fused_attention.decode_attention_args(c.q, c.k, c.v, c.lengths_t, c.H)
    ctx = ppk.context(device)
    assert ppk.fused_attention.plan(auto, ctx) != ppk.fused_attention.plan(per_row, ctx)
    got, _ = c.step(lengths_host=lengths)
    assert_close(got, c.expected(), atol=ATOL, rtol=RTOL, what="auto balanced step")
    c.check_store()


@pytest.mark.parametrize("new_dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_step_new_token_dtypes(device, new_dtype):
    lengths = [100, 0, 255]
    for kv in (torch.bfloat16, torch.float32):
        c = StepCase(device, 3, 2, 128, 256, kv, lengths, new_dtype=new_dtype, seed=SEED + 14)
        got, _ = c.step()
        assert_close(got, c.expected(), atol=ATOL, rtol=RTOL, what=f"new {new_dtype} into {kv}")
        c.check_store()


def test_step_rows_past_max_length_give_nan(device):
    lengths = [10, 60, 49, 50]
    c = StepCase(device, 4, 2, 64, 128, torch.float32, lengths, seed=SEED + 15)
    got, _ = c.step(max_length=50)
    ref = c.expected(max_length=50)
    assert np.isnan(got[2:4]).all() and np.isnan(got[6:8]).all() and not np.isnan(got[0:2]).any()
    assert_close(got, ref, atol=ATOL, rtol=RTOL, what="step within max_length")
    c.check_store()  # rows past max_length are still written (their slot is inside the store)


def test_step_equals_write_then_attention(device):
    """The step against the reference's own sequence run on the device: the token written into the store,
    then ppk_float_decode_attention over lengths + 1."""
    lengths = [700, 0, 1023, 64]
    c = StepCase(device, 4, 4, 128, 1024, torch.bfloat16, lengths, seed=SEED + 16)
    got, _ = c.step()
    k_after, v_after = c.k.clone(), c.v.clone()
    plus = (c.lengths_t + 1).contiguous()
    out = ppk.fused_attention.decode_attention(c.q, k_after, v_after, plus, c.H)
    torch.cuda.synchronize()
    two_calls = out.float().reshape(c.rows, c.D).cpu().numpy()
    assert_close(got, two_calls, atol=ATOL, rtol=RTOL, what="fused vs write + attention")


def test_prepared_step_replays_in_a_graph(device):
    """FloatDecodeStep builds its block once; a HIP graph of it replays bit for bit (the same token written
    again at the same slot)."""
    lengths = [500, 20, 333]
    c = StepCase(device, 3, 4, 64, 512, torch.bfloat16, lengths, seed=SEED + 17)
    st = ppk.FloatDecodeStep(c.q, c.k, c.v, c.lengths_t, c.H, c.k_new, c.v_new)
    eager = st().clone()
    torch.cuda.synchronize()
    assert_close(eager.reshape(c.rows, c.D).cpu().numpy(), c.expected(), atol=ATOL, rtol=RTOL, what="prepared")
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
    c.check_store()


def test_step_refuses_missing_lengths(device):
    """The step needs the device lengths: the binding refuses None, and the library refuses a block without
    them (status 1, nothing enqueued: the store is untouched)."""
    import ctypes

    c = StepCase(device, 1, 2, 64, 64, torch.float32, [10], seed=SEED + 18)
    with pytest.raises(ValueError):
        ppk.fused_attention.decode_step(c.q, c.k, c.v, None, c.H, c.k_new, c.v_new)
    a, _ = ppk.fused_attention.decode_attention_args(c.q, c.k, c.v, c.lengths_t, c.H)
    step = ppk.fused_attention._step_args(a, c.k_new, c.v_new, None, c.lengths_t)
    step.attn.lengths = None
    lib = ppk._abi.lib()
    assert lib.ppk_float_decode_step(ppk.context(device), None, ctypes.byref(step)) == ppk._abi.PPK_PRECONDITION
    assert "lengths" in ppk._abi.last_error()
    torch.cuda.synchronize()
    assert torch.equal(c.k.cpu(), c.before[0]) and torch.equal(c.v.cpu(), c.before[1])
