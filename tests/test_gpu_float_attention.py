"""GPU parity of the float-KV decode attention (ppk_float_decode_attention)
against the f64 oracle (oracle_attention_float).

Bar: max |gpu - oracle| <= 1e-4, the reference's own acceptance bar for this
kernel pair (hip_attention::validate_split_k, app/src/model/hip_attention.rs:36-41),
and max relative error <= 1e-2 over |oracle| >= 1e-3, each checked on its own;
fp32 accumulation over up to 8192 tokens stays well inside both.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import ppk
from helpers import SEED, assert_close, bf16_bits_to_f32, to_bf16_bits

pytestmark = pytest.mark.gpu
ATOL, RTOL = 1e-4, 1e-2


class FloatCase:
    """A seeded float-KV store [rows, cap, D] on the device; rows attend `lengths` (or the whole view)."""

    def __init__(self, device, B, H, D, size, kv_dtype, lengths=None, cap=None, seed=SEED):
        rng = np.random.default_rng(seed)
        self.B, self.H, self.D, self.size = B, H, D, size
        self.rows = rows = B * H
        cap = cap or size
        k32 = rng.standard_normal((rows, cap, D), dtype=np.float32)
        v32 = rng.standard_normal((rows, cap, D), dtype=np.float32)
        self.q32 = rng.standard_normal((rows, 1, D), dtype=np.float32)
        if kv_dtype == torch.bfloat16:
            self.k_host, self.v_host = to_bf16_bits(k32), to_bf16_bits(v32)
            self.k = torch.from_numpy(self.k_host.view(np.int16)).to(device).view(torch.bfloat16)
            self.v = torch.from_numpy(self.v_host.view(np.int16)).to(device).view(torch.bfloat16)
        else:
            self.k_host, self.v_host = k32, v32
            self.k, self.v = torch.from_numpy(k32).to(device), torch.from_numpy(v32).to(device)
        self.k, self.v = self.k[:, :size], self.v[:, :size]  # a narrowed view when cap > size
        self.k_host, self.v_host = self.k_host[:, :size], self.v_host[:, :size]
        self.q = torch.from_numpy(self.q32).to(device)
        self.lengths = None if lengths is None else np.asarray(lengths, np.uint32)
        self.lengths_t = None if lengths is None else torch.from_numpy(self.lengths.view(np.int32)).to(device)

    def run(self, split=0, q=None, **kw):
        out = ppk.fused_attention.decode_attention(self.q if q is None else q, self.k, self.v, self.lengths_t,
                                                   self.H, split, **kw)
        torch.cuda.synchronize()
        return out.float().reshape(self.rows, self.D).cpu().numpy()

    def reference(self, scale=None):
        return oracle.attention_float(self.q32, self.k_host, self.v_host, self.lengths, self.H, scale=scale)


@pytest.mark.parametrize("kv", [torch.bfloat16, torch.float32])
def test_reference_graph_decode_shape(device, kv):
    """graph_decode.rs:298-305: a 1024-token store per row, D = 64, ragged valid lengths."""
    c = FloatCase(device, 4, 16, 64, 1024, kv, lengths=[1, 300, 1024, 777])
    assert_close(c.run(), c.reference(), atol=ATOL, rtol=RTOL, what=f"graph decode {kv}")
    # The reference's Split-K setting (split_tokens = 128) gives the same result.
    assert_close(c.run(128), c.reference(), atol=ATOL, rtol=RTOL, what=f"graph decode split 128 {kv}")


@pytest.mark.parametrize("kv", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("d", [64, 128, 256])
def test_head_dims_and_dtypes(device, kv, d):
    c = FloatCase(device, 2, 4, d, 513, kv, lengths=[513, 200], seed=SEED + d)
    assert_close(c.run(), c.reference(), atol=ATOL, rtol=RTOL, what=f"d{d} {kv}")


@pytest.mark.parametrize("kv", [torch.bfloat16, torch.float32])
def test_no_lengths_attends_the_whole_view(device, kv):
    """mod.rs:713-714 and batch.rs:207: lengths = None, the view's length is the attended length."""
    c = FloatCase(device, 1, 16, 64, 257, kv, seed=SEED + 5)
    assert_close(c.run(), c.reference(), atol=ATOL, rtol=RTOL, what="no lengths")


def test_narrowed_store_and_strided_query(device):
    """Row strides: K/V narrowed from a larger store, q a slice of a packed [rows, 3, D] tensor."""
    c = FloatCase(device, 2, 8, 128, 300, torch.bfloat16, lengths=[300, 123], cap=512, seed=SEED + 6)
    assert c.k.stride(0) == 512 * 128 and not c.k.is_contiguous()
    packed = torch.randn((c.rows, 3, c.D), device=device)
    packed[:, 1:2] = c.q
    q = packed[:, 1:2]
    assert q.stride(0) == 3 * c.D
    assert_close(c.run(q=q), c.reference(), atol=ATOL, rtol=RTOL, what="strided views")


def test_invalid_lengths_give_nan(device):
    c = FloatCase(device, 4, 2, 64, 100, torch.float32, lengths=[0, 100, 101, 37], seed=SEED + 7)
    got = c.run()
    ref = c.reference()
    assert np.isnan(got[0:2]).all() and np.isnan(got[4:6]).all()
    assert np.isnan(ref[0:2]).all() and np.isnan(ref[4:6]).all()
    ok = np.r_[2:4, 6:8]
    assert_close(got[ok], ref[ok], atol=ATOL, rtol=RTOL, what="valid rows")
    # max_length bounds the plan; a row beyond it gives NaN rather than a wrong value.
    got = c.run(max_length=50)
    assert np.isnan(got[2:4]).all()
    assert_close(got[6:8], ref[6:8], atol=ATOL, rtol=RTOL, what="rows within max_length")


@pytest.mark.parametrize("split", [0, 32, 100, 512])
def test_split_invariance(device, split):
    c = FloatCase(device, 2, 4, 128, 2000, torch.bfloat16, lengths=[2000, 1111], seed=SEED + 8)
    assert_close(c.run(split), c.reference(), atol=ATOL, rtol=RTOL, what=f"split {split}")


@pytest.mark.parametrize("kv", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("split", [0, 100, 1000])
def test_rotated_batch_order_counts_every_token_once(device, kv, split):
    """Each wave takes its batches in its own rotated order, wrapping at its last batch. Here the stores hold
    exactly 4096 tokens (power-of-two row strides), the lengths leave odd batch counts and partial last
    batches, and the splits give waves of 4 to 32 batches. With q = 0 every score is equal, so each row's
    output is the plain mean of its V rows: a batch skipped or taken twice moves it by about 1e-3."""
    lengths = [4096, 4095, 1000, 33]
    c = FloatCase(device, 4, 16, 64, 4096, kv, lengths=lengths, seed=SEED + 41)
    assert c.k.stride(0) == 4096 * 64
    assert_close(c.run(split), c.reference(), atol=ATOL, rtol=RTOL, what=f"split {split} {kv}")
    v = (bf16_bits_to_f32(c.v_host) if kv == torch.bfloat16 else c.v_host).astype(np.float64)
    mean = np.stack([v[r, :lengths[r // c.H]].mean(axis=0) for r in range(c.rows)])
    got = c.run(split, q=torch.zeros_like(c.q))
    np.testing.assert_allclose(got, mean, rtol=0, atol=1e-5)


def test_output_and_query_dtypes(device):
    c = FloatCase(device, 2, 4, 64, 333, torch.bfloat16, lengths=[333, 64], seed=SEED + 9)
    f32 = c.run()
    for dt in (torch.bfloat16, torch.float16):
        out = ppk.fused_attention.decode_attention(c.q, c.k, c.v, c.lengths_t, c.H, out_dtype=dt)
        torch.cuda.synchronize()
        # Same arithmetic, rounded once at the store.
        expect = torch.from_numpy(f32).to(dt).float().numpy()
        np.testing.assert_array_equal(out.float().reshape(c.rows, c.D).cpu().numpy(), expect)
    # A bf16 query computes exactly what an f32 query holding the same values computes.
    qb = c.q.to(torch.bfloat16)
    np.testing.assert_array_equal(c.run(q=qb), c.run(q=qb.float()))


def test_softmax_scale(device):
    c = FloatCase(device, 1, 4, 64, 200, torch.float32, seed=SEED + 10)
    assert_close(c.run(softmax_scale=0.37), c.reference(scale=0.37), atol=ATOL, rtol=RTOL, what="scale")


@pytest.mark.parametrize("kv", [torch.bfloat16, torch.float32])
def test_reference_split_k_validation(device, kv):
    """hip_attention::validate_split_k (hip_attention.rs:18-45): a 257-token store, split 0 and 128
    agree with the f32 softmax reference within 1e-4, and zeros give zero (mod.rs:440-451)."""
    from test_oracle_float import reference_kat_inputs

    bf16 = kv == torch.bfloat16
    q, k, v = reference_kat_inputs(bf16)
    dev = lambda a: (torch.from_numpy(a.view(np.int16)).to(device).view(torch.bfloat16) if bf16
                     else torch.from_numpy(a).to(device))
    qt, kt, vt = torch.from_numpy(q.reshape(1, 1, 64)).to(device), dev(k), dev(v)
    ref = oracle.attention_float(q, k, v, None, 1)
    outs = []
    for split in (0, 128):
        out = ppk.fused_attention.decode_attention(qt, kt, vt, None, 1, split)
        torch.cuda.synchronize()
        outs.append(out.reshape(1, 64).cpu().numpy())
        assert np.max(np.abs(outs[-1] - ref)) <= 1e-4
    assert np.max(np.abs(outs[0] - outs[1])) <= 1e-4
    z = torch.zeros((1, 257, 64), dtype=kv, device=device)
    out = ppk.fused_attention.decode_attention(torch.zeros((1, 1, 64), device=device), z, z, None, 1, 128)
    assert torch.all(out.abs() <= 1e-6).item()


def test_full_size_bf16_b32_h16_ctx8192_sampled_rows(device):
    """The bandwidth workload (512 rows x 8192 bf16 tokens, D = 128, 2 GiB of K+V): GPU output on
    a sample of rows against the oracle on the same rows."""
    gen = torch.Generator(device=device).manual_seed(SEED)
    rows, size, d = 32 * 16, 8192, 128
    k = torch.randn((rows, size, d), generator=gen, device=device, dtype=torch.bfloat16)
    v = torch.randn((rows, size, d), generator=gen, device=device, dtype=torch.bfloat16)
    q = torch.randn((rows, 1, d), generator=gen, device=device, dtype=torch.float32)
    lengths = torch.full((32,), size, dtype=torch.int32, device=device)
    lengths[3] = 4097
    out = ppk.fused_attention.decode_attention(q, k, v, lengths, 16)
    torch.cuda.synchronize()
    sample = np.array([0, 1, 48, 49, 63, 200, 511])
    idx = torch.from_numpy(sample).to(device)
    kh = k[idx].view(torch.int16).cpu().numpy().view(np.uint16)
    vh = v[idx].view(torch.int16).cpu().numpy().view(np.uint16)
    lh = lengths.cpu().numpy().astype(np.uint32)
    ref = np.stack([oracle.attention_float(q[r].cpu().numpy(), kh[i:i + 1], vh[i:i + 1],
                                           lh[r // 16:r // 16 + 1], 1)[0] for i, r in enumerate(sample)])
    got = out.reshape(rows, d)[idx].cpu().numpy()
    assert_close(got, ref, atol=ATOL, rtol=RTOL, what="full size sampled rows")
    assert np.isfinite(out.cpu().numpy()).all()
    del k, v


def test_rows_past_4_gib_of_their_store(device):
    """16 rows of a bf16 store of 2^21 tokens x D = 128 (8 GiB per tensor), so rows 8-15 start past 4 GiB;
    the first 600 tokens of each row hold data. Every row against the oracle."""
    B, H, D, cap = 2, 8, 128, 1 << 21
    lengths = np.array([600, 431], np.uint32)
    L = int(lengths.max())
    rows = B * H
    print(f"float rows past 4 GiB: rows={rows} D={D} cap={cap} lengths={lengths.tolist()}", flush=True)
    rng = np.random.default_rng(SEED + 62)
    kh = to_bf16_bits(rng.standard_normal((rows, L, D), dtype=np.float32))
    vh = to_bf16_bits(rng.standard_normal((rows, L, D), dtype=np.float32))
    q32 = rng.standard_normal((rows, 1, D), dtype=np.float32)
    k = torch.empty((rows, cap, D), dtype=torch.bfloat16, device=device)
    v = torch.empty_like(k)
    assert (rows - 1) * cap * D * 2 > 1 << 32
    k[:, :L] = torch.from_numpy(kh.view(np.int16)).to(device).view(torch.bfloat16)
    v[:, :L] = torch.from_numpy(vh.view(np.int16)).to(device).view(torch.bfloat16)
    lt = torch.from_numpy(lengths.view(np.int32)).to(device)
    out = ppk.fused_attention.decode_attention(torch.from_numpy(q32).to(device), k, v, lt, H, max_length=L)
    torch.cuda.synchronize()
    got = out.float().reshape(rows, D).cpu().numpy()
    assert_close(got, oracle.attention_float(q32, kh, vh, lengths, H), atol=ATOL, rtol=RTOL,
                 what="float rows past 4 GiB of the store")
    del k, v


@pytest.mark.parametrize("kv", [torch.bfloat16, torch.float32])
def test_long_rows_merge_more_than_64_groups(device, kv):
    """Two rows of 65000 live tokens: hundreds of blocks per row, so the merge takes its second pass over
    the (m, z) records beyond the first 64."""
    c = FloatCase(device, 1, 2, 128, 65536, kv, lengths=[65000], seed=SEED + 22)
    call = ppk.FloatDecodeAttention(c.q, c.k, c.v, c.lengths_t, c.H)
    assert call.ngroups > 64
    got = call().float().reshape(c.rows, c.D).cpu().numpy()
    assert_close(got, c.reference(), atol=ATOL, rtol=RTOL, what=f"65000 tokens, {call.ngroups} groups")


@pytest.mark.parametrize("B,D,size,want", [(18, 64, 2048, (296, 3, 3)), (20, 128, 2048, (344, 3, 2))])
def test_rows_beyond_the_cus_spread_over_small_blocks(device, B, D, size, want):
    """288 / 320 rows: one block per row would give the busiest CUs two rows against a mean of 1.1-1.3, so each
    row's waves go to 2- or 3-wave blocks joined by the merge; ragged lengths, some empty."""
    lengths = [size - (53 * i) % (size // 2) for i in range(B)]
    lengths[3], lengths[7] = 0, 1
    c = FloatCase(device, B, 16, D, size, torch.bfloat16, lengths=lengths, seed=SEED + 31 + B)
    call = ppk.FloatDecodeAttention(c.q, c.k, c.v, c.lengths_t, c.H, max_length=size)
    info = call.plan_info
    assert (info["split_tokens"], info["nsplits"], info["waves_per_block"]) == want
    got = call().float().reshape(c.rows, c.D).cpu().numpy()
    assert_close(got, c.reference(), atol=ATOL, rtol=RTOL, what=f"{c.rows} rows x {size} at D = {D}")


def test_few_long_rows_take_larger_blocks_that_land_evenly(device):
    """64 rows of up to 8192 tokens at D = 64: 32 waves of 256 tokens a row in four 8-wave blocks (256 blocks,
    one a CU) joined by the merge, instead of 4-wave blocks; ragged lengths, one sequence empty."""
    size = 8192
    c = FloatCase(device, 4, 16, 64, size, torch.bfloat16, lengths=[8192, 0, 5000, 8191], seed=SEED + 37)
    call = ppk.FloatDecodeAttention(c.q, c.k, c.v, c.lengths_t, c.H, max_length=size)
    info = call.plan_info
    assert (info["split_tokens"], info["nsplits"], info["waves_per_block"]) == (256, 4, 8)
    got = call().float().reshape(c.rows, c.D).cpu().numpy()
    ref = c.reference()
    assert np.isnan(got[16:32]).all() and np.isnan(ref[16:32]).all()
    keep = np.r_[0:16, 32:64]
    assert_close(got[keep], ref[keep], atol=ATOL, rtol=RTOL, what="64 rows x 8192 at D = 64, 8-wave blocks")


def test_hip_graph_replay(device):
    """A prepared call captured in a HIP graph replays bit-identically to the eager call."""
    c = FloatCase(device, 1, 16, 64, 1024, torch.bfloat16, lengths=[900], seed=SEED + 11)
    call = ppk.FloatDecodeAttention(c.q, c.k, c.v, c.lengths_t, c.H)
    assert call.ngroups > 1  # the merge kernel is part of the graph
    eager = call().clone()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        call(s)  # warm up on the capture stream
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            call(s)
    for _ in range(3):
        call.out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(call.out, eager)
    assert_close(eager.reshape(c.rows, c.D).cpu().numpy(), c.reference(), atol=ATOL, rtol=RTOL, what="graph")


def test_float_prepare_self_check(device):
    """ppk_float_attention_prepare runs the reference's Split-K validation on the device."""
    ppk.fused_attention.prepare(device)
