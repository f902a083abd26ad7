"""GPU tests of int8 KV arenas: the reference's Int8LayerCache tests
(app/src/model/int8_cache.rs:14-266, including the device batch-attention
test at :210-266) and the AMD variant's self-check (known-answer test v,
app/native/aten_hip/cpp/kv_int8.cpp:167-196), restated through the C-ABI.
Codes and scales are compared bit for bit with the oracle's quantisation;
attention with the reference's own bars (1e-4 for the bf16-history host
formula, 0.005 for the AMD variant's bf16 output)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle
import ppk
from ppk import _abi
from ppk.kv_arena import LayerCache, WritePlan, read
from helpers import bf16_bits_to_f32, to_bf16_bits

pytestmark = pytest.mark.gpu


def data(heads, count, bias, device="cuda"):
    """int8_cache.rs:19-23: sin(0.173 i) * 2 + bias over [heads, count, 64]."""
    i = torch.arange(heads * count * 64, dtype=torch.float32)
    return ((i * 0.173).sin() * 2 + bias).reshape(heads, count, 64).to(device)


def prefix(view, heads, row, count):
    """int8_cache.rs:30-33: codes and scales of sequence `row`, slots [0, count)."""
    codes = read(view, "k", max(view.length, count))[row * heads:(row + 1) * heads, :count]
    scales = read(view, "k_scales", max(view.length, count))[row * heads:(row + 1) * heads, :count]
    return codes.cpu().numpy(), scales.cpu().numpy()


def same(a, b):
    return np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def prefilled(n: int, heads: int, tokens: int) -> list[LayerCache]:
    """n int8 caches with `tokens` committed rows each (data bias = row index). Built in a helper so no
    loop variable keeps a cache object, and with it its slot ownership, alive in the test."""
    caches = [LayerCache("int8", heads, 64) for _ in range(n)]
    for row in range(n):
        x = data(heads, tokens, float(row))
        caches[row].query(x, x, 0, True)
    return caches


def test_history_is_persistently_eight_bit_with_fp32_token_head_scales(device):
    c = LayerCache("int8", 2, 64)
    k, v = data(2, 3, 0.0), data(2, 3, 1.0)
    view = c.query(k, v, 0, True)
    assert len(c) == 3 and (view.rows, view.capacity, view.head_dim) == (2, 64, 64)
    assert read(view, "k").dtype == torch.uint8 and read(view, "k_scales").dtype == torch.float32
    info = c.info()
    assert info.reserved_bytes == 2 * 64 * (64 * 2 + 4 * 2)
    assert info.scale_bytes == 2 * 64 * 4 * 2
    assert info.reserved_bytes * 1000 // (2 * 64 * 64 * 4) == 531  # 136 B per head-token vs 256 for bf16 K+V
    codes, scales, _ = oracle.quantize(k.cpu().numpy())
    assert np.array_equal(read(view, "k").cpu().numpy(), codes)
    assert np.array_equal(read(view, "k_scales").cpu().numpy(), scales)


def test_nine_partial_attributes_preserve_history_and_clone_commit_is_copy_on_write(device):
    c = LayerCache("int8", 2, 64)
    initial = data(2, 3, 0.0)
    expected = prefix(c.query(initial, initial, 0, True), 2, 0, 3)
    branch = c.clone()
    for field in range(9):
        scratch = data(2, 1, field * 5.0)
        assert same(prefix(c.query(scratch, scratch, 3, False), 2, 0, 3), expected)
        assert len(c) == 3
    complete = data(2, 1, -5.0)
    c.query(complete, complete, 3, True)
    assert len(c) == 4 and len(branch) == 3
    assert same(prefix(branch.query(complete, complete, 3, False), 2, 0, 3), expected)
    with pytest.raises(ppk.PpkPreconditionError):
        c.query(complete, complete, 3, True)


def test_ragged_batch_reuses_packed_arenas_without_losing_independent_history(device):
    heads, lengths = 2, [1, 3, 2]
    caches = [LayerCache("int8", heads, 64) for _ in lengths]
    expected = []
    for row, (n, c) in enumerate(zip(lengths, caches)):
        x = data(heads, n, float(row))
        expected.append(prefix(c.query(x, x, 0, True), heads, 0, n))
    saved = caches[0].clone()
    current = torch.stack([data(heads, 1, 10.0 + row) for row in range(3)])
    plan = WritePlan(lengths, heads, 64)
    view = LayerCache.query_batch(caches, current, current, lengths, False, plan)
    assert (view.rows, view.capacity) == (3 * heads, 64)
    arena = caches[0].info().arena_id
    for row in range(3):
        assert same(prefix(view, heads, row, lengths[row]), expected[row])
    nxt = LayerCache.query_batch(caches, current, current, lengths, True, plan)
    assert caches[0].info().arena_id == arena, "stable batch arena should be reused"
    for row in range(3):
        assert len(caches[row]) == lengths[row] + 1
        assert same(prefix(nxt, heads, row, lengths[row]), expected[row])
        codes, scales, _ = oracle.quantize(current[row].cpu().numpy())
        got = prefix(nxt, heads, row, lengths[row] + 1)
        assert np.array_equal(got[0][:, lengths[row]:], codes) and np.array_equal(got[1][:, lengths[row]:], scales)
    scratch = data(heads, 1, -99.0)
    assert same(prefix(saved.query(scratch, scratch, lengths[0], False), heads, 0, lengths[0]), expected[0])


def test_geometric_growth_copies_quantized_values_and_scales_without_requantizing(device):
    c = LayerCache("int8", 2, 64)
    initial = data(2, 63, 0.0)
    expected = prefix(c.query(initial, initial, 0, True), 2, 0, 63)
    tail = data(2, 2, 4.0)
    after = c.query(tail, tail, 63, True)
    assert len(c) == 65 and after.capacity == 128
    assert same(prefix(after, 2, 0, 63), expected)
    rebuilt = LayerCache("int8", 2, 64)
    rebuilt.query(tail, tail, 0, True)
    assert len(rebuilt) == 2 and len(c) == 65


def test_prefill_uses_original_current_chunk_and_only_expands_history_temporarily(device):
    c = LayerCache("int8", 2, 64)
    a = data(2, 3, 0.0)
    keys, _ = c.query_int8_prefill(a, a, 0, True)
    assert torch.equal(keys, a)
    b = data(2, 2, 7.0)
    keys, _ = c.query_int8_prefill(b, b, 3, True)
    assert torch.equal(keys[:, 3:5], b)
    # The prefix is the bf16 dequantisation of a's codes (int8_cache.rs:363-371).
    codes, scales, _ = oracle.quantize(a.cpu().numpy())
    deq = oracle.dequantize(codes, scales, round_bf16=True)
    assert np.array_equal(keys[:, :3].cpu().numpy(), deq)
    view = c.query(b[:, :1], b[:, :1], 5, False)
    history = ppk.dequantize(read(view, "k", 5), read(view, "k_scales", 5))
    assert tuple(history.shape) == (2, 5, 64) and len(c) == 5


@pytest.mark.parametrize("changed", [0, 1, 2])
def test_rebuilt_row_reuses_packed_and_scale_slots_with_one_history_copy(device, changed):
    heads = 2
    caches = prefilled(3, heads, 3)
    current = torch.stack([data(heads, 1, 8.0 + row) for row in range(3)])
    first = LayerCache.query_batch(caches, current, current, [3, 3, 3], False)
    expected = [prefix(first, heads, row, 3) for row in range(3)]
    arena = caches[0].info().arena_id
    copied = caches[(changed + 1) % 3].info().arena_copied_rows
    caches[changed] = LayerCache("int8", heads, 64)
    rebuilt = data(heads, 2, 20.0)
    rebuilt_expected = prefix(caches[changed].query(rebuilt, rebuilt, 0, True), heads, 0, 2)
    lengths = [2 if row == changed else 3 for row in range(3)]
    nxt = LayerCache.query_batch(caches, current, current, lengths, True)
    assert caches[0].info().arena_id == arena
    for row in range(3):
        assert same(prefix(nxt, heads, row, lengths[row]), rebuilt_expected if row == changed else expected[row])
    assert caches[0].info().arena_copied_rows - copied == 1


def test_truncated_int8_cache_keeps_reserve_and_snapshot_values(device):
    c = LayerCache("int8", 2, 64)
    initial = data(2, 5, 0.0)
    old = prefix(c.query(initial, initial, 0, True), 2, 0, 5)
    snapshot = c.clone()
    reserved = c.info().reserved_bytes
    with pytest.raises(ppk.PpkPreconditionError):
        c.truncate_committed(6)
    assert len(c) == 5
    c.truncate_committed(2)
    assert len(c) == 2 and c.info().reserved_bytes == reserved
    tail = data(2, 1, 7.0)
    nxt = c.query(tail, tail, 2, True)
    assert len(c) == 3
    got = prefix(nxt, 2, 0, 2)
    assert np.array_equal(got[0], old[0][:, :2]) and np.array_equal(got[1], old[1][:, :2])
    assert len(snapshot) == 5 and same(prefix(snapshot.query(tail, tail, 5, False), 2, 0, 5), old)
    c.truncate_committed(0)
    assert len(c) == 0 and c.info().reserved_bytes == reserved
    c.query(tail, tail, 0, True)
    assert len(c) == 1


def test_detached_int8_snapshot_blocks_slot_reuse(device):
    caches = prefilled(2, 2, 3)
    current = torch.stack([data(2, 1, 8.0), data(2, 1, 9.0)])
    old = LayerCache.query_batch(caches, current, current, [3, 3], False)
    old_arena = caches[0].info().arena_id
    expected = prefix(old, 2, 1, 3)
    snapshot = caches[1].clone()
    caches[1] = LayerCache("int8", 2, 64)
    rebuilt = data(2, 2, 30.0)
    caches[1].query(rebuilt, rebuilt, 0, True)
    LayerCache.query_batch(caches, current, current, [3, 2], True)
    assert caches[0].info().arena_id != old_arena
    assert same(prefix(snapshot.query(data(2, 1, -5.0), data(2, 1, -5.0), 3, False), 2, 0, 3), expected)


def _bf16(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("split", [32, 128])
def test_device_batch_attention_preserves_scratch_history_and_cow(device, split):
    """int8_cache.rs:210-266 (the reference's device test, tolerance 1e-4): a prototype cache cloned into a
    2-row batch; a partial batch write, then attention (bf16 history, reference-exact mode) against the
    host formula; then a commit; the prototype keeps its history."""
    heads = 2
    proto = LayerCache("int8", heads, 64)
    initial = _bf16(data(heads, 3, 0.0))
    expected = prefix(proto.query(initial, initial, 0, True), heads, 0, 3)
    caches = [proto.clone(), proto.clone()]
    current = _bf16(torch.stack([data(heads, 1, 0.37), data(heads, 1, -0.51)]))
    q = torch.stack([data(heads, 1, 0.07), data(heads, 1, -0.19)]).reshape(4, 1, 64)
    scratch = current.float().reshape(4, 1, 64).contiguous()
    view = LayerCache.query_batch(caches, current, current, [3, 3], False)
    assert same(prefix(view, heads, 0, 3), expected) and same(prefix(view, heads, 1, 3), expected)
    cap = view.capacity
    hist = oracle.dequantize(read(view, "k", cap).cpu().numpy(), read(view, "k_scales", cap).cpu().numpy(),
                             round_bf16=True)
    qc, sc = q.cpu().numpy().reshape(4, 64), scratch.cpu().numpy().reshape(4, 64)
    ref = np.empty((4, 64), np.float32)
    for row in range(4):
        keys = np.concatenate([hist[row, :3], sc[row:row + 1]])
        s = (keys @ qc[row]).astype(np.float32) * np.float32(0.125)
        p = np.exp(s - s.max())
        ref[row] = (p[:, None] * keys).sum(0) / p.sum()
    out = torch.empty((4, 1, 64), device=device)
    a = _abi.PpkAttentionArgs(struct_size=ctypes.sizeof(_abi.PpkAttentionArgs), flags=_abi.PPK_ATTN_BF16_HISTORY,
                              rows=4, heads=heads, capacity=cap, head_dim=64, split_tokens=split, q=q.data_ptr(),
                              k_codes=view.k, v_codes=view.v, k_scales=view.k_scales, v_scales=view.v_scales,
                              sk=scratch.data_ptr(), sv=scratch.data_ptr(), past=view.past, out=out.data_ptr())
    _, _, nbytes = ppk.int8_kv_ops.plan(a, ppk.context(device))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
    a.workspace, a.workspace_bytes = ws.data_ptr(), nbytes
    _abi.check(_abi.lib().ppk_decode_attention(ppk.context(device), None, ctypes.byref(a)), "attention")
    torch.cuda.synchronize()
    got = out.reshape(4, 64).cpu().numpy()
    assert np.all(np.isfinite(got)) and np.max(np.abs(got - ref)) < 1e-4
    LayerCache.query_batch(caches, current, current, [3, 3], True)
    assert all(len(c) == 4 for c in caches) and len(proto) == 3
    still = proto.query(current[0], current[0], 3, False)
    assert same(prefix(still, heads, 0, 3), expected)


def test_amd_variant_self_check_known_answer_v(device):
    """kv_int8.cpp:167-196 restated where the Candle API has the feature: B=2, H=2, C=257 bf16 K/V
    (sin 0.013 i / cos 0.019 i), bf16 q (cos 0.017 i); its chunk quantisation (kv_int8.cpp:162-165,
    absmax / 127 with IEEE division) is the a1 rule; attention over 256 history slots + the current slot
    within its 0.005 bar (bf16 output); the ragged commit at slot C-1-2b bit-exact in codes, scales
    within 1e-8. The validity mask of its batch 0 exists only in the AMD variant and is not restated."""
    B, H, C, D = 2, 2, 257, 64
    f = lambda n, a, fn: fn(torch.arange(n, dtype=torch.float32) * a)
    k = f(B * H * C * D, 0.013, torch.sin).reshape(B * H, C, D).to(torch.bfloat16)
    v = f(B * H * C * D, 0.019, torch.cos).reshape(B * H, C, D).to(torch.bfloat16)
    q = f(B * H * D, 0.017, torch.cos).reshape(B * H, 1, D).to(torch.bfloat16)
    caches = [LayerCache("int8", H, D, max_context=1024) for _ in range(B)]
    for b in range(B):
        caches[b].query(k[b * H:(b + 1) * H, :C - 1].to(device), v[b * H:(b + 1) * H, :C - 1].to(device), 0, True)
    sk = k[:, C - 1:C].contiguous()
    sv = v[:, C - 1:C].contiguous()
    view = LayerCache.query_batch(caches, sk.reshape(B, H, 1, D).to(device), sv.reshape(B, H, 1, D).to(device),
                                  [C - 1] * B, True)
    kc, ks, _ = oracle.quantize(k.float().numpy())
    vc, vs, _ = oracle.quantize(v.float().numpy())
    assert np.array_equal(read(view, "k", C).cpu().numpy(), kc)
    assert np.array_equal(read(view, "k_scales", C).cpu().numpy(), ks)
    assert np.array_equal(read(view, "v", C).cpu().numpy(), vc)
    # Attention (bf16 q, bf16 current token, bf16 output) vs the variant's reference formula.
    out = torch.empty((B * H, 1, D), dtype=torch.bfloat16, device=device)
    qd, skd, svd = q.to(device), sk.to(device), sv.to(device)
    a = _abi.PpkAttentionArgs(struct_size=ctypes.sizeof(_abi.PpkAttentionArgs), q_dtype=_abi.PPK_BF16,
                              scratch_dtype=_abi.PPK_BF16, out_dtype=_abi.PPK_BF16, rows=B * H, heads=H,
                              capacity=view.capacity, head_dim=D, q=qd.data_ptr(), k_codes=view.k, v_codes=view.v,
                              k_scales=view.k_scales, v_scales=view.v_scales, sk=skd.data_ptr(), sv=svd.data_ptr(),
                              past=view.past, out=out.data_ptr())
    _, _, nbytes = ppk.int8_kv_ops.plan(a, ppk.context(device))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
    a.workspace, a.workspace_bytes = ws.data_ptr(), nbytes
    _abi.check(_abi.lib().ppk_decode_attention(ppk.context(device), None, ctypes.byref(a)), "attention")
    torch.cuda.synchronize()
    dk = bf16_bits_to_f32(to_bf16_bits(oracle.dequantize(kc, ks)))
    dv = bf16_bits_to_f32(to_bf16_bits(oracle.dequantize(vc, vs)))
    dk[:, C - 1] = sk.float().numpy()[:, 0]
    dv[:, C - 1] = sv.float().numpy()[:, 0]
    qf = q.float().numpy()[:, 0]
    ref = np.empty((B * H, D), np.float32)
    for r in range(B * H):
        s = (dk[r] @ qf[r]) * np.float32(0.125)
        p = np.exp(s - s.max())
        ref[r] = (p[:, None] * dv[r]).sum(0) / p.sum()
    ref = bf16_bits_to_f32(to_bf16_bits(ref))
    assert np.max(np.abs(out.float().reshape(B * H, D).cpu().numpy() - ref)) <= 0.005
    # Ragged commit (kv_int8.cpp:184-195): scratch sin(0.031 i), written at slot C-1-2b of sequence b.
    scratch = f(B * H * D, 0.031, torch.sin).reshape(B, H, 1, D).to(torch.bfloat16)
    commit = [LayerCache("int8", H, D, max_context=1024) for _ in range(B)]
    slots = [C - 1 - 2 * b for b in range(B)]
    filler = torch.zeros((H, C, D), dtype=torch.bfloat16, device=device)
    for b in range(B):
        commit[b].query(filler[:, :slots[b]], filler[:, :slots[b]], 0, True)
    view = LayerCache.query_batch(commit, scratch.to(device), scratch.to(device), slots, True)
    codes, scales, _ = oracle.quantize(scratch.float().numpy().reshape(B * H, 1, D))
    got_c = read(view, "k", C).cpu().numpy()
    got_s = read(view, "k_scales", C).cpu().numpy()
    for b in range(B):
        rows = slice(b * H, (b + 1) * H)
        assert np.array_equal(got_c[rows, slots[b]], codes[rows, 0])
        assert np.max(np.abs(got_s[rows, slots[b]] - scales[rows, 0])) < 1e-8


def _view_attention(view, q, sk, sv, heads):
    """ppk_decode_attention over a batch view (history [0, past[b]) plus the current token sk/sv)."""
    rows, d = view.rows, view.head_dim
    out = torch.empty((rows, 1, d), dtype=torch.float32, device=q.device)
    a = _abi.PpkAttentionArgs(
        struct_size=ctypes.sizeof(_abi.PpkAttentionArgs), q_dtype=_abi.PPK_BF16, scratch_dtype=_abi.PPK_BF16,
        out_dtype=_abi.PPK_F32, flags=0, rows=rows, heads=heads, capacity=view.capacity, head_dim=d,
        split_tokens=0, max_past=view.length - 1, softmax_scale=0.0, q=q.data_ptr(), k_codes=view.k,
        v_codes=view.v, k_scales=view.k_scales, v_scales=view.v_scales, sk=sk.data_ptr(), sv=sv.data_ptr(),
        past=view.past, out=out.data_ptr(), workspace=None, workspace_bytes=0, past_host=None)
    ctx = ppk.context(q.device)
    nbytes = ppk.int8_kv_ops.workspace_bytes(a, ctx)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    a.workspace, a.workspace_bytes = ws.data_ptr(), nbytes
    stream = ctypes.c_void_p(torch.cuda.current_stream(q.device).cuda_stream)
    _abi.check(_abi.lib().ppk_decode_attention(ctx, stream, ctypes.byref(a)), "ppk_decode_attention")
    return out


def test_reserved_batch_write_and_fused_step_equal_write_then_attention(device):
    """ppk_kv_query_batch with NULL sources (no counterpart in the reference) reserves slot past[b]; the fused
    decode step on the returned view then quantises the token there and attends in one launch. Over a join
    round and two steady rounds of ragged sequences, the arenas (codes and scales of every committed slot) and
    the outputs equal the two-call path (write, then ppk_decode_attention) bit for bit."""
    from ppk import kv_arena

    heads, d, lengths = 4, 128, [37, 0, 120]
    g = torch.Generator(device=device).manual_seed(11)
    sets = []
    for _ in range(2):
        caches = [LayerCache("int8", heads, d) for _ in lengths]
        for c, n in zip(caches, lengths):
            if n:
                x = torch.randn((heads, n, d), generator=torch.Generator(device=device).manual_seed(n), device=device)
                c.query(x, x, 0, True)
        sets.append(caches)
    past = list(lengths)
    for rnd in range(3):
        q = torch.randn((len(past) * heads, d), generator=g, device=device).to(torch.bfloat16)
        kn = torch.randn((len(past), heads, 1, d), generator=g, device=device).to(torch.bfloat16)
        vn = torch.randn((len(past), heads, 1, d), generator=g, device=device).to(torch.bfloat16)
        va = LayerCache.query_batch(sets[0], kn, vn, past, True, WritePlan(past, heads, d))
        out_a = _view_attention(va, q, kn, vn, heads)
        vb = LayerCache.query_batch(sets[1], None, None, past, True, WritePlan(past, heads, d))
        out_b = kv_arena.decode_step(vb, q, kn.reshape(-1, d), vn.reshape(-1, d), heads)
        torch.cuda.synchronize()
        assert torch.equal(out_a, out_b), f"round {rnd}"
        assert torch.isfinite(out_a).all()
        n = max(past) + 1
        for which in ("k", "v", "k_scales", "v_scales"):
            ra, rb = read(va, which, n), read(vb, which, n)
            for row, p in enumerate(past):
                rows = slice(row * heads, (row + 1) * heads)
                assert torch.equal(ra[rows, :p + 1], rb[rows, :p + 1]), f"round {rnd} {which} sequence {row}"
        assert [len(c) for c in sets[1]] == [p + 1 for p in past]
        past = [p + 1 for p in past]


def test_refused_step_after_a_reserving_write_is_undone_by_truncation(device):
    """A reserving write commits slot past[b] unwritten; a fused step refused after it (status 1, nothing
    enqueued: here the balanced plan without host lengths) leaves that commit in place. Truncating each
    cache back to past[b] undoes it, and the round then runs as if the reservation had never happened: codes,
    scales and output equal those of a second set of caches that only ever saw the plain write."""
    from ppk import kv_arena

    heads, d, lengths = 4, 128, [37, 0, 120]
    sets = []
    for _ in range(2):
        caches = [LayerCache("int8", heads, d) for _ in lengths]
        for c, n in zip(caches, lengths):
            if n:
                x = torch.randn((heads, n, d), generator=torch.Generator(device=device).manual_seed(n), device=device)
                c.query(x, x, 0, True)
        sets.append(caches)
    g = torch.Generator(device=device).manual_seed(12)
    q = torch.randn((len(lengths) * heads, d), generator=g, device=device).to(torch.bfloat16)
    kn = torch.randn((len(lengths), heads, 1, d), generator=g, device=device).to(torch.bfloat16)
    vn = torch.randn((len(lengths), heads, 1, d), generator=g, device=device).to(torch.bfloat16)
    view = LayerCache.query_batch(sets[1], None, None, lengths, True)
    assert [len(c) for c in sets[1]] == [p + 1 for p in lengths]  # committed, not yet written
    with pytest.raises(ppk.PpkError) as e:
        kv_arena.decode_step(view, q, kn.reshape(-1, d), vn.reshape(-1, d), heads, plan="balanced")
    assert e.value.status == _abi.PPK_PRECONDITION
    assert [len(c) for c in sets[1]] == [p + 1 for p in lengths]  # the refusal left the commit in place
    for c, p in zip(sets[1], lengths):
        c.truncate_committed(p)
    assert [len(c) for c in sets[1]] == lengths
    va = LayerCache.query_batch(sets[0], kn, vn, lengths, True)
    out_a = _view_attention(va, q, kn, vn, heads)
    vb = LayerCache.query_batch(sets[1], kn, vn, lengths, True)
    out_b = _view_attention(vb, q, kn, vn, heads)
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b) and torch.isfinite(out_a).all()
    n = max(lengths) + 1
    for which in ("k", "v", "k_scales", "v_scales"):
        ra, rb = read(va, which, n), read(vb, which, n)
        for row, p in enumerate(lengths):
            rows = slice(row * heads, (row + 1) * heads)
            assert torch.equal(ra[rows, :p + 1], rb[rows, :p + 1]), f"{which} sequence {row}"


def test_reserving_write_needs_int8_bf16_or_f32_caches(device):
    """F16 caches have no fused step (the float attention reads bf16 and f32 stores): a reserving write is
    refused before anything changes."""
    caches = [LayerCache(torch.float16, 2, 64) for _ in range(2)]
    with pytest.raises(ppk.PpkError) as e:
        LayerCache.query_batch(caches, None, None, [0, 0], True)
    assert e.value.status == _abi.PPK_PRECONDITION
    assert [len(c) for c in caches] == [0, 0]


@pytest.mark.parametrize("kind", [torch.bfloat16, torch.float32])
def test_reserved_float_batch_write_and_fused_step_equal_write_then_attention(device, kind):
    """The float caches' reserve + ppk_float_decode_step against the two-call path (the token written by
    ppk_kv_query_batch, then ppk_float_decode_attention over past + 1): the arenas bit for bit over a join
    round and two steady rounds of ragged sequences; outputs within the float path's bars (the fused step
    folds the current token from registers, a different fp32 order)."""
    from helpers import assert_close
    from ppk import kv_arena

    heads, d, lengths = 4, 128, [37, 0, 120]
    g = torch.Generator(device=device).manual_seed(12)
    sets = []
    for _ in range(2):
        caches = [LayerCache(kind, heads, d) for _ in lengths]
        for c, n in zip(caches, lengths):
            if n:
                x = torch.randn((heads, n, d), generator=torch.Generator(device=device).manual_seed(n),
                                device=device).to(kind)
                c.query(x, x, 0, True)
        sets.append(caches)
    past = list(lengths)
    for rnd in range(3):
        q = torch.randn((len(past) * heads, d), generator=g, device=device)
        kn = torch.randn((len(past), heads, 1, d), generator=g, device=device).to(kind)
        vn = torch.randn((len(past), heads, 1, d), generator=g, device=device).to(kind)
        va = LayerCache.query_batch(sets[0], kn, vn, past, True, WritePlan(past, heads, d))
        view_len = va.length
        k_view, v_view = read(va, "k"), read(va, "v")
        lengths_after = torch.tensor([p + 1 for p in past], dtype=torch.int32, device=device)
        out_a = ppk.fused_attention.decode_attention(q.reshape(-1, 1, d), k_view, v_view, lengths_after, heads)
        vb = LayerCache.query_batch(sets[1], None, None, past, True, WritePlan(past, heads, d))
        out_b = kv_arena.decode_step(vb, q, kn.reshape(-1, d), vn.reshape(-1, d), heads, past_host=past)
        torch.cuda.synchronize()
        assert torch.isfinite(out_b).all()
        assert_close(out_b.reshape(-1, d).cpu().numpy(), out_a.reshape(-1, d).cpu().numpy(), atol=1e-4, rtol=1e-2,
                     what=f"{kind} round {rnd}")
        assert vb.length == view_len
        for which in ("k", "v"):
            ra, rb = read(va, which), read(vb, which)
            for row, p in enumerate(past):
                rows = slice(row * heads, (row + 1) * heads)
                assert torch.equal(ra[rows, :p + 1], rb[rows, :p + 1]), f"round {rnd} {which} sequence {row}"
        assert [len(c) for c in sets[1]] == [p + 1 for p in past]
        past = [p + 1 for p in past]
