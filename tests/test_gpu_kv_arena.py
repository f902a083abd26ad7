"""GPU tests of the KV arena manager (ppk_kv_*), through the C-ABI.

The scenarios restate the reference's own LayerCache / BatchWritePlan tests
(app/src/model/cache.rs:545-1479, app/src/model/write_plan.rs:104-163) and
check every visible slot against a host model that concatenates what was
written (the reference's cat oracle, cache.rs:551-556): float stores
bit-exact, int8 stores against the oracle's quantisation bit-exact, and
attention over the returned views against the f64 oracle.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle
import ppk
from ppk import _abi
from ppk.kv_arena import LayerCache, WritePlan, read
from helpers import SEED, assert_close

pytestmark = pytest.mark.gpu
F32 = torch.float32


def data(heads, length, width, base, dtype=F32, device="cuda"):
    """cache.rs:557-566: base + 0.25 * i over [heads, length, width]."""
    x = base + 0.25 * torch.arange(heads * length * width, dtype=torch.float64)
    return x.reshape(heads, length, width).to(dtype).to(device)


def batch_data(batch, heads, width, base, dtype=F32):
    """cache.rs:576-585: [batch, heads, 1, width], row b offset by 100 * b."""
    return torch.stack([data(heads, 1, width, base + 100.0 * b, dtype) for b in range(batch)])


def cat(old, cur):
    return cur if old is None else torch.cat([old, cur], 1)


def rows_of(view, b, heads, tokens, which="k"):
    full = read(view, which, tokens)
    return full[b * heads:(b + 1) * heads]


def expect_status(status, fn):
    with pytest.raises(ppk.PpkError) as e:
        fn()
    assert e.value.status == status


def grouped_rows(dtype=F32):
    """cache.rs:586-598: three caches with 3 committed tokens each, then one partial batch write."""
    caches = [LayerCache(dtype, 2, 3) for _ in range(3)]
    for row, c in enumerate(caches):
        p = data(2, 3, 3, row * 10.0, dtype)
        c.query(p, p, 0, True)
    cur = batch_data(3, 2, 3, 100.0, dtype)
    LayerCache.query_batch(caches, cur, cur, [3, 3, 3], False)
    return caches


def test_preallocated_commit_matches_dynamic_cat_oracle(device):
    c = LayerCache(F32, 3, 4)
    old_k = old_v = None
    for step, n in enumerate([3, 1, 5, 2]):
        k, v = data(3, n, 4, step * 10.0), data(3, n, 4, 100 + step * 10.0)
        ek, ev = cat(old_k, k), cat(old_v, v)
        prev = len(c)
        view = c.query(k, v, prev, True)
        assert torch.equal(read(view, "k"), ek) and torch.equal(read(view, "v"), ev)
        assert len(c) == prev + n and torch.equal(c.key(), ek)
        old_k, old_v = ek, ev


def test_capacity_grows_by_powers_of_two_without_losing_committed_prefix(device):
    c = LayerCache(F32, 2, 3)
    assert c.info().capacity == 0
    old_k = old_v = None
    for step, (n, cap) in enumerate(zip([1, 63, 1, 63, 1, 127, 1, 255, 1, 511],
                                        [64, 64, 128, 128, 256, 256, 512, 512, 1024, 1024])):
        k, v = data(2, n, 3, step * 1000.0), data(2, n, 3, step * 1000.0 + 500)
        ek, ev = cat(old_k, k), cat(old_v, v)
        prev = len(c)
        before = c.info()
        view = c.query(k, v, prev, True)
        assert c.info().capacity == cap and len(c) == prev + n
        # A sole owner writes in place while the capacity holds (cache.rs:249-266): same storage, no copy.
        assert (c.info().storage_id == before.storage_id) == (before.capacity == cap), step
        assert torch.equal(read(view, "k"), ek) and torch.equal(read(view, "v"), ev)
        old_k, old_v = ek, ev
    assert len(c) == 1024
    expect_status(_abi.PPK_PRECONDITION, lambda: c.query(data(2, 1, 3, 2.0), data(2, 1, 3, 2.0), 1024, True))
    assert len(c) == 1024


def test_cow_retains_current_reserve_and_growth_copies_no_uncommitted_scratch(device):
    original = LayerCache(F32, 2, 3)
    prefix = data(2, 70, 3, 1.0)
    original.query(prefix, prefix, 0, True)
    assert original.info().capacity == 128
    scratch = data(2, 10, 3, 9000.0)
    original.query(scratch, scratch, 70, False)
    branch = original.clone()
    assert branch.info().shared == 1
    one = data(2, 1, 3, 55.0)
    bview = branch.query(one, one, 70, False)
    assert branch.info().capacity == 128 and len(branch) == 70
    assert torch.equal(branch.key(), prefix)
    assert torch.all(read(bview, "k", 73)[:, 72] == 0)             # scratch was not copied
    assert not torch.all(read(original.view(), "k", 73)[:, 72] == 0)
    growing = original.clone()
    nxt = data(2, 80, 3, 200.0)
    growing.query(nxt, nxt, 70, False)
    assert growing.info().capacity == 256 and len(growing) == 70
    assert original.info().capacity == 128 and len(original) == 70
    assert torch.equal(growing.key(), prefix)
    view = growing.query(nxt, nxt, 70, True)
    assert growing.info().capacity == 256 and len(growing) == 150
    assert torch.equal(read(view, "k"), cat(prefix, nxt))
    assert torch.equal(original.key(), prefix)


def test_partial_overwrites_scratch_without_committing_or_touching_prefix(device):
    c = LayerCache(F32, 2, 3)
    k, v = data(2, 4, 3, 1.0), data(2, 4, 3, 20.0)
    c.query(k, v, 0, True)
    prefix = c.key()
    first, second = data(2, 1, 3, 100.0), data(2, 1, 3, 200.0)
    first_snapshot = read(c.query(first, first, 4, False), "k")
    second_view = c.query(second, second, 4, False)
    assert len(c) == 4 and torch.equal(c.key(), prefix)
    assert not torch.equal(first_snapshot, read(second_view, "k"))
    assert torch.equal(read(second_view, "k"), cat(k, second))
    assert torch.equal(read(c.query(second, second, 4, True), "k"), cat(k, second)) and len(c) == 5


def test_cloned_cache_detaches_before_partial_or_commit_and_does_not_copy_scratch(device):
    original = LayerCache(F32, 2, 4)
    prefix = data(2, 3, 4, 1.0)
    original.query(prefix, prefix, 0, True)
    original.query(data(2, 1, 4, 999.0), data(2, 1, 4, 999.0), 3, False)
    branch = original.clone()
    assert branch.info().storage_id == original.info().storage_id
    q = data(2, 1, 4, 80.0)
    bview = branch.query(q, q, 3, False)
    assert branch.info().storage_id != original.info().storage_id
    assert len(original) == 3 and len(branch) == 3
    assert torch.equal(original.key(), prefix)
    assert torch.equal(read(original.view(), "k", 4)[:, 3:4], data(2, 1, 4, 999.0))
    assert torch.all(read(bview, "k", 5)[:, 4] == 0)
    branch.query(q, q, 3, True)
    assert len(original) == 3 and len(branch) == 4 and torch.equal(original.key(), prefix)


def test_default_clones_allocate_separately_and_validate_boundary_and_lengths(device):
    first = LayerCache(F32, 1, 2)
    second = first.clone()
    a, b = data(1, 1, 2, 1.0), data(1, 1, 2, 50.0)
    first.query(a, a, 0, True)
    second.query(b, b, 0, True)
    assert not torch.equal(first.key(), second.key())
    expect_status(_abi.PPK_PRECONDITION, lambda: first.query(a, a, 0, False))       # past != length
    assert len(first) == 1
    with pytest.raises(ValueError):
        first.query(data(2, 1, 2, 0.0), data(2, 1, 2, 0.0), 1, True)               # heads differ
    expect_status(_abi.PPK_PRECONDITION, lambda: first.query(a.half(), a.half(), 1, True))  # dtype differs
    full = LayerCache(F32, 1, 1)
    block = data(1, 1024, 1, 0.0)
    full.query(block, block, 0, True)
    assert len(full) == 1024
    expect_status(_abi.PPK_PRECONDITION, lambda: full.query(data(1, 1, 1, 2.0), data(1, 1, 1, 2.0), 1024, True))
    assert len(full) == 1024


def test_partial_only_cache_has_no_valid_prefix(device):
    source = data(2, 4, 3, 7.0)[:, 1:3]
    c = LayerCache(F32, 2, 3)
    view = c.query(source, source, 0, False)
    assert torch.equal(read(view, "k"), source)
    assert len(c) == 0 and c.key() is None and c.value() is None
    clone = c.clone()
    clone.query(data(2, 1, 3, 1.0), data(2, 1, 3, 2.0), 0, True)
    assert len(c) == 0 and len(clone) == 1


def test_batch_arena_matches_each_cat_oracle_and_reuses_one_storage(device):
    caches = [LayerCache(F32, 2, 4) for _ in range(3)]
    expected = []
    for row, c in enumerate(caches):
        p = data(2, 3, 4, row * 10.0)
        c.query(p, p, 0, True)
        expected.append(p)
    first = batch_data(3, 2, 4, 500.0)
    view = LayerCache.query_batch(caches, first, first, [3, 3, 3], False)
    assert (view.rows, view.length, view.batch) == (6, 4, 3)
    for row in range(3):
        oracle_rows = cat(expected[row], first[row].reshape(2, 1, 4))
        assert torch.equal(rows_of(view, row, 2, 4), oracle_rows)
        assert torch.equal(rows_of(view, row, 2, 4, "v"), oracle_rows)
        assert len(caches[row]) == 3 and torch.equal(caches[row].key(), expected[row])
    arena = caches[0].info().arena_id
    second = batch_data(3, 2, 4, 900.0)
    view = LayerCache.query_batch(caches, second, second, [3, 3, 3], True)
    assert caches[2].info().arena_id == arena
    for row in range(3):
        assert torch.equal(rows_of(view, row, 2, 4), cat(expected[row], second[row].reshape(2, 1, 4)))
        assert len(caches[row]) == 4


def test_ragged_batch_has_maskable_tails_and_invalid_last_row_writes_nothing(device):
    lengths = [0, 2, 5]
    caches = [LayerCache(F32, 2, 3) for _ in range(3)]
    old = []
    for row, c in enumerate(caches):
        if lengths[row]:
            p = data(2, lengths[row], 3, row * 10.0)
            c.query(p, p, 0, True)
            old.append(p)
        else:
            old.append(None)
    cur = batch_data(3, 2, 3, 600.0)
    view = LayerCache.query_batch(caches, cur, cur, lengths, False)
    assert (view.rows, view.length) == (6, 6)
    for row in range(3):
        visible = rows_of(view, row, 2, 6)[:, :lengths[row] + 1]
        assert torch.equal(visible, cat(old[row], cur[row].reshape(2, 1, 3)))
        assert len(caches[row]) == lengths[row]
        assert (caches[row].key() is None) == (lengths[row] == 0)
    before = read(view, "k", 6).clone()
    other = batch_data(3, 2, 3, 800.0)
    expect_status(_abi.PPK_PRECONDITION, lambda: LayerCache.query_batch(caches, other, other, [0, 2, 4], True))
    assert torch.equal(read(view, "k", 6), before)
    assert [len(c) for c in caches] == lengths


def test_cloned_batch_detaches_before_partial_and_commit(device):
    original = [LayerCache(F32, 2, 3) for _ in range(2)]
    first = batch_data(2, 2, 3, 10.0)
    LayerCache.query_batch(original, first, first, [0, 0], True)
    before = [c.key().clone() for c in original]
    branch = [c.clone() for c in original]
    other = batch_data(2, 2, 3, 700.0)
    LayerCache.query_batch(branch, other, other, [1, 1], False)
    assert original[0].info().arena_id != branch[0].info().arena_id
    LayerCache.query_batch(branch, other, other, [1, 1], True)
    for row in range(2):
        assert len(original[row]) == 1 and len(branch[row]) == 2
        assert torch.equal(original[row].key(), before[row])


def test_batch_growth_and_single_row_detach_can_rejoin_without_losing_prefix(device):
    caches = [LayerCache(F32, 2, 3) for _ in range(2)]
    for row, c in enumerate(caches):
        p = data(2, 63, 3, row * 100.0)
        c.query(p, p, 0, True)
    cur = batch_data(2, 2, 3, 700.0)
    LayerCache.query_batch(caches, cur, cur, [63, 63], True)
    assert all(c.info().capacity == 64 for c in caches)
    old = [c.clone() for c in caches]
    nxt = data(2, 1, 3, 2000.0)
    caches[0].query(nxt, nxt, 64, True)
    assert caches[0].info().grouped == 0 and caches[0].info().capacity == 128
    assert len(old[0]) == 64
    before = [c.key().clone() for c in caches]
    tail = batch_data(2, 2, 3, 3000.0)
    view = LayerCache.query_batch(caches, tail, tail, [65, 64], True)
    for row in range(2):
        assert caches[row].info().capacity == 128
        expected = cat(before[row], tail[row].reshape(2, 1, 3))
        assert torch.equal(rows_of(view, row, 2, view.length)[:, :expected.shape[1]], expected)
        assert len(old[row]) == 64


def test_aliased_input_is_snapshotted_before_batch_write(device):
    caches = [LayerCache(F32, 1, 3)]
    first = batch_data(1, 1, 3, 10.0)
    view = LayerCache.query_batch(caches, first, first, [0], True)
    # The source is slot 0 of the arena itself (a raw view of the storage being written).
    w = _abi.PpkKvWrite(struct_size=ctypes.sizeof(_abi.PpkKvWrite), src_dtype=_abi.PPK_F32, tokens=1, commit=1,
                        k=view.k, v=view.k)
    handles = (ctypes.c_void_p * 1)(caches[0].handle.value)
    lens = (ctypes.c_uint32 * 1)(1)
    out = _abi.PpkKvView(struct_size=ctypes.sizeof(_abi.PpkKvView))
    ppk._abi.check(_abi.lib().ppk_kv_query_batch(caches[0].ctx, None, handles, 1, lens, ctypes.byref(w), None,
                                                 ctypes.byref(out)), "ppk_kv_query_batch")
    torch.cuda.synchronize()
    assert read(out, "k").flatten().tolist() == [10.0, 10.25, 10.5, 10.0, 10.25, 10.5]


def test_one_write_plan_is_reused_by_thirty_five_layers_without_local_offset_uploads(device):
    offsets = [1, 3]
    plan = WritePlan(offsets, 2, 3)
    layers = []
    for layer in range(35):
        rows = [LayerCache(F32, 2, 3) for _ in range(2)]
        for row, c in enumerate(rows):
            c.query(data(2, offsets[row], 3, layer * 1000.0 + row * 100),
                    data(2, offsets[row], 3, layer * 1000.0 + row * 100 + 50), 0, True)
        layers.append(rows)
    for layer, caches in enumerate(layers):
        old_k = [c.key().clone() for c in caches]
        old_v = [c.value().clone() for c in caches]
        k = batch_data(2, 2, 3, layer * 1000.0 + 500)
        v = batch_data(2, 2, 3, layer * 1000.0 + 700)
        view = LayerCache.query_batch(caches, k, v, offsets, False, plan)
        for row in range(2):
            n = offsets[row] + 1
            assert torch.equal(rows_of(view, row, 2, view.length)[:, :n], cat(old_k[row], k[row].reshape(2, 1, 3)))
            assert torch.equal(rows_of(view, row, 2, view.length, "v")[:, :n], cat(old_v[row], v[row].reshape(2, 1, 3)))
            assert len(caches[row]) == offsets[row] and torch.equal(caches[row].key(), old_k[row])
        assert caches[0].info().arena_offset_uploads == 0


@pytest.mark.parametrize("batch", [40, 70])
def test_write_plan_offsets_reach_the_device_for_small_and_large_batches(device, batch):
    """Plans of up to 64 sequences upload their offsets in a kernel's arguments, larger ones by a copy;
    either way every sequence's token lands at its own slot (ragged lengths, some empty)."""
    lengths = [(7 * b) % 13 for b in range(batch)]
    caches = [LayerCache(F32, 2, 3) for _ in range(batch)]
    old = []
    for b, c in enumerate(caches):
        if lengths[b]:
            p = data(2, lengths[b], 3, b * 10.0)
            c.query(p, p, 0, True)
            old.append(p)
        else:
            old.append(None)
    cur = batch_data(batch, 2, 3, 600.0)
    view = LayerCache.query_batch(caches, cur, cur, lengths, True, WritePlan(lengths, 2, 3))
    width = max(lengths) + 1
    for b in range(batch):
        visible = rows_of(view, b, 2, width)[:, :lengths[b] + 1]
        assert torch.equal(visible, cat(old[b], cur[b].reshape(2, 1, 3))), f"sequence {b}"
        assert len(caches[b]) == lengths[b] + 1


def test_wrong_shared_write_plan_is_rejected_before_history_or_scratch_is_touched(device):
    for offsets in ([1, 3], [1, 1]):
        caches = [LayerCache(F32, 2, 3) for _ in range(2)]
        for row, c in enumerate(caches):
            c.query(data(2, offsets[row], 3, row * 100.0), data(2, offsets[row], 3, row * 100.0 + 50), 0, True)
        cur = batch_data(2, 2, 3, 500.0)
        view = LayerCache.query_batch(caches, cur, cur, offsets, False, WritePlan(offsets, 2, 3))
        before_k = read(view, "k", view.capacity).clone()
        before_v = read(view, "v", view.capacity).clone()
        owners = [c.info().storage_id for c in caches]
        for wrong in (WritePlan([0, offsets[1]], 2, 3), WritePlan(offsets, 1, 3), WritePlan(offsets, 2, 2)):
            expect_status(_abi.PPK_PRECONDITION,
                          lambda: LayerCache.query_batch(caches, cur, cur, offsets, True, wrong))
            assert torch.equal(read(view, "k", view.capacity), before_k)
            assert torch.equal(read(view, "v", view.capacity), before_v)
            for row in range(2):
                assert len(caches[row]) == offsets[row] and caches[row].info().storage_id == owners[row]


def _read_u32(ptr, n):
    out = torch.empty(n, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    ppk.kv_arena._hip_runtime().hipMemcpy2DAsync(out.data_ptr(), 4 * n, ptr, 4 * n, 4 * n, 1, 3, None)
    torch.cuda.synchronize()
    return out.tolist()


def test_write_plan_is_refused_on_another_stream_and_recycled_on_its_own(device):
    """A plan's device vector is uploaded and recycled in its creation stream's order, so a batch write on
    another stream is refused (status 1, nothing touched); released plans hand their vectors to the next
    plans on the same stream, which wait for the release event before uploading."""
    offsets = [2, 0, 1]
    caches = [LayerCache(F32, 2, 3) for _ in range(3)]
    for row, c in enumerate(caches):
        if offsets[row]:
            c.query(data(2, offsets[row], 3, row * 10.0), data(2, offsets[row], 3, row * 10.0 + 5), 0, True)
    cur = batch_data(3, 2, 3, 300.0)
    plan = WritePlan(offsets, 2, 3)
    owners = [c.info().storage_id for c in caches]
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        expect_status(_abi.PPK_PRECONDITION, lambda: LayerCache.query_batch(caches, cur, cur, offsets, True, plan))
    torch.cuda.current_stream(device).wait_stream(side)
    assert [len(c) for c in caches] == offsets and [c.info().storage_id for c in caches] == owners
    # On its own stream the plan works; then a chain of plans, each released before the next is created,
    # recycles vectors and every upload lands.
    view = LayerCache.query_batch(caches, cur, cur, offsets, False, plan)
    assert _read_u32(view.past, 3) == offsets
    del plan
    for step in range(12):
        lens = [offsets[row] + (step + row) % 4 for row in range(3)]
        plan = WritePlan(lens, 2, 3)
        for row, c in enumerate(caches):
            if len(c) != lens[row]:
                c.truncate_committed(min(len(c), lens[row]))
                extra = lens[row] - len(c)
                if extra:
                    c.query(data(2, extra, 3, 40.0 + row), data(2, extra, 3, 70.0 + row), len(c), True)
        view = LayerCache.query_batch(caches, cur, cur, lens, False, plan)
        assert _read_u32(view.past, 3) == lens and _read_u32(view.lengths, 3) == [n + 1 for n in lens], step
        for row in range(3):
            assert torch.equal(rows_of(view, row, 2, view.length)[:, lens[row]], cur[row].reshape(2, 3))
        del plan


def test_committed_offsets_require_a_fresh_shared_plan(device):
    caches = [LayerCache(F32, 1, 2) for _ in range(2)]
    for row, c in enumerate(caches):
        p = data(1, row + 1, 2, row * 10.0)
        c.query(p, p, 0, True)
    initial = WritePlan([1, 2], 1, 2)
    cur = batch_data(2, 1, 2, 50.0)
    LayerCache.query_batch(caches, cur, cur, [1, 2], True, initial)
    committed = [c.key().clone() for c in caches]
    expect_status(_abi.PPK_PRECONDITION, lambda: LayerCache.query_batch(caches, cur, cur, [2, 3], True, initial))
    for row in range(2):
        assert torch.equal(caches[row].key(), committed[row])
    refreshed = WritePlan([2, 3], 1, 2)
    LayerCache.query_batch(caches, cur, cur, [2, 3], False, refreshed)
    assert [len(c) for c in caches] == [2, 3]
    for row in range(2):
        assert torch.equal(caches[row].key(), committed[row])


def test_ragged_offsets_are_reused_across_partials_and_refreshed_after_commit(device):
    caches = [LayerCache(F32, 2, 3) for _ in range(2)]
    ek, ev = [], []
    for row, c in enumerate(caches):
        n = 1 if row == 0 else 3
        k, v = data(2, n, 3, 10.0 + row * 20), data(2, n, 3, 110.0 + row * 20)
        c.query(k, v, 0, True)
        ek.append(k)
        ev.append(v)
    arena = None
    uploads = []
    for step, commit in enumerate([False, False, True, False]):
        offsets = [1, 3] if step < 3 else [2, 4]
        k = batch_data(2, 2, 3, 500.0 + step * 100)
        v = batch_data(2, 2, 3, 1500.0 + step * 100)
        view = LayerCache.query_batch(caches, k, v, offsets, commit)
        info = caches[0].info()
        if arena is not None:
            assert info.arena_id == arena
        arena = info.arena_id
        uploads.append(info.arena_offset_uploads)
        past = torch.empty(4, dtype=torch.int32, device="cuda")
        ppk.kv_arena._hip_runtime().hipMemcpy2DAsync(past.data_ptr(), 8, view.past, 8, 8, 1, 3, None)
        torch.cuda.synchronize()
        assert past[:2].tolist() == offsets
        for row in range(2):
            ok = cat(ek[row], k[row].reshape(2, 1, 3))
            ov = cat(ev[row], v[row].reshape(2, 1, 3))
            assert torch.equal(rows_of(view, row, 2, view.length)[:, :offsets[row] + 1], ok)
            assert torch.equal(rows_of(view, row, 2, view.length, "v")[:, :offsets[row] + 1], ov)
            if commit:
                ek[row], ev[row] = ok, ov
            assert torch.equal(caches[row].key(), ek[row]) and torch.equal(caches[row].value(), ev[row])
    assert uploads == [1, 1, 1, 2]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, F32])
def test_ragged_scatter_keeps_data_types(device, dtype):
    caches = [LayerCache(dtype, 1, 2) for _ in range(2)]
    for row, c in enumerate(caches):
        p = data(1, row + 1, 2, row + 1.0, dtype)
        c.query(p, p, 0, True)
    cur = batch_data(2, 1, 2, 4.0, dtype)
    before = [c.key().clone() for c in caches]
    view = LayerCache.query_batch(caches, cur, cur, [1, 2], True)
    assert read(view, "k").dtype == dtype
    for row in range(2):
        expected = cat(before[row], cur[row].reshape(1, 1, 2))
        assert torch.equal(rows_of(view, row, 1, view.length)[:, :row + 2], expected)


@pytest.mark.parametrize("dtype", [torch.bfloat16, F32])
def test_independent_reprefill_rejoins_its_orphan_slot_without_copying_other_rows(device, dtype):
    for changed in range(3):
        caches = grouped_rows(dtype)
        arena = caches[(changed + 1) % 3].info().arena_id
        copied = caches[(changed + 1) % 3].info().arena_copied_rows
        owners = [c.info().storage_id for c in caches]
        before = [c.key().clone() for c in caches]
        caches[changed] = LayerCache(dtype, 2, 3)
        rebuilt = data(2, 2, 3, 900.0, dtype)
        caches[changed].query(rebuilt, rebuilt, 0, True)
        lengths = [2 if r == changed else 3 for r in range(3)]
        cur = batch_data(3, 2, 3, 500.0, dtype)
        view = LayerCache.query_batch(caches, cur, cur, lengths, True)
        assert caches[0].info().arena_id == arena
        assert caches[0].info().arena_copied_rows - copied == 1
        for row in range(3):
            prior = rebuilt if row == changed else before[row]
            assert torch.equal(rows_of(view, row, 2, view.length)[:, :lengths[row] + 1],
                               cat(prior, cur[row].reshape(2, 1, 3)))
            if row != changed:
                assert caches[row].info().storage_id == owners[row]


def test_detached_snapshot_of_replaced_slot_forces_new_batch_arena(device):
    caches = grouped_rows()
    snapshot = caches[1].clone()
    saved = snapshot.key().clone()
    arena = caches[0].info().arena_id
    caches[1] = LayerCache(F32, 2, 3)
    rebuilt = data(2, 2, 3, 900.0)
    caches[1].query(rebuilt, rebuilt, 0, True)
    cur = batch_data(3, 2, 3, 500.0)
    LayerCache.query_batch(caches, cur, cur, [3, 2, 3], True)
    assert caches[0].info().arena_id != arena
    assert torch.equal(snapshot.key(), saved)
    snapshot.query(data(2, 1, 3, -80.0), data(2, 1, 3, -70.0), 3, True)
    assert torch.equal(snapshot.key()[:, :3], saved)


def test_empty_replacement_row_reuses_orphan_slot_without_history_copy(device):
    caches = grouped_rows()
    arena = caches[1].info().arena_id
    copied = caches[1].info().arena_copied_rows
    caches[0] = LayerCache(F32, 2, 3)
    cur = batch_data(3, 2, 3, 700.0)
    LayerCache.query_batch(caches, cur, cur, [0, 3, 3], True)
    assert caches[0].info().arena_id == arena and caches[0].info().arena_copied_rows == copied
    assert torch.equal(caches[0].key(), cur[0].reshape(2, 1, 3))


@pytest.mark.parametrize("case", ["permuted", "shared_owner", "capacity_growth"])
def test_unsafe_reuse_falls_back_to_a_new_arena(device, case):
    caches = grouped_rows()
    arena = caches[0].info().arena_id
    snapshot = caches[2].clone() if case == "shared_owner" else None
    saved = snapshot.key().clone() if snapshot is not None else None
    lengths = [3, 3, 3]
    if case == "permuted":
        caches[0], caches[1] = caches[1], caches[0]
    elif case == "capacity_growth":
        caches[1] = LayerCache(F32, 2, 3)
        p = data(2, 65, 3, 800.0)
        caches[1].query(p, p, 0, True)
        lengths[1] = 65
    cur = batch_data(3, 2, 3, 500.0)
    LayerCache.query_batch(caches, cur, cur, lengths, True)
    assert caches[0].info().arena_id != arena, case
    if snapshot is not None:
        assert torch.equal(snapshot.key(), saved)


def test_adopted_alias_of_the_batch_arena_keeps_the_safe_fallback(device):
    """cache.rs:664-681, case 3: row 1 replaced by a graph view adopted over the batch arena's own rows
    of that slot; the next batch write must not reuse the arena (the view aliases it) and still carries
    the adopted history."""
    caches = grouped_rows()
    arena = caches[0].info().arena_id
    own = caches[1].view()
    history = caches[1].key().clone()
    assert torch.equal(history, data(2, 3, 3, 10.0))
    old = caches[1]
    caches[1] = LayerCache._adopt(own.k, own.v, 2, 3, own.capacity, 3, device=device, keep=(caches[0],))
    del old                                            # its slot is orphaned; the memory stays (caches[0])
    assert caches[1].info().arena_id != arena and len(caches[1]) == 3
    cur = batch_data(3, 2, 3, 500.0)
    view = LayerCache.query_batch(caches, cur, cur, [3, 3, 3], True)
    assert caches[0].info().arena_id != arena
    assert caches[1].info().arena_id == caches[0].info().arena_id
    assert torch.equal(rows_of(view, 1, 2, 4), cat(history, cur[1]))
    assert torch.equal(rows_of(view, 0, 2, 4), cat(data(2, 3, 3, 0.0), cur[0]))


def test_adopted_graph_view_commits_in_place_and_advances_by_one(device):
    """graph_decode.rs:335-383 over cache.rs:55-73: the first graph commit adopts the graph's f32 buffers
    with the new length, later commits advance it by exactly one; the identity follows the storage."""
    heads, cap, d = 2, 64, 4
    key = torch.zeros(heads, cap, d, device=device)
    value = torch.zeros_like(key)
    key[:, :3], value[:, :3] = data(heads, 3, d, 1.0), data(heads, 3, d, 2.0)
    c = LayerCache.adopt_graph_view(key, value, cap, 3)
    ident = c.graph_storage_identity()
    assert ident is not None and len(c) == 3
    assert c.info().reserved_bytes == 2 * key.numel() * 4 and c.info().capacity == cap
    assert torch.equal(c.key(), key[:, :3]) and torch.equal(c.value(), value[:, :3])
    key[:, 3], value[:, 3] = 7.0, 8.0                  # the graph wrote slot 3
    c.advance_graph_length(3, 4)
    assert len(c) == 4 and c.graph_storage_identity() == ident and torch.equal(c.key(), key[:, :4])
    for prev, nxt in ((3, 4), (4, 6), (4, 4), (5, 6)):
        expect_status(_abi.PPK_PRECONDITION, lambda: c.advance_graph_length(prev, nxt))
    assert len(c) == 4
    nxt = data(heads, 1, d, 50.0)
    c.query(nxt, nxt, 4, True)                         # fits: written into the adopted memory in place
    torch.cuda.synchronize()
    assert c.graph_storage_identity() == ident and torch.equal(key[:, 4:5], nxt)
    snap = c.clone()
    saved = key.clone()
    s2 = data(heads, 1, d, 60.0)
    snap.query(s2, s2, 5, True)                        # shared: the snapshot copies first
    torch.cuda.synchronize()
    assert snap.graph_storage_identity() != ident and torch.equal(key, saved)
    assert torch.equal(snap.key(), torch.cat([saved[:, :5], s2], 1)) and len(c) == 5
    c.truncate_committed(2)
    assert c.graph_storage_identity() == ident
    grow = data(heads, 70, d, 90.0)
    c.query(grow, grow, 2, True)                       # past the adopted capacity: own storage
    torch.cuda.synchronize()
    assert c.graph_storage_identity() != ident and c.info().capacity == 128 and torch.equal(key, saved)
    assert torch.equal(c.key(), torch.cat([saved[:, :2], grow], 1))
    full = LayerCache.adopt_graph_view(key, value, cap, cap)
    expect_status(_abi.PPK_PRECONDITION, lambda: full.advance_graph_length(cap, cap + 1))


def test_adopt_graph_view_rejects_invalid_views(device):
    """cache.rs:55-63: shape, dtype, length and capacity checks fail with "invalid graph KV view"."""
    key = torch.zeros(2, 8, 4, device=device)
    value = torch.zeros_like(key)
    k, v = key.data_ptr(), value.data_ptr()
    for bad in (dict(committed_len=9), dict(max_context=4), dict(v_ptr=k + 16), dict(k_ptr=k + 2),
                dict(k_ptr=0), dict(heads=0)):
        args = dict(k_ptr=k, v_ptr=v, heads=2, head_dim=4, capacity=8, committed_len=3, max_context=0)
        args.update(bad)
        with pytest.raises(ppk.PpkError, match="invalid graph KV view"):
            LayerCache._adopt(args["k_ptr"], args["v_ptr"], args["heads"], args["head_dim"], args["capacity"],
                              args["committed_len"], max_context=args["max_context"], device=device)
    cfg = _abi.PpkKvConfig(struct_size=ctypes.sizeof(_abi.PpkKvConfig), kind=_abi.PPK_KV_BF16, heads=2, head_dim=4)
    h = ctypes.c_void_p()
    status = _abi.lib().ppk_kv_cache_adopt(ppk.context(device), ctypes.byref(cfg), k, v, 8, 3, ctypes.byref(h))
    assert status == _abi.PPK_PRECONDITION and not h.value
    assert b"invalid graph KV view" in _abi.lib().ppk_last_error()
    for kk, vv in ((key.half(), value.half()), (key[:, :4], value[:, :4]), (key, value[:1])):
        with pytest.raises(ValueError, match="invalid graph KV view"):
            LayerCache.adopt_graph_view(kk, vv, 8, 0)


@pytest.mark.parametrize("kind", [F32, "int8"])
def test_reused_storage_of_released_caches_reads_as_zeros_past_the_new_history(device, kind):
    """Storage of released caches is reused for the next arena of the same size: the new cache sees only
    its own history and zeros in every other slot (the reference's Tensor::zeros, cache.rs:241-247),
    never the released cache's data; single caches and a batch arena alike."""
    d = 64
    old = [LayerCache(kind, 2, d) for _ in range(3)]
    for c in old:
        p = data(2, 50, d, 7.0)
        c.query(p, p, 0, True)
    LayerCache.query_batch(old, batch_data(3, 2, d, 9.0), batch_data(3, 2, d, 9.0), [50, 50, 50], True)
    old_single = LayerCache(kind, 2, d)
    old_single.query(data(2, 60, d, 3.0), data(2, 60, d, 3.0), 0, True)
    ptrs = {old[0].view().k, old_single.view().k}
    del old, old_single
    fresh = [LayerCache(kind, 2, d) for _ in range(3)]
    for c in fresh:
        p = data(2, 5, d, 100.0)
        c.query(p, p, 0, True)
    view = LayerCache.query_batch(fresh, batch_data(3, 2, d, 200.0), batch_data(3, 2, d, 200.0), [5, 5, 5], True)
    single = LayerCache(kind, 2, d)
    sview = single.query(data(2, 4, d, 300.0), data(2, 4, d, 300.0), 0, True)
    torch.cuda.synchronize()
    assert ptrs & {view.k, sview.k}, "no released storage was reused"
    for v, used in ((view, 6), (sview, 4)):
        full = read(v, "k", v.capacity)
        assert not full[:, used:].any(), "stale data past the new history"
        if kind == "int8":
            assert not read(v, "k_scales", v.capacity)[:, used:].any()
    if kind == F32:
        assert torch.equal(rows_of(view, 1, 2, 6), cat(data(2, 5, d, 100.0), batch_data(3, 2, d, 200.0)[1]))


def test_context_trim_returns_kept_storage_and_caches_stay_valid(device):
    """ppk_context_trim (no counterpart in the reference): the storage of released caches that the context
    keeps for reuse is freed once, live caches keep their contents, and new caches allocate as before."""
    ctx = ppk.context(device)
    trimmed = ctypes.c_uint64()
    _abi.check(_abi.lib().ppk_context_trim(ctx, ctypes.byref(trimmed)), "ppk_context_trim")  # start empty
    keep = LayerCache(F32, 2, 16)
    keep.query(data(2, 40, 16, 1.0), data(2, 40, 16, 1.0), 0, True)
    gone = [LayerCache(F32, 2, 16) for _ in range(3)]
    for c in gone:
        c.query(data(2, 30, 16, 5.0), data(2, 30, 16, 5.0), 0, True)
    reserved = sum(c.info().reserved_bytes for c in gone)
    del gone, c
    _abi.check(_abi.lib().ppk_context_trim(ctx, ctypes.byref(trimmed)), "ppk_context_trim")
    assert trimmed.value >= reserved
    _abi.check(_abi.lib().ppk_context_trim(ctx, ctypes.byref(trimmed)), "ppk_context_trim")
    assert trimmed.value == 0
    assert torch.equal(keep.key(), data(2, 40, 16, 1.0))
    fresh = LayerCache(F32, 2, 16)
    fresh.query(data(2, 3, 16, 9.0), data(2, 3, 16, 9.0), 0, True)
    assert torch.equal(fresh.key(), data(2, 3, 16, 9.0))


def test_allocation_that_runs_out_of_memory_drains_the_kept_storage(device):
    """Released caches are kept for reuse at an equal size only. An arena of another size that does not fit
    beside them (device memory otherwise full) frees them and succeeds on the second try, instead of failing
    while that memory sits idle."""
    gib = 1 << 30
    ppk.kv_arena.trim(device)
    torch.cuda.empty_cache()
    tok = torch.arange(16 * 256, dtype=F32, device=device).reshape(16, 1, 256)
    # Four released caches of 2 GiB each (16 rows x 65536 slots x 256 f32, K and V).
    kept = [LayerCache(F32, 16, 256, max_context=65536, min_capacity=65536) for _ in range(4)]
    for c in kept:
        c.query(tok, tok, 0, True)
    assert kept[0].info().reserved_bytes >= 2 * gib
    del kept, c
    torch.cuda.synchronize()
    free, _ = torch.cuda.mem_get_info(device)
    filler = torch.empty(free - 2 * gib, dtype=torch.uint8, device=device)  # leaves 2 GiB
    try:
        tok24 = torch.arange(24 * 256, dtype=F32, device=device).reshape(24, 1, 256)
        big = LayerCache(F32, 24, 256, max_context=65536, min_capacity=65536)
        big.query(tok24, tok24, 0, True)  # 3 GiB: fits only once the 8 GiB kept are freed
        assert big.info().reserved_bytes >= 3 * gib
        assert torch.equal(big.key(), tok24)
        del big
    finally:
        del filler
        torch.cuda.empty_cache()
    assert ppk.kv_arena.trim(device) < 4 * gib, "the kept storage was not handed back"


def test_truncate_is_metadata_only_and_append_preserves_longer_snapshots(device):
    cache = grouped_rows()[0]
    snapshot = cache.clone()
    saved = snapshot.key().clone()
    owner, nbytes = cache.info().storage_id, cache.info().reserved_bytes
    expect_status(_abi.PPK_PRECONDITION, lambda: cache.truncate_committed(4))
    assert len(cache) == 3
    cache.truncate_committed(1)
    assert cache.info().storage_id == owner and cache.info().reserved_bytes == nbytes
    nxt = data(2, 1, 3, 900.0)
    cache.query(nxt, nxt, 1, True)
    assert cache.info().storage_id != owner
    assert len(snapshot) == 3 and torch.equal(snapshot.key(), saved)
    owner = cache.info().storage_id
    cache.truncate_committed(0)
    assert cache.info().storage_id == owner and cache.key() is None


def test_int8_arena_codes_and_attention_match_the_oracle(device):
    """Int8LayerCache::query_batch (int8_cache.rs:325-359): ragged prefill, grouped decode steps and a
    snapshot branch; codes and scales bit-exact vs the oracle; attention over the arena view (its device
    past vector) vs the f64 oracle."""
    rng = np.random.default_rng(SEED)
    B, H, D = 3, 4, 64
    lens = [5, 1, 33]
    hist = [rng.standard_normal((H, n, D)).astype(np.float32) for n in lens]
    caches = [LayerCache("int8", H, D) for _ in range(B)]
    for b in range(B):
        t = torch.from_numpy(hist[b]).to(device)
        caches[b].query(t, t * 0.5, 0, True)
    model_k = [oracle.quantize(h) for h in hist]
    model_v = [oracle.quantize(h * np.float32(0.5)) for h in hist]
    for step in range(3):
        kn = rng.standard_normal((B, H, 1, D)).astype(np.float32)
        vn = rng.standard_normal((B, H, 1, D)).astype(np.float32)
        past = [len(c) for c in caches]
        view = LayerCache.query_batch(caches, torch.from_numpy(kn).to(device).to(torch.bfloat16),
                                      torch.from_numpy(vn).to(device).to(torch.bfloat16), past, True)
        kb = torch.from_numpy(kn).to(torch.bfloat16).float().numpy()
        vb = torch.from_numpy(vn).to(torch.bfloat16).float().numpy()
        codes_k = read(view, "k", view.length).cpu().numpy()
        scales_k = read(view, "k_scales", view.length).cpu().numpy()
        codes_v = read(view, "v", view.length).cpu().numpy()
        for b in range(B):
            ck, sk, _ = oracle.quantize(kb[b])
            cv, sv, _ = oracle.quantize(vb[b])
            model_k[b] = (np.concatenate([model_k[b][0], ck], 1), np.concatenate([model_k[b][1], sk], 1), 0)
            model_v[b] = (np.concatenate([model_v[b][0], cv], 1), np.concatenate([model_v[b][1], sv], 1), 0)
            n = past[b] + 1
            assert np.array_equal(codes_k[b * H:(b + 1) * H, :n], model_k[b][0])
            assert np.array_equal(scales_k[b * H:(b + 1) * H, :n], model_k[b][1])
            assert np.array_equal(codes_v[b * H:(b + 1) * H, :n], model_v[b][0])
        # Attention over the arena: history [0, past) from the arena, current token unquantised.
        q = rng.standard_normal((B * H, 1, D)).astype(np.float32)
        qt = torch.from_numpy(q).to(device)
        skt = torch.from_numpy(kb.reshape(B * H, 1, D)).to(device)
        svt = torch.from_numpy(vb.reshape(B * H, 1, D)).to(device)
        out = torch.empty((B * H, 1, D), dtype=torch.float32, device=device)
        args = _abi.PpkAttentionArgs(
            struct_size=ctypes.sizeof(_abi.PpkAttentionArgs), rows=B * H, heads=H, capacity=view.capacity,
            head_dim=D, max_past=0, q=qt.data_ptr(), k_codes=view.k, v_codes=view.v, k_scales=view.k_scales,
            v_scales=view.v_scales, sk=skt.data_ptr(), sv=svt.data_ptr(), past=view.past, out=out.data_ptr())
        split, groups, nbytes = ppk.int8_kv_ops.plan(args, ppk.context(device))
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
        args.workspace, args.workspace_bytes = ws.data_ptr(), nbytes
        ppk._abi.check(_abi.lib().ppk_decode_attention(ppk.context(device), None, ctypes.byref(args)), "attn")
        torch.cuda.synchronize()
        cap = view.capacity
        full_k = np.zeros((B * H, cap, D), np.uint8)
        full_v = np.zeros((B * H, cap, D), np.uint8)
        ks = np.ones((B * H, cap), np.float32)
        vs = np.ones((B * H, cap), np.float32)
        for b in range(B):
            n = past[b]
            full_k[b * H:(b + 1) * H, :n] = model_k[b][0][:, :n]
            full_v[b * H:(b + 1) * H, :n] = model_v[b][0][:, :n]
            ks[b * H:(b + 1) * H, :n] = model_k[b][1][:, :n]
            vs[b * H:(b + 1) * H, :n] = model_v[b][1][:, :n]
        ref = oracle.attention(q, full_k, full_v, ks, vs, kb.reshape(B * H, D), vb.reshape(B * H, D),
                               np.array(past, np.uint32), H)
        assert_close(out.reshape(B * H, D).cpu().numpy(), ref, what=f"int8 arena step {step}")
    # A snapshot branch detaches; the original keeps its history.
    branch = [c.clone() for c in caches]
    past = [len(c) for c in caches]
    cur = torch.zeros((B, H, 1, D), device=device)
    LayerCache.query_batch(branch, cur, cur, past, True)
    assert branch[0].info().arena_id != caches[0].info().arena_id
    assert [len(c) for c in caches] == past


def test_float_arena_view_feeds_float_attention(device):
    """A bf16 batch arena (the graph-decode layout) with ragged lengths: ppk_float_decode_attention over
    the view's lengths vector equals the f64 oracle on the model history."""
    rng = np.random.default_rng(SEED + 1)
    B, H, D = 4, 2, 64
    lens = [0, 7, 100, 31]
    caches = [LayerCache(torch.bfloat16, H, D) for _ in range(B)]
    model = []
    for b in range(B):
        h = torch.from_numpy(rng.standard_normal((H, lens[b], D)).astype(np.float32)).to(torch.bfloat16).to(device)
        if lens[b]:
            caches[b].query(h, h, 0, True)
        model.append(h)
    cur = torch.from_numpy(rng.standard_normal((B, H, 1, D)).astype(np.float32)).to(torch.bfloat16).to(device)
    view = LayerCache.query_batch(caches, cur, cur, lens, True)
    q = torch.from_numpy(rng.standard_normal((B * H, 1, D)).astype(np.float32)).to(device)
    out = torch.empty((B * H, 1, D), dtype=torch.float32, device=device)
    a = _abi.PpkFloatAttentionArgs(struct_size=ctypes.sizeof(_abi.PpkFloatAttentionArgs), kv_dtype=_abi.PPK_BF16,
                                   q_dtype=_abi.PPK_F32, out_dtype=_abi.PPK_F32, rows=B * H, heads=H,
                                   size=view.length, head_dim=D, k_row_stride=view.capacity * D,
                                   v_row_stride=view.capacity * D, q=q.data_ptr(), k=view.k, v=view.v,
                                   lengths=view.lengths, out=out.data_ptr())
    _, _, nbytes = ppk.fused_attention.plan(a, ppk.context(device))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
    a.workspace, a.workspace_bytes = ws.data_ptr(), nbytes
    ppk._abi.check(_abi.lib().ppk_float_decode_attention(ppk.context(device), None, ctypes.byref(a)), "fattn")
    torch.cuda.synchronize()
    size = view.length
    kh = np.zeros((B * H, size, D), np.uint16)
    for b in range(B):
        full = torch.cat([model[b], cur[b].reshape(H, 1, D)], 1)
        kh[b * H:(b + 1) * H, :lens[b] + 1] = full.view(torch.int16).cpu().numpy().view(np.uint16)
    ref = oracle.attention_float(q.cpu().numpy(), kh, kh, np.array(lens, np.uint32) + 1, H)
    assert_close(out.reshape(B * H, D).cpu().numpy(), ref, atol=1e-4, rtol=1e-2, what="float arena attention")
