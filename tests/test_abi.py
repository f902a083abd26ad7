"""C-ABI checks that need no GPU: the library loads, exports every function
include/ppk_int8_kv.h declares, its argument structs match the C layout, and
host-side validation refuses bad arguments with status 1 before any launch."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

import ppk
from ppk import _abi
from helpers import SEED

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ppk_int8_kv.h")


def declared_functions() -> list[str]:
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^PPK_API\s+[\w\s\*]+?\b(ppk_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = _abi.lib()
    names = declared_functions()
    assert len(names) >= 14
    for name in names:
        assert hasattr(lib, name), f"libppk.so does not export {name}"
        assert name in _abi.FUNCTIONS, f"ctypes binding lacks {name}"
    out = subprocess.run(["nm", "-D", "--defined-only", _abi.LIB_PATH], capture_output=True, text=True, check=True)
    exported = sorted(set(re.findall(r" T (ppk_\w+)", out.stdout)))
    assert exported == names, "exported C symbols differ from the header's declarations"


def test_code_object_is_built_for_gfx950():
    assert os.path.exists(_abi.HSACO_PATH)
    blob = open(_abi.HSACO_PATH, "rb").read()
    assert b"gfx950" in blob
    for kernel in (b"ppk_quantize_d128", b"ppk_decode_d128", b"ppk_decode_bf16h_d128", b"ppk_attn_merge_d128",
                   b"ppk_dequantize", b"ppk_fdecode_bf16_d64", b"ppk_fdecode_f32_d64", b"ppk_fmerge_d64",
                   b"ppk_renyi_sample", b"ppk_quantize_dense_d64", b"ppk_quantize_dense_d128",
                   b"ppk_quantize_dense_d256", b"ppk_quantize_append_d128", b"ppk_kv_scatter_u16",
                   b"ppk_copy2d_batch"):
        assert kernel in blob


def test_abi_version():
    assert _abi.lib().ppk_abi_version() == _abi.PPK_ABI_VERSION == 1


@pytest.fixture(scope="module")
def c_layout(tmp_path_factory):
    """sizeof/offsetof of every argument struct, as the C compiler lays them out."""
    src = tmp_path_factory.mktemp("abi") / "layout.c"
    exe = src.with_suffix("")
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void){"]
    for cls in (_abi.PpkQuantizeArgs, _abi.PpkAppendArgs, _abi.PpkDequantizeArgs, _abi.PpkAttentionArgs,
                _abi.PpkDecodeStepArgs, _abi.PpkFloatAttentionArgs, _abi.PpkFloatDecodeStepArgs,
                _abi.PpkRenyiSampleArgs, _abi.PpkKvConfig, _abi.PpkKvView, _abi.PpkKvInfo, _abi.PpkKvWrite,
                _abi.PpkInt8KvStatus):
        name = cls.__name__
        lines.append(f'printf("{name} __sizeof__ %zu\\n", sizeof({name}));')
        for field, _ in cls._fields_:
            lines.append(f'printf("{name} {field} %zu\\n", offsetof({name}, {field}));')
    lines.append("return 0;}")
    src.write_text("\n".join(lines))
    subprocess.run(["gcc", "-std=c11", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    return {tuple(line.split()[:2]): int(line.split()[2]) for line in out.splitlines()}


@pytest.mark.parametrize("cls", [_abi.PpkQuantizeArgs, _abi.PpkAppendArgs, _abi.PpkDequantizeArgs,
                                 _abi.PpkAttentionArgs, _abi.PpkDecodeStepArgs, _abi.PpkFloatAttentionArgs,
                                 _abi.PpkFloatDecodeStepArgs, _abi.PpkRenyiSampleArgs, _abi.PpkKvConfig,
                                 _abi.PpkKvView, _abi.PpkKvInfo, _abi.PpkKvWrite, _abi.PpkInt8KvStatus])
def test_struct_layout_matches_c(c_layout, cls):
    name = cls.__name__
    assert c_layout[(name, "__sizeof__")] == ctypes.sizeof(cls)
    for field, _ in cls._fields_:
        assert c_layout[(name, field)] == getattr(cls, field).offset, f"{name}.{field}"


def _attn_args(**kw) -> _abi.PpkAttentionArgs:
    a = _abi.PpkAttentionArgs(struct_size=ctypes.sizeof(_abi.PpkAttentionArgs), q_dtype=0, scratch_dtype=0,
                              out_dtype=0, flags=0, rows=512, heads=16, capacity=8193, head_dim=128,
                              split_tokens=0, max_past=8192, softmax_scale=0.0)
    host = kw.pop("past_host", None)
    for k, v in kw.items():
        setattr(a, k, v)
    if host is not None:
        a._past_host = (ctypes.c_uint32 * len(host))(*[int(x) for x in host])
        a.past_host = ctypes.cast(a._past_host, ctypes.c_void_p).value
    return a


def test_plan_sizes_workspace_without_a_device():
    # Config 5 on 256 CUs: 4 waves x 2048 tokens cover a row (8 waves per CU over
    # the launch), so one block per row finishes the step in one launch and needs
    # no workspace.
    split, groups, nbytes = ppk.int8_kv_ops.plan(_attn_args())
    assert (split, groups, nbytes) == (2048, 1, 0)
    # An explicit per-wave split is honoured (rounded up to whole 1 KiB tiles);
    # int8 blocks hold up to 8 waves, so ceil(ceil(8192/104)/8) blocks per row.
    split, groups, nbytes = ppk.int8_kv_ops.plan(_attn_args(split_tokens=100))
    assert (split, groups) == (104, -(-(-(-8192 // 104)) // 8))
    assert ppk.int8_kv_ops.plan_info(_attn_args(split_tokens=100))["waves_per_block"] == 8
    assert nbytes == 512 * groups * 128 * 4 + -(-(512 * groups * 2 * 4) // 256) * 256
    # Few long rows (config 3 shape): rows split into blocks so the launch covers all 256 CUs, joined by the
    # merge kernel; the waves' shares halved to 32 tokens (one batch at D = 128) so that each block has four
    # waves, one per SIMD of its CU. At D = 64 a batch is 64 tokens: 2-wave blocks stay.
    split, groups, nbytes = ppk.int8_kv_ops.plan(_attn_args(rows=16, capacity=2049, max_past=2048))
    assert split == 32 and groups == 16 and nbytes == 16 * 16 * 128 * 4 + 16 * 16 * 2 * 4
    assert ppk.int8_kv_ops.plan_info(_attn_args(rows=16, capacity=2049, max_past=2048))["waves_per_block"] == 4
    info64 = ppk.int8_kv_ops.plan_info(_attn_args(rows=16, capacity=2049, max_past=2048, head_dim=64))
    assert (info64["split_tokens"], info64["nsplits"], info64["waves_per_block"]) == (64, 16, 2)
    # Uniform host lengths keep the per-row plan.
    assert ppk.int8_kv_ops.plan(_attn_args(rows=16, capacity=2049, max_past=2048, past_host=[2048])) == \
        (split, groups, nbytes)
    # Ragged host lengths whose per-row plan loads one CU with 1.2 x what the balanced plan's busiest CU
    # streams: the balanced plan over 2048 waves (8 per CU). 4 sequences of 8192 tokens beside 28 of 512: the
    # least unit (>= 64 tokens) whose units fit is 456, so rows of 8192 tokens are 18 units (record slots).
    skew = [8192] * 4 + [512] * 28
    split, groups, nbytes = ppk.int8_kv_ops.plan(_attn_args(past_host=skew))
    assert split == 456 and groups == 18 and nbytes == 512 * 18 * 128 * 4 + 512 * 18 * 2 * 4
    # Few ragged rows: the per-row plan already spreads them over every CU (16 four-wave blocks per row), while
    # the balanced plan's 384 units would fill only 96 CUs: per-row kept.
    assert ppk.int8_kv_ops.plan(_attn_args(rows=16, heads=8, capacity=2049, max_past=2048,
                                           past_host=[2048, 1000])) == (32, 16, 16 * 16 * 128 * 4 + 16 * 16 * 8)
    # Short ragged rows with host lengths: the per-row plan covers the longest live row (64 tokens) instead of
    # the span (900: rows cut into four blocks, merged from the workspace), so one block per row, one launch;
    # the same plan as a call whose max_past is that longest row. PPK_ATTN_PLAN_PER_ROW plans as without them.
    span_plan = ppk.int8_kv_ops.plan(_attn_args(rows=64, heads=16, capacity=1024, max_past=900))
    assert span_plan[1] == 4
    host = [10, 0, 60, 64]
    assert ppk.int8_kv_ops.plan(_attn_args(rows=64, heads=16, capacity=1024, max_past=900, past_host=host)) == \
        ppk.int8_kv_ops.plan(_attn_args(rows=64, heads=16, capacity=1024, max_past=64)) == (64, 1, 0)
    assert ppk.int8_kv_ops.plan(_attn_args(rows=64, heads=16, capacity=1024, max_past=900, past_host=host,
                                           flags=_abi.PPK_ATTN_PLAN_PER_ROW)) == span_plan
    # Every host length beyond the span (or zero): the plan covers one token (one 8-token tile per row).
    assert ppk.int8_kv_ops.plan(_attn_args(rows=64, heads=16, capacity=1024, max_past=900,
                                           past_host=[0, 901, 1024, 0])) == (8, 1, 0)
    # Few short rows (config 1 shape): one block per row, one launch.
    assert ppk.int8_kv_ops.plan(_attn_args(rows=16, capacity=513, max_past=512, head_dim=64)) == (64, 1, 0)
    # A row one block covers (at most 128 KiB of history) that the budget would give 15 waves of 64 tokens
    # keeps at most 8 int8 waves, each a longer share: 900 / 8 = 113 -> 128 (16-token tiles at D = 64).
    info = ppk.int8_kv_ops.plan_info(_attn_args(rows=64, capacity=1024, max_past=900, head_dim=64))
    assert (info["split_tokens"], info["nsplits"], info["waves_per_block"], info["launches"]) == (128, 1, 8, 1)
    # Fewer rows than CUs whose blocks would not all fit the CUs' eight int8 wave slots at once (192 rows x
    # 4096 tokens at D = 64: 3 groups of 4-wave blocks, 576 > 512 resident): one 8-wave block per row, 4096 / 8
    # = 512 tokens a wave, one launch. Rows eight waves cannot cover (2048 tokens a wave at most) keep a
    # split plan; so do grids that fit one round.
    for rows, span, d, want in ((192, 4096, 64, (512, 1, 8, 192, 1)), (160, 1024, 128, (128, 1, 8, 160, 1)),
                                (192, 1500, 128, (192, 1, 8, 192, 1)), (224, 8192, 64, (1024, 1, 8, 224, 1))):
        info = ppk.int8_kv_ops.plan_info(_attn_args(rows=rows, capacity=span + 1, max_past=span, head_dim=d))
        got = (info["split_tokens"], info["nsplits"], info["waves_per_block"], info["blocks"], info["launches"])
        assert got == want, (rows, span, d, got)
    # Larger blocks where they land evenly (the row's waves split exactly, the busiest CU within 7 % of the
    # mean): 128 rows x 8192 as two 8-wave blocks a row (256 blocks, one a CU) instead of sixteen 1-wave
    # blocks; 48 rows x 8192 keeps 2-wave blocks (4-wave ones would give the busiest CUs 8 waves, mean 6).
    for rows, span, want in ((128, 8192, (512, 2, 8)), (48, 8192, (256, 16, 2))):
        info = ppk.int8_kv_ops.plan_info(_attn_args(rows=rows, capacity=span + 1, max_past=span))
        assert (info["split_tokens"], info["nsplits"], info["waves_per_block"]) == want, (rows, span, info)
    # And smaller blocks where the chosen ones land unevenly and smaller ones evenly, at most 16 a row: 80 rows
    # x 1024 at D = 128 (four 4-wave blocks, 320 on 256 CUs) takes sixteen 1-wave blocks (1280, five a CU);
    # 48 x 4096 at D = 64 two-wave blocks; 16 rows x 3000 at D = 128 keeps its plan (an even split would be 47
    # blocks a row).
    for rows, span, d, want in ((80, 1024, 128, (64, 16, 1)), (48, 4096, 64, (128, 16, 2)),
                                (16, 3000, 128, (32, 24, 4))):
        info = ppk.int8_kv_ops.plan_info(_attn_args(rows=rows, capacity=span + 1, max_past=span, head_dim=d))
        assert (info["split_tokens"], info["nsplits"], info["waves_per_block"]) == want, (rows, span, d, info)
    for rows, span in ((192, 8192), (144, 4096)):
        info = ppk.int8_kv_ops.plan_info(_attn_args(rows=rows, capacity=span + 1, max_past=span))
        assert info["launches"] == 2 and info["blocks"] * info["waves_per_block"] <= 256 * 8, (rows, span, info)
    info = ppk.int8_kv_ops.plan_info(_attn_args(rows=240, capacity=20001, max_past=20000))
    assert info["split_tokens"] <= 2048 and info["launches"] == 2
    # At least as many rows as CUs, where the budget gives each row 3, 5, 6 or 7 waves (one block each, a second
    # round): short rows take a power-of-two number of waves in one block (384 x 1024 at D = 64: 4 waves of 256
    # tokens; the busiest CUs stream 139 KB a row more than the mean share, half a row), longer ones keep their
    # waves in 1- or 2-wave blocks that fill the CUs' slots, joined by the merge (384 x 8192 at D = 128: five
    # 1640-token waves as 1-wave blocks; 320 x 4096: six waves as three 2-wave blocks).
    for rows, span, d, want in ((384, 1024, 64, (256, 1, 4, 384, 1)), (384, 8192, 128, (1640, 5, 1, 1920, 2)),
                                (320, 4096, 128, (688, 3, 2, 960, 2)), (288, 700, 128, (176, 1, 4, 288, 1))):
        info = ppk.int8_kv_ops.plan_info(_attn_args(rows=rows, capacity=span + 1, max_past=span, head_dim=d))
        got = (info["split_tokens"], info["nsplits"], info["waves_per_block"], info["blocks"], info["launches"])
        assert got == want, (rows, span, d, got)
    for rows in range(256, 1100, 16):
        for span in (700, 1024, 3000, 4096, 8192):
            for d in (64, 128):
                info = ppk.int8_kv_ops.plan_info(_attn_args(rows=rows, capacity=span + 1, max_past=span, head_dim=d))
                resident = 256 * (8 // info["waves_per_block"])
                waves = rows * -(-span // info["split_tokens"])
                assert info["blocks"] <= resident or waves > 256 * 8, (rows, span, d, info)
    # Spans that are no multiple of the power-of-two split: each row gets as many waves as the budget holds
    # (2048 / 512 rows = 4) with equal shares rounded up to whole tiles (1100 / 4 = 275 -> 280 for the int8
    # path's 8-token tiles, 276 for bf16's 4-token tiles at D = 128), one block per row.
    assert ppk.int8_kv_ops.plan(_attn_args(capacity=1101, max_past=1100)) == (280, 1, 0)
    assert ppk.int8_kv_ops.plan(_attn_args(rows=256, capacity=1501, max_past=1500)) == (192, 1, 0)
    assert ppk.fused_attention.plan(_float_args(size=1100)) == (276, 1, 0)
    # The float path with at least as many rows as CUs: one block per row leaves the busiest CUs a whole row
    # more than the mean (288 rows: 2 against 1.125), so the row's waves go to small blocks spread evenly over
    # the CUs (seven 1-wave blocks of 588 tokens, 2016 blocks) and the merge; at 448 rows (1.75 of 2) HBM sets
    # the time and the one-block plan stays; 512 rows are even already.
    for rows, size, d, want in ((288, 4096, 128, (588, 7, 1)), (576, 1024, 128, (344, 3, 1)),
                                (448, 4096, 128, (1024, 1, 4)), (512, 8192, 128, (2048, 1, 4))):
        info = ppk.fused_attention.plan_info(_float_args(rows=rows, size=size, head_dim=d))
        assert (info["split_tokens"], info["nsplits"], info["waves_per_block"]) == want, (rows, size, d, info)


def _cu_peaks(lens, heads, per_row, share, cus=256, waves_per_block=4):
    """Most live tokens one CU streams under the per-row plan (split S, W waves per block, G groups; block
    g * rows + r on CU (g * rows + r) mod cus) and under the balanced plan (unit u on block u / 4, same
    placement); lens are the live lengths per sequence."""
    S, W, G = per_row
    rows = len(lens) * heads
    row_cu = np.zeros(cus, np.int64)
    for r in range(rows):
        n = lens[r // heads]
        for g in range(G):
            row_cu[(g * rows + r) % cus] += max(0, min(W * S, n - g * W * S))
    flat_cu = np.zeros(cus, np.int64)
    u = 0
    for n in lens:
        for _ in range(heads):
            for s in range(max(1, -(-n // share))):
                flat_cu[(u // waves_per_block) % cus] += max(0, min(share, n - s * share))
                u += 1
    return int(row_cu.max()), int(flat_cu.max())


def _balanced_pays(lens, heads, per_row, share, flat_groups, token_bytes):
    """The library's pick between the plans: a modelled step of a fixed cost (per-row 4.75 us for one launch,
    7.3 us with the merge; balanced 7.0 / 9.9 us), plus the live history streamed at 27.8 (per-row) / 27.2
    (balanced) GB/s per CU over 256 CUs, plus the busiest CU's bytes beyond the mean at 64 / 63 GB/s; balanced
    when modelled faster, or when per-row waves stream 256 KiB or more each and the per-row plan's busiest CU
    streams at least 1.2 x the balanced plan's."""
    S, W, G = per_row
    row_peak, flat_peak = _cu_peaks(lens, heads, per_row, share, waves_per_block=W)
    flat_peak = _cu_peaks(lens, heads, per_row, share)[1]
    total = sum(lens) * heads * token_bytes

    def modelled(peak, merge, one, merged, stream, excess):
        return (merged if merge else one) + total / (stream * 256) + max(0.0, peak * token_bytes - total / 256) / excess

    return (modelled(flat_peak, flat_groups > 1, 7.0, 9.9, 27.2e3, 63e3)
            < modelled(row_peak, G > 1, 4.75, 7.3, 27.8e3, 64e3)
            or (S * token_bytes >= 256 << 10 and 5 * row_peak >= 6 * flat_peak))


def _flat_units(past, heads, rows, capacity, span, waves, min_unit=64):
    """Units per row of the balanced plan from the host lengths: live length past[b] (0 beyond
    min(capacity, span)), a row of len tokens is max(1, ceil(len / Q)) units of at most Q tokens, Q the least
    share >= 64 whose units fit the waves (found here by a linear scan); returns (units per row, Q)."""
    lens = [p if p <= capacity and p <= span else 0 for p in past]
    share = min_unit
    while sum(heads * max(1, -(-length // share)) for length in lens) > waves:
        share += 1
    return [max(1, -(-length // share)) for length in lens for _ in range(heads)], share


@pytest.mark.parametrize("heads,d", [(16, 128), (1, 64), (4, 256), (8, 128)])
def test_balanced_plan_covers_every_row_within_the_waves(heads, d):
    """Ragged batches of up to 64 sequences (zero, tiny, capacity-long and past-capacity rows) with host
    lengths: the balanced plan is taken when the longest live row exceeds 1.1 x the mean (and rows fit half
    the waves) and the timing model of both plans favours it (_balanced_pays); its units cover every live token, never outnumber the launched waves (2048 on the 256 CUs assumed without a
    context), and the record slots per row are the most units of any row."""
    rng = np.random.default_rng(SEED + heads + d)
    checked = 0
    for trial in range(500):
        batch = int(rng.integers(1, 65))
        cap = int(rng.choice([64, 700, 4096, 30000]))
        span = int(rng.choice([cap, max(1, cap // 3)]))
        kind = trial % 4
        if kind == 0:
            past = rng.integers(0, span + 1, batch)
        elif kind == 1:  # one long row among empty ones
            past = np.zeros(batch, np.int64)
            past[int(rng.integers(batch))] = span
        elif kind == 2:  # all at the span, one past the capacity
            past = np.full(batch, span)
            past[0] = cap + 1
        else:  # tiny rows and a few long ones
            past = rng.integers(0, 3, batch)
            past[rng.integers(0, batch, 3)] = span
        rows = batch * heads
        a = _attn_args(rows=rows, heads=heads, capacity=cap, max_past=span, head_dim=d, past_host=past)
        live = [int(p) if p <= min(cap, span) else 0 for p in past]
        # The per-row plan with host lengths covers the longest live row (at least one token).
        cover = max(1, max(live))
        per_row_args = _attn_args(rows=rows, heads=heads, capacity=cap, max_past=cover, head_dim=d)
        per_row = ppk.int8_kv_ops.plan(per_row_args)
        # The per-row plan's block size as the library reports it (its sizing rules are pinned by the plan
        # tests above); the balanced-or-per-row choice below is restated independently.
        per_row_waves = ppk.int8_kv_ops.plan_info(per_row_args)["waves_per_block"]
        split, groups, nbytes = ppk.int8_kv_ops.plan(a)
        if 2 * rows > 2048 or max(live) * batch * 10 <= sum(live) * 11:  # too many rows, or not ragged
            assert (split, groups, nbytes) == per_row
            continue
        units, share = _flat_units([int(p) for p in past], heads, rows, cap, span, 2048)
        S, G = per_row[:2]
        if not _balanced_pays(live, heads, (S, per_row_waves, G), share, max(units),
                              2 * d + 8):
            assert (split, groups, nbytes) == per_row, "per-row plan kept"
            # The balanced plan, forced, still covers the rows as below.
            a = _attn_args(rows=rows, heads=heads, capacity=cap, max_past=span, head_dim=d, past_host=past,
                           flags=_abi.PPK_ATTN_PLAN_BALANCED)
            split, groups, nbytes = ppk.int8_kv_ops.plan(a)
        assert split == share and groups == max(units)
        assert sum(units) <= 2048, "every unit has a wave"
        for p, u in zip(np.repeat(past, heads), units):
            live = int(p) if p <= min(cap, span) else 0
            assert u * share >= live and (u - 1) * share < max(live, 1)
        assert nbytes == (0 if groups == 1 else rows * groups * d * 4 + -(-(rows * groups * 8) // 256) * 256)
        checked += 1
    assert checked > 60


@pytest.mark.parametrize("bad", [dict(head_dim=96), dict(rows=30, heads=16), dict(heads=0), dict(capacity=0),
                                 dict(q_dtype=7), dict(flags=8), dict(max_past=9000),
                                 dict(softmax_scale=float("nan")), dict(struct_size=8)])
def test_invalid_attention_arguments_are_refused_before_launch(bad):
    with pytest.raises(ppk.PpkPreconditionError):
        ppk.int8_kv_ops.plan(_attn_args(**bad))
    assert "HIP_PREPARATION" in _abi.lib().ppk_last_error().decode()


def test_null_context_calls_return_status_1():
    lib = _abi.lib()
    a = _attn_args()
    assert lib.ppk_decode_attention(None, None, ctypes.byref(a)) == _abi.PPK_PRECONDITION
    q = _abi.PpkQuantizeArgs(struct_size=ctypes.sizeof(_abi.PpkQuantizeArgs))
    assert lib.ppk_quantize(None, None, ctypes.byref(q)) == _abi.PPK_PRECONDITION
    assert lib.ppk_prepare(None) == _abi.PPK_PRECONDITION
    step = _abi.PpkDecodeStepArgs(struct_size=ctypes.sizeof(_abi.PpkDecodeStepArgs), attn=a)
    assert lib.ppk_decode_step(None, None, ctypes.byref(step)) == _abi.PPK_PRECONDITION
    assert lib.ppk_context_release(None) == _abi.PPK_OK


def _float_args(**kw) -> _abi.PpkFloatAttentionArgs:
    a = _abi.PpkFloatAttentionArgs(struct_size=ctypes.sizeof(_abi.PpkFloatAttentionArgs), kv_dtype=_abi.PPK_BF16,
                                   q_dtype=0, out_dtype=0, rows=512, heads=16, size=8192, head_dim=128,
                                   split_tokens=0, max_length=0, softmax_scale=0.0)
    host = kw.pop("lengths_host", None)
    for k, v in kw.items():
        setattr(a, k, v)
    if host is not None:
        a._lengths_host = (ctypes.c_uint32 * len(host))(*[int(x) for x in host])
        a.lengths_host = ctypes.cast(a._lengths_host, ctypes.c_void_p).value
    return a


def test_float_plan_without_a_device():
    # Long rows, many of them: one 4-wave block per row, a single launch.
    assert ppk.fused_attention.plan(_float_args()) == (2048, 1, 0)
    # The reference's graph-decode shape (16 rows of a 1024-token bf16 store, D = 64):
    # 16 one-wave groups per row cover the CUs; merge workspace y + (m, z) records.
    split, groups, nbytes = ppk.fused_attention.plan(_float_args(rows=16, size=1024, head_dim=64))
    assert (split, groups) == (64, 16)
    assert nbytes == 16 * 16 * 64 * 4 + -(-(16 * 16 * 2 * 4) // 256) * 256
    # Few long rows with blocks of fewer than four waves: the waves' share is halved while a wave keeps at
    # least 16 KiB of K and V: bf16 D = 128 x 2048 tokens, 32-token waves (16 KiB) in 4-wave blocks; the
    # graph-decode shape above (bf16 D = 64, 16 KiB per 64-token wave) keeps its one-wave blocks.
    info = ppk.fused_attention.plan_info(_float_args(rows=16, size=2048, head_dim=128))
    assert (info["split_tokens"], info["nsplits"], info["waves_per_block"]) == (32, 16, 4)
    assert ppk.fused_attention.plan_info(_float_args(rows=16, size=1024, head_dim=64))["waves_per_block"] == 1
    # Explicit split: whole wave loads of tokens (f32, D = 128: 2 tokens per 1 KiB load).
    split, groups, _ = ppk.fused_attention.plan(_float_args(kv_dtype=_abi.PPK_F32, split_tokens=33))
    assert split == 34 and groups == -(-(-(-8192 // 34)) // 16)
    # max_length bounds the planned span.
    assert ppk.fused_attention.plan(_float_args(max_length=1024, lengths=8))[:2] == (256, 1)


def test_float_balanced_plan_without_a_device():
    """Host lengths of a ragged batch take the balanced plan of the int8 path (the same table from the same
    rule); uniform lengths, an explicit split or a batch beyond 64 sequences keep the per-row plan (sized for the
    longest host length)."""
    skew = [8192] * 4 + [512] * 28
    per_row = ppk.fused_attention.plan(_float_args(lengths=8))
    split, groups, nbytes = ppk.fused_attention.plan(_float_args(lengths=8, lengths_host=skew))
    units, share = _flat_units(skew, 16, 512, 8192, 8192, 2048)
    assert (split, groups) == (share, max(units)) and groups > 1
    assert nbytes == 512 * groups * 128 * 4 + -(-(512 * groups * 8) // 256) * 256
    # The same table as the int8 plan of the same lengths.
    assert ppk.int8_kv_ops.plan(_attn_args(rows=512, capacity=8192, max_past=8192, past_host=skew))[:2] == \
        (split, groups)
    assert ppk.fused_attention.plan(_float_args(lengths=8, lengths_host=[8192] * 32)) == per_row
    assert ppk.fused_attention.plan(_float_args(lengths=8, lengths_host=skew, split_tokens=128)) == \
        ppk.fused_attention.plan(_float_args(split_tokens=128))
    # Beyond 64 sequences: the per-row plan, covering the longest host length (5000 of the 8192 slots) as a call
    # with that max_length would; PPK_ATTN_PLAN_PER_ROW plans as without the host lengths.
    many = [5000] + [10] * 79
    assert ppk.fused_attention.plan(_float_args(rows=80, heads=1, lengths=8, lengths_host=many)) == \
        ppk.fused_attention.plan(_float_args(rows=80, heads=1, lengths=8, max_length=5000)) != \
        ppk.fused_attention.plan(_float_args(rows=80, heads=1, lengths=8))
    assert ppk.fused_attention.plan(_float_args(rows=80, heads=1, lengths=8, lengths_host=many,
                                                flags=_abi.PPK_ATTN_PLAN_PER_ROW)) == \
        ppk.fused_attention.plan(_float_args(rows=80, heads=1, lengths=8))
    # Lengths beyond max_length count as empty rows (NaN): one live long row among them.
    host = [8000, 9000, 10, 0] + [600] * 28
    split, groups, _ = ppk.fused_attention.plan(_float_args(max_length=8100, lengths=8, lengths_host=host))
    units, share = _flat_units(host, 16, 512, 8192, 8100, 2048)
    assert (split, groups) == (share, max(units))
    # Few rows: the per-row plan's waves (128 tokens, 33 per row of 4000) are already even; kept.
    few = _float_args(rows=64, heads=16, max_length=4000, lengths=8)
    assert ppk.fused_attention.plan(_float_args(rows=64, heads=16, max_length=4000, lengths=8,
                                                lengths_host=[4000, 9000, 10, 0])) == ppk.fused_attention.plan(few)
    # Even per-row waves in a large batch: 8 sequences of 4096 tokens beside 24 of 1024 take 1024-token waves
    # everywhere (the balanced plan measured slower there); kept.
    even = [4096] * 8 + [1024] * 24
    assert ppk.fused_attention.plan(_float_args(size=4096, lengths=8, lengths_host=even)) == \
        ppk.fused_attention.plan(_float_args(size=4096, lengths=8))
    # A ragged batch whose longest row holds at most 512 KiB of K and V keeps the per-row plan (one launch
    # there beats the balanced plan's two): bf16, D = 64, 1024 tokens is 256 KiB; f32 is 512 KiB.
    short = [1024] * 4 + [64] * 28
    for kv, d, flat in ((_abi.PPK_BF16, 64, False), (_abi.PPK_F32, 64, False), (_abi.PPK_F32, 128, True)):
        base = dict(kv_dtype=kv, head_dim=d, size=1024, lengths=8)
        got = ppk.fused_attention.plan(_float_args(lengths_host=short, **base))
        assert (got != ppk.fused_attention.plan(_float_args(**base))) == flat, (kv, d)
    # Host lengths need the device lengths; an argument block that ends before lengths_host is still taken.
    with pytest.raises(ppk.PpkPreconditionError):
        ppk.fused_attention.plan(_float_args(lengths_host=skew))
    old = _float_args(lengths=8, lengths_host=skew)
    old.struct_size = _abi.PpkFloatAttentionArgs.lengths_host.offset
    assert ppk.fused_attention.plan(old) == per_row


def test_plan_flags_fix_the_choice():
    """PPK_ATTN_PLAN_PER_ROW / _BALANCED override the library's choice between its two plans (int8 and float);
    BALANCED needs host lengths, split_tokens == 0 and a batch within the balanced plan's limits."""
    P, B = _abi.PPK_ATTN_PLAN_PER_ROW, _abi.PPK_ATTN_PLAN_BALANCED
    skew, uniform = [8192] * 4 + [512] * 28, [8192] * 32
    per_row = ppk.int8_kv_ops.plan(_attn_args())
    balanced = ppk.int8_kv_ops.plan(_attn_args(past_host=skew))
    assert balanced != per_row
    assert ppk.int8_kv_ops.plan(_attn_args(past_host=skew, flags=P)) == per_row
    units, share = _flat_units(uniform, 16, 512, 8193, 8192, 2048)
    assert ppk.int8_kv_ops.plan(_attn_args(past_host=uniform, flags=B))[:2] == (share, max(units))
    assert ppk.int8_kv_ops.plan(_attn_args(past_host=uniform, flags=B | _abi.PPK_ATTN_BF16_HISTORY))[:2] == \
        (share, max(units))
    # Short rows that the library keeps per-row: forced balanced, every row one unit (no records, no merge).
    assert ppk.int8_kv_ops.plan(_attn_args(rows=64, heads=16, capacity=1024, max_past=900, flags=B,
                                           past_host=[10, 0, 60, 64])) == (64, 1, 0)
    fl_per_row = ppk.fused_attention.plan(_float_args(lengths=8))
    assert ppk.fused_attention.plan(_float_args(lengths=8, lengths_host=skew, flags=P)) == fl_per_row
    assert ppk.fused_attention.plan(_float_args(lengths=8, lengths_host=uniform, flags=B))[:2] == (share, max(units))
    for bad in (dict(flags=P | B, past_host=skew), dict(flags=B), dict(flags=B, past_host=skew, split_tokens=128),
                dict(flags=B, rows=65 * 16, heads=16, past_host=[100] * 65),
                dict(flags=B, rows=1040, heads=1040, past_host=[100])):
        with pytest.raises(ppk.PpkPreconditionError):
            ppk.int8_kv_ops.plan(_attn_args(**bad))
    for bad in (dict(flags=P | B, lengths_host=skew), dict(flags=B), dict(flags=B, lengths_host=skew, split_tokens=64),
                dict(flags=8, lengths_host=skew), dict(flags=_abi.PPK_ATTN_BF16_HISTORY)):
        with pytest.raises(ppk.PpkPreconditionError):
            ppk.fused_attention.plan(_float_args(lengths=8, **bad))
    assert "PPK_ATTN_PLAN" in _abi.lib().ppk_last_error().decode() or "flags" in _abi.lib().ppk_last_error().decode()
    with pytest.raises(ValueError):
        _abi.plan_flags("fastest")


@pytest.mark.parametrize("bad", [dict(kv_dtype=_abi.PPK_F16), dict(head_dim=96), dict(size=0), dict(rows=30),
                                 dict(q_dtype=5), dict(out_dtype=9), dict(k_row_stride=8191 * 128),
                                 dict(v_row_stride=8192 * 128 + 4), dict(max_length=8193),
                                 dict(max_length=100), dict(softmax_scale=-1.0), dict(struct_size=16)])
def test_invalid_float_attention_arguments_are_refused_before_launch(bad):
    with pytest.raises(ppk.PpkPreconditionError):
        ppk.fused_attention.plan(_float_args(**bad))
    assert "HIP_PREPARATION" in _abi.lib().ppk_last_error().decode()


def test_float_attention_null_context_returns_status_1():
    a = _float_args()
    assert _abi.lib().ppk_float_decode_attention(None, None, ctypes.byref(a)) == _abi.PPK_PRECONDITION


def _sample_args(**kw) -> _abi.PpkRenyiSampleArgs:
    a = _abi.PpkRenyiSampleArgs(struct_size=ctypes.sizeof(_abi.PpkRenyiSampleArgs), batch=2, choices=128,
                                guidance=1, alpha=3.5, cfg=1.0, token_offset=100, raw=8, uniforms=8, bounds=8, out=8)
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("bad", [dict(alpha=1.0), dict(alpha=0.0), dict(alpha=float("nan")), dict(alpha=float("inf")),
                                 dict(cfg=-1.0), dict(cfg=float("nan")), dict(cfg=float("inf")), dict(cfg=2.0),
                                 dict(guidance=3), dict(token_offset=2**32 - 1), dict(choices=2049),
                                 dict(choices=0), dict(batch=0), dict(raw=None), dict(out=6),
                                 dict(struct_size=8)])
def test_invalid_sampler_metadata_is_refused_before_launch(bad):
    """hip_sampling.rs:209-245 (validates_metadata_and_refuses_host_mathematics,
    supports_cfg_pairs_offsets_and_rejects_wrong_shapes): the same rules, at the C-ABI."""
    # A stand-in context pointer: every case fails validation, which precedes any use of the context.
    a = _sample_args(**bad)
    assert _abi.lib().ppk_renyi_sample(ctypes.c_void_p(16), None, ctypes.byref(a)) == _abi.PPK_PRECONDITION
    msg = _abi.lib().ppk_last_error().decode()
    assert msg.startswith("HIP_PREPARATION") and "null context" not in msg


def test_sampler_python_mirror_refuses_cpu_tensors_and_bad_shapes():
    import torch

    raw = torch.zeros((4, 270))
    u = torch.zeros((2, 1))
    b = torch.zeros((2, 2), dtype=torch.int32)
    with pytest.raises(RuntimeError, match="no CPU/CUDA fallback"):
        ppk.sampling.sample(raw, u, b, 3.5, 2.5, 2, 2048)
    with pytest.raises(ValueError):
        ppk.sampling.sample(torch.zeros((4, 2049)), u, b, 4.0, 2.0, 2, 0)
    with pytest.raises(ValueError):
        ppk.sampling.sample(raw.to(torch.bfloat16), u, b, 4.0, 2.0, 2, 0)
    with pytest.raises(ValueError):
        ppk.sampling.sample(raw, torch.zeros((2, 2))[:, :1], b, 4.0, 2.0, 2, 0)
    with pytest.raises(ValueError):
        ppk.sampling.sample(raw, u, b, 4.0, 2.0, 1, 0)


def test_kv_arena_entry_points_refuse_null_arguments():
    lib = _abi.lib()
    cfg = _abi.PpkKvConfig(struct_size=ctypes.sizeof(_abi.PpkKvConfig), kind=0, heads=2, head_dim=64)
    out = ctypes.c_void_p(123)
    assert lib.ppk_kv_cache_create(None, ctypes.byref(cfg), ctypes.byref(out)) == _abi.PPK_PRECONDITION
    assert out.value is None
    assert lib.ppk_kv_cache_clone(None, ctypes.byref(out)) == _abi.PPK_PRECONDITION
    assert lib.ppk_kv_cache_info(None, None) == _abi.PPK_PRECONDITION
    assert lib.ppk_kv_cache_truncate(None, 0) == _abi.PPK_PRECONDITION
    out = ctypes.c_void_p(123)
    cfg.kind = _abi.PPK_KV_F32
    assert lib.ppk_kv_cache_adopt(None, ctypes.byref(cfg), 256, 4096, 8, 0, ctypes.byref(out)) == _abi.PPK_PRECONDITION
    assert out.value is None
    assert lib.ppk_kv_cache_advance(None, 0, 1) == _abi.PPK_PRECONDITION
    released = ctypes.c_uint64(7)
    assert lib.ppk_context_trim(None, ctypes.byref(released)) == _abi.PPK_PRECONDITION
    assert released.value == 0
    w = _abi.PpkKvWrite(struct_size=ctypes.sizeof(_abi.PpkKvWrite))
    assert lib.ppk_kv_query(None, None, None, 0, ctypes.byref(w), None) == _abi.PPK_PRECONDITION
    assert lib.ppk_kv_query_batch(None, None, None, 0, None, ctypes.byref(w), None, None) == _abi.PPK_PRECONDITION
    assert lib.ppk_write_plan_create(None, None, None, 0, 1, 1, ctypes.byref(out)) == _abi.PPK_PRECONDITION
    assert lib.ppk_kv_cache_release(None) == _abi.PPK_OK
    assert lib.ppk_write_plan_release(None) == _abi.PPK_OK


def test_int8_gate_refuses_null_context():
    st = _abi.PpkInt8KvStatus(struct_size=ctypes.sizeof(_abi.PpkInt8KvStatus))
    assert _abi.lib().ppk_prepare_int8_kv(None, 1, 64, ctypes.byref(st)) == _abi.PPK_PRECONDITION


def test_error_text_is_thread_local():
    """Two threads failing different checks concurrently each read back their own message
    (the reference keeps its last error per thread, painter_ffi.cpp:12,18-19). Host-only calls."""
    import threading

    lib = _abi.lib()
    bad = {"max_past": "max_past exceeds capacity", "q_dtype": "dtype must be f32, bf16 or f16"}
    seen = {k: set() for k in bad}

    def worker(field):
        a = _abi.PpkAttentionArgs(struct_size=ctypes.sizeof(_abi.PpkAttentionArgs), rows=16, heads=16,
                                  capacity=64, head_dim=64)
        setattr(a, field, 1000 if field == "max_past" else 7)
        for _ in range(2000):
            assert lib.ppk_attention_plan(None, ctypes.byref(a), None, None, None) == _abi.PPK_PRECONDITION
            seen[field].add(lib.ppk_last_error().decode())

    threads = [threading.Thread(target=worker, args=(f,)) for f in bad]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    for field, texts in seen.items():
        assert len(texts) == 1 and bad[field] in next(iter(texts)), (field, texts)


def test_plan_info_reports_the_plan_taken():
    """ppk_attention_plan_info / ppk_float_attention_plan_info (no device: 256 CUs): the plan kind the
    library takes, its grid and launches, consistent with ppk_attention_plan."""
    skew = [8192] * 4 + [512] * 28
    info = ppk.int8_kv_ops.plan_info(_attn_args())  # config 5: one 4-wave block per row, one launch
    assert info == {"kind": "per-row", "split_tokens": 2048, "nsplits": 1, "waves_per_block": 4, "blocks": 512,
                    "launches": 1, "workspace_bytes": 0}
    info = ppk.int8_kv_ops.plan_info(_attn_args(split_tokens=100))  # 8-wave blocks, merge launch
    split, groups, nbytes = ppk.int8_kv_ops.plan(_attn_args(split_tokens=100))
    assert (info["split_tokens"], info["nsplits"], info["workspace_bytes"]) == (split, groups, nbytes)
    assert info["kind"] == "per-row" and info["waves_per_block"] == 8 and info["blocks"] == 512 * groups
    assert info["launches"] == 2
    info = ppk.int8_kv_ops.plan_info(_attn_args(past_host=skew))
    assert info["kind"] == "balanced" and info["launches"] == 2
    assert (info["split_tokens"], info["nsplits"], info["workspace_bytes"]) == ppk.int8_kv_ops.plan(
        _attn_args(past_host=skew))
    info = ppk.int8_kv_ops.plan_info(_attn_args(past_host=skew, flags=_abi.PPK_ATTN_PLAN_PER_ROW))
    assert info["kind"] == "per-row"
    finfo = ppk.fused_attention.plan_info(_float_args(lengths=8, lengths_host=skew))
    assert finfo["kind"] == "balanced"
    assert ppk.fused_attention.plan_info(_float_args(lengths=8))["kind"] == "per-row"
    small = _abi.PpkAttentionPlanInfo(struct_size=8)
    assert _abi.lib().ppk_attention_plan_info(None, ctypes.byref(_attn_args()), ctypes.byref(small)) == \
        _abi.PPK_PRECONDITION


def test_auto_plans_respect_the_kernels_limits():
    """Every automatic plan, over row counts around the CU count and its multiples, spans from one token to
    65536 and D = 64 / 128 / 256: int8 blocks of 1-8 waves, float blocks of 1-16, at most 16384 tokens per
    block (one float of LDS per token), and the groups cover the span."""
    rows_list = [1, 3, 16, 100, 255, 256, 257, 288, 384, 448, 511, 512, 513, 640, 1000, 2048, 4096]
    spans = [1, 63, 64, 65, 300, 1024, 1445, 2048, 3000, 8192, 12000, 20000, 65536]
    for rows in rows_list:
        for span in spans:
            for d in (64, 128, 256):
                i = ppk.int8_kv_ops.plan_info(_attn_args(rows=rows, heads=1, capacity=span + 1, max_past=span,
                                                         head_dim=d))
                w, s = i["waves_per_block"], i["split_tokens"]
                assert 1 <= w <= 8 and w * s <= 16384 and i["nsplits"] * w * s >= span, (rows, span, d, i)
                i = ppk.fused_attention.plan_info(_float_args(rows=rows, heads=1, size=span + 1, max_length=span,
                                                              head_dim=d, lengths=8))
                w, s = i["waves_per_block"], i["split_tokens"]
                assert 1 <= w <= 16 and w * s <= 16384 and i["nsplits"] * w * s >= span, (rows, span, d, i)
