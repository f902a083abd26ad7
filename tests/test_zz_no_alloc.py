"""GPU checks of ppk_decode_step_noalloc, the decode step that allocates nothing.

It must give what ppk_decode_step gives on the same inputs (same kernels and
plan: outputs and appended arena slots bit-identical), on two calls in a row,
the second with a smaller input, and stay within the oracle's bar; a plan
whose workspace exceeds the library's scratch array is refused with status 1
before anything is enqueued. Calls go through the C-ABI (ctypes).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import ppk
from helpers import SEED, assert_close
from ppk import _abi
from test_gpu_attention import Case

pytestmark = pytest.mark.gpu


def _step_args(c: Case, out: torch.Tensor, workspace: torch.Tensor | None, split: int = 0):
    a, _ = ppk.int8_kv_ops.attention_args(c.q, c.kc, c.vc, c.ks, c.vs, c.sk, c.sv, c.past_t, c.H, split,
                                          max_past=int(c.past.max()), out=out)
    step = ppk.int8_kv_ops._step_args(a, c.sk, c.sv, None, c.D)
    if workspace is not None:
        step.attn.workspace = workspace.data_ptr()
        step.attn.workspace_bytes = workspace.numel()
    return step


def _run_both(device, c: Case) -> tuple[np.ndarray, int]:
    """ppk_decode_step on one copy of the arenas, ppk_decode_step_noalloc on another; both compared."""
    lib = _abi.lib()
    ctx = ppk.context(device)
    stream = ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
    arenas = [t.clone() for t in (c.kc, c.vc, c.ks, c.vs)]
    out_ref = torch.full((c.rows, 1, c.D), float("nan"), dtype=torch.float32, device=device)
    probe = _step_args(c, out_ref, None)
    _, ngroups, nbytes = ppk.int8_kv_ops.plan(probe.attn, ctx)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
    step = _step_args(c, out_ref, ws)
    assert lib.ppk_decode_step(ctx, stream, ctypes.byref(step)) == 0, _abi.last_error()
    ref_arenas = [t.clone() for t in (c.kc, c.vc, c.ks, c.vs)]
    for t, saved in zip((c.kc, c.vc, c.ks, c.vs), arenas):  # same starting arenas for the second call
        t.copy_(saved)
    out = torch.full_like(out_ref, float("nan"))
    step = _step_args(c, out, None)  # no workspace: the library's scratch array serves it
    assert lib.ppk_decode_step_noalloc(ctx, stream, ctypes.byref(step)) == 0, _abi.last_error()
    torch.cuda.synchronize()
    assert torch.equal(out, out_ref), "no-alloc output differs from ppk_decode_step"
    for got, exp in zip((c.kc, c.vc, c.ks, c.vs), ref_arenas):
        assert torch.equal(got.view(torch.uint8), exp.view(torch.uint8)), "no-alloc append differs"
    return out.reshape(c.rows, c.D).cpu().numpy(), nbytes


def test_noalloc_step_matches_decode_step_twice_second_smaller(device):
    # First call: few long ragged rows, so rows span several blocks and the plan needs a workspace.
    big = Case(device, 2, 8, 128, [3000, 1501], 4096, q_dtype=torch.bfloat16, scratch_dtype=torch.bfloat16,
               seed=SEED + 901)
    got, nbytes = _run_both(device, big)
    assert nbytes > 0, "the first case must use the scratch"
    assert_close(got, big.reference(), what="no-alloc call 1")
    # Second call on the same GPU: a smaller problem, whose records overwrite fewer scratch bytes.
    small = Case(device, 1, 4, 64, [2000], 2048, seed=SEED + 902)
    got2, nbytes2 = _run_both(device, small)
    assert 0 < nbytes2 < nbytes
    assert_close(got2, small.reference(), what="no-alloc call 2")


def test_noalloc_step_single_launch_plan(device):
    """A plan with one block per row needs no scratch at all; the result is still the decode step's."""
    c = Case(device, 4, 4, 64, [100, 0, 37, 513], 640, seed=SEED + 903)
    got, nbytes = _run_both(device, c)
    assert nbytes == 0
    assert_close(got, c.reference(), what="no-alloc single launch")


def test_noalloc_step_refuses_a_plan_beyond_the_scratch(device):
    """8 rows x 2^20 slots of D = 256 at 64 tokens per wave: 1024 blocks per row, so the records need
    8 MiB + 64 KiB, more than PPK_NOALLOC_SCRATCH_BYTES. Status 1, nothing enqueued (output untouched)."""
    rows, cap, d = 8, 1 << 20, 256
    kc = torch.empty((rows, cap, d), dtype=torch.uint8, device=device)
    vc = torch.empty_like(kc)
    ks = torch.empty((rows, cap), dtype=torch.float32, device=device)
    vs = torch.empty_like(ks)
    q = torch.zeros((rows, 1, d), dtype=torch.float32, device=device)
    past = torch.full((1,), cap - 1, dtype=torch.int32, device=device)
    out = torch.full((rows, 1, d), 7.0, dtype=torch.float32, device=device)
    a, _ = ppk.int8_kv_ops.attention_args(q, kc, vc, ks, vs, q, q, past, rows, 64, out=out)
    step = ppk.int8_kv_ops._step_args(a, q, q, None, d)
    ctx = ppk.context(device)
    _, _, nbytes = ppk.int8_kv_ops.plan(step.attn, ctx)
    assert nbytes > _abi.PPK_NOALLOC_SCRATCH_BYTES
    stream = ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
    rc = _abi.lib().ppk_decode_step_noalloc(ctx, stream, ctypes.byref(step))
    torch.cuda.synchronize()
    assert rc == _abi.PPK_PRECONDITION
    assert "no-alloc scratch holds" in _abi.last_error()
    assert torch.all(out == 7.0)
