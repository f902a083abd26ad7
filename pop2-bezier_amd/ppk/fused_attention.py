"""Torch-tensor mirror of the reference's float-KV decode attention.

fused_attention::decode_attention(q, k, v, lengths, heads, split_tokens)
(app/src/model/fused_attention.rs:8-30, its ROCm branch
app/src/model/hip_attention.rs:47-113): single-query attention of
q F32[batch*heads, 1, D] over unquantised bf16/f32 K/V [batch*heads, length, D]
that already hold the current token, optionally limited per sequence by
lengths U32[batch]. Every computation runs in the gfx950 kernels behind
libppk.so (ppk_float_decode_attention); CPU tensors are refused as the
reference refuses them (fused_attention.rs:28, hip_attention.rs:51-53).

Beyond the reference: head_dim 64/128/256 (reference: 64), any length
(reference: <= 1024), bf16/f16 q and output dtypes.
"""
from __future__ import annotations

import ctypes

import torch

from . import _abi
from ._abi import check, lib
from .int8_kv_ops import _DTYPES, _HEAD_DIMS, _require, _stream, context, current_stream_handle

_KV_DTYPES = {torch.bfloat16: _abi.PPK_BF16, torch.float32: _abi.PPK_F32}


def decode_attention_args(q, k, v, lengths, heads: int, split_tokens: int = 0, *, max_length: int = 0,
                          out: torch.Tensor | None = None, out_dtype: torch.dtype = torch.float32,
                          softmax_scale: float = 0.0, lengths_host=None,
                          plan: str = "auto") -> tuple[_abi.PpkFloatAttentionArgs, torch.Tensor]:
    """Validate like fused_attention::decode_attention and build the ABI block (workspace unset).
    lengths_host: an optional host copy of `lengths` (a sequence of ints), with which the library balances
    ragged batches or sizes its per-row plan for the longest one; plan: "auto", "per-row" (plans as without
    lengths_host) or "balanced" (PPK_ATTN_PLAN_*)."""
    _require(q.dim() == 3 and k.dim() == 3 and v.dim() == 3, "fused decode attention requires 3-d q/k/v")
    rows, query, width = q.shape
    key_rows, length, key_width = k.shape
    _require(heads > 0 and rows > 0 and rows % heads == 0 and query == 1 and width in _HEAD_DIMS
             and key_rows == rows and key_width == width and length > 0 and v.shape == k.shape
             and q.dtype in _DTYPES and k.dtype in _KV_DTYPES and k.dtype == v.dtype
             and q.device == k.device == v.device,
             "fused decode attention requires float[batch*heads,1,D] Q and same-device BF16/F32 K/V")
    for t in (q, k, v):
        _require(t.stride(2) == 1 and t.stride(1) == width, "fused attention requires dense width and token strides")
    if lengths is not None:
        _require(lengths.dim() == 1 and lengths.shape[0] == rows // heads
                 and lengths.dtype in (torch.int32, torch.uint32) and lengths.is_contiguous()
                 and lengths.device == q.device, "fused attention row lengths require same-device U32[batch]")
    if q.device.type != "cuda":
        raise RuntimeError("fused decode attention needs a HIP device; use ordinary attention on this backend")
    if out is None:
        out = torch.empty((rows, 1, width), dtype=out_dtype, device=q.device)
    _require(out.numel() == rows * width and out.dtype in _DTYPES and out.is_contiguous() and out.device == q.device,
             "fused attention output must be a dense float tensor of rows*D elements")
    a = _abi.PpkFloatAttentionArgs(
        struct_size=ctypes.sizeof(_abi.PpkFloatAttentionArgs), kv_dtype=_KV_DTYPES[k.dtype],
        q_dtype=_DTYPES[q.dtype], out_dtype=_DTYPES[out.dtype], rows=rows, heads=heads, size=length,
        head_dim=width, split_tokens=split_tokens, max_length=max_length, softmax_scale=softmax_scale,
        flags=_abi.plan_flags(plan),
        q_row_stride=q.stride(0), k_row_stride=k.stride(0), v_row_stride=v.stride(0),
        q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(),
        lengths=lengths.data_ptr() if lengths is not None else None, out=out.data_ptr(), workspace=None,
        workspace_bytes=0, lengths_host=None)
    if lengths_host is not None:
        host = [int(x) for x in lengths_host]
        _require(lengths is not None and len(host) == rows // heads and all(0 <= x < 2 ** 32 for x in host),
                 "fused attention host lengths require device lengths of the same batch")
        a._lengths_host = (ctypes.c_uint32 * len(host))(*host)  # kept alive with the argument block
        a.lengths_host = ctypes.cast(a._lengths_host, ctypes.c_void_p).value
    return a, out


def plan(args: _abi.PpkFloatAttentionArgs, ctx: ctypes.c_void_p | None = None) -> tuple[int, int, int]:
    """(tokens per wave, blocks per row, workspace bytes) the library chooses for args."""
    split, nsplits, nbytes = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint64()
    check(lib().ppk_float_attention_plan(ctx, ctypes.byref(args), ctypes.byref(split), ctypes.byref(nsplits),
                                         ctypes.byref(nbytes)), "ppk_float_attention_plan")
    return split.value, nsplits.value, nbytes.value


def plan_info(args: _abi.PpkFloatAttentionArgs, ctx: ctypes.c_void_p | None = None) -> dict:
    """The whole launch plan the library takes for args (ppk_float_attention_plan_info): kind ("per-row" or
    "balanced"), split_tokens, nsplits, waves_per_block, blocks, launches and workspace_bytes."""
    info = _abi.PpkAttentionPlanInfo(struct_size=ctypes.sizeof(_abi.PpkAttentionPlanInfo))
    check(lib().ppk_float_attention_plan_info(ctx, ctypes.byref(args), ctypes.byref(info)),
          "ppk_float_attention_plan_info")
    return {"kind": "balanced" if info.kind == _abi.PPK_ATTN_PLAN_BALANCED else "per-row",
            "split_tokens": info.split_tokens, "nsplits": info.nsplits, "waves_per_block": info.waves_per_block,
            "blocks": info.blocks, "launches": info.launches, "workspace_bytes": info.workspace_bytes}


# The parameter `plan` of the calls below shadows the function inside them.
launch_plan = plan


def decode_attention(q, k, v, lengths, heads: int, split_tokens: int = 0, *, max_length: int = 0,
                     out_dtype: torch.dtype = torch.float32, softmax_scale: float = 0.0,
                     lengths_host=None, plan: str = "auto") -> torch.Tensor:
    """fused_attention::decode_attention -> out [rows, 1, D] (float32 by default). lengths_host: optional
    host copy of lengths."""
    a, out = decode_attention_args(q, k, v, lengths, heads, split_tokens, max_length=max_length,
                                   out_dtype=out_dtype, softmax_scale=softmax_scale, lengths_host=lengths_host,
                                   plan=plan)
    ctx = context(q.device)
    nbytes = launch_plan(a, ctx)[2]
    # Stream-ordered caching allocator: the block outlives the queued kernels.
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    a.workspace = ws.data_ptr()
    a.workspace_bytes = nbytes
    check(lib().ppk_float_decode_attention(ctx, _stream(q), ctypes.byref(a)), "ppk_float_decode_attention")
    return out


def _step_args(a: _abi.PpkFloatAttentionArgs, k_new: torch.Tensor, v_new: torch.Tensor, flags,
               lengths) -> _abi.PpkFloatDecodeStepArgs:
    _require(lengths is not None, "the float decode step needs the device lengths")
    _require(k_new.dtype == v_new.dtype and k_new.dtype in _DTYPES and k_new.numel() == a.rows * a.head_dim
             and v_new.numel() == a.rows * a.head_dim and k_new.is_contiguous() and v_new.is_contiguous()
             and k_new.is_cuda and v_new.is_cuda, "float decode step new token must be float[rows,D] on the device")
    if flags is not None:
        _require(flags.dtype in (torch.int32, torch.uint32) and flags.numel() >= 1, "flags must be one 32-bit word")
    step = _abi.PpkFloatDecodeStepArgs(struct_size=ctypes.sizeof(_abi.PpkFloatDecodeStepArgs),
                                       new_dtype=_DTYPES[k_new.dtype], k_new=k_new.data_ptr(),
                                       v_new=v_new.data_ptr(), flags=flags.data_ptr() if flags is not None else None,
                                       attn=a)
    step._lengths_host = getattr(a, "_lengths_host", None)  # the copied block points at it
    return step


def decode_step(q, k, v, lengths, heads: int, k_new: torch.Tensor, v_new: torch.Tensor, split_tokens: int = 0, *,
                flags: torch.Tensor | None = None, max_length: int = 0, out_dtype: torch.dtype = torch.float32,
                softmax_scale: float = 0.0, lengths_host=None, plan: str = "auto") -> torch.Tensor:
    """The float path's fused decode step (ppk_float_decode_step): write k_new / v_new [rows, D] (rounded to the
    store's dtype) at slot lengths[b] of the stores k / v [rows, size, D], then attend over the lengths[b] stored
    tokens plus that one; the graph-decode session's scatter_set pair + decode_attention(lengths + 1)
    (app/src/model/graph_decode.rs:290-305) in one launch. A row whose slot is past the store is not written
    (PPK_FLAG_OVERFLOW in `flags`) and gives NaN."""
    a, out = decode_attention_args(q, k, v, lengths, heads, split_tokens, max_length=max_length,
                                   out_dtype=out_dtype, softmax_scale=softmax_scale, lengths_host=lengths_host,
                                   plan=plan)
    step = _step_args(a, k_new, v_new, flags, lengths)
    ctx = context(q.device)
    nbytes = launch_plan(a, ctx)[2]
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    step.attn.workspace = ws.data_ptr()
    step.attn.workspace_bytes = nbytes
    check(lib().ppk_float_decode_step(ctx, _stream(q), ctypes.byref(step)), "ppk_float_decode_step")
    return out


def _replan(obj, attn: _abi.PpkFloatAttentionArgs, lengths_host) -> None:
    """Point attn at a new host copy of lengths[] (or none), re-plan, and grow obj's workspace if the new plan
    needs more (the old workspace is released to torch's stream-ordered allocator)."""
    if lengths_host is None:
        obj._lengths_host = None
        attn.lengths_host = None
    else:
        host = [int(x) for x in lengths_host]
        _require(attn.lengths is not None and len(host) == attn.rows // attn.heads
                 and all(0 <= x < 2 ** 32 for x in host),
                 "fused attention host lengths require device lengths of the same batch")
        obj._lengths_host = (ctypes.c_uint32 * len(host))(*host)
        attn.lengths_host = ctypes.cast(obj._lengths_host, ctypes.c_void_p).value
    obj.split_tokens, obj.ngroups, nbytes = launch_plan(attn, obj.ctx)
    obj.plan_info = plan_info(attn, obj.ctx)
    if nbytes > obj.workspace.numel():
        obj.workspace = torch.empty(nbytes, dtype=torch.uint8, device=obj.device)
    attn.workspace = obj.workspace.data_ptr()
    attn.workspace_bytes = nbytes


class FloatDecodeAttention:
    """A prepared float-KV attention call for fixed buffers: argument block and workspace are built once;
    __call__ only enqueues the kernels (bench and serving loops, graph capture).

    lengths_host, if given, is the host copy of lengths[] for the calls that follow: the plan is sized from
    it and every call checks it against the device lengths (a differing sequence gives NaN rows, never wrong
    ones). A caller whose lengths move between calls passes each call's copy to set_lengths_host() first, or
    builds the call without one (device lengths only)."""

    def __init__(self, q, k, v, lengths, heads: int, split_tokens: int = 0, *, max_length: int = 0,
                 out: torch.Tensor | None = None, out_dtype: torch.dtype = torch.float32, lengths_host=None,
                 plan: str = "auto"):
        self.args, self.out = decode_attention_args(q, k, v, lengths, heads, split_tokens, max_length=max_length,
                                                    out=out, out_dtype=out_dtype, lengths_host=lengths_host,
                                                    plan=plan)
        self.ctx = context(q.device)
        self.split_tokens, self.ngroups, nbytes = launch_plan(self.args, self.ctx)
        self.plan_info = plan_info(self.args, self.ctx)
        self.workspace = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
        self.args.workspace = self.workspace.data_ptr()
        self.args.workspace_bytes = nbytes
        self._keep = (q, k, v, lengths)
        self._ref = ctypes.byref(self.args)
        self._fn = lib().ppk_float_decode_attention
        self.device = q.device

    def set_lengths_host(self, lengths_host) -> None:
        """Replace the host copy of lengths[] (None: none) and re-plan for it."""
        _replan(self, self.args, lengths_host)

    def __call__(self, stream: torch.cuda.Stream | None = None) -> torch.Tensor:
        s = current_stream_handle(self.device) if stream is None else ctypes.c_void_p(stream.cuda_stream)
        check(self._fn(self.ctx, s, self._ref), "ppk_float_decode_attention")
        return self.out


def prepare(device: torch.device | int | None = None) -> None:
    """hip_attention::validate_split_k on the device (raises PpkInvalidOutputError on a mismatch)."""
    check(lib().ppk_float_attention_prepare(context(device)), "ppk_float_attention_prepare")


class FloatDecodeStep:
    """A prepared fused float decode step for fixed buffers (the graph-decode session's per-layer call):
    argument block and workspace are built once; __call__ only enqueues the kernels.

    lengths_host is the host copy of lengths[] for the calls that follow (see FloatDecodeAttention): in a
    graph-decode session, whose lengths grow by one every step, pass each step's copy to set_lengths_host()
    before the call, or build the step without one (device lengths only)."""

    def __init__(self, q, k, v, lengths, heads: int, k_new: torch.Tensor, v_new: torch.Tensor,
                 split_tokens: int = 0, *, flags: torch.Tensor | None = None, max_length: int = 0,
                 out: torch.Tensor | None = None, out_dtype: torch.dtype = torch.float32, lengths_host=None,
                 plan: str = "auto"):
        a, self.out = decode_attention_args(q, k, v, lengths, heads, split_tokens, max_length=max_length, out=out,
                                            out_dtype=out_dtype, lengths_host=lengths_host, plan=plan)
        self.args = _step_args(a, k_new, v_new, flags, lengths)
        self.ctx = context(q.device)
        self.split_tokens, self.ngroups, nbytes = launch_plan(self.args.attn, self.ctx)
        self.plan_info = plan_info(self.args.attn, self.ctx)
        self.workspace = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
        self.args.attn.workspace = self.workspace.data_ptr()
        self.args.attn.workspace_bytes = nbytes
        self._keep = (q, k, v, lengths, k_new, v_new, flags)
        self._ref = ctypes.byref(self.args)
        self._fn = lib().ppk_float_decode_step
        self.device = q.device

    def set_lengths_host(self, lengths_host) -> None:
        """Replace the host copy of lengths[] (None: none) and re-plan for it."""
        _replan(self, self.args.attn, lengths_host)

    def __call__(self, stream: torch.cuda.Stream | None = None) -> torch.Tensor:
        s = current_stream_handle(self.device) if stream is None else ctypes.c_void_p(stream.cuda_stream)
        check(self._fn(self.ctx, s, self._ref), "ppk_float_decode_step")
        return self.out
