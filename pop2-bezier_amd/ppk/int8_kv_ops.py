"""Torch-tensor mirror of the reference's int8 KV custom-op API.

Same entry points, argument meaning and error behaviour as
app/src/model/int8_kv_ops.rs (quantize :11-29, dequantize :30-40,
attention :41-55, prepare :56-103), plus `append`, the fused commit that
Int8LayerCache::query_batch performs (app/src/model/int8_cache.rs:326-359).
torch supplies device memory and the stream; every computation runs in the
gfx950 kernels behind libppk.so. CPU tensors are refused, as the reference's
device-only branches refuse them (int8_kv_ops.rs:28,54).
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _abi
from ._abi import check, lib

_DTYPES = {torch.float32: _abi.PPK_F32, torch.bfloat16: _abi.PPK_BF16, torch.float16: _abi.PPK_F16}
_HEAD_DIMS = (64, 128, 256)
_contexts: dict[int, ctypes.c_void_p] = {}


def context(device: torch.device | int | None = None) -> ctypes.c_void_p:
    """The library context of a HIP device (code object loaded once per device)."""
    if device is None:
        index = torch.cuda.current_device()
    elif isinstance(device, int):
        index = device
    else:
        index = torch.device(device).index
        if index is None:
            index = torch.cuda.current_device()
    ctx = _contexts.get(index)
    if ctx is None:
        ctx = ctypes.c_void_p()
        check(lib().ppk_context_create(index, None, ctypes.byref(ctx)), "ppk_context_create")
        _contexts[index] = ctx
    return ctx


def current_stream_handle(device: torch.device) -> ctypes.c_void_p:
    """The device's current HIP stream as a raw handle, without building a torch Stream object (the prepared
    calls below run once per layer of a decode step, where that object cost more than the C-ABI call)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    return ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(index))


def _stream(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _require(cond: bool, message: str) -> None:
    if not cond:
        raise ValueError(message)


def _device_only(*tensors: torch.Tensor, what: str) -> None:
    dev = tensors[0].device
    if dev.type != "cuda":
        raise RuntimeError(f"{what} is unavailable on this native provider")
    for t in tensors:
        _require(t.device == dev, "INT8 attention device mismatch")


def _geometry(t: torch.Tensor) -> tuple[int, int]:
    """geometry() of int8_kv_ops.rs:5-10, with D in {64, 128, 256}."""
    _require(t.dim() == 3 and t.shape[0] > 0 and t.shape[1] > 0 and t.shape[2] in _HEAD_DIMS and t.is_contiguous(),
             "INT8 KV requires dense [heads,tokens,D] with D in {64,128,256}")
    return t.shape[0], t.shape[1]


def quantize(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """[heads, tokens, D] float -> (uint8 codes [heads, tokens, D], float32 scales [heads, tokens])."""
    h, n = _geometry(x)
    _require(x.dtype in _DTYPES, "INT8 KV quantize input must be float32, bfloat16 or float16")
    _device_only(x, what="KV INT8")
    codes = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    scales = torch.empty((h, n), dtype=torch.float32, device=x.device)
    a = _abi.PpkQuantizeArgs(struct_size=ctypes.sizeof(_abi.PpkQuantizeArgs), src_dtype=_DTYPES[x.dtype],
                             src=x.data_ptr(), codes=codes.data_ptr(), scales=scales.data_ptr(), rows=h * n,
                             head_dim=x.shape[2], flags=None)
    check(lib().ppk_quantize(context(x.device), _stream(x), ctypes.byref(a)), "ppk_quantize")
    return codes, scales


def dequantize(packed: torch.Tensor, scale: torch.Tensor, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """codes * scale, rounded to `dtype` (bf16: round-to-nearest-even of the f32 product)."""
    h, n = _geometry(packed)
    _require(packed.dtype == torch.uint8 and scale.dtype == torch.float32 and tuple(scale.shape) == (h, n)
             and scale.is_contiguous() and packed.device == scale.device, "INT8 KV scales differ")
    _require(dtype in _DTYPES, "INT8 dequantize dtype must be float32, bfloat16 or float16")
    _device_only(packed, scale, what="KV INT8 dequantization")
    out = torch.empty(packed.shape, dtype=dtype, device=packed.device)
    a = _abi.PpkDequantizeArgs(struct_size=ctypes.sizeof(_abi.PpkDequantizeArgs), out_dtype=_DTYPES[dtype],
                               codes=packed.data_ptr(), scales=scale.data_ptr(), out=out.data_ptr(), rows=h * n,
                               head_dim=packed.shape[2], round_bf16=0)
    check(lib().ppk_dequantize(context(packed.device), _stream(packed), ctypes.byref(a)), "ppk_dequantize")
    return out


def append(k_new: torch.Tensor, v_new: torch.Tensor, past: torch.Tensor, k_codes: torch.Tensor,
           v_codes: torch.Tensor, k_scales: torch.Tensor, v_scales: torch.Tensor,
           flags: torch.Tensor | None = None) -> None:
    """Quantize k_new/v_new [B, H, T, D] and write them at slots past[b]..past[b]+T-1 of the
    arenas [B*H, capacity, D] (codes) and [B*H, capacity] (scales), in place."""
    _require(k_new.dim() == 4 and k_new.shape == v_new.shape and k_new.dtype == v_new.dtype
             and k_new.dtype in _DTYPES and k_new.is_contiguous() and v_new.is_contiguous(),
             "INT8 batch requires [B,H,T,D] scratch and matching row histories")
    b, h, t, d = k_new.shape
    _require(d in _HEAD_DIMS and b > 0 and h > 0 and t > 0, "INT8 batch requires [B,H,T,D] with D in {64,128,256}")
    rows, cap = _geometry(k_codes)[0], k_codes.shape[1]
    _require(rows == b * h and k_codes.shape == v_codes.shape and k_codes.shape[2] == d
             and k_codes.dtype == torch.uint8 and v_codes.dtype == torch.uint8 and v_codes.is_contiguous(),
             "INT8 packed arenas must be uint8 [B*H, capacity, D]")
    for s in (k_scales, v_scales):
        _require(tuple(s.shape) == (rows, cap) and s.dtype == torch.float32 and s.is_contiguous(),
                 "INT8 scale arenas must be float32 [B*H, capacity]")
    _require(tuple(past.shape) == (b,) and past.dtype in (torch.int32, torch.uint32) and past.is_contiguous(),
             "INT8 append lengths must be U32[B]")
    if flags is not None:
        _require(flags.dtype in (torch.int32, torch.uint32) and flags.numel() >= 1, "flags must be one 32-bit word")
    _device_only(k_new, v_new, past, k_codes, v_codes, k_scales, v_scales, what="KV INT8")
    a = _abi.PpkAppendArgs(struct_size=ctypes.sizeof(_abi.PpkAppendArgs), src_dtype=_DTYPES[k_new.dtype],
                           k_src=k_new.data_ptr(), v_src=v_new.data_ptr(), past=past.data_ptr(),
                           k_codes=k_codes.data_ptr(), v_codes=v_codes.data_ptr(), k_scales=k_scales.data_ptr(),
                           v_scales=v_scales.data_ptr(), batch=b, heads=h, tokens=t, head_dim=d, capacity=cap,
                           flags=flags.data_ptr() if flags is not None else None)
    check(lib().ppk_quantize_append(context(k_new.device), _stream(k_new), ctypes.byref(a)), "ppk_quantize_append")


def attention_args(q, k, v, ks, vs, sk, sv, past, heads: int, split_tokens: int = 0, *, bf16_history: bool = False,
                   max_past: int = 0, out: torch.Tensor | None = None, out_dtype: torch.dtype = torch.float32,
                   softmax_scale: float = 0.0, past_host=None,
                   plan: str = "auto") -> tuple[_abi.PpkAttentionArgs, torch.Tensor]:
    """Validate like int8_kv_ops::attention and build the ABI argument block (workspace unset). past_host: an
    optional host copy of `past` (a sequence of ints), with which the library balances ragged batches or sizes
    its per-row plan for the longest one; plan: "auto" (the library chooses from past_host), "per-row" (plans as
    without past_host) or "balanced" (PPK_ATTN_PLAN_*)."""
    rows, capacity = _geometry(k)
    d = k.shape[2]
    _require(heads > 0 and rows % heads == 0 and v.shape == k.shape and v.is_contiguous()
             and k.dtype == torch.uint8 and v.dtype == torch.uint8, "INT8 attention geometry differs")
    for t in (q, sk, sv):
        _require(t.numel() == rows * d and t.shape[0] == rows and t.shape[-1] == d and t.dtype in _DTYPES
                 and t.is_contiguous(), "INT8 scratch must be float[head_rows,1,D]")
    _require(sk.dtype == sv.dtype, "INT8 scratch key/value dtypes differ")
    for t in (ks, vs):
        _require(tuple(t.shape) == (rows, capacity) and t.dtype == torch.float32 and t.is_contiguous(),
                 "INT8 scales must be F32[head_rows,capacity]")
    _require(tuple(past.shape) == (rows // heads,) and past.dtype in (torch.int32, torch.uint32)
             and past.is_contiguous(), "INT8 attention lengths differ")
    _device_only(q, k, v, ks, vs, sk, sv, past, what="KV INT8 fused attention")
    if out is None:
        out = torch.empty((rows, 1, d), dtype=out_dtype, device=q.device)
    _require(out.numel() == rows * d and out.dtype in _DTYPES and out.is_contiguous() and out.device == q.device,
             "INT8 attention output must be a dense float tensor of rows*D elements")
    a = _abi.PpkAttentionArgs(
        struct_size=ctypes.sizeof(_abi.PpkAttentionArgs), q_dtype=_DTYPES[q.dtype], scratch_dtype=_DTYPES[sk.dtype],
        out_dtype=_DTYPES[out.dtype],
        flags=(_abi.PPK_ATTN_BF16_HISTORY if bf16_history else 0) | _abi.plan_flags(plan), rows=rows,
        heads=heads, capacity=capacity, head_dim=d, split_tokens=split_tokens, max_past=max_past,
        softmax_scale=softmax_scale, q=q.data_ptr(), k_codes=k.data_ptr(), v_codes=v.data_ptr(),
        k_scales=ks.data_ptr(), v_scales=vs.data_ptr(), sk=sk.data_ptr(), sv=sv.data_ptr(), past=past.data_ptr(),
        out=out.data_ptr(), workspace=None, workspace_bytes=0, past_host=None)
    if past_host is not None:
        host = [int(x) for x in past_host]
        _require(len(host) == rows // heads and all(0 <= x < 2 ** 32 for x in host), "INT8 attention lengths differ")
        a._past_host = (ctypes.c_uint32 * len(host))(*host)  # kept alive with the argument block
        a.past_host = ctypes.cast(a._past_host, ctypes.c_void_p).value
    return a, out


def workspace_bytes(args: _abi.PpkAttentionArgs, ctx: ctypes.c_void_p | None = None) -> int:
    n = ctypes.c_uint64()
    check(lib().ppk_attention_workspace_bytes(ctx, ctypes.byref(args), ctypes.byref(n)),
          "ppk_attention_workspace_bytes")
    return n.value


def plan(args: _abi.PpkAttentionArgs, ctx: ctypes.c_void_p | None = None) -> tuple[int, int, int]:
    """(history tokens per wave, blocks per row, workspace bytes) the library chooses for args.
    One block per row means the whole step is a single launch (no workspace)."""
    split, nsplits, nbytes = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint64()
    check(lib().ppk_attention_plan(ctx, ctypes.byref(args), ctypes.byref(split), ctypes.byref(nsplits),
                                   ctypes.byref(nbytes)), "ppk_attention_plan")
    return split.value, nsplits.value, nbytes.value


def plan_info(args: _abi.PpkAttentionArgs, ctx: ctypes.c_void_p | None = None) -> dict:
    """The whole launch plan the library takes for args (ppk_attention_plan_info): kind ("per-row" or
    "balanced"), split_tokens, nsplits, waves_per_block, blocks, launches and workspace_bytes."""
    info = _abi.PpkAttentionPlanInfo(struct_size=ctypes.sizeof(_abi.PpkAttentionPlanInfo))
    check(lib().ppk_attention_plan_info(ctx, ctypes.byref(args), ctypes.byref(info)),
          "ppk_attention_plan_info")
    return {"kind": "balanced" if info.kind == _abi.PPK_ATTN_PLAN_BALANCED else "per-row",
            "split_tokens": info.split_tokens, "nsplits": info.nsplits, "waves_per_block": info.waves_per_block,
            "blocks": info.blocks, "launches": info.launches, "workspace_bytes": info.workspace_bytes}


# The parameter `plan` of the calls below shadows the function inside them.
launch_plan = plan


def attention(q, k, v, ks, vs, sk, sv, past, heads: int, split_tokens: int = 0, *, bf16_history: bool = False,
              max_past: int = 0, out_dtype: torch.dtype = torch.float32, softmax_scale: float = 0.0,
              past_host=None, plan: str = "auto") -> torch.Tensor:
    """int8_kv_ops::attention: q/sk/sv [rows,1,D], k/v uint8 [rows,cap,D], ks/vs f32 [rows,cap],
    past U32 [rows/heads] -> out [rows,1,D] (float32 by default). past_host: optional host copy of past."""
    a, out = attention_args(q, k, v, ks, vs, sk, sv, past, heads, split_tokens, bf16_history=bf16_history,
                            max_past=max_past, out_dtype=out_dtype, softmax_scale=softmax_scale, past_host=past_host,
                            plan=plan)
    ctx = context(q.device)
    nbytes = workspace_bytes(a, ctx)
    # The caching allocator is stream-ordered: the block is not reused before
    # the kernels queued on this stream have consumed it.
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    a.workspace = ws.data_ptr()
    a.workspace_bytes = nbytes
    check(lib().ppk_decode_attention(ctx, _stream(q), ctypes.byref(a)), "ppk_decode_attention")
    return out


def decode_step(q, k, v, ks, vs, sk, sv, past, heads: int, k_new: torch.Tensor | None = None,
                v_new: torch.Tensor | None = None, split_tokens: int = 0, *, flags: torch.Tensor | None = None,
                bf16_history: bool = False, max_past: int = 0, out_dtype: torch.dtype = torch.float32,
                softmax_scale: float = 0.0, past_host=None, plan: str = "auto") -> torch.Tensor:
    """Commit + attend in one call: quantise k_new/v_new [rows, D] (default: sk/sv) into slot past[b] of the
    arenas, then attention over [0, past[b]) plus the current token, as forward_embedding's commit path does
    (query_int8 then int8_kv_ops::attention, app/src/model/mod.rs:699-705)."""
    a, out = attention_args(q, k, v, ks, vs, sk, sv, past, heads, split_tokens, bf16_history=bf16_history,
                            max_past=max_past, out_dtype=out_dtype, softmax_scale=softmax_scale, past_host=past_host,
                            plan=plan)
    step = _step_args(a, sk if k_new is None else k_new, sv if v_new is None else v_new, flags, k.shape[2])
    ctx = context(q.device)
    nbytes = workspace_bytes(a, ctx)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    step.attn.workspace = ws.data_ptr()
    step.attn.workspace_bytes = nbytes
    check(lib().ppk_decode_step(ctx, _stream(q), ctypes.byref(step)), "ppk_decode_step")
    return out


def _step_args(a: _abi.PpkAttentionArgs, k_new: torch.Tensor, v_new: torch.Tensor, flags, d: int
               ) -> _abi.PpkDecodeStepArgs:
    _require(k_new.dtype == v_new.dtype and k_new.dtype in _DTYPES and k_new.numel() == a.rows * d
             and v_new.numel() == a.rows * d and k_new.is_contiguous() and v_new.is_contiguous(),
             "INT8 decode step new token must be float[rows,D]")
    if flags is not None:
        _require(flags.dtype in (torch.int32, torch.uint32) and flags.numel() >= 1, "flags must be one 32-bit word")
    step = _abi.PpkDecodeStepArgs(struct_size=ctypes.sizeof(_abi.PpkDecodeStepArgs), new_dtype=_DTYPES[k_new.dtype],
                                  k_new=k_new.data_ptr(), v_new=v_new.data_ptr(),
                                  flags=flags.data_ptr() if flags is not None else None, attn=a)
    step._past_host = getattr(a, "_past_host", None)  # the copied block points at it
    return step


def _replan(obj, attn: _abi.PpkAttentionArgs, past_host) -> None:
    """Point attn at a new host copy of past[] (or none), re-plan, and grow obj's workspace if the new plan
    needs more (the old workspace is released to torch's stream-ordered allocator)."""
    if past_host is None:
        obj._past_host = None
        attn.past_host = None
    else:
        host = [int(x) for x in past_host]
        _require(len(host) == attn.rows // attn.heads and all(0 <= x < 2 ** 32 for x in host),
                 "INT8 attention lengths differ")
        obj._past_host = (ctypes.c_uint32 * len(host))(*host)
        attn.past_host = ctypes.cast(obj._past_host, ctypes.c_void_p).value
    obj.split_tokens, obj.ngroups, nbytes = launch_plan(attn, obj.ctx)
    obj.plan_info = plan_info(attn, obj.ctx)
    if nbytes > obj.workspace.numel():
        obj.workspace = torch.empty(nbytes, dtype=torch.uint8, device=obj.device)
    attn.workspace = obj.workspace.data_ptr()
    attn.workspace_bytes = nbytes


class DecodeAttention:
    """A prepared attention call for a fixed set of buffers (bench / serving loops): the argument
    block and workspace are built once; __call__ only enqueues the two kernels.

    past_host, if given, is the host copy of past[] for the calls that follow: the plan is sized from it and
    every call checks it against the device past[] (a differing sequence gives NaN rows, never wrong ones).
    A caller whose lengths move between calls passes each call's copy to set_past_host() first, or builds
    the call without one (device lengths only)."""

    def __init__(self, q, k, v, ks, vs, sk, sv, past, heads: int, split_tokens: int = 0, *,
                 bf16_history: bool = False, max_past: int = 0, out: torch.Tensor | None = None,
                 out_dtype: torch.dtype = torch.float32, past_host=None, plan: str = "auto"):
        self.args, self.out = attention_args(q, k, v, ks, vs, sk, sv, past, heads, split_tokens,
                                             bf16_history=bf16_history, max_past=max_past, out=out,
                                             out_dtype=out_dtype, past_host=past_host, plan=plan)
        self.ctx = context(q.device)
        self.split_tokens, self.ngroups, nbytes = launch_plan(self.args, self.ctx)
        self.plan_info = plan_info(self.args, self.ctx)
        self.workspace = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
        self.args.workspace = self.workspace.data_ptr()
        self.args.workspace_bytes = nbytes
        self._keep = (q, k, v, ks, vs, sk, sv, past)
        self._ref = ctypes.byref(self.args)
        self._fn = lib().ppk_decode_attention
        self.device = q.device

    def set_past_host(self, past_host) -> None:
        """Replace the host copy of past[] (None: none) and re-plan for it."""
        _replan(self, self.args, past_host)

    def __call__(self, stream: torch.cuda.Stream | None = None) -> torch.Tensor:
        s = current_stream_handle(self.device) if stream is None else ctypes.c_void_p(stream.cuda_stream)
        check(self._fn(self.ctx, s, self._ref), "ppk_decode_attention")
        return self.out


class DecodeStep:
    """A prepared decode step (append of the current token + attention) for fixed buffers: the argument
    block and workspace are built once; __call__ enqueues one launch (two when the plan splits rows).

    past_host is the host copy of past[] for the calls that follow (see DecodeAttention): a decode loop
    whose lengths grow every step passes each step's copy to set_past_host() before the call, or builds the
    step without one."""

    def __init__(self, q, k, v, ks, vs, sk, sv, past, heads: int, k_new=None, v_new=None, split_tokens: int = 0, *,
                 flags=None, bf16_history: bool = False, max_past: int = 0, out: torch.Tensor | None = None,
                 out_dtype: torch.dtype = torch.float32, past_host=None, plan: str = "auto"):
        a, self.out = attention_args(q, k, v, ks, vs, sk, sv, past, heads, split_tokens, bf16_history=bf16_history,
                                     max_past=max_past, out=out, out_dtype=out_dtype, past_host=past_host,
                                     plan=plan)
        k_new = sk if k_new is None else k_new
        v_new = sv if v_new is None else v_new
        self.args = _step_args(a, k_new, v_new, flags, k.shape[2])
        self.ctx = context(q.device)
        self.split_tokens, self.ngroups, nbytes = launch_plan(self.args.attn, self.ctx)
        self.plan_info = plan_info(self.args.attn, self.ctx)
        self.workspace = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
        self.args.attn.workspace = self.workspace.data_ptr()
        self.args.attn.workspace_bytes = nbytes
        self._keep = (q, k, v, ks, vs, sk, sv, past, k_new, v_new, flags)
        self._ref = ctypes.byref(self.args)
        self._fn = lib().ppk_decode_step
        self.device = q.device

    def set_past_host(self, past_host) -> None:
        """Replace the host copy of past[] (None: none) and re-plan for it."""
        _replan(self, self.args.attn, past_host)

    def __call__(self, stream: torch.cuda.Stream | None = None) -> torch.Tensor:
        s = current_stream_handle(self.device) if stream is None else ctypes.c_void_p(stream.cuda_stream)
        check(self._fn(self.ctx, s, self._ref), "ppk_decode_step")
        return self.out


class AppendKV:
    """A prepared quantize-and-append call for fixed buffers."""

    def __init__(self, k_new, v_new, past, k_codes, v_codes, k_scales, v_scales, flags=None):
        b, h, t, d = k_new.shape
        self.args = _abi.PpkAppendArgs(
            struct_size=ctypes.sizeof(_abi.PpkAppendArgs), src_dtype=_DTYPES[k_new.dtype], k_src=k_new.data_ptr(),
            v_src=v_new.data_ptr(), past=past.data_ptr(), k_codes=k_codes.data_ptr(), v_codes=v_codes.data_ptr(),
            k_scales=k_scales.data_ptr(), v_scales=v_scales.data_ptr(), batch=b, heads=h, tokens=t, head_dim=d,
            capacity=k_codes.shape[1], flags=flags.data_ptr() if flags is not None else None)
        # Validate through the one-shot path's checks once.
        _require(k_new.is_contiguous() and v_new.is_contiguous() and k_codes.shape[0] == b * h,
                 "INT8 batch requires [B,H,T,D] scratch and matching row histories")
        self.ctx = context(k_new.device)
        self._keep = (k_new, v_new, past, k_codes, v_codes, k_scales, v_scales, flags)
        self._ref = ctypes.byref(self.args)
        self._fn = lib().ppk_quantize_append
        self.device = k_new.device

    def __call__(self, stream: torch.cuda.Stream | None = None) -> None:
        s = current_stream_handle(self.device) if stream is None else ctypes.c_void_p(stream.cuda_stream)
        check(self._fn(self.ctx, s, self._ref), "ppk_quantize_append")


def prepare(device: torch.device | int | None = None) -> None:
    """int8_kv_ops::prepare: run the private known-answer checks on the device."""
    check(lib().ppk_prepare(context(device)), "ppk_prepare")


def prepare_int8_kv(requested: bool, head_dim: int = 64, device: torch.device | int | None = None) -> dict:
    """PrimitiveModel::prepare_int8_kv (int8_policy.rs:26-55): the Int8KvStatus fields as a dict. A failed
    self-check raises (PpkInvalidOutputError etc.) after recording the reason, as the reference returns Err."""
    st = _abi.PpkInt8KvStatus(struct_size=ctypes.sizeof(_abi.PpkInt8KvStatus))
    check(lib().ppk_prepare_int8_kv(context(device), int(bool(requested)), head_dim, ctypes.byref(st)),
          "ppk_prepare_int8_kv")
    return {"requested": bool(st.requested), "available": bool(st.available), "ready": bool(st.ready),
            "enabled": bool(st.enabled), "format": st.format.decode(), "reason": st.reason.decode(),
            "packed_bytes_per_token_head": st.packed_bytes_per_token_head,
            "scale_bytes_per_token_head": st.scale_bytes_per_token_head}


def set_profiling(enable: bool, device: torch.device | int | None = None) -> None:
    check(lib().ppk_context_set_profiling(context(device), int(bool(enable))), "ppk_context_set_profiling")


def kernel_stats(kernel: int, device: torch.device | int | None = None, reset: bool = False) -> tuple[int, float]:
    """(launches, total milliseconds) of a traced kernel (PPK_KERNEL_*)."""
    n = ctypes.c_uint64()
    ms = ctypes.c_double()
    check(lib().ppk_context_kernel_stats(context(device), kernel, ctypes.byref(n), ctypes.byref(ms), int(reset)),
          "ppk_context_kernel_stats")
    return n.value, ms.value


def default_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)
