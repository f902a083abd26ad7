"""Torch-facing mirror of the reference's KV cache layer over the C-ABI arena
manager (include/ppk_int8_kv.h, ppk_kv_*).

LayerCache follows app/src/model/cache.rs:40-531 (query, query_batch[_with_plan],
clone = snapshot, truncate_committed, key/value, len) with int8 storage as
Int8LayerCache (app/src/model/int8_cache.rs:292-359); WritePlan follows
BatchWritePlan (app/src/model/write_plan.rs:12-102). Storage lives in
device arenas owned by libppk; views are returned as the C view block plus
`read()`, which copies a view's rows into a new torch tensor.
"""
from __future__ import annotations

import ctypes
import sys

import torch

from . import _abi
from ._abi import check, lib
from .int8_kv_ops import _DTYPES, _stream, context

KINDS = {"int8": _abi.PPK_KV_INT8, torch.bfloat16: _abi.PPK_KV_BF16, torch.float16: _abi.PPK_KV_F16,
         torch.float32: _abi.PPK_KV_F32}
_KIND_DTYPE = {_abi.PPK_KV_INT8: torch.uint8, _abi.PPK_KV_BF16: torch.bfloat16, _abi.PPK_KV_F16: torch.float16,
               _abi.PPK_KV_F32: torch.float32}
_hip = None


def _hip_runtime() -> ctypes.CDLL:
    """The HIP runtime already loaded by torch and libppk (one SONAME, one instance)."""
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so.7")
        _hip.hipMemcpy2DAsync.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t,
                                          ctypes.c_size_t, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p]
        _hip.hipMemcpy2DAsync.restype = ctypes.c_int
    return _hip


def _write(k: torch.Tensor, v: torch.Tensor, tokens: int, commit: bool) -> _abi.PpkKvWrite:
    if k.dtype not in _DTYPES or v.dtype != k.dtype or k.shape != v.shape or not (k.is_cuda and v.is_cuda):
        raise ValueError("K/V query precision, shape or device mismatch")
    return _abi.PpkKvWrite(struct_size=ctypes.sizeof(_abi.PpkKvWrite), src_dtype=_DTYPES[k.dtype], tokens=tokens,
                           commit=int(bool(commit)), k=k.data_ptr(), v=v.data_ptr())


def read(view: _abi.PpkKvView, which: str = "k", tokens: int | None = None,
         device: torch.device | None = None) -> torch.Tensor:
    """Copy of a view's [rows, tokens, head_dim] values (`k` / `v`) or [rows, tokens] scales
    (`k_scales` / `v_scales`); tokens defaults to the view's length."""
    n = view.length if tokens is None else tokens
    device = device or torch.device("cuda", torch.cuda.current_device())
    src = getattr(view, which)
    if which in ("k", "v"):
        dtype = _KIND_DTYPE[view.kind]
        shape, inner = (view.rows, n, view.head_dim), view.head_dim
    else:
        dtype, shape, inner = torch.float32, (view.rows, n), 1
    out = torch.empty(shape, dtype=dtype, device=device)
    if out.numel() == 0 or not src:
        return out
    eb = out.element_size()
    st = _hip_runtime().hipMemcpy2DAsync(out.data_ptr(), n * inner * eb, src, view.capacity * inner * eb,
                                         n * inner * eb, view.rows, 3, _stream(out))
    if st != 0:
        raise RuntimeError(f"hipMemcpy2DAsync failed with {st}")
    return out


class LayerCache:
    """One sequence's K/V history for one layer (cache.rs LayerCache / int8_cache.rs Int8LayerCache)."""

    def __init__(self, kind, heads: int, head_dim: int, *, max_context: int = 0, min_capacity: int = 0,
                 device: torch.device | int | None = None, _handle: ctypes.c_void_p | None = None):
        self.kind = KINDS[kind] if not isinstance(kind, int) else kind
        self.heads, self.head_dim = heads, head_dim
        self.ctx = context(device)
        self.device = device
        if _handle is not None:
            self.handle = _handle
        else:
            cfg = _abi.PpkKvConfig(struct_size=ctypes.sizeof(_abi.PpkKvConfig), kind=self.kind, heads=heads,
                                   head_dim=head_dim, max_context=max_context, min_capacity=min_capacity)
            self.handle = ctypes.c_void_p()
            check(lib().ppk_kv_cache_create(self.ctx, ctypes.byref(cfg), ctypes.byref(self.handle)),
                  "ppk_kv_cache_create")

    def __del__(self):
        # At interpreter shutdown the HIP runtime may already be gone; the process frees everything.
        h = getattr(self, "handle", None)
        if h is not None and h.value and not sys.is_finalizing():
            lib().ppk_kv_cache_release(h)
            self.handle = None

    def clone(self) -> "LayerCache":
        """A snapshot sharing storage; the next write through either side copies first."""
        h = ctypes.c_void_p()
        check(lib().ppk_kv_cache_clone(self.handle, ctypes.byref(h)), "ppk_kv_cache_clone")
        out = LayerCache(self.kind, self.heads, self.head_dim, device=self.device, _handle=h)
        out._adopted = getattr(self, "_adopted", None)  # adopted memory stays referenced by every snapshot
        return out

    @staticmethod
    def adopt_graph_view(key: torch.Tensor, value: torch.Tensor, capacity: int, committed_len: int,
                         *, max_context: int = 0) -> "LayerCache":
        """LayerCache::adopt_graph_view (cache.rs:55-64): a cache over f32 K/V [heads, capacity, D] that
        the caller owns (a graph decode session's buffers), holding committed_len tokens. The tensors stay
        referenced by the cache; the library writes into them in place while writes fit."""
        if (key.dim() != 3 or value.shape != key.shape or key.shape[1] != capacity or key.dtype != torch.float32
                or value.dtype != key.dtype or key.device != value.device or not key.is_cuda
                or not (key.is_contiguous() and value.is_contiguous()) or 0 in (key.shape[0], key.shape[2])):
            raise ValueError("invalid graph KV view")
        return LayerCache._adopt(key.data_ptr(), value.data_ptr(), key.shape[0], key.shape[2], capacity,
                                 committed_len, max_context=max_context, device=key.device, keep=(key, value))

    @staticmethod
    def _adopt(k_ptr: int, v_ptr: int, heads: int, head_dim: int, capacity: int, committed_len: int, *,
               max_context: int = 0, device=None, keep=()) -> "LayerCache":
        """ppk_kv_cache_adopt over raw device addresses; `keep` holds whatever owns that memory."""
        cfg = _abi.PpkKvConfig(struct_size=ctypes.sizeof(_abi.PpkKvConfig), kind=_abi.PPK_KV_F32, heads=heads,
                               head_dim=head_dim, max_context=max_context, min_capacity=0)
        h = ctypes.c_void_p()
        check(lib().ppk_kv_cache_adopt(context(device), ctypes.byref(cfg), k_ptr, v_ptr, capacity, committed_len,
                                       ctypes.byref(h)), "ppk_kv_cache_adopt")
        out = LayerCache(_abi.PPK_KV_F32, heads, head_dim, device=device, _handle=h)
        out._adopted = keep
        return out

    def advance_graph_length(self, previous: int, next_len: int) -> None:
        """LayerCache::advance_graph_length (cache.rs:66-73): commit the slot a graph wrote."""
        check(lib().ppk_kv_cache_advance(self.handle, previous, next_len), "ppk_kv_cache_advance")

    def graph_storage_identity(self) -> int | None:
        """LayerCache::graph_storage_identity (cache.rs:51-53): identity of the storage owner, None without storage."""
        return self.info().storage_id or None

    def info(self) -> _abi.PpkKvInfo:
        out = _abi.PpkKvInfo(struct_size=ctypes.sizeof(_abi.PpkKvInfo))
        check(lib().ppk_kv_cache_info(self.handle, ctypes.byref(out)), "ppk_kv_cache_info")
        return out

    def __len__(self) -> int:
        return self.info().length

    def truncate_committed(self, new_len: int) -> None:
        check(lib().ppk_kv_cache_truncate(self.handle, new_len), "ppk_kv_cache_truncate")

    def view(self) -> _abi.PpkKvView:
        out = _abi.PpkKvView(struct_size=ctypes.sizeof(_abi.PpkKvView))
        check(lib().ppk_kv_cache_view(self.handle, ctypes.byref(out)), "ppk_kv_cache_view")
        return out

    def key(self) -> torch.Tensor | None:
        """Copy of the committed keys [heads, len, D] (codes for int8), or None when empty."""
        v = self.view()
        return read(v, "k") if v.length else None

    def value(self) -> torch.Tensor | None:
        v = self.view()
        return read(v, "v") if v.length else None

    def query(self, k: torch.Tensor, v: torch.Tensor, past: int, commit: bool) -> _abi.PpkKvView:
        """k/v [heads, tokens, D] at slot `past` (= len(self)); returns the view of [0, past + tokens)."""
        if k.dim() != 3 or k.shape[0] != self.heads or k.shape[2] != self.head_dim:
            raise ValueError("K/V query shape differs from the cache geometry")
        k, v = k.contiguous(), v.contiguous()
        w = _write(k, v, k.shape[1], commit)
        out = _abi.PpkKvView(struct_size=ctypes.sizeof(_abi.PpkKvView))
        check(lib().ppk_kv_query(self.ctx, _stream(k), self.handle, past, ctypes.byref(w), ctypes.byref(out)),
              "ppk_kv_query")
        return out

    def query_int8_prefill(self, k: torch.Tensor, v: torch.Tensor, past: int, commit: bool
                           ) -> tuple[torch.Tensor, torch.Tensor]:
        """LayerCache::query_int8_prefill (cache.rs:133-141, int8_cache.rs:363-371): the committed int8
        history dequantised through bf16 (ppk_dequantize) and cast to k's dtype, concatenated with the
        original k/v chunk; the chunk itself is committed (quantised) as query() does. Only prefill
        uses this transient floating prefix."""
        from .int8_kv_ops import dequantize

        if self.kind != _abi.PPK_KV_INT8:
            raise ValueError("query_int8_prefill needs an INT8 cache")
        view = self.view()
        prefix = None
        if view.length:
            codes_k, codes_v = read(view, "k"), read(view, "v")
            sk, sv = read(view, "k_scales"), read(view, "v_scales")
            prefix = (dequantize(codes_k, sk, torch.bfloat16).to(k.dtype),
                      dequantize(codes_v, sv, torch.bfloat16).to(v.dtype))
        self.query(k, v, past, commit)
        if prefix is None:
            return k, v
        return torch.cat([prefix[0], k], 1), torch.cat([prefix[1], v], 1)

    @staticmethod
    def query_batch(caches: list["LayerCache"], k: torch.Tensor | None, v: torch.Tensor | None, past_lens,
                    commit: bool, plan: "WritePlan | None" = None) -> _abi.PpkKvView:
        """k/v [B, H, 1, D]: one token per sequence at slot past_lens[b]; returns the arena view
        [B*H, capacity, D] with length max(past) + 1 and device past / lengths vectors. k = v = None (int8
        caches) reserves the slot without writing it, for `decode_step(view, ...)` on the current stream."""
        b = len(caches)
        if k is None and v is None:
            w = _abi.PpkKvWrite(struct_size=ctypes.sizeof(_abi.PpkKvWrite), src_dtype=_abi.PPK_BF16, tokens=1,
                                commit=int(bool(commit)), k=None, v=None)
            stream = ctypes.c_void_p(torch.cuda.current_stream(caches[0].device).cuda_stream) if b else None
        else:
            if k.dim() != 4 or k.shape[0] != b or k.shape[2] != 1:
                raise ValueError("batch KV requires [B,H,1,D] scratch and matching row histories")
            k, v = k.contiguous(), v.contiguous()
            w = _write(k, v, 1, commit)
            stream = _stream(k)
        handles = (ctypes.c_void_p * b)(*[c.handle.value for c in caches])
        lens = (ctypes.c_uint32 * b)(*[int(x) for x in past_lens])
        out = _abi.PpkKvView(struct_size=ctypes.sizeof(_abi.PpkKvView))
        check(lib().ppk_kv_query_batch(caches[0].ctx, stream, handles, b, lens, ctypes.byref(w),
                                       plan.handle if plan is not None else None, ctypes.byref(out)),
              "ppk_kv_query_batch")
        return out


def decode_step(view: _abi.PpkKvView, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, heads: int, *,
                out_dtype: torch.dtype = torch.float32, past_host=None, flags: torch.Tensor | None = None,
                bf16_history: bool = False, plan: str = "auto") -> torch.Tensor:
    """The fused decode step over a reserved batch view (LayerCache.query_batch with k = v = None): write
    k_new / v_new (the current token, [B*H, D] or [B, H, 1, D]) into slot past[b] of the view's arenas and
    attend over [0, past[b]) plus that token, in one launch (two when rows span blocks); returns out
    [B*H, 1, D]. Int8 caches (ppk_decode_step): the token is quantised there and attended unquantised, the
    commit path of forward_batched_embedding (app/src/model/batch.rs:152-161) with query_int8 and
    int8_kv_ops::attention joined. Bf16 / f32 caches (ppk_float_decode_step): the token is rounded to the
    cache's dtype, written and attended, the float cache's commit + fused_attention::decode_attention
    (app/src/model/mod.rs:699-720) joined; bf16_history does not apply."""
    from .int8_kv_ops import _step_args, workspace_bytes

    if not view.batch or not view.past:
        raise ValueError("decode_step needs a batch view")
    if view.kind in (_abi.PPK_KV_BF16, _abi.PPK_KV_F32):
        return _float_decode_step(view, q, k_new, v_new, heads, out_dtype=out_dtype, past_host=past_host,
                                  flags=flags, plan=plan)
    if view.kind != _abi.PPK_KV_INT8:
        raise ValueError("decode_step needs the batch view of int8, bf16 or f32 caches")
    rows, d, cap = view.rows, view.head_dim, view.capacity
    for t in (q, k_new, v_new):
        if t.numel() != rows * d or t.dtype not in _DTYPES or not t.is_contiguous() or not t.is_cuda:
            raise ValueError("INT8 decode step operands must be dense float [B*H, D] on the device")
    if heads <= 0 or rows % heads or rows // heads != view.batch:
        raise ValueError("INT8 attention geometry differs")
    out = torch.empty((rows, 1, d), dtype=out_dtype, device=q.device)
    a = _abi.PpkAttentionArgs(
        struct_size=ctypes.sizeof(_abi.PpkAttentionArgs), q_dtype=_DTYPES[q.dtype], scratch_dtype=_DTYPES[k_new.dtype],
        out_dtype=_DTYPES[out_dtype],
        flags=(_abi.PPK_ATTN_BF16_HISTORY if bf16_history else 0) | _abi.plan_flags(plan), rows=rows,
        heads=heads, capacity=cap, head_dim=d, split_tokens=0, max_past=view.length - 1, softmax_scale=0.0,
        q=q.data_ptr(), k_codes=view.k, v_codes=view.v, k_scales=view.k_scales, v_scales=view.v_scales,
        sk=k_new.data_ptr(), sv=v_new.data_ptr(), past=view.past, out=out.data_ptr(), workspace=None,
        workspace_bytes=0, past_host=None)
    if past_host is not None:
        a._past_host = (ctypes.c_uint32 * view.batch)(*[int(x) for x in past_host])
        a.past_host = ctypes.cast(a._past_host, ctypes.c_void_p).value
    step = _step_args(a, k_new, v_new, flags, d)
    ctx = context(q.device)
    nbytes = workspace_bytes(a, ctx)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    step.attn.workspace = ws.data_ptr()
    step.attn.workspace_bytes = nbytes
    check(lib().ppk_decode_step(ctx, _stream(q), ctypes.byref(step)), "ppk_decode_step")
    return out


def _float_decode_step(view: _abi.PpkKvView, q, k_new, v_new, heads: int, *, out_dtype, past_host, flags,
                       plan: str) -> torch.Tensor:
    rows, d, cap = view.rows, view.head_dim, view.capacity
    for t in (q, k_new, v_new):
        if t.numel() != rows * d or t.dtype not in _DTYPES or not t.is_contiguous() or not t.is_cuda:
            raise ValueError("float decode step operands must be dense float [B*H, D] on the device")
    if heads <= 0 or rows % heads or rows // heads != view.batch or k_new.dtype != v_new.dtype:
        raise ValueError("float decode step geometry differs")
    if flags is not None and (flags.dtype not in (torch.int32, torch.uint32) or flags.numel() < 1):
        raise ValueError("flags must be one 32-bit word")
    out = torch.empty((rows, 1, d), dtype=out_dtype, device=q.device)
    a = _abi.PpkFloatAttentionArgs(
        struct_size=ctypes.sizeof(_abi.PpkFloatAttentionArgs),
        kv_dtype=_abi.PPK_BF16 if view.kind == _abi.PPK_KV_BF16 else _abi.PPK_F32, q_dtype=_DTYPES[q.dtype],
        out_dtype=_DTYPES[out_dtype], rows=rows, heads=heads, size=cap, head_dim=d, split_tokens=0,
        max_length=view.length, softmax_scale=0.0, flags=_abi.plan_flags(plan), q_row_stride=0, k_row_stride=0,
        v_row_stride=0, q=q.data_ptr(), k=view.k, v=view.v, lengths=view.past, out=out.data_ptr(), workspace=None,
        workspace_bytes=0, lengths_host=None)
    if past_host is not None:
        a._lengths_host = (ctypes.c_uint32 * view.batch)(*[int(x) for x in past_host])
        a.lengths_host = ctypes.cast(a._lengths_host, ctypes.c_void_p).value
    step = _abi.PpkFloatDecodeStepArgs(struct_size=ctypes.sizeof(_abi.PpkFloatDecodeStepArgs),
                                       new_dtype=_DTYPES[k_new.dtype], k_new=k_new.data_ptr(), v_new=v_new.data_ptr(),
                                       flags=flags.data_ptr() if flags is not None else None, attn=a)
    ctx = context(q.device)
    split, nsplits, nbytes = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint64()
    check(lib().ppk_float_attention_plan(ctx, ctypes.byref(step.attn), ctypes.byref(split), ctypes.byref(nsplits),
                                         ctypes.byref(nbytes)), "ppk_float_attention_plan")
    ws = torch.empty(max(nbytes.value, 1), dtype=torch.uint8, device=q.device)
    step.attn.workspace = ws.data_ptr()
    step.attn.workspace_bytes = nbytes.value
    check(lib().ppk_float_decode_step(ctx, _stream(q), ctypes.byref(step)), "ppk_float_decode_step")
    return out


def trim(device: torch.device | int | None = None) -> int:
    """ppk_context_trim: free the storage of released caches that the device's context keeps for reuse
    (and the unused memory of its pool); returns the bytes of kept storage freed."""
    released = ctypes.c_uint64()
    check(lib().ppk_context_trim(context(device), ctypes.byref(released)), "ppk_context_trim")
    return released.value


class WritePlan:
    """BatchWritePlan: one decode round's per-sequence write offsets on the device, shared by every layer."""

    def __init__(self, past_lens, heads: int, head_dim: int, device: torch.device | int | None = None):
        self.offsets = [int(x) for x in past_lens]
        b = len(self.offsets)
        lens = (ctypes.c_uint32 * max(b, 1))(*self.offsets)
        self.handle = ctypes.c_void_p()
        dev = device if device is not None else torch.cuda.current_device()
        stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        check(lib().ppk_write_plan_create(context(dev), stream, lens, b, heads, head_dim, ctypes.byref(self.handle)),
              "ppk_write_plan_create")

    def __del__(self):
        h = getattr(self, "handle", None)
        if h is not None and h.value and not sys.is_finalizing():
            lib().ppk_write_plan_release(h)
            self.handle = None
