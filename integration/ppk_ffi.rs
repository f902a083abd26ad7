//! Rust bindings of `include/ppk_int8_kv.h`, for the reference's Candle host
//! side (`app/src/model/`). Drop this file in as `app/src/model/ppk_ffi.rs`
//! and declare it with `#[cfg(feature = "rocm")] mod ppk_ffi;` in
//! `app/src/model/mod.rs`; link against `libppk.so`, shipped with its code
//! object `ppk_kernels.hsaco` beside it.
//!
//! Every `#[repr(C)]` block below mirrors the header field for field, in the
//! same order and with the same widths; `tests/test_rust_binding.py` parses
//! this file and checks each layout against the C compiler's. All-zero is a
//! valid value of every argument block (null pointers, zero sizes, dtype
//! PPK_F32), so build them with `zeroed()` and set the fields used.
//!
//! Status codes: 0 = ok; 1 = "HIP_PREPARATION: ..." (a precondition failed,
//! nothing was enqueued, a caller may fall back); 2 = a result failed its
//! check (self-checks); 3 = "HIP_EXECUTION_UNCERTAIN: ..." (work may have been
//! enqueued: never replay). These are the prefixes the reference's provider
//! classifies (app/src/inference/inference.rs:84-92,
//! app/src/model/hip_kernel.rs:150-165).

#![allow(non_camel_case_types, dead_code)]

use candle_core::{backend::BackendStorage, DType, Device, Layout, RocmStorage, Shape, Storage, Tensor};
use std::{
    collections::HashMap,
    ffi::{c_char, c_void, CStr},
    sync::{Mutex, OnceLock, RwLockReadGuard},
};

pub const PPK_ABI_VERSION: u32 = 1;

pub const PPK_OK: i32 = 0;
pub const PPK_PRECONDITION: i32 = 1;
pub const PPK_INVALID_OUTPUT: i32 = 2;
pub const PPK_EXECUTION_UNCERTAIN: i32 = 3;

/// Element types of floating tensors crossing the boundary.
pub const PPK_F32: u32 = 0;
pub const PPK_BF16: u32 = 1;
pub const PPK_F16: u32 = 2;

/// Device-side status bits OR-ed into an optional flags word.
pub const PPK_FLAG_NONFINITE: u32 = 1;
pub const PPK_FLAG_OVERFLOW: u32 = 2;
pub const PPK_FLAG_STALE_LENGTHS: u32 = 4;

/// Attention flags: dequantise history as bf16(code * scale) before the dot
/// products, exactly as pp_i8_load does (app/src/model/int8_kv.cu:23-27).
pub const PPK_ATTN_BF16_HISTORY: u32 = 1;
/// Launch plan with host lengths: force the per-row plan, or the balanced
/// plan for ragged batches (default: the library chooses).
pub const PPK_ATTN_PLAN_PER_ROW: u32 = 2;
pub const PPK_ATTN_PLAN_BALANCED: u32 = 4;

/// Bytes of the per-GPU array behind `ppk_decode_step_noalloc`.
pub const PPK_NOALLOC_SCRATCH_BYTES: u32 = 8 << 20;

/// KV cache kinds.
pub const PPK_KV_INT8: u32 = 0;
pub const PPK_KV_BF16: u32 = 1;
pub const PPK_KV_F16: u32 = 2;
pub const PPK_KV_F32: u32 = 3;

/// Kernel ids of `ppk_context_kernel_stats`.
pub const PPK_KERNEL_QUANTIZE: u32 = 0;
pub const PPK_KERNEL_APPEND: u32 = 1;
pub const PPK_KERNEL_DEQUANTIZE: u32 = 2;
pub const PPK_KERNEL_ATTENTION: u32 = 3;
pub const PPK_KERNEL_ATTN_MERGE: u32 = 4;
pub const PPK_KERNEL_FLOAT_ATTENTION: u32 = 5;
pub const PPK_KERNEL_FLOAT_MERGE: u32 = 6;
pub const PPK_KERNEL_RENYI_SAMPLE: u32 = 7;
pub const PPK_KERNEL_COPY: u32 = 8;
pub const PPK_KERNEL_COUNT: u32 = 9;

/// Opaque handles.
#[repr(C)]
pub struct ppk_context {
    _opaque: [u8; 0],
}
#[repr(C)]
pub struct ppk_kv_cache {
    _opaque: [u8; 0],
}
#[repr(C)]
pub struct ppk_write_plan {
    _opaque: [u8; 0],
}

/// Dense quantize (int8_kv_ops::quantize, app/src/model/int8_kv_ops.rs:11-29).
#[repr(C)]
#[derive(Clone, Copy)]
pub struct PpkQuantizeArgs {
    pub struct_size: u32,
    pub src_dtype: u32,
    pub src: *const c_void,
    pub codes: *mut u8,
    pub scales: *mut f32,
    pub rows: u64,
    pub head_dim: u32,
    pub reserved: u32,
    pub flags: *mut u32,
}

/// Fused quantize + append into the arenas at slot past[b] + j (the commit
/// path of Int8LayerCache::query / query_batch, app/src/model/int8_cache.rs:293-359).
#[repr(C)]
#[derive(Clone, Copy)]
pub struct PpkAppendArgs {
    pub struct_size: u32,
    pub src_dtype: u32,
    pub k_src: *const c_void,
    pub v_src: *const c_void,
    pub past: *const u32,
    pub k_codes: *mut u8,
    pub v_codes: *mut u8,
    pub k_scales: *mut f32,
    pub v_scales: *mut f32,
    pub batch: u32,
    pub heads: u32,
    pub tokens: u32,
    pub head_dim: u32,
    pub capacity: u32,
    pub reserved: u32,
    pub flags: *mut u32,
}

/// int8_kv_ops::dequantize (int8_kv_ops.rs:30-40).
#[repr(C)]
#[derive(Clone, Copy)]
pub struct PpkDequantizeArgs {
    pub struct_size: u32,
    pub out_dtype: u32,
    pub codes: *const u8,
    pub scales: *const f32,
    pub out: *mut c_void,
    pub rows: u64,
    pub head_dim: u32,
    pub round_bf16: u32,
}

/// int8_kv_ops::attention (int8_kv_ops.rs:41-55). `past_host` is optional
/// (null): the host copy of `past` that lets the library balance a ragged
/// batch (or size its per-row plan for the longest length); the device
/// `past` is still read, and a length the plan does not cover gives NaN rows.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct PpkAttentionArgs {
    pub struct_size: u32,
    pub q_dtype: u32,
    pub scratch_dtype: u32,
    pub out_dtype: u32,
    pub flags: u32,
    pub rows: u32,
    pub heads: u32,
    pub capacity: u32,
    pub head_dim: u32,
    pub split_tokens: u32,
    pub max_past: u32,
    pub softmax_scale: f32,
    pub q: *const c_void,
    pub k_codes: *const u8,
    pub v_codes: *const u8,
    pub k_scales: *const f32,
    pub v_scales: *const f32,
    pub sk: *const c_void,
    pub sv: *const c_void,
    pub past: *const u32,
    pub out: *mut c_void,
    pub workspace: *mut c_void,
    pub workspace_bytes: u64,
    pub past_host: *const u32,
}

/// One decode step: append the current token, then attend (mod.rs:699-705).
#[repr(C)]
#[derive(Clone, Copy)]
pub struct PpkDecodeStepArgs {
    pub struct_size: u32,
    pub new_dtype: u32,
    pub k_new: *const c_void,
    pub v_new: *const c_void,
    pub flags: *mut u32,
    pub attn: PpkAttentionArgs,
}

/// Float-KV decode attention (hip_attention::decode_attention, app/src/model/hip_attention.rs:47-113).
#[repr(C)]
#[derive(Clone, Copy)]
pub struct PpkFloatAttentionArgs {
    pub struct_size: u32,
    pub kv_dtype: u32,
    pub q_dtype: u32,
    pub out_dtype: u32,
    pub rows: u32,
    pub heads: u32,
    pub size: u32,
    pub head_dim: u32,
    pub split_tokens: u32,
    pub max_length: u32,
    pub softmax_scale: f32,
    pub flags: u32,
    pub q_row_stride: u64,
    pub k_row_stride: u64,
    pub v_row_stride: u64,
    pub q: *const c_void,
    pub k: *const c_void,
    pub v: *const c_void,
    pub lengths: *const u32,
    pub out: *mut c_void,
    pub workspace: *mut c_void,
    pub workspace_bytes: u64,
    pub lengths_host: *const u32,
}

/// The float path's fused decode step (the graph-decode session's scatter_set
/// pair + decode_attention, app/src/model/graph_decode.rs:290-305).
#[repr(C)]
#[derive(Clone, Copy)]
pub struct PpkFloatDecodeStepArgs {
    pub struct_size: u32,
    pub new_dtype: u32,
    pub k_new: *const c_void,
    pub v_new: *const c_void,
    pub flags: *mut u32,
    pub attn: PpkFloatAttentionArgs,
}

/// CFG + Renyi sampler (hip_sampling::sample, app/src/inference/hip_sampling.rs:71-106).
#[repr(C)]
#[derive(Clone, Copy)]
pub struct PpkRenyiSampleArgs {
    pub struct_size: u32,
    pub batch: u32,
    pub choices: u32,
    pub guidance: u32,
    pub alpha: f32,
    pub cfg: f32,
    pub token_offset: u32,
    pub reserved: u32,
    pub raw: *const f32,
    pub uniforms: *const f32,
    pub bounds: *const u32,
    pub out: *mut u32,
}

/// LayerCache geometry (app/src/model/cache.rs:40-531).
#[repr(C)]
#[derive(Clone, Copy)]
pub struct PpkKvConfig {
    pub struct_size: u32,
    pub kind: u32,
    pub heads: u32,
    pub head_dim: u32,
    pub max_context: u32,
    pub min_capacity: u32,
}

/// Device view of cache storage (single cache or batch arena).
#[repr(C)]
#[derive(Clone, Copy)]
pub struct PpkKvView {
    pub struct_size: u32,
    pub kind: u32,
    pub rows: u32,
    pub capacity: u32,
    pub head_dim: u32,
    pub length: u32,
    pub batch: u32,
    pub reserved: u32,
    pub k: *mut c_void,
    pub v: *mut c_void,
    pub k_scales: *mut f32,
    pub v_scales: *mut f32,
    pub past: *const u32,
    pub lengths: *const u32,
}

#[repr(C)]
#[derive(Clone, Copy)]
pub struct PpkKvInfo {
    pub struct_size: u32,
    pub length: u32,
    pub capacity: u32,
    pub grouped: u32,
    pub slot: u32,
    pub shared: u32,
    pub reserved_bytes: u64,
    pub storage_id: u64,
    pub arena_id: u64,
    pub arena_copied_rows: u64,
    pub arena_offset_uploads: u64,
    pub scale_bytes: u64,
}

/// Source of a cache write.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct PpkKvWrite {
    pub struct_size: u32,
    pub src_dtype: u32,
    pub tokens: u32,
    pub commit: u32,
    pub k: *const c_void,
    pub v: *const c_void,
}

/// Int8KvStatus (app/src/model/int8_policy.rs:3-56).
#[repr(C)]
#[derive(Clone, Copy)]
pub struct PpkInt8KvStatus {
    pub struct_size: u32,
    pub requested: u32,
    pub available: u32,
    pub ready: u32,
    pub enabled: u32,
    pub packed_bytes_per_token_head: u32,
    pub scale_bytes_per_token_head: u32,
    pub reserved: u32,
    pub format: [c_char; 64],
    pub reason: [c_char; 256],
}

/// The whole launch plan (no counterpart in the reference).
#[repr(C)]
#[derive(Clone, Copy)]
pub struct PpkAttentionPlanInfo {
    pub struct_size: u32,
    pub kind: u32,
    pub split_tokens: u32,
    pub nsplits: u32,
    pub waves_per_block: u32,
    pub blocks: u32,
    pub launches: u32,
    pub reserved: u32,
    pub workspace_bytes: u64,
}

#[link(name = "ppk")]
extern "C" {
    pub fn ppk_abi_version() -> u32;
    pub fn ppk_last_error() -> *const c_char;
    pub fn ppk_context_create(device: i32, code_object_path: *const c_char, out: *mut *mut ppk_context) -> i32;
    pub fn ppk_context_release(ctx: *mut ppk_context) -> i32;
    pub fn ppk_context_trim(ctx: *mut ppk_context, released_bytes: *mut u64) -> i32;
    pub fn ppk_quantize(ctx: *mut ppk_context, stream: *mut c_void, args: *const PpkQuantizeArgs) -> i32;
    pub fn ppk_quantize_append(ctx: *mut ppk_context, stream: *mut c_void, args: *const PpkAppendArgs) -> i32;
    pub fn ppk_dequantize(ctx: *mut ppk_context, stream: *mut c_void, args: *const PpkDequantizeArgs) -> i32;
    pub fn ppk_attention_workspace_bytes(ctx: *mut ppk_context, args: *const PpkAttentionArgs, bytes: *mut u64) -> i32;
    pub fn ppk_attention_plan(
        ctx: *mut ppk_context,
        args: *const PpkAttentionArgs,
        split_tokens: *mut u32,
        nsplits: *mut u32,
        workspace_bytes: *mut u64,
    ) -> i32;
    pub fn ppk_decode_attention(ctx: *mut ppk_context, stream: *mut c_void, args: *const PpkAttentionArgs) -> i32;
    pub fn ppk_decode_step(ctx: *mut ppk_context, stream: *mut c_void, args: *const PpkDecodeStepArgs) -> i32;
    pub fn ppk_decode_step_noalloc(ctx: *mut ppk_context, stream: *mut c_void, args: *const PpkDecodeStepArgs) -> i32;
    pub fn ppk_attention_plan_info(
        ctx: *mut ppk_context,
        args: *const PpkAttentionArgs,
        info: *mut PpkAttentionPlanInfo,
    ) -> i32;
    pub fn ppk_float_attention_plan_info(
        ctx: *mut ppk_context,
        args: *const PpkFloatAttentionArgs,
        info: *mut PpkAttentionPlanInfo,
    ) -> i32;
    pub fn ppk_float_attention_plan(
        ctx: *mut ppk_context,
        args: *const PpkFloatAttentionArgs,
        split_tokens: *mut u32,
        nsplits: *mut u32,
        workspace_bytes: *mut u64,
    ) -> i32;
    pub fn ppk_float_decode_attention(ctx: *mut ppk_context, stream: *mut c_void, args: *const PpkFloatAttentionArgs) -> i32;
    pub fn ppk_float_decode_step(ctx: *mut ppk_context, stream: *mut c_void, args: *const PpkFloatDecodeStepArgs) -> i32;
    pub fn ppk_float_attention_prepare(ctx: *mut ppk_context) -> i32;
    pub fn ppk_renyi_sample(ctx: *mut ppk_context, stream: *mut c_void, args: *const PpkRenyiSampleArgs) -> i32;
    pub fn ppk_kv_cache_create(ctx: *mut ppk_context, config: *const PpkKvConfig, out: *mut *mut ppk_kv_cache) -> i32;
    pub fn ppk_kv_cache_clone(cache: *const ppk_kv_cache, out: *mut *mut ppk_kv_cache) -> i32;
    pub fn ppk_kv_cache_release(cache: *mut ppk_kv_cache) -> i32;
    pub fn ppk_kv_cache_info(cache: *const ppk_kv_cache, out: *mut PpkKvInfo) -> i32;
    pub fn ppk_kv_cache_truncate(cache: *mut ppk_kv_cache, new_len: u32) -> i32;
    pub fn ppk_kv_cache_adopt(
        ctx: *mut ppk_context,
        config: *const PpkKvConfig,
        k: *mut c_void,
        v: *mut c_void,
        capacity: u32,
        committed_len: u32,
        out: *mut *mut ppk_kv_cache,
    ) -> i32;
    pub fn ppk_kv_cache_advance(cache: *mut ppk_kv_cache, previous: u32, next: u32) -> i32;
    pub fn ppk_kv_cache_view(cache: *const ppk_kv_cache, out: *mut PpkKvView) -> i32;
    pub fn ppk_kv_query(
        ctx: *mut ppk_context,
        stream: *mut c_void,
        cache: *mut ppk_kv_cache,
        past: u32,
        write: *const PpkKvWrite,
        out: *mut PpkKvView,
    ) -> i32;
    pub fn ppk_write_plan_create(
        ctx: *mut ppk_context,
        stream: *mut c_void,
        past_lens: *const u32,
        batch: u32,
        heads: u32,
        head_dim: u32,
        out: *mut *mut ppk_write_plan,
    ) -> i32;
    pub fn ppk_write_plan_release(plan: *mut ppk_write_plan) -> i32;
    pub fn ppk_kv_query_batch(
        ctx: *mut ppk_context,
        stream: *mut c_void,
        caches: *const *mut ppk_kv_cache,
        batch: u32,
        past_lens: *const u32,
        write: *const PpkKvWrite,
        plan: *const ppk_write_plan,
        out: *mut PpkKvView,
    ) -> i32;
    pub fn ppk_prepare(ctx: *mut ppk_context) -> i32;
    pub fn ppk_prepare_int8_kv(ctx: *mut ppk_context, requested: u32, head_dim: u32, out: *mut PpkInt8KvStatus) -> i32;
    pub fn ppk_context_set_profiling(ctx: *mut ppk_context, enable: i32) -> i32;
    pub fn ppk_context_set_wave_clock(ctx: *mut ppk_context, buffer: *mut c_void, bytes: u64) -> i32;
    pub fn ppk_context_kernel_stats(
        ctx: *mut ppk_context,
        kernel: u32,
        launches: *mut u64,
        total_ms: *mut f64,
        reset: u32,
    ) -> i32;
}

/// An argument block with every field zero and `struct_size` set.
pub fn args<T: Copy>() -> T {
    // SAFETY: every argument block above is plain data for which all-zero is
    // a valid value (null pointers, zero sizes, PPK_F32).
    let mut value: T = unsafe { std::mem::zeroed() };
    let size = std::mem::size_of::<T>() as u32;
    // SAFETY: each block starts with `struct_size: u32`.
    unsafe { *(&mut value as *mut T as *mut u32) = size };
    value
}

/// The calling thread's last library error.
pub fn last_error() -> String {
    // SAFETY: ppk_last_error returns a NUL-terminated thread-local string.
    unsafe { CStr::from_ptr(ppk_last_error()) }.to_string_lossy().into_owned()
}

/// Status -> Candle error, keeping the library's message (and with it the
/// HIP_PREPARATION / HIP_EXECUTION_UNCERTAIN prefix the provider classifies).
pub fn check(status: i32) -> candle_core::Result<()> {
    match status {
        PPK_OK => Ok(()),
        _ => Err(candle_core::Error::Msg(last_error())),
    }
}

// ---- Candle helpers shared by the ROCm ops ------------------------------------
// (int8_kv_ops_rocm.rs, hip_attention_rocm.rs, hip_sampling_rocm.rs)

/// The stream of every library call: the null HIP stream, the one the
/// reference's own HIP kernels are launched on (hip_kernel::launch ->
/// HipModule::launch), so the calls stay ordered with them.
pub const STREAM: *mut c_void = std::ptr::null_mut();

struct Context(*mut ppk_context);
// SAFETY: a ppk_context may be used from any thread; the library serialises
// its own state.
unsafe impl Send for Context {}

/// The library context of a HIP device, created once per process (the module
/// cache of app/src/model/hip_kernel.rs:45,107) and kept until exit. Creation
/// loads the gfx950 code object beside libppk.so and resolves every kernel.
pub fn context(ordinal: usize) -> candle_core::Result<*mut ppk_context> {
    static CONTEXTS: OnceLock<Mutex<HashMap<usize, Context>>> = OnceLock::new();
    let mut map = CONTEXTS
        .get_or_init(|| Mutex::new(HashMap::new()))
        .lock()
        .map_err(|_| candle_core::Error::Msg("HIP_PREPARATION: ppk context cache poisoned".into()))?;
    if let Some(ctx) = map.get(&ordinal) {
        return Ok(ctx.0);
    }
    if unsafe { ppk_abi_version() } != PPK_ABI_VERSION {
        candle_core::bail!("HIP_PREPARATION: libppk ABI version differs from ppk_ffi.rs");
    }
    let mut ctx = std::ptr::null_mut();
    check(unsafe { ppk_context_create(ordinal as i32, std::ptr::null(), &mut ctx) })?;
    map.insert(ordinal, Context(ctx));
    Ok(ctx)
}

pub fn device_context(device: &Device) -> candle_core::Result<*mut ppk_context> {
    match device {
        Device::Rocm(d) => context(d.ordinal()),
        _ => candle_core::bail!("HIP_PREPARATION: libppk op on a non-ROCm device"),
    }
}

pub fn dtype_code(dtype: DType) -> candle_core::Result<u32> {
    match dtype {
        DType::F32 => Ok(PPK_F32),
        DType::BF16 => Ok(PPK_BF16),
        DType::F16 => Ok(PPK_F16),
        other => candle_core::bail!("HIP_PREPARATION: libppk does not take {other:?} tensors"),
    }
}

/// Device address of a dense view of `elems` elements, after checking that
/// the view lies inside its storage (as checked_span does, hip_attention.rs:63-69).
pub fn span(
    storage: &RocmStorage,
    layout: &Layout,
    elems: usize,
    elem_bytes: usize,
    what: &str,
) -> candle_core::Result<*mut c_void> {
    let (start, end) = layout
        .contiguous_offsets()
        .ok_or_else(|| candle_core::Error::Msg(format!("HIP_PREPARATION: {what} is not contiguous")))?;
    if end - start != elems || end.checked_mul(elem_bytes).is_none_or(|n| n > storage.byte_len()) {
        candle_core::bail!("HIP_PREPARATION: {what} view exceeds its storage");
    }
    Ok(unsafe { storage.device_ptr().add(start * elem_bytes) } as *mut c_void)
}

/// The read guards of the side tensors an op reads or writes, held until the
/// library call has been enqueued (as the reference holds its `lengths`
/// storage, hip_attention.rs:93-101).
pub struct Bound<'a> {
    guards: Vec<RwLockReadGuard<'a, Storage>>,
}

impl<'a> Bound<'a> {
    pub fn new() -> Self {
        Bound { guards: Vec::new() }
    }

    pub fn ptr(&mut self, t: &'a Tensor, dtype: DType, what: &str) -> candle_core::Result<*mut c_void> {
        if t.dtype() != dtype {
            candle_core::bail!("HIP_PREPARATION: {what} must be {dtype:?}");
        }
        let (guard, layout) = t.storage_and_layout();
        let ptr = match &*guard {
            Storage::Rocm(s) => span(s, layout, t.elem_count(), dtype.size_in_bytes(), what)?,
            _ => candle_core::bail!("HIP_PREPARATION: {what} is not on the ROCm device"),
        };
        self.guards.push(guard);
        Ok(ptr)
    }
}

/// Device scratch of `bytes` (None for 0), released when the op returns, as
/// the reference releases its `partial` buffer (hip_attention.rs:87-110).
pub fn workspace(device: &candle_core::rocm_backend::RocmDevice, bytes: u64) -> candle_core::Result<Option<RocmStorage>> {
    use candle_core::backend::BackendDevice;
    if bytes == 0 {
        return Ok(None);
    }
    // hipMalloc memory: 256-byte aligned, as the library requires.
    Ok(Some(unsafe { device.alloc_uninit(&Shape::from(bytes as usize), DType::U8)? }))
}
