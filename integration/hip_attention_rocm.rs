//! The float-KV decode attention (app/src/model/hip_attention.rs) over the
//! MI355X library `libppk.so`: the same three functions, `prepare`,
//! `validate_split_k` and `decode_attention`, with the hiprtc module and the
//! pp_attention_* launches replaced by `ppk_float_decode_attention`.
//!
//! Install: copy this file over `app/src/model/hip_attention.rs` (and
//! `ppk_ffi.rs` to `app/src/model/ppk_ffi.rs`, declared in `mod.rs` with
//! `#[cfg(feature = "rocm")] mod ppk_ffi;`). Callers keep their calls. The
//! NVIDIA-only limits of fused_attention::decode_attention (D == 64, length
//! <= 1024, F32 q; app/src/model/fused_attention.rs:11-16) sit before its
//! ROCm dispatch (:27-28); move that dispatch above them to let the ROCm
//! branch take D = 128 / 256, longer stores and bf16 / f16 queries, which
//! this file validates itself.
//!
//! The graph-decode session (app/src/model/graph_decode.rs:298-305) holds the
//! attended lengths on the host too (`expected_lengths[row] + 1`, :224-253):
//! passing them to `decode_attention_with_host_lengths` lets the library
//! balance a ragged batch (a 4-sequence x 8192 beside 28 x 512 bf16 batch at
//! D = 128: 111.8 -> 67.2 us per call). Every call runs on the null HIP
//! stream, and there is no CPU fallback (hip_attention.rs:75).

use crate::model::ppk_ffi as ffi;
use crate::model::ppk_ffi::{context, device_context, dtype_code, workspace, Bound, STREAM};
use anyhow::{bail, ensure, Result};
use candle_core::{backend::BackendStorage, CpuStorage, CustomOp3, DType, Layout, RocmStorage, Shape, Tensor};
use std::ffi::c_void;

/// hip_attention::prepare (hip_attention.rs:7-13): the library context of the
/// device, which loads the gfx950 code object and resolves every kernel, the
/// float path's among them. A failure is HIP_PREPARATION.
pub(crate) fn prepare(device: &candle_core::Device) -> Result<()> {
    device_context(device)?;
    Ok(())
}

/// hip_attention::validate_split_k (hip_attention.rs:15-45): the same private
/// inputs (a 257-token bf16 and f32 store, D = 64), split 0 and 128 against an
/// f32 softmax reference and each other within 1e-4, and zero inputs giving
/// zero, run on the device by the library. A numeric mismatch withholds the
/// capability (HIP_PREPARATION, as the reference bails); a failed readback
/// is HIP_EXECUTION_UNCERTAIN.
pub(crate) fn validate_split_k(device: &candle_core::Device) -> Result<()> {
    let ctx = device_context(device)?;
    let status = unsafe { ffi::ppk_float_attention_prepare(ctx) };
    if status == ffi::PPK_INVALID_OUTPUT {
        bail!("HIP_PREPARATION: Split-K private numerical check failed: {}", ffi::last_error());
    }
    Ok(ffi::check(status)?)
}

/// hip_attention::decode_attention (hip_attention.rs:47-61): q [rows, 1, D]
/// against K/V [rows, length, D] (BF16 or F32, the current token already
/// stored), each row attending lengths[row / heads] tokens, or `length`
/// without lengths; F32 [rows, 1, D] out. Beyond the reference: D of 64, 128
/// or 256, any length, and BF16 / F16 queries. `split_tokens` is a hint: the
/// result does not depend on it. A row whose length is 0 or beyond the store
/// gives NaN, as the reference's kernels do (decode_attention.hip:15,50).
pub(super) fn decode_attention(
    q: &Tensor,
    k: &Tensor,
    v: &Tensor,
    lengths: Option<&Tensor>,
    heads: usize,
    split_tokens: usize,
) -> Result<Tensor> {
    decode_attention_with_host_lengths(q, k, v, lengths, None, heads, split_tokens)
}

/// decode_attention with the host's copy of `lengths` (no counterpart in the
/// reference): the library plans a ragged batch from it and compares every
/// device length with it; a sequence whose values differ gives NaN rows,
/// never a wrong result.
pub(super) fn decode_attention_with_host_lengths(
    q: &Tensor,
    k: &Tensor,
    v: &Tensor,
    lengths: Option<&Tensor>,
    lengths_host: Option<&[u32]>,
    heads: usize,
    split_tokens: usize,
) -> Result<Tensor> {
    let op = decode_attention_op(q, k, v, lengths, lengths_host, heads, split_tokens)?;
    Ok(q.apply_op3_no_bwd(k, v, &op)?)
}

/// The op of one attention call after the checks of hip_attention.rs:48-60
/// (widened to D = 64 / 128 / 256, any length and F32 / BF16 / F16 queries).
fn decode_attention_op(
    q: &Tensor,
    k: &Tensor,
    v: &Tensor,
    lengths: Option<&Tensor>,
    lengths_host: Option<&[u32]>,
    heads: usize,
    split_tokens: usize,
) -> Result<Decode> {
    let (rows, query, width) = q.dims3()?;
    let (key_rows, length, key_width) = k.dims3()?;
    ensure!(
        heads > 0
            && rows > 0
            && rows <= u32::MAX as usize
            && rows % heads == 0
            && query == 1
            && matches!(width, 64 | 128 | 256)
            && key_rows == rows
            && key_width == width
            && length > 0
            && length <= u32::MAX as usize
            && v.dims() == k.dims()
            && matches!(q.dtype(), DType::F32 | DType::BF16 | DType::F16)
            && matches!(k.dtype(), DType::BF16 | DType::F32)
            && k.dtype() == v.dtype()
            && q.device().is_rocm()
            && q.device().same_device(k.device())
            && q.device().same_device(v.device()),
        "HIP decode requires same-device float[batch*heads,1,D] Q and BF16/F32[batch*heads,length,D] K/V, D in 64/128/256"
    );
    for tensor in [q, k, v] {
        ensure!(
            tensor.stride()[2] == 1 && tensor.stride()[1] == width,
            "HIP attention requires dense width/token strides"
        );
    }
    if let Some(lengths) = lengths {
        ensure!(
            lengths.dims1()? == rows / heads
                && lengths.dtype() == DType::U32
                && lengths.is_contiguous()
                && q.device().same_device(lengths.device()),
            "HIP attention lengths require same-device U32[batch]"
        );
    }
    if let Some(host) = lengths_host {
        ensure!(lengths.is_some() && host.len() == rows / heads, "HIP attention host lengths differ from the batch");
    }
    Ok(Decode {
        heads,
        rows,
        length,
        width,
        split: split_tokens,
        lengths: lengths.cloned(),
        lengths_host: lengths_host.map(<[u32]>::to_vec),
        step: None,
    })
}

/// The graph-decode session's per-layer commit + attend
/// (app/src/model/graph_decode.rs:290-305: scatter_set of the current K/V at
/// write_indices, then decode_attention over lengths + 1) in one call
/// (no counterpart fuses them in the reference): k_new / v_new [rows, 1, D]
/// (F32, BF16 or F16) are rounded to the store's dtype and written at slot
/// lengths[b] of k / v [rows, length, D], which the op writes in place (they
/// must be the caller's alone, as the session's own buffers are), and each
/// row attends its lengths[b] stored tokens plus that one. `lengths` holds
/// the stored counts before this step (the session's `lengths`, not
/// `valid_lengths`); `lengths_host` its host copy (`expected_lengths`). A row
/// whose slot is past the store is not written, sets PPK_FLAG_OVERFLOW in
/// `flags` (optional U32[1]) and gives NaN.
#[allow(clippy::too_many_arguments)]
pub(super) fn decode_step(
    q: &Tensor,
    k: &Tensor,
    v: &Tensor,
    lengths: &Tensor,
    lengths_host: Option<&[u32]>,
    heads: usize,
    k_new: &Tensor,
    v_new: &Tensor,
    flags: Option<&Tensor>,
) -> Result<Tensor> {
    let (rows, _, width) = q.dims3()?;
    ensure!(
        k_new.dims() == [rows, 1, width] && v_new.dims() == k_new.dims() && k_new.dtype() == v_new.dtype(),
        "HIP decode step current token must be [batch*heads,1,D]"
    );
    if let Some(flags) = flags {
        ensure!(flags.dims1()? >= 1 && flags.dtype() == DType::U32, "HIP decode step flags must be U32[1]");
    }
    // The shape, dtype and stride checks of the attention (the op below is the same one with the step's
    // operands attached).
    let checked = decode_attention_op(q, k, v, Some(lengths), lengths_host, heads, 0)?;
    let op = Decode { step: Some((k_new.clone(), v_new.clone(), flags.cloned())), ..checked };
    Ok(q.apply_op3_no_bwd(k, v, &op)?)
}

struct Decode {
    heads: usize,
    rows: usize,
    length: usize,
    width: usize,
    split: usize,
    lengths: Option<Tensor>,
    lengths_host: Option<Vec<u32>>,
    step: Option<(Tensor, Tensor, Option<Tensor>)>,
}

/// Start address and row stride (elements) of a [rows, n, D] view whose
/// tokens are dense, after checking that its last element lies inside the
/// storage (hip_attention.rs:63-69).
fn rows_view(
    storage: &RocmStorage,
    layout: &Layout,
    rows: usize,
    n: usize,
    width: usize,
    what: &str,
) -> candle_core::Result<(*mut c_void, u64)> {
    let elem_bytes = storage.dtype().size_in_bytes();
    let stride = layout.stride()[0];
    let last = (rows - 1)
        .checked_mul(stride)
        .and_then(|x| x.checked_add(n * width))
        .and_then(|x| x.checked_add(layout.start_offset()))
        .and_then(|x| x.checked_mul(elem_bytes));
    if last.is_none_or(|last| last > storage.byte_len()) {
        candle_core::bail!("HIP_PREPARATION: HIP attention {what} view exceeds underlying storage");
    }
    let ptr = unsafe { storage.device_ptr().add(layout.start_offset() * elem_bytes) } as *mut c_void;
    Ok((ptr, stride as u64))
}

impl CustomOp3 for Decode {
    fn name(&self) -> &'static str {
        if self.step.is_some() {
            "ppk-float-decode-step"
        } else {
            "ppk-float-decode-attention"
        }
    }

    fn cpu_fwd(
        &self,
        _: &CpuStorage,
        _: &Layout,
        _: &CpuStorage,
        _: &Layout,
        _: &CpuStorage,
        _: &Layout,
    ) -> candle_core::Result<(CpuStorage, Shape)> {
        candle_core::bail!("HIP attention never falls back to CPU")
    }

    fn rocm_fwd(
        &self,
        q: &RocmStorage,
        ql: &Layout,
        k: &RocmStorage,
        kl: &Layout,
        v: &RocmStorage,
        vl: &Layout,
    ) -> candle_core::Result<(RocmStorage, Shape)> {
        use candle_core::backend::BackendDevice;
        let device = q.rocm_device();
        let ctx = context(device.ordinal())?;
        let (qp, qs) = rows_view(q, ql, self.rows, 1, self.width, "query")?;
        let (kp, ks) = rows_view(k, kl, self.rows, self.length, self.width, "key")?;
        let (vp, vs) = rows_view(v, vl, self.rows, self.length, self.width, "value")?;
        let mut bound = Bound::new();
        let mut a: ffi::PpkFloatAttentionArgs = ffi::args();
        a.kv_dtype = if k.dtype() == DType::BF16 { ffi::PPK_BF16 } else { ffi::PPK_F32 };
        a.q_dtype = dtype_code(q.dtype())?;
        a.out_dtype = ffi::PPK_F32;
        a.rows = self.rows as u32;
        a.heads = self.heads as u32;
        a.size = self.length as u32;
        a.head_dim = self.width as u32;
        a.split_tokens = self.split as u32;
        a.q_row_stride = qs;
        a.k_row_stride = ks;
        a.v_row_stride = vs;
        a.q = qp;
        a.k = kp;
        a.v = vp;
        if let Some(lengths) = &self.lengths {
            a.lengths = bound.ptr(lengths, DType::U32, "HIP attention lengths")? as *const u32;
        }
        if let Some(host) = &self.lengths_host {
            // The plan covers the longest live row only; a row beyond it gives NaN.
            a.max_length = host.iter().copied().filter(|&n| n as usize <= self.length).max().unwrap_or(0);
            a.lengths_host = host.as_ptr();
        }
        let shape: Shape = (self.rows, 1, self.width).into();
        let mut out = unsafe { device.alloc_uninit(&shape, DType::F32)? };
        a.out = out.device_ptr_mut() as *mut c_void;
        let mut bytes = 0u64;
        ffi::check(unsafe {
            ffi::ppk_float_attention_plan(ctx, &a, std::ptr::null_mut(), std::ptr::null_mut(), &mut bytes)
        })?;
        let mut ws = workspace(device, bytes)?;
        if let Some(ws) = ws.as_mut() {
            a.workspace = ws.device_ptr_mut() as *mut c_void;
            a.workspace_bytes = bytes;
        }
        match &self.step {
            None => ffi::check(unsafe { ffi::ppk_float_decode_attention(ctx, STREAM, &a) })?,
            Some((k_new, v_new, flags)) => {
                let mut s: ffi::PpkFloatDecodeStepArgs = ffi::args();
                s.new_dtype = dtype_code(k_new.dtype())?;
                s.k_new = bound.ptr(k_new, k_new.dtype(), "HIP decode step key")?;
                s.v_new = bound.ptr(v_new, k_new.dtype(), "HIP decode step value")?;
                if let Some(flags) = flags {
                    s.flags = bound.ptr(flags, DType::U32, "HIP decode step flags")? as *mut u32;
                }
                s.attn = a;
                ffi::check(unsafe { ffi::ppk_float_decode_step(ctx, STREAM, &s) })?;
            }
        }
        Ok((out, shape))
    }
}
