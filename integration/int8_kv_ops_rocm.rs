//! ROCm branches of `int8_kv_ops` (app/src/model/int8_kv_ops.rs) over the
//! MI355X library `libppk.so`, as Candle custom ops on a Candle build with a
//! ROCm backend (the `rocm` feature that app/src/model/hip_attention.rs and
//! app/src/inference/hip_sampling.rs are written against).
//!
//! Install: copy this file to `app/src/model/int8_kv_ops_rocm.rs` and
//! `ppk_ffi.rs` to `app/src/model/ppk_ffi.rs`, then
//!
//! * in `app/src/model/mod.rs`: `#[cfg(feature = "rocm")] mod ppk_ffi;`
//! * in `app/src/model/int8_kv_ops.rs`, beside `mod cuda`:
//!   `#[cfg(feature = "rocm")] #[path = "int8_kv_ops_rocm.rs"] mod rocm;`
//!   and one branch per function, after its existing checks and before its
//!   `#[cfg(feature = "cuda")]` branch:
//!   - quantize (:11-29):   `#[cfg(feature="rocm")] if input.device().is_rocm(){return rocm::quantize(input);}`
//!   - dequantize (:30-40): `#[cfg(feature="rocm")] if packed.device().is_rocm(){return rocm::dequantize(packed,scale,dtype);}`
//!   - attention (:41-55):  `#[cfg(feature="rocm")] if q.device().is_rocm(){return rocm::attention(q,k,v,ks,vs,sk,sv,past,heads,split_tokens,None);}`
//!   - prepare (:57-103):   `#[cfg(feature="rocm")] if device.is_rocm(){return rocm::prepare(device);}`
//! * in `Int8LayerCache::query` / `query_batch` (app/src/model/int8_cache.rs:292-359),
//!   on a ROCm device with `commit == true`: `rocm::commit_append` in place
//!   of `encoded(..)` + the two `LayerCache::query` writes, once the arenas
//!   hold `past + tokens` slots;
//! * in the decode step of `forward_embedding` / `forward_batched_embedding`
//!   (app/src/model/mod.rs:699-720, app/src/model/batch.rs:152-222):
//!   `rocm::decode_step` in place of `query_int8(.., commit = true)` followed
//!   by `int8_kv_ops::attention`, passing the host lengths the batch builder
//!   already holds (batch.rs:152-161) as `past_host`.
//!
//! Every op refuses CPU storage, as the reference's device-only branches do
//! (hip_attention.rs:75); there is no CPU fallback. Calls run on the null HIP
//! stream, the stream the reference's own HIP kernels are launched on
//! (hip_kernel::launch -> HipModule::launch), so they stay ordered with them.

use super::*;
use crate::model::ppk_ffi as ffi;
use crate::model::ppk_ffi::{context, device_context, dtype_code, span, workspace, Bound, STREAM};
use candle_core::{
    backend::BackendStorage, CpuStorage, CustomOp1, CustomOp2, CustomOp3, InplaceOp1, Layout, RocmStorage, Shape,
};
use std::ffi::c_void;

/// History dequantisation of the attention ops. 0 (the default) dequantises
/// every history value in f32, the arithmetic of the fp32-dequantised
/// attention the decode path is specified and measured against;
/// PPK_ATTN_BF16_HISTORY instead rounds each dequantised value to bf16 as
/// the reference kernel's pp_i8_load does (app/src/model/int8_kv.cu:23-27),
/// for bit-level agreement with the CUDA path's own 2e-5 checks, at a higher
/// cost per step (more arithmetic per history byte).
pub const HISTORY: u32 = 0;

// ---- quantize / dequantize -------------------------------------------------

/// int8_kv_ops::quantize: codes and scales in one launch. The codes are the
/// op's output; the scales go into `scales`, allocated by the caller for it.
struct Quantize {
    rows: usize,
    width: usize,
    scales: Tensor,
}

impl CustomOp1 for Quantize {
    fn name(&self) -> &'static str {
        "ppk-int8-quantize"
    }

    fn cpu_fwd(&self, _: &CpuStorage, _: &Layout) -> candle_core::Result<(CpuStorage, Shape)> {
        candle_core::bail!("ROCm INT8 quantize never falls back to CPU")
    }

    fn rocm_fwd(&self, x: &RocmStorage, xl: &Layout) -> candle_core::Result<(RocmStorage, Shape)> {
        use candle_core::backend::BackendDevice;
        let device = x.rocm_device();
        let ctx = context(device.ordinal())?;
        let src_dtype = dtype_code(x.dtype())?;
        let src = span(x, xl, self.rows * self.width, x.dtype().size_in_bytes(), "INT8 KV input")?;
        let mut bound = Bound::new();
        let scales = bound.ptr(&self.scales, DType::F32, "INT8 KV scales")?;
        let shape = xl.shape().clone();
        let mut codes = unsafe { device.alloc_uninit(&shape, DType::U8)? };
        let mut a: ffi::PpkQuantizeArgs = ffi::args();
        a.src_dtype = src_dtype;
        a.src = src;
        a.codes = codes.device_ptr_mut() as *mut u8;
        a.scales = scales as *mut f32;
        a.rows = self.rows as u64;
        a.head_dim = self.width as u32;
        ffi::check(unsafe { ffi::ppk_quantize(ctx, STREAM, &a) })?;
        Ok((codes, shape))
    }
}

/// `input`: dense [heads, tokens, D] in F32, BF16 or F16 (geometry() checked
/// it). Same codes and scales as the reference's Scale + Pack (int8_kv.cu:8-18)
/// from the input's f32 values: widening bf16/f16 to f32 is exact, so the
/// reference's `to_dtype(F32)` is not needed first.
pub(super) fn quantize(input: &Tensor) -> Result<(Tensor, Tensor)> {
    let (h, n, d) = input.dims3()?;
    let scales = Tensor::zeros((h, n), DType::F32, input.device())?;
    let codes = input.apply_op1_no_bwd(&Quantize { rows: h * n, width: d, scales: scales.clone() })?;
    Ok((codes, scales))
}

struct Dequantize {
    rows: usize,
    width: usize,
    dtype: DType,
}

impl CustomOp2 for Dequantize {
    fn name(&self) -> &'static str {
        "ppk-int8-dequantize"
    }

    fn cpu_fwd(&self, _: &CpuStorage, _: &Layout, _: &CpuStorage, _: &Layout) -> candle_core::Result<(CpuStorage, Shape)> {
        candle_core::bail!("ROCm INT8 dequantize never falls back to CPU")
    }

    fn rocm_fwd(
        &self,
        codes: &RocmStorage,
        cl: &Layout,
        scales: &RocmStorage,
        sl: &Layout,
    ) -> candle_core::Result<(RocmStorage, Shape)> {
        use candle_core::backend::BackendDevice;
        let device = codes.rocm_device();
        let ctx = context(device.ordinal())?;
        let shape = cl.shape().clone();
        let mut out = unsafe { device.alloc_uninit(&shape, self.dtype)? };
        let mut a: ffi::PpkDequantizeArgs = ffi::args();
        a.out_dtype = dtype_code(self.dtype)?;
        a.codes = span(codes, cl, self.rows * self.width, 1, "INT8 KV codes")? as *const u8;
        a.scales = span(scales, sl, self.rows, 4, "INT8 KV scales")? as *const f32;
        a.out = out.device_ptr_mut() as *mut c_void;
        a.rows = self.rows as u64;
        a.head_dim = self.width as u32;
        ffi::check(unsafe { ffi::ppk_dequantize(ctx, STREAM, &a) })?;
        Ok((out, shape))
    }
}

/// int8_kv_ops::dequantize: code * scale in f32, then the requested dtype.
/// BF16 and F16 are produced by the kernel with the same round-to-nearest-even
/// as the reference's `to_dtype`; other dtypes convert from the F32 result.
pub(super) fn dequantize(packed: &Tensor, scale: &Tensor, dtype: DType) -> Result<Tensor> {
    let (h, n, d) = packed.dims3()?;
    let direct = matches!(dtype, DType::F32 | DType::BF16 | DType::F16);
    let op = Dequantize { rows: h * n, width: d, dtype: if direct { dtype } else { DType::F32 } };
    let out = packed.apply_op2_no_bwd(scale, &op)?;
    Ok(if direct { out } else { out.to_dtype(dtype)? })
}

// ---- attention and the fused decode step -----------------------------------

/// Attention over the int8 arenas plus the current token (and, for the step,
/// the append of k_new/v_new at slot past[b] first).
struct Attention {
    ks: Tensor,
    vs: Tensor,
    sk: Tensor,
    sv: Tensor,
    past: Tensor,
    new: Option<(Tensor, Tensor, Option<Tensor>)>,
    rows: usize,
    heads: usize,
    capacity: usize,
    width: usize,
    split: usize,
    past_host: Option<Vec<u32>>,
}

impl CustomOp3 for Attention {
    fn name(&self) -> &'static str {
        if self.new.is_some() {
            "ppk-int8-decode-step"
        } else {
            "ppk-int8-attention"
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
        candle_core::bail!("ROCm INT8 attention never falls back to CPU")
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
        let (rows, d) = (self.rows, self.width);
        let mut bound = Bound::new();
        let mut a: ffi::PpkAttentionArgs = ffi::args();
        a.q_dtype = dtype_code(q.dtype())?;
        a.scratch_dtype = dtype_code(self.sk.dtype())?;
        a.out_dtype = ffi::PPK_F32;
        a.flags = HISTORY;
        a.rows = rows as u32;
        a.heads = self.heads as u32;
        a.capacity = self.capacity as u32;
        a.head_dim = d as u32;
        a.split_tokens = self.split as u32;
        a.q = span(q, ql, rows * d, q.dtype().size_in_bytes(), "INT8 attention query")?;
        a.k_codes = span(k, kl, rows * self.capacity * d, 1, "INT8 key arena")? as *const u8;
        a.v_codes = span(v, vl, rows * self.capacity * d, 1, "INT8 value arena")? as *const u8;
        a.k_scales = bound.ptr(&self.ks, DType::F32, "INT8 key scales")? as *const f32;
        a.v_scales = bound.ptr(&self.vs, DType::F32, "INT8 value scales")? as *const f32;
        a.sk = bound.ptr(&self.sk, self.sk.dtype(), "current key")?;
        a.sv = bound.ptr(&self.sv, self.sv.dtype(), "current value")?;
        a.past = bound.ptr(&self.past, DType::U32, "INT8 attention lengths")? as *const u32;
        if let Some(host) = &self.past_host {
            if host.len() != rows / self.heads {
                candle_core::bail!("HIP_PREPARATION: host lengths differ from the batch");
            }
            a.past_host = host.as_ptr();
        }
        let shape: Shape = (rows, 1, d).into();
        let mut out = unsafe { device.alloc_uninit(&shape, DType::F32)? };
        a.out = out.device_ptr_mut() as *mut c_void;
        let mut bytes = 0u64;
        ffi::check(unsafe { ffi::ppk_attention_workspace_bytes(ctx, &a, &mut bytes) })?;
        let mut ws = workspace(device, bytes)?;
        if let Some(ws) = ws.as_mut() {
            a.workspace = ws.device_ptr_mut() as *mut c_void;
            a.workspace_bytes = bytes;
        }
        match &self.new {
            None => ffi::check(unsafe { ffi::ppk_decode_attention(ctx, STREAM, &a) })?,
            Some((k_new, v_new, flags)) => {
                let mut s: ffi::PpkDecodeStepArgs = ffi::args();
                s.new_dtype = dtype_code(k_new.dtype())?;
                s.k_new = bound.ptr(k_new, k_new.dtype(), "new key")?;
                s.v_new = bound.ptr(v_new, k_new.dtype(), "new value")?;
                if let Some(flags) = flags {
                    s.flags = bound.ptr(flags, DType::U32, "step flags")? as *mut u32;
                }
                s.attn = a;
                ffi::check(unsafe { ffi::ppk_decode_step(ctx, STREAM, &s) })?;
            }
        }
        // `ws` is released when the op returns, as the reference releases its
        // `partial` buffer (hip_attention.rs:87-110).
        Ok((out, shape))
    }
}

fn attention_shape(q: &Tensor, k: &Tensor, sk: &Tensor, past: &Tensor, heads: usize) -> Result<(usize, usize, usize)> {
    let (rows, capacity, width) = k.dims3()?;
    ensure!(matches!(width, 64 | 128 | 256), "INT8 attention head width must be 64, 128 or 256");
    ensure!(heads > 0 && rows % heads == 0, "INT8 attention geometry differs");
    ensure!(q.dims() == [rows, 1, width] && sk.dims() == [rows, 1, width], "INT8 scratch must be [head_rows,1,D]");
    ensure!(past.dims() == [rows / heads] && past.dtype() == DType::U32, "INT8 attention lengths differ");
    Ok((rows, capacity, width))
}

/// int8_kv_ops::attention (int8_kv_ops.rs:41-55) in one or two launches.
/// Unlike the reference, D may be 64, 128 or 256 and capacity is not capped at
/// 1024; `split_tokens` is a hint (the result does not depend on it, as the
/// reference's does not). `past_host` (optional) is the host copy of `past`.
#[allow(clippy::too_many_arguments)]
pub(super) fn attention(
    q: &Tensor,
    k: &Tensor,
    v: &Tensor,
    ks: &Tensor,
    vs: &Tensor,
    sk: &Tensor,
    sv: &Tensor,
    past: &Tensor,
    heads: usize,
    split_tokens: usize,
    past_host: Option<&[u32]>,
) -> Result<Tensor> {
    let (rows, capacity, width) = attention_shape(q, k, sk, past, heads)?;
    let op = Attention {
        ks: ks.clone(),
        vs: vs.clone(),
        sk: sk.clone(),
        sv: sv.clone(),
        past: past.clone(),
        new: None,
        rows,
        heads,
        capacity,
        width,
        split: split_tokens,
        past_host: past_host.map(<[u32]>::to_vec),
    };
    Ok(q.apply_op3_no_bwd(k, v, &op)?)
}

/// One decode step (mod.rs:699-705, batch.rs:152-222): quantise k_new/v_new
/// ([rows, 1, D], the current token) into slot past[b] of the arenas k/v and
/// ks/vs, then attend over [0, past[b]) plus the unquantised current token
/// sk/sv; the same result as `query_int8(.., commit = true)` followed by
/// `attention`. The arenas are written in place: they must be the caller's
/// alone (an Int8LayerCache's own storage, not a shared snapshot). A row at
/// its capacity is not appended and sets PPK_FLAG_OVERFLOW in `flags`
/// (optional U32[1]).
#[allow(clippy::too_many_arguments)]
pub(super) fn decode_step(
    q: &Tensor,
    k: &Tensor,
    v: &Tensor,
    ks: &Tensor,
    vs: &Tensor,
    k_new: &Tensor,
    v_new: &Tensor,
    sk: &Tensor,
    sv: &Tensor,
    past: &Tensor,
    past_host: Option<&[u32]>,
    heads: usize,
    flags: Option<&Tensor>,
) -> Result<Tensor> {
    let (rows, capacity, width) = attention_shape(q, k, sk, past, heads)?;
    ensure!(k_new.dims() == [rows, 1, width] && v_new.dims() == k_new.dims(), "INT8 step tokens must be [head_rows,1,D]");
    let op = Attention {
        ks: ks.clone(),
        vs: vs.clone(),
        sk: sk.clone(),
        sv: sv.clone(),
        past: past.clone(),
        new: Some((k_new.clone(), v_new.clone(), flags.cloned())),
        rows,
        heads,
        capacity,
        width,
        split: 0,
        past_host: past_host.map(<[u32]>::to_vec),
    };
    Ok(q.apply_op3_no_bwd(k, v, &op)?)
}

// ---- commit-append into the arenas -----------------------------------------

/// The commit of Int8LayerCache::query / query_batch (int8_cache.rs:292-359):
/// quantise `tokens` new K/V tokens per row and write codes and scales at
/// slots past[b] .. past[b] + tokens of the arenas, in one launch. Applied in
/// place to the key-code arena; the other three arenas are written through
/// the same call.
struct CommitAppend {
    v_codes: Tensor,
    k_scales: Tensor,
    v_scales: Tensor,
    k_src: Tensor,
    v_src: Tensor,
    past: Tensor,
    batch: usize,
    heads: usize,
    tokens: usize,
    width: usize,
    capacity: usize,
}

impl InplaceOp1 for CommitAppend {
    fn name(&self) -> &'static str {
        "ppk-int8-commit-append"
    }

    fn cpu_fwd(&self, _: &mut CpuStorage, _: &Layout) -> candle_core::Result<()> {
        candle_core::bail!("ROCm INT8 commit never falls back to CPU")
    }

    fn rocm_fwd(&self, k_codes: &mut RocmStorage, layout: &Layout) -> candle_core::Result<()> {
        let device = k_codes.rocm_device();
        let ctx = context(device.ordinal())?;
        let rows = self.batch * self.heads;
        let mut bound = Bound::new();
        let mut a: ffi::PpkAppendArgs = ffi::args();
        a.src_dtype = dtype_code(self.k_src.dtype())?;
        a.k_src = bound.ptr(&self.k_src, self.k_src.dtype(), "INT8 commit keys")?;
        a.v_src = bound.ptr(&self.v_src, self.k_src.dtype(), "INT8 commit values")?;
        a.past = bound.ptr(&self.past, DType::U32, "INT8 commit lengths")? as *const u32;
        a.k_codes = span(k_codes, layout, rows * self.capacity * self.width, 1, "INT8 key arena")? as *mut u8;
        a.v_codes = bound.ptr(&self.v_codes, DType::U8, "INT8 value arena")? as *mut u8;
        a.k_scales = bound.ptr(&self.k_scales, DType::F32, "INT8 key scale arena")? as *mut f32;
        a.v_scales = bound.ptr(&self.v_scales, DType::F32, "INT8 value scale arena")? as *mut f32;
        a.batch = self.batch as u32;
        a.heads = self.heads as u32;
        a.tokens = self.tokens as u32;
        a.head_dim = self.width as u32;
        a.capacity = self.capacity as u32;
        ffi::check(unsafe { ffi::ppk_quantize_append(ctx, STREAM, &a) })
    }
}

/// Quantise and commit k/v ([batch, heads, tokens, D] in F32/BF16/F16) into
/// the arenas (codes [batch*heads, capacity, D] U8, scales [batch*heads,
/// capacity] F32) at slot past[b] (device U32[batch]). The caller has checked
/// past[b] + tokens <= capacity on the host, as LayerCache does before a write
/// (cache.rs:122-154); a row that would still overflow is left unwritten.
/// The four arenas are distinct tensors (Candle holds the key arena's write
/// lock while the op runs and read-locks the others).
#[allow(clippy::too_many_arguments)]
pub(super) fn commit_append(
    k_codes: &Tensor,
    v_codes: &Tensor,
    k_scales: &Tensor,
    v_scales: &Tensor,
    k: &Tensor,
    v: &Tensor,
    past: &Tensor,
) -> Result<()> {
    let (batch, heads, tokens, width) = k.dims4()?;
    let (rows, capacity, arena_width) = k_codes.dims3()?;
    ensure!(rows == batch * heads && arena_width == width, "INT8 commit arena differs from the tokens");
    ensure!(v_codes.dims() == k_codes.dims() && v.dims() == k.dims(), "INT8 commit K/V shapes differ");
    ensure!(k_scales.dims() == [rows, capacity] && v_scales.dims() == [rows, capacity], "INT8 commit scales differ");
    ensure!(past.dims() == [batch] && past.dtype() == DType::U32, "INT8 commit lengths differ");
    let op = CommitAppend {
        v_codes: v_codes.clone(),
        k_scales: k_scales.clone(),
        v_scales: v_scales.clone(),
        k_src: k.contiguous()?,
        v_src: v.contiguous()?,
        past: past.clone(),
        batch,
        heads,
        tokens,
        width,
        capacity,
    };
    Ok(k_codes.inplace_op1(&op)?)
}

// ---- prepare -----------------------------------------------------------------

/// int8_kv_ops::prepare (int8_kv_ops.rs:57-103): the same three known-answer
/// checks (quantise round trip within 0.009; two-row attention and the
/// offset / multi-head / unequal-length / split case within 2e-5 of an f32
/// softmax over bf16-rounded history), plus their f32-history twins, run on
/// the device by the library. A mismatch fails naming the check that failed.
pub(super) fn prepare(device: &Device) -> Result<()> {
    let ctx = device_context(device)?;
    let status = unsafe { ffi::ppk_prepare(ctx) };
    if status == ffi::PPK_INVALID_OUTPUT {
        bail!("{}", ffi::last_error());
    }
    Ok(ffi::check(status)?)
}
