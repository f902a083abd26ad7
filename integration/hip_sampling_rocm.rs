//! The ROCm body of the CFG + Rényi sampler op (app/src/inference/hip_sampling.rs)
//! over the MI355X library `libppk.so`: `HipSampler::rocm_fwd` (:120-214)
//! without the hiprtc module load and kernel launch, one `ppk_renyi_sample`
//! call instead. Validation (`validate`, :18-69), the op's shape and its
//! [3, batch] U32 output (tokens, valid flags, supports) are unchanged.
//!
//! Install: copy this file to `app/src/inference/hip_sampling_rocm.rs` (and
//! `ppk_ffi.rs` to `app/src/model/ppk_ffi.rs`); in hip_sampling.rs declare
//! `#[cfg(feature = "rocm")] #[path = "hip_sampling_rocm.rs"] mod rocm;` and
//! make the body of `rocm_fwd`
//! `rocm::rocm_fwd(self, raw, raw_layout, uniforms, uniform_layout, bounds, bounds_layout)`.
//! As a child module it reads the private fields of `HipSampler`.

use crate::model::ppk_ffi as ffi;
use crate::model::ppk_ffi::{context, span, STREAM};
use candle_core::{backend::BackendStorage, DType, Layout, RocmStorage, Shape};

/// The sampler over `raw` [batch * guidance, choices] F32, `uniforms`
/// [batch, 1] F32 and `bounds` [batch, 2] U32 (contiguous, view offsets
/// allowed, as `validate` required): one block per logical row; bad device
/// values give valid = 0 and the reference's placeholder token.
pub(super) fn rocm_fwd(
    op: &super::HipSampler,
    raw: &RocmStorage,
    raw_layout: &Layout,
    uniforms: &RocmStorage,
    uniform_layout: &Layout,
    bounds: &RocmStorage,
    bounds_layout: &Layout,
) -> candle_core::Result<(RocmStorage, Shape)> {
    use candle_core::backend::BackendDevice;
    let device = raw.rocm_device();
    let ctx = context(device.ordinal())?;
    let mut a: ffi::PpkRenyiSampleArgs = ffi::args();
    a.batch = op.batch as u32;
    a.choices = op.choices as u32;
    a.guidance = op.guidance as u32;
    a.alpha = op.alpha;
    a.cfg = op.cfg;
    a.token_offset = op.offset;
    a.raw = span(raw, raw_layout, op.batch * op.guidance * op.choices, 4, "HIP sampler raw logits")? as *const f32;
    a.uniforms = span(uniforms, uniform_layout, op.batch, 4, "HIP sampler uniforms")? as *const f32;
    a.bounds = span(bounds, bounds_layout, op.batch * 2, 4, "HIP sampler bounds")? as *const u32;
    let shape: Shape = (3usize, op.batch).into();
    // The kernel writes all three cells of every row on every path.
    let mut output = unsafe { device.alloc_uninit(&shape, DType::U32)? };
    a.out = output.device_ptr_mut() as *mut u32;
    ffi::check(unsafe { ffi::ppk_renyi_sample(ctx, STREAM, &a) })?;
    Ok((output, shape))
}
