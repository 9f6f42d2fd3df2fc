// The `rocm` bodies of the two private entry points of src/iq2_matmul.rs
// (iq2_matmul_metal, src/iq2_matmul.rs:197-365, and
// iq2_dequantize_to_f16_metal, :367-505), to be added as src/hip/mod.rs and
// declared in src/iq2_matmul.rs as
//     #[cfg(feature = "rocm")] #[path = "hip/mod.rs"] mod hip;
// so that they see the module's private items (parse_x_shape) as a child
// module.  The call sites dispatch on the feature:
//     #[cfg(feature = "rocm")] return hip::iq2_matmul_rocm(x, weight_bytes, ...);
// The checks and error texts are the reference's (:170-311); candle has no
// ROCm device, so CPU tensors are staged through device buffers of the C ABI.
// Not built in this repository (no Rust toolchain in the build image).
pub mod ffi;

use super::{parse_x_shape, Iq2MatmulVariant};
use crate::activation_quant::ActivationQuantMode;
use candle_core::{DType, Result, Tensor};

/// A device buffer from the C ABI's allocator, freed on drop.
struct DevBuf(*mut std::ffi::c_void);
impl DevBuf {
    fn new(bytes: usize) -> Result<Self> {
        let mut p = std::ptr::null_mut();
        ffi::check(unsafe { ffi::cmk_malloc(&mut p, bytes.max(1)) })?;
        Ok(DevBuf(p))
    }
    fn upload<T: Copy>(host: &[T]) -> Result<Self> {
        let bytes = std::mem::size_of_val(host);
        let b = Self::new(bytes)?;
        ffi::check(unsafe {
            ffi::cmk_memcpy_htod(b.0, host.as_ptr().cast(), bytes, std::ptr::null_mut())
        })?;
        Ok(b)
    }
}
impl Drop for DevBuf { fn drop(&mut self) { unsafe { ffi::cmk_free(self.0); } } }

pub(super) fn iq2_matmul_rocm(x: &Tensor, weight_bytes: &Tensor, weight_scales: &Tensor, out_dim: usize,
                   in_dim: usize, variant: Iq2MatmulVariant,
                   activation_quant_mode: ActivationQuantMode) -> Result<Tensor> {
    use self::ffi::*;
    if out_dim == 0 || in_dim == 0 { candle_core::bail!("iq2_matmul expects non-zero dimensions") }
    if weight_bytes.dtype() != DType::U8 || weight_scales.dtype() != DType::U8 {
        candle_core::bail!("iq2_matmul expects U8 weight bytes/scales, got bytes={:?}, scales={:?}",
                           weight_bytes.dtype(), weight_scales.dtype());
    }
    let (x2, m, squeeze_out) = parse_x_shape(x, in_dim)?;
    // candle has no ROCm device: the tensors live on the CPU and are staged here (a serving loop
    // keeps the weights resident, keyed by storage id and offset, and reuses one workspace)
    let (xd, xbuf) = match x2.dtype() {
        DType::F32 => (CmkDtype::F32, DevBuf::upload(&x2.flatten_all()?.to_vec1::<f32>()?)?),
        DType::F16 => (CmkDtype::F16, DevBuf::upload(&x2.flatten_all()?.to_vec1::<half::f16>()?)?),
        DType::BF16 => (CmkDtype::BF16, DevBuf::upload(&x2.flatten_all()?.to_vec1::<half::bf16>()?)?),
        dt => candle_core::bail!("iq2_matmul unsupported x dtype: {:?}", dt),
    };
    let wb = weight_bytes.flatten_all()?.to_vec1::<u8>()?;
    let ws = weight_scales.flatten_all()?.to_vec1::<u8>()?;
    let (wbuf, sbuf) = (DevBuf::upload(&wb)?, DevBuf::upload(&ws)?);
    let mode = match activation_quant_mode {
        ActivationQuantMode::Off => CmkActQuant::Off,
        ActivationQuantMode::W8A8 => CmkActQuant::W8A8,
        ActivationQuantMode::W4A8 => candle_core::bail!("W4A8 kernel path is not implemented yet"),
    };
    let var = variant as u32 as i32; // the reference's variant order is the ABI's
    let var: CmkVariant = unsafe { std::mem::transmute(var) };
    let mut ws_bytes = 0usize;
    check(unsafe { cmk_iq2_matmul_workspace_size(xd, m, out_dim, in_dim, var, mode, &mut ws_bytes) })?;
    let work = if ws_bytes > 0 { Some(DevBuf::new(ws_bytes)?) } else { None };
    let out_len = m.checked_mul(out_dim)
        .ok_or_else(|| candle_core::Error::msg("iq2_matmul output size overflow"))?;
    let obuf = DevBuf::new(out_len * 4)?;
    check(unsafe {
        cmk_iq2_matmul(xbuf.0, xd, m * in_dim, m, wbuf.0.cast(), wb.len(), sbuf.0.cast(), ws.len(),
                       out_dim, in_dim, var, mode, 0, obuf.0.cast(),
                       work.as_ref().map_or(std::ptr::null_mut(), |w| w.0), ws_bytes,
                       std::ptr::null_mut())
    })?;
    let mut host = vec![0f32; out_len];
    check(unsafe { cmk_memcpy_dtoh(host.as_mut_ptr().cast(), obuf.0, out_len * 4, std::ptr::null_mut()) })?;
    check(unsafe { cmk_stream_synchronize(std::ptr::null_mut()) })?;
    let out = Tensor::from_vec(host, (m, out_dim), x.device())?;
    if squeeze_out { out.squeeze(0) } else { Ok(out) }
}

pub(super) fn iq2_dequantize_to_f16_rocm(weight_bytes: &Tensor, weight_scales: &Tensor, out_dim: usize,
                              in_dim: usize, variant: Iq2MatmulVariant) -> Result<Tensor> {
    use self::ffi::*;
    if out_dim == 0 || in_dim == 0 {
        candle_core::bail!("iq2_dequantize_to_f16 expects non-zero dimensions")
    }
    let wb = weight_bytes.flatten_all()?.to_vec1::<u8>()?;
    let ws = weight_scales.flatten_all()?.to_vec1::<u8>()?;
    let (wbuf, sbuf) = (DevBuf::upload(&wb)?, DevBuf::upload(&ws)?);
    let n = out_dim.checked_mul(in_dim)
        .ok_or_else(|| candle_core::Error::msg("iq2_dequantize_to_f16 output size overflow"))?;
    let obuf = DevBuf::new(n * 2)?;
    let var: CmkVariant = unsafe { std::mem::transmute(variant as u32 as i32) };
    check(unsafe {
        cmk_iq2_dequantize(wbuf.0.cast(), wb.len(), sbuf.0.cast(), ws.len(), out_dim, in_dim, var,
                           CmkDtype::F16, obuf.0, std::ptr::null_mut())
    })?;
    let mut host = vec![half::f16::ZERO; n];
    check(unsafe { cmk_memcpy_dtoh(host.as_mut_ptr().cast(), obuf.0, n * 2, std::ptr::null_mut()) })?;
    check(unsafe { cmk_stream_synchronize(std::ptr::null_mut()) })?;
    Tensor::from_vec(host, (out_dim, in_dim), weight_bytes.device())
}
