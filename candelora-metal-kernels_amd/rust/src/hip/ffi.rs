// Rust FFI of libcmk_iq2.so (include/cmk_iq2.h) for the `rocm` feature of
// candelora-metal-kernels: to be added as src/hip/ffi.rs.  Not built in this
// repository (no Rust toolchain in the build image); the C ABI it binds is
// tested through ctypes (tests/test_abi.py) and the C++ host layer.
use std::ffi::{c_char, c_int, c_void, CStr};

#[repr(C)] #[derive(Clone, Copy)] pub enum CmkDtype { F32 = 0, F16 = 1, BF16 = 2 }
#[repr(C)] #[derive(Clone, Copy)] pub enum CmkVariant { Iq2Xxs = 0, Iq2Xs = 1, Iq2S = 2, Iq3S = 3 }
#[repr(C)] #[derive(Clone, Copy)] pub enum CmkActQuant { Off = 0, W8A8 = 1, W4A8 = 2 }

#[link(name = "cmk_iq2")]
extern "C" {
    pub fn cmk_iq2_matmul(x: *const c_void, x_dtype: CmkDtype, x_len: usize, m: usize,
                          weight_bytes: *const u8, weight_bytes_len: usize,
                          weight_scales: *const u8, weight_scales_len: usize,
                          out_dim: usize, in_dim: usize, variant: CmkVariant,
                          mode: CmkActQuant, strict: c_int, out: *mut f32,
                          workspace: *mut c_void, workspace_bytes: usize,
                          stream: *mut c_void) -> c_int;
    pub fn cmk_iq2_matmul_noalloc(x: *const c_void, x_dtype: CmkDtype, x_len: usize, m: usize,
                                  weight_bytes: *const u8, weight_bytes_len: usize,
                                  weight_scales: *const u8, weight_scales_len: usize,
                                  out_dim: usize, in_dim: usize, variant: CmkVariant,
                                  mode: CmkActQuant, strict: c_int, out: *mut f32,
                                  stream: *mut c_void) -> c_int;
    pub fn cmk_iq2_matmul_workspace_size(x_dtype: CmkDtype, m: usize, out_dim: usize,
                                         in_dim: usize, variant: CmkVariant,
                                         mode: CmkActQuant, bytes: *mut usize) -> c_int;
    pub fn cmk_iq2_dequantize(weight_bytes: *const u8, weight_bytes_len: usize,
                              weight_scales: *const u8, weight_scales_len: usize,
                              out_dim: usize, in_dim: usize, variant: CmkVariant,
                              out_dtype: CmkDtype, out: *mut c_void,
                              stream: *mut c_void) -> c_int;
    pub fn cmk_swiglu(gate: *const f32, up: *const f32, n: usize, out_dtype: CmkDtype,
                      out: *mut c_void, stream: *mut c_void) -> c_int;
    pub fn cmk_iq2_matmul_swiglu(x: *const c_void, x_dtype: CmkDtype, x_len: usize, m: usize,
                                 weight_bytes: *const u8, weight_bytes_len: usize,
                                 weight_scales: *const u8, weight_scales_len: usize,
                                 out_dim: usize, in_dim: usize, gate: *const f32,
                                 gate_len: usize, out: *mut f32, workspace: *mut c_void,
                                 workspace_bytes: usize, stream: *mut c_void) -> c_int;
    pub fn cmk_iq2_split_gguf_blocks(blocks: *const u8, blocks_len: usize, n_blocks: usize,
                                     variant: CmkVariant, weight_bytes: *mut u8,
                                     weight_bytes_len: usize, weight_scales: *mut u8,
                                     weight_scales_len: usize, stream: *mut c_void) -> c_int;
    pub fn cmk_last_error() -> *const c_char;
    pub fn cmk_abi_version() -> c_int;
    pub fn cmk_malloc(ptr: *mut *mut c_void, bytes: usize) -> c_int;
    pub fn cmk_free(ptr: *mut c_void) -> c_int;
    pub fn cmk_memcpy_htod(dst: *mut c_void, src: *const c_void, bytes: usize, s: *mut c_void) -> c_int;
    pub fn cmk_memcpy_dtoh(dst: *mut c_void, src: *const c_void, bytes: usize, s: *mut c_void) -> c_int;
    pub fn cmk_stream_synchronize(s: *mut c_void) -> c_int;
}

pub fn check(rc: c_int) -> candle_core::Result<()> {
    if rc == 0 { return Ok(()); }
    let msg = unsafe { CStr::from_ptr(cmk_last_error()) }.to_string_lossy().into_owned();
    Err(candle_core::Error::msg(msg))
}
