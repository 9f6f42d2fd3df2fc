// iq2xxs_kernels.h — internal launcher interface between the C ABI (cmk_iq2.cpp)
// and the HIP kernels.  Not part of the public ABI (include/cmk_iq2.h).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace cmk {

// dtype / output kind codes shared with the ABI: 0 = f32, 1 = f16, 2 = bf16.

// Dense dequantisation, out[out_dim, in_dim].  Needs 8-byte aligned
// weight_bytes and 2-byte aligned weight_scales.
hipError_t launch_iq2xxs_dequant(const uint8_t* wb, const uint8_t* ws, void* out, int out_kind,
                                 uint32_t out_dim, uint32_t in_dim, int num_cus,
                                 hipStream_t stream);

// Decode-shaped matmul (int8-MFMA GEMV), any m: the one-row kernel for m = 1,
// the multi-row kernel on groups of up to 16 rows (W8A8: 32) otherwise; shapes where
// gemv_supported() holds (m = 1: K up to about 31000; weights and x below
// 2 GB).  Needs 16-byte aligned weight_bytes and 2-byte aligned weight_scales.
// gate non-null: out = silu(gate) * (x . w) with gate [m, out_dim] f32 (not
// overlapping out), the gated MLP step in the epilogue.
// split_ws: workspace of the multi-row kernel's split over K (16-byte
// aligned, split_ws_bytes >= gemv_rows_split_bytes(m, ...)); without it the
// kernel runs unsplit.
bool gemv_supported(uint32_t m, uint32_t out_dim, uint32_t in_dim, int x_dtype);
hipError_t launch_iq2xxs_gemv(const void* x, int x_dtype, uint32_t m, const uint8_t* wb,
                              const uint8_t* ws, float* out, uint32_t out_dim, uint32_t in_dim,
                              bool w8a8, int num_cus, hipStream_t stream,
                              const float* gate = nullptr, void* split_ws = nullptr,
                              size_t split_ws_bytes = 0);
// The multi-row kernel alone (1 <= m <= 16; W8A8: 1 <= m <= 32).
bool gemv_rows_supported(uint32_t m, uint32_t out_dim, uint32_t in_dim, int x_dtype,
                         bool w8a8 = false);
hipError_t launch_iq2xxs_gemv_rows(const void* x, int x_dtype, uint32_t m, const uint8_t* wb,
                                   const uint8_t* ws, float* out, uint32_t out_dim,
                                   uint32_t in_dim, bool w8a8, int num_cus, hipStream_t stream,
                                   const float* gate = nullptr, void* split_ws = nullptr,
                                   size_t split_ws_bytes = 0);
// Workspace bytes the multi-row kernel's split over K uses for m rows (any
// m: launches of up to 16 rows, W8A8 32, share it one after another) on
// num_cus CUs; 0 where it does not split (m = 1, or the row groups fill the
// CUs).  Any format: the split depends on the shape only.
size_t gemv_rows_split_bytes(uint32_t m, uint32_t out_dim, uint32_t in_dim, bool w8a8,
                             int num_cus);

// W8A8 per-row inverse scale: inv[r] = 127 / max|x_r| (1 when max < 1e-8).
hipError_t launch_iq2xxs_row_inv_scale(const void* x, int x_dtype, uint32_t m, uint32_t in_dim,
                                       float* inv_out, hipStream_t stream);

// Portable matmul for any alignment / shape (one wave per output row).
// row_inv: W8A8 per-row scales (from launch_iq2xxs_row_inv_scale) or null.
hipError_t launch_iq2xxs_matmul_simple(const void* x, int x_dtype, uint32_t m, const uint8_t* wb,
                                       const uint8_t* ws, float* out, uint32_t out_dim,
                                       uint32_t in_dim, const float* row_inv, int num_cus,
                                       hipStream_t stream);

// Prefill matmul (MFMA GEMM, weights dequantised into LDS as f16);
// x_dtype 0 (f32), 1 (f16) or 2 (bf16), on shapes where gemm_supported() holds
// (in_dim % 8 == 0, x and weights below 2 GB).  Needs 16-byte aligned x and
// weight_bytes and 2-byte aligned weight_scales.
// With row_inv non-null the activations are first written to xq (16-byte
// aligned) as f16 from v = x * row_inv[r], and each output row is divided by
// row_inv[r]:
//  - w8a8: q = clamp(round_half_away(v), +-127) (exact in f16), inv from
//    launch_iq2xxs_row_inv_scale; xq holds gemm_w8a8_scratch_bytes (f16 /
//    bf16 x) or gemm_f32_scratch_bytes(m, in_dim, true) (f32 x);
//  - bf16 x without w8a8: the launch writes row_inv[r] = 2^(14 - floor(log2
//    max|x_r|)) itself and stages v as f16 (exact); xq holds
//    gemm_w8a8_scratch_bytes;
//  - f32 x without w8a8: row_inv as for bf16; row r is staged as the f16 head
//    rne(v) and tail rne(v - head), two GEMM rows whose products are summed in
//    the epilogue; xq holds gemm_f32_scratch_bytes(m, in_dim, false), and
//    gemm_supported must hold for 2m rows.
// f32 and bf16 x always need row_inv and xq.
bool gemm_supported(uint32_t m, uint32_t out_dim, uint32_t in_dim);
size_t gemm_w8a8_scratch_bytes(uint32_t m, uint32_t in_dim);
size_t gemm_f32_scratch_bytes(uint32_t m, uint32_t in_dim, bool w8a8);
// Shapes whose tiles cannot fill the GPU split k over grid z; the launch then
// writes partial products to `partials` (this many bytes, 16-byte aligned; 0 =
// no split, partials may be null) and sums them into out in split order.
// rows: GEMM rows (2m for staged f32 pairs), out_rows: rows of out (m).
size_t gemm_split_scratch_bytes(uint32_t rows, uint32_t out_rows, uint32_t out_dim,
                                uint32_t in_dim);
hipError_t launch_iq2xxs_gemm(const void* x, int x_dtype, uint32_t m, const uint8_t* wb,
                              const uint8_t* ws, float* out, uint32_t out_dim, uint32_t in_dim,
                              const float* row_inv, void* xq, bool w8a8, float* partials,
                              hipStream_t stream);

// IQ2_XS (1), IQ2_S (2), IQ3_S (3): bytes / scales per 256-weight block
// (0 for any other variant), and the portable matmul (any m, any alignment;
// row_inv as for the simple path) and dequantisation of those formats.
size_t variant_bytes_per_block(int variant);
size_t variant_scales_per_block(int variant);
hipError_t launch_iq_variant_matmul(int variant, const void* x, int x_dtype, uint32_t m,
                                    const uint8_t* wb, const uint8_t* ws, float* out,
                                    uint32_t out_dim, uint32_t in_dim, const float* row_inv,
                                    int num_cus, hipStream_t stream);
// The multi-row decode kernel for IQ2_XS (1), IQ2_S (2), IQ3_S (3): any m, in
// launches of up to 16 rows (W8A8: 32, int8 activations; row scales computed in
// the kernel).  Needs
// weight_bytes 16-byte and weight_scales 2-byte aligned.
// IQ2_XS (variant 1), IQ2_S (2) and IQ3_S (3) at m = 1 on the one-row GEMV
// (iq2xxs_gemv.hip): whether the launch fits (alignment of x and the weight
// buffers, K in whole 1024-column slices, one chunk per workgroup), and the
// launch.
bool iq_variant_gemv_fits(int variant, const void* x, const uint8_t* wb, const uint8_t* ws,
                          uint32_t out_dim, uint32_t in_dim, int x_dtype, int num_cus);
hipError_t launch_iq_variant_gemv(int variant, const void* x, int x_dtype, const uint8_t* wb,
                                  const uint8_t* ws, float* out, uint32_t out_dim,
                                  uint32_t in_dim, bool w8a8, int num_cus, hipStream_t stream);
bool variant_rows_supported(int variant, uint32_t out_dim, uint32_t in_dim, int x_dtype);
hipError_t launch_iq_variant_rows(int variant, const void* x, int x_dtype, uint32_t m,
                                  const uint8_t* wb, const uint8_t* ws, float* out,
                                  uint32_t out_dim, uint32_t in_dim, bool w8a8, int num_cus,
                                  hipStream_t stream, void* split_ws = nullptr,
                                  size_t split_ws_bytes = 0);
hipError_t launch_iq_variant_dequant(int variant, const uint8_t* wb, const uint8_t* ws, void* out,
                                     int out_kind, uint32_t out_dim, uint32_t in_dim, int num_cus,
                                     hipStream_t stream);

// GGUF (ggml) blocks of code_bytes + scale_bytes bytes each -> weight_bytes
// (codes) and weight_scales (d, then the packed scales).  Any alignment.
hipError_t launch_gguf_split(const uint8_t* blocks, uint64_t n_blocks, uint32_t code_bytes,
                             uint32_t scale_bytes, uint8_t* wb, uint8_t* ws, int num_cus,
                             hipStream_t stream);

// h[i] = silu(gate[i]) * up[i] for i < n, written as f32 (out_kind 0), f16 (1)
// or bf16 (2).  Any alignment.
hipError_t launch_swiglu(const float* gate, const float* up, void* out, int out_kind, uint64_t n,
                         int num_cus, hipStream_t stream);

}  // namespace cmk
