/*
 * cmk_iq2.h — C ABI of the MI355X (gfx950) IQ2 matmul library, libcmk_iq2.so.
 *
 * This is the drop-in boundary for the crate candelora-metal-kernels: the
 * crate keeps its public Rust API (module candelora_metal_kernels::iq2_matmul,
 * src/iq2_matmul.rs:31-37,535-670; candelora_metal_kernels::activation_quant,
 * src/activation_quant.rs:7-44) and, under a `rocm` cargo feature, its bodies
 * call the entry points below instead of the Metal dispatch helpers
 * iq2_matmul_metal (src/iq2_matmul.rs:197-365) and
 * iq2_dequantize_to_f16_metal (src/iq2_matmul.rs:367-505).
 *
 * Conventions
 *  - Plain pointers and sizes only.  Device pointers are HIP device memory
 *    (from cmk_device_malloc or any hipMalloc'd buffer); `stream` is a
 *    hipStream_t passed as void* (NULL = the default stream).
 *  - Launch entry points are asynchronous on `stream` and never allocate
 *    device memory.  Callers synchronise (cmk_stream_synchronize), the same
 *    contract as the reference's encoder-based dispatch, whose callers call
 *    device.synchronize() (src/iq2_matmul.rs:1101).
 *  - Return value: CMK_OK (0) or a negative cmk_status.  On error the
 *    message is available from cmk_last_error() (thread-local, valid until the
 *    next call on the same thread).  Message texts follow the reference's
 *    bail! texts (src/iq2_matmul.rs:210-311,367-433).
 *  - Thread safety: entry points may be called concurrently from several
 *    host threads; launches on the same stream are ordered by that stream.
 */
#ifndef CMK_IQ2_H
#define CMK_IQ2_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 2: cmk_iq2_matmul_noalloc and cmk_iq2_matmul_swiglu exported; f32 x at 9-16
 * rows and W8A8 at 17-32 rows run on the multi-row decode kernel, with the
 * workspace sizes that follow from it.
 * 3: the multi-row decode kernel splits K over several workgroups when its
 * row groups leave CUs idle, in an optional workspace that
 * cmk_iq2_matmul_workspace_size now reports (m >= 2, N <= 4096 on 256 CUs);
 * cmk_iq2_matmul_swiglu takes a workspace. */
#define CMK_IQ2_ABI_VERSION 3

/* Status codes. */
typedef enum cmk_status {
    CMK_OK = 0,
    CMK_ERR_INVALID_ARGUMENT = -1, /* shape/size/dtype contract violated */
    CMK_ERR_UNSUPPORTED = -2,      /* a variant or mode this build does not implement */
    CMK_ERR_HIP = -3,              /* a HIP runtime call failed */
    CMK_ERR_NO_DEVICE = -4         /* no usable gfx950 device */
} cmk_status;

/* Element types of x / the dequantized output.  Mirrors the candle DTypes the
 * reference accepts for x: F32, F16, BF16 (src/iq2_matmul.rs:59-75). */
typedef enum cmk_dtype { CMK_F32 = 0, CMK_F16 = 1, CMK_BF16 = 2 } cmk_dtype;

/* Iq2MatmulVariant (src/iq2_matmul.rs:31-37).  All four are implemented.  IQ2_XXS
 * runs on the one-row GEMV (m = 1; 2-4 rows where out_dim <= 16 per CU, 2 rows
 * also at larger out_dim when in_dim <= 4096), the multi-row decode kernel (up
 * to 16 rows per launch, W8A8 32) and the MFMA GEMM (larger m).  IQ2_XS / IQ2_S /
 * IQ3_S run on the one-row GEMV at m = 1 and on the multi-row decode kernel
 * otherwise when the buffers are aligned (weight_bytes 16-byte or 8-byte,
 * weight_scales 2-byte), and on a byte-load kernel for any other alignment.
 * Bytes / scales per 256-weight block: 64/2, 64/10, 72/10, 104/6
 * (src/iq2_matmul.rs:13-29). */
typedef enum cmk_iq2_variant {
    CMK_IQ2_XXS = 0,
    CMK_IQ2_XS = 1,
    CMK_IQ2_S = 2,
    CMK_IQ3_S = 3
} cmk_iq2_variant;

/* ActivationQuantMode (src/activation_quant.rs:7-15). */
typedef enum cmk_act_quant_mode {
    CMK_ACT_QUANT_OFF = 0,
    CMK_ACT_QUANT_W8A8 = 1,
    CMK_ACT_QUANT_W4A8 = 2
} cmk_act_quant_mode;

/* ------------------------------------------------------------------------ */
/* Launch entry points                                                       */
/* ------------------------------------------------------------------------ */

/*
 * out[m, out_dim] (fp32) = x[m, in_dim] . W^T, W the matrix [out_dim, in_dim]
 * in format `variant`, held as the reference's split super-blocks:
 *   weight_bytes : out_dim * ceil(in_dim/256) blocks x bytes_per_block
 *                  (IQ2_XXS: 64 B, 32 x u16 qs)
 *   weight_scales: out_dim * ceil(in_dim/256) blocks x scales_per_block
 *                  (IQ2_XXS: 2 B, fp16 d, LE)
 * (src/iq2_matmul.rs:13-29; block index = row * blocks_per_row + blk).
 *
 * Replaces iq2_matmul_metal (src/iq2_matmul.rs:197-365) as reached from
 * iq2_matmul / iq2_xxs_matmul (:535-553, :604-619) with mode OFF, and from
 * iq2_matmul_with_activation_quant (:559-591) for every mode:
 *   OFF  -> plain matmul;
 *   W8A8 -> x is first fake-quantised per row (inv = 127/max|x_row|, or 1 when
 *           max < 1e-8; q = clamp(round_half_away(x*inv), +-127); x' = q/inv),
 *           iq2_matmul.metal:85-126;
 *   W4A8 -> error when `strict` != 0, else runs as OFF (:581-589).
 * x_len / weight_bytes_len / weight_scales_len are the element counts the
 * caller's buffers hold; like the reference, larger weight buffers are fine
 * (:237-259) and x must hold at least m*in_dim elements.
 * Dimensions must be non-zero and fit in u32 (:210-212, :305-311).
 * `workspace` may be NULL when cmk_iq2_matmul_workspace_size reports 0.  The
 * MFMA GEMM (m > 16, in_dim % 8 == 0) needs one for W8A8, for f32 x (each row
 * scaled by a power of two and staged as an f16 head / tail pair, so x keeps
 * about 22 bits) and for shapes too small to fill the GPU, whose k is split
 * (partials summed in a fixed order: results are the same on every run).
 * The multi-row decode kernel (2 <= m, decode shapes) uses the workspace when
 * it is given and large enough, and runs without it otherwise: its 32-row
 * groups fill at most N / 32 CUs, so where that leaves CUs idle it splits K
 * into parts, one workgroup each, whose sums meet in the workspace and are
 * added in part order by the part that finishes last (the same results on
 * every run, equal to the unsplit launch up to fp32 rounding).  The workspace
 * needs no initial contents; launches that share one must be ordered (one
 * stream).
 */
int cmk_iq2_matmul(const void *x, cmk_dtype x_dtype, size_t x_len, size_t m,
                   const uint8_t *weight_bytes, size_t weight_bytes_len,
                   const uint8_t *weight_scales, size_t weight_scales_len,
                   size_t out_dim, size_t in_dim, cmk_iq2_variant variant,
                   cmk_act_quant_mode mode, int strict,
                   float *out, void *workspace, size_t workspace_bytes, void *stream);

/*
 * cmk_iq2_matmul without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * hosts that forbid allocation).  No counterpart in the reference, whose
 * dispatch allocates its output per call (src/iq2_matmul.rs:261).  Same
 * arguments, checks, kernels and results as cmk_iq2_matmul; the scratch the
 * launch needs (the MFMA GEMM's staged rows, row scales and k-split partials)
 * comes from an array inside the library, one per device, of
 * CMK_IQ2_NOALLOC_SCRATCH_BYTES bytes.  Arguments that need more fail with
 * CMK_ERR_INVALID_ARGUMENT before anything is launched.  The call performs no
 * device allocation: the array is part of the code object and lives until the
 * process ends; the first call on a device looks up its address once.  All
 * calls on one device share that device's array and nothing clears it between
 * calls (every launch writes what it reads): calls that can overlap on one
 * device -- different streams, or host threads without ordering -- race on it.
 */
#define CMK_IQ2_NOALLOC_SCRATCH_BYTES (32u << 20)
int cmk_iq2_matmul_noalloc(const void *x, cmk_dtype x_dtype, size_t x_len, size_t m,
                           const uint8_t *weight_bytes, size_t weight_bytes_len,
                           const uint8_t *weight_scales, size_t weight_scales_len,
                           size_t out_dim, size_t in_dim, cmk_iq2_variant variant,
                           cmk_act_quant_mode mode, int strict, float *out, void *stream);

/* Device scratch (bytes) that cmk_iq2_matmul needs for these arguments.  The
 * launch never allocates; callers that get a non-zero size pass a buffer of at
 * least that many bytes.  Same argument validation as cmk_iq2_matmul.  The
 * size includes the multi-row kernel's optional split over K, counted for
 * 256 CUs (a device with fewer CUs never splits more). */
int cmk_iq2_matmul_workspace_size(cmk_dtype x_dtype, size_t m, size_t out_dim, size_t in_dim,
                                  cmk_iq2_variant variant, cmk_act_quant_mode mode,
                                  size_t *bytes);

/*
 * out[out_dim, in_dim] = dequantised W in out_dtype (F16, BF16 or F32).
 * Replaces iq2_dequantize_to_f16_metal (src/iq2_matmul.rs:367-505) reached
 * from iq2_dequantize_to_f16 (:594-602), whose kernels are the four
 * *_dequantize_f16 kernels (iq2_matmul.metal:868-950, decodes :701-866).
 * Every value is the single round-to-nearest-even of the exact product
 * dl*g*sign (dl = d*(0.5+s)*0.25 for the IQ2 formats, d*(1+2s) for IQ3_S);
 * F32 output is that exact product.  F16 is the reference's output type;
 * BF16/F32 are this build's extensions on the same boundary.  IQ2_XXS needs
 * 8-byte aligned weight_bytes and 2-byte aligned weight_scales; the other
 * variants take any alignment.
 */
int cmk_iq2_dequantize(const uint8_t *weight_bytes, size_t weight_bytes_len,
                       const uint8_t *weight_scales, size_t weight_scales_len,
                       size_t out_dim, size_t in_dim, cmk_iq2_variant variant,
                       cmk_dtype out_dtype, void *out, void *stream);

/*
 * Splits n_blocks GGUF (ggml) blocks of `variant` into the reference's pair:
 * weight_bytes (the code bytes, bytes_per_block each) and weight_scales (the
 * fp16 d, then the packed scales; scales_per_block each).  A ggml block is
 * {d; codes; scales}: 66, 74, 82 or 110 bytes for IQ2_XXS, IQ2_XS, IQ2_S,
 * IQ3_S (ggml's block_iq2_xxs / block_iq2_xs / block_iq2_s / block_iq3_s).
 * No counterpart in the reference, which expects callers to have split the
 * blocks already (src/iq2_matmul.rs:13-17); it is the on-disk format step for
 * GGUF weights.  Device pointers, any alignment, asynchronous on `stream`.
 */
int cmk_iq2_split_gguf_blocks(const uint8_t *blocks, size_t blocks_len, size_t n_blocks,
                              cmk_iq2_variant variant, uint8_t *weight_bytes,
                              size_t weight_bytes_len, uint8_t *weight_scales,
                              size_t weight_scales_len, void *stream);

/*
 * out[i] = silu(gate[i]) * up[i], i < n, silu(g) = g / (1 + exp(-g)) in fp32;
 * out in F32, F16 or BF16 (one round-to-nearest-even).  The step between the
 * gate/up and down projections of a Llama-style MLP: gate and up are the fp32
 * outputs of cmk_iq2_matmul, out feeds the down projection's cmk_iq2_matmul
 * (F32 for the GEMV at small m, F16/BF16 for the MFMA GEMM).  No counterpart in
 * the reference, whose callers compose it from candle ops.  Device pointers,
 * asynchronous on `stream`.
 */
int cmk_swiglu(const float *gate, const float *up, size_t n, cmk_dtype out_dtype, void *out,
               void *stream);

/*
 * The up projection of a gated MLP with the step above folded into its
 * epilogue: out[m, out_dim] = silu(gate) * iq2_matmul(x) for the IQ2_XXS
 * weights, elementwise, with gate the gate projection's output ([m, out_dim]
 * f32, `gate_len` elements, not overlapping out).  Equal, bit for bit, to
 * cmk_iq2_matmul into a buffer u followed by cmk_swiglu(gate, u, F32): the
 * epilogue evaluates the same fp32 expression on the same sum.  Serves the
 * decode-shaped kernels only (m <= 16, no
 * activation quantisation, weight_bytes 16-byte and weight_scales 2-byte
 * aligned); CMK_ERR_UNSUPPORTED otherwise.  `workspace` as for cmk_iq2_matmul
 * with mode OFF (cmk_iq2_matmul_workspace_size): the bit-for-bit equality
 * holds between calls given the same workspace size (both split K or
 * neither).  No counterpart in the reference, whose callers compose the MLP
 * from candle ops.  Device pointers, asynchronous on `stream`.
 */
int cmk_iq2_matmul_swiglu(const void *x, cmk_dtype x_dtype, size_t x_len, size_t m,
                          const uint8_t *weight_bytes, size_t weight_bytes_len,
                          const uint8_t *weight_scales, size_t weight_scales_len,
                          size_t out_dim, size_t in_dim, const float *gate, size_t gate_len,
                          float *out, void *workspace, size_t workspace_bytes, void *stream);

/* ------------------------------------------------------------------------ */
/* Errors and introspection                                                  */
/* ------------------------------------------------------------------------ */

/* Message of the last failed call on this thread ("" if none). */
const char *cmk_last_error(void);
/* CMK_IQ2_ABI_VERSION of the loaded library. */
int cmk_abi_version(void);
/* Which kernel family cmk_iq2_matmul picks for these arguments:
 * 0 = GEMV (small m), 1 = MFMA GEMM.  Host-only, no device needed. */
int cmk_iq2_matmul_path(cmk_dtype x_dtype, size_t m, size_t out_dim, size_t in_dim,
                        cmk_act_quant_mode mode);

/* ------------------------------------------------------------------------ */
/* Thin HIP runtime wrappers for hosts that do not link HIP themselves (the   */
/* Rust crate's src/hip/ffi.rs).  All return cmk_status.                      */
/* ------------------------------------------------------------------------ */

int cmk_device_count(int *count);
int cmk_set_device(int ordinal);
/* Name, CU count, LDS bytes per workgroup, peak memory clock (kHz) and bus
 * width (bits) of the current device; name_len includes the terminator. */
int cmk_device_props(char *name, size_t name_len, int *cu_count, size_t *lds_bytes,
                     int *mem_clock_khz, int *mem_bus_bits);
int cmk_malloc(void **ptr, size_t bytes);
int cmk_free(void *ptr);
int cmk_memcpy_htod(void *dst, const void *src, size_t bytes, void *stream);
int cmk_memcpy_dtoh(void *dst, const void *src, size_t bytes, void *stream);
int cmk_memset(void *dst, int value, size_t bytes, void *stream);
int cmk_stream_create(void **stream);
int cmk_stream_destroy(void *stream);
int cmk_stream_synchronize(void *stream);
int cmk_device_synchronize(void);
int cmk_event_create(void **event);
int cmk_event_destroy(void *event);
int cmk_event_record(void *event, void *stream);
/* Milliseconds between two recorded, completed events. */
int cmk_event_elapsed_ms(void *start, void *stop, float *ms);

#ifdef __cplusplus
}
#endif

#endif /* CMK_IQ2_H */
