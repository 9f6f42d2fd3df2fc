/*
 * TEST INFRASTRUCTURE ONLY — the CPU oracle for the IQ2_XS, IQ2_S and IQ3_S
 * variants of the matmul path.
 *
 * Plain-C restatement of the other branches of the reference crate's scalar
 * CPU reference (Steboss/candelora-metal-kernels, src/iq2_matmul.rs:884-1016,
 * with accum_word_grid :789-809 and accum_word_grid_u32 :811-831) and of the
 * Metal element decodes (src/metal_src/iq2_matmul.metal:736-866).  Same build,
 * same loading rules and same pinning approach as iq2xxs_oracle.h; variant 0
 * (IQ2_XXS) forwards to the functions declared there.
 */
#ifndef IQ_VARIANTS_ORACLE_H
#define IQ_VARIANTS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Iq2MatmulVariant (src/iq2_matmul.rs:31-37) in declaration order. */
#define ORACLE_IQ2_XXS 0
#define ORACLE_IQ2_XS 1
#define ORACLE_IQ2_S 2
#define ORACLE_IQ3_S 3

/* bytes_per_block / scales_per_block (src/iq2_matmul.rs:13-29,39-57); 0 for an
 * unknown variant. */
size_t oracle_iq_bytes_per_block(int variant);
size_t oracle_iq_scales_per_block(int variant);

/* The decoded codebook of a variant as little-endian values (IQ3_S entries are
 * u32 values widened to u64).  Returns the entry count (256, 512, 1024, 512)
 * and writes that many values when grid is non-null. */
size_t oracle_iq_grid(int variant, uint64_t *grid);

/* iq2_matmul_reference, src/iq2_matmul.rs:833-1016: sequential fp32
 * accumulation in the loop order row -> out -> blk -> ib32 -> word -> j.
 * out is [m, out_dim] fp32. */
void oracle_iq_matmul_reference(int variant, const float *x, size_t m, size_t out_dim,
                                size_t in_dim, const uint8_t *weight_bytes,
                                const uint8_t *weight_scales, float *out);

/* iq2_matmul_reference_w8a8, src/iq2_matmul.rs:1044-1063. */
void oracle_iq_matmul_reference_w8a8(int variant, const float *x, size_t m, size_t out_dim,
                                     size_t in_dim, const uint8_t *weight_bytes,
                                     const uint8_t *weight_scales, float *out);

/* Element decodes decode_iq2_xs_value / decode_iq2_s_value /
 * decode_iq3_s_value (iq2_matmul.metal:736-866): the dense fp32 matrix
 * [out_dim, in_dim], and its RNE to f16 / bf16. */
void oracle_iq_dequantize_f32(int variant, const uint8_t *weight_bytes,
                              const uint8_t *weight_scales, size_t out_dim, size_t in_dim,
                              float *out);
void oracle_iq_dequantize_f16(int variant, const uint8_t *weight_bytes,
                              const uint8_t *weight_scales, size_t out_dim, size_t in_dim,
                              uint16_t *out);
void oracle_iq_dequantize_bf16(int variant, const uint8_t *weight_bytes,
                               const uint8_t *weight_scales, size_t out_dim, size_t in_dim,
                               uint16_t *out);

/* GGUF (ggml) block layout to the reference's split pair (src/iq2_matmul.rs:
 * 13-17: weight_bytes + weight_scales).  ggml's block structs (ggml-common.h,
 * the format the reference's tables come from, iq2_tables.metal:1-2) store,
 * per 256-weight block, the fp16 d first, then the code bytes, then (IQ2_XS,
 * IQ2_S, IQ3_S) the packed 4-bit scales last:
 *   iq2_xxs {d; qs[64]}                        66 B -> 64 + 2
 *   iq2_xs  {d; qs[64]; scales[8]}             74 B -> 64 + 10
 *   iq2_s   {d; qs[64]; qh[8]; scales[8]}      82 B -> 72 + 10
 *   iq3_s   {d; qs[64]; qh[8]; signs[32]; scales[4]}  110 B -> 104 + 6
 * weight_scales = d followed by the scales; weight_bytes = everything between.
 * Returns the GGUF block size, 0 for an unknown variant. */
size_t oracle_gguf_block_bytes(int variant);
void oracle_gguf_to_split(int variant, const uint8_t *blocks, size_t n_blocks,
                          uint8_t *weight_bytes, uint8_t *weight_scales);

/* Error-metric helper (not a restatement): fp64 accumulation of the decoded
 * products plus the condition scale sum_k |x_k * w_nk|, both [m, out_dim]. */
void oracle_iq_matmul_f64(int variant, const float *x, size_t m, size_t out_dim, size_t in_dim,
                          const uint8_t *weight_bytes, const uint8_t *weight_scales, double *out,
                          double *abs_scale);

#ifdef __cplusplus
}
#endif

#endif
