/*
 * TEST INFRASTRUCTURE ONLY — the CPU oracle for the IQ2_XXS matmul path.
 *
 * This is a plain-C restatement of the reference crate's scalar CPU reference
 * (Steboss/candelora-metal-kernels, src/iq2_matmul.rs, test module) and of the
 * Metal decode it mirrors.  It is the checker for the HIP kernels and the CPU
 * baseline timed by bench.py; nothing on the product path may call it.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this library.  Every function cites the reference file:line it follows.
 *
 * Pinning (what keeps this restatement honest) is listed per function in
 * iq2xxs_oracle.c; the tests that perform it live in tests/test_oracle*.py.
 *
 * Build: oracle/Makefile (gcc -O3 -ffp-contract=off, no -ffast-math): Rust
 * does not contract a*b+c into an FMA, so neither may the restatement.
 */
#ifndef IQ2XXS_ORACLE_H
#define IQ2XXS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Format constants: src/iq2_matmul.rs:13-17 (IQ2_QK, IQ2_XXS_BYTES_PER_BLOCK,
 * IQ2_XXS_SCALES_PER_BLOCK). */
#define ORACLE_QK 256
#define ORACLE_XXS_BYTES_PER_BLOCK 64
#define ORACLE_XXS_SCALES_PER_BLOCK 2

/* Table images (little-endian values), decoded from the oracle's own copy of
 * the codebook.  kmask: iq2_tables.metal:4-6, ksigns: :8-17, grid: :19-84. */
void oracle_tables(uint8_t kmask[8], uint8_t ksigns[128], uint64_t grid[256]);

/* IEEE binary16 -> binary32, exact widening (half 2.7.1 f16::to_f32,
 * src/iq2_matmul.rs:856). */
float oracle_f16_to_f32(uint16_t h);
/* binary32 -> binary16 / bfloat16, round-to-nearest-even (Metal half(float),
 * iq2_matmul.metal:886; candle to_dtype). NaN maps to a quiet NaN. */
uint16_t oracle_f32_to_f16(float f);
uint16_t oracle_f32_to_bf16(float f);

/* Reference input generators.
 * lcg_fill: src/iq2_matmul.rs:765-773 (and examples/iq2_matmul_bench.rs:215-223).
 * deterministic_x: src/iq2_matmul.rs:775-779.
 * force_f16_one_per_block: src/iq2_matmul.rs:781-787. */
void oracle_lcg_fill(uint8_t *out, size_t len, uint32_t seed);
void oracle_deterministic_x(float *out, size_t len);
void oracle_force_f16_one_per_block(uint8_t *scales, size_t len, size_t scales_per_block);

/* iq2_matmul_reference, IQ2_XXS branch: src/iq2_matmul.rs:833-883 with
 * accum_word_grid :789-809 and read_u16_le :761-763.  Sequential fp32
 * accumulation in the loop order row -> out -> blk -> ib32 -> g -> j.
 * out is [m, out_dim] fp32. */
void oracle_iq2xxs_matmul_reference(const float *x, size_t m, size_t out_dim, size_t in_dim,
                                    const uint8_t *weight_bytes, const uint8_t *weight_scales,
                                    float *out);

/* Same loop, OpenMP over (row, out) pairs with identical per-output arithmetic,
 * so results are bit-identical to oracle_iq2xxs_matmul_reference. Used only as
 * the multi-core CPU baseline.  Returns the thread count used. */
int oracle_iq2xxs_matmul_reference_mt(const float *x, size_t m, size_t out_dim, size_t in_dim,
                                      const uint8_t *weight_bytes, const uint8_t *weight_scales,
                                      float *out, int threads);

/* rowwise_quant_dequant_w8a8: src/iq2_matmul.rs:1025-1042 (Metal
 * row_inv_scale_w8a8/qdq_w8a8, iq2_matmul.metal:85-102). */
void oracle_rowwise_qdq_w8a8(const float *x, size_t m, size_t in_dim, float *out);

/* iq2_matmul_reference_w8a8: src/iq2_matmul.rs:1044-1063. */
void oracle_iq2xxs_matmul_reference_w8a8(const float *x, size_t m, size_t out_dim, size_t in_dim,
                                         const uint8_t *weight_bytes, const uint8_t *weight_scales,
                                         float *out);

/* Element decode, decode_iq2_xxs_value: iq2_matmul.metal:701-734.  Writes the
 * dense fp32 matrix [out_dim, in_dim] (columns >= in_dim are not produced). */
void oracle_iq2xxs_dequantize_f32(const uint8_t *weight_bytes, const uint8_t *weight_scales,
                                  size_t out_dim, size_t in_dim, float *out);

/* iq2_xxs_dequantize_f16 (iq2_matmul.metal:868-887): RNE of each fp32 value.
 * The bf16 variant is the build's extension (same decode, bf16 RNE). */
void oracle_iq2xxs_dequantize_f16(const uint8_t *weight_bytes, const uint8_t *weight_scales,
                                  size_t out_dim, size_t in_dim, uint16_t *out);
void oracle_iq2xxs_dequantize_bf16(const uint8_t *weight_bytes, const uint8_t *weight_scales,
                                   size_t out_dim, size_t in_dim, uint16_t *out);

/* Error-metric helpers (not a restatement of any reference function):
 * fp64 accumulation of the same products in the same order, plus the
 * condition scale sum_k |x_k * w_nk| for each output.  Both [m, out_dim]. */
void oracle_iq2xxs_matmul_f64(const float *x, size_t m, size_t out_dim, size_t in_dim,
                              const uint8_t *weight_bytes, const uint8_t *weight_scales,
                              double *out, double *abs_scale);

#ifdef __cplusplus
}
#endif

#endif
