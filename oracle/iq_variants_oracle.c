/*
 * TEST INFRASTRUCTURE ONLY — CPU oracle for the IQ2_XS, IQ2_S and IQ3_S
 * variants.  See iq_variants_oracle.h for the contract.  Loaded only by
 * tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline leg.
 *
 * Pinning, per function (tests in tests/test_oracle_variants.py):
 *  - oracle_iq_grid: SHA-256 of the decoded little-endian images equal the
 *    digests recorded from the reference's table text; value sets {8,25,43}
 *    (IQ2) and odd 1..15 (IQ3_S); sorted and unique; byte-equal to the
 *    reference text when it is present.
 *  - dequantize: each element against the closed form d*(0.5+s)/4*g*sign
 *    (IQ2) or d*(1+2s)*g*sign (IQ3_S) computed in exact rational arithmetic
 *    from fields placed by hand into otherwise zero blocks (a grid index, a
 *    sign pattern, a scale nibble, the IQ2_S / IQ3_S high bits at each of
 *    their positions), so a wrong bit offset, nibble or byte fails.
 *  - matmul reference: one-hot x = e_k reproduces column k of the dequantized
 *    matrix exactly; numpy float64 x @ W^T agrees to fp32 rounding; columns
 *    >= in_dim never contribute; W8A8 = plain reference on qdq(x).
 */
#include "iq_variants_oracle.h"

#include "iq2xxs_oracle.h"
#include "iq_variants_oracle_tables.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- tables ------------------------------------------------------------- */

static uint8_t v_kmask[8];
static uint8_t v_ksigns[128];
static uint64_t v_iq2xs[512];
static uint64_t v_iq2s[1024];
static uint32_t v_iq3s[512];
static int v_ready = 0;

static uint64_t decode2(uint16_t code) {
    static const uint8_t lv[3] = {8, 25, 43};
    uint64_t v = 0;
    for (int j = 0; j < 8; ++j) v |= (uint64_t)lv[(code >> (2 * j)) & 3u] << (8 * j);
    return v;
}

static uint32_t decode3(uint16_t code) {
    uint32_t v = 0;
    for (int j = 0; j < 4; ++j) v |= (uint32_t)(2u * ((code >> (3 * j)) & 7u) + 1u) << (8 * j);
    return v;
}

static void build_variant_tables(void) {
    if (v_ready) return;
    uint64_t xxs[256];
    oracle_tables(v_kmask, v_ksigns, xxs);
    for (int i = 0; i < 512; ++i) v_iq2xs[i] = decode2(ORACLE_IQ2XS_CODES[i]);
    for (int i = 0; i < 1024; ++i) v_iq2s[i] = decode2(ORACLE_IQ2S_CODES[i]);
    for (int i = 0; i < 512; ++i) v_iq3s[i] = decode3(ORACLE_IQ3S_CODES[i]);
    v_ready = 1;
}

size_t oracle_iq_bytes_per_block(int variant) {
    switch (variant) {
        case ORACLE_IQ2_XXS: return 64;
        case ORACLE_IQ2_XS: return 64;
        case ORACLE_IQ2_S: return 72;
        case ORACLE_IQ3_S: return 104;
        default: return 0;
    }
}

size_t oracle_iq_scales_per_block(int variant) {
    switch (variant) {
        case ORACLE_IQ2_XXS: return 2;
        case ORACLE_IQ2_XS: return 10;
        case ORACLE_IQ2_S: return 10;
        case ORACLE_IQ3_S: return 6;
        default: return 0;
    }
}

size_t oracle_iq_grid(int variant, uint64_t *grid) {
    build_variant_tables();
    switch (variant) {
        case ORACLE_IQ2_XXS: {
            uint8_t km[8], ks[128];
            uint64_t g[256];
            oracle_tables(km, ks, g);
            if (grid) memcpy(grid, g, sizeof(g));
            return 256;
        }
        case ORACLE_IQ2_XS:
            if (grid) memcpy(grid, v_iq2xs, sizeof(v_iq2xs));
            return 512;
        case ORACLE_IQ2_S:
            if (grid) memcpy(grid, v_iq2s, sizeof(v_iq2s));
            return 1024;
        case ORACLE_IQ3_S:
            if (grid)
                for (int i = 0; i < 512; ++i) grid[i] = v_iq3s[i];
            return 512;
        default: return 0;
    }
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* accum_word_grid (src/iq2_matmul.rs:789-809) and accum_word_grid_u32
 * (:811-831): n magnitudes of grid_pack, signs tested against kmask[0..n),
 * `acc += x * (dl * gv * sign)` left to right, no contraction. */
static void accum(uint64_t grid_pack, int n, uint8_t signs, const uint8_t *kmask, float dl,
                  size_t base_col, size_t in_dim, const float *x_row, float *acc) {
    for (int j = 0; j < n; ++j) {
        size_t col = base_col + (size_t)j;
        if (col >= in_dim) break;
        uint8_t gv = (uint8_t)((grid_pack >> (8 * j)) & 0xFFu);
        float sign = (signs & kmask[j]) ? -1.0f : 1.0f;
        float w = dl * (float)gv;
        w = w * sign;
        *acc = *acc + x_row[col] * w;
    }
}

/* dl = d * (0.5 + nib) * 0.25, as the reference writes it (IQ2 formats). */
static float dl_iq2(float d, unsigned nib) {
    float dl = d * (0.5f + (float)nib);
    return dl * 0.25f;
}

/* One output of iq2_matmul_reference for the IQ2_XS / IQ2_S / IQ3_S branches
 * (src/iq2_matmul.rs:884-1016). */
static float reference_one(int variant, const float *x_row, size_t out_idx, size_t in_dim,
                           size_t bpr, const uint8_t *wb, const uint8_t *ws) {
    const size_t bb = oracle_iq_bytes_per_block(variant), sb = oracle_iq_scales_per_block(variant);
    float acc = 0.0f;
    for (size_t blk = 0; blk < bpr; ++blk) {
        size_t block_idx = out_idx * bpr + blk;
        const uint8_t *q = wb + block_idx * bb;
        const uint8_t *sc = ws + block_idx * sb;
        float d = oracle_f16_to_f32(rd16(sc));
        for (size_t ib32 = 0; ib32 < 8; ++ib32) {
            size_t col0 = blk * ORACLE_QK + ib32 * 32;
            if (variant == ORACLE_IQ2_XS) {
                /* :884-918 */
                uint8_t scale_byte = sc[2 + ib32];
                float dl0 = dl_iq2(d, scale_byte & 0x0Fu);
                float dl1 = dl_iq2(d, (scale_byte >> 4) & 0x0Fu);
                for (int w = 0; w < 4; ++w) {
                    uint16_t qw = rd16(q + ib32 * 8 + 2 * w);
                    accum(v_iq2xs[qw & 0x1FFu], 8, v_ksigns[(qw >> 9) & 0x7Fu], v_kmask,
                          w < 2 ? dl0 : dl1, col0 + 8 * (size_t)w, in_dim, x_row, &acc);
                }
            } else if (variant == ORACLE_IQ2_S) {
                /* :919-970 */
                const uint8_t *qs = q, *qh = q + 64;
                uint8_t qh_byte = qh[ib32], scale_byte = sc[2 + ib32];
                for (size_t il = 0; il < 2; ++il) {
                    size_t qs_off = 4 * ib32 + 2 * il;
                    uint8_t qh_nib = (uint8_t)(qh_byte >> (4 * il));
                    float dl = dl_iq2(d, (scale_byte >> (4 * il)) & 0x0Fu);
                    size_t g0 = (size_t)qs[qs_off] | (((size_t)qh_nib << 8) & 0x300u);
                    size_t g1 = (size_t)qs[qs_off + 1] | (((size_t)qh_nib << 6) & 0x300u);
                    size_t base = col0 + il * 16;
                    accum(v_iq2s[g0], 8, qs[32 + qs_off], v_kmask, dl, base, in_dim, x_row, &acc);
                    accum(v_iq2s[g1], 8, qs[32 + qs_off + 1], v_kmask, dl, base + 8, in_dim, x_row,
                          &acc);
                }
            } else {
                /* IQ3_S, :971-1014 */
                const uint8_t *qs = q, *qh = q + 64, *signs = q + 72;
                uint8_t qh_byte = qh[ib32];
                unsigned nib = (sc[2 + ib32 / 2] >> (4 * (ib32 % 2))) & 0x0Fu;
                float dl = d * (1.0f + 2.0f * (float)nib);
                for (size_t l = 0; l < 4; ++l) {
                    size_t i1 = (size_t)qs[8 * ib32 + 2 * l] | ((qh_byte & v_kmask[2 * l]) ? 256u : 0u);
                    size_t i2 =
                        (size_t)qs[8 * ib32 + 2 * l + 1] | ((qh_byte & v_kmask[2 * l + 1]) ? 256u : 0u);
                    uint8_t sign_byte = signs[4 * ib32 + l];
                    size_t base = col0 + l * 8;
                    accum(v_iq3s[i1], 4, sign_byte, v_kmask, dl, base, in_dim, x_row, &acc);
                    accum(v_iq3s[i2], 4, sign_byte, v_kmask + 4, dl, base + 4, in_dim, x_row, &acc);
                }
            }
        }
    }
    return acc;
}

void oracle_iq_matmul_reference(int variant, const float *x, size_t m, size_t out_dim,
                                size_t in_dim, const uint8_t *weight_bytes,
                                const uint8_t *weight_scales, float *out) {
    if (variant == ORACLE_IQ2_XXS) {
        oracle_iq2xxs_matmul_reference(x, m, out_dim, in_dim, weight_bytes, weight_scales, out);
        return;
    }
    build_variant_tables();
    size_t bpr = (in_dim + ORACLE_QK - 1) / ORACLE_QK;
    for (size_t row = 0; row < m; ++row)
        for (size_t o = 0; o < out_dim; ++o)
            out[row * out_dim + o] = reference_one(variant, x + row * in_dim, o, in_dim, bpr,
                                                   weight_bytes, weight_scales);
}

void oracle_iq_matmul_reference_w8a8(int variant, const float *x, size_t m, size_t out_dim,
                                     size_t in_dim, const uint8_t *weight_bytes,
                                     const uint8_t *weight_scales, float *out) {
    size_t n = m * in_dim;
    float *xq = (float *)malloc((n ? n : 1) * sizeof(float));
    if (!xq) return;
    oracle_rowwise_qdq_w8a8(x, m, in_dim, xq);
    oracle_iq_matmul_reference(variant, xq, m, out_dim, in_dim, weight_bytes, weight_scales, out);
    free(xq);
}

/* decode_iq2_xs_value / decode_iq2_s_value / decode_iq3_s_value
 * (iq2_matmul.metal:736-866): dl * gv * sgn evaluated left to right. */
static float decode_value(int variant, const uint8_t *wb, const uint8_t *ws, size_t block_idx,
                          size_t local_col) {
    const size_t bb = oracle_iq_bytes_per_block(variant), sb = oracle_iq_scales_per_block(variant);
    const uint8_t *q = wb + block_idx * bb;
    const uint8_t *sc = ws + block_idx * sb;
    float d = oracle_f16_to_f32(rd16(sc));
    size_t ib32 = local_col / 32, within32 = local_col % 32;
    uint8_t gv, signs, mask;
    float dl;
    if (variant == ORACLE_IQ2_XS) {
        size_t word = within32 / 8, j = within32 % 8;
        uint16_t qw = rd16(q + ib32 * 8 + 2 * word);
        uint8_t scale_byte = sc[2 + ib32];
        dl = word < 2 ? dl_iq2(d, scale_byte & 0x0Fu) : dl_iq2(d, (scale_byte >> 4) & 0x0Fu);
        gv = (uint8_t)((v_iq2xs[qw & 0x1FFu] >> (8 * j)) & 0xFFu);
        signs = v_ksigns[(qw >> 9) & 0x7Fu];
        mask = v_kmask[j];
    } else if (variant == ORACLE_IQ2_S) {
        size_t il = within32 / 16, within16 = within32 % 16, j = within16 % 8;
        const uint8_t *qs = q, *qh = q + 64;
        uint8_t qh_nib = (uint8_t)(qh[ib32] >> (4 * il));
        dl = dl_iq2(d, (sc[2 + ib32] >> (4 * il)) & 0x0Fu);
        size_t qs_off = 4 * ib32 + 2 * il, gi;
        if (within16 < 8) {
            gi = (size_t)qs[qs_off] | (((size_t)qh_nib << 8) & 0x300u);
            signs = qs[32 + qs_off];
        } else {
            gi = (size_t)qs[qs_off + 1] | (((size_t)qh_nib << 6) & 0x300u);
            signs = qs[32 + qs_off + 1];
        }
        gv = (uint8_t)((v_iq2s[gi] >> (8 * j)) & 0xFFu);
        mask = v_kmask[j];
    } else {
        size_t l = within32 / 8, within8 = within32 % 8;
        const uint8_t *qs = q, *qh = q + 64, *sg = q + 72;
        uint8_t qh_byte = qh[ib32];
        unsigned nib = (sc[2 + ib32 / 2] >> (4 * (ib32 % 2))) & 0x0Fu;
        dl = d * (1.0f + 2.0f * (float)nib);
        size_t i1 = (size_t)qs[8 * ib32 + 2 * l] | ((qh_byte & v_kmask[2 * l]) ? 256u : 0u);
        size_t i2 = (size_t)qs[8 * ib32 + 2 * l + 1] | ((qh_byte & v_kmask[2 * l + 1]) ? 256u : 0u);
        signs = sg[4 * ib32 + l];
        if (within8 < 4) {
            gv = (uint8_t)((v_iq3s[i1] >> (8 * within8)) & 0xFFu);
            mask = v_kmask[within8];
        } else {
            gv = (uint8_t)((v_iq3s[i2] >> (8 * (within8 - 4))) & 0xFFu);
            mask = v_kmask[within8];
        }
    }
    float sgn = (signs & mask) ? -1.0f : 1.0f;
    float v = dl * (float)gv;
    return v * sgn;
}

void oracle_iq_dequantize_f32(int variant, const uint8_t *weight_bytes,
                              const uint8_t *weight_scales, size_t out_dim, size_t in_dim,
                              float *out) {
    if (variant == ORACLE_IQ2_XXS) {
        oracle_iq2xxs_dequantize_f32(weight_bytes, weight_scales, out_dim, in_dim, out);
        return;
    }
    build_variant_tables();
    size_t bpr = (in_dim + ORACLE_QK - 1) / ORACLE_QK;
    for (size_t o = 0; o < out_dim; ++o)
        for (size_t c = 0; c < in_dim; ++c)
            out[o * in_dim + c] = decode_value(variant, weight_bytes, weight_scales,
                                               o * bpr + c / ORACLE_QK, c % ORACLE_QK);
}

void oracle_iq_dequantize_f16(int variant, const uint8_t *weight_bytes,
                              const uint8_t *weight_scales, size_t out_dim, size_t in_dim,
                              uint16_t *out) {
    if (variant == ORACLE_IQ2_XXS) {
        oracle_iq2xxs_dequantize_f16(weight_bytes, weight_scales, out_dim, in_dim, out);
        return;
    }
    build_variant_tables();
    size_t bpr = (in_dim + ORACLE_QK - 1) / ORACLE_QK;
    for (size_t o = 0; o < out_dim; ++o)
        for (size_t c = 0; c < in_dim; ++c)
            out[o * in_dim + c] = oracle_f32_to_f16(decode_value(
                variant, weight_bytes, weight_scales, o * bpr + c / ORACLE_QK, c % ORACLE_QK));
}

void oracle_iq_dequantize_bf16(int variant, const uint8_t *weight_bytes,
                               const uint8_t *weight_scales, size_t out_dim, size_t in_dim,
                               uint16_t *out) {
    if (variant == ORACLE_IQ2_XXS) {
        oracle_iq2xxs_dequantize_bf16(weight_bytes, weight_scales, out_dim, in_dim, out);
        return;
    }
    build_variant_tables();
    size_t bpr = (in_dim + ORACLE_QK - 1) / ORACLE_QK;
    for (size_t o = 0; o < out_dim; ++o)
        for (size_t c = 0; c < in_dim; ++c)
            out[o * in_dim + c] = oracle_f32_to_bf16(decode_value(
                variant, weight_bytes, weight_scales, o * bpr + c / ORACLE_QK, c % ORACLE_QK));
}

void oracle_iq_matmul_f64(int variant, const float *x, size_t m, size_t out_dim, size_t in_dim,
                          const uint8_t *weight_bytes, const uint8_t *weight_scales, double *out,
                          double *abs_scale) {
    if (variant == ORACLE_IQ2_XXS) {
        oracle_iq2xxs_matmul_f64(x, m, out_dim, in_dim, weight_bytes, weight_scales, out,
                                 abs_scale);
        return;
    }
    build_variant_tables();
    size_t bpr = (in_dim + ORACLE_QK - 1) / ORACLE_QK;
    float *w = (float *)malloc((in_dim ? in_dim : 1) * sizeof(float));
    if (!w) return;
    for (size_t o = 0; o < out_dim; ++o) {
        for (size_t c = 0; c < in_dim; ++c)
            w[c] = decode_value(variant, weight_bytes, weight_scales, o * bpr + c / ORACLE_QK,
                                c % ORACLE_QK);
        for (size_t row = 0; row < m; ++row) {
            const float *xr = x + row * in_dim;
            double acc = 0.0, s = 0.0;
            for (size_t c = 0; c < in_dim; ++c) {
                double p = (double)xr[c] * (double)w[c];
                acc += p;
                s += fabs(p);
            }
            out[row * out_dim + o] = acc;
            if (abs_scale) abs_scale[row * out_dim + o] = s;
        }
    }
    free(w);
}

/* ---- GGUF block layout ---------------------------------------------------- */

size_t oracle_gguf_block_bytes(int variant) {
    size_t b = oracle_iq_bytes_per_block(variant), s = oracle_iq_scales_per_block(variant);
    return b ? b + s : 0;
}

void oracle_gguf_to_split(int variant, const uint8_t *blocks, size_t n_blocks,
                          uint8_t *weight_bytes, uint8_t *weight_scales) {
    const size_t bb = oracle_iq_bytes_per_block(variant), sb = oracle_iq_scales_per_block(variant);
    const size_t gb = bb + sb;
    for (size_t i = 0; i < n_blocks; ++i) {
        const uint8_t *src = blocks + i * gb;
        uint8_t *ws = weight_scales + i * sb;
        memcpy(ws, src, 2);                             /* d */
        memcpy(weight_bytes + i * bb, src + 2, bb);     /* codes */
        memcpy(ws + 2, src + 2 + bb, sb - 2);           /* packed scales (none for IQ2_XXS) */
    }
}
