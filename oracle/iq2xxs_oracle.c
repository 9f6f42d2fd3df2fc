/*
 * TEST INFRASTRUCTURE ONLY — CPU oracle for the IQ2_XXS matmul path.
 * See iq2xxs_oracle.h for the contract.  Loaded only by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg.
 *
 * Pinning, per function (tests named in brackets):
 *  - oracle_tables: SHA-256 of the LE images of kmask/ksigns/grid equal the
 *    digests recorded from the reference text; ksigns closed form
 *    i | parity(i) << 7; kmask[j] == 1 << j; grid sorted, unique, bytes in
 *    {8,25,43}; byte-equal to the reference's table text when it is present
 *    [tests/test_oracle_tables.py].
 *  - f16/bf16 conversions: exhaustive over all 65536 half patterns against
 *    numpy's IEEE float16; f32->f16/bf16 RNE against numpy/torch on edge and
 *    random values [tests/test_oracle_numerics.py].
 *  - lcg_fill / deterministic_x: recurrence checked against an independent
 *    jump-ahead form and hand-derived first values [test_oracle_numerics.py].
 *  - matmul reference: (a) one-hot x = e_k reproduces column k of the
 *    dequantized weights exactly; (b) numpy float64 matmul of x with the
 *    dequantized matrix agrees to fp32 rounding; (c) fp64 variant agrees;
 *    (d) partial final super-block: columns >= in_dim never contribute
 *    [tests/test_oracle_matmul.py].
 *  - dequantize: closed form +-d*(2s+1)*g/8 computed in exact rational
 *    arithmetic (Python fractions) for every element of small cases; special
 *    cases d=0, scale nibble 0, grid index 0, subnormal d
 *    [tests/test_oracle_matmul.py].
 *  - W8A8 qdq: exact special cases (all-zero row -> inv=1, +-max -> +-127,
 *    ties round away from zero, tiny rows below 1e-8) and a float64
 *    restatement with explicit f32 rounding [tests/test_oracle_numerics.py].
 */
#include "iq2xxs_oracle.h"
#include "iq2xxs_oracle_tables.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* ---- tables ------------------------------------------------------------- */

static uint8_t g_kmask[8];
static uint8_t g_ksigns[128];
static uint64_t g_grid[256];
static int g_tables_ready = 0;

static void build_tables(void) {
    if (g_tables_ready) return;
    for (int j = 0; j < 8; ++j) g_kmask[j] = (uint8_t)(1u << j);
    for (int i = 0; i < 128; ++i) {
        int pop = 0;
        for (int b = 0; b < 7; ++b) pop += (i >> b) & 1;
        g_ksigns[i] = (uint8_t)(i | ((pop & 1) << 7));
    }
    for (int e = 0; e < 256; ++e) {
        uint64_t v = 0;
        for (int j = 0; j < 8; ++j) {
            unsigned code = (ORACLE_GRID_CODES[e] >> (2 * j)) & 3u;
            v |= (uint64_t)ORACLE_GRID_LEVELS[code] << (8 * j);
        }
        g_grid[e] = v;
    }
    g_tables_ready = 1;
}

void oracle_tables(uint8_t kmask[8], uint8_t ksigns[128], uint64_t grid[256]) {
    build_tables();
    memcpy(kmask, g_kmask, sizeof g_kmask);
    memcpy(ksigns, g_ksigns, sizeof g_ksigns);
    memcpy(grid, g_grid, sizeof g_grid);
}

/* ---- half / bfloat16 ---------------------------------------------------- */

float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    if (exp == 0) {
        if (man == 0) return bits_f32(sign);
        /* subnormal: man * 2^-24, renormalise */
        int e = -1;
        do {
            man <<= 1;
            ++e;
        } while ((man & 0x400u) == 0);
        man &= 0x3FFu;
        return bits_f32(sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13));
    }
    if (exp == 31) return bits_f32(sign | 0x7F800000u | (man << 13));
    return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t oracle_f32_to_f16(float f) {
    uint32_t x = f32_bits(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) {                                   /* below 2^-14: subnormal result */
        if (ax < 0x33000000u) return sign;                    /* below 2^-25: rounds to zero */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        uint32_t s = 126u - e; /* 14..24 */
        uint32_t r = m >> s;
        uint32_t rem = m & ((1u << s) - 1u);
        uint32_t half = 1u << (s - 1u);
        if (rem > half || (rem == half && (r & 1u))) ++r;
        return (uint16_t)(sign | r);
    }
    uint32_t r = (((ax >> 23) - 112u) << 10) | ((ax & 0x7FFFFFu) >> 13);
    uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
}

uint16_t oracle_f32_to_bf16(float f) {
    uint32_t x = f32_bits(f);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)(((x >> 16) & 0x8000u) | 0x7FC0u);
    x += 0x7FFFu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

/* ---- reference input generators ----------------------------------------- */

void oracle_lcg_fill(uint8_t *out, size_t len, uint32_t seed) {
    /* src/iq2_matmul.rs:765-773: state = state*1664525 + 1013904223 (wrapping),
     * emit state >> 24. */
    uint32_t state = seed;
    for (size_t i = 0; i < len; ++i) {
        state = state * 1664525u + 1013904223u;
        out[i] = (uint8_t)(state >> 24);
    }
}

void oracle_deterministic_x(float *out, size_t len) {
    /* src/iq2_matmul.rs:775-779: (((i*17) % 41) as f32 - 20.0) / 13.0 */
    for (size_t i = 0; i < len; ++i) out[i] = ((float)((i * 17u) % 41u) - 20.0f) / 13.0f;
}

void oracle_force_f16_one_per_block(uint8_t *scales, size_t len, size_t scales_per_block) {
    /* src/iq2_matmul.rs:781-787: chunks_exact_mut -> a trailing partial chunk
     * is left untouched. */
    for (size_t b = 0; b + scales_per_block <= len; b += scales_per_block) {
        scales[b] = 0x00;
        scales[b + 1] = 0x3C;
    }
}

/* ---- matmul reference ---------------------------------------------------- */

static uint16_t read_u16_le(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* accum_word_grid, src/iq2_matmul.rs:789-809.  `acc += x * (dl * gv * sign)`
 * evaluated left-to-right inside the parentheses, no FMA contraction. */
static void accum_word_grid(uint64_t grid_pack, uint8_t signs, float dl, size_t base_col,
                            size_t in_dim, const float *x_row, float *acc) {
    for (int j = 0; j < 8; ++j) {
        size_t col = base_col + (size_t)j;
        if (col >= in_dim) break;
        uint8_t gv = (uint8_t)((grid_pack >> (8 * j)) & 0xFFu);
        float sign = (signs & g_kmask[j]) ? -1.0f : 1.0f;
        float w = dl * (float)gv;
        w = w * sign;
        *acc = *acc + x_row[col] * w;
    }
}

/* One output of iq2_matmul_reference (IQ2_XXS), src/iq2_matmul.rs:841-883. */
static float reference_one(const float *x_row, size_t out_idx, size_t in_dim, size_t blocks_per_row,
                           const uint8_t *wb, const uint8_t *ws) {
    float acc = 0.0f;
    for (size_t blk = 0; blk < blocks_per_row; ++blk) {
        size_t block_idx = out_idx * blocks_per_row + blk;
        size_t byte_base = block_idx * ORACLE_XXS_BYTES_PER_BLOCK;
        size_t scale_base = block_idx * ORACLE_XXS_SCALES_PER_BLOCK;
        float d = oracle_f16_to_f32(read_u16_le(ws + scale_base));
        for (size_t ib32 = 0; ib32 < 8; ++ib32) {
            size_t q2 = byte_base + ib32 * 8;
            uint32_t aux_g = (uint32_t)read_u16_le(wb + q2) | ((uint32_t)read_u16_le(wb + q2 + 2) << 16);
            uint32_t aux_s = (uint32_t)read_u16_le(wb + q2 + 4) | ((uint32_t)read_u16_le(wb + q2 + 6) << 16);
            float dl = d * (0.5f + (float)((aux_s >> 28) & 0xFu));
            dl = dl * 0.25f;
            for (size_t g = 0; g < 4; ++g) {
                size_t grid_idx = (aux_g >> (8 * g)) & 0xFFu;
                size_t signs_idx = (aux_s >> (7 * g)) & 0x7Fu;
                size_t base_col = blk * ORACLE_QK + ib32 * 32 + g * 8;
                accum_word_grid(g_grid[grid_idx], g_ksigns[signs_idx], dl, base_col, in_dim, x_row,
                                &acc);
            }
        }
    }
    return acc;
}

void oracle_iq2xxs_matmul_reference(const float *x, size_t m, size_t out_dim, size_t in_dim,
                                    const uint8_t *weight_bytes, const uint8_t *weight_scales,
                                    float *out) {
    build_tables();
    size_t bpr = (in_dim + ORACLE_QK - 1) / ORACLE_QK;
    for (size_t row = 0; row < m; ++row)
        for (size_t o = 0; o < out_dim; ++o)
            out[row * out_dim + o] =
                reference_one(x + row * in_dim, o, in_dim, bpr, weight_bytes, weight_scales);
}

int oracle_iq2xxs_matmul_reference_mt(const float *x, size_t m, size_t out_dim, size_t in_dim,
                                      const uint8_t *weight_bytes, const uint8_t *weight_scales,
                                      float *out, int threads) {
    build_tables();
    size_t bpr = (in_dim + ORACLE_QK - 1) / ORACLE_QK;
    long total = (long)(m * out_dim);
    int used = 1;
#ifdef _OPENMP
    if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(threads)
    for (long t = 0; t < total; ++t) {
        size_t row = (size_t)t / out_dim, o = (size_t)t % out_dim;
        out[t] = reference_one(x + row * in_dim, o, in_dim, bpr, weight_bytes, weight_scales);
    }
    used = threads;
#else
    (void)threads;
    for (long t = 0; t < total; ++t) {
        size_t row = (size_t)t / out_dim, o = (size_t)t % out_dim;
        out[t] = reference_one(x + row * in_dim, o, in_dim, bpr, weight_bytes, weight_scales);
    }
#endif
    return used;
}

/* ---- W8A8 ----------------------------------------------------------------- */

void oracle_rowwise_qdq_w8a8(const float *x, size_t m, size_t in_dim, float *out) {
    for (size_t row = 0; row < m; ++row) {
        const float *xr = x + row * in_dim;
        float *orow = out + row * in_dim;
        float max_abs = 0.0f;
        for (size_t c = 0; c < in_dim; ++c) max_abs = fmaxf(max_abs, fabsf(xr[c]));
        float inv_scale = (max_abs < 1e-8f) ? 1.0f : 127.0f / max_abs;
        for (size_t c = 0; c < in_dim; ++c) {
            float q = roundf(xr[c] * inv_scale); /* f32::round: half away from zero */
            if (q < -127.0f) q = -127.0f;        /* f32::clamp keeps NaN */
            if (q > 127.0f) q = 127.0f;
            orow[c] = q / inv_scale;
        }
    }
}

void oracle_iq2xxs_matmul_reference_w8a8(const float *x, size_t m, size_t out_dim, size_t in_dim,
                                         const uint8_t *weight_bytes, const uint8_t *weight_scales,
                                         float *out) {
    /* Workspace on the stack is not an option for big rows; the caller-sized
     * heap buffer keeps this a faithful two-step restatement. */
    size_t n = m * in_dim;
    float *xq = (float *)malloc(n * sizeof(float));
    if (!xq) return;
    oracle_rowwise_qdq_w8a8(x, m, in_dim, xq);
    oracle_iq2xxs_matmul_reference(xq, m, out_dim, in_dim, weight_bytes, weight_scales, out);
    free(xq);
}

/* ---- dequantize ------------------------------------------------------------ */

/* decode_iq2_xxs_value, iq2_matmul.metal:701-734: dl * gv * sgn with
 * dl = d * (0.5 + s) * 0.25, evaluated left to right in fp32. */
static float decode_value(const uint8_t *wb, const uint8_t *ws, size_t block_idx, size_t local_col) {
    size_t byte_base = block_idx * ORACLE_XXS_BYTES_PER_BLOCK;
    float d = oracle_f16_to_f32(read_u16_le(ws + block_idx * ORACLE_XXS_SCALES_PER_BLOCK));
    size_t ib32 = local_col / 32, within = local_col % 32, g = within / 8, j = within % 8;
    size_t q2 = byte_base + ib32 * 8;
    uint32_t aux_g = (uint32_t)read_u16_le(wb + q2) | ((uint32_t)read_u16_le(wb + q2 + 2) << 16);
    uint32_t aux_s = (uint32_t)read_u16_le(wb + q2 + 4) | ((uint32_t)read_u16_le(wb + q2 + 6) << 16);
    float dl = d * (0.5f + (float)((aux_s >> 28) & 0xFu));
    dl = dl * 0.25f;
    uint8_t gv = (uint8_t)((g_grid[(aux_g >> (8 * g)) & 0xFFu] >> (8 * j)) & 0xFFu);
    uint8_t signs = g_ksigns[(aux_s >> (7 * g)) & 0x7Fu];
    float sgn = (signs & g_kmask[j]) ? -1.0f : 1.0f;
    float v = dl * (float)gv;
    return v * sgn;
}

void oracle_iq2xxs_dequantize_f32(const uint8_t *weight_bytes, const uint8_t *weight_scales,
                                  size_t out_dim, size_t in_dim, float *out) {
    build_tables();
    size_t bpr = (in_dim + ORACLE_QK - 1) / ORACLE_QK;
    for (size_t o = 0; o < out_dim; ++o)
        for (size_t c = 0; c < in_dim; ++c)
            out[o * in_dim + c] =
                decode_value(weight_bytes, weight_scales, o * bpr + c / ORACLE_QK, c % ORACLE_QK);
}

void oracle_iq2xxs_dequantize_f16(const uint8_t *weight_bytes, const uint8_t *weight_scales,
                                  size_t out_dim, size_t in_dim, uint16_t *out) {
    build_tables();
    size_t bpr = (in_dim + ORACLE_QK - 1) / ORACLE_QK;
    for (size_t o = 0; o < out_dim; ++o)
        for (size_t c = 0; c < in_dim; ++c)
            out[o * in_dim + c] = oracle_f32_to_f16(
                decode_value(weight_bytes, weight_scales, o * bpr + c / ORACLE_QK, c % ORACLE_QK));
}

void oracle_iq2xxs_dequantize_bf16(const uint8_t *weight_bytes, const uint8_t *weight_scales,
                                   size_t out_dim, size_t in_dim, uint16_t *out) {
    build_tables();
    size_t bpr = (in_dim + ORACLE_QK - 1) / ORACLE_QK;
    for (size_t o = 0; o < out_dim; ++o)
        for (size_t c = 0; c < in_dim; ++c)
            out[o * in_dim + c] = oracle_f32_to_bf16(
                decode_value(weight_bytes, weight_scales, o * bpr + c / ORACLE_QK, c % ORACLE_QK));
}

/* ---- fp64 metric helper ----------------------------------------------------- */

void oracle_iq2xxs_matmul_f64(const float *x, size_t m, size_t out_dim, size_t in_dim,
                              const uint8_t *weight_bytes, const uint8_t *weight_scales,
                              double *out, double *abs_scale) {
    build_tables();
    size_t bpr = (in_dim + ORACLE_QK - 1) / ORACLE_QK;
    for (size_t row = 0; row < m; ++row) {
        const float *xr = x + row * in_dim;
        for (size_t o = 0; o < out_dim; ++o) {
            double acc = 0.0, sc = 0.0;
            for (size_t c = 0; c < in_dim; ++c) {
                /* the dequantized weight is an exact fp32 value (<= 22 significant bits) */
                double w = (double)decode_value(weight_bytes, weight_scales, o * bpr + c / ORACLE_QK,
                                                c % ORACLE_QK);
                double p = (double)xr[c] * w;
                acc += p;
                sc += fabs(p);
            }
            out[row * out_dim + o] = acc;
            if (abs_scale) abs_scale[row * out_dim + o] = sc;
        }
    }
}
