// iq2xxs_device.h — device-side helpers shared by the gfx950 IQ2_XXS kernels.
//
// All kernels expand the compact codebook (iq2xxs_format.h) into LDS at
// launch, so no global table exists and no table is read from HBM.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "iq2xxs_format.h"

namespace cmk {

// Per-translation-unit device copy of the codebook codes.
static __constant__ uint16_t kGridCodesDev[256] = {CMK_IQ2XXS_GRID_CODES};

// Codebook entry e as 8 magnitude bytes (little-endian u64: byte j = weight j).
__device__ __forceinline__ uint64_t expand_grid_entry(int e) {
  uint32_t c = kGridCodesDev[e];
  uint64_t v = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    uint32_t code = (c >> (2 * j)) & 3u;
    uint32_t lvl = code == 0 ? 8u : (code == 1 ? 25u : 43u);
    v |= (uint64_t)lvl << (8 * j);
  }
  return v;
}

// Byte mask of the sign pattern ksigns(i): byte j = 0xFF where weight j is negative.
__device__ __forceinline__ uint64_t expand_sign_mask(int i) {
  uint32_t s = (uint32_t)i | ((__popc((uint32_t)i) & 1u) << 7);
  uint64_t v = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (s & (1u << j)) v |= (uint64_t)0xFF << (8 * j);
  return v;
}

// Fill the LDS grid (256 x u64) and sign-mask (128 x u64) tables cooperatively.
__device__ __forceinline__ void build_lds_tables(uint64_t* lds_grid, uint64_t* lds_smask, int tid,
                                                 int nthreads) {
  for (int e = tid; e < 256 + 128; e += nthreads) {
    if (e < 256)
      lds_grid[e] = expand_grid_entry(e);
    else
      lds_smask[e - 256] = expand_sign_mask(e - 256);
  }
}

// Signed int8 weights of one group of 4 columns: magnitudes G (4 bytes) with the
// bytes selected by M (0xFF) negated.  Per byte: (g ^ 0xFF) + 1 = -g, and since
// g <= 43 the +1 never carries out of its byte.
__device__ __forceinline__ uint32_t apply_signs(uint32_t g, uint32_t m) {
  return (g ^ m) + (m & 0x01010101u);
}

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
  return __half2float(__ushort_as_half(h));
}

__device__ __forceinline__ float bf16_bits_to_float(uint16_t h) {
  return __uint_as_float((uint32_t)h << 16);
}

// Load element i of x (dtype 0 = f32, 1 = f16, 2 = bf16) as fp32.
__device__ __forceinline__ float load_x(const void* x, int dtype, size_t i) {
  if (dtype == 0) return static_cast<const float*>(x)[i];
  uint16_t h = static_cast<const uint16_t*>(x)[i];
  return dtype == 1 ? half_bits_to_float(h) : bf16_bits_to_float(h);
}

// W8A8 fake quantisation of one activation (src/metal_src/iq2_matmul.metal:98-102):
// q = clamp(round_half_away(x * inv), -127, 127); return q / inv.
__device__ __forceinline__ float qdq_w8a8(float x, float inv_scale) {
  float q = roundf(x * inv_scale);
  q = fminf(fmaxf(q, -127.0f), 127.0f);
  return q / inv_scale;
}

// ---------------------------------------------------------------------------
// Activation digits for the int8 MFMA GEMV.
//
// A 32-column chunk of fp32 activations with max |x| < 2^e is mapped to
// integers v = rint(x * 2^(22-e)), |v| <= 2^22.  u = v + 2^23 is a 24-bit
// unsigned value; its bytes b0,b1,b2 give signed digits s_k = b_k - 128, i.e.
// the bytes of D = u ^ 0x808080 read as int8.  Then
//     v = 65536*s2 + 256*s1 + s0 + 32896,   32896 = 128*(65536+256+1) - 2^23,
// exactly, so sum_k v_k w_k = 65536*C2 + 256*C1 + C0 + 32896*sum_k w_k where
// C_p = sum_k s_p,k w_k.  The MFMA forms C0..C2 from three digit planes and
// sum_k w_k from a fourth plane of ones.
// The chunk scale 2^(e-22) is kept as a float per chunk.
// ---------------------------------------------------------------------------
constexpr int kDigitShift = 22;
constexpr int kDigitOffset = 32896;  // 128 * (65536 + 256 + 1) - 2^23

__device__ __forceinline__ uint32_t digitize(float x, int e) {
  int v = __float2int_rn(ldexpf(x, kDigitShift - e));
  return ((uint32_t)(v + (1 << 23))) ^ 0x808080u;
}

}  // namespace cmk
