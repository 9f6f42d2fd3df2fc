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

// Codebook entry with level codes `c` (2 bits per byte) as 8 magnitude bytes
// (little-endian u64: byte j = weight j).
__device__ __forceinline__ uint64_t grid_entry_from_code(uint32_t c) {
  uint64_t v = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t code = (c >> (2 * j)) & 3u;
    const uint32_t lvl = code == 0 ? 8u : (code == 1 ? 25u : 43u);
    v |= (uint64_t)lvl << (8 * j);
  }
  return v;
}

__device__ __forceinline__ uint64_t expand_grid_entry(int e) {
  return grid_entry_from_code(kGridCodesDev[e]);
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

// This thread's codebook word (0 for tid >= 256).  Kernels that want the
// codebook read issued before their other loads fetch it first: global loads
// return in order, so a later wait on it does not wait for loads issued after.
__device__ __forceinline__ uint32_t fetch_grid_code(uint32_t tid) {
  return tid < 256 ? kGridCodesDev[tid] : 0u;
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

// Raw bits of element i of x for a dtype known at compile time (no branches,
// so the load's result is not waited for until it is used).
template <int XD>
__device__ __forceinline__ uint32_t load_x_bits(const void* x, size_t i) {
  if constexpr (XD == 0)
    return static_cast<const uint32_t*>(x)[i];
  else
    return static_cast<const uint16_t*>(x)[i];
}

template <int XD>
__device__ __forceinline__ float x_bits_to_float(uint32_t b) {
  if constexpr (XD == 0)
    return __uint_as_float(b);
  else if constexpr (XD == 1)
    return half_bits_to_float((uint16_t)b);
  else
    return bf16_bits_to_float((uint16_t)b);
}

// silu(g) * u = g / (1 + exp(-g)) * u in fp32: the step between a gated MLP's
// gate/up and down projections.  The swiglu kernel and the matmul epilogues
// that fold the step in evaluate this same expression, so both routes give the
// same bits.
__device__ __forceinline__ float silu_mul(float g, float u) {
  return (g / (1.0f + expf(-g))) * u;
}


// Eight consecutive activations x[base + c0 .. +8) as raw bits.  A task that
// is out of range issues no load at all (its registers stay undefined) and
// in-range elements are never selected right after the load: the validity
// mask is applied in get(), at the point of use, so that nothing forces the
// wave to wait for the load early.  kVec: the 8 elements are 16-byte aligned
// and in_dim % 8 == 0, so they go out as one (16-bit types) or two (f32)
// 16-byte loads.
template <int XD, bool kVec>
struct XOctet {
  uint32_t raw[kVec && XD != 0 ? 4 : 8];
  uint32_t okmask;  // bit k: element k is in range

  __device__ __forceinline__ void load(const void* x, size_t base, uint32_t c0, uint32_t in_dim,
                                       bool valid) {
    if constexpr (kVec) {
      okmask = valid ? 0xFFu : 0u;
      if (valid) {
        if constexpr (XD == 0) {
          const uint4* p = reinterpret_cast<const uint4*>(static_cast<const float*>(x) + base + c0);
          const uint4 a = p[0], b = p[1];
          raw[0] = a.x; raw[1] = a.y; raw[2] = a.z; raw[3] = a.w;
          raw[4] = b.x; raw[5] = b.y; raw[6] = b.z; raw[7] = b.w;
        } else {
          const uint4 a =
              *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + base + c0);
          raw[0] = a.x; raw[1] = a.y; raw[2] = a.z; raw[3] = a.w;
        }
      }
    } else {
      okmask = 0;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const bool ok = valid && c0 + k < in_dim;
        okmask |= ok ? (1u << k) : 0u;
        if (ok) raw[k] = load_x_bits<XD>(x, base + c0 + k);
      }
    }
  }

  // Blocks until the loads of this octet have returned (an empty asm that
  // reads the registers; the compiler places the wait in front of it).
  __device__ __forceinline__ void wait_arrived() const {
#pragma unroll
    for (int k = 0; k < (int)(sizeof(raw) / sizeof(raw[0])); ++k) asm volatile("" ::"v"(raw[k]));
  }

  __device__ __forceinline__ float get(int k) const {
    uint32_t b;
    if constexpr (kVec && XD != 0)
      b = (k & 1) ? (raw[k >> 1] >> 16) : (raw[k >> 1] & 0xFFFFu);
    else
      b = raw[k];
    const float v = x_bits_to_float<XD>(b);
    return ((okmask >> k) & 1u) ? v : 0.0f;
  }
};

// The exact fp32 weight at (row, col), evaluated as the reference does:
// (d * (0.5 + s) * 0.25) * g, negated under its sign bit
// (src/iq2_matmul.rs:853-866 with accum_word_grid :789-809;
// iq2_matmul.metal:8-28,201-232).  Byte loads, any alignment.
__device__ inline float iq2xxs_weight_at(const uint8_t* wb, const uint8_t* ws, uint32_t row,
                                         uint32_t col, uint32_t bpr) {
  const size_t block = (size_t)row * bpr + col / kQK;
  const uint32_t ib32 = (col % kQK) / 32, g = (col % 32) / 8, j = col % 8;
  const uint8_t* q = wb + block * kBytesPerBlock + ib32 * 8;
  const uint32_t aux_s =
      (uint32_t)q[4] | ((uint32_t)q[5] << 8) | ((uint32_t)q[6] << 16) | ((uint32_t)q[7] << 24);
  const uint8_t* sp = ws + block * kScalesPerBlock;
  const float d = half_bits_to_float((uint16_t)(sp[0] | (sp[1] << 8)));
  const float dl = d * (0.5f + (float)(aux_s >> 28)) * 0.25f;
  const uint32_t sidx = (aux_s >> (7 * g)) & 127u;
  const uint32_t sbyte = sidx | ((__popc(sidx) & 1u) << 7);
  const uint32_t code = ((uint32_t)kGridCodesDev[q[g]] >> (2 * j)) & 3u;
  const float mag = dl * (code == 0 ? 8.0f : (code == 1 ? 25.0f : 43.0f));
  return ((sbyte >> j) & 1u) ? -mag : mag;
}

// Activations that are NaN or infinite.  The digit paths hold x as finite
// integers, so those values are set aside: they enter the digits as zeros, and
// the sum over them, x_c * w_rc, is added to each output afterwards.  Every
// such term is NaN or an infinity, so the sum only depends on which kinds
// occur, never on their order:
//   NaN term, or infinities of both signs -> NaN; otherwise the infinity;
// and a finite partial sum plus that value is what the reference's
// sequential fp32 loop yields (src/iq2_matmul.rs:789-809).
constexpr uint32_t kAbsMask = 0x7FFFFFFFu;
constexpr uint32_t kInfBits = 0x7F800000u;  // |x| bits at or above: not finite
constexpr uint32_t kSpecialNaN = 1u, kSpecialPosInf = 2u, kSpecialNegInf = 4u;

__device__ __forceinline__ uint32_t special_kind(float t) {
  return t != t ? kSpecialNaN : (t > 0.0f ? kSpecialPosInf : kSpecialNegInf);
}

// The sum of the set-aside terms of an output from the kinds that occurred
// (0 when none did).
__device__ __forceinline__ float special_value(uint32_t kinds) {
  if ((kinds & kSpecialNaN) || (kinds & (kSpecialPosInf | kSpecialNegInf)) ==
                                   (kSpecialPosInf | kSpecialNegInf))
    return __uint_as_float(0x7FC00000u);
  if (kinds & kSpecialPosInf) return __uint_as_float(kInfBits);
  if (kinds & kSpecialNegInf) return -__uint_as_float(kInfBits);
  return 0.0f;
}

// W8A8 quantisation of one activation (src/iq2_matmul.rs:1025-1048,
// iq2_matmul.metal:98-102): q = clamp(round_half_away(x * inv), -127, 127), an
// integer in a float.  A NaN stays NaN, as in the reference's CPU path
// (f32::clamp); the Metal clamp (fmin/fmax) would give -127 instead.
__device__ __forceinline__ float quant_w8a8(float x, float inv_scale) {
  float q = roundf(x * inv_scale);
  q = q < -127.0f ? -127.0f : q;
  return q > 127.0f ? 127.0f : q;
}

// The reference's fake quantisation: q / inv.
__device__ __forceinline__ float qdq_w8a8(float x, float inv_scale) {
  return quant_w8a8(x, inv_scale) / inv_scale;
}

// ---------------------------------------------------------------------------
// Activation digits for the int8 MFMA GEMV.
//
// A 32-column chunk of activations with max|x| < 2^e is mapped to integers
// v = rint(x * 2^(D-e)), |v| <= 2^D (IQ2_XXS: D = kDigitShift = 22, the
// other formats 21).  The rounding is one fma against the magic constant
// 1.5*2^23: for |v| <= 2^22 the sum lies in [2^23, 2^24] and its bits are
// bits(1.5*2^23) + v exactly (v = 2^22 carries into the exponent field).
// u = v + 0x808080 is a 24-bit unsigned value whose bytes b0,b1,b2 give signed
// digits s_k = b_k - 128 (the bytes of D = u ^ 0x808080 read as int8) with
//     v = 65536*s2 + 256*s1 + s0      exactly,
// so sum_k v_k w_k = 65536*C2 + 256*C1 + C0 with C_p = sum_k s_p,k w_k, the
// three integer dot products the MFMA forms from three digit planes.  Over a
// 32-column sub-block with |w| <= 43 and D = 22 the sum passes 2^31
// (32*43*2^22), so the kernels form 256*C2 + C1 in int32 and add C0 in fp32.
// The chunk scale 2^(e-D) is kept as a float per chunk.
// ---------------------------------------------------------------------------
constexpr int kDigitShift = 22;
constexpr float kDigitMagic = 12582912.0f;       // 1.5 * 2^23
constexpr uint32_t kDigitBias = 0x4ABF7F80u;     // bits(1.5*2^23) - 0x808080

// Clamp of the chunk exponent so 2^(D-e) and 2^(e-D-3) stay finite and normal
// for digit widths D <= 22.
__device__ __forceinline__ int digit_exponent(float max_abs) {
  int e;
  (void)frexpf(max_abs, &e);
  return e < -100 ? -100 : e;
}

// The three digit bytes of x (bits 0..23) each plus 128, for chunk scale
// 2^(D-e): the bytes of v + 0x808080.
__device__ __forceinline__ uint32_t digitize_biased(float x, float scale) {
  const uint32_t bits = __float_as_uint(fmaf(x, scale, kDigitMagic));
  return bits - kDigitBias;
}

// Three signed digit bytes (bits 0..23) of x for chunk exponent e.
__device__ __forceinline__ uint32_t digitize(float x, float scale) {
  return digitize_biased(x, scale) ^ 0x808080u;
}

// Transpose the digit bytes of 4 values into one dword per plane.
__device__ __forceinline__ void digits_to_planes(uint32_t d0, uint32_t d1, uint32_t d2, uint32_t d3,
                                                 uint32_t& p0, uint32_t& p1, uint32_t& p2) {
  // v_perm_b32(s0, s1, sel): bytes 0-3 of the pool are s1, bytes 4-7 are s0.
  const uint32_t a = __builtin_amdgcn_perm(d1, d0, 0x05010400u);  // d0.b0 d1.b0 d0.b1 d1.b1
  const uint32_t b = __builtin_amdgcn_perm(d3, d2, 0x05010400u);  // d2.b0 d3.b0 d2.b1 d3.b1
  p0 = __builtin_amdgcn_perm(b, a, 0x05040100u);
  p1 = __builtin_amdgcn_perm(b, a, 0x07060302u);
  const uint32_t c = __builtin_amdgcn_perm(d1, d0, 0x0c0c0602u);  // d0.b2 d1.b2
  const uint32_t f = __builtin_amdgcn_perm(d3, d2, 0x0c0c0602u);  // d2.b2 d3.b2
  p2 = __builtin_amdgcn_perm(f, c, 0x05040100u);
}

// (g ^ m) + (m & 0x01010101): magnitudes g negated where the byte mask m is 0xFF
// (per byte (g ^ 0xFF) + 1 = -g; g <= 43 so the +1 never carries).  The
// compiler selects v_and + v_xad_u32 for it.  Kept in plain C on purpose: the
// result feeds v_mfma, and only compiler-visible instructions get the
// VALU-write -> MFMA-read wait states inserted.
__device__ __forceinline__ uint32_t apply_signs(uint32_t g, uint32_t m) {
  return (g ^ m) + (m & 0x01010101u);
}

}  // namespace cmk
