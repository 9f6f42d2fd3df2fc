// iq2xxs_gemv_common.h — pieces shared by the decode-shaped IQ2_XXS kernels
// (iq2xxs_gemv.hip: one activation row; iq2xxs_gemv_rows.hip: up to 16 rows,
// W8A8 32):
// the LDS expansion tables of the codebook and sign masks, LDS and buffer
// access helpers, and the activation loads of a digitisation task.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "iq2xxs_device.h"

namespace cmk {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kGemvLdsLimit = 160 * 1024;
// Buffer offset past every num_records used here (buffers are < 2^31 bytes).
constexpr uint32_t kOutOfRange = 0x80000000u;
// Word 3 of a gfx9 raw buffer resource (32-bit data format, no swizzle).
constexpr int kBufferWord3 = 0x00020000;
// Cache policy of the weight loads: nontemporal (read once).
constexpr int kStreamLoad = 2;

// Table layouts at LDS offset 0.
//  wide:   [0, 64K)   codebook row e (256 B) = 16 copies of {g lo, g hi, -g lo, -g hi}
//          [64K, 80K) sign row i (128 B) = 16 copies of the 8-byte mask of ksigns(i);
//          the 128-byte stride puts the index of sign field g (bits 7g..7g+6
//          of aux_s) at address bits 7..13 with one shift and one v_and_or
//          (field 1 needs no shift)
//  narrow: [0, 64K)   row r (256 B): bytes [0,128) 8 codebook copies of entry r,
//          bytes [128, 256) 16 copies of the sign mask of ksigns(r & 127); the
//          sign index then needs no masking (a byte of aux_s << g carries one
//          unrelated bit on top), at the price of 2-way bank conflicts.
// Lane l reads copy l & 15 of a row, so the 16 lanes the LDS serves together
// hit 16 different bank groups (measured on gfx950 with 16 waves: about 3.0
// clocks per wave-wide 16-byte read with 16 copies against 4.9 with 8, and
// 2.6 per 8-byte read with 16 copies against 2.4 with 32).
template <bool kWide>
struct GemvTables {
  static constexpr uint32_t kBytes = kWide ? 80 * 1024 : 64 * 1024;
  static constexpr uint32_t kGridCopies = kWide ? 16 : 8;
  static constexpr uint32_t kSignCopies = 16;
  static constexpr uint32_t kSignBase = kWide ? 65536 : 128;
  static constexpr uint32_t kSignStride = kWide ? 128 : 256;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes,
                                           kBufferWord3);
}

// Four level codes (2 bits each, x4 = bits 0..7) as four magnitude bytes
// {8, 25, 43}: the codes are spread to one per byte with two multiplies
// (fields 0 and 2, and fields 1 and 3, land in disjoint bits), then select
// from the byte pool {8, 25, 43, 0} with one v_perm.
__device__ __forceinline__ uint32_t level_bytes(uint32_t x4) {
  const uint32_t even = ((x4 & 0x33u) * 0x1001u) & 0x00030003u;   // codes 0, 2 -> bytes 0, 2
  const uint32_t odd = ((x4 & 0xCCu) * 0x40040u) & 0x03000300u;   // codes 1, 3 -> bytes 1, 3
  return __builtin_amdgcn_perm(0u, 0x002B1908u, even | odd);
}

// Bit j of the nibble n as byte j of the result: 0xFF where set.  The nibble's
// copies at shifts 0, 7, 14, 21 do not overlap, so the multiply places bit j at
// bit 8j without carries.
__device__ __forceinline__ uint32_t byte_mask4(uint32_t n) {
  const uint32_t t = (n * 0x00204081u) & 0x01010101u;
  return (t << 8) - t;
}

// All copies of codebook row e (code c: 2-bit level codes of its 8 bytes); the
// copy order is rotated by e so the 16 lanes the LDS serves together write 16
// different bank groups.
template <bool kWide>
__device__ __forceinline__ void store_grid_row(uint8_t* lds, uint32_t e, uint32_t c) {
  const uint32_t lo = level_bytes(c & 0xFFu), hi = level_bytes(c >> 8);
  // per-byte negation: (~g) + 1 never carries across bytes since g >= 8
  const u32x4 v = {lo, hi, ~lo + 0x01010101u, ~hi + 0x01010101u};
  constexpr uint32_t C = GemvTables<kWide>::kGridCopies;
  const uint32_t row = e * 256, rot = 16 * e;
  // (a short unroll: callers hold many live registers while they build tables)
#pragma unroll 2
  for (uint32_t k = 0; k < C; ++k)
    *reinterpret_cast<u32x4*>(lds + (row | ((rot + 16 * k) & (16 * C - 16)))) = v;
}

// The 8-byte mask of ksigns(i) = i | parity(i) << 7.
__device__ __forceinline__ u32x2 sign_mask(uint32_t i) {
  const uint32_t sb = i | ((__popc(i) & 1u) << 7);
  return u32x2{byte_mask4(sb & 0xFu), byte_mask4(sb >> 4)};
}

// Copies [k0, k0 + n) of sign row i (rotated like the codebook rows).
template <bool kWide>
__device__ __forceinline__ void store_sign_row(uint8_t* lds, uint32_t i, u32x2 v, uint32_t k0,
                                               uint32_t n) {
  using TL = GemvTables<kWide>;
  constexpr uint32_t C = TL::kSignCopies;
  uint8_t* const row = lds + TL::kSignBase + i * TL::kSignStride;
#pragma unroll 2
  for (uint32_t k = k0; k < k0 + n; ++k)
    *reinterpret_cast<u32x2*>(row + 8 * ((k + i) & (C - 1))) = v;
}

// Table address  256 * byte G of w + low byte of cbase  as one v_perm
// (result bytes: cbase.b0, w.bG, 0, 0).
template <int G>
__device__ __forceinline__ uint32_t perm_addr(uint32_t w, uint32_t cbase) {
  return __builtin_amdgcn_perm(w, cbase, 0x0C0C0000u | ((0x04u + G) << 8));
}

// LDS reads at byte addresses (the kernel's dynamic LDS starts at 0).
__device__ __forceinline__ u32x2 lds_u2(uint32_t addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) u32x2*>(
      static_cast<uintptr_t>(addr));
}
__device__ __forceinline__ uint32_t lds_u16(uint32_t addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) uint16_t*>(
      static_cast<uintptr_t>(addr));
}
__device__ __forceinline__ u32x4 lds_u4(uint32_t addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
      static_cast<uintptr_t>(addr));
}

// Bits of a where m is set, of b elsewhere (one v_bitop3 on gfx950).  Kept in
// plain C: the result feeds v_mfma, and only compiler-visible instructions
// get the VALU-write -> MFMA-read wait states inserted.
__device__ __forceinline__ uint32_t bit_select(uint32_t m, uint32_t a, uint32_t b) {
  return (m & a) | (~m & b);
}

// Max over the 4 lanes of an aligned quad (DPP quad_perm [1,0,3,2], [2,3,0,1]).
__device__ __forceinline__ uint32_t quad_max_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
  return max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
}

// Eight consecutive activations (one digitisation task) by buffer loads.  An
// absent task or element reads at an offset past the buffer and gets zeros,
// with no branch, so the count of outstanding loads is the same on every path.
// kVec: the 8 elements are 16-byte aligned and in_dim % 8 == 0.
template <int XD, bool kVec>
struct XTask {
  static constexpr uint32_t kRegs = (kVec && XD != 0) ? 4 : 8;
  uint32_t raw[kRegs];

  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rx, uint32_t elem0, uint32_t c0,
                                       uint32_t in_dim, bool valid) {
    constexpr uint32_t es = XD == 0 ? 4 : 2;
    if constexpr (kVec) {
      const uint32_t off = valid ? elem0 * es : kOutOfRange;
      const u32x4 v0 = __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0);
      raw[0] = v0.x; raw[1] = v0.y; raw[2] = v0.z; raw[3] = v0.w;
      if constexpr (XD == 0) {
        const u32x4 v1 = __builtin_amdgcn_raw_buffer_load_b128(rx, off + 16, 0, 0);
        raw[4] = v1.x; raw[5] = v1.y; raw[6] = v1.z; raw[7] = v1.w;
      }
    } else {
#pragma unroll
      for (uint32_t k = 0; k < 8; ++k) {
        const uint32_t off = (valid && c0 + k < in_dim) ? (elem0 + k) * es : kOutOfRange;
        if constexpr (XD == 0)
          raw[k] = __builtin_amdgcn_raw_buffer_load_b32(rx, off, 0, 0);
        else
          raw[k] = __builtin_amdgcn_raw_buffer_load_b16(rx, off, 0, 0);
      }
    }
  }

  __device__ __forceinline__ float get(int k) const {
    uint32_t b;
    if constexpr (kVec && XD != 0)
      b = (k & 1) ? (raw[k >> 1] >> 16) : (raw[k >> 1] & 0xFFFFu);
    else
      b = raw[k];
    return x_bits_to_float<XD>(b);
  }
};

}  // namespace cmk
