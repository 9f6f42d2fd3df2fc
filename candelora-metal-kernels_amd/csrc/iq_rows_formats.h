// iq_rows_formats.h — the per-format parts of the multi-row decode kernel
// (iq2xxs_gemv_rows.hip): LDS tables, the loads of a unit (32 weight rows x
// half a super-block), and the expansion of a lane's codes into signed int8
// weights for the MFMA.
//
// Activation digits have F::kDigitShift bits (at most 22, the widest the
// magic-number digitisation gives: |rint| <= 2^22 keeps fma(x, 2^(D-e),
// 1.5 * 2^23) in [2^23, 2^24], where its bits are 0x4B400000 + rint).  The
// plane sums of one MFMA, (columns) x 2^kDigitShift x (largest code
// magnitude), are combined in int32 where they stay below 2^31, and as
// 256 * (256 C2 + C1) + C0 in fp32 otherwise (F::kSplitSum).
//
// Every format's weight is w = dl * g * sign with g a small odd or level
// magnitude (IQ2: {8, 25, 43}; IQ3_S: odd 1..15) and dl = d * (2s+1) / 8
// (IQ2_*), d * (2s+1) (IQ3_S) for a 4-bit sub-scale s.  The kernel multiplies
// the int8 values +-g against the activation digits exactly and applies
// (2s+1) and d in fp32.  Formats whose sub-scale covers 16 weights (IQ2_XS,
// IQ2_S) run one v_mfma_i32_32x32x16_i8 per 16 columns ("half" formats); the
// others one v_mfma_i32_32x32x32_i8 per 32-column sub-block.
//
// Scales: the kernel stages each K slice's scale bytes for the workgroup's
// rows in LDS (coalesced), and fill_scales reads a unit's d and sub-scales
// from there (`addr`: the LDS address of the row's block scales); loading
// them per unit from global memory took one wave-wide load per field, each
// touching 32 rows' lines for 2 bytes.
//
// Lane roles: lane l = 32 h + n holds weight row n of the unit.  In a
// 32-column MFMA it supplies columns 16 h .. 16 h + 15 of the sub-block
// (groups 2h and 2h+1 of 8 weights); in a 16-column MFMA of half hf it
// supplies columns 16 hf + 8 h .. + 7 (group 2 hf + h).  A lane loads half of
// its row's bytes of the unit and v_permlane32_swap hands each lane the other
// half, so every lane ends up with its row's codes for all 4 sub-blocks.
//
// Byte layouts (src/iq2_matmul.rs:884-1016; iq2_matmul.metal:8-28, 242-434):
//   IQ2_XXS 64 B / 2 B per block: sub-block b = aux_g (4 grid bytes) and
//           aux_s (4 x 7-bit ksigns indices, scale in bits 28-31) at 8 b.
//   IQ2_XS  64 B / 10 B: sub-block b = four LE u16 at 8 b (grid index bits
//           0-8, ksigns index bits 9-15); scales: d, then byte 2 + b (low
//           nibble groups 0-1, high nibble groups 2-3).
//   IQ2_S   72 B / 10 B: grid low bytes qs[4 b + g], sign bytes at 32 + 4 b +
//           g, grid high bits (qh[64 + b] >> 2 g) & 3; scales as IQ2_XS.
//   IQ3_S   104 B / 6 B: grid low bytes qs[8 b + 2 g], qs[8 b + 2 g + 1] (two
//           4-value entries per group), high bits (qh[64 + b] >> 2 g) & 1 and
//           >> (2 g + 1) & 1, sign bytes at 72 + 4 b + g; scale nibble b & 1 of
//           byte 2 + b / 2.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "iq2xxs_device.h"
#include "iq2xxs_gemv_common.h"
#include "iq_variants_format.h"

namespace cmk {

// Cache policy of the unit loads: default.  A unit reads 32 bytes of each of
// 32 rows, so the four units of a 128-byte line come from four waves; with
// the nontemporal hint a line could leave the cache between them (M=4, N=14336:
// 12.5 us with the hint, 11.5 us without).
constexpr int kUnitLoad = 0;

static __constant__ uint16_t kRowsXsCodes[512] = {CMK_IQ2XS_GRID_CODES};
static __constant__ uint16_t kRowsSCodes[1024] = {CMK_IQ2S_GRID_CODES};
static __constant__ uint16_t kRowsS3Codes[512] = {CMK_IQ3S_GRID_CODES};

// C copies of an entry (row of C * S bytes at `row`), copy k stored at slot
// (k + entry) mod C so the 16 lanes the LDS serves together write 16
// different bank groups.
template <uint32_t C, typename T>
__device__ __forceinline__ void store_copies(uint8_t* row, uint32_t entry, T v, uint32_t k0,
                                             uint32_t n) {
#pragma unroll 2
  for (uint32_t k = k0; k < k0 + n; ++k)
    *reinterpret_cast<T*>(row + sizeof(T) * ((k + entry) & (C - 1))) = v;
}

// The 8-byte mask of an explicit sign byte: byte j = 0xFF where bit j is set.
__device__ __forceinline__ u32x2 byte_sign_mask(uint32_t b) {
  return u32x2{byte_mask4(b & 0xFu), byte_mask4(b >> 4)};
}

// {g, -g} for one dword of magnitudes (per byte: (~g) + 1 never carries, g >= 1).
__device__ __forceinline__ uint32_t neg_bytes(uint32_t g) { return ~g + 0x01010101u; }

// Magnitude bytes of an IQ3_S entry (3-bit codes (v-1)/2 of 4 values).
__device__ __forceinline__ uint32_t iq3_bytes(uint32_t c) {
  uint32_t v = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) v |= (2u * ((c >> (3 * j)) & 7u) + 1u) << (8 * j);
  return v;
}

__device__ __forceinline__ uint32_t swap_lo(uint32_t v) {
  return __builtin_amdgcn_permlane32_swap(v, v, false, false)[0];
}

// ---------------------------------------------------------------------------
// IQ2_XXS: tables as the one-row kernel's wide layout (80 KB).
// ---------------------------------------------------------------------------
struct RowsFmtXXS {
  static constexpr bool kHalf = false;
  // activation digits of 22 bits: 32 columns x 2^22 x 43 pass 2^31, so the
  // planes combine as 256 * (256 C2 + C1) + C0: the inner sum is exact in
  // int32 (|C2| <= 32 x 64 x 43, below 2^25) and is converted and added to C0
  // with two fp32 roundings of 2^-24 relative, against the digits' 2^-23
  static constexpr int kDigitShift = 22;
  static constexpr bool kSplitSum = true;
  static constexpr uint32_t kTableBytes = GemvTables<true>::kBytes;
  static constexpr uint32_t kBlockBytes = 64, kScaleBytes = 2;
  struct Consts {
    uint32_t cg, cs, sel0, sel1, rot0, rot1, k27;
  };
  struct Unit {
    u32x4 q;
    uint32_t d;
  };
  struct Words {
    uint32_t g[4], s[4];
  };

  __device__ static Consts consts(uint32_t lane) {
    const uint32_t h = lane >> 5;
    Consts k;
    k.cg = 16 * (lane & 15);
    k.cs = GemvTables<true>::kSignBase + 8 * (lane & 15);
    k.sel0 = 0x0C0C0000u | ((4u + 2u * h) << 8);  // codebook byte 2h of aux_g
    k.sel1 = k.sel0 + 0x100u;                       // byte 2h + 1
    k.rot0 = h ? 7u : 25u;                          // sign fields 2h, 2h + 1
    k.rot1 = h ? 14u : 0u;
    uint32_t k27 = 0x07FFFFFFu;
    asm volatile("" : "+v"(k27));
    k.k27 = k27;
    return k;
  }
  __device__ static uint32_t seed(uint32_t tid) { return tid < 256 ? kGridCodesDev[tid] : 0u; }
  __device__ static void tables(uint8_t* lds, uint32_t tid, uint32_t code) {
    if (tid < 256) {
      store_grid_row<true>(lds, tid, code);
    } else if (tid < 512) {
      const uint32_t i = (tid - 256) >> 1, half = tid & 1;
      store_sign_row<true>(lds, i, sign_mask(i), half * 8, 8);
    }
  }
  // Lane (n, h) of unit `half` of super-block sb: pair 2 half + h of row.
  __device__ static Unit load(__amdgpu_buffer_rsrc_t rw, bool ok, uint32_t blk, uint32_t half,
                              uint32_t h) {
    Unit u;
    const uint32_t off = ok ? blk * kBlockBytes + half * 32 + 16 * h : kOutOfRange;
    u.q = __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, kUnitLoad);
    return u;
  }
  __device__ static void fill_scales(Unit& u, uint32_t addr, uint32_t) { u.d = lds_u16(addr); }
  // d times the factor that cancels the 2^27 of pair_scale
  __device__ static float unit_scale(const Unit& u) {
    return half_bits_to_float((uint16_t)u.d) * 0x1p-27f;
  }
  // lane (n, 0) holds the unit's first pair, (n, 1) its second; swapping a
  // register with itself gives every lane both halves' values
  __device__ static Words unpack(const Unit& u) {
    Words w;
#pragma unroll
    for (uint32_t c = 0; c < 4; ++c) {
      const auto r = __builtin_amdgcn_permlane32_swap(u.q[c], u.q[c], false, false);
      const uint32_t j0 = c >> 1, j1 = j0 + 2;
      if (c & 1) {
        w.s[j0] = r[0];
        w.s[j1] = r[1];
      } else {
        w.g[j0] = r[0];
        w.g[j1] = r[1];
      }
    }
    return w;
  }
  // groups 2h and 2h + 1 of sub-block j as 16 signed bytes
  __device__ static v4i pair(const Words& w, uint32_t j, const Consts& k) {
    const uint32_t ga0 = __builtin_amdgcn_perm(w.g[j], k.cg, k.sel0);
    const uint32_t ga1 = __builtin_amdgcn_perm(w.g[j], k.cg, k.sel1);
    const uint32_t sa0 = (__builtin_amdgcn_alignbit(w.s[j], w.s[j], k.rot0) & 0x3F80u) | k.cs;
    const uint32_t sa1 = (__builtin_amdgcn_alignbit(w.s[j], w.s[j], k.rot1) & 0x3F80u) | k.cs;
    const u32x4 g0 = lds_u4(ga0), g1 = lds_u4(ga1);
    const u32x2 m0 = lds_u2(sa0), m1 = lds_u2(sa1);
    return v4i{(int)bit_select(m0.x, g0.z, g0.x), (int)bit_select(m0.y, g0.w, g0.y),
               (int)bit_select(m1.x, g1.z, g1.x), (int)bit_select(m1.y, g1.w, g1.y)};
  }
  // (2s+1) * 2^27: the conversion of s * 2^28 + 2^27 - 1 rounds to it exactly
  // (one v_and_or with the low constant in a register)
  __device__ static float pair_scale(const Words& w, uint32_t j, const Consts& k) {
    return (float)((w.s[j] & 0xF0000000u) | k.k27);
  }
  __device__ static float weight_at(const uint8_t* wb, const uint8_t* ws, uint32_t row,
                                    uint32_t col, uint32_t bpr) {
    return iq2xxs_weight_at(wb, ws, row, col, bpr);
  }
};

// ---------------------------------------------------------------------------
// IQ2_XS: grid rows (512 x 128 B) of 8 copies of {g, -g} at [0, 64K); the
// ksigns rows of the IQ2_XXS wide layout at [64K, 80K).
// ---------------------------------------------------------------------------
struct RowsFmtXS {
  static constexpr bool kHalf = true;
  // 21-bit digits: 16 columns x 2^21 x 43 stay below 2^31
  static constexpr int kDigitShift = 21;
  static constexpr bool kSplitSum = false;
  static constexpr uint32_t kTableBytes = 80 * 1024;
  static constexpr uint32_t kBlockBytes = 64, kScaleBytes = 10;
  struct Consts {
    uint32_t cg, cs, h16;
  };
  struct Unit {
    u32x4 q;
    uint32_t d, s01, s23;
  };
  struct Words {
    uint32_t lo[4], hi[4];  // u16 words 0-1 and 2-3 of each sub-block
    uint32_t sc;            // scale byte of sub-block j at bits 8j
  };

  __device__ static Consts consts(uint32_t lane) {
    return Consts{16 * (lane & 7), 65536u + 8 * (lane & 15), 16 * (lane >> 5)};
  }
  __device__ static uint32_t seed(uint32_t tid) { return tid < 512 ? kRowsXsCodes[tid] : 0u; }
  __device__ static void tables(uint8_t* lds, uint32_t tid, uint32_t code) {
    if (tid < 512) {
      const uint32_t lo = level_bytes(code & 0xFFu), hi = level_bytes(code >> 8);
      store_copies<8>(lds + tid * 128, tid, u32x4{lo, hi, neg_bytes(lo), neg_bytes(hi)}, 0, 8);
    } else if (tid < 768) {
      const uint32_t i = (tid - 512) >> 1, half = tid & 1;
      store_sign_row<true>(lds, i, sign_mask(i), half * 8, 8);
    }
  }
  __device__ static Unit load(__amdgpu_buffer_rsrc_t rw, bool ok, uint32_t blk, uint32_t half,
                              uint32_t h) {
    Unit u;
    const uint32_t off = ok ? blk * kBlockBytes + half * 32 + 16 * h : kOutOfRange;
    u.q = __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, kUnitLoad);
    return u;
  }
  // d, then the scale bytes of sub-blocks 4 half .. 4 half + 3
  __device__ static void fill_scales(Unit& u, uint32_t addr, uint32_t half) {
    u.d = lds_u16(addr);
    u.s01 = lds_u16(addr + 2 + 4 * half);
    u.s23 = lds_u16(addr + 4 + 4 * half);
  }
  __device__ static float unit_scale(const Unit& u) {
    return half_bits_to_float((uint16_t)u.d);
  }
  __device__ static Words unpack(const Unit& u) {
    Words w;
#pragma unroll
    for (uint32_t c = 0; c < 4; ++c) {
      const auto r = __builtin_amdgcn_permlane32_swap(u.q[c], u.q[c], false, false);
      const uint32_t j0 = c >> 1, j1 = j0 + 2;
      if (c & 1) {
        w.hi[j0] = r[0];
        w.hi[j1] = r[1];
      } else {
        w.lo[j0] = r[0];
        w.lo[j1] = r[1];
      }
    }
    w.sc = (u.s01 & 0xFFFFu) | (u.s23 << 16);
    return w;
  }
  // group 2 hf + h of sub-block j as 8 signed bytes
  __device__ static u32x2 group(const Words& w, uint32_t j, uint32_t hf, const Consts& k) {
    const uint32_t word = hf ? w.hi[j] : w.lo[j];
    const uint32_t ga = (__builtin_amdgcn_ubfe(word, k.h16, 9) << 7) | k.cg;
    const uint32_t sa = (__builtin_amdgcn_ubfe(word, k.h16 + 9, 7) << 7) | k.cs;
    const u32x4 g = lds_u4(ga);
    const u32x2 m = lds_u2(sa);
    return u32x2{bit_select(m.x, g.z, g.x), bit_select(m.y, g.w, g.y)};
  }
  __device__ static float group_scale(const Words& w, uint32_t j, uint32_t hf) {
    return (float)(2u * ((w.sc >> (8 * j + 4 * hf)) & 0xFu) + 1u);
  }
  __device__ static float weight_at(const uint8_t* wb, const uint8_t* ws, uint32_t row,
                                    uint32_t col, uint32_t bpr) {
    const size_t blk = (size_t)row * bpr + col / kQK;
    const uint32_t ib32 = (col % kQK) / 32, g = (col % 32) / 8, j = col % 8;
    const uint8_t* q = wb + blk * kBlockBytes + 8 * ib32 + 2 * g;
    const uint32_t qw = (uint32_t)q[0] | ((uint32_t)q[1] << 8);
    const uint8_t* sc = ws + blk * kScaleBytes;
    const float d = half_bits_to_float((uint16_t)(sc[0] | (sc[1] << 8)));
    const uint32_t nib = (sc[2 + ib32] >> (g < 2 ? 0 : 4)) & 0xFu;
    const float dl = d * (0.5f + (float)nib) * 0.25f;
    const uint32_t code = ((uint32_t)kRowsXsCodes[qw & 0x1FFu] >> (2 * j)) & 3u;
    const float mag = dl * (code == 0 ? 8.0f : (code == 1 ? 25.0f : 43.0f));
    const uint32_t sidx = qw >> 9;
    const uint32_t sb = sidx | ((__popc(sidx) & 1u) << 7);
    return ((sb >> j) & 1u) ? -mag : mag;
  }
};

// ---------------------------------------------------------------------------
// IQ2_S: grid rows (1024 x 64 B) of 4 copies of {g, -g} at [0, 64K); rows of
// 16 copies of the 8-byte mask of each sign byte (256 x 128 B) at [64K, 96K).
// ---------------------------------------------------------------------------
struct RowsFmtS {
  static constexpr bool kHalf = true;
  static constexpr int kDigitShift = 21;  // as IQ2_XS
  static constexpr bool kSplitSum = false;
  static constexpr uint32_t kTableBytes = 96 * 1024;
  static constexpr uint32_t kBlockBytes = 72, kScaleBytes = 10;
  struct Consts {
    uint32_t cg, cs, h8, h2;
  };
  struct Unit {
    u32x2 qs, sg;
    uint32_t qh, d, s01, s23;
  };
  struct Words {
    uint32_t qs[4], sg[4];  // grid low bytes and sign bytes of sub-block j
    uint32_t qh, sc;        // byte j: sub-block j's high bits / scale byte
  };

  __device__ static Consts consts(uint32_t lane) {
    const uint32_t h = lane >> 5;
    return Consts{16 * (lane & 3), 65536u + 8 * (lane & 15), 8 * h, 2 * h};
  }
  __device__ static uint32_t seed(uint32_t tid) { return kRowsSCodes[tid]; }
  __device__ static void tables(uint8_t* lds, uint32_t tid, uint32_t code) {
    // every thread: grid row tid, and a quarter of sign row tid / 4
    const uint32_t lo = level_bytes(code & 0xFFu), hi = level_bytes(code >> 8);
    store_copies<4>(lds + tid * 64, tid, u32x4{lo, hi, neg_bytes(lo), neg_bytes(hi)}, 0, 4);
    const uint32_t b = tid >> 2;
    store_copies<16>(lds + 65536 + b * 128, b, byte_sign_mask(b), 4 * (tid & 3), 4);
  }
  __device__ static Unit load(__amdgpu_buffer_rsrc_t rw, bool ok, uint32_t blk, uint32_t half,
                              uint32_t h) {
    Unit u;
    const uint32_t base = blk * kBlockBytes;
    u.qs = __builtin_amdgcn_raw_buffer_load_b64(
        rw, ok ? base + 16 * half + 8 * h : kOutOfRange, 0, kUnitLoad);
    u.sg = __builtin_amdgcn_raw_buffer_load_b64(
        rw, ok ? base + 32 + 16 * half + 8 * h : kOutOfRange, 0, kUnitLoad);
    u.qh = __builtin_amdgcn_raw_buffer_load_b32(rw, ok ? base + 64 + 4 * half : kOutOfRange,
                                                0, kUnitLoad);
    return u;
  }
  __device__ static void fill_scales(Unit& u, uint32_t addr, uint32_t half) {
    u.d = lds_u16(addr);
    u.s01 = lds_u16(addr + 2 + 4 * half);
    u.s23 = lds_u16(addr + 4 + 4 * half);
  }
  __device__ static float unit_scale(const Unit& u) {
    return half_bits_to_float((uint16_t)u.d);
  }
  __device__ static Words unpack(const Unit& u) {
    Words w;
#pragma unroll
    for (uint32_t c = 0; c < 2; ++c) {
      const auto r = __builtin_amdgcn_permlane32_swap(u.qs[c], u.qs[c], false, false);
      w.qs[c] = r[0];
      w.qs[c + 2] = r[1];
      const auto t = __builtin_amdgcn_permlane32_swap(u.sg[c], u.sg[c], false, false);
      w.sg[c] = t[0];
      w.sg[c + 2] = t[1];
    }
    w.qh = u.qh;
    w.sc = (u.s01 & 0xFFFFu) | (u.s23 << 16);
    return w;
  }
  __device__ static u32x2 group(const Words& w, uint32_t j, uint32_t hf, const Consts& k) {
    // group g = 2 hf + h: grid index qs byte g | ((qh byte j >> 2 g) & 3) << 8
    const uint32_t lo = __builtin_amdgcn_ubfe(w.qs[j], 16 * hf + k.h8, 8);
    const uint32_t hb = __builtin_amdgcn_ubfe(w.qh, 8 * j + 4 * hf + k.h2, 2);
    const uint32_t ga = (((hb << 8) | lo) << 6) | k.cg;
    const uint32_t sa = (__builtin_amdgcn_ubfe(w.sg[j], 16 * hf + k.h8, 8) << 7) | k.cs;
    const u32x4 g = lds_u4(ga);
    const u32x2 m = lds_u2(sa);
    return u32x2{bit_select(m.x, g.z, g.x), bit_select(m.y, g.w, g.y)};
  }
  __device__ static float group_scale(const Words& w, uint32_t j, uint32_t hf) {
    return (float)(2u * ((w.sc >> (8 * j + 4 * hf)) & 0xFu) + 1u);
  }
  __device__ static float weight_at(const uint8_t* wb, const uint8_t* ws, uint32_t row,
                                    uint32_t col, uint32_t bpr) {
    const size_t blk = (size_t)row * bpr + col / kQK;
    const uint32_t ib32 = (col % kQK) / 32, g = (col % 32) / 8, j = col % 8;
    const uint8_t* q = wb + blk * kBlockBytes;
    const uint32_t idx = (uint32_t)q[4 * ib32 + g] | (((q[64 + ib32] >> (2 * g)) & 3u) << 8);
    const uint32_t sbyte = q[32 + 4 * ib32 + g];
    const uint8_t* sc = ws + blk * kScaleBytes;
    const float d = half_bits_to_float((uint16_t)(sc[0] | (sc[1] << 8)));
    const uint32_t nib = (sc[2 + ib32] >> (g < 2 ? 0 : 4)) & 0xFu;
    const float dl = d * (0.5f + (float)nib) * 0.25f;
    const uint32_t code = ((uint32_t)kRowsSCodes[idx] >> (2 * j)) & 3u;
    const float mag = dl * (code == 0 ? 8.0f : (code == 1 ? 25.0f : 43.0f));
    return ((sbyte >> j) & 1u) ? -mag : mag;
  }
};

// ---------------------------------------------------------------------------
// IQ3_S: grid rows (512 x 128 B) of 16 copies of {g, -g} (4 magnitudes each)
// at [0, 64K); sign-byte mask rows as IQ2_S at [64K, 96K).
// ---------------------------------------------------------------------------
struct RowsFmtS3 {
  static constexpr bool kHalf = false;
  // 21-bit digits: 32 columns x 2^21 x 15 stay below 2^31 (22 bits would let
  // rint reach 2^22, past the range of the magic-number digitisation)
  static constexpr int kDigitShift = 21;
  static constexpr bool kSplitSum = false;
  static constexpr uint32_t kTableBytes = 96 * 1024;
  static constexpr uint32_t kBlockBytes = 104, kScaleBytes = 6;
  struct Consts {
    uint32_t cg, cs, h, h4, h16;
  };
  struct Unit {
    u32x4 qs;
    u32x2 sg;
    uint32_t qh, d, sc;
  };
  struct Words {
    uint32_t q0[4], q1[4];  // grid low bytes of groups 0-1 / 2-3 of sub-block j
    uint32_t sg[4];         // sign bytes of sub-block j
    uint32_t qh, sc;        // high-bit byte j; scale nibble j at bits 4j
  };

  __device__ static Consts consts(uint32_t lane) {
    const uint32_t h = lane >> 5;
    return Consts{8 * (lane & 15), 65536u + 8 * (lane & 15), h, 4 * h, 16 * h};
  }
  __device__ static uint32_t seed(uint32_t tid) { return tid < 512 ? kRowsS3Codes[tid] : 0u; }
  __device__ static void tables(uint8_t* lds, uint32_t tid, uint32_t code) {
    if (tid < 512) {
      const uint32_t g = iq3_bytes(code);
      store_copies<16>(lds + tid * 128, tid, u32x2{g, neg_bytes(g)}, 0, 16);
    } else {
      const uint32_t b = (tid - 512) >> 1, half = tid & 1;
      store_copies<16>(lds + 65536 + b * 128, b, byte_sign_mask(b), 8 * half, 8);
    }
  }
  __device__ static Unit load(__amdgpu_buffer_rsrc_t rw, bool ok, uint32_t blk, uint32_t half,
                              uint32_t h) {
    Unit u;
    const uint32_t base = blk * kBlockBytes;
    // (blocks are 8-byte aligned only: the 16 code bytes as two 8-byte loads)
    const uint32_t qo = ok ? base + 32 * half + 16 * h : kOutOfRange;
    const u32x2 q0 = __builtin_amdgcn_raw_buffer_load_b64(rw, qo, 0, kUnitLoad);
    const u32x2 q1 = __builtin_amdgcn_raw_buffer_load_b64(rw, ok ? qo + 8 : kOutOfRange, 0,
                                                          kUnitLoad);
    u.qs = u32x4{q0.x, q0.y, q1.x, q1.y};
    u.sg = __builtin_amdgcn_raw_buffer_load_b64(
        rw, ok ? base + 72 + 16 * half + 8 * h : kOutOfRange, 0, kUnitLoad);
    u.qh = __builtin_amdgcn_raw_buffer_load_b32(rw, ok ? base + 64 + 4 * half : kOutOfRange,
                                                0, kUnitLoad);
    return u;
  }
  // d, then the scale byte of sub-blocks 4 half .. 4 half + 3 (two nibbles each)
  __device__ static void fill_scales(Unit& u, uint32_t addr, uint32_t half) {
    u.d = lds_u16(addr);
    u.sc = lds_u16(addr + 2 + 2 * half);
  }
  // d * 8: the activation scales carry the 1/8 of the IQ2 formats' dl
  __device__ static float unit_scale(const Unit& u) {
    return half_bits_to_float((uint16_t)u.d) * 8.0f;
  }
  __device__ static Words unpack(const Unit& u) {
    Words w;
#pragma unroll
    for (uint32_t c = 0; c < 4; ++c) {
      const auto r = __builtin_amdgcn_permlane32_swap(u.qs[c], u.qs[c], false, false);
      const uint32_t j0 = c >> 1, j1 = j0 + 2;
      if (c & 1) {
        w.q1[j0] = r[0];
        w.q1[j1] = r[1];
      } else {
        w.q0[j0] = r[0];
        w.q0[j1] = r[1];
      }
    }
#pragma unroll
    for (uint32_t c = 0; c < 2; ++c) {
      const auto r = __builtin_amdgcn_permlane32_swap(u.sg[c], u.sg[c], false, false);
      w.sg[c] = r[0];
      w.sg[c + 2] = r[1];
    }
    w.qh = u.qh;
    w.sc = u.sc;
    return w;
  }
  // groups 2h and 2h + 1 of sub-block j (two 4-value entries each)
  __device__ static v4i pair(const Words& w, uint32_t j, const Consts& k) {
    const uint32_t q = k.h ? w.q1[j] : w.q0[j];
    const uint32_t hb = __builtin_amdgcn_ubfe(w.qh, 8 * j + k.h4, 4);
    uint32_t v[4];
#pragma unroll
    for (uint32_t l = 0; l < 2; ++l) {
      // group 2h + l: sign byte l of the lane's half, entries 2l and 2l + 1
      const uint32_t sbyte = __builtin_amdgcn_ubfe(w.sg[j], k.h16 + 8 * l, 8);
      const u32x2 m = lds_u2((sbyte << 7) | k.cs);
#pragma unroll
      for (uint32_t e = 2 * l; e < 2 * l + 2; ++e) {
        // entry e: grid index byte e of q, high bit e of hb
        const uint32_t idx = __builtin_amdgcn_ubfe(q, 8 * e, 8) | (((hb >> e) & 1u) << 8);
        const u32x2 g = lds_u2((idx << 7) | k.cg);
        v[e] = bit_select((e & 1) ? m.y : m.x, g.y, g.x);
      }
    }
    return v4i{(int)v[0], (int)v[1], (int)v[2], (int)v[3]};
  }
  __device__ static float pair_scale(const Words& w, uint32_t j, const Consts&) {
    return (float)(2u * ((w.sc >> (4 * j)) & 0xFu) + 1u);
  }
  __device__ static float weight_at(const uint8_t* wb, const uint8_t* ws, uint32_t row,
                                    uint32_t col, uint32_t bpr) {
    const size_t blk = (size_t)row * bpr + col / kQK;
    const uint32_t ib32 = (col % kQK) / 32, l = (col % 32) / 8, j = col % 8;
    const uint8_t* q = wb + blk * kBlockBytes;
    const uint32_t half = j >> 2;  // the group's first or second entry
    const uint32_t idx =
        (uint32_t)q[8 * ib32 + 2 * l + half] | (((q[64 + ib32] >> (2 * l + half)) & 1u) << 8);
    const uint32_t sbyte = q[72 + 4 * ib32 + l];
    const uint8_t* sc = ws + blk * kScaleBytes;
    const float d = half_bits_to_float((uint16_t)(sc[0] | (sc[1] << 8)));
    const uint32_t nib = (sc[2 + ib32 / 2] >> (4 * (ib32 & 1))) & 0xFu;
    const float dl = d * (1.0f + 2.0f * (float)nib);
    const float mag = dl * (float)(2u * ((kRowsS3Codes[idx] >> (3 * (j & 3))) & 7u) + 1u);
    return ((sbyte >> j) & 1u) ? -mag : mag;
  }
};

}  // namespace cmk
