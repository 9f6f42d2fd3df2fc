// iq_variants.hip — IQ2_XS, IQ2_S and IQ3_S matmul and dequantisation for gfx950.
//
// The reference serves these formats with the same one-thread-per-output
// kernels as IQ2_XXS (iq2_xs / iq2_s / iq3_s matmul kernels,
// src/metal_src/iq2_matmul.metal:242-434, 501-699; element decodes :736-866;
// CPU reference src/iq2_matmul.rs:884-1016).  Here every format reduces to one
// sub-block decode: a 32-weight sub-block is four groups of 8 weights, each a
// codebook entry of 8 magnitudes (IQ3_S: two entries of 4), a sign byte (bit j
// negates weight j) and a sub-block scale dl.  Every weight is the exact fp32
// product dl * g * sign:
//   IQ2_XS, IQ2_S: dl = d * (0.5 + nibble) * 0.25, g in {8, 25, 43};
//   IQ3_S:         dl = d * (1 + 2 * nibble),      g odd in 1..15;
// (at most 22 significant bits, so exact and independent of evaluation order).
//
// Layouts (weight_bytes / weight_scales per 256-weight block):
//   IQ2_XS 64 / 10:  sub-block ib32 = four LE u16 words at 8*ib32; word w:
//                    grid index bits 0..8, ksigns index bits 9..15; scales:
//                    d, then byte 2+ib32 (low nibble words 0-1, high 2-3).
//   IQ2_S  72 / 10:  qs[0..32) grid low bytes, qs[32..64) sign bytes, qh[64..72)
//                    grid high bits (two per group, nibble il per half);
//                    scales: d, then byte 2+ib32 (nibble il per 16 weights).
//   IQ3_S 104 / 6:   qs[0..64) grid low bytes (two per group), qh[64..72) one
//                    high bit per entry, signs[72..104) one byte per group;
//                    scales: d, then nibble ib32 of bytes 2..5.
//
// Matmul: the workgroup stages up to four activation rows in LDS as fp32
// (W8A8: after the reference's qdq), padded by 4 floats per 32 so that the
// lanes' 16-byte reads of their sub-blocks' columns are conflict-free; each
// wave then takes four weight rows at once, lanes over sub-blocks, exact
// weights into fp32 FMA, and reduces across the wave.  Shapes whose staged
// rows do not fit LDS read x from global memory with one row per wave.
// Dequantisation: one thread per sub-block, each output the single RNE of its
// exact weight.  Codebooks are expanded from compact codes into LDS at launch.
// All code and scale bytes are read with byte loads (any alignment).
#include "iq2xxs_device.h"
#include "iq2xxs_kernels.h"
#include "iq_variants_format.h"

namespace cmk {

static __constant__ uint16_t kIq2xsCodes[512] = {CMK_IQ2XS_GRID_CODES};
static __constant__ uint16_t kIq2sCodes[1024] = {CMK_IQ2S_GRID_CODES};
static __constant__ uint16_t kIq3sCodes[512] = {CMK_IQ3S_GRID_CODES};

template <int V>
struct VariantFmt;
template <>
struct VariantFmt<1> {  // IQ2_XS
  static constexpr uint32_t kBytes = 64, kScales = 10, kGrid = 512;
};
template <>
struct VariantFmt<2> {  // IQ2_S
  static constexpr uint32_t kBytes = 72, kScales = 10, kGrid = 1024;
};
template <>
struct VariantFmt<3> {  // IQ3_S
  static constexpr uint32_t kBytes = 104, kScales = 6, kGrid = 512;
};

size_t variant_bytes_per_block(int v) { return v == 1 ? 64 : v == 2 ? 72 : v == 3 ? 104 : 0; }
size_t variant_scales_per_block(int v) { return v == 1 ? 10 : v == 2 ? 10 : v == 3 ? 6 : 0; }

// Codebook entry e as magnitude bytes (IQ3_S: four bytes in the low half).
template <int V>
__device__ __forceinline__ uint64_t variant_grid_entry(uint32_t e) {
  if constexpr (V == 3) {
    const uint32_t c = kIq3sCodes[e];
    uint32_t v = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) v |= (2u * ((c >> (3 * j)) & 7u) + 1u) << (8 * j);
    return v;
  } else {
    return grid_entry_from_code(V == 1 ? kIq2xsCodes[e] : kIq2sCodes[e]);
  }
}

template <int V>
__device__ __forceinline__ void build_variant_grid(uint64_t* g) {
  for (uint32_t e = threadIdx.x; e < VariantFmt<V>::kGrid; e += blockDim.x)
    g[e] = variant_grid_entry<V>(e);
}

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8);
}

// Little-endian loads: byte by byte for any alignment, or (kAligned: weight
// bytes 4-byte and scales 2-byte aligned; every offset used below is then a
// multiple of the access size) one load each.
template <bool kAligned>
struct Ld {
  static __device__ __forceinline__ uint32_t u16(const uint8_t* p) {
    if constexpr (kAligned) return *reinterpret_cast<const uint16_t*>(p);
    return ld_u16(p);
  }
  static __device__ __forceinline__ uint32_t u32(const uint8_t* p) {
    if constexpr (kAligned) return *reinterpret_cast<const uint32_t*>(p);
    return ld_u16(p) | (ld_u16(p + 2) << 16);
  }
};

// ksigns(i) = i | parity(i) << 7 (the reference's ksigns_iq2xs table).
__device__ __forceinline__ uint32_t ksigns7(uint32_t i) {
  return i | ((__popc(i) & 1u) << 7);
}

// The four 8-weight groups of sub-block ib32 of a block: magnitudes, sign
// bits, scale.
struct SubBlock {
  uint64_t mag[4];
  uint32_t sgn[4];
  float dl[4];
};

template <int V, bool kAligned = false>
__device__ __forceinline__ SubBlock decode_sub_block(const uint8_t* q, const uint8_t* sc, float d,
                                                     uint32_t ib32, const uint64_t* grid) {
  using L = Ld<kAligned>;
  SubBlock s;
  if constexpr (V == 1) {
    const uint32_t sbyte = sc[2 + ib32];
    const float dl0 = (d * (0.5f + (float)(sbyte & 0x0Fu))) * 0.25f;
    const float dl1 = (d * (0.5f + (float)(sbyte >> 4))) * 0.25f;
    const uint32_t w01 = L::u32(q + 8 * ib32), w23 = L::u32(q + 8 * ib32 + 4);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t qw = ((w < 2 ? w01 : w23) >> (16 * (w & 1))) & 0xFFFFu;
      s.mag[w] = grid[qw & 0x1FFu];
      s.sgn[w] = ksigns7((qw >> 9) & 0x7Fu);
      s.dl[w] = w < 2 ? dl0 : dl1;
    }
  } else if constexpr (V == 2) {
    const uint32_t qh = q[64 + ib32], sbyte = sc[2 + ib32];
    const uint32_t qs4 = L::u32(q + 4 * ib32), sg4 = L::u32(q + 32 + 4 * ib32);
#pragma unroll
    for (int il = 0; il < 2; ++il) {
      const uint32_t nib = qh >> (4 * il);
      const float dl = (d * (0.5f + (float)((sbyte >> (4 * il)) & 0x0Fu))) * 0.25f;
      const uint32_t b0 = (qs4 >> (16 * il)) & 0xFFu, b1 = (qs4 >> (16 * il + 8)) & 0xFFu;
      s.mag[2 * il] = grid[b0 | ((nib << 8) & 0x300u)];
      s.mag[2 * il + 1] = grid[b1 | ((nib << 6) & 0x300u)];
      s.sgn[2 * il] = (sg4 >> (16 * il)) & 0xFFu;
      s.sgn[2 * il + 1] = (sg4 >> (16 * il + 8)) & 0xFFu;
      s.dl[2 * il] = dl;
      s.dl[2 * il + 1] = dl;
    }
  } else {
    const uint32_t qh = q[64 + ib32];
    const uint32_t nib = (sc[2 + ib32 / 2] >> (4 * (ib32 & 1))) & 0x0Fu;
    const float dl = d * (1.0f + 2.0f * (float)nib);
    const uint32_t lo = L::u32(q + 8 * ib32), hi = L::u32(q + 8 * ib32 + 4);
    const uint32_t sg4 = L::u32(q + 72 + 4 * ib32);
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const uint32_t w = l < 2 ? lo : hi;
      const uint32_t i1 = ((w >> (16 * (l & 1))) & 0xFFu) | (((qh >> (2 * l)) & 1u) << 8);
      const uint32_t i2 = ((w >> (16 * (l & 1) + 8)) & 0xFFu) | (((qh >> (2 * l + 1)) & 1u) << 8);
      s.mag[l] = grid[i1] | (grid[i2] << 32);
      s.sgn[l] = (sg4 >> (8 * l)) & 0xFFu;
      s.dl[l] = dl;
    }
  }
  return s;
}

// Exact weight j of a group.
__device__ __forceinline__ float group_weight(const SubBlock& s, int g, int j) {
  const float mag = s.dl[g] * (float)((s.mag[g] >> (8 * j)) & 0xFFu);
  return ((s.sgn[g] >> j) & 1u) ? -mag : mag;
}

// Staged activation column c of row mm: 36 floats per 32 columns.
__device__ __forceinline__ uint32_t xs_index(uint32_t mm, uint32_t c, uint32_t pitch) {
  return mm * pitch + c + (c >> 5) * 4;
}

template <int V, bool kAligned>
__global__ __launch_bounds__(256) void iq_variant_matmul_lds_kernel(
    const void* x, int x_dtype, uint32_t m, const uint8_t* wb, const uint8_t* ws, float* out,
    uint32_t out_dim, uint32_t in_dim, uint32_t bpr, const float* row_inv, uint32_t mc_max) {
  using F = VariantFmt<V>;
  __shared__ uint64_t grid[F::kGrid];
  extern __shared__ __align__(16) float xs[];
  build_variant_grid<V>(grid);
  const int lane = threadIdx.x & 63;
  const uint32_t wave = threadIdx.x >> 6;
  const uint32_t nsb = bpr * kSubBlocksPerBlock;
  const uint32_t pitch = nsb * 36;  // staged floats per activation row
  for (uint32_t m0 = 0; m0 < m; m0 += mc_max) {
    const uint32_t mc = m - m0 < mc_max ? m - m0 : mc_max;
    __syncthreads();  // the previous rows' readers are done
    // eight loads in flight per thread before their stores
    const uint32_t total = mc * in_dim;
    for (uint32_t base = threadIdx.x; base < total; base += 8 * blockDim.x) {
      float xv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const uint32_t i = base + u * blockDim.x;
        xv[u] = i < total ? load_x(x, x_dtype, (size_t)m0 * in_dim + i) : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const uint32_t i = base + u * blockDim.x;
        if (i < total) {
          const uint32_t mm = i / in_dim, c = i - mm * in_dim;
          xs[xs_index(mm, c, pitch)] = row_inv ? qdq_w8a8(xv[u], row_inv[m0 + mm]) : xv[u];
        }
      }
    }
    __syncthreads();
    for (uint32_t r0 = (blockIdx.x * 4 + wave) * 4; r0 < out_dim; r0 += gridDim.x * 16) {
      float acc[4][4];
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int mm = 0; mm < 4; ++mm) acc[r][mm] = 0.0f;
      for (uint32_t sb = lane; sb < nsb; sb += 64) {
        const uint32_t col0 = sb * 32;
        if (col0 >= in_dim) continue;
        SubBlock s[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t row = r0 + r < out_dim ? r0 + r : out_dim - 1;
          const size_t block = (size_t)row * bpr + sb / 8;
          const uint8_t* q = wb + block * F::kBytes;
          const uint8_t* sc = ws + block * F::kScales;
          s[r] = decode_sub_block<V, kAligned>(
              q, sc, half_bits_to_float((uint16_t)Ld<kAligned>::u16(sc)), sb % 8, grid);
        }
        const uint32_t ncol = in_dim - col0 < 32 ? in_dim - col0 : 32;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
#pragma unroll
          for (int mm = 0; mm < 4; ++mm) {
            if ((uint32_t)mm >= mc) break;
            // eight staged activations of this group (zero past in_dim)
            float xv[8];
            const float* xp = xs + xs_index(mm, col0 + 8 * g, pitch);
#pragma unroll
            for (int j = 0; j < 8; ++j) xv[j] = (uint32_t)(8 * g + j) < ncol ? xp[j] : 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
              for (int j = 0; j < 8; ++j) acc[r][mm] = fmaf(xv[j], group_weight(s[r], g, j), acc[r][mm]);
          }
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int mm = 0; mm < 4; ++mm) {
          float v = acc[r][mm];
#pragma unroll
          for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
          if (lane == 0 && r0 + r < out_dim && (uint32_t)mm < mc)
            out[(size_t)(m0 + mm) * out_dim + r0 + r] = v;
        }
    }
  }
}

template <int V>
__global__ __launch_bounds__(256) void iq_variant_matmul_kernel(
    const void* x, int x_dtype, uint32_t m, const uint8_t* wb, const uint8_t* ws, float* out,
    uint32_t out_dim, uint32_t in_dim, uint32_t bpr, const float* row_inv) {
  using F = VariantFmt<V>;
  __shared__ uint64_t grid[F::kGrid];
  build_variant_grid<V>(grid);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const uint32_t nsb = bpr * kSubBlocksPerBlock;
  for (uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6); row < out_dim; row += gridDim.x * 4) {
    for (uint32_t m0 = 0; m0 < m; m0 += 4) {
      float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      for (uint32_t sb = lane; sb < nsb; sb += 64) {
        const uint32_t col0 = sb * 32;
        if (col0 >= in_dim) continue;
        const size_t block = (size_t)row * bpr + sb / 8;
        const uint8_t* q = wb + block * F::kBytes;
        const uint8_t* sc = ws + block * F::kScales;
        const float d = half_bits_to_float((uint16_t)ld_u16(sc));
        const SubBlock s = decode_sub_block<V>(q, sc, d, sb % 8, grid);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          for (int j = 0; j < 8; ++j) {
            const uint32_t c = col0 + 8 * g + j;
            if (c >= in_dim) break;
            const float w = group_weight(s, g, j);
#pragma unroll
            for (int mm = 0; mm < 4; ++mm) {
              if (m0 + mm < m) {
                float xv = load_x(x, x_dtype, (size_t)(m0 + mm) * in_dim + c);
                if (row_inv) xv = qdq_w8a8(xv, row_inv[m0 + mm]);
                acc[mm] = fmaf(xv, w, acc[mm]);
              }
            }
          }
        }
      }
#pragma unroll
      for (int mm = 0; mm < 4; ++mm) {
        float v = acc[mm];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
        if (lane == 0 && m0 + mm < m) out[(size_t)(m0 + mm) * out_dim + row] = v;
      }
    }
  }
}

__device__ __forceinline__ uint16_t variant_f16_rne(float v) {
  return __half_as_ushort(__float2half_rn(v));
}

__device__ __forceinline__ uint16_t variant_bf16_rne(float v) {
  uint32_t b = __float_as_uint(v);
  if ((b & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)(((b >> 16) & 0x8000u) | 0x7FC0u);
  b += 0x7FFFu + ((b >> 16) & 1u);
  return (uint16_t)(b >> 16);
}

// kind: 0 = f32 out, 1 = f16 out, 2 = bf16 out.
template <int V, int kind>
__global__ __launch_bounds__(256) void iq_variant_dequant_kernel(const uint8_t* wb,
                                                                 const uint8_t* ws, void* out,
                                                                 uint32_t out_dim,
                                                                 uint32_t in_dim, uint32_t bpr) {
  using F = VariantFmt<V>;
  __shared__ uint64_t grid[F::kGrid];
  build_variant_grid<V>(grid);
  __syncthreads();
  const uint64_t nsb_row = (uint64_t)bpr * kSubBlocksPerBlock;
  const uint64_t total = (uint64_t)out_dim * nsb_row;
  for (uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t row = t / nsb_row;
    const uint32_t sb = (uint32_t)(t - row * nsb_row);
    const uint32_t col0 = sb * 32;
    if (col0 >= in_dim) continue;
    const uint64_t block = row * bpr + sb / 8;
    const uint8_t* q = wb + block * F::kBytes;
    const uint8_t* sc = ws + block * F::kScales;
    const float d = half_bits_to_float((uint16_t)ld_u16(sc));
    const SubBlock s = decode_sub_block<V>(q, sc, d, sb % 8, grid);
    const size_t obase = row * (uint64_t)in_dim + col0;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t c = col0 + 8 * g + j;
        if (c < in_dim) {
          const float w = group_weight(s, g, j);
          if constexpr (kind == 0)
            static_cast<float*>(out)[obase + 8 * g + j] = w;
          else if constexpr (kind == 1)
            static_cast<uint16_t*>(out)[obase + 8 * g + j] = variant_f16_rne(w);
          else
            static_cast<uint16_t*>(out)[obase + 8 * g + j] = variant_bf16_rne(w);
        }
      }
    }
  }
}

// LDS for the staged activation rows: at most 128 KB next to the codebook.
constexpr size_t kVariantStageLimit = 128 * 1024;

template <int V>
static hipError_t launch_matmul_v(const void* x, int x_dtype, uint32_t m, const uint8_t* wb,
                                  const uint8_t* ws, float* out, uint32_t out_dim,
                                  uint32_t in_dim, const float* row_inv, int num_cus,
                                  hipStream_t stream) {
  const uint32_t bpr = (in_dim + kQK - 1) / kQK;
  const size_t row_bytes = (size_t)bpr * kSubBlocksPerBlock * 36 * sizeof(float);
  if (row_bytes <= kVariantStageLimit) {
    uint32_t mc = (uint32_t)(kVariantStageLimit / row_bytes);
    if (mc > 4) mc = 4;
    if (mc > m) mc = m;
    const bool al = reinterpret_cast<uintptr_t>(wb) % 4 == 0 &&
                    reinterpret_cast<uintptr_t>(ws) % 2 == 0;
    auto kern = al ? &iq_variant_matmul_lds_kernel<V, true> : &iq_variant_matmul_lds_kernel<V, false>;
    static bool attr_set[2] = {false, false};
    if (!attr_set[al]) {
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize,
                                         (int)kVariantStageLimit);
      if (e != hipSuccess) return e;
      attr_set[al] = true;
    }
    uint32_t blocks = (out_dim + 15) / 16;
    const uint32_t cap = (uint32_t)num_cus * 4;
    if (blocks > cap) blocks = cap;
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), (size_t)mc * row_bytes, stream, x, x_dtype,
                       m, wb, ws, out, out_dim, in_dim, bpr, row_inv, mc);
    return hipGetLastError();
  }
  uint32_t blocks = (out_dim + 3) / 4;
  const uint32_t cap = (uint32_t)num_cus * 8;
  if (blocks > cap) blocks = cap;
  hipLaunchKernelGGL(iq_variant_matmul_kernel<V>, dim3(blocks), dim3(256), 0, stream, x, x_dtype,
                     m, wb, ws, out, out_dim, in_dim, bpr, row_inv);
  return hipGetLastError();
}

hipError_t launch_iq_variant_matmul(int variant, const void* x, int x_dtype, uint32_t m,
                                    const uint8_t* wb, const uint8_t* ws, float* out,
                                    uint32_t out_dim, uint32_t in_dim, const float* row_inv,
                                    int num_cus, hipStream_t stream) {
  switch (variant) {
    case 1:
      return launch_matmul_v<1>(x, x_dtype, m, wb, ws, out, out_dim, in_dim, row_inv, num_cus,
                                stream);
    case 2:
      return launch_matmul_v<2>(x, x_dtype, m, wb, ws, out, out_dim, in_dim, row_inv, num_cus,
                                stream);
    case 3:
      return launch_matmul_v<3>(x, x_dtype, m, wb, ws, out, out_dim, in_dim, row_inv, num_cus,
                                stream);
    default:
      return hipErrorInvalidValue;
  }
}

template <int V>
static hipError_t launch_dequant_v(const uint8_t* wb, const uint8_t* ws, void* out, int out_kind,
                                   uint32_t out_dim, uint32_t in_dim, int num_cus,
                                   hipStream_t stream) {
  const uint32_t bpr = (in_dim + kQK - 1) / kQK;
  const uint64_t total = (uint64_t)out_dim * bpr * kSubBlocksPerBlock;
  uint64_t blocks = (total + 255) / 256;
  const uint64_t cap = (uint64_t)num_cus * 16;
  if (blocks > cap) blocks = cap;
  if (blocks == 0) blocks = 1;
  if (out_kind == 0)
    hipLaunchKernelGGL((iq_variant_dequant_kernel<V, 0>), dim3((uint32_t)blocks), dim3(256), 0,
                       stream, wb, ws, out, out_dim, in_dim, bpr);
  else if (out_kind == 1)
    hipLaunchKernelGGL((iq_variant_dequant_kernel<V, 1>), dim3((uint32_t)blocks), dim3(256), 0,
                       stream, wb, ws, out, out_dim, in_dim, bpr);
  else
    hipLaunchKernelGGL((iq_variant_dequant_kernel<V, 2>), dim3((uint32_t)blocks), dim3(256), 0,
                       stream, wb, ws, out, out_dim, in_dim, bpr);
  return hipGetLastError();
}

hipError_t launch_iq_variant_dequant(int variant, const uint8_t* wb, const uint8_t* ws, void* out,
                                     int out_kind, uint32_t out_dim, uint32_t in_dim, int num_cus,
                                     hipStream_t stream) {
  switch (variant) {
    case 1:
      return launch_dequant_v<1>(wb, ws, out, out_kind, out_dim, in_dim, num_cus, stream);
    case 2:
      return launch_dequant_v<2>(wb, ws, out, out_kind, out_dim, in_dim, num_cus, stream);
    case 3:
      return launch_dequant_v<3>(wb, ws, out, out_kind, out_dim, in_dim, num_cus, stream);
    default:
      return hipErrorInvalidValue;
  }
}

// ---------------------------------------------------------------------------
// GGUF (ggml) blocks -> the reference's split pair.  A ggml block stores the
// fp16 d first, then the code bytes, then the packed scales (none for
// IQ2_XXS); weight_scales receives d and the scales, weight_bytes the codes.
// Code bytes are gathered a dword per thread (code_bytes is a multiple of 4,
// so a dword never straddles blocks; neighbouring threads read neighbouring
// bytes), then scale bytes one per thread.  kAligned: weight_bytes is 4-byte
// aligned and takes dword stores.
// ---------------------------------------------------------------------------
template <bool kAligned>
__global__ __launch_bounds__(256) void gguf_split_kernel(const uint8_t* __restrict__ src,
                                                         uint64_t n_blocks, uint32_t code_bytes,
                                                         uint32_t scale_bytes,
                                                         uint8_t* __restrict__ wb,
                                                         uint8_t* __restrict__ ws) {
  const uint64_t gb = code_bytes + scale_bytes;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  const uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t n_words = n_blocks * (code_bytes / 4);
  for (uint64_t t = tid; t < n_words; t += stride) {
    const uint64_t o = 4 * t;
    const uint64_t b = o / code_bytes;
    const uint8_t* s = src + b * gb + 2 + (o - b * code_bytes);
    const uint32_t v = (uint32_t)s[0] | ((uint32_t)s[1] << 8) | ((uint32_t)s[2] << 16) |
                       ((uint32_t)s[3] << 24);
    if constexpr (kAligned) {
      *reinterpret_cast<uint32_t*>(wb + o) = v;
    } else {
      wb[o] = (uint8_t)v;
      wb[o + 1] = (uint8_t)(v >> 8);
      wb[o + 2] = (uint8_t)(v >> 16);
      wb[o + 3] = (uint8_t)(v >> 24);
    }
  }
  const uint64_t n_sc = n_blocks * scale_bytes;
  for (uint64_t t = tid; t < n_sc; t += stride) {
    const uint64_t b = t / scale_bytes;
    const uint32_t jb = (uint32_t)(t - b * scale_bytes);
    ws[t] = src[b * gb + (jb < 2 ? jb : code_bytes + jb)];
  }
}

hipError_t launch_gguf_split(const uint8_t* blocks, uint64_t n_blocks, uint32_t code_bytes,
                             uint32_t scale_bytes, uint8_t* wb, uint8_t* ws, int num_cus,
                             hipStream_t stream) {
  const uint64_t work = n_blocks * (code_bytes / 4);
  uint64_t grid = (work + 255) / 256;
  const uint64_t cap = (uint64_t)num_cus * 32;
  if (grid > cap) grid = cap;
  if (grid == 0) grid = 1;
  if (reinterpret_cast<uintptr_t>(wb) % 4 == 0)
    hipLaunchKernelGGL(gguf_split_kernel<true>, dim3((uint32_t)grid), dim3(256), 0, stream,
                       blocks, n_blocks, code_bytes, scale_bytes, wb, ws);
  else
    hipLaunchKernelGGL(gguf_split_kernel<false>, dim3((uint32_t)grid), dim3(256), 0, stream,
                       blocks, n_blocks, code_bytes, scale_bytes, wb, ws);
  return hipGetLastError();
}

}  // namespace cmk
