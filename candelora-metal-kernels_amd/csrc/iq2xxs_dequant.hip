// iq2xxs_dequant.hip — IQ2_XXS -> dense [out_dim, in_dim] in f16 / bf16 / f32.
//
// Replaces the reference kernel iq2_xxs_dequantize_f16
// (src/metal_src/iq2_matmul.metal:868-887, decode :701-734), which runs one
// thread per output element and re-reads d and 8 bytes of codes for every one
// of the 256 elements of a block.  Here one thread owns one 32-weight
// sub-block: it reads its 8 code bytes and the block's fp16 d once and writes
// 32 outputs (64 B for f16) as 16-byte stores.
//
// Every output is the single round-to-nearest-even of the exact fp32 product
// d * (0.5 + s) * 0.25 * g * sign (exact: <= 22 significant bits), so the
// result is bit-identical to the reference's half(float) conversion.
//
// Bound: HBM.  Algorithmic bytes per weight: 66/256 read + sizeof(out) written.
#include "iq2xxs_device.h"
#include "iq2xxs_kernels.h"

namespace cmk {

template <typename OutT>
__device__ __forceinline__ OutT to_out(float v);
template <>
__device__ __forceinline__ float to_out<float>(float v) { return v; }
template <>
__device__ __forceinline__ uint16_t to_out<uint16_t>(float v) {  // f16 RNE
  return __half_as_ushort(__float2half_rn(v));
}

__device__ __forceinline__ uint16_t to_bf16_rne(float v) {
  uint32_t x = __float_as_uint(v);
  if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)(((x >> 16) & 0x8000u) | 0x7FC0u);
  x += 0x7FFFu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}

// kind: 0 = f32 out, 1 = f16 out, 2 = bf16 out.  kVec: in_dim % 8 == 0 and the
// output pointer is 16-byte aligned, so each group of 8 goes out as one 16-byte
// (f16/bf16) or two 16-byte (f32) stores.
template <int kind, bool kVec>
__global__ __launch_bounds__(256) void iq2xxs_dequant_kernel(const uint8_t* __restrict__ wb,
                                                             const uint8_t* __restrict__ ws,
                                                             void* __restrict__ out,
                                                             uint32_t out_dim, uint32_t in_dim,
                                                             uint32_t bpr) {
  __shared__ uint64_t lds_grid[256];
  __shared__ uint64_t lds_smask[128];
  build_lds_tables(lds_grid, lds_smask, threadIdx.x, blockDim.x);
  __syncthreads();

  const uint64_t nsb_row = (uint64_t)bpr * kSubBlocksPerBlock;
  const uint64_t total = (uint64_t)out_dim * nsb_row;
  for (uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (uint64_t)gridDim.x * blockDim.x) {
    const uint64_t row = t / nsb_row;
    const uint32_t sb = (uint32_t)(t - row * nsb_row);
    const uint32_t col0 = sb * kSubBlock;
    if (col0 >= in_dim) continue;  // padding sub-blocks of a partial final block
    const uint64_t block = row * bpr + sb / kSubBlocksPerBlock;
    // unaligned-safe byte loads are not needed: the launcher only selects this
    // kernel for 8-byte aligned weight_bytes and 2-byte aligned weight_scales.
    const uint2 q = *reinterpret_cast<const uint2*>(wb + block * kBytesPerBlock +
                                                    (sb % kSubBlocksPerBlock) * 8);
    const uint16_t dbits = *reinterpret_cast<const uint16_t*>(ws + block * kScalesPerBlock);
    const float d = half_bits_to_float(dbits);
    // dl = d * (0.5 + s) * 0.25, exactly as the reference orders it.
    const float dl = (d * (0.5f + (float)(q.y >> 28))) * 0.25f;
    const uint64_t obase = row * (uint64_t)in_dim + col0;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint64_t gv = lds_grid[(q.x >> (8 * g)) & 0xFFu];
      const uint64_t sm = lds_smask[(q.y >> (7 * g)) & 0x7Fu];
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float mag = dl * (float)((gv >> (8 * j)) & 0xFFu);
        v[j] = ((sm >> (8 * j)) & 1u) ? -mag : mag;
      }
      const uint32_t c = col0 + 8 * g;
      // in_dim % 8 == 0 on the vector path, so a group is either fully inside
      // the row or fully past its end.
      if (kVec && c >= in_dim) break;
      if (kVec) {
        if (kind == 0) {
          float4* o = reinterpret_cast<float4*>(static_cast<float*>(out) + obase + 8 * g);
          o[0] = make_float4(v[0], v[1], v[2], v[3]);
          o[1] = make_float4(v[4], v[5], v[6], v[7]);
        } else {
          uint32_t p[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            uint16_t lo = kind == 1 ? to_out<uint16_t>(v[2 * k]) : to_bf16_rne(v[2 * k]);
            uint16_t hi = kind == 1 ? to_out<uint16_t>(v[2 * k + 1]) : to_bf16_rne(v[2 * k + 1]);
            p[k] = (uint32_t)lo | ((uint32_t)hi << 16);
          }
          *reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + obase + 8 * g) =
              make_uint4(p[0], p[1], p[2], p[3]);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (c + j < in_dim) {
            if (kind == 0)
              static_cast<float*>(out)[obase + 8 * g + j] = v[j];
            else if (kind == 1)
              static_cast<uint16_t*>(out)[obase + 8 * g + j] = to_out<uint16_t>(v[j]);
            else
              static_cast<uint16_t*>(out)[obase + 8 * g + j] = to_bf16_rne(v[j]);
          }
        }
      }
    }
  }
}

template <int kind>
static hipError_t launch_kind(const uint8_t* wb, const uint8_t* ws, void* out, uint32_t out_dim,
                              uint32_t in_dim, uint32_t bpr, bool vec, int num_cus,
                              hipStream_t stream) {
  const uint64_t total = (uint64_t)out_dim * bpr * kSubBlocksPerBlock;
  uint64_t blocks = (total + 255) / 256;
  const uint64_t cap = (uint64_t)num_cus * 16;
  if (blocks > cap) blocks = cap;
  if (blocks == 0) blocks = 1;
  if (vec)
    hipLaunchKernelGGL((iq2xxs_dequant_kernel<kind, true>), dim3((unsigned)blocks), dim3(256), 0,
                       stream, wb, ws, out, out_dim, in_dim, bpr);
  else
    hipLaunchKernelGGL((iq2xxs_dequant_kernel<kind, false>), dim3((unsigned)blocks), dim3(256), 0,
                       stream, wb, ws, out, out_dim, in_dim, bpr);
  return hipGetLastError();
}

hipError_t launch_iq2xxs_dequant(const uint8_t* wb, const uint8_t* ws, void* out, int out_kind,
                                 uint32_t out_dim, uint32_t in_dim, int num_cus,
                                 hipStream_t stream) {
  const uint32_t bpr = (in_dim + kQK - 1) / kQK;
  const size_t esize = out_kind == 0 ? 4 : 2;
  const bool vec = (in_dim % 8 == 0) && ((reinterpret_cast<uintptr_t>(out) & 15) == 0) &&
                   ((8 * esize) % 16 == 0);
  switch (out_kind) {
    case 0:
      return launch_kind<0>(wb, ws, out, out_dim, in_dim, bpr, vec, num_cus, stream);
    case 1:
      return launch_kind<1>(wb, ws, out, out_dim, in_dim, bpr, vec, num_cus, stream);
    default:
      return launch_kind<2>(wb, ws, out, out_dim, in_dim, bpr, vec, num_cus, stream);
  }
}

}  // namespace cmk
