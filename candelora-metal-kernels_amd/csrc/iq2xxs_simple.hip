// iq2xxs_simple.hip — portable IQ2_XXS matmul for gfx950 and the W8A8 row
// scale pre-pass.
//
// The portable kernel serves shapes and alignments the MFMA paths do not take
// (unaligned weight buffers, K beyond the GEMV's LDS budget, f32 activations
// with many rows).  It follows iq2_xxs_matmul_kernel
// (src/metal_src/iq2_matmul.metal:188-240): exact fp32 weights, fp32 FMA.
#include "iq2xxs_device.h"
#include "iq2xxs_kernels.h"

namespace cmk {

// ---------------------------------------------------------------------------
// Portable path: any alignment, any K.  One wave per output row; lanes walk
// the row's sub-blocks with byte loads and accumulate exact fp32 weights with
// fp32 FMA for up to 4 activation rows at a time.
// ---------------------------------------------------------------------------
// W8A8 row scale: 127 / max|x_row| (1 when max < 1e-8).
__global__ __launch_bounds__(256) void iq2xxs_row_inv_scale_kernel(const void* x, int x_dtype,
                                                                   uint32_t in_dim,
                                                                   float* inv_out) {
  __shared__ float s_red[4];
  const size_t base = (size_t)blockIdx.x * in_dim;
  float mx = 0.0f;
  if (x_dtype == 0 && in_dim % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0) {
    // f32 rows: 16-byte loads, four independent maxima (fmaxf ignores NaN and
    // the maximum does not depend on the order, so the result is the same)
    const float4* r4 = reinterpret_cast<const float4*>(static_cast<const float*>(x) + base);
    float m1 = 0.0f, m2 = 0.0f, m3 = 0.0f;
#pragma unroll 4
    for (uint32_t c = threadIdx.x; c < in_dim / 4; c += blockDim.x) {
      const float4 v = r4[c];
      mx = fmaxf(mx, fabsf(v.x));
      m1 = fmaxf(m1, fabsf(v.y));
      m2 = fmaxf(m2, fabsf(v.z));
      m3 = fmaxf(m3, fabsf(v.w));
    }
    mx = fmaxf(fmaxf(mx, m1), fmaxf(m2, m3));
  } else {
    for (uint32_t c = threadIdx.x; c < in_dim; c += blockDim.x)
      mx = fmaxf(mx, fabsf(load_x(x, x_dtype, base + c)));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = mx;
  __syncthreads();
  if (threadIdx.x == 0) {
    float m = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    inv_out[blockIdx.x] = (m < 1e-8f) ? 1.0f : 127.0f / m;
  }
}

__device__ __forceinline__ uint32_t load_u32_bytes(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

__global__ __launch_bounds__(256) void iq2xxs_matmul_simple_kernel(
    const void* x, int x_dtype, uint32_t m, const uint8_t* wb, const uint8_t* ws, float* out,
    uint32_t out_dim, uint32_t in_dim, uint32_t bpr, const float* row_inv) {
  __shared__ uint64_t lds_grid[256];
  __shared__ uint64_t lds_smask[128];
  build_lds_tables(lds_grid, lds_smask, threadIdx.x, blockDim.x);
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
        const uint8_t* q = wb + block * kBytesPerBlock + (sb % 8) * 8;
        const uint32_t aux_g = load_u32_bytes(q), aux_s = load_u32_bytes(q + 4);
        const uint8_t* sp = ws + block * kScalesPerBlock;
        const float d = half_bits_to_float((uint16_t)(sp[0] | (sp[1] << 8)));
        const float dl = (d * (0.5f + (float)(aux_s >> 28))) * 0.25f;
        for (int g = 0; g < 4; ++g) {
          const uint64_t gv = lds_grid[(aux_g >> (8 * g)) & 0xFFu];
          const uint64_t sm = lds_smask[(aux_s >> (7 * g)) & 0x7Fu];
          for (int jj = 0; jj < 8; ++jj) {
            const uint32_t c = col0 + 8 * g + jj;
            if (c >= in_dim) break;
            const float mag = dl * (float)((gv >> (8 * jj)) & 0xFFu);
            const float w = ((sm >> (8 * jj)) & 1u) ? -mag : mag;
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

hipError_t launch_iq2xxs_row_inv_scale(const void* x, int x_dtype, uint32_t m, uint32_t in_dim,
                                       float* inv_out, hipStream_t stream) {
  hipLaunchKernelGGL(iq2xxs_row_inv_scale_kernel, dim3(m), dim3(256), 0, stream, x, x_dtype,
                     in_dim, inv_out);
  return hipGetLastError();
}

hipError_t launch_iq2xxs_matmul_simple(const void* x, int x_dtype, uint32_t m, const uint8_t* wb,
                                       const uint8_t* ws, float* out, uint32_t out_dim,
                                       uint32_t in_dim, const float* row_inv, int num_cus,
                                       hipStream_t stream) {
  const uint32_t bpr = (in_dim + kQK - 1) / kQK;
  uint32_t blocks = (out_dim + 3) / 4;
  const uint32_t cap = (uint32_t)num_cus * 8;
  if (blocks > cap) blocks = cap;
  hipLaunchKernelGGL(iq2xxs_matmul_simple_kernel, dim3(blocks), dim3(256), 0, stream, x, x_dtype,
                     m, wb, ws, out, out_dim, in_dim, bpr, row_inv);
  return hipGetLastError();
}

}  // namespace cmk
