// iq2xxs_gemm.hip — prefill-shaped IQ2_XXS matmul (large m, x in f16/bf16).
//
// out[m, n] = sum_k x[m, k] * W[n, k] with W dequantised per tile into LDS in
// the activation's type (f16 or bf16, each value the RNE of the exact fp32
// weight, i.e. exactly what iq2_dequantize_to_f16 produces), then fed to
// v_mfma_f32_16x16x32_{f16,bf16} with fp32 accumulation.
//
// The reference has no dedicated prefill kernel: its iq2_xxs_matmul_kernel
// (src/metal_src/iq2_matmul.metal:188-240) serves every m with one thread per
// output.  This kernel is the large-m replacement on the same boundary.
//
// W8A8 (iq2_matmul.metal:436-499): x is replaced by q = clamp(round(x*inv),
// +-127) (exact small integers in f16/bf16) and the fp32 result is divided by
// the row's inv, i.e. sum(q/inv * w) up to fp32 rounding.
//
// Tile: 128 (m) x 128 (n) x 64 (k) per workgroup of 4 waves (2 x 2), each wave
// 64 x 64 = 4 x 4 MFMA tiles.  LDS rows are padded by 8 halves so the 16
// rows read by one MFMA operand fall in different banks.
//
// Bound: MFMA (arithmetic intensity ~1200 flop/B at m = 512).
#include "iq2xxs_device.h"
#include "iq2xxs_kernels.h"

namespace cmk {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int kBM = 128;
constexpr int kBN = 128;
constexpr int kBK = 64;
constexpr int kLdsStride = kBK + 8;  // halves per LDS row
constexpr int kGemmThreads = 256;

__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) {
  return __half_as_ushort(__float2half_rn(v));
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float v) {
  uint32_t x = __float_as_uint(v);
  if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)(((x >> 16) & 0x8000u) | 0x7FC0u);
  x += 0x7FFFu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}

template <bool kBf16>
__device__ __forceinline__ uint16_t to_operand(float v) {
  return kBf16 ? f32_to_bf16_bits(v) : f32_to_f16_bits(v);
}

template <bool kBf16>
__device__ __forceinline__ float4v mfma16(const uint4& a, const uint4& b, float4v c) {
  if constexpr (kBf16) {
    bf16x8 av, bv;
    __builtin_memcpy(&av, &a, 16);
    __builtin_memcpy(&bv, &b, 16);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, c, 0, 0, 0);
  } else {
    half8 av, bv;
    __builtin_memcpy(&av, &a, 16);
    __builtin_memcpy(&bv, &b, 16);
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, c, 0, 0, 0);
  }
}

struct GemmArgs {
  const uint16_t* x;  // f16 or bf16 bits, [m, in_dim]
  const uint8_t* wb;
  const uint8_t* ws;
  float* out;
  const float* row_inv;  // W8A8 per-row inv scale, or null
  uint32_t m, out_dim, in_dim, bpr, nk;  // nk = ceil(in_dim / 64)
};

// Staged global data for one k-step.
struct Stage {
  uint4 xa[4];     // 4 x 8 halves of the x tile (rows tid/8 + 32*i, cols 8*(tid%8))
  uint2 q;         // this thread's sub-block codes
  uint32_t dbits;  // fp16 d of its block
};

template <bool kBf16, bool kVecX>
__device__ __forceinline__ void load_stage(const GemmArgs& a, uint32_t m0, uint32_t n0, uint32_t kt,
                                           int tid, Stage& s) {
  const uint32_t c = kt * kBK + 8 * (tid & 7);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t r = m0 + (tid >> 3) + 32 * i;
    if (kVecX) {
      if (r < a.m && c < a.in_dim)
        s.xa[i] = *reinterpret_cast<const uint4*>(a.x + (size_t)r * a.in_dim + c);
      else
        s.xa[i] = make_uint4(0, 0, 0, 0);
    } else {
      uint16_t e[8];
#pragma unroll
      for (int k = 0; k < 8; ++k)
        e[k] = (r < a.m && c + k < a.in_dim) ? a.x[(size_t)r * a.in_dim + c + k] : (uint16_t)0;
      s.xa[i] = make_uint4(e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16),
                           e[6] | (e[7] << 16));
    }
  }
  // W: 128 rows x 2 sub-blocks; thread -> (row tid/2, sub-block tid%2).
  const uint32_t row = n0 + (tid >> 1);
  const uint32_t sb = kt * 2 + (tid & 1);
  if (row < a.out_dim) {
    const size_t block = (size_t)row * a.bpr + sb / 8;
    s.q = *reinterpret_cast<const uint2*>(a.wb + block * kBytesPerBlock + (sb % 8) * 8);
    s.dbits = *reinterpret_cast<const uint16_t*>(a.ws + block * kScalesPerBlock);
  } else {
    s.q = make_uint2(0, 0);
    s.dbits = 0;
  }
}

template <bool kBf16>
__device__ __forceinline__ void store_stage(const GemmArgs& a, const Stage& s, uint16_t* As,
                                            uint16_t* Bs, const uint64_t* lds_grid,
                                            const uint64_t* lds_smask, float inv0, float inv1,
                                            float inv2, float inv3, int tid) {
  // x tile -> LDS (optionally W8A8-quantised)
  const float invs[4] = {inv0, inv1, inv2, inv3};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint4 v = s.xa[i];
    if (a.row_inv) {
      uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float lo = kBf16 ? bf16_bits_to_float((uint16_t)w[k]) : half_bits_to_float((uint16_t)w[k]);
        float hi = kBf16 ? bf16_bits_to_float((uint16_t)(w[k] >> 16))
                         : half_bits_to_float((uint16_t)(w[k] >> 16));
        float ql = fminf(fmaxf(roundf(lo * invs[i]), -127.0f), 127.0f);
        float qh = fminf(fmaxf(roundf(hi * invs[i]), -127.0f), 127.0f);
        w[k] = (uint32_t)to_operand<kBf16>(ql) | ((uint32_t)to_operand<kBf16>(qh) << 16);
      }
      v = make_uint4(w[0], w[1], w[2], w[3]);
    }
    *reinterpret_cast<uint4*>(As + ((tid >> 3) + 32 * i) * kLdsStride + 8 * (tid & 7)) = v;
  }
  // W sub-block -> 32 dequantised values
  const float d = half_bits_to_float((uint16_t)s.dbits);
  const float dl = (d * (0.5f + (float)(s.q.y >> 28))) * 0.25f;
  uint16_t* dst = Bs + (tid >> 1) * kLdsStride + 32 * (tid & 1);
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const uint64_t gv = lds_grid[(s.q.x >> (8 * g)) & 0xFFu];
    const uint64_t sm = lds_smask[(s.q.y >> (7 * g)) & 0x7Fu];
    uint32_t p[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float v0 = dl * (float)((gv >> (16 * k)) & 0xFFu);
      float v1 = dl * (float)((gv >> (16 * k + 8)) & 0xFFu);
      if ((sm >> (16 * k)) & 1u) v0 = -v0;
      if ((sm >> (16 * k + 8)) & 1u) v1 = -v1;
      p[k] = (uint32_t)to_operand<kBf16>(v0) | ((uint32_t)to_operand<kBf16>(v1) << 16);
    }
    *reinterpret_cast<uint4*>(dst + 8 * g) = make_uint4(p[0], p[1], p[2], p[3]);
  }
}

template <bool kBf16, bool kVecX>
__global__ __launch_bounds__(kGemmThreads) void iq2xxs_gemm_kernel(GemmArgs a) {
  __shared__ __align__(16) uint16_t As[2][kBM * kLdsStride];
  __shared__ __align__(16) uint16_t Bs[2][kBN * kLdsStride];
  __shared__ uint64_t lds_grid[256];
  __shared__ uint64_t lds_smask[128];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const uint32_t m0 = blockIdx.y * kBM;
  const uint32_t n0 = blockIdx.x * kBN;

  build_lds_tables(lds_grid, lds_smask, tid, kGemmThreads);

  float inv[4] = {1.0f, 1.0f, 1.0f, 1.0f};
  if (a.row_inv) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t r = m0 + (tid >> 3) + 32 * i;
      inv[i] = r < a.m ? a.row_inv[r] : 1.0f;
    }
  }

  float4v acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int jn = 0; jn < 4; ++jn) acc[i][jn] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

  Stage st;
  load_stage<kBf16, kVecX>(a, m0, n0, 0, tid, st);
  __syncthreads();  // tables ready
  store_stage<kBf16>(a, st, As[0], Bs[0], lds_grid, lds_smask, inv[0], inv[1], inv[2], inv[3],
                     tid);
  __syncthreads();

  const int lr = lane & 15;       // operand row within a 16-row tile
  const int lk = 8 * (lane >> 4);  // operand k offset within a 32-wide k-step
  for (uint32_t kt = 0; kt < a.nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < a.nk;
    if (more) load_stage<kBf16, kVecX>(a, m0, n0, kt + 1, tid, st);
    const uint16_t* A = As[cur];
    const uint16_t* B = Bs[cur];
#pragma unroll
    for (int ks = 0; ks < kBK / 32; ++ks) {
      uint4 af[4], bfr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[i] = *reinterpret_cast<const uint4*>(A + (wm * 64 + i * 16 + lr) * kLdsStride +
                                                ks * 32 + lk);
#pragma unroll
      for (int jn = 0; jn < 4; ++jn)
        bfr[jn] = *reinterpret_cast<const uint4*>(B + (wn * 64 + jn * 16 + lr) * kLdsStride +
                                                  ks * 32 + lk);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jn = 0; jn < 4; ++jn) acc[i][jn] = mfma16<kBf16>(af[i], bfr[jn], acc[i][jn]);
    }
    if (more)
      store_stage<kBf16>(a, st, As[cur ^ 1], Bs[cur ^ 1], lds_grid, lds_smask, inv[0], inv[1],
                         inv[2], inv[3], tid);
    __syncthreads();
  }

  // Epilogue: C[m][n], lane holds rows 4*(lane/16)+r, column lane%16 of each tile.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t row = m0 + wm * 64 + i * 16 + 4 * (lane >> 4) + r;
      if (row >= a.m) continue;
      const float scale = a.row_inv ? a.row_inv[row] : 1.0f;
#pragma unroll
      for (int jn = 0; jn < 4; ++jn) {
        const uint32_t col = n0 + wn * 64 + jn * 16 + (lane & 15);
        if (col < a.out_dim) {
          float v = acc[i][jn][r];
          if (a.row_inv) v = v / scale;
          a.out[(size_t)row * a.out_dim + col] = v;
        }
      }
    }
  }
}

hipError_t launch_iq2xxs_gemm(const void* x, int x_dtype, uint32_t m, const uint8_t* wb,
                              const uint8_t* ws, float* out, uint32_t out_dim, uint32_t in_dim,
                              const float* row_inv, hipStream_t stream) {
  GemmArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.wb = wb;
  a.ws = ws;
  a.out = out;
  a.row_inv = row_inv;
  a.m = m;
  a.out_dim = out_dim;
  a.in_dim = in_dim;
  a.bpr = (in_dim + kQK - 1) / kQK;
  a.nk = (in_dim + kBK - 1) / kBK;
  const bool vec = (in_dim % 8 == 0) && ((reinterpret_cast<uintptr_t>(x) & 15) == 0);
  dim3 grid((out_dim + kBN - 1) / kBN, (m + kBM - 1) / kBM);
  const bool bf = x_dtype == 2;
  if (bf) {
    if (vec)
      hipLaunchKernelGGL((iq2xxs_gemm_kernel<true, true>), grid, dim3(kGemmThreads), 0, stream, a);
    else
      hipLaunchKernelGGL((iq2xxs_gemm_kernel<true, false>), grid, dim3(kGemmThreads), 0, stream, a);
  } else {
    if (vec)
      hipLaunchKernelGGL((iq2xxs_gemm_kernel<false, true>), grid, dim3(kGemmThreads), 0, stream, a);
    else
      hipLaunchKernelGGL((iq2xxs_gemm_kernel<false, false>), grid, dim3(kGemmThreads), 0, stream,
                         a);
  }
  return hipGetLastError();
}

}  // namespace cmk
