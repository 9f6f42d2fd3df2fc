// mlp_ops.hip — the step between the MLP's matmuls: h = silu(gate) * up.
//
// The reference has no such op (its callers compose candle ops); in a
// Llama-style MLP the gate and up projections (fp32 outputs of the matmul)
// meet here and h feeds the down projection.  One pass reads gate and up
// once and writes h in the type the next matmul takes: f32 for the GEMV
// (small m), f16 / bf16 for the MFMA GEMM (large m).
//
// silu(g) = g / (1 + exp(-g)) in fp32 with the device expf; finite g below
// about -88 gives exp(-g) = inf and silu = -0; g = -inf gives NaN (as
// g * sigmoid(g) does), and NaN propagates.  f16 / bf16 outputs are
// one round-to-nearest-even of the fp32 product.
//
// Bound: HBM.  Bytes per element: 8 read + sizeof(out) written.
#include "iq2xxs_device.h"
#include "iq2xxs_kernels.h"

namespace cmk {

__device__ __forceinline__ uint16_t mlp_f16_rne(float v) {
  return __half_as_ushort(__float2half_rn(v));
}

__device__ __forceinline__ uint16_t mlp_bf16_rne(float v) {
  uint32_t b = __float_as_uint(v);
  if ((b & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)(((b >> 16) & 0x8000u) | 0x7FC0u);
  b += 0x7FFFu + ((b >> 16) & 1u);
  return (uint16_t)(b >> 16);
}

template <int kind>
__device__ __forceinline__ void store_h(void* out, uint64_t i, float h) {
  if constexpr (kind == 0)
    static_cast<float*>(out)[i] = h;
  else
    static_cast<uint16_t*>(out)[i] = kind == 1 ? mlp_f16_rne(h) : mlp_bf16_rne(h);
}

// kind: 0 = f32 out, 1 = f16 out, 2 = bf16 out.  kVec: the three pointers are
// 16-byte aligned (4 elements per step as vectors, then the n % 4 tail).
template <int kind, bool kVec>
__global__ __launch_bounds__(256) void swiglu_kernel(const float* __restrict__ gate,
                                                     const float* __restrict__ up, void* out,
                                                     uint64_t n) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  const uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint64_t first = 0;  // first element of the scalar loop
  if constexpr (kVec) {
    const uint64_t n4 = n / 4;
    for (uint64_t q = tid; q < n4; q += stride) {
      const float4 g = reinterpret_cast<const float4*>(gate)[q];
      const float4 u = reinterpret_cast<const float4*>(up)[q];
      const float h0 = silu_mul(g.x, u.x), h1 = silu_mul(g.y, u.y);
      const float h2 = silu_mul(g.z, u.z), h3 = silu_mul(g.w, u.w);
      if constexpr (kind == 0) {
        reinterpret_cast<float4*>(out)[q] = make_float4(h0, h1, h2, h3);
      } else {
        const uint32_t a0 = kind == 1 ? mlp_f16_rne(h0) : mlp_bf16_rne(h0);
        const uint32_t a1 = kind == 1 ? mlp_f16_rne(h1) : mlp_bf16_rne(h1);
        const uint32_t a2 = kind == 1 ? mlp_f16_rne(h2) : mlp_bf16_rne(h2);
        const uint32_t a3 = kind == 1 ? mlp_f16_rne(h3) : mlp_bf16_rne(h3);
        reinterpret_cast<uint2*>(out)[q] = make_uint2(a0 | (a1 << 16), a2 | (a3 << 16));
      }
    }
    first = n4 * 4;
  }
  for (uint64_t i = first + tid; i < n; i += stride) store_h<kind>(out, i, silu_mul(gate[i], up[i]));
}

hipError_t launch_swiglu(const float* gate, const float* up, void* out, int out_kind, uint64_t n,
                         int num_cus, hipStream_t stream) {
  const bool vec = reinterpret_cast<uintptr_t>(gate) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(up) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(out) % 16 == 0;
  const uint64_t work = vec ? (n + 3) / 4 : n;
  uint64_t grid = (work + 255) / 256;
  const uint64_t cap = (uint64_t)num_cus * 16;
  if (grid > cap) grid = cap;
  if (grid == 0) grid = 1;
  const dim3 g((uint32_t)grid), b(256);
#define CMK_SWIGLU_LAUNCH(K, V) hipLaunchKernelGGL((swiglu_kernel<K, V>), g, b, 0, stream, gate, up, out, n)
  if (vec) {
    if (out_kind == 0) CMK_SWIGLU_LAUNCH(0, true);
    else if (out_kind == 1) CMK_SWIGLU_LAUNCH(1, true);
    else CMK_SWIGLU_LAUNCH(2, true);
  } else {
    if (out_kind == 0) CMK_SWIGLU_LAUNCH(0, false);
    else if (out_kind == 1) CMK_SWIGLU_LAUNCH(1, false);
    else CMK_SWIGLU_LAUNCH(2, false);
  }
#undef CMK_SWIGLU_LAUNCH
  return hipGetLastError();
}

}  // namespace cmk
