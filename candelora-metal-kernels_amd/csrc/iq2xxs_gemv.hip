// iq2xxs_gemv.hip — decode-shaped IQ2_XXS matmul (small m) for gfx950.
//
// Replaces iq2_xxs_matmul_kernel / iq2_xxs_matmul_w8a8_kernel
// (src/metal_src/iq2_matmul.metal:188-240, 436-499), which run one thread per
// output walking all of K serially with byte loads, and (for W8A8) rescan the
// whole x row per thread to find its max.
//
// Design (one launch, no scratch memory):
//  * Activations are turned into exact integer digits once per workgroup:
//    each 32-column chunk with max|x| < 2^e becomes v = rint(x*2^(22-e)) split
//    into three signed 8-bit digit planes (see iq2xxs_device.h), held in LDS.
//  * The weights stream from HBM with 16-byte loads, one pair of 32-weight
//    sub-blocks per lane; codes are expanded with two LDS lookups per group of
//    8 (codebook bytes and a sign byte-mask) and one xor/add per 4 weights into
//    signed int8.
//  * v_mfma_i32_4x4x4_16b_i8 does the dot products: in each of the 16 4x4
//    blocks, the A rows are the three digit planes plus a plane of ones, the B
//    columns are 4 weight rows, so one instruction yields, for 4 rows, the
//    three digit sums and sum(w) of 4 columns.  Eight instructions cover a
//    sub-block; the per-sub-block scale d*(2s+1)/8 * 2^(e-22) is applied in
//    fp32 when the sub-block's sums are folded into the row accumulator.
//  * Lanes keep one partial per (row, slice); the workgroup reduces them in
//    a fixed order at the end, so results are deterministic.
//
// Bound: HBM.  Algorithmic bytes per weight row: ceil(K/256)*66, plus x and
// out once.
#include <atomic>

#include "iq2xxs_device.h"
#include "iq2xxs_kernels.h"

namespace cmk {

typedef int v4i __attribute__((ext_vector_type(4)));

// Lane roles in v_mfma_i32_4x4x4_16b_i8: lane L belongs to 4x4 block L/4; it
// supplies row L%4 of A and column L%4 of B, and receives column L%4 of C
// (rows in the four result registers).
__device__ __forceinline__ v4i mfma4x4(int a_xdigits, int b_weights, v4i c) {
  return __builtin_amdgcn_mfma_i32_4x4x4i8(a_xdigits, b_weights, c, 0, 0, 0);
}

constexpr int kGemvThreads = 512;  // 8 waves
constexpr int kGemvWaves = kGemvThreads / 64;
constexpr int kMaxPairs = 512;  // npairs per row handled by one launch (K <= 32768)
constexpr uint32_t kSignTableOffset = 256 * 8;  // LDS byte offset of the sign-mask table

// Row groups each wave loads up front: 8 / T keeps the weight registers at 40.
template <int T>
constexpr int rows_per_wave() {
  return T == 1 ? 8 : (T == 2 ? 4 : 2);
}

// Makes v look modified here (emits no instruction).  Used on the weight
// registers right before they are decoded, so the decode's address arithmetic
// cannot be hoisted out of the activation-row loop, where it would wait for
// every weight load and hold all addresses in registers at once.
__device__ __forceinline__ void pin_here(uint4& v, uint32_t& d) {
  asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w), "+v"(d));
}

// 8-byte LDS read at a byte address (the kernel's dynamic LDS starts at 0),
// returned as two dwords so the sign step stays 32-bit (v_and + v_xad_u32).
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u32x2 lds_load_u2(uint32_t addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) u32x2*>(
      static_cast<uintptr_t>(addr));
}

struct GemvArgs {
  const void* x;
  const uint8_t* wb;
  const uint8_t* ws;
  float* out;
  int x_dtype;
  uint32_t m, out_dim, in_dim, bpr;
  uint32_t npairs;     // sub-block pairs per row = 4 * bpr
  uint32_t slices;     // waves per row group (1, 2, 4, 8)
  uint32_t rg_per_wg;  // row groups (4 rows) per workgroup
  int w8a8;
};

// LDS layout (dynamic):  grid[256] u64 | smask[128] u64 | xsc[8*npairs] f32 |
//                        red[rg_per_wg * slices * 64] f32 | xdig[3][256*bpr] u8 |
//                        wave maxima[8] f32
//
// T: sub-block pairs per lane per 4-row group (the wave's K-slice is 32T
//    sub-blocks); R: row groups per wave (all loaded up front);
// XT: digitisation tasks (8 columns each) per thread whose activations are
//    loaded before the weights; XD: activation dtype (0 f32, 1 f16, 2 bf16);
// kVecX: activations can be read as aligned 16-byte vectors (in_dim % 8 == 0).
// All global loads are branch-free (clamped addresses, zeroed results), so the
// compiler waits for a load only where its value is used.
template <int T, int R, int XT, int XD, bool kVecX>
__global__ __launch_bounds__(kGemvThreads) void iq2xxs_gemv_kernel(GemvArgs a) {
  extern __shared__ __align__(16) uint8_t lds[];
  uint64_t* lds_grid = reinterpret_cast<uint64_t*>(lds);
  uint64_t* lds_smask = lds_grid + 256;
  float* xsc = reinterpret_cast<float*>(lds_smask + 128);
  const uint32_t nsb = a.npairs * 2;
  float* red = xsc + nsb;
  const uint32_t red_n = a.rg_per_wg * a.slices * 64;
  const uint32_t kp = nsb * 32;  // padded K = 256 * bpr
  uint8_t* xdig = reinterpret_cast<uint8_t*>(red + red_n);
  float* s_wred = reinterpret_cast<float*>(xdig + 3 * kp);  // kGemvWaves floats

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int b = lane >> 2;  // 4x4 block within the wave
  const int j = lane & 3;   // row of the 4-row group this lane loads / column of C it gets
  const uint32_t slice = wave % a.slices;
  const uint32_t team = wave / a.slices;
  const uint32_t teams = kGemvWaves / a.slices;

  const uint32_t rg_begin = blockIdx.x * a.rg_per_wg;
  const uint32_t n_rg_total = (a.out_dim + 3) / 4;
  const uint32_t rg_end = min(rg_begin + a.rg_per_wg, n_rg_total);
  const uint32_t ntasks = nsb * 4;

  // ---- loads in the order they are needed (they complete in issue order):
  // this thread's codebook word, then the activations of row 0 for its first
  // XT digitisation tasks, then every weight this wave will use.
  const uint32_t grid_code = fetch_grid_code(tid);
  XOctet<XD, kVecX> xo[XT];
  auto load_x_tasks = [&](uint32_t task0, size_t xbase) {
#pragma unroll
    for (int u = 0; u < XT; ++u) {
      const uint32_t task = task0 + tid + u * kGemvThreads;
      const uint32_t c0 = (task >> 2) * 32 + (task & 3) * 8;
      xo[u].load(a.x, xbase, c0, a.in_dim, task < ntasks && c0 < a.in_dim);
    }
  };
  load_x_tasks(0, 0);

  // ---- R row groups x T sub-block pairs of weights.
  const size_t row_bytes = (size_t)a.bpr * kBytesPerBlock;
  // Lanes whose (row, pair) is out of range read row 0 / pair 0 instead and get
  // a zero scale at the point of use (wmask), which cancels their products.
  // The 2-byte scales go first: the compiler widens each one right after its
  // load, and that wait should not cover the 16-byte code loads behind it.
  uint4 q[R][T];
  uint32_t dbits[R][T];
  size_t qoff[R][T];
  uint32_t wmask = 0;  // bit r*T+t: (row, pair) in range
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint32_t rg = rg_begin + team + r * teams;
    const uint32_t row = rg * 4 + j;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const uint32_t pair = slice * (16 * T) + t * 16 + b;
      const bool ok = rg < rg_end && row < a.out_dim && pair < a.npairs;
      wmask |= ok ? (1u << (r * T + t)) : 0u;
      const size_t rr = ok ? row : 0;
      const uint32_t pp = ok ? pair : 0;
      qoff[r][t] = rr * row_bytes + (size_t)pp * 16;
      dbits[r][t] = *reinterpret_cast<const uint16_t*>(
          a.ws + (rr * a.bpr + pp / 4) * kScalesPerBlock);
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int t = 0; t < T; ++t) q[r][t] = *reinterpret_cast<const uint4*>(a.wb + qoff[r][t]);

  store_lds_tables(lds_grid, lds_smask, tid, grid_code);

  for (uint32_t mrow = 0; mrow < a.m; ++mrow) {
    const size_t xbase = (size_t)mrow * a.in_dim;
    if (mrow > 0) load_x_tasks(0, xbase);
    // ---- W8A8 row scale (iq2_matmul.metal:86-96), reduced over the whole row.
    float inv_scale = 1.0f;
    if (a.w8a8) {
      float mx0 = 0.0f, mx1 = 0.0f, mx2 = 0.0f, mx3 = 0.0f;
      for (uint32_t c = tid; c < a.in_dim; c += 4 * kGemvThreads) {
        const uint32_t c1 = c + kGemvThreads, c2 = c + 2 * kGemvThreads, c3 = c + 3 * kGemvThreads;
        const uint32_t b0 = load_x_bits<XD>(a.x, xbase + c);
        const uint32_t b1 = load_x_bits<XD>(a.x, c1 < a.in_dim ? xbase + c1 : xbase);
        const uint32_t b2 = load_x_bits<XD>(a.x, c2 < a.in_dim ? xbase + c2 : xbase);
        const uint32_t b3 = load_x_bits<XD>(a.x, c3 < a.in_dim ? xbase + c3 : xbase);
        mx0 = fmaxf(mx0, fabsf(x_bits_to_float<XD>(b0)));
        mx1 = fmaxf(mx1, fabsf(x_bits_to_float<XD>(b1)));
        mx2 = fmaxf(mx2, fabsf(x_bits_to_float<XD>(b2)));
        mx3 = fmaxf(mx3, fabsf(x_bits_to_float<XD>(b3)));
      }
      float mx = fmaxf(fmaxf(mx0, mx1), fmaxf(mx2, mx3));
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
      if (lane == 0) s_wred[wave] = mx;
      __syncthreads();
      mx = 0.0f;
#pragma unroll
      for (int w = 0; w < kGemvWaves; ++w) mx = fmaxf(mx, s_wred[w]);
      inv_scale = (mx < 1e-8f) ? 1.0f : 127.0f / mx;
    }
    // ---- digit planes: 4 threads per 32-column chunk, 8 columns each.
    for (uint32_t task0 = 0; task0 < ntasks; task0 += kGemvThreads * XT) {
      if (task0 > 0) load_x_tasks(task0, xbase);  // activations beyond the first XT tasks
#pragma unroll
      for (int u = 0; u < XT; ++u) {
        const uint32_t task = task0 + tid + u * kGemvThreads;
        // the 4 tasks of a chunk sit in 4 consecutive lanes: all active or none
        if (task0 + u * kGemvThreads >= ntasks) break;
        float xv[8];
        float mx = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          xv[k] = xo[u].get(k);
          if (a.w8a8) xv[k] = qdq_w8a8(xv[k], inv_scale);
          mx = fmaxf(mx, fabsf(xv[k]));
        }
        mx = fmaxf(mx, __shfl_xor(mx, 1));
        mx = fmaxf(mx, __shfl_xor(mx, 2));
        if (task < ntasks) {
          const int e = digit_exponent(mx);
          const float scale = ldexpf(1.0f, kDigitShift - e);
          uint32_t dg[8];
#pragma unroll
          for (int k = 0; k < 8; ++k) dg[k] = digitize(xv[k], scale);
          uint32_t p0[2], p1[2], p2[2];
          digits_to_planes(dg[0], dg[1], dg[2], dg[3], p0[0], p1[0], p2[0]);
          digits_to_planes(dg[4], dg[5], dg[6], dg[7], p0[1], p1[1], p2[1]);
          const uint32_t c0 = (task >> 2) * 32 + (task & 3) * 8;
          *reinterpret_cast<uint2*>(xdig + c0) = make_uint2(p0[0], p0[1]);
          *reinterpret_cast<uint2*>(xdig + kp + c0) = make_uint2(p1[0], p1[1]);
          *reinterpret_cast<uint2*>(xdig + 2 * kp + c0) = make_uint2(p2[0], p2[1]);
          if ((task & 3) == 0) xsc[task >> 2] = ldexpf(1.0f, e - kDigitShift - 3);
        }
        __builtin_amdgcn_sched_barrier(0);  // one task at a time: bounds register use
      }
    }
    // Fence the scheduler on both sides of the barrier: weight-dependent work
    // hoisted above it would make every wave wait for all of its weights here.
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);

    // ---- per-lane activation registers for this wave's slice.
    // Lane (b, i=j) holds digit plane i (i < 3; row 3 of A is zero) of the two
    // sub-blocks of pair  p = slice*16T + t*16 + b  for t < T.
    uint32_t xr[T][2][8];
    float xs[T][2];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const uint32_t pair = slice * (16 * T) + t * 16 + b;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t sb = 2 * pair + h;
        const bool ok = pair < a.npairs;
        xs[t][h] = ok ? xsc[sb] : 0.0f;
        if (ok && j < 3) {
          const uint4* src = reinterpret_cast<const uint4*>(xdig + j * kp + sb * 32);
          uint4 lo = src[0], hi = src[1];
          xr[t][h][0] = lo.x; xr[t][h][1] = lo.y; xr[t][h][2] = lo.z; xr[t][h][3] = lo.w;
          xr[t][h][4] = hi.x; xr[t][h][5] = hi.y; xr[t][h][6] = hi.z; xr[t][h][7] = hi.w;
        } else {
#pragma unroll
          for (int k = 0; k < 8; ++k) xr[t][h][k] = 0u;
        }
      }
    }

    // ---- the dot products, one 4-row group at a time.  The codebook table is
    // at LDS address 0 and the sign table at 2048 (no static LDS in this kernel).
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t rg = rg_begin + team + r * teams;
      if (rg >= rg_end) break;  // wave-uniform
      float acc = 0.0f;
#pragma unroll
      for (int t = 0; t < T; ++t) {
        pin_here(q[r][t], dbits[r][t]);
        const float d =
            ((wmask >> (r * T + t)) & 1u) ? half_bits_to_float((uint16_t)dbits[r][t]) : 0.0f;
        const uint32_t words[4] = {q[r][t].x, q[r][t].y, q[r][t].z, q[r][t].w};
        // signed int8 weights of both sub-blocks of the pair: w[h][2g], w[h][2g+1]
        uint32_t w[2][8];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t aux_g = words[2 * h];
          const uint32_t aux_s = words[2 * h + 1];
          uint32_t goff[4];
          goff[0] = byte_times8<0>(aux_g);
          goff[1] = byte_times8<1>(aux_g);
          goff[2] = byte_times8<2>(aux_g);
          goff[3] = byte_times8<3>(aux_g);
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const u32x2 gv = lds_load_u2(goff[g]);
            const u32x2 sm = lds_load_u2(kSignTableOffset + (((aux_s >> (7 * g)) & 0x7Fu) << 3));
            w[h][2 * g] = apply_signs(gv.x, sm.x);
            w[h][2 * g + 1] = apply_signs(gv.y, sm.y);
          }
        }
        // two independent accumulation chains, interleaved
        v4i c0 = {0, 0, 0, 0}, c1 = {0, 0, 0, 0};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          c0 = mfma4x4((int)xr[t][0][k], (int)w[0][k], c0);
          c1 = mfma4x4((int)xr[t][1][k], (int)w[1][k], c1);
        }
        // c[p] = sum over the 32 columns of digit-plane p times w
        const float f0 = fmaf((float)(c0[2] * 256 + c0[1]), 256.0f, (float)c0[0]);
        const float f1 = fmaf((float)(c1[2] * 256 + c1[1]), 256.0f, (float)c1[0]);
        const float coef0 = (float)((words[1] >> 27) | 1u) * (d * xs[t][0]);
        const float coef1 = (float)((words[3] >> 27) | 1u) * (d * xs[t][1]);
        acc = fmaf(f0, coef0, acc);
        acc = fmaf(f1, coef1, acc);
      }
      red[((rg - rg_begin) * a.slices + slice) * 64 + lane] = acc;
      // keep row groups apart: interleaving them only raises register pressure
      __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();
    // ---- fixed-order reduction of the partials: sum over slices and blocks.
    const uint32_t rows_here = (rg_end > rg_begin) ? (rg_end - rg_begin) * 4 : 0;
    for (uint32_t rr = tid; rr < rows_here; rr += kGemvThreads) {
      const uint32_t rgl = rr >> 2, jj = rr & 3;
      const uint32_t row = rg_begin * 4 + rr;
      float sum = 0.0f;
      for (uint32_t sl = 0; sl < a.slices; ++sl) {
        const float* p = red + (rgl * a.slices + sl) * 64 + jj;
#pragma unroll
        for (int bb = 0; bb < 16; ++bb) sum += p[4 * bb];
      }
      if (row < a.out_dim) a.out[(size_t)mrow * a.out_dim + row] = sum;
    }
    __syncthreads();  // xdig / red are rewritten for the next activation row
  }
}

// ---------------------------------------------------------------------------
// Portable path: any alignment, any K.  One wave per output row; lanes walk
// the row's sub-blocks with byte loads and accumulate exact fp32 weights with
// fp32 FMA for up to 4 activation rows at a time.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void iq2xxs_row_inv_scale_kernel(const void* x, int x_dtype,
                                                                   uint32_t in_dim,
                                                                   float* inv_out) {
  __shared__ float s_red[4];
  const size_t base = (size_t)blockIdx.x * in_dim;
  float mx = 0.0f;
  for (uint32_t c = threadIdx.x; c < in_dim; c += blockDim.x)
    mx = fmaxf(mx, fabsf(load_x(x, x_dtype, base + c)));
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

// ---------------------------------------------------------------------------
// GEMV launch policy.
// ---------------------------------------------------------------------------
bool gemv_supported(uint32_t in_dim) {
  const uint32_t bpr = (in_dim + kQK - 1) / kQK;
  return bpr * 4 <= kMaxPairs;
}

static void gemv_shape(uint32_t npairs, int* T, uint32_t* slices) {
  // Pairs per wave slice is 16*T.  T = 2 (two 16-byte loads per lane per row
  // group) unless eight slices cannot cover the row.
  int t = 2;
  uint32_t s = (npairs + 31) / 32;
  if (s > 8) {
    t = 4;
    s = (npairs + 63) / 64;
  }
  uint32_t p2 = 1;
  while (p2 < s) p2 <<= 1;
  *T = t;
  *slices = p2;
}

size_t gemv_lds_bytes(uint32_t in_dim, uint32_t rg_per_wg, uint32_t slices) {
  const uint32_t bpr = (in_dim + kQK - 1) / kQK;
  const uint32_t nsb = bpr * 8;
  return 256 * 8 + 128 * 8 + (size_t)nsb * 4 + (size_t)rg_per_wg * slices * 64 * 4 +
         (size_t)3 * nsb * 32 + kGemvWaves * 4;
}

// Dynamic LDS above 64 KB must be enabled per kernel.  The limit granted so far
// is remembered per instantiation; it only ever grows (at most 160 KB).
template <int T, int XT, int XD, bool V>
static hipError_t launch_gemv_t(const GemvArgs& a, uint32_t grid, size_t lds,
                                hipStream_t stream) {
  constexpr int R = rows_per_wave<T>();
  static std::atomic<size_t> granted{64 * 1024};
  if (lds > granted.load()) {
    hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&iq2xxs_gemv_kernel<T, R, XT, XD, V>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    size_t cur = granted.load();
    while (lds > cur && !granted.compare_exchange_weak(cur, lds)) {
    }
  }
  hipLaunchKernelGGL((iq2xxs_gemv_kernel<T, R, XT, XD, V>), dim3(grid), dim3(kGemvThreads), lds,
                     stream, a);
  return hipGetLastError();
}

template <int T, int XT, int XD>
static hipError_t launch_gemv_v(const GemvArgs& a, bool vec, uint32_t grid, size_t lds,
                                hipStream_t stream) {
  return vec ? launch_gemv_t<T, XT, XD, true>(a, grid, lds, stream)
             : launch_gemv_t<T, XT, XD, false>(a, grid, lds, stream);
}

template <int T, int XT>
static hipError_t launch_gemv_d(const GemvArgs& a, bool vec, uint32_t grid, size_t lds,
                                hipStream_t stream) {
  switch (a.x_dtype) {
    case 0: return launch_gemv_v<T, XT, 0>(a, vec, grid, lds, stream);
    case 1: return launch_gemv_v<T, XT, 1>(a, vec, grid, lds, stream);
    default: return launch_gemv_v<T, XT, 2>(a, vec, grid, lds, stream);
  }
}

template <int T>
static hipError_t launch_gemv_x(const GemvArgs& a, bool vec, uint32_t grid, size_t lds,
                                hipStream_t stream) {
  // Activations of up to 4 digitisation tasks per thread are loaded up front
  // (T = 4 keeps 1 for registers).
  const uint32_t tasks = (a.npairs * 8 + kGemvThreads - 1) / kGemvThreads;
  if (tasks <= 1 || T == 4) return launch_gemv_d<T, 1>(a, vec, grid, lds, stream);
  return launch_gemv_d<T, 4>(a, vec, grid, lds, stream);
}

hipError_t launch_iq2xxs_gemv(const void* x, int x_dtype, uint32_t m, const uint8_t* wb,
                              const uint8_t* ws, float* out, uint32_t out_dim, uint32_t in_dim,
                              bool w8a8, int num_cus, hipStream_t stream) {
  GemvArgs a;
  a.x = x;
  a.wb = wb;
  a.ws = ws;
  a.out = out;
  a.x_dtype = x_dtype;
  a.m = m;
  a.out_dim = out_dim;
  a.in_dim = in_dim;
  a.bpr = (in_dim + kQK - 1) / kQK;
  a.npairs = a.bpr * 4;
  a.w8a8 = w8a8 ? 1 : 0;
  int T;
  gemv_shape(a.npairs, &T, &a.slices);
  const uint32_t teams = kGemvWaves / a.slices;
  const uint32_t n_rg = (out_dim + 3) / 4;
  // One workgroup per CU when the row groups allow; each wave holds at most
  // R row groups of weights in registers.
  uint32_t rg_per_wg = (n_rg + num_cus - 1) / num_cus;
  const uint32_t cap = teams * (T == 2 ? rows_per_wave<2>() : rows_per_wave<4>());
  if (rg_per_wg > cap) rg_per_wg = cap;
  if (rg_per_wg == 0) rg_per_wg = 1;
  a.rg_per_wg = rg_per_wg;
  const uint32_t grid = (n_rg + rg_per_wg - 1) / rg_per_wg;
  const size_t lds = gemv_lds_bytes(in_dim, rg_per_wg, a.slices);
  const size_t esize = x_dtype == 0 ? 4 : 2;
  const bool vec = (in_dim % 8 == 0) && (reinterpret_cast<uintptr_t>(x) % 16 == 0) &&
                   ((size_t)in_dim * esize % 16 == 0);
  if (T == 2) return launch_gemv_x<2>(a, vec, grid, lds, stream);
  return launch_gemv_x<4>(a, vec, grid, lds, stream);
}

}  // namespace cmk
