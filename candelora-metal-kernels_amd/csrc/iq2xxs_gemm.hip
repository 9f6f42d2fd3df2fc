// iq2xxs_gemm.hip — prefill-shaped IQ2_XXS matmul (large m, x in f16/bf16).
//
// out[m, n] = sum_k x[m, k] * W[n, k], W dequantised per tile into LDS in the
// activation's type, then fed to v_mfma_f32_16x16x32_{f16,bf16} with fp32
// accumulation.  Every dequantised value is the single round-to-nearest-even
// of the exact weight d*(2s+1)*g/8, i.e. exactly what iq2_dequantize_to_f16
// produces.
//
// The reference has no dedicated prefill kernel: its iq2_xxs_matmul_kernel
// (src/metal_src/iq2_matmul.metal:188-240) serves every m with one thread per
// output.  This kernel is the large-m replacement on the same boundary.
//
// W8A8 (iq2_matmul.metal:436-499): x is replaced by q = clamp(round(x*inv),
// +-127) (exact small integers in f16/bf16) and the fp32 result is divided by
// the row's inv, i.e. sum(q/inv * w) up to fp32 rounding.
//
// Work split.  A workgroup computes a 128 x BN tile of out (BN = 224 gives
// 4 x 64 = 256 workgroups for m = 512, n = 14336: one per CU).  Its 8 waves
// split into two roles around a double-buffered LDS stage of 32 columns of k
// (one sub-block of every weight row):
//  * waves 0-3 (consumers, 2 x 2): each owns a 64 x BN/2 block of the tile and
//    runs the MFMAs of one stage while the next is being written;
//  * waves 4-7 (producers): load the x tile and the weights' codes two stages
//    ahead, and write a stage: x as is, W dequantised.
// One barrier per stage separates writing a buffer from reading it.
//
// Dequantisation of a sub-block (32 weights of one row): the three level
// values RNE(l*d*(2s+1)/8), l in {8, 25, 43}, are formed once in fp32 (exact
// products) and packed into two dwords; a selector table (one v_perm selector
// per pair of weights of each codebook entry) then assembles each pair with
// one v_perm, and a sign table (16-bit sign masks) applies ksigns with one xor.
//
// Bound: MFMA (arithmetic intensity ~1200 flop/B at m = 512).
#include <atomic>

#include "iq2xxs_device.h"
#include "iq2xxs_kernels.h"

namespace cmk {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kGemmBM = 128;
constexpr int kGemmBK = 32;                       // columns of k per stage
constexpr int kGemmPitch = (kGemmBK + 8) * 2;     // LDS bytes per tile row (80)
constexpr int kGemmThreads = 512;
constexpr int kGemmProducer0 = 256;               // first producer thread
constexpr int kGemmTableCopies = 16;              // lane l reads copy l & 15
constexpr uint32_t kGemmSelBytes = 256 * kGemmTableCopies * 16;   // 64 KB
constexpr uint32_t kGemmSignBytes = 128 * kGemmTableCopies * 16;  // 32 KB
constexpr uint32_t kGemmLdsLimit = 160 * 1024;
constexpr uint32_t kGemmOutOfRange = 0x80000000u;
constexpr int kGemmBufferWord3 = 0x00020000;

template <int BN>
struct GemmLayout {
  static constexpr uint32_t kA = kGemmBM * kGemmPitch;  // bytes of the x tile
  static constexpr uint32_t kB = BN * kGemmPitch;       // bytes of the weight tile
  static constexpr uint32_t kStage = kA + kB;
  static constexpr uint32_t kSel = 2 * kStage;          // selector table
  static constexpr uint32_t kSign = kSel + kGemmSelBytes;
  static constexpr uint32_t kTotal = kSign + kGemmSignBytes;
  static constexpr int kNTiles = BN / 32;                // 16-wide MFMA tiles per consumer in n
};

template <bool kBf16>
__device__ __forceinline__ float4v mfma16(const u32x4& a, const u32x4& b, float4v c) {
  if constexpr (kBf16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a),
                                                  __builtin_bit_cast(half8, b), c, 0, 0, 0);
}

// Two floats as a packed pair of f16 / bf16 (each one round-to-nearest-even).
template <bool kBf16>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (kBf16) {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    const b2 v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
  } else {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 v = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, v);
  }
}

__device__ __forceinline__ u32x4 gemm_lds_u4(uint32_t addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
      static_cast<uintptr_t>(addr));
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t gemm_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes,
                                           kGemmBufferWord3);
}

struct GemmArgs {
  const uint16_t* x;  // f16 or bf16 bits, [m, in_dim]
  const uint8_t* wb;
  const uint8_t* ws;
  float* out;
  const float* row_inv;  // W8A8 per-row inv scale, or null
  uint32_t m, out_dim, in_dim, bpr, nk;  // nk = ceil(in_dim / 32)
  uint32_t x_records, wb_records, ws_records;
};

// Builds the selector and sign tables (all copies) with the workgroup's 512
// threads: 256 selector entries and 128 sign entries, 16 copies each.
template <int BN>
__device__ __forceinline__ void build_gemm_tables(uint8_t* lds, uint32_t tid) {
  using L = GemmLayout<BN>;
  for (uint32_t u = tid; u < 256 + 128; u += kGemmThreads) {
    u32x4 v;
    uint32_t base;
    if (u < 256) {
      // pair p of entry u: bytes (2c, 2c+1) of level code c of each weight
      const uint32_t code = kGridCodesDev[u];
      uint32_t w[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const uint32_t c0 = (code >> (4 * p)) & 3u, c1 = (code >> (4 * p + 2)) & 3u;
        w[p] = (2 * c0) | ((2 * c0 + 1) << 8) | ((2 * c1) << 16) | ((2 * c1 + 1) << 24);
      }
      v = u32x4{w[0], w[1], w[2], w[3]};
      base = L::kSel + u * kGemmTableCopies * 16;
    } else {
      const uint32_t i = u - 256;
      const uint32_t s = i | ((__popc(i) & 1u) << 7);  // ksigns(i)
      uint32_t w[4];
#pragma unroll
      for (int p = 0; p < 4; ++p)
        w[p] = (((s >> (2 * p)) & 1u) ? 0x8000u : 0u) | (((s >> (2 * p + 1)) & 1u) ? 0x80000000u : 0u);
      v = u32x4{w[0], w[1], w[2], w[3]};
      base = L::kSign + i * kGemmTableCopies * 16;
    }
#pragma unroll 4
    for (uint32_t k = 0; k < (uint32_t)kGemmTableCopies; ++k)
      *reinterpret_cast<u32x4*>(lds + base + 16 * ((k + u) & (kGemmTableCopies - 1))) = v;
  }
}

template <bool kBf16, int BN>
__global__ __launch_bounds__(kGemmThreads) void iq2xxs_gemm_kernel(GemmArgs a) {
  using L = GemmLayout<BN>;
  extern __shared__ __align__(16) uint8_t lds[];
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t m0 = blockIdx.y * kGemmBM;
  const uint32_t n0 = blockIdx.x * BN;

  build_gemm_tables<BN>(lds, tid);

  if (wave >= 4) {
    // ======== producers ========
    const uint32_t p = tid - kGemmProducer0;  // 0..255
    const __amdgpu_buffer_rsrc_t rx = gemm_rsrc(a.x, a.x_records);
    const __amdgpu_buffer_rsrc_t rw = gemm_rsrc(a.wb, a.wb_records);
    const __amdgpu_buffer_rsrc_t rs = gemm_rsrc(a.ws, a.ws_records);
    // x tile: 128 rows x 32 halves = 512 chunks of 16 B, two per producer
    // (row = c / 4, 16-byte column chunk c % 4).
    uint32_t xrow[2], xinv_ok[2];
    float xinv[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const uint32_t c = p + 256 * u;
      xrow[u] = m0 + (c >> 2);
      xinv_ok[u] = xrow[u] < a.m;
      xinv[u] = (a.row_inv && xinv_ok[u]) ? a.row_inv[xrow[u]] : 1.0f;
    }
    // weight row of this producer (BN <= 256 rows: one sub-block each per stage)
    const uint32_t wrow = n0 + p;
    const bool wrow_ok = p < (uint32_t)BN && wrow < a.out_dim;
    const uint32_t cs = 16 * (lane & (kGemmTableCopies - 1));

    struct Regs {
      u32x4 xv[2];
      u32x2 q;
      uint32_t dbits;
    };
    auto issue = [&](uint32_t kt, Regs& r) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const uint32_t c = p + 256 * u;
        const uint32_t col = kt * kGemmBK + 8 * (c & 3);
        // in_dim % 8 == 0 and x 16-byte aligned on this path: a chunk is in or out
        const bool ok = xinv_ok[u] && col < a.in_dim;
        r.xv[u] = __builtin_amdgcn_raw_buffer_load_b128(
            rx, ok ? ((xrow[u] * a.in_dim) + col) * 2 : kGemmOutOfRange, 0, 0);
      }
      const uint32_t sb = kt;  // sub-block index along the row
      const uint32_t blk = sb >> 3;
      const bool ok = wrow_ok && kt < a.nk;
      r.q = __builtin_amdgcn_raw_buffer_load_b64(
          rw, ok ? (wrow * a.bpr + blk) * kBytesPerBlock + (sb & 7) * 8 : kGemmOutOfRange, 0, 0);
      r.dbits = __builtin_amdgcn_raw_buffer_load_b16(
          rs, ok ? (wrow * a.bpr + blk) * kScalesPerBlock : kGemmOutOfRange, 0, 0);
    };
    auto write_stage = [&](uint32_t stage, const Regs& r) {
      uint8_t* A = lds + stage * L::kStage;
      uint8_t* B = A + L::kA;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const uint32_t c = p + 256 * u;
        u32x4 v = r.xv[u];
        if (a.row_inv) {
          uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const float lo = kBf16 ? bf16_bits_to_float((uint16_t)w[k]) : half_bits_to_float((uint16_t)w[k]);
            const float hi = kBf16 ? bf16_bits_to_float((uint16_t)(w[k] >> 16))
                                   : half_bits_to_float((uint16_t)(w[k] >> 16));
            const float ql = fminf(fmaxf(roundf(lo * xinv[u]), -127.0f), 127.0f);
            const float qh = fminf(fmaxf(roundf(hi * xinv[u]), -127.0f), 127.0f);
            w[k] = pack2<kBf16>(ql, qh);
          }
          v = u32x4{w[0], w[1], w[2], w[3]};
        }
        *reinterpret_cast<u32x4*>(A + (c >> 2) * kGemmPitch + 16 * (c & 3)) = v;
      }
      if (p < (uint32_t)BN) {
        const uint32_t aux_g = r.q.x, aux_s = r.q.y;
        // exact fp32 level values l * d * (2s + 1) / 8, then one rounding each
        const float tdf = half_bits_to_float((uint16_t)r.dbits) * (float)((aux_s >> 27) | 1u) * 0.125f;
        const uint32_t pool_lo = pack2<kBf16>(8.0f * tdf, 25.0f * tdf);
        const uint32_t pool_hi = pack2<kBf16>(43.0f * tdf, 0.0f);
        uint8_t* dst = B + p * kGemmPitch;
        // all table reads first: the stores below may alias them as far as the
        // compiler knows, so interleaving would serialise on LDS latency
        u32x4 sel[4], sgn[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const uint32_t e = (aux_g >> (8 * g)) & 0xFFu;
          const uint32_t i = (aux_s >> (7 * g)) & 0x7Fu;
          sel[g] = gemm_lds_u4(L::kSel + e * (kGemmTableCopies * 16) + cs);
          sgn[g] = gemm_lds_u4(L::kSign + i * (kGemmTableCopies * 16) + cs);
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const u32x4 v = {__builtin_amdgcn_perm(pool_hi, pool_lo, sel[g].x) ^ sgn[g].x,
                           __builtin_amdgcn_perm(pool_hi, pool_lo, sel[g].y) ^ sgn[g].y,
                           __builtin_amdgcn_perm(pool_hi, pool_lo, sel[g].z) ^ sgn[g].z,
                           __builtin_amdgcn_perm(pool_hi, pool_lo, sel[g].w) ^ sgn[g].w};
          *reinterpret_cast<u32x4*>(dst + 16 * g) = v;
        }
      }
    };

    Regs r0, r1;
    issue(0, r0);
    issue(1, r1);
    __syncthreads();  // tables ready
    write_stage(0, r0);
    __syncthreads();  // stage 0 ready
    // iteration kt: consumers read stage kt & 1; producers write stage (kt+1) & 1
    // from the registers loaded two iterations earlier, then reload them.
    for (uint32_t kt = 0; kt < a.nk; kt += 2) {
      issue(kt + 2, r0);
      if (kt + 1 < a.nk) write_stage(1, r1);
      __syncthreads();
      if (kt + 1 >= a.nk) break;
      issue(kt + 3, r1);
      if (kt + 2 < a.nk) write_stage(0, r0);
      __syncthreads();
    }
    return;
  }

  // ======== consumers ========
  const uint32_t wm = wave >> 1, wn = wave & 1;
  constexpr int NT = L::kNTiles;  // n tiles of 16 per consumer
  float4v acc[4][NT];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int jn = 0; jn < NT; ++jn) acc[i][jn] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

  const uint32_t lr = lane & 15;        // operand row within a 16-row tile
  const uint32_t lk = 16 * (lane >> 4);  // byte offset of the lane's 8 k-values
  __syncthreads();  // tables ready
  __syncthreads();  // stage 0 ready
  for (uint32_t kt = 0; kt < a.nk; ++kt) {
    const uint8_t* A = lds + (kt & 1) * L::kStage;
    const uint8_t* B = A + L::kA;
    u32x4 af[4], bfr[NT];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      af[i] = *reinterpret_cast<const u32x4*>(A + (wm * 64 + i * 16 + lr) * kGemmPitch + lk);
#pragma unroll
    for (int jn = 0; jn < NT; ++jn)
      bfr[jn] = *reinterpret_cast<const u32x4*>(B + (wn * (BN / 2) + jn * 16 + lr) * kGemmPitch + lk);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int jn = 0; jn < NT; ++jn) acc[i][jn] = mfma16<kBf16>(af[i], bfr[jn], acc[i][jn]);
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
      for (int jn = 0; jn < NT; ++jn) {
        const uint32_t col = n0 + wn * (BN / 2) + jn * 16 + (lane & 15);
        if (col < a.out_dim) {
          float v = acc[i][jn][r];
          if (a.row_inv) v = v / scale;
          a.out[(size_t)row * a.out_dim + col] = v;
        }
      }
    }
  }
}

// The x tile is loaded in 16-byte chunks that are wholly in or out of range
// (in_dim % 8 == 0), and every buffer offset stays below kGemmOutOfRange.
bool gemm_supported(uint32_t m, uint32_t out_dim, uint32_t in_dim) {
  return in_dim % 8 == 0 && (uint64_t)m * in_dim * 2 < kGemmOutOfRange - 4096 &&
         (uint64_t)out_dim * ((in_dim + kQK - 1) / kQK) * kBytesPerBlock < kGemmOutOfRange - 4096;
}

template <bool kBf16, int BN>
static hipError_t launch_gemm_t(const GemmArgs& a, hipStream_t stream) {
  using L = GemmLayout<BN>;
  static std::atomic<bool> attr_set{false};
  if (!attr_set.load()) {
    hipError_t e =
        hipFuncSetAttribute(reinterpret_cast<const void*>(&iq2xxs_gemm_kernel<kBf16, BN>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGemmLdsLimit);
    if (e != hipSuccess) return e;
    attr_set.store(true);
  }
  dim3 grid((a.out_dim + BN - 1) / BN, (a.m + kGemmBM - 1) / kGemmBM);
  hipLaunchKernelGGL((iq2xxs_gemm_kernel<kBf16, BN>), grid, dim3(kGemmThreads), L::kTotal, stream,
                     a);
  return hipGetLastError();
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
  a.nk = (in_dim + kGemmBK - 1) / kGemmBK;
  a.x_records = m * in_dim * 2;
  a.wb_records = out_dim * a.bpr * kBytesPerBlock;
  a.ws_records = out_dim * a.bpr * kScalesPerBlock;
  // tile width: 224 when it fills the CUs better than 128
  const uint64_t mt = (m + kGemmBM - 1) / kGemmBM;
  const uint64_t t224 = mt * ((out_dim + 223) / 224), t128 = mt * ((out_dim + 127) / 128);
  const bool wide = t224 >= 200 || t224 * 224 <= t128 * 128;
  const bool bf = x_dtype == 2;
  if (wide) return bf ? launch_gemm_t<true, 224>(a, stream) : launch_gemm_t<false, 224>(a, stream);
  return bf ? launch_gemm_t<true, 128>(a, stream) : launch_gemm_t<false, 128>(a, stream);
}

}  // namespace cmk
