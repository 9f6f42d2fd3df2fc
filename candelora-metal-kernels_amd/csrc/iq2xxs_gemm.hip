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
// W8A8 (iq2_matmul.metal:436-499): a pre-pass writes q = clamp(round(x*inv),
// +-127) (exact small integers in f16/bf16) to the caller's workspace; the
// GEMM runs on q and divides each fp32 result by its row's inv, i.e.
// sum(q/inv * w) up to fp32 rounding.
//
// Work split.  A workgroup computes a 128 x BN tile of out (BN = 224 gives
// 4 x 64 = 256 workgroups for m = 512, n = 14336: one per CU).  k advances in
// stages of 64 columns (two 32-weight sub-blocks of every weight row).
//  * Waves 0-3 (consumers, 2 x 2) each own a 64 x BN/2 block of the tile.  They
//    load their activation fragments straight from global memory (L2-resident
//    x, one stage ahead) and read the weight fragments from LDS.
//  * Waves 4-7 (producers) own one weight row per lane: they load the row's
//    codes 128 bytes (eight stages) at a time, dequantise one stage per step
//    into a double-buffered LDS tile, and a barrier publishes each stage.
// Only the weight tile passes through LDS: LDS writes run at about 100 B/clk
// and reads at about 270 B/clk per CU on gfx950, and an activation tile in LDS
// as well would cost more LDS time per stage than the stage's MFMAs take.
//
// LDS layout (64 KB aligned tables, so one v_perm forms a selector address):
//   [0, 64K)      selector table: 256 codebook entries x 16 copies x 16 B
//   [64K, 96K)    sign table: 128 sign indices x 16 copies x 16 B
//   [96K, ...)    two weight tiles of BN rows x 128 B, 16-byte chunk c of row
//                 r stored at chunk position c ^ (r & 7) (conflict-free reads
//                 of the MFMA fragment pattern; measured on gfx950).
//
// Dequantisation of a sub-block (32 weights of one row): the three level
// values RNE(l*d*(2s+1)/8), l in {8, 25, 43}, are formed once in fp32 (exact
// products) and packed into two dwords; the selector table (one v_perm
// selector per pair of weights of each codebook entry) then assembles each
// pair with one v_perm, and the sign table (16-bit sign masks) applies ksigns
// with one xor.
//
// Bound: MFMA (arithmetic intensity ~1200 flop/B at m = 512).
#include <atomic>

#include "iq2xxs_device.h"
#include "iq2xxs_kernels.h"

namespace cmk {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kGemmBM = 128;
constexpr int kGemmBK = 64;                  // columns of k per stage
constexpr int kGemmRowBytes = kGemmBK * 2;   // LDS bytes per weight-tile row
constexpr int kGemmThreads = 512;
constexpr int kGemmProducer0 = 256;          // first producer thread
constexpr int kGemmGroup = 8;                // stages per 128-byte code load
constexpr uint32_t kGemmSel = 0;             // selector table
constexpr uint32_t kGemmSign = 0x10000;      // sign table
constexpr uint32_t kGemmTiles = 0x18000;     // weight tiles
constexpr uint32_t kGemmLdsLimit = 160 * 1024;
constexpr uint32_t kGemmOutOfRange = 0x80000000u;
constexpr int kGemmBufferWord3 = 0x00020000;

template <int BN>
struct GemmLayout {
  static constexpr uint32_t kStage = BN * kGemmRowBytes;
  static constexpr uint32_t kTotal = kGemmTiles + 2 * kStage;
  static constexpr int kNTiles = BN / 32;  // 16-wide MFMA tiles per consumer in n
  static_assert(kTotal <= kGemmLdsLimit, "LDS budget");
  static_assert((BN / 2) % 16 == 0, "consumer column block of whole MFMA tiles");
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

__device__ __forceinline__ void gemm_lds_store(uint32_t addr, const u32x4& v) {
  *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(static_cast<uintptr_t>(addr)) = v;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t gemm_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes,
                                           kGemmBufferWord3);
}

struct GemmArgs {
  const uint16_t* x;  // f16 or bf16 bits, [m, in_dim] (q for W8A8)
  const uint8_t* wb;
  const uint8_t* ws;
  float* out;
  const float* row_inv;  // W8A8 per-row inv scale, or null
  uint32_t m, out_dim, in_dim, bpr;
  uint32_t nk;      // ceil(in_dim / 64) stages
  uint32_t nk_pad;  // nk rounded up to whole pairs of code loads (2 kGemmGroup stages)
  uint32_t x_records, wb_records, ws_records;
};

// Builds the selector and sign tables (16 copies each) with the workgroup's
// 512 threads: 256 selector entries and 128 sign entries, one per thread.
__device__ __forceinline__ void build_gemm_tables(uint32_t tid) {
  if (tid >= 256 + 128) return;
  u32x4 v;
  uint32_t base;
  if (tid < 256) {
    // pair p of entry tid: bytes (2c, 2c+1) of level code c of each weight
    const uint32_t code = kGridCodesDev[tid];
    uint32_t w[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint32_t c0 = (code >> (4 * p)) & 3u, c1 = (code >> (4 * p + 2)) & 3u;
      w[p] = (2 * c0) | ((2 * c0 + 1) << 8) | ((2 * c1) << 16) | ((2 * c1 + 1) << 24);
    }
    v = u32x4{w[0], w[1], w[2], w[3]};
    base = kGemmSel + tid * 256;
  } else {
    const uint32_t i = tid - 256;
    const uint32_t s = i | ((__popc(i) & 1u) << 7);  // ksigns(i)
    uint32_t w[4];
#pragma unroll
    for (int p = 0; p < 4; ++p)
      w[p] = (((s >> (2 * p)) & 1u) ? 0x8000u : 0u) | (((s >> (2 * p + 1)) & 1u) ? 0x80000000u : 0u);
    v = u32x4{w[0], w[1], w[2], w[3]};
    base = kGemmSign + i * 256;
  }
#pragma unroll
  for (uint32_t k = 0; k < 16; ++k) gemm_lds_store(base + 16 * ((k + tid) & 15), v);
}

template <bool kBf16, int BN, bool kQ>
__global__ __launch_bounds__(kGemmThreads) void iq2xxs_gemm_kernel(GemmArgs a) {
  using L = GemmLayout<BN>;
  extern __shared__ __align__(16) uint8_t lds[];
  (void)lds;  // addressed through the layout constants above
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t m0 = blockIdx.y * kGemmBM;
  const uint32_t n0 = blockIdx.x * BN;

  build_gemm_tables(tid);

  if (wave >= 4) {
    // ======== producers: weight row n0 + p ========
    const uint32_t p = tid - kGemmProducer0;  // 0..255
    const bool row_ok = p < (uint32_t)BN && n0 + p < a.out_dim;
    const __amdgpu_buffer_rsrc_t rw = gemm_rsrc(a.wb, a.wb_records);
    const __amdgpu_buffer_rsrc_t rs = gemm_rsrc(a.ws, a.ws_records);
    const uint32_t row_blk = (n0 + p) * a.bpr;
    const uint32_t cs = 16 * (lane & 15);  // table copy of this lane
    const uint32_t wdst = kGemmTiles + p * kGemmRowBytes;
    const uint32_t swz = p & 7;

    // Codes of eight stages (blocks 2g, 2g+1 of the row: 128 bytes) and their
    // two scales.  Past the row's end the loads read zeros or the next row:
    // such stages are padding that no consumer reads.
    struct Codes {
      u32x4 q[kGemmGroup];
      uint32_t d[2];
    };
    // Scales first, in a fixed order with the codes: a stage then waits only
    // for loads of its own set, never for the set issued after it.
    auto load_codes = [&](uint32_t g, Codes& c) {
      const uint32_t blk = row_blk + 2 * g;
#pragma unroll
      for (int h = 0; h < 2; ++h)
        c.d[h] = __builtin_amdgcn_raw_buffer_load_b16(
            rs, row_ok ? (blk + h) * kScalesPerBlock : kGemmOutOfRange, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < kGemmGroup; ++j)
        c.q[j] = __builtin_amdgcn_raw_buffer_load_b128(
            rw, row_ok ? blk * kBytesPerBlock + 16 * j : kGemmOutOfRange, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    };
    // Dequantise one stage (sub-blocks 2s, 2s+1 of the row) into a tile.
    auto write_stage = [&](uint32_t tile, const u32x4& q, uint32_t dbits) {
      if (p >= (uint32_t)BN) return;
      const float d = half_bits_to_float((uint16_t)dbits);
      const uint32_t aux[2][2] = {{q.x, q.y}, {q.z, q.w}};
      u32x4 sel[2][4], sgn[2][4];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          // selector entry aux_g.byte(g): address (e << 8) | cs in one v_perm
          const uint32_t sa = kGemmSel + __builtin_amdgcn_perm(aux[h][0], cs, 0x0C0C0000u | ((4u + g) << 8));
          const uint32_t ia = kGemmSign + (__builtin_amdgcn_ubfe(aux[h][1], 7 * g, 7) << 8) + cs;
          sel[h][g] = gemm_lds_u4(sa);
          sgn[h][g] = gemm_lds_u4(ia);
        }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        // exact fp32 level values l * d * (2s + 1) / 8, then one rounding each
        const float tdf = d * (float)((aux[h][1] >> 27) | 1u) * 0.125f;
        const uint32_t pool_lo = pack2<kBf16>(8.0f * tdf, 25.0f * tdf);
        const uint32_t pool_hi = pack2<kBf16>(43.0f * tdf, 0.0f);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const u32x4 v = {__builtin_amdgcn_perm(pool_hi, pool_lo, sel[h][g].x) ^ sgn[h][g].x,
                           __builtin_amdgcn_perm(pool_hi, pool_lo, sel[h][g].y) ^ sgn[h][g].y,
                           __builtin_amdgcn_perm(pool_hi, pool_lo, sel[h][g].z) ^ sgn[h][g].z,
                           __builtin_amdgcn_perm(pool_hi, pool_lo, sel[h][g].w) ^ sgn[h][g].w};
          gemm_lds_store(tile + wdst + 16 * ((4 * h + g) ^ swz), v);
        }
      }
    };

    // Two code sets alternate (no register copies: a copy of a set still
    // being loaded would wait for it).  Stage s goes to tile s & 1; the
    // barrier after it publishes it.  The loop runs whole pairs of code loads
    // (nk_pad stages) so that its body is one straight-line sequence and the
    // compiler's wait counts stay exact.
    Codes c0, c1;
    load_codes(0, c0);
    load_codes(1, c1);
    __syncthreads();  // tables ready
    for (uint32_t g = 0; g * kGemmGroup < a.nk_pad; g += 2) {
#pragma unroll
      for (int j = 0; j < kGemmGroup; ++j) {
        write_stage((j & 1) * L::kStage, c0.q[j], c0.d[j >> 2]);
        __syncthreads();
      }
      load_codes(g + 2, c0);
#pragma unroll
      for (int j = 0; j < kGemmGroup; ++j) {
        write_stage((j & 1) * L::kStage, c1.q[j], c1.d[j >> 2]);
        __syncthreads();
      }
      load_codes(g + 3, c1);
    }
    return;
  }

  // ======== consumers ========
  const uint32_t wm = wave >> 1, wn = wave & 1;
  constexpr int NT = L::kNTiles;
  float4v acc[4][NT];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int jn = 0; jn < NT; ++jn) acc[i][jn] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

  // Activation fragments: rows m0 + 64 wm + 16 i + (lane & 15), the lane's 8
  // columns at 8 (lane >> 4) + 32 kh of the stage.  in_dim % 8 == 0 on this
  // path, so a 16-byte chunk is wholly in or out of the row.
  const __amdgpu_buffer_rsrc_t rx = gemm_rsrc(a.x, a.x_records);
  uint32_t arow[4];
  bool arow_ok[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t row = m0 + wm * 64 + i * 16 + (lane & 15);
    arow_ok[i] = row < a.m;
    arow[i] = row * a.in_dim * 2 + 16 * (lane >> 4);
  }
  const uint32_t acol = 8 * (lane >> 4);
  struct AFrags {
    u32x4 f[2][4];  // [kh][i]
  };
  auto load_a = [&](uint32_t st, AFrags& A) {
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool ok = arow_ok[i] && st * kGemmBK + 32 * kh + acol < a.in_dim;
        A.f[kh][i] = __builtin_amdgcn_raw_buffer_load_b128(
            rx, ok ? arow[i] + st * (kGemmBK * 2) + 64 * kh : kGemmOutOfRange, 0, 0);
      }
  };
  // Weight fragments of k-half kh from tile t: row wn*BN/2 + 16 jn + (lane & 15),
  // chunk (lane >> 4) + 4 kh stored at position chunk ^ (row & 7) = ... ^ (lane & 7).
  const uint32_t brow = kGemmTiles + (wn * (BN / 2) + (lane & 15)) * kGemmRowBytes;
  const uint32_t bofs0 = brow + 16 * (((lane >> 4) + 0) ^ (lane & 7));
  const uint32_t bofs1 = brow + 16 * (((lane >> 4) + 4) ^ (lane & 7));
  typedef u32x4 BFrags[NT];
  auto read_b = [&](uint32_t t, int kh, BFrags& F) {
    const uint32_t base = t * L::kStage + (kh ? bofs1 : bofs0);
#pragma unroll
    for (int jn = 0; jn < NT; ++jn) F[jn] = gemm_lds_u4(base + jn * 16 * kGemmRowBytes);
  };
  auto mfma_half = [&](const u32x4 (&A)[4], const BFrags& F) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int jn = 0; jn < NT; ++jn) acc[i][jn] = mfma16<kBf16>(A[i], F[jn], acc[i][jn]);
  };

  AFrags a0, a1;
  BFrags fb0, fb1;
  load_a(0, a0);
  load_a(1, a1);
  __syncthreads();  // tables ready
  __syncthreads();  // stage 0 published
  read_b(0, 0, fb0);
  // Two stages per trip (tiles 0 and 1, activation sets a0 and a1).  Each
  // stage: read its second k-half, MFMAs of the first half, the barrier that
  // publishes the next stage, read the next stage's first half, MFMAs of the
  // second half, then load the activations of the stage two ahead.
  // sched_barrier keeps the phases in this order.
  uint32_t s = 0;
  for (; s + 2 < a.nk; s += 2) {
    read_b(0, 1, fb1);
    __builtin_amdgcn_sched_barrier(0);
    mfma_half(a0.f[0], fb0);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    read_b(1, 0, fb0);
    __builtin_amdgcn_sched_barrier(0);
    mfma_half(a0.f[1], fb1);
    __builtin_amdgcn_sched_barrier(0);
    load_a(s + 2, a0);
    read_b(1, 1, fb1);
    __builtin_amdgcn_sched_barrier(0);
    mfma_half(a1.f[0], fb0);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    read_b(0, 0, fb0);
    __builtin_amdgcn_sched_barrier(0);
    mfma_half(a1.f[1], fb1);
    __builtin_amdgcn_sched_barrier(0);
    load_a(s + 3, a1);
  }
  // the last one or two stages
  read_b(0, 1, fb1);
  mfma_half(a0.f[0], fb0);
  mfma_half(a0.f[1], fb1);
  if (s + 1 < a.nk) {
    __syncthreads();
    read_b(1, 0, fb0);
    read_b(1, 1, fb1);
    mfma_half(a1.f[0], fb0);
    mfma_half(a1.f[1], fb1);
  }
  // the producers' barriers of the padding stages
  for (uint32_t e = a.nk; e < a.nk_pad; ++e) __syncthreads();

  // Epilogue: C[m][n], lane holds rows 4*(lane/16)+r, column lane%16 of each tile.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t row = m0 + wm * 64 + i * 16 + 4 * (lane >> 4) + r;
      if (row >= a.m) continue;
      const float scale = kQ ? a.row_inv[row] : 1.0f;
#pragma unroll
      for (int jn = 0; jn < NT; ++jn) {
        const uint32_t col = n0 + wn * (BN / 2) + jn * 16 + (lane & 15);
        if (col < a.out_dim) {
          float v = acc[i][jn][r];
          if constexpr (kQ) v = v / scale;
          a.out[(size_t)row * a.out_dim + col] = v;
        }
      }
    }
  }
}

// W8A8 pre-pass: q = clamp(round_half_away(x * inv_row), -127, 127) in the
// activation's type (exact), eight activations per thread.
template <bool kBf16>
__global__ __launch_bounds__(256) void iq2xxs_quantize_rows_kernel(const uint16_t* x, uint32_t m,
                                                                   uint32_t in_dim,
                                                                   const float* row_inv,
                                                                   uint16_t* q) {
  const uint32_t chunks_per_row = in_dim / 8;
  const uint64_t total = (uint64_t)m * chunks_per_row;
  for (uint64_t c = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; c < total;
       c += (uint64_t)gridDim.x * blockDim.x) {
    const uint32_t row = (uint32_t)(c / chunks_per_row);
    const float inv = row_inv[row];
    const u32x4 v = *reinterpret_cast<const u32x4*>(x + c * 8);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float lo = kBf16 ? bf16_bits_to_float((uint16_t)w[k]) : half_bits_to_float((uint16_t)w[k]);
      const float hi = kBf16 ? bf16_bits_to_float((uint16_t)(w[k] >> 16))
                             : half_bits_to_float((uint16_t)(w[k] >> 16));
      const float ql = fminf(fmaxf(roundf(lo * inv), -127.0f), 127.0f);
      const float qh = fminf(fmaxf(roundf(hi * inv), -127.0f), 127.0f);
      o[k] = pack2<kBf16>(ql, qh);
    }
    *reinterpret_cast<u32x4*>(q + c * 8) = u32x4{o[0], o[1], o[2], o[3]};
  }
}

// The activation fragments are loaded in 16-byte chunks that are wholly in or
// out of range (in_dim % 8 == 0), and every buffer offset stays below
// kGemmOutOfRange.
bool gemm_supported(uint32_t m, uint32_t out_dim, uint32_t in_dim) {
  return in_dim % 8 == 0 && (uint64_t)m * in_dim * 2 < kGemmOutOfRange - 4096 &&
         (uint64_t)out_dim * ((in_dim + kQK - 1) / kQK) * kBytesPerBlock < kGemmOutOfRange - 4096;
}

size_t gemm_w8a8_scratch_bytes(uint32_t m, uint32_t in_dim) { return (size_t)m * in_dim * 2; }

template <bool kBf16, int BN, bool kQ>
static hipError_t launch_gemm_t(const GemmArgs& a, hipStream_t stream) {
  using L = GemmLayout<BN>;
  static std::atomic<bool> attr_set{false};
  if (!attr_set.load()) {
    hipError_t e =
        hipFuncSetAttribute(reinterpret_cast<const void*>(&iq2xxs_gemm_kernel<kBf16, BN, kQ>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGemmLdsLimit);
    if (e != hipSuccess) return e;
    attr_set.store(true);
  }
  dim3 grid((a.out_dim + BN - 1) / BN, (a.m + kGemmBM - 1) / kGemmBM);
  hipLaunchKernelGGL((iq2xxs_gemm_kernel<kBf16, BN, kQ>), grid, dim3(kGemmThreads), L::kTotal,
                     stream, a);
  return hipGetLastError();
}

hipError_t launch_iq2xxs_gemm(const void* x, int x_dtype, uint32_t m, const uint8_t* wb,
                              const uint8_t* ws, float* out, uint32_t out_dim, uint32_t in_dim,
                              const float* row_inv, void* xq, hipStream_t stream) {
  const bool bf = x_dtype == 2;
  if (row_inv) {
    const uint64_t chunks = (uint64_t)m * (in_dim / 8);
    const uint32_t blocks = (uint32_t)((chunks + 255) / 256 < 8192 ? (chunks + 255) / 256 : 8192);
    if (bf)
      hipLaunchKernelGGL(iq2xxs_quantize_rows_kernel<true>, dim3(blocks), dim3(256), 0, stream,
                         static_cast<const uint16_t*>(x), m, in_dim, row_inv,
                         static_cast<uint16_t*>(xq));
    else
      hipLaunchKernelGGL(iq2xxs_quantize_rows_kernel<false>, dim3(blocks), dim3(256), 0, stream,
                         static_cast<const uint16_t*>(x), m, in_dim, row_inv,
                         static_cast<uint16_t*>(xq));
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    x = xq;
  }
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
  a.nk_pad = (a.nk + 2 * kGemmGroup - 1) / (2 * kGemmGroup) * (2 * kGemmGroup);
  a.x_records = m * in_dim * 2;
  a.wb_records = out_dim * a.bpr * kBytesPerBlock;
  a.ws_records = out_dim * a.bpr * kScalesPerBlock;
  // tile width: 224 when it fills the CUs better than 128
  const uint64_t mt = (m + kGemmBM - 1) / kGemmBM;
  const uint64_t t224 = mt * ((out_dim + 223) / 224), t128 = mt * ((out_dim + 127) / 128);
  const bool wide = t224 >= 200 || t224 * 224 <= t128 * 128;
  if (row_inv) {
    if (wide)
      return bf ? launch_gemm_t<true, 224, true>(a, stream) : launch_gemm_t<false, 224, true>(a, stream);
    return bf ? launch_gemm_t<true, 128, true>(a, stream) : launch_gemm_t<false, 128, true>(a, stream);
  }
  if (wide)
    return bf ? launch_gemm_t<true, 224, false>(a, stream) : launch_gemm_t<false, 224, false>(a, stream);
  return bf ? launch_gemm_t<true, 128, false>(a, stream) : launch_gemm_t<false, 128, false>(a, stream);
}

}  // namespace cmk
