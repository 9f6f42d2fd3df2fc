// iq2xxs_gemm.hip — prefill-shaped IQ2_XXS matmul (large m).
//
// out[m, n] = sum_k x[m, k] * W[n, k], W dequantised per tile into LDS as
// f16, then fed to v_mfma_f32_16x16x32_f16 with fp32 accumulation.  Every
// dequantised value is the single round-to-nearest-even of the exact weight
// d*(2s+1)*g/8, i.e. exactly what iq2_dequantize_to_f16 produces.  The
// activations reach the kernel as f16: f16 x as given; bf16 x staged as f16
// after scaling each row by a power of two (exact); f32 x staged as f16 head /
// tail row pairs (about 22 bits of each value); W8A8 rows as their integer q.
//
// The reference has no dedicated prefill kernel: its iq2_xxs_matmul_kernel
// (src/metal_src/iq2_matmul.metal:188-240) serves every m with one thread per
// output.  This kernel is the large-m replacement on the same boundary.
//
// W8A8 (iq2_matmul.metal:436-499): a pre-pass writes q = clamp(round(x*inv),
// +-127) (exact small integers in f16) to the caller's workspace; the
// GEMM runs on q and divides each fp32 result by its row's inv, i.e.
// sum(q/inv * w) up to fp32 rounding.
//
// Work split.  A workgroup computes a BM x BN tile of out; k advances in
// stages of 32 columns (one 32-weight sub-block of every weight row).  For
// m = 512, n = 14336 the tile is 256 x 112: 2 x 128 = 256 workgroups, one per
// CU, and every weight sub-block is dequantised by two CUs only (256 x 128 or
// 128 x 128 where those fill the CUs better; see plan_gemm).
//  * Waves 0-3 (consumers) each own a 64 x BN/WN block of the tile.  They only
//    read fragments from LDS and issue MFMAs: on gfx950 a wave's VALU work and
//    memory-issue stalls do not overlap its own MFMAs, while work of another
//    wave on the same SIMD does.
//  * Waves 4-7 (producers) dequantise the weights: two lanes per weight row,
//    two 8-weight groups each per stage; the table reads of the next stage
//    are issued after the current stage is written and stay in flight across
//    the barrier.  They also copy the activations two stages ahead into four
//    rotating LDS tiles with global-to-LDS DMA (buffer_load ... lds).  A
//    barrier per stage publishes it.
// Layout and load shapes follow measurements on gfx950: vector loads run at
// full rate only when each quad of lanes reads 64 contiguous bytes; LDS reads
// run at about 270 B/clk per CU when conflict-free, writes at about 100 B/clk;
// VALU work of a wave sharing a SIMD with an MFMA stream issues at about one
// instruction per 6-8 clocks.
//
// LDS layout (64 KB aligned tables, so one v_perm forms a selector address):
//   [0, 64K)      selector table: 256 codebook entries x 16 copies x 16 B
//                 (lane l reads copy l & 15: conflict-free)
//   [64K, 80K)    sign table: 128 sign indices x 8 copies x 16 B (lane l
//                 reads copy l & 7; lanes l and l + 8 may meet in a bank)
//   [80K, ...)    four activation tiles (BM rows x 64 B), then two weight
//                 tiles (BN rows x 64 B); 16-byte chunk c of row r is stored
//                 at position c ^ ((r >> 1) & 3), which makes the MFMA
//                 fragment reads conflict-free.
//
// Dequantisation of a sub-block (32 weights of one row): the three level
// values RNE(l*d*(2s+1)/8), l in {8, 25, 43}, are formed in fp32 (exact
// products) and packed into two dwords; the selector table (one v_perm
// selector per pair of weights of each codebook entry) then assembles each
// pair with one v_perm, and the sign table (16-bit sign masks) applies ksigns
// with one xor.
//
// Bound: MFMA (arithmetic intensity ~1200 flop/B at m = 512).
#include <algorithm>
#include <atomic>
#include <cstdint>
#include <initializer_list>
#include <type_traits>

#include "iq2xxs_device.h"
#include "iq2xxs_kernels.h"

namespace cmk {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kGemmBK = 32;                  // columns of k per stage
constexpr int kGemmThreads = 512;
constexpr int kGemmProducer0 = 256;          // first producer thread
constexpr int kGemmUnroll = 16;              // producer steps per loop trip
constexpr uint32_t kGemmSel = 0;             // selector table
constexpr uint32_t kGemmSign = 0x10000;      // sign table
constexpr uint32_t kGemmSignCopies = 8;
constexpr uint32_t kGemmTiles = 0x14000;     // activation and weight tiles
constexpr uint32_t kGemmLdsLimit = 160 * 1024;
constexpr uint32_t kGemmOutOfRange = 0x80000000u;
constexpr int kGemmBufferWord3 = 0x00020000;

// Tile geometry: BM x BN per workgroup, consumer waves WM x WN of 64 x TN.
template <int BM, int BN>
struct GemmLayout {
  static constexpr int WM = BM / 64, WN = 4 / WM, TN = BN / WN;
  static constexpr int NT = TN / 16;                  // 16-wide MFMA tiles per consumer in n
  static constexpr uint32_t kAStage = BM * 64;        // one activation tile
  static constexpr uint32_t kBStage = BN * 64;        // one weight tile
  static constexpr uint32_t kA = kGemmTiles;          // four activation tiles
  static constexpr uint32_t kB = kA + 4 * kAStage;    // two weight tiles
  static constexpr uint32_t kTotal = kB + 2 * kBStage;
  static constexpr int kDma = BM / 64;                // DMA instructions per producer wave per stage
  static_assert(WM * WN == 4 && TN % 16 == 0, "four consumer waves of whole MFMA tiles");
  static_assert(2 * BN <= 256, "two producer lanes per weight row");
  static_assert(kTotal <= kGemmLdsLimit, "LDS budget");
};

__device__ __forceinline__ float4v mfma16(const u32x4& a, const u32x4& b, float4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a),
                                                __builtin_bit_cast(half8, b), c, 0, 0, 0);
}

// Two floats as a packed pair of f16 (each one round-to-nearest-even).
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 v = {(_Float16)lo, (_Float16)hi};
  return __builtin_bit_cast(uint32_t, v);
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
  const uint16_t* x;  // f16 bits, [m, in_dim] (staged rows, or q for W8A8)
  const uint8_t* wb;
  const uint8_t* ws;
  float* out;
  const float* row_inv;  // W8A8 per-row inv scale, or null
  uint32_t m, out_dim, in_dim, bpr;
  uint32_t nk;      // ceil(in_dim / 32) stages
  uint32_t nk_pad;  // 1 + (nk - 1) rounded up to whole producer loop trips
  uint32_t x_records, wb_records, ws_records;
  // Split over k (grid z): workgroup z covers blocks [z, z + 1) * split_blocks
  // of each row and writes its partial products at out + z * out_split.
  uint32_t split_blocks;
  uint64_t out_split;
};

// Barrier of the main loop without a memory fence: waits until at most kVm of
// this wave's vector-memory operations and at most kLgkm of its LDS accesses
// are in flight (both complete in issue order), then s_barrier.  A workgroup
// fence would also wait for the activation DMA of later stages, which is
// meant to stay in flight.  The memory clobber keeps the compiler from moving
// LDS accesses across it.
template <int kVm, int kLgkm = 0>
__device__ __forceinline__ void stage_barrier() {
  static_assert(kVm >= 0 && kVm < 64 && kLgkm >= 0 && kLgkm < 16, "waitcnt fields");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(%1)\n\ts_barrier" ::"n"(kVm), "n"(kLgkm) : "memory");
}

// Builds the selector table (16 copies) and the sign table (8 copies) with the
// workgroup's 512 threads: 256 selector entries and 128 sign entries, one per
// thread.
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
    base = kGemmSign + i * (16 * kGemmSignCopies);
#pragma unroll
    for (uint32_t k = 0; k < kGemmSignCopies; ++k)
      gemm_lds_store(base + 16 * ((k + i) & (kGemmSignCopies - 1)), v);
    return;
  }
#pragma unroll
  for (uint32_t k = 0; k < 16; ++k) gemm_lds_store(base + 16 * ((k + tid) & 15), v);
}

// kQ: 0 = plain output; 1 = output row r divided by row_inv[r]; 2 = staged
// row pairs (2r: the f16 head of x_r * row_inv[r], 2r + 1: the f16 of what
// the head leaves), output row r = (C[2r] + C[2r+1]) / row_inv[r].
template <int BM, int BN, int kQ>
__global__ __launch_bounds__(kGemmThreads) void iq2xxs_gemm_kernel(GemmArgs a) {
  using L = GemmLayout<BM, BN>;
  extern __shared__ __align__(16) uint8_t lds[];
  (void)lds;  // addressed through the layout constants above
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t m0 = blockIdx.y * BM;
  const uint32_t n0 = blockIdx.x * BN;
  const uint32_t blk0 = blockIdx.z * a.split_blocks;  // first block of this k split
  const uint32_t k0 = blk0 * kQK;
  // Stages of this workgroup's k range.  Splits cover split_blocks blocks each
  // except the last, which ends at the row's end (an uneven split is shorter).
  uint32_t nk = a.nk, nk_pad = a.nk_pad;
  if (a.split_blocks) {
    const uint32_t k_end = min(k0 + a.split_blocks * (uint32_t)kQK, a.in_dim);
    nk = (k_end - k0 + kGemmBK - 1) / kGemmBK;
    nk_pad = 1 + (nk - 1 + kGemmUnroll - 1) / kGemmUnroll * kGemmUnroll;
  }

  build_gemm_tables(tid);

  if (wave >= 4) {
    // ======== producers: lanes 2r, 2r + 1 own weight row n0 + r ========
    const uint32_t p = tid - kGemmProducer0;  // 0..255
    // row, group pair (groups 2h, 2h + 1).  When 2 * BN < 256 the lanes past
    // the tile redo rows 0.. (same loads, same values written to the same
    // place), which keeps every lane on the same branch-free path.
    const uint32_t r = (p >> 1) % (uint32_t)BN, h = p & 1;
    const bool row_ok = n0 + r < a.out_dim;
    const __amdgpu_buffer_rsrc_t rw = gemm_rsrc(a.wb, a.wb_records);
    const __amdgpu_buffer_rsrc_t rs = gemm_rsrc(a.ws, a.ws_records);
    const uint32_t row_blk = (n0 + r) * a.bpr + blk0;
    const uint32_t cs = 16 * (lane & 15);  // selector-table copy of this lane
    const uint32_t css = 16 * (lane & (kGemmSignCopies - 1));  // sign-table copy
    const uint32_t wdst0 = L::kB + r * 64 + 16 * ((2 * h + 0) ^ ((r >> 1) & 3));
    const uint32_t wdst1 = L::kB + r * 64 + 16 * ((2 * h + 1) ^ ((r >> 1) & 3));

    // Codes of one block (eight stages) and its scale.  Stages past nk (the
    // padding that completes the last loop trip) load codes past this
    // workgroup's k range -- zeros past the buffer's end, or the blocks that
    // follow -- and are written to LDS but never read: the consumers stop at
    // stage nk.
    struct Codes {
      u32x4 q[4];  // sub-blocks 2j, 2j + 1 of the block
      uint32_t d;
    };
    // The scale first and the order pinned: a stage then waits only for
    // loads of its own set.
    auto load_codes = [&](uint32_t g, Codes& c) {
      const uint32_t blk = row_blk + g;
      c.d = __builtin_amdgcn_raw_buffer_load_b16(
          rs, row_ok ? blk * kScalesPerBlock : kGemmOutOfRange, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        c.q[j] = __builtin_amdgcn_raw_buffer_load_b128(
            rw, row_ok ? blk * kBytesPerBlock + 16 * j : kGemmOutOfRange, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    };
    // Dequantisation of this lane's two groups of a sub-block, in two parts:
    // the table reads, then the assembly into weight tile t (one step later).
    struct Tables {
      u32x4 sel[2], sgn[2];
    };
    auto read_tables = [&](uint32_t aux_g, uint32_t aux_s, Tables& T) {
#pragma unroll
      for (int gg = 0; gg < 2; ++gg) {
        const uint32_t g = 2 * h + gg;
        // selector entry aux_g.byte(g): address (e << 8) | cs in one v_perm
        T.sel[gg] = gemm_lds_u4(kGemmSel + __builtin_amdgcn_perm(aux_g, cs, 0x0C0C0000u | ((4u + g) << 8)));
        T.sgn[gg] = gemm_lds_u4(kGemmSign + __builtin_amdgcn_ubfe(aux_s, 7 * g, 7) * (16 * kGemmSignCopies) + css);
      }
    };
    // The level values l * d * (2s + 1) / 8 of a sub-block, l in {8, 25, 43},
    // each rounded once to f16 (exact in fp32 before the rounding): the
    // conversion of s * 2^28 + 2^27 - 1 rounds to (2s + 1) * 2^27 exactly,
    // and d * 2^-30 is exact.
    struct Pool {
      uint32_t lo, hi;
    };
    auto level_pool = [](uint32_t aux_s, uint32_t dbits) {
      const float s27 = (float)((aux_s & 0xF0000000u) | 0x07FFFFFFu);
      const float tdf = s27 * (half_bits_to_float((uint16_t)dbits) * 0x1p-30f);
      return Pool{pack2(8.0f * tdf, 25.0f * tdf), pack2(43.0f * tdf, 0.0f)};
    };
    // group pair gg of weight tile t from the tables read one step earlier
    auto store_group = [&](int gg, uint32_t t, const Pool& P, const Tables& T) {
      const u32x4 v = {__builtin_amdgcn_perm(P.hi, P.lo, T.sel[gg].x) ^ T.sgn[gg].x,
                       __builtin_amdgcn_perm(P.hi, P.lo, T.sel[gg].y) ^ T.sgn[gg].y,
                       __builtin_amdgcn_perm(P.hi, P.lo, T.sel[gg].z) ^ T.sgn[gg].z,
                       __builtin_amdgcn_perm(P.hi, P.lo, T.sel[gg].w) ^ T.sgn[gg].w};
      gemm_lds_store((gg ? wdst1 : wdst0) + t * L::kBStage, v);
    };
    // codes of the stage at sub-block sb of its block, from set c
    auto aux_of = [](const Codes& c, int sb, uint32_t& aux_g, uint32_t& aux_s) {
      const u32x4& q = c.q[sb >> 1];
      aux_g = (sb & 1) ? q.z : q.x;
      aux_s = (sb & 1) ? q.w : q.y;
    };

    // Activations of stage s by DMA into tile s & 3: producer wave pw copies
    // row groups kDma * pw + k (16 rows of 64 bytes each); lane l lands at
    // byte 16 l of the group, i.e. row (l >> 2), position l & 3, which holds
    // chunk (l & 3) ^ ((row >> 1) & 3) = (l & 3) ^ ((l >> 3) & 3).  A quad of
    // lanes reads one row's 64 contiguous bytes.  Rows past m and columns past
    // in_dim read as zeros: a row past m starts at kGemmOutOfRange, which
    // stays out of range at every stage's offset, and a stage that reaches
    // past in_dim checks each lane's chunk.
    const uint32_t pw = wave - 4;
    const __amdgpu_buffer_rsrc_t rx = gemm_rsrc(a.x, a.x_records);
    const uint32_t xkc = (lane & 3) ^ ((lane >> 3) & 3);
    // (fixed-size arrays: with arrays sized by L::kDma next to the DMA builtin,
    // hipcc's host pass silently emits no stub for the kernel)
    uint32_t xsrc[4];
    static_assert(L::kDma <= 4, "activation DMA per producer");
#pragma unroll
    for (int k = 0; k < L::kDma; ++k) {
      const uint32_t row = 16 * (L::kDma * pw + k) + (lane >> 2);
      xsrc[k] = m0 + row < a.m ? ((m0 + row) * a.in_dim + k0 + 8 * xkc) * 2 : kGemmOutOfRange;
    }
    // Instruction k of stage s's DMA; `whole`: every column of the stage lies
    // before in_dim (no per-lane check).
    auto dma_one = [&](uint32_t s, int k, bool whole) {
      if (k < L::kDma) {
        const uint32_t dst = L::kA + (s & 3) * L::kAStage + (L::kDma * pw + k) * 1024;
        const bool col_ok = whole || k0 + kGemmBK * s + 8 * xkc < a.in_dim;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rx, reinterpret_cast<__attribute__((address_space(3))) void*>(static_cast<uintptr_t>(dst)),
            16, col_ok ? xsrc[k] + 64 * s : kGemmOutOfRange, 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    auto dma_x = [&](uint32_t s) {
#pragma unroll
      for (int k = 0; k < L::kDma; ++k) dma_one(s, k, false);
    };

    Codes c0, c1;
    Tables t0, t1;
    load_codes(0, c0);
    load_codes(1, c1);
    dma_x(0);
    __syncthreads();  // tables ready
    // prologue: stage 0, the activations of stages 1 and 2, and the table
    // reads of stage 1
    dma_x(1);
    dma_x(2);
    {
      uint32_t g0, s0v, g1, s1v;
      aux_of(c0, 0, g0, s0v);
      read_tables(g0, s0v, t0);
      aux_of(c0, 1, g1, s1v);
      read_tables(g1, s1v, t1);
      const Pool P = level_pool(s0v, c0.d);
      store_group(0, 0, P, t0);
      store_group(1, 0, P, t0);
    }
    __syncthreads();  // stage 0 published (with its activations)
    // Step s issues the DMA of the activations of stage s + 2 (their tile,
    // (s + 2) & 3, held stage s - 2, whose fragments were read before the
    // previous barrier), writes stage s (weight tile s & 1) from the tables
    // read one step earlier, then reads the tables of stage s + 1, and after
    // the last stage of a block reloads that code set with the block two
    // ahead.  The DMA instructions are spread over the step (one before the
    // level values, one before each group store, one after): a wave that
    // issues them back to back waits for the memory pipeline to take each
    // one, and its dequantisation waits with it.  Its barrier publishes
    // stage s: the weight writes must be done (the four table reads issued
    // after them may stay in flight), and the DMA of stage s (issued two
    // steps earlier) must have landed while the DMA of stages s + 1 and
    // s + 2 and code loads may stay in flight.  A trip covers kGemmUnroll
    // steps from s0 = 1 (mod 16), so every set choice and wait count below is
    // a compile-time constant and the body is one straight-line sequence
    // (exact wait counts).  `whole`: the trip's DMA stages all end at or
    // before in_dim.
    auto trip = [&](uint32_t s0, auto whole_t) {
      constexpr bool kWhole = decltype(whole_t)::value;
#pragma unroll
      for (int j = 0; j < kGemmUnroll; ++j) {
        const uint32_t s = s0 + j;
        const int cj = 1 + j;  // s modulo 16
        Codes& cc = ((cj >> 3) & 1) ? c1 : c0;        // block of stage s
        Codes& cn = (((cj + 1) >> 3) & 1) ? c1 : c0;  // block of stage s + 1
        Tables& tc = (cj & 1) ? t1 : t0;
        Tables& tn = (cj & 1) ? t0 : t1;
        uint32_t gn, sn, gc, sc;
        aux_of(cc, cj & 7, gc, sc);
        dma_one(s + 2, 0, kWhole);
        const Pool P = level_pool(sc, cc.d);
        __builtin_amdgcn_sched_barrier(0);
        dma_one(s + 2, 1, kWhole);
        store_group(0, (uint32_t)(cj & 1), P, tc);
        __builtin_amdgcn_sched_barrier(0);
        dma_one(s + 2, 2, kWhole);
        store_group(1, (uint32_t)(cj & 1), P, tc);
        __builtin_amdgcn_sched_barrier(0);
        dma_one(s + 2, 3, kWhole);
        aux_of(cn, (cj + 1) & 7, gn, sn);
        read_tables(gn, sn, tn);
        if ((cj & 7) == 7) load_codes((s >> 3) + 2, cc);
        // in flight after the DMA of stage s: code loads of steps s - 2 and
        // s - 1, the DMA of stages s + 1 and s + 2, code loads of step s (5
        // loads per code set; at most one of the three steps loads codes).
        // cj is a constant once the loop is unrolled, so one branch remains.
        if (((cj - 2) & 7) == 7 || ((cj - 1) & 7) == 7 || (cj & 7) == 7)
          stage_barrier<2 * L::kDma + 5, 4>();
        else
          stage_barrier<2 * L::kDma, 4>();
      }
    };
    for (uint32_t s0 = 1; s0 < nk_pad; s0 += kGemmUnroll) {
      if (k0 + kGemmBK * (s0 + kGemmUnroll + 2) <= a.in_dim)
        trip(s0, std::true_type());
      else
        trip(s0, std::false_type());
    }
    return;
  }

  // ======== consumers ========
  constexpr int NT = L::NT;
  const uint32_t wm = wave / L::WN, wn = wave % L::WN;
  float4v acc[4][NT];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int jn = 0; jn < NT; ++jn) acc[i][jn] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

  // Fragment addresses: row (16-aligned base) + (lane & 15), chunk lane >> 4,
  // stored at position chunk ^ ((row >> 1) & 3) = chunk ^ ((lane >> 1) & 3).
  const uint32_t fpos = 16 * ((lane >> 4) ^ ((lane >> 1) & 3));
  const uint32_t aofs = L::kA + (wm * 64 + (lane & 15)) * 64 + fpos;
  const uint32_t bofs = L::kB + (wn * L::TN + (lane & 15)) * 64 + fpos;
  struct Frags {
    u32x4 a[4], b[NT];
  };
  // fragments of stage s: activation tile abuf (s & 3), weight tile s & 1
  auto read_frags = [&](uint32_t abuf, uint32_t s, Frags& F) {
    const uint32_t abase = aofs + abuf * L::kAStage;
#pragma unroll
    for (int i = 0; i < 4; ++i) F.a[i] = gemm_lds_u4(abase + i * 16 * 64);
    const uint32_t bbase = bofs + (s & 1) * L::kBStage;
#pragma unroll
    for (int jn = 0; jn < NT; ++jn) F.b[jn] = gemm_lds_u4(bbase + jn * 16 * 64);
  };
  auto mfma_rows = [&](const Frags& F, int i0) {
#pragma unroll
    for (int i = i0; i < i0 + 2; ++i)
#pragma unroll
      for (int jn = 0; jn < NT; ++jn) acc[i][jn] = mfma16(F.a[i], F.b[jn], acc[i][jn]);
  };
  // Rows 2-3 of stage F with the fragment reads of the next stage (into Fn)
  // interleaved one per MFMA, so that the MFMA pipe restarts right after a
  // barrier instead of waiting behind the read issue.
  auto mfma_rows_reading = [&](const Frags& F, uint32_t abuf, uint32_t s_next, Frags& Fn) {
    const uint32_t abase = aofs + abuf * L::kAStage;
    const uint32_t bbase = bofs + (s_next & 1) * L::kBStage;
    int k = 0;
#pragma unroll
    for (int i = 2; i < 4; ++i)
#pragma unroll
      for (int jn = 0; jn < NT; ++jn) {
        if (k < 4)
          Fn.a[k] = gemm_lds_u4(abase + k * 16 * 64);
        else if (k < 4 + NT)
          Fn.b[k - 4] = gemm_lds_u4(bbase + (k - 4) * 16 * 64);
        acc[i][jn] = mfma16(F.a[i], F.b[jn], acc[i][jn]);
        __builtin_amdgcn_sched_barrier(0);
        ++k;
      }
  };

  auto next_tile = [](uint32_t b) { return (b + 1) & 3u; };
  // Rows 0-1 of stage F, one MFMA after another.
  auto mfma_rows01 = [&](const Frags& F) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int jn = 0; jn < NT; ++jn) {
        acc[i][jn] = mfma16(F.a[i], F.b[jn], acc[i][jn]);
        __builtin_amdgcn_sched_barrier(0);
      }
  };

  __syncthreads();  // tables ready
  __syncthreads();  // stage 0 published
  // Stage s: MFMAs of rows 0-1, the barrier that publishes stage s + 1, the
  // reads of stage s + 1 (landing while rows 2-3 of stage s run).
  // sched_barrier keeps the phases in this order.
  Frags f0, f1;
  uint32_t ab = 0;  // activation tile of stage s
  read_frags(ab, 0, f0);
  uint32_t s = 0;
  for (; s + 2 < nk; s += 2) {
    mfma_rows01(f0);
    stage_barrier<0>();
    ab = next_tile(ab);
    mfma_rows_reading(f0, ab, s + 1, f1);
    mfma_rows01(f1);
    stage_barrier<0>();
    ab = next_tile(ab);
    mfma_rows_reading(f1, ab, s + 2, f0);
  }
  // the last one or two stages
  mfma_rows(f0, 0);
  mfma_rows(f0, 2);
  if (s + 1 < nk) {
    __syncthreads();
    read_frags(next_tile(ab), s + 1, f1);
    mfma_rows(f1, 0);
    mfma_rows(f1, 2);
  }
  // the producers' barriers of the padding stages
  for (uint32_t e = nk; e < nk_pad; ++e) __syncthreads();

  // Epilogue: C[m][n], lane holds rows 4*(lane/16)+r, column lane%16 of each tile
  // (so a staged pair 2r, 2r + 1 sits in one lane).
  float* const out = a.out + (size_t)blockIdx.z * a.out_split;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int r = 0; r < 4; r += (kQ == 2 ? 2 : 1)) {
      const uint32_t row = m0 + wm * 64 + i * 16 + 4 * (lane >> 4) + r;
      if (row >= a.m) continue;  // a.m is even for kQ == 2: row + 1 is in range too
      const uint32_t orow = kQ == 2 ? row >> 1 : row;
      const float scale = kQ ? a.row_inv[orow] : 1.0f;
#pragma unroll
      for (int jn = 0; jn < NT; ++jn) {
        const uint32_t col = n0 + wn * L::TN + jn * 16 + (lane & 15);
        if (col < a.out_dim) {
          float v = acc[i][jn][r];
          if constexpr (kQ == 2) v += acc[i][jn][r + 1];
          if constexpr (kQ != 0) v = v / scale;
          out[(size_t)orow * a.out_dim + col] = v;
        }
      }
    }
  }
}

// W8A8 pre-pass: q = clamp(round_half_away(x * inv_row), -127, 127) from f16
// or bf16 activations, written as f16 (exact), eight activations per thread.
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
      const float ql = quant_w8a8(lo, inv);
      const float qh = quant_w8a8(hi, inv);
      o[k] = pack2(ql, qh);
    }
    *reinterpret_cast<u32x4*>(q + c * 8) = u32x4{o[0], o[1], o[2], o[3]};
  }
}

// bf16 rows for the f16 GEMM (f16 weights carry 11 significant bits, bf16
// weights 8): one workgroup per row scales the row by the power of two inv
// that brings its largest finite magnitude into [2^14, 2^15) and writes
// x * inv as f16, exact for every value at or above 2^-31 of the row's
// largest (bf16 has 8 significant bits); inv goes to row_inv, which the
// epilogue divides by.  NaN and infinities stay what they are.
__global__ __launch_bounds__(256) void iq2xxs_scale_stage_bf16_rows_kernel(
    const uint16_t* __restrict__ x, uint32_t in_dim, float* __restrict__ row_inv,
    uint16_t* __restrict__ q) {
  __shared__ uint32_t s_red[4];
  const uint32_t row = blockIdx.x;
  const u32x4* r8 = reinterpret_cast<const u32x4*>(x + (size_t)row * in_dim);
  // magnitudes as integer bits (bf16 bits << 16); NaN and infinities count as 0
  auto fin = [](uint32_t h) {
    const uint32_t b = (h << 16) & kAbsMask;
    return b < kInfBits ? b : 0u;
  };
  uint32_t mb = 0;
#pragma unroll 4
  for (uint32_t c = threadIdx.x; c < in_dim / 8; c += 256) {
    const u32x4 v = r8[c];
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) mb = max(mb, max(fin(w[k] & 0xFFFFu), fin(w[k] >> 16)));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mb = max(mb, (uint32_t)__shfl_xor((int)mb, off));
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = mb;
  __syncthreads();
  const float mx = __uint_as_float(max(max(s_red[0], s_red[1]), max(s_red[2], s_red[3])));
  const float inv = mx > 0.0f ? ldexpf(1.0f, min(14 - ilogbf(mx), 126)) : 1.0f;
  if (threadIdx.x == 0) row_inv[row] = inv;
  u32x4* const o8 = reinterpret_cast<u32x4*>(q + (size_t)row * in_dim);
#pragma unroll 4
  for (uint32_t c = threadIdx.x; c < in_dim / 8; c += 256) {
    const u32x4 v = r8[c];
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      o[k] = pack2(bf16_bits_to_float((uint16_t)w[k]) * inv,
                   bf16_bits_to_float((uint16_t)(w[k] >> 16)) * inv);
    o8[c] = u32x4{o[0], o[1], o[2], o[3]};
  }
}

// f32 W8A8 staging pre-pass, eight activations per thread: q = clamp(
// round_half_away(x * row_inv[r]), -127, 127) to staged row r (exact in f16).
__global__ __launch_bounds__(256) void iq2xxs_stage_f32_w8a8_kernel(const float* x, uint32_t m,
                                                                    uint32_t in_dim,
                                                                    const float* row_inv,
                                                                    uint16_t* q) {
  const uint32_t chunks_per_row = in_dim / 8;
  const uint64_t total = (uint64_t)m * chunks_per_row;
  for (uint64_t c = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; c < total;
       c += (uint64_t)gridDim.x * blockDim.x) {
    const float inv = row_inv[c / chunks_per_row];
    const float4 lo = *reinterpret_cast<const float4*>(x + c * 8);
    const float4 hi = *reinterpret_cast<const float4*>(x + c * 8 + 4);
    const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      o[k] = pack2(quant_w8a8(v[2 * k], inv), quant_w8a8(v[2 * k + 1], inv));
    *reinterpret_cast<u32x4*>(q + c * 8) = u32x4{o[0], o[1], o[2], o[3]};
  }
}

// f32 staging pass, one workgroup of 256 per row r: the power of two
// inv = 2^(14 - floor(log2 max|x_r|)) (capped at 2^126; 1 for a zero max),
// with the max taken over the row's finite values, brings the row's largest
// finite magnitude into [2^14, 2^15), so v = x * inv is exact.  The row is
// then read again (from L2) and staged as the f16 head h = rne(v) in row 2r
// and the f16 tail rne(v - h) in row 2r + 1 (v - h is exact in fp32): the
// pair carries v to about 2^-22 of its size.  A NaN or an infinity is staged
// as itself in the head with a zero tail, so the MFMA products carry it to the
// output as the reference's fp32 loop would.
__global__ __launch_bounds__(256) void iq2xxs_scale_stage_f32_rows_kernel(
    const float* __restrict__ x, uint32_t in_dim, float* __restrict__ row_inv,
    uint16_t* __restrict__ q) {
  __shared__ float s_red[4];
  const uint32_t row = blockIdx.x;
  const float4* r4 = reinterpret_cast<const float4*>(x + (size_t)row * in_dim);
  // magnitudes as integer bits; NaN and infinities count as 0
  auto fin = [](float v) {
    const uint32_t b = __float_as_uint(v) & kAbsMask;
    return b < kInfBits ? b : 0u;
  };
  uint32_t m0 = 0, m1 = 0, m2 = 0, m3 = 0;
#pragma unroll 8
  for (uint32_t c = threadIdx.x; c < in_dim / 4; c += 256) {
    const float4 v = r4[c];
    m0 = max(m0, fin(v.x));
    m1 = max(m1, fin(v.y));
    m2 = max(m2, fin(v.z));
    m3 = max(m3, fin(v.w));
  }
  float mx = __uint_as_float(max(max(m0, m1), max(m2, m3)));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
  const float inv = mx > 0.0f ? ldexpf(1.0f, min(14 - ilogbf(mx), 126)) : 1.0f;
  if (threadIdx.x == 0) row_inv[row] = inv;
  uint16_t* const head = q + (size_t)(2 * row) * in_dim;
#pragma unroll 4
  for (uint32_t c = threadIdx.x; c < in_dim / 8; c += 256) {
    const float4 lo = r4[2 * c], hi = r4[2 * c + 1];
    const float v[8] = {lo.x * inv, lo.y * inv, lo.z * inv, lo.w * inv,
                        hi.x * inv, hi.y * inv, hi.z * inv, hi.w * inv};
    uint32_t oh[4], ot[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float h0 = (float)(_Float16)v[2 * k], h1 = (float)(_Float16)v[2 * k + 1];
      oh[k] = pack2(h0, h1);
      ot[k] = pack2(fin(v[2 * k]) ? v[2 * k] - h0 : 0.0f,
                    fin(v[2 * k + 1]) ? v[2 * k + 1] - h1 : 0.0f);
    }
    *reinterpret_cast<u32x4*>(head + c * 8) = u32x4{oh[0], oh[1], oh[2], oh[3]};
    *reinterpret_cast<u32x4*>(head + in_dim + c * 8) = u32x4{ot[0], ot[1], ot[2], ot[3]};
  }
}

// The same staging with the row held in registers between its maximum and
// its split (read once): one 1024-thread workgroup per row, kV 16-byte
// chunks per thread (in_dim <= 4096 kV), 8-byte stores of 4 halves.  Results
// are those of iq2xxs_scale_stage_f32_rows_kernel bit for bit.
template <int kV>
__global__ __launch_bounds__(1024) void iq2xxs_stage_f32_rows_held_kernel(
    const float* __restrict__ x, uint32_t in_dim, float* __restrict__ row_inv,
    uint16_t* __restrict__ q) {
  __shared__ float s_red[16];
  const uint32_t row = blockIdx.x, tid = threadIdx.x;
  const uint32_t n4 = in_dim / 4;
  const float4* r4 = reinterpret_cast<const float4*>(x + (size_t)row * in_dim);
  auto fin = [](float v) {
    const uint32_t b = __float_as_uint(v) & kAbsMask;
    return b < kInfBits ? b : 0u;
  };
  float4 v[kV];
  uint32_t mb = 0;
#pragma unroll
  for (int j = 0; j < kV; ++j) {
    const uint32_t c = tid + 1024u * j;
    v[j] = c < n4 ? r4[c] : float4{0.0f, 0.0f, 0.0f, 0.0f};
    mb = max(mb, max(max(fin(v[j].x), fin(v[j].y)), max(fin(v[j].z), fin(v[j].w))));
  }
  float mx = __uint_as_float(mb);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  if ((tid & 63) == 0) s_red[tid >> 6] = mx;
  __syncthreads();
  mx = s_red[0];
#pragma unroll
  for (int w = 1; w < 16; ++w) mx = fmaxf(mx, s_red[w]);
  const float inv = mx > 0.0f ? ldexpf(1.0f, min(14 - ilogbf(mx), 126)) : 1.0f;
  if (tid == 0) row_inv[row] = inv;
  uint16_t* const head = q + (size_t)(2 * row) * in_dim;
#pragma unroll
  for (int j = 0; j < kV; ++j) {
    const uint32_t c = tid + 1024u * j;
    if (c >= n4) break;
    const float e[4] = {v[j].x * inv, v[j].y * inv, v[j].z * inv, v[j].w * inv};
    uint32_t oh[2], ot[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const float h0 = (float)(_Float16)e[2 * k], h1 = (float)(_Float16)e[2 * k + 1];
      oh[k] = pack2(h0, h1);
      ot[k] = pack2(fin(e[2 * k]) ? e[2 * k] - h0 : 0.0f,
                    fin(e[2 * k + 1]) ? e[2 * k + 1] - h1 : 0.0f);
    }
    *reinterpret_cast<uint2*>(head + c * 4) = make_uint2(oh[0], oh[1]);
    *reinterpret_cast<uint2*>(head + in_dim + c * 4) = make_uint2(ot[0], ot[1]);
  }
}

// The activations are loaded in 16-byte chunks that are wholly in or out of
// range (in_dim % 8 == 0), and every buffer offset stays below
// kGemmOutOfRange.
bool gemm_supported(uint32_t m, uint32_t out_dim, uint32_t in_dim) {
  return in_dim % 8 == 0 && (uint64_t)m * in_dim * 2 < kGemmOutOfRange - 4096 &&
         (uint64_t)out_dim * ((in_dim + kQK - 1) / kQK) * kBytesPerBlock < kGemmOutOfRange - 4096;
}

size_t gemm_w8a8_scratch_bytes(uint32_t m, uint32_t in_dim) { return (size_t)m * in_dim * 2; }

size_t gemm_f32_scratch_bytes(uint32_t m, uint32_t in_dim, bool w8a8) {
  return (w8a8 ? 1 : 2) * (size_t)m * in_dim * 2;
}

// Sum of the k-split partials in split order (deterministic).  The loads of
// up to kReduceBatch splits are issued before their adds, so a thread waits
// for one memory round trip per batch rather than one per split; the adds
// keep split order.
constexpr uint32_t kReduceBatch = 16;

__global__ __launch_bounds__(256) void gemm_split_reduce_kernel(const float* __restrict__ part,
                                                                uint32_t splits, uint64_t n,
                                                                float* __restrict__ out) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (uint64_t)gridDim.x * blockDim.x) {
    float v = part[i];
    for (uint32_t zb = 1; zb < splits; zb += kReduceBatch) {
      float w[kReduceBatch];
#pragma unroll
      for (uint32_t j = 0; j < kReduceBatch; ++j)
        if (zb + j < splits) w[j] = part[(uint64_t)(zb + j) * n + i];
#pragma unroll
      for (uint32_t j = 0; j < kReduceBatch; ++j)
        if (zb + j < splits) v += w[j];
    }
    out[i] = v;
  }
}

// The same sum over 16-byte chunks (n4 = n / 4; 16-byte aligned buffers).
__global__ __launch_bounds__(256) void gemm_split_reduce4_kernel(const float4* __restrict__ part,
                                                                 uint32_t splits, uint64_t n4,
                                                                 float4* __restrict__ out) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4;
       i += (uint64_t)gridDim.x * blockDim.x) {
    float4 v = part[i];
    for (uint32_t zb = 1; zb < splits; zb += kReduceBatch) {
      float4 w[kReduceBatch];
#pragma unroll
      for (uint32_t j = 0; j < kReduceBatch; ++j)
        if (zb + j < splits) w[j] = part[(uint64_t)(zb + j) * n4 + i];
#pragma unroll
      for (uint32_t j = 0; j < kReduceBatch; ++j) {
        if (zb + j < splits) {
          v.x += w[j].x;
          v.y += w[j].y;
          v.z += w[j].z;
          v.w += w[j].w;
        }
      }
    }
    out[i] = v;
  }
}

// Tile shape and k split of one launch.  256-row tiles halve the
// dequantisation per CU and are used, above 128 rows, when they still give
// most CUs a tile, and for 129-256 rows (one row block, where 128-row tiles
// would decode every weight twice).  Up to 128 rows one 128-row block holds
// them all: 256-row tiles would run half their MFMAs on padding rows (config
// 4's gate / up at M = 128, f16 x: 97 us on 256 x 112 tiles).  When the tiles
// cannot fill half of the 256 CUs, k is split (at least two blocks per split)
// until they do.  The 256-row tiles are 112 or 128 columns wide, whichever
// leaves the busiest CU less work (rounds of 256 workgroups x columns x
// blocks per split): 112 fills the CUs at N = 14336 and 28672 (128 or 256
// tiles), 128 at N = 8192 (64 tiles, split four ways, where 112 gives 74
// tiles split three ways: 222 workgroups).
struct GemmPlan {
  bool wide;    // 256-row tiles (else 128 x 128)
  uint32_t bn;  // columns of a 256-row tile: 112 or 128
  uint32_t splits, split_blocks;
};

static GemmPlan plan_gemm(uint32_t rows, uint32_t out_dim, uint32_t in_dim) {
  GemmPlan p;
  const uint32_t bpr = (in_dim + kQK - 1) / kQK;
  const uint64_t row_tiles = (rows + 255) / 256;
  const uint64_t t256 = row_tiles * ((out_dim + 111) / 112);
  p.wide = rows > 128 && (t256 >= 192 || rows <= 256);
  auto split_of = [&](uint64_t tiles, uint32_t& splits, uint32_t& split_blocks) {
    uint64_t sp = 1;
    if (tiles <= 128 && bpr >= 4) sp = std::min<uint64_t>(256 / tiles, bpr / 2);
    split_blocks = (uint32_t)((bpr + sp - 1) / sp);
    splits = (bpr + split_blocks - 1) / split_blocks;
  };
  if (!p.wide) {
    p.bn = 128;
    split_of((uint64_t)((rows + 127) / 128) * ((out_dim + 127) / 128), p.splits, p.split_blocks);
    return p;
  }
  uint64_t best = UINT64_MAX;
  for (const uint32_t bn : {112u, 128u}) {
    const uint64_t tiles = row_tiles * ((out_dim + bn - 1) / bn);
    uint32_t sp, sb;
    split_of(tiles, sp, sb);
    const uint64_t cost = (tiles * sp + 255) / 256 * bn * sb;
    if (cost < best) {  // (ties keep 112)
      best = cost;
      p.bn = bn;
      p.splits = sp;
      p.split_blocks = sb;
    }
  }
  return p;
}

size_t gemm_split_scratch_bytes(uint32_t rows, uint32_t out_rows, uint32_t out_dim,
                                uint32_t in_dim) {
  const GemmPlan p = plan_gemm(rows, out_dim, in_dim);
  return p.splits > 1 ? (size_t)p.splits * out_rows * out_dim * sizeof(float) : 0;
}

template <int BM, int BN, int kQ>
static hipError_t launch_gemm_t(const GemmArgs& a, uint32_t splits, hipStream_t stream) {
  using L = GemmLayout<BM, BN>;
  static std::atomic<bool> attr_set{false};
  if (!attr_set.load()) {
    hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&iq2xxs_gemm_kernel<BM, BN, kQ>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGemmLdsLimit);
    if (e != hipSuccess) return e;
    attr_set.store(true);
  }
  dim3 grid((a.out_dim + BN - 1) / BN, (a.m + BM - 1) / BM, splits);
  hipLaunchKernelGGL((iq2xxs_gemm_kernel<BM, BN, kQ>), grid, dim3(kGemmThreads),
                     L::kTotal, stream, a);
  return hipGetLastError();
}

// out_rows: rows of the output (a.m / 2 for staged pairs).  With a k split
// the workgroups write partials (the caller's buffer of
// gemm_split_scratch_bytes) that a second kernel sums into out.
template <int kQ>
static hipError_t launch_gemm_shape(GemmArgs a, uint32_t out_rows, float* partials,
                                    hipStream_t stream) {
  const GemmPlan p = plan_gemm(a.m, a.out_dim, a.in_dim);
  float* const out = a.out;
  const uint64_t n = (uint64_t)out_rows * a.out_dim;
  if (p.splits > 1) {
    if (!partials) return hipErrorInvalidValue;
    a.split_blocks = p.split_blocks;
    a.nk = p.split_blocks * (kQK / kGemmBK);
    a.nk_pad = 1 + (a.nk - 1 + kGemmUnroll - 1) / kGemmUnroll * kGemmUnroll;
    a.out = partials;
    a.out_split = n;
  }
  const hipError_t e = !p.wide       ? launch_gemm_t<128, 128, kQ>(a, p.splits, stream)
                       : p.bn == 128 ? launch_gemm_t<256, 128, kQ>(a, p.splits, stream)
                                     : launch_gemm_t<256, 112, kQ>(a, p.splits, stream);
  if (e != hipSuccess || p.splits == 1) return e;
  if (n % 4 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0 &&
      reinterpret_cast<uintptr_t>(partials) % 16 == 0) {
    const uint64_t want = (n / 4 + 255) / 256;
    const uint32_t blocks = (uint32_t)(want < 4096 ? want : 4096);
    hipLaunchKernelGGL(gemm_split_reduce4_kernel, dim3(blocks), dim3(256), 0, stream,
                       reinterpret_cast<const float4*>(partials), p.splits, n / 4,
                       reinterpret_cast<float4*>(out));
    return hipGetLastError();
  }
  const uint64_t want = (n + 255) / 256;
  const uint32_t blocks = (uint32_t)(want < 4096 ? want : 4096);
  hipLaunchKernelGGL(gemm_split_reduce_kernel, dim3(blocks), dim3(256), 0, stream, partials,
                     p.splits, n, out);
  return hipGetLastError();
}

hipError_t launch_iq2xxs_gemm(const void* x, int x_dtype, uint32_t m, const uint8_t* wb,
                              const uint8_t* ws, float* out, uint32_t out_dim, uint32_t in_dim,
                              const float* row_inv, void* xq, bool w8a8, float* partials,
                              hipStream_t stream) {
  const bool bf = x_dtype == 2;
  const uint32_t out_rows = m;
  if (x_dtype == 0) {
    if (!row_inv || !xq) return hipErrorInvalidValue;
    const uint64_t chunks = (uint64_t)m * (in_dim / 8);
    const uint32_t blocks = (uint32_t)((chunks + 255) / 256 < 8192 ? (chunks + 255) / 256 : 8192);
    if (w8a8)
      hipLaunchKernelGGL(iq2xxs_stage_f32_w8a8_kernel, dim3(blocks), dim3(256), 0, stream,
                         static_cast<const float*>(x), m, in_dim, row_inv,
                         static_cast<uint16_t*>(xq));
    else {
      // the row held in registers where it fits (up to 32768 columns)
      const float* xf = static_cast<const float*>(x);
      float* ri = const_cast<float*>(row_inv);
      uint16_t* q16 = static_cast<uint16_t*>(xq);
      const uint32_t n4 = in_dim / 4;
      if (n4 <= 1024)
        hipLaunchKernelGGL(iq2xxs_stage_f32_rows_held_kernel<1>, dim3(m), dim3(1024), 0, stream,
                           xf, in_dim, ri, q16);
      else if (n4 <= 2048)
        hipLaunchKernelGGL(iq2xxs_stage_f32_rows_held_kernel<2>, dim3(m), dim3(1024), 0, stream,
                           xf, in_dim, ri, q16);
      else if (n4 <= 4096)
        hipLaunchKernelGGL(iq2xxs_stage_f32_rows_held_kernel<4>, dim3(m), dim3(1024), 0, stream,
                           xf, in_dim, ri, q16);
      else if (n4 <= 8192)
        hipLaunchKernelGGL(iq2xxs_stage_f32_rows_held_kernel<8>, dim3(m), dim3(1024), 0, stream,
                           xf, in_dim, ri, q16);
      else
        hipLaunchKernelGGL(iq2xxs_scale_stage_f32_rows_kernel, dim3(m), dim3(256), 0, stream, xf,
                           in_dim, ri, q16);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    x = xq;
    if (!w8a8) m *= 2;  // the staged head / tail rows
  } else if (w8a8) {
    if (!row_inv || !xq) return hipErrorInvalidValue;
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
  } else if (bf) {
    // bf16 rows staged as scaled f16: the f16 GEMM with f16 weights
    if (!row_inv || !xq) return hipErrorInvalidValue;
    hipLaunchKernelGGL(iq2xxs_scale_stage_bf16_rows_kernel, dim3(m), dim3(256), 0, stream,
                       static_cast<const uint16_t*>(x), in_dim, const_cast<float*>(row_inv),
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
  a.nk_pad = 1 + (a.nk - 1 + kGemmUnroll - 1) / kGemmUnroll * kGemmUnroll;
  a.x_records = m * in_dim * 2;
  a.wb_records = out_dim * a.bpr * kBytesPerBlock;
  a.ws_records = out_dim * a.bpr * kScalesPerBlock;
  a.split_blocks = 0;
  a.out_split = 0;
  // every row set runs on f16 weights: f16 x as given, bf16 and f32 rows and
  // W8A8's q staged as f16 (row_inv: the scale the epilogue divides by)
  if (x_dtype == 0 && !w8a8) return launch_gemm_shape<2>(a, out_rows, partials, stream);
  if (row_inv) return launch_gemm_shape<1>(a, out_rows, partials, stream);
  return launch_gemm_shape<0>(a, out_rows, partials, stream);
}

}  // namespace cmk
