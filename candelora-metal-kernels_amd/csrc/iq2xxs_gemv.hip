// iq2xxs_gemv.hip — decode-shaped IQ2_XXS matmul, one activation row, for
// gfx950; also 2 to 4 rows where the multi-row kernel (iq2xxs_gemv_rows.hip,
// which serves more rows) would leave CUs idle (out_dim <= 16 per CU), and 2
// rows at any out_dim for K <= 4096: the rows then take the places of the
// digit planes in the MFMA's A operand (kM4, below).
//
// Replaces iq2_xxs_matmul_kernel / iq2_xxs_matmul_w8a8_kernel
// (src/metal_src/iq2_matmul.metal:188-240, 436-499), which run one thread per
// output walking all of K serially with byte loads, and (for W8A8) rescan the
// whole x row per thread to find its max.
//
// Work split.  One workgroup of 16 waves per CU.  A workgroup owns a chunk of
// consecutive 4-row groups; a *tile* is one row group x 16 sub-block pairs
// (1024 columns), i.e. one 16-byte weight load per lane.  Tiles are numbered
// slice-major (tile = slice * n_rg + rg) and each wave takes a contiguous run
// of them, so a wave mostly reuses one slice of activation digits, and the
// tile counts of the 4 waves that share a SIMD differ by at most one.
//
// Arithmetic.
//  * Activations become exact integer digits: each 32-column chunk with
//    max|x| < 2^e gives v = rint(x*2^(22-e)) split into three signed 8-bit
//    digit planes (iq2xxs_device.h), held in LDS.
//  * Codes expand through two LDS tables: a codebook row holds 16 copies of
//    {g, -g} (8 magnitude bytes and their negations), a sign row 16 copies of
//    the 8-byte sign mask; lane l reads copy l & 15, so the 16 lanes the LDS
//    serves together never share a bank.  One v_bitop3 (bit select) per dword
//    picks g or -g under the mask.
//  * v_mfma_i32_4x4x4_16b_i8: in each of the 16 4x4 blocks the A rows are the
//    three digit planes (the fourth row is unused) and the B columns are 4 weight
//    rows; eight instructions give, for 4 rows, the three digit sums of a
//    32-column sub-block, combined as 256 * (256 C2 + C1) + C0 (the inner sum
//    exact in int32, then two fp32 roundings of 2^-24 relative, against the
//    digits' 2^-23).  The scale d*(2s+1)/8 * 2^(e-22) is applied in fp32.
//  * A wave sums its 16 blocks with DPP and lane-swap moves; the workgroup
//    adds the slices of a row in slice order.  Results are deterministic.
//  * W8A8 (true int8): the reference's q = clamp(round(x * inv), +-127) is
//    digit plane 0 as it stands (planes 1 and 2 are zero), so the sub-block
//    sums of q times the codes are exact; each output is divided by inv once.
//
// Schedule.  A CU's memory pipeline serves requests roughly in issue order and
// a wave that issues a load stalls while the pipeline is full, so the order of
// issue matters:
//   1. every wave issues its set-up loads (codebook word, the chunk's scales,
//      its share of the activation row) and the workgroup meets at a barrier,
//      so those loads are ahead of every weight load;
//   2. every wave issues its first two weight tiles;
//   3. waves 0-7 build the tables, waves 15, 14, ... digitise, everyone stages
//      the scales; barrier;
//   4. once tile k has arrived, each wave issues tile k+3 and computes tile k;
//      a workgroup with more chunks then issues the next chunk's tile k into
//      the registers tile k has freed, so the next chunk is in flight while
//      this one is reduced.
// Weight loads carry the nontemporal hint: every code byte is read once.
// All waves run the same code with the same sequence of loads, so the
// compiler's count of outstanding loads (s_waitcnt vmcnt) is exact: a wave
// waits for exactly the load it is about to use.  The first chunk is
// straight-line code for the same reason; further chunks (large out_dim) loop
// behind it.
//
// Bound: HBM.  Algorithmic bytes per weight row: ceil(K/256)*66, plus x and
// out once.
#include <atomic>

#include "iq2xxs_device.h"
#include "iq2xxs_gemv_common.h"
#include "iq2xxs_kernels.h"
#include "iq_rows_formats.h"

namespace cmk {

// Lane roles in v_mfma_i32_4x4x4_16b_i8: lane L belongs to 4x4 block L/4; it
// supplies row L%4 of A and column L%4 of B, and receives column L%4 of C
// (rows in the four result registers).
__device__ __forceinline__ v4i mfma4x4(int a_xdigits, int b_weights, v4i c) {
  return __builtin_amdgcn_mfma_i32_4x4x4i8(a_xdigits, b_weights, c, 0, 0, 0);
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kGemvWaves = 16;
constexpr uint32_t kGemvThreads = kGemvWaves * 64;
constexpr uint32_t kSlicePairs = 16;   // sub-block pairs per tile (one per 4x4 block)
constexpr uint32_t kTilesPerWave = 4;  // weight tiles a wave holds
constexpr uint32_t kTilesEarly = 2;    // tiles issued before the set-up work
constexpr uint32_t kScaleLoads = 2;    // staged scales per thread and chunk

// Sign-row address of group G of aux_s for this lane's copy base cs (whose
// bits 7..13 are clear).
template <bool kWide, int G>
__device__ __forceinline__ uint32_t sign_addr(uint32_t aux_s, uint32_t cs) {
  if constexpr (kWide) {
    const uint32_t f = G == 0 ? aux_s << 7 : (G == 1 ? aux_s : aux_s >> (7 * G - 7));
    return (f & 0x3F80u) | cs;
  } else {
    return perm_addr<G>(aux_s << G, cs);
  }
}

// 65536 c[2] + 256 c[1] + c[0] in 32-bit arithmetic (exact when the result
// fits in an int32: the 21-bit digits of the other formats).
__device__ __forceinline__ int plane_sum(v4i c) {
  const uint32_t hi = ((uint32_t)c[2] << 8) + (uint32_t)c[1];
  return (int)((hi << 8) + (uint32_t)c[0]);
}

// The same sum in fp32 for the 22-bit IQ2_XXS digits, where it can pass
// 2^31 (32 x 43 x 2^22): 256 c[2] + c[1] exactly in int32 (|c[2]| <= 32 x 64
// x 43), then converted and added to c[0] with one fma.
__device__ __forceinline__ float plane_sum_f(v4i c) {
  const uint32_t hi = ((uint32_t)c[2] << 8) + (uint32_t)c[1];
  return fmaf((float)(int)hi, 256.0f, (float)c[0]);
}

// Sum over the 16 lanes that share lane & 3 (the 16 4x4 blocks) of one
// tile, with VALU lane moves only: lanes l and l ^ 32, then l and l ^ 16, then
// the row's four blocks (row_ror:4, row_ror:8).  Every add sees the same
// operands as in sum_over_blocks4, so a row's result does not depend on which
// of the two reductions the kernel took (results do not depend on m).
__device__ __forceinline__ float sum_over_blocks(float v) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  v = __uint_as_float(s[0]) + __uint_as_float(s[1]);
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));
  return v;
}

// The sums over the 16 blocks of four tiles at once: afterwards every lane l
// holds the sum for tile l >> 4 and row l & 3.  v_permlane32_swap swaps the
// upper 32 lanes of its first operand with the lower 32 lanes of its second,
// so adding the two results leaves tile a in lanes 0-31 and tile b in lanes
// 32-63 (each summed over lanes l and l ^ 32); v_permlane16_swap does the same
// with the odd rows of the first operand and the even rows of the second,
// leaving tile 0, 1, 2, 3 in rows 0, 1, 2, 3; two row rotations then add the
// row's four blocks.  Three swaps and five adds for four tiles, in a fixed
// order.
__device__ __forceinline__ float sum_over_blocks4(float a0, float a1, float a2, float a3) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a0), __float_as_uint(a2), false,
                                            false);
  const float t02 = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a1), __float_as_uint(a3), false, false);
  const float t13 = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  r = __builtin_amdgcn_permlane16_swap(__float_as_uint(t02), __float_as_uint(t13), false, false);
  float v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));
  return v;
}

struct GemvArgs {
  const void* x;
  const uint8_t* wb;
  const uint8_t* ws;
  float* out;
  uint32_t m, out_dim, in_dim;
  uint32_t bpr;           // super-blocks per row
  uint32_t spr;           // staged scales per row: bpr rounded up to whole slices
  uint32_t spr_magic;     // ceil(2^32 / spr): i / spr = umulhi(i, spr_magic) for i < 2^16
  int scale_dw;           // spr == bpr and weight_scales 4-byte aligned: dword scale loads
  uint32_t npairs;        // sub-block pairs per row = 4 * bpr
  uint32_t nslices;       // tiles per row group = ceil(npairs / 16)
  uint32_t rg_per_chunk;  // row groups per chunk
  uint32_t nchunks;
  uint32_t ntasks;        // digitisation tasks (8 columns each): m * ntasks_row
  uint32_t ntasks_row;    // digitisation tasks per activation row
  uint32_t ntasks_magic;  // ceil(2^32 / ntasks_row): t / ntasks_row = umulhi(t, magic), t < 2^11
  uint32_t wb_records, ws_records, x_records;  // bytes addressable by the buffer loads
  uint32_t plane_stride;  // LDS bytes between the three digit planes
  uint32_t scale_ofs, xsc_ofs, xdig_ofs, red_ofs, wred_ofs, flag_ofs;  // LDS layout
  int w8a8;
  // Non-null: out = silu(gate) * (x . w), the gated MLP step in the epilogue
  // (gate: [m, out_dim] f32, the gate projection's output).
  const float* gate;
};

// XD: activation dtype (0 f32, 1 f16, 2 bf16); kVecX: activations can be read
// as aligned 16-byte vectors; kWide: table layout; kXT: digitisation tasks
// per thread per round; kW8A8: fake-quantise x per row first; kMulti: more
// than one chunk per workgroup or more than one digitisation round (the loops
// are compiled out otherwise).
// kFmt: the weight format.  kGemvXXS: IQ2_XXS.  kGemvXS: IQ2_XS (the same 64
// code bytes per block; 9-bit codebook indices into the multi-row kernel's
// IQ2_XS table, 8 copies of {g, -g} per 128-byte row, and the IQ2_XXS wide sign
// rows).  kGemvS: IQ2_S (72 code bytes per block: grid low bytes, sign bytes
// and 2 high index bits per group in three arrays, so a tile is three loads
// per lane; the multi-row kernel's IQ2_S tables, 1024 rows x 4 copies and 256
// sign-byte masks x 16 copies, 96 KB).  Both take a 4-bit sub-scale per 16
// weights from 10 scale bytes per block, four 16-column MFMA chains per tile
// and 21-bit digits (16 x 2^21 x 43 < 2^31), one chunk per workgroup and
// dword-copied scales only.  kGemvS3: IQ3_S (104 code bytes per block: two
// 4-value entries per group, 9-bit indices from a low byte and one qh bit,
// explicit sign bytes; four loads per lane per tile; the multi-row kernel's
// IQ3_S tables, 512 rows x 16 copies of {g, -g} and the sign-byte masks, 96
// KB), a sub-scale per 32 weights from 6 scale bytes per block, two chains per
// tile as IQ2_XXS, dl = d (2s+1) and 21-bit digits (32 x 2^21 x 15 < 2^31).
constexpr int kGemvXXS = 0, kGemvXS = 1, kGemvS = 2, kGemvS3 = 3;

// kM4: 2 to 4 activation rows (IQ2_XXS, one chunk per workgroup, every
// digitisation task in registers at once): A row j of the MFMA is activation
// row j instead of digit plane j, one chain pair per digit plane (W8A8: one
// plane, q), and a lane's four results are the four rows' sums for its weight
// row.  The weights are still decoded once per launch.
template <int XD, bool kVecX, bool kWide, int kXT, bool kW8A8, bool kMulti, int kFmt = kGemvXXS,
          bool kM4 = false>
__global__ __launch_bounds__(kGemvThreads) void iq2xxs_gemv_kernel(GemvArgs a) {
  constexpr bool kXS = kFmt == kGemvXS, kS = kFmt == kGemvS, kS3 = kFmt == kGemvS3;
  constexpr bool kH16 = kXS || kS;  // a sub-scale per 16 weights, 10 scale bytes per block
  constexpr bool kOther = kFmt != kGemvXXS;
  static_assert(!kOther || (kWide && !kMulti), "other formats: wide tables, one chunk per workgroup");
  static_assert(!kM4 || (!kOther && !kMulti), "2 to 4 rows: IQ2_XXS, one chunk per workgroup");
  constexpr uint32_t kP = kW8A8 ? 1 : 3;  // digit planes per activation row (kM4 layout)
  extern __shared__ __align__(16) uint8_t lds[];
  using TL = GemvTables<kWide>;
  constexpr int kDS = kOther ? RowsFmtXS::kDigitShift : kDigitShift;  // digit bits
  // scale bytes per block, and staged scale dwords per thread
  constexpr uint32_t kSB =
      kH16 ? RowsFmtXS::kScaleBytes : (kS3 ? RowsFmtS3::kScaleBytes : kScalesPerBlock);
  constexpr uint32_t kSL = kH16 ? 3 : kScaleLoads;
  constexpr uint32_t kLPT = kS ? 3 : (kS3 ? 4 : 1);  // load instructions per tile
  // Tiles in flight ahead of the one computed, and those of them issued
  // before the set-up work.  Mode Off keeps one (IQ2_XS three), timed side by
  // side against three: IQ2_S 9.3 against 11.0 us, IQ3_S 11.0 against 12.4 us
  // (three and four loads a tile); IQ2_XXS 6.99 against 7.13 us at K=4096
  // N=14336, 7.80 against 8.00 us at K=14336 N=4096, 1-2 % slower at K=8192.
  // W8A8 was level or slower with fewer.
  constexpr uint32_t kTilesAhead = (!kXS && !kW8A8) ? 1 : 3;
  constexpr uint32_t kTilesFirst = kTilesEarly < kTilesAhead ? kTilesEarly : kTilesAhead;
  uint16_t* sscale = reinterpret_cast<uint16_t*>(lds + a.scale_ofs);
  float* xsc = reinterpret_cast<float*>(lds + a.xsc_ofs);
  uint8_t* xdig = lds + a.xdig_ofs;
  float* red = reinterpret_cast<float*>(lds + a.red_ofs);
  float* s_wred = reinterpret_cast<float*>(lds + a.wred_ofs);
  // Generation number of the last digitised row that held a NaN or an
  // infinity (rows are numbered by `gen` below; 0 = none yet).
  uint32_t* s_special = reinterpret_cast<uint32_t*>(lds + a.flag_ofs);
  uint32_t* s_kinds = reinterpret_cast<uint32_t*>(lds + a.red_ofs);

  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t rtid = kGemvThreads - 1 - tid;  // digitisation order: last waves first
  const uint32_t b = lane >> 2;                  // 4x4 block of this lane
  const uint32_t j = lane & 3;                   // row in the row group / digit plane
  const uint32_t n_rg_total = (a.out_dim + 3) / 4;
  const uint32_t row_bytes =
      a.bpr * (kS ? RowsFmtS::kBlockBytes : (kS3 ? RowsFmtS3::kBlockBytes : kBytesPerBlock));
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(a.x, a.x_records);
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(a.wb, a.wb_records);
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(a.ws, a.ws_records);
  const uint32_t round = kGemvThreads * kXT;  // tasks per digitisation round

  // ---- chunk geometry and this wave's tiles (all uniform)
  struct ChunkGeom {
    uint32_t row_begin, n_rg, rows, t0, cnt;
  };
  auto geom_of = [&](uint32_t c) {
    ChunkGeom g;
    const uint32_t rg_begin = c * a.rg_per_chunk;
    const uint32_t rg_end = min(rg_begin + a.rg_per_chunk, n_rg_total);
    g.n_rg = rg_end - rg_begin;
    g.row_begin = rg_begin * 4;
    g.rows = min(rg_end * 4, a.out_dim) - g.row_begin;
    const uint32_t ntiles = g.n_rg * a.nslices;
    const uint32_t base = ntiles / kGemvWaves, extra = ntiles - base * kGemvWaves;
    g.cnt = base + (wave < extra ? 1u : 0u);
    g.t0 = wave * base + min(wave, extra);
    return g;
  };
  uint32_t chunk = blockIdx.x;
  uint32_t row_begin, n_rg, rows, t0, cnt;  // the current chunk's
  // slice and row group of this wave's tiles t0 + k of the current chunk
  // (uniform; one division per chunk, then a carry per tile)
  uint32_t tslice[kTilesPerWave], trgl[kTilesPerWave];
  auto set_chunk = [&](const ChunkGeom& g) {
    row_begin = g.row_begin;
    n_rg = g.n_rg;
    rows = g.rows;
    t0 = g.t0;
    cnt = g.cnt;
    uint32_t sl = t0 / n_rg, rg = t0 - sl * n_rg;
#pragma unroll
    for (uint32_t k = 0; k < kTilesPerWave; ++k) {
      tslice[k] = sl;
      trgl[k] = rg;
      if (++rg == n_rg) {
        rg = 0;
        ++sl;
      }
    }
  };
  // Lane (b, j) loads pair b of row j of the tile: byte offset
  // (first row of the tile's row group) * row_bytes + slice * 256 (uniform)
  // plus j * row_bytes + 16 b (this lane's constant).  Rows past out_dim lie
  // past the buffer's end and read zeros; pairs past the row end read other
  // codes, whose staged scale d is 0; tiles past this wave's count are sent
  // past the buffer.
  const uint32_t tile_lane_ofs =
      kS    ? j * row_bytes + (b >> 2) * RowsFmtS::kBlockBytes + 8 * (b & 3)
      : kS3 ? j * row_bytes + (b >> 2) * RowsFmtS3::kBlockBytes + 16 * (b & 3)
            : j * row_bytes + 16 * b;
  // IQ2_S: the 2 high-bit bytes of the lane's sub-blocks (the grid low bytes
  // and the sign bytes are the tile's x, y and z, w)
  uint32_t qhs[kS || kS3 ? kTilesPerWave : 1];
  u32x2 sgs[kS3 ? kTilesPerWave : 1];  // IQ3_S: the sign bytes of the lane's sub-blocks
  auto load_tile_at = [&](uint32_t slice, uint32_t rgl, uint32_t g_row_begin, bool present,
                          uint32_t k) -> u32x4 {
    if constexpr (kS) {
      const uint32_t base = present ? (g_row_begin + rgl * 4) * row_bytes +
                                            slice * (kSlicePairs / 4) * RowsFmtS::kBlockBytes
                                      : kOutOfRange;  // uniform
      const u32x2 qs = __builtin_amdgcn_raw_buffer_load_b64(rw, base + tile_lane_ofs, 0,
                                                            kStreamLoad);
      const u32x2 sg = __builtin_amdgcn_raw_buffer_load_b64(rw, base + tile_lane_ofs + 32, 0,
                                                            kStreamLoad);
      qhs[k] = __builtin_amdgcn_raw_buffer_load_b16(
          rw, base + tile_lane_ofs + 64 - 6 * (b & 3), 0, kStreamLoad);
      return u32x4{qs.x, qs.y, sg.x, sg.y};
    }
    if constexpr (kS3) {
      // (blocks are 8-byte aligned only: the 16 grid bytes as two 8-byte loads)
      const uint32_t base = present ? (g_row_begin + rgl * 4) * row_bytes +
                                            slice * (kSlicePairs / 4) * RowsFmtS3::kBlockBytes
                                      : kOutOfRange;  // uniform
      const uint32_t o = base + tile_lane_ofs;
      const u32x2 q0 = __builtin_amdgcn_raw_buffer_load_b64(rw, o, 0, kStreamLoad);
      const u32x2 q1 = __builtin_amdgcn_raw_buffer_load_b64(rw, o + 8, 0, kStreamLoad);
      sgs[k] = __builtin_amdgcn_raw_buffer_load_b64(rw, o + 72 - 8 * (b & 3), 0, kStreamLoad);
      qhs[k] = __builtin_amdgcn_raw_buffer_load_b16(rw, o + 64 - 14 * (b & 3), 0, kStreamLoad);
      return u32x4{q0.x, q0.y, q1.x, q1.y};
    }
    const uint32_t base = present
                              ? (g_row_begin + rgl * 4) * row_bytes + slice * (kSlicePairs * 16)
                              : kOutOfRange;  // uniform
    return __builtin_amdgcn_raw_buffer_load_b128(rw, base + tile_lane_ofs, 0, kStreamLoad);
  };
  auto load_tile_of = [&](const ChunkGeom& g, uint32_t k) -> u32x4 {
    const uint32_t tau = g.t0 + k;
    const uint32_t slice = tau / g.n_rg;
    const uint32_t rgl = tau - slice * g.n_rg;
    return load_tile_at(slice, rgl, g.row_begin, k < g.cnt, k);
  };
  // (the current chunk's tile k: positions from tslice / trgl)
  auto load_tile = [&](uint32_t k) -> u32x4 {
    return load_tile_at(tslice[k], trgl[k], row_begin, k < cnt, k);
  };
  // Super-block scales of the chunk, staged as rows of a.spr entries (blocks
  // padded to whole slices) with zeros for padding rows and blocks.
  uint32_t sraw[kSL];
  // (the looping kernels keep the 2-byte loads and the one-tile reductions:
  // they are at the 128-VGPR limit, and the alternatives cost spills)
  auto load_scales_of = [&](const ChunkGeom& g) {
    const uint32_t row_begin = g.row_begin, rows = g.rows;
    if (!kMulti && a.scale_dw) {
      // a chunk's scales are contiguous and staged as they lie: rows*bpr*kSB/4
      // dwords (rows is a multiple of 4 or the chunk ends the matrix, and bpr is
      // then even); dwords past them read zeros
      const uint32_t ndw = kOther ? (rows * a.bpr * kSB + 3) / 4 : (rows * a.bpr + 1) / 2;
#pragma unroll
      for (uint32_t k = 0; k < kSL; ++k) {
        const uint32_t t = tid + k * kGemvThreads;
        sraw[k] = __builtin_amdgcn_raw_buffer_load_b32(
            rs, t < ndw ? row_begin * a.bpr * kSB + 4 * t : kOutOfRange, 0, 0);
      }
      return;
    }
#pragma unroll
    for (uint32_t k = 0; k < kScaleLoads; ++k) {
      const uint32_t i = tid + k * kGemvThreads;
      const uint32_t rl = __umulhi(i, a.spr_magic), blk = i - rl * a.spr;  // i / spr, exact
      const bool ok = rl < rows && blk < a.bpr;
      sraw[k] = __builtin_amdgcn_raw_buffer_load_b16(
          rs, ok ? ((row_begin + rl) * a.bpr + blk) * kScalesPerBlock : kOutOfRange, 0, 0);
    }
  };
  auto load_scales = [&]() { load_scales_of(ChunkGeom{row_begin, n_rg, rows, t0, cnt}); };
  auto stage_scales = [&]() {
    const uint32_t nstaged = a.rg_per_chunk * 4 * a.spr;
    if (!kMulti && a.scale_dw) {
#pragma unroll
      for (uint32_t k = 0; k < kSL; ++k) {
        const uint32_t t = tid + k * kGemvThreads;
        if (kOther ? 4 * t < nstaged * kSB : 2 * t < nstaged)
          reinterpret_cast<uint32_t*>(sscale)[t] = sraw[k];
      }
      return;
    }
#pragma unroll
    for (uint32_t k = 0; k < kScaleLoads; ++k) {
      const uint32_t i = tid + k * kGemvThreads;
      if (i < nstaged) sscale[i] = (uint16_t)sraw[k];
    }
  };

  // ---- activation digits
  XTask<XD, kVecX> xo[kXT];
  auto load_x = [&](uint32_t r0, uint32_t mrow) {
#pragma unroll
    for (uint32_t u = 0; u < (uint32_t)kXT; ++u) {
      const uint32_t task = r0 + u * kGemvThreads + rtid;
      if constexpr (kM4) {
        // task = row * ntasks_row + tr over all the rows
        const uint32_t row = __umulhi(task, a.ntasks_magic), tr = task - row * a.ntasks_row;
        const uint32_t c0 = (tr >> 2) * 32 + (tr & 3) * 8;
        xo[u].load(rx, row * a.in_dim + c0, c0, a.in_dim, task < a.ntasks && c0 < a.in_dim);
      } else {
        const uint32_t c0 = (task >> 2) * 32 + (task & 3) * 8;
        xo[u].load(rx, mrow * a.in_dim + c0, c0, a.in_dim, task < a.ntasks && c0 < a.in_dim);
      }
    }
  };
  // W8A8 row scale (iq2_matmul.metal:86-96) from the row's values in xo (the
  // row fits in one round) or by a second pass over the row; ends in a barrier.
  auto w8a8_inv_scale = [&](uint32_t mrow) -> float {
    float mx = 0.0f;
    if (a.ntasks <= round) {
#pragma unroll
      for (uint32_t u = 0; u < (uint32_t)kXT; ++u)
#pragma unroll
        for (int k = 0; k < 8; ++k) mx = fmaxf(mx, fabsf(xo[u].get(k)));
    } else {
      const size_t xbase = (size_t)mrow * a.in_dim;
      for (uint32_t c = tid; c < a.in_dim; c += kGemvThreads)
        mx = fmaxf(mx, fabsf(x_bits_to_float<XD>(load_x_bits<XD>(a.x, xbase + c))));
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if (lane == 0) s_wred[wave] = mx;
    __syncthreads();
    mx = 0.0f;
#pragma unroll
    for (uint32_t w = 0; w < kGemvWaves; ++w) mx = fmaxf(mx, s_wred[w]);
    return (mx < 1e-8f) ? 1.0f : 127.0f / mx;
  };
  // Digits of the round of tasks held in xo: 4 threads per 32-column chunk
  // (an aligned quad of lanes), 8 columns each.
  // The chunk maximum is taken over the magnitude bits as integers, so a NaN
  // (or an infinity) shows up as a value at or above kInfBits; such a chunk
  // (rare) has those values set to zero and marks the row for the fix-up in
  // reduce_and_store.  The condition is the same on the 4 lanes of a quad.
  auto digitize_round = [&](uint32_t r0, float inv_scale, uint32_t gen) {
#pragma unroll
    for (uint32_t u = 0; u < (uint32_t)kXT; ++u) {
      const uint32_t task = r0 + u * kGemvThreads + rtid;
      float xv[8], qv[8];
      uint32_t mb = 0;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        xv[k] = xo[u].get(k);
        if constexpr (kW8A8) xv[k] = qv[k] = quant_w8a8(xv[k], inv_scale);
      }
      if constexpr (kW8A8) {
        // xv only flags values whose q / inv is not finite: for inv >= 2^-100,
        // |q / inv| <= 127 * 2^100 is finite unless q is NaN
        if (inv_scale < 0x1p-100f) {
#pragma unroll
          for (int k = 0; k < 8; ++k) xv[k] = qv[k] / inv_scale;
        }
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) mb = max(mb, __float_as_uint(xv[k]) & kAbsMask);
      mb = quad_max_u32(mb);
      if (mb >= kInfBits) {
        mb = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const uint32_t ab = __float_as_uint(xv[k]) & kAbsMask;
          if (ab >= kInfBits) {
            xv[k] = 0.0f;
            if constexpr (kW8A8) qv[k] = 0.0f;
          }
          mb = max(mb, ab < kInfBits ? ab : 0u);
        }
        mb = quad_max_u32(mb);
        if (task < a.ntasks) *s_special = gen;
      }
      if (kW8A8 && task < a.ntasks) {
        // q as plane 0, planes 1 and 2 zero; the scale keeps the weights' 1/8
        uint32_t qb[2] = {0, 0};
#pragma unroll
        for (int k = 0; k < 8; ++k) qb[k >> 2] |= ((uint32_t)(int)qv[k] & 0xFFu) << (8 * (k & 3));
        const uint32_t c0 = (task >> 2) * 32 + (task & 3) * 8;
        *reinterpret_cast<uint2*>(xdig + c0) = make_uint2(qb[0], qb[1]);
        *reinterpret_cast<uint2*>(xdig + a.plane_stride + c0) = make_uint2(0u, 0u);
        *reinterpret_cast<uint2*>(xdig + 2 * a.plane_stride + c0) = make_uint2(0u, 0u);
        if ((task & 3) == 0) xsc[task >> 2] = 0.125f;
      } else if (task < a.ntasks) {
        const int e = digit_exponent(__uint_as_float(mb));
        const float scale = ldexpf(1.0f, kDS - e);
        // biased digit bytes (each digit + 128), transposed into planes, then
        // the bias removed from four digits at a time
        uint32_t dg[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) dg[k] = digitize_biased(xv[k], scale);
        uint32_t p0[2], p1[2], p2[2];
        digits_to_planes(dg[0], dg[1], dg[2], dg[3], p0[0], p1[0], p2[0]);
        digits_to_planes(dg[4], dg[5], dg[6], dg[7], p0[1], p1[1], p2[1]);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          p0[h] ^= 0x80808080u;
          p1[h] ^= 0x80808080u;
          p2[h] ^= 0x80808080u;
        }
        const uint32_t c0 = (task >> 2) * 32 + (task & 3) * 8;
        *reinterpret_cast<uint2*>(xdig + c0) = make_uint2(p0[0], p0[1]);
        *reinterpret_cast<uint2*>(xdig + a.plane_stride + c0) = make_uint2(p1[0], p1[1]);
        *reinterpret_cast<uint2*>(xdig + 2 * a.plane_stride + c0) = make_uint2(p2[0], p2[1]);
        if ((task & 3) == 0) xsc[task >> 2] = ldexpf(1.0f, e - kDS - 3);
      }
    }
  };
  // Digits of row mrow whose first round is in xo; rounds beyond the first
  // (in_dim > 8192 * kXT) load behind the first weight tiles.
  float inv_row = 1.0f;  // W8A8 scale of the digitised row
  uint32_t gen = 0;      // number of rows digitised so far
  auto digitize_row = [&](uint32_t mrow) {
    ++gen;
    inv_row = 1.0f;
    if constexpr (kW8A8) inv_row = w8a8_inv_scale(mrow);
    digitize_round(0, inv_row, gen);
    if constexpr (kMulti) {
      for (uint32_t r0 = round; r0 < a.ntasks; r0 += round) {
        load_x(r0, mrow);
        digitize_round(r0, inv_row, gen);
      }
    }
  };
  // kM4: the W8A8 scale of each of the (up to 4) rows, from the values in xo;
  // ends in a barrier.  Layout: digit plane p of row r at (r * kP + p) *
  // plane_stride, chunk scales of row r at xsc[r * 8 * bpr ...].
  // (four variables, not an array: selects between array elements by a
  // lane's row index get turned into a scratch table)
  float inv4_0 = 1.0f, inv4_1 = 1.0f, inv4_2 = 1.0f, inv4_3 = 1.0f;
  auto inv_of = [&](uint32_t r) {
    return r == 0 ? inv4_0 : (r == 1 ? inv4_1 : (r == 2 ? inv4_2 : inv4_3));
  };
  auto w8a8_inv4 = [&]() {
    float mx[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (uint32_t u = 0; u < (uint32_t)kXT; ++u) {
      const uint32_t row = __umulhi(u * kGemvThreads + rtid, a.ntasks_magic);
      float v = 0.0f;
#pragma unroll
      for (int k = 0; k < 8; ++k) v = fmaxf(v, fabsf(xo[u].get(k)));
#pragma unroll
      for (uint32_t r = 0; r < 4; ++r) mx[r] = row == r ? fmaxf(mx[r], v) : mx[r];
    }
#pragma unroll
    for (uint32_t r = 0; r < 4; ++r) {
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) mx[r] = fmaxf(mx[r], __shfl_xor(mx[r], off));
      if (lane == 0) s_wred[r * kGemvWaves + wave] = mx[r];
    }
    __syncthreads();
    float inv[4];
#pragma unroll
    for (uint32_t r = 0; r < 4; ++r) {
      float m = 0.0f;
#pragma unroll
      for (uint32_t w = 0; w < kGemvWaves; ++w) m = fmaxf(m, s_wred[r * kGemvWaves + w]);
      inv[r] = (m < 1e-8f) ? 1.0f : 127.0f / m;
    }
    inv4_0 = inv[0];
    inv4_1 = inv[1];
    inv4_2 = inv[2];
    inv4_3 = inv[3];
  };
  // kM4: digits of every row from the tasks in xo (as digitize_round; a
  // non-finite value sets bit `row` of s_special).
  auto digitize4 = [&]() {
    const uint32_t nsb = a.bpr * 8;
#pragma unroll
    for (uint32_t u = 0; u < (uint32_t)kXT; ++u) {
      const uint32_t task = u * kGemvThreads + rtid;
      const uint32_t row = __umulhi(task, a.ntasks_magic), tr = task - row * a.ntasks_row;
      const bool ok = task < a.ntasks;
      const float inv = kW8A8 ? inv_of(row) : 1.0f;
      float xv[8], qv[8];
      uint32_t mb = 0;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        xv[k] = xo[u].get(k);
        if constexpr (kW8A8) xv[k] = qv[k] = quant_w8a8(xv[k], inv);
      }
      if constexpr (kW8A8) {
        if (inv < 0x1p-100f) {
#pragma unroll
          for (int k = 0; k < 8; ++k) xv[k] = qv[k] / inv;
        }
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) mb = max(mb, __float_as_uint(xv[k]) & kAbsMask);
      mb = quad_max_u32(mb);
      if (mb >= kInfBits) {
        mb = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const uint32_t ab = __float_as_uint(xv[k]) & kAbsMask;
          if (ab >= kInfBits) {
            xv[k] = 0.0f;
            if constexpr (kW8A8) qv[k] = 0.0f;
          }
          mb = max(mb, ab < kInfBits ? ab : 0u);
        }
        mb = quad_max_u32(mb);
        if (ok) atomicOr(s_special, 1u << row);
      }
      if (!ok) continue;
      const uint32_t c0 = (tr >> 2) * 32 + (tr & 3) * 8;
      uint8_t* const dst = xdig + row * kP * a.plane_stride + c0;
      if constexpr (kW8A8) {
        uint32_t qb[2] = {0, 0};
#pragma unroll
        for (int k = 0; k < 8; ++k) qb[k >> 2] |= ((uint32_t)(int)qv[k] & 0xFFu) << (8 * (k & 3));
        *reinterpret_cast<uint2*>(dst) = make_uint2(qb[0], qb[1]);
        if ((tr & 3) == 0) xsc[row * nsb + (tr >> 2)] = 0.125f;
      } else {
        const int e = digit_exponent(__uint_as_float(mb));
        const float scale = ldexpf(1.0f, kDS - e);
        uint32_t dg[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) dg[k] = digitize_biased(xv[k], scale);
        uint32_t p0[2], p1[2], p2[2];
        digits_to_planes(dg[0], dg[1], dg[2], dg[3], p0[0], p1[0], p2[0]);
        digits_to_planes(dg[4], dg[5], dg[6], dg[7], p0[1], p1[1], p2[1]);
        *reinterpret_cast<uint2*>(dst) = make_uint2(p0[0] ^ 0x80808080u, p0[1] ^ 0x80808080u);
        *reinterpret_cast<uint2*>(dst + a.plane_stride) =
            make_uint2(p1[0] ^ 0x80808080u, p1[1] ^ 0x80808080u);
        *reinterpret_cast<uint2*>(dst + 2 * a.plane_stride) =
            make_uint2(p2[0] ^ 0x80808080u, p2[1] ^ 0x80808080u);
        if ((tr & 3) == 0) xsc[row * nsb + (tr >> 2)] = ldexpf(1.0f, e - kDS - 3);
      }
    }
  };
  auto sync = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
  };

  // ---- dot products of one tile
  const uint32_t cg = 16 * (lane & (TL::kGridCopies - 1));  // this lane's codebook copy
  const uint32_t cg8 = 16 * (lane & 7);  // IQ2_XS: 8 codebook copies
  const uint32_t cg4 = 16 * (lane & 3);  // IQ2_S: 4 codebook copies
  const uint32_t cs3 = 8 * (lane & 15);  // IQ3_S: 16 codebook copies of 8 bytes
  const uint32_t cs = TL::kSignBase + 8 * (lane & (TL::kSignCopies - 1));
  // Digit plane of this lane's A row.  Lanes with j = 3 load plane 2 as well:
  // A row 3 only feeds C row 3, which is never read, so its contents do not
  // matter and the reload needs no branch.
  const uint32_t plane = min(j, 2u);
  uint32_t xr[2][8];  // digit plane of the tile's two sub-blocks
  float xs[2];        // their chunk scales
  uint32_t cur_slice;
  u32x4 q[kTilesPerWave];
  float acc[kTilesPerWave];
  float dsc[kTilesPerWave];  // d * 2^-27 of each tile's (row, pair); 0 when out of range
  // IQ2_XS: d (no 2^-27), and the lane's two sub-scale bytes of each tile
  uint32_t ssc[kOther ? kTilesPerWave : 1];
  // d of all of this wave's tiles, from the staged scales (one LDS round trip).
  // Staged entry of (row j, pair b): (rgl * 4) * spr + slice * 4 (uniform)
  // plus j * spr + b / 4 (this lane's constant).
  const uint32_t scale_lane_ofs = j * a.spr + (b >> 2);
  // (branch-free: the four reads are in flight together; an absent tile's
  // entry index is clamped into the staged copy and its d replaced by 0)
  auto load_tile_scales = [&]() {
    const uint32_t ent_max = a.rg_per_chunk * 4 * a.spr - 1;  // last staged entry
#pragma unroll
    for (uint32_t k = 0; k < kTilesPerWave; ++k) {
      const uint32_t base = trgl[k] * 4 * a.spr + tslice[k] * (kSlicePairs / 4);  // uniform
      const uint32_t e = min(base + scale_lane_ofs, ent_max);
      if constexpr (kOther) {
        // block (row, blk) at byte kSB * (row * bpr + blk) of the staged copy
        const uint32_t ent = a.scale_ofs + kSB * e;
        const float dv = half_bits_to_float(lds_u16(ent));
        dsc[k] = k < cnt ? dv : 0.0f;
        // IQ2_XS / IQ2_S: the lane's two sub-scale bytes; IQ3_S: its byte (two
        // nibbles), from an aligned 2-byte read
        ssc[k] = kS3 ? lds_u16(ent + 2 + (b & 2)) >> (8 * (b & 1))
                     : lds_u16(ent + 2 + 2 * (b & 3));
      } else {
        const float dv = half_bits_to_float(sscale[e]) * 0x1p-27f;
        dsc[k] = k < cnt ? dv : 0.0f;
      }
    }
  };
  uint32_t k27 = 0x07FFFFFFu;
  asm volatile("" : "+v"(k27));
  // This lane's partial of tile k (before the sum over the 16 blocks).
  auto compute_tile = [&](uint32_t k) -> float {
    const uint32_t slice = tslice[k];
    if (slice != cur_slice) {  // uniform
      cur_slice = slice;
      // a pair past the row end reads the last pair's digits: its d is 0
      const uint32_t pair = min(slice * kSlicePairs + b, a.npairs - 1);
#pragma unroll
      for (uint32_t h = 0; h < 2; ++h) {
        const uint32_t sb = 2 * pair + h;
        xs[h] = xsc[sb];
        const u32x4* src = reinterpret_cast<const u32x4*>(xdig + plane * a.plane_stride + sb * 32);
        const u32x4 lo = src[0], hi = src[1];
        xr[h][0] = lo.x; xr[h][1] = lo.y; xr[h][2] = lo.z; xr[h][3] = lo.w;
        xr[h][4] = hi.x; xr[h][5] = hi.y; xr[h][6] = hi.z; xr[h][7] = hi.w;
      }
    }
    const uint32_t words[4] = {q[k].x, q[k].y, q[k].z, q[k].w};
    if constexpr (kH16) {
      uint32_t w[2][8];
#pragma unroll
      for (uint32_t h = 0; h < 2; ++h) {
        u32x4 gv[4];
        u32x2 sm[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          if constexpr (kXS) {
            // sub-block h: u16 codes of groups 0, 1 in words[2h], of groups 2, 3
            // in words[2h + 1] (codebook index bits 0-8, ksigns index bits 9-15)
            const uint32_t word = words[2 * h + (g >> 1)];
            const uint32_t sh = 16 * (g & 1);
            gv[g] = lds_u4((__builtin_amdgcn_ubfe(word, sh, 9) << 7) | cg8);
            sm[g] = lds_u2((__builtin_amdgcn_ubfe(word, sh + 9, 7) << 7) | cs);
          } else {
            // sub-block h: grid low byte g of words[h], its 2 high bits at bit
            // 2g of byte h of qhs[k]; sign byte g of words[2 + h] (rows of 16
            // copies of its 8-byte mask at 64K)
            const uint32_t idx = __builtin_amdgcn_ubfe(words[h], 8 * g, 8) |
                                 (__builtin_amdgcn_ubfe(qhs[k], 8 * h + 2 * g, 2) << 8);
            gv[g] = lds_u4((idx << 6) | cg4);
            sm[g] = lds_u2((__builtin_amdgcn_ubfe(words[2 + h], 8 * g, 8) << 7) | cs);
          }
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          w[h][2 * g] = bit_select(sm[g].x, gv[g].z, gv[g].x);
          w[h][2 * g + 1] = bit_select(sm[g].y, gv[g].w, gv[g].y);
        }
      }
      // four chains: sub-block h, columns 16 q .. 16 q + 15 (a sub-scale each)
      v4i c[2][2] = {{v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}}, {v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}}};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (uint32_t h = 0; h < 2; ++h)
#pragma unroll
          for (uint32_t qq = 0; qq < 2; ++qq)
            c[h][qq] = mfma4x4((int)xr[h][4 * qq + kk], (int)w[h][4 * qq + kk], c[h][qq]);
      // |plane sum| <= 16 * 43 * 2^21 < 2^31; dl = d * (2 s + 1) / 8 (the 1/8 is
      // in the activation scale)
      const uint32_t sc = ssc[k];
      float r = 0.0f;
#pragma unroll
      for (uint32_t h = 0; h < 2; ++h) {
        float t = 0.0f;
#pragma unroll
        for (uint32_t qq = 0; qq < 2; ++qq)
          t = fmaf((float)plane_sum(c[h][qq]),
                   (float)(2u * __builtin_amdgcn_ubfe(sc, 8 * h + 4 * qq, 4) + 1u), t);
        r = fmaf(t * dsc[k], xs[h], r);
      }
      return r;
    }
    if constexpr (kS3) {
      // sub-block h: grid bytes in words[2h] (entries 0-3) and words[2h + 1]
      // (entries 4-7), high index bits in byte h of qhs[k], sign bytes in
      // sgs[k] word h; group l = entries 2l, 2l + 1 under sign byte l
      uint32_t w[2][8];
#pragma unroll
      for (uint32_t h = 0; h < 2; ++h) {
        const uint32_t sgw = h ? sgs[k].y : sgs[k].x;
#pragma unroll
        for (int l = 0; l < 4; ++l) {
          const u32x2 m = lds_u2((__builtin_amdgcn_ubfe(sgw, 8 * l, 8) << 7) | cs);
          u32x2 ge[2];
#pragma unroll
          for (int e2 = 0; e2 < 2; ++e2) {
            const int e = 2 * l + e2;
            const uint32_t idx = __builtin_amdgcn_ubfe(words[2 * h + (e >> 2)], 8 * (e & 3), 8) |
                                 (__builtin_amdgcn_ubfe(qhs[k], 8 * h + e, 1) << 8);
            ge[e2] = lds_u2((idx << 7) | cs3);
          }
          w[h][2 * l] = bit_select(m.x, ge[0].y, ge[0].x);
          w[h][2 * l + 1] = bit_select(m.y, ge[1].y, ge[1].x);
        }
      }
      v4i c[2] = {v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}};
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        c[0] = mfma4x4((int)xr[0][kk], (int)w[0][kk], c[0]);
        c[1] = mfma4x4((int)xr[1][kk], (int)w[1][kk], c[1]);
      }
      // |plane sum| <= 32 * 15 * 2^21 < 2^31; dl = d (2s+1), times 8 against the
      // 1/8 the activation scales carry
      const uint32_t sc = ssc[k];
      const float d8 = dsc[k] * 8.0f;
      const float t0 = (float)plane_sum(c[0]) * (float)(2u * (sc & 0xFu) + 1u);
      const float t1 = (float)plane_sum(c[1]) * (float)(2u * ((sc >> 4) & 0xFu) + 1u);
      return fmaf(t1 * d8, xs[1], (t0 * d8) * xs[0]);
    }
    // signed int8 weights of both sub-blocks: g where the mask is clear, -g where set
    uint32_t w[2][8];
#pragma unroll
    for (uint32_t h = 0; h < 2; ++h) {
      const uint32_t aux_g = words[2 * h];
      const uint32_t aux_s = words[2 * h + 1];
      const uint32_t ga[4] = {perm_addr<0>(aux_g, cg), perm_addr<1>(aux_g, cg),
                              perm_addr<2>(aux_g, cg), perm_addr<3>(aux_g, cg)};
      const uint32_t sa[4] = {sign_addr<kWide, 0>(aux_s, cs), sign_addr<kWide, 1>(aux_s, cs),
                              sign_addr<kWide, 2>(aux_s, cs), sign_addr<kWide, 3>(aux_s, cs)};
      u32x4 gv[4];
      u32x2 sm[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        gv[g] = lds_u4(ga[g]);
        sm[g] = lds_u2(sa[g]);
      }
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        w[h][2 * g] = bit_select(sm[g].x, gv[g].z, gv[g].x);
        w[h][2 * g + 1] = bit_select(sm[g].y, gv[g].w, gv[g].y);
      }
    }
    // two independent accumulation chains, interleaved
    v4i c[2] = {v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}};
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      c[0] = mfma4x4((int)xr[0][kk], (int)w[0][kk], c[0]);
      c[1] = mfma4x4((int)xr[1][kk], (int)w[1][kk], c[1]);
    }
    // c[h][p] = sum over the 32 columns of digit plane p times w; the
    // sub-block's dot product 65536 c2 + 256 c1 + c0 (W8A8: c0 alone)
    const float f0 = plane_sum_f(c[0]);
    const float f1 = plane_sum_f(c[1]);
    // (2s+1) * 2^27 for the sub-block scale s in bits 28-31 of aux_s: the
    // conversion of s * 2^28 + 2^27 - 1 rounds to (2s+1) * 2^27 exactly (one
    // v_and_or with the low constant in a register: a VOP3 takes one literal)
    const float d = dsc[k];
    const float ud0 = (float)((words[1] & 0xF0000000u) | k27) * d;
    const float ud1 = (float)((words[3] & 0xF0000000u) | k27) * d;
    return fmaf(f1 * ud1, xs[1], (f0 * ud0) * xs[0]);
  };
  // kM4: this lane's partials of tile k for activation rows 0..3 (before the
  // sum over the 16 blocks).  A row j is activation row j (rows past m read
  // zeros); per digit plane, from the highest, two chains of eight MFMAs, and
  // the planes combine as ((C2 * 256 + C1) * 256 + C0) in fp32 (two roundings
  // of 2^-24 relative); two rows in mode Off pack their six (row, plane) pairs
  // into two A operands instead.  The digits are read per tile: the three
  // planes of a row do not fit in registers next to the rest.
  auto compute_tile4 = [&](uint32_t k) -> f32x4 {
    const uint32_t pair = min(tslice[k] * kSlicePairs + b, a.npairs - 1);
    const uint32_t nsb = a.bpr * 8;
    const bool arow = j < a.m;
    const uint32_t jrow = min(j, a.m - 1);
    const uint32_t words[4] = {q[k].x, q[k].y, q[k].z, q[k].w};
    uint32_t w[2][8];
#pragma unroll
    for (uint32_t h = 0; h < 2; ++h) {
      const uint32_t aux_g = words[2 * h];
      const uint32_t aux_s = words[2 * h + 1];
      const uint32_t ga[4] = {perm_addr<0>(aux_g, cg), perm_addr<1>(aux_g, cg),
                              perm_addr<2>(aux_g, cg), perm_addr<3>(aux_g, cg)};
      const uint32_t sa[4] = {sign_addr<kWide, 0>(aux_s, cs), sign_addr<kWide, 1>(aux_s, cs),
                              sign_addr<kWide, 2>(aux_s, cs), sign_addr<kWide, 3>(aux_s, cs)};
      u32x4 gv[4];
      u32x2 sm[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        gv[g] = lds_u4(ga[g]);
        sm[g] = lds_u2(sa[g]);
      }
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        w[h][2 * g] = bit_select(sm[g].x, gv[g].z, gv[g].x);
        w[h][2 * g + 1] = bit_select(sm[g].y, gv[g].w, gv[g].y);
      }
    }
    const float d = dsc[k];
    const float ud0 = (float)((words[1] & 0xF0000000u) | k27) * d;
    const float ud1 = (float)((words[3] & 0xF0000000u) | k27) * d;
    if (!kW8A8 && a.m <= 2) {  // uniform
      // Two rows: the six (row, plane) pairs in two A operands, A row j of
      // the first = plane j >> 1 of row j & 1, of the second = plane 2 of row
      // j (j < 2), so two chain pairs per tile instead of three.
      float f2[2][2];
#pragma unroll
      for (int set = 1; set >= 0; --set) {
        const uint32_t row = j & 1, plane = set ? 2u : (j >> 1);
        const bool valid = (set ? j < 2 : true) && row < a.m;
        const uint32_t rr = min(row, a.m - 1);
        uint32_t xa[2][8];
#pragma unroll
        for (uint32_t h = 0; h < 2; ++h) {
          const u32x4* src = reinterpret_cast<const u32x4*>(
              xdig + (rr * kP + plane) * a.plane_stride + (2 * pair + h) * 32);
          const u32x4 lo = src[0], hi = src[1];
          xa[h][0] = lo.x; xa[h][1] = lo.y; xa[h][2] = lo.z; xa[h][3] = lo.w;
          xa[h][4] = hi.x; xa[h][5] = hi.y; xa[h][6] = hi.z; xa[h][7] = hi.w;
#pragma unroll
          for (int kk = 0; kk < 8; ++kk) xa[h][kk] = valid ? xa[h][kk] : 0u;
        }
        v4i c[2] = {v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}};
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          c[0] = mfma4x4((int)xa[0][kk], (int)w[0][kk], c[0]);
          c[1] = mfma4x4((int)xa[1][kk], (int)w[1][kk], c[1]);
        }
        // first pass: plane 2 of rows 0, 1 (C rows 0, 1); second: planes 0
        // and 1 of row r in C rows r and 2 + r
#pragma unroll
        for (uint32_t h = 0; h < 2; ++h)
#pragma unroll
          for (uint32_t r = 0; r < 2; ++r)
            f2[h][r] = set ? (float)c[h][r]
                           : fmaf(fmaf(f2[h][r], 256.0f, (float)c[h][2 + r]), 256.0f,
                                  (float)c[h][r]);
      }
      f32x4 res2 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (uint32_t r = 0; r < 2; ++r) {
        const float* xs_r = xsc + min(r, a.m - 1) * nsb + 2 * pair;
        res2[r] = fmaf(f2[1][r] * ud1, xs_r[1], (f2[0][r] * ud0) * xs_r[0]);
      }
      return res2;
    }
    float f[2][4];
#pragma unroll
    for (int p = (int)kP - 1; p >= 0; --p) {
      uint32_t xa[2][8];
#pragma unroll
      for (uint32_t h = 0; h < 2; ++h) {
        const u32x4* src = reinterpret_cast<const u32x4*>(
            xdig + (jrow * kP + (uint32_t)p) * a.plane_stride + (2 * pair + h) * 32);
        const u32x4 lo = src[0], hi = src[1];
        xa[h][0] = lo.x; xa[h][1] = lo.y; xa[h][2] = lo.z; xa[h][3] = lo.w;
        xa[h][4] = hi.x; xa[h][5] = hi.y; xa[h][6] = hi.z; xa[h][7] = hi.w;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) xa[h][kk] = arow ? xa[h][kk] : 0u;
      }
      v4i c[2] = {v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}};
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        c[0] = mfma4x4((int)xa[0][kk], (int)w[0][kk], c[0]);
        c[1] = mfma4x4((int)xa[1][kk], (int)w[1][kk], c[1]);
      }
#pragma unroll
      for (uint32_t h = 0; h < 2; ++h)
#pragma unroll
        for (uint32_t r = 0; r < 4; ++r)
          f[h][r] = p == (int)kP - 1 ? (float)c[h][r] : fmaf(f[h][r], 256.0f, (float)c[h][r]);
    }
    f32x4 res;
#pragma unroll
    for (uint32_t r = 0; r < 4; ++r) {
      const float* xs_r = xsc + min(r, a.m - 1) * nsb + 2 * pair;
      res[r] = fmaf(f[1][r] * ud1, xs_r[1], (f[0][r] * ud0) * xs_r[0]);
    }
    return res;
  };
  // Adds the set-aside terms of activation row mrow (NaN or infinite x) to the
  // chunk's outputs: every thread scans its columns of x; for each such column
  // it forms x_c * w_rc for the chunk's rows and records the kind of the term.
  // Only runs for rows that held such a value.
  auto fix_up_special = [&](uint32_t mrow) {
    sync();  // the partial sums in red are consumed: red holds the kinds now
    if (kW8A8 && inv_row == 0.0f) {
      // an infinite activation makes the row's max infinite and inv 0: every
      // q / inv is NaN, and so is every output, as in the reference (uniform;
      // each thread writes the rows it wrote the sums of)
      for (uint32_t rl = tid; rl < rows; rl += kGemvThreads)
        a.out[(size_t)mrow * a.out_dim + row_begin + rl] = __builtin_nanf("");
      return;
    }
    for (uint32_t rl = tid; rl < rows; rl += kGemvThreads) s_kinds[rl] = 0;
    sync();
    const size_t xbase = (size_t)mrow * a.in_dim;
    for (uint32_t c = tid; c < a.in_dim; c += kGemvThreads) {
      float v = x_bits_to_float<XD>(load_x_bits<XD>(a.x, xbase + c));
      if constexpr (kW8A8) v = qdq_w8a8(v, inv_row);
      if ((__float_as_uint(v) & kAbsMask) < kInfBits) continue;
      for (uint32_t rl = 0; rl < rows; ++rl)
        atomicOr(&s_kinds[rl],
                 special_kind(v * (kXS ? RowsFmtXS::weight_at(a.wb, a.ws, row_begin + rl, c, a.bpr)
                                   : kS ? RowsFmtS::weight_at(a.wb, a.ws, row_begin + rl, c, a.bpr)
                                   : kS3 ? RowsFmtS3::weight_at(a.wb, a.ws, row_begin + rl, c, a.bpr)
                                         : iq2xxs_weight_at(a.wb, a.ws, row_begin + rl, c, a.bpr))));
    }
    sync();
    for (uint32_t rl = tid; rl < rows; rl += kGemvThreads) {
      const uint32_t kinds = s_kinds[rl];
      float* o = a.out + (size_t)mrow * a.out_dim + row_begin + rl;
      if (kinds) *o = *o + special_value(kinds);
    }
  };
  // Row sums of the chunk's tiles for activation row mrow, into out.
  static_assert(kTilesPerWave == 4, "sum_over_blocks4 reduces four tiles");
  f32x4 acc4[kM4 ? kTilesPerWave : 1];
  auto reduce_and_store = [&](uint32_t mrow) {
    if constexpr (kM4) {
      // per tile: lane l then holds activation row l >> 4, weight row l & 3
      const uint32_t rgc = a.rg_per_chunk;
#pragma unroll
      for (uint32_t k = 0; k < kTilesPerWave; ++k) {
        if (k >= cnt) break;  // uniform
        const float v = sum_over_blocks4(acc4[k][0], acc4[k][1], acc4[k][2], acc4[k][3]);
        if ((lane & 12) == 0 && (lane >> 4) < a.m)
          red[(((lane >> 4) * rgc + trgl[k]) * a.nslices + tslice[k]) * 4 + j] = v;
      }
      sync();
      const uint32_t special = *s_special;  // bit r: row r held a non-finite value (uniform)
      for (uint32_t r = 0; r < a.m; ++r) {
        const bool gated = a.gate != nullptr && !((special >> r) & 1u);
        for (uint32_t rl = tid; rl < rows; rl += kGemvThreads) {
          const float* p = red + ((r * rgc + (rl >> 2)) * a.nslices) * 4 + (rl & 3);
          float sum = 0.0f;
          for (uint32_t sl = 0; sl < a.nslices; ++sl) sum += p[sl * 4];
          const size_t o = (size_t)r * a.out_dim + row_begin + rl;
          const float v = kW8A8 ? sum / inv_of(r) : sum;  // W8A8: q / inv
          a.out[o] = gated ? silu_mul(a.gate[o], v) : v;
        }
      }
      for (uint32_t r = 0; r < a.m; ++r) {
        if (!((special >> r) & 1u)) continue;  // uniform
        inv_row = inv_of(r);
        fix_up_special(r);
        if (a.gate != nullptr) {
          // (each thread rereads the outputs it wrote)
          for (uint32_t rl = tid; rl < rows; rl += kGemvThreads) {
            const size_t o = (size_t)r * a.out_dim + row_begin + rl;
            a.out[o] = silu_mul(a.gate[o], a.out[o]);
          }
        }
      }
      return;
    }
    if constexpr (!kMulti) {
      // acc[k] is 0 for k >= cnt
      const float v = sum_over_blocks4(acc[0], acc[1], acc[2], acc[3]);
      const uint32_t tk = lane >> 4;  // the tile this lane's row holds
      uint32_t ofs = 0;
#pragma unroll
      for (uint32_t k = 0; k < kTilesPerWave; ++k)
        ofs = tk == k ? (trgl[k] * a.nslices + tslice[k]) * 4 : ofs;
      if ((lane & 12) == 0 && tk < cnt) red[ofs + j] = v;
    } else {
#pragma unroll
      for (uint32_t k = 0; k < kTilesPerWave; ++k) {
        if (k >= cnt) break;  // uniform
        const float v = sum_over_blocks(acc[k]);
        if (lane < 4) red[(trgl[k] * a.nslices + tslice[k]) * 4 + j] = v;
      }
    }
    sync();
    const bool special = *s_special == gen;  // uniform
    const bool gated = a.gate != nullptr && !special;
    for (uint32_t rl = tid; rl < rows; rl += kGemvThreads) {
      const float* p = red + (rl >> 2) * a.nslices * 4 + (rl & 3);
      float sum = 0.0f;
      for (uint32_t sl = 0; sl < a.nslices; ++sl) sum += p[sl * 4];
      const size_t o = (size_t)mrow * a.out_dim + row_begin + rl;
      const float v = kW8A8 ? sum / inv_row : sum;  // W8A8: q / inv
      a.out[o] = gated ? silu_mul(a.gate[o], v) : v;
    }
    if (special) {
      fix_up_special(mrow);
      // the gated step on the completed sums (each thread rereads the rows
      // it wrote)
      if (a.gate != nullptr) {
        for (uint32_t rl = tid; rl < rows; rl += kGemvThreads) {
          const size_t o = (size_t)mrow * a.out_dim + row_begin + rl;
          a.out[o] = silu_mul(a.gate[o], a.out[o]);
        }
      }
    }
  };

  // ======== first chunk (straight-line) ========
  set_chunk(geom_of(chunk));
  // the next chunk of this workgroup (looping kernels only)
  uint32_t next = chunk + gridDim.x;
  ChunkGeom gn = geom_of(kMulti && next < a.nchunks ? next : chunk);
  // 1. set-up loads, ahead of every weight load
  const uint32_t code = kXS ? RowsFmtXS::seed(tid)
                        : kS ? RowsFmtS::seed(tid)
                        : kS3 ? RowsFmtS3::seed(tid) : (tid < 256 ? kGridCodesDev[tid] : 0u);
  if (tid == 0) *s_special = 0;
  load_scales();
  load_x(0, 0);
  sync();
  // 2. the first tiles
#pragma unroll
  for (uint32_t k = 0; k < kTilesFirst; ++k) q[k] = load_tile(k);
  __builtin_amdgcn_sched_barrier(0);
  // 3. tables (waves 0-7), digits (waves from 15 down), scales
  if constexpr (kXS) {
    RowsFmtXS::tables(lds, tid, code);
  } else if constexpr (kS) {
    RowsFmtS::tables(lds, tid, code);
  } else if constexpr (kS3) {
    RowsFmtS3::tables(lds, tid, code);
  } else if (tid < 256) {
    store_grid_row<kWide>(lds, tid, code);
    if (!kWide) store_sign_row<kWide>(lds, tid, sign_mask(tid & 127), 0, TL::kSignCopies);
  } else if (kWide && tid < 512) {
    const uint32_t i = (tid - 256) >> 1, half = tid & 1;
    store_sign_row<kWide>(lds, i, sign_mask(i), half * (TL::kSignCopies / 2),
                          TL::kSignCopies / 2);
  }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (kM4) {
    if constexpr (kW8A8) w8a8_inv4();
    digitize4();
  } else {
    digitize_row(0);
  }
  stage_scales();
  // the rest of the first tiles, then a barrier that leaves them in flight
  // (the set-up loads were consumed above; the tiles are the last loads issued)
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (uint32_t k = kTilesFirst; k < kTilesAhead; ++k) q[k] = load_tile(k);
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(kTilesAhead * kLPT)
               : "memory");
  __builtin_amdgcn_sched_barrier(0);
  // 4. once tile k has arrived, issue tile k + kTilesAhead, then compute tile k
  load_tile_scales();
  cur_slice = ~0u;
#pragma unroll
  for (uint32_t k = 0; k < kTilesPerWave; ++k) {
    acc[k] = 0.0f;
    asm volatile("" ::"v"(q[k].x), "v"(q[k].y), "v"(q[k].z), "v"(q[k].w));
    if constexpr (kS || kS3) asm volatile("" ::"v"(qhs[k]));
    if constexpr (kS3) asm volatile("" ::"v"(sgs[k].x), "v"(sgs[k].y));
    __builtin_amdgcn_sched_barrier(0);
    if (k + kTilesAhead < kTilesPerWave) q[k + kTilesAhead] = load_tile(k + kTilesAhead);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kM4) {
      acc4[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      if (k < cnt) acc4[k] = compute_tile4(k);  // uniform
    } else {
      if (k < cnt) acc[k] = compute_tile(k);  // uniform
    }
    if constexpr (kMulti) {
      // tile k's registers are free: the next chunk's scales (once), then its tile k
      if (next < a.nchunks) {
        if (k == 0) load_scales_of(gn);
        q[k] = load_tile_of(gn, k);
      }
    }
  }
  reduce_and_store(0);

  // ======== further chunks (large out_dim): their tiles are in flight ========
  if constexpr (!kMulti) return;
  while (next < a.nchunks) {
    chunk = next;
    set_chunk(gn);
    next = chunk + gridDim.x;
    if (next < a.nchunks) gn = geom_of(next);
    sync();  // the previous chunk's scales and partial sums are consumed
    stage_scales();
    sync();
    load_tile_scales();
    cur_slice = ~0u;
#pragma unroll
    for (uint32_t k = 0; k < kTilesPerWave; ++k) {
      acc[k] = 0.0f;
      if (k < cnt) acc[k] = compute_tile(k);  // uniform
      if (next < a.nchunks) {
        if (k == 0) load_scales_of(gn);
        q[k] = load_tile_of(gn, k);
      }
    }
    reduce_and_store(0);
  }
}

// ---------------------------------------------------------------------------
// Launch policy.
// ---------------------------------------------------------------------------
struct GemvPlan {
  uint32_t nslices, rg_per_chunk, nchunks, grid, ntasks, ntasks_row, xt, plane_stride;
  uint32_t scale_ofs, xsc_ofs, xdig_ofs, red_ofs, wred_ofs, flag_ofs;
  size_t lds;
  bool wide;
};

static uint32_t align16(uint64_t v) { return (uint32_t)((v + 15) & ~15ull); }

// Launch shape for m x out_dim x in_dim on num_cus CUs; false when the shape
// does not fit (LDS budget, 31-bit buffer offsets).
// sb_bytes / scale_loads: scale bytes per block and staged scale dwords per
// thread (IQ2_XS: 10 and 3).
// table_bytes: a format's fixed table size (0: the IQ2_XXS wide or narrow layout).
// xrows / planes: activation rows digitised and digit planes per row (the
// 2-4 row kernel: m and 3, W8A8 1; else 1 and 3).
static bool plan_gemv(uint32_t m, uint32_t out_dim, uint32_t in_dim, int x_dtype, int num_cus,
                      GemvPlan* p, uint32_t sb_bytes = kScalesPerBlock,
                      uint32_t scale_loads = kScaleLoads, uint32_t table_bytes = 0,
                      uint32_t xrows = 1, uint32_t planes = 3) {
  const uint64_t bpr = (in_dim + kQK - 1) / kQK;
  const uint64_t npairs = bpr * 4;
  const uint64_t nsb = bpr * 8;
  const uint64_t esize = x_dtype == 0 ? 4 : 2;
  if ((uint64_t)out_dim * bpr * kBytesPerBlock > kOutOfRange - 4096) return false;
  if ((uint64_t)m * in_dim * esize > kOutOfRange - 4096) return false;
  const uint64_t nslices = (npairs + kSlicePairs - 1) / kSlicePairs;
  const uint64_t n_rg = (out_dim + 3) / 4;
  const uint64_t cus = num_cus > 0 ? (uint64_t)num_cus : 1;
  const uint64_t target = (n_rg + cus - 1) / cus;  // row groups per CU
  uint64_t rg_per_chunk = (kGemvWaves * kTilesPerWave) / nslices;
  if (rg_per_chunk < 1) return false;
  // as few chunks per workgroup as the tile budget allows, evenly sized
  const uint64_t per_wg_chunks = (target + rg_per_chunk - 1) / rg_per_chunk;
  rg_per_chunk = (target + per_wg_chunks - 1) / per_wg_chunks;
  const uint64_t spr = nslices * (kSlicePairs / 4);  // staged scales per row
  if (sb_bytes == kScalesPerBlock) {
    if (rg_per_chunk * 4 * spr > (uint64_t)scale_loads * kGemvThreads) {
      rg_per_chunk = (scale_loads * kGemvThreads) / (4 * spr);
      if (rg_per_chunk < 1) return false;
    }
  } else if (rg_per_chunk * 4 * spr * sb_bytes > (uint64_t)scale_loads * kGemvThreads * 4) {
    // (the staged copy is rows * blocks * sb_bytes bytes, scale_loads dwords a thread)
    rg_per_chunk = (scale_loads * kGemvThreads * 4) / (4 * spr * sb_bytes);
    if (rg_per_chunk < 1) return false;
  }
  p->nslices = (uint32_t)nslices;
  p->rg_per_chunk = (uint32_t)rg_per_chunk;
  p->nchunks = (uint32_t)((n_rg + rg_per_chunk - 1) / rg_per_chunk);
  p->grid = p->nchunks < cus ? p->nchunks : (uint32_t)cus;
  p->ntasks_row = (uint32_t)(nsb * 4);
  p->ntasks = p->ntasks_row * xrows;
  // two rounds' worth of activations per thread at most (more would spill);
  // longer rows digitise in further rounds
  p->xt = p->ntasks <= kGemvThreads ? 1 : 2;
  p->plane_stride = (uint32_t)(nsb * 32 + 16);
  const uint64_t scale_bytes = align16(rg_per_chunk * 4 * nslices * (kSlicePairs / 4) * sb_bytes);
  // per-wave maxima of the W8A8 row scales: one row, or four (the 2-4 row kernel)
  const uint32_t wred_bytes = kGemvWaves * 4 * (xrows > 1 ? 4 : 1);
  const uint64_t rest = scale_bytes + align16(xrows * nsb * 4) +
                        (uint64_t)planes * xrows * p->plane_stride +
                        align16(xrows * rg_per_chunk * nslices * 16) + wred_bytes + 16;
  p->wide = (table_bytes ? table_bytes : GemvTables<true>::kBytes) + rest <= kGemvLdsLimit;
  if (table_bytes && !p->wide) return false;
  const uint32_t tb =
      table_bytes ? table_bytes : (p->wide ? GemvTables<true>::kBytes : GemvTables<false>::kBytes);
  p->scale_ofs = tb;
  p->xsc_ofs = p->scale_ofs + (uint32_t)scale_bytes;
  p->xdig_ofs = p->xsc_ofs + align16(xrows * nsb * 4);
  p->red_ofs = p->xdig_ofs + planes * xrows * p->plane_stride;
  p->wred_ofs = p->red_ofs + align16(xrows * rg_per_chunk * nslices * 16);
  p->flag_ofs = p->wred_ofs + wred_bytes;
  p->lds = p->flag_ofs + 16;
  return p->lds <= kGemvLdsLimit;
}

bool gemv_supported(uint32_t m, uint32_t out_dim, uint32_t in_dim, int x_dtype) {
  if (m > 1)
    return gemv_rows_supported(m < 16 ? m : 16, out_dim, in_dim, x_dtype, false) &&
           gemv_rows_supported(m < 32 ? m : 32, out_dim, in_dim, x_dtype, true);
  GemvPlan p;
  return plan_gemv(m, out_dim, in_dim, x_dtype, 1, &p);
}

template <int XD, bool V, bool W, int XT, bool Q, bool M, int F = kGemvXXS, bool M4 = false>
static hipError_t launch_gemv_t(const GemvArgs& a, const GemvPlan& p, hipStream_t stream) {
  // The tables alone exceed the default 64 KB of dynamic LDS: raise the
  // limit once per instantiation.
  static std::atomic<bool> attr_set{false};
  if (!attr_set.load()) {
    hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&iq2xxs_gemv_kernel<XD, V, W, XT, Q, M, F, M4>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGemvLdsLimit);
    if (e != hipSuccess) return e;
    attr_set.store(true);
  }
  hipLaunchKernelGGL((iq2xxs_gemv_kernel<XD, V, W, XT, Q, M, F, M4>), dim3(p.grid),
                     dim3(kGemvThreads), p.lds, stream, a);
  return hipGetLastError();
}

template <int XD, bool V, bool W, bool Q>
static hipError_t launch_gemv_m(const GemvArgs& a, const GemvPlan& p, hipStream_t stream) {
  const bool multi = a.nchunks > p.grid || a.ntasks > kGemvThreads * p.xt;
  if (multi)
    return p.xt <= 1 ? launch_gemv_t<XD, V, W, 1, Q, true>(a, p, stream)
                     : launch_gemv_t<XD, V, W, 2, Q, true>(a, p, stream);
  return p.xt <= 1 ? launch_gemv_t<XD, V, W, 1, Q, false>(a, p, stream)
                   : launch_gemv_t<XD, V, W, 2, Q, false>(a, p, stream);
}

template <int XD, bool V, bool W>
static hipError_t launch_gemv_xt(const GemvArgs& a, const GemvPlan& p, hipStream_t stream) {
  return a.w8a8 ? launch_gemv_m<XD, V, W, true>(a, p, stream)
                : launch_gemv_m<XD, V, W, false>(a, p, stream);
}

template <int XD>
static hipError_t launch_gemv_v(const GemvArgs& a, const GemvPlan& p, bool vec,
                                hipStream_t stream) {
  if (vec) return p.wide ? launch_gemv_xt<XD, true, true>(a, p, stream)
                         : launch_gemv_xt<XD, true, false>(a, p, stream);
  return p.wide ? launch_gemv_xt<XD, false, true>(a, p, stream)
                : launch_gemv_xt<XD, false, false>(a, p, stream);
}

// The kernel arguments of a one-row launch planned as p (sb_bytes: scale
// bytes per block).
static GemvArgs gemv_args(const void* x, int x_dtype, uint32_t m, const uint8_t* wb,
                          const uint8_t* ws, float* out, uint32_t out_dim, uint32_t in_dim,
                          bool w8a8, const float* gate, const GemvPlan& p, uint32_t sb_bytes,
                          uint32_t block_bytes = kBytesPerBlock) {
  GemvArgs a;
  a.x = x;
  a.wb = wb;
  a.ws = ws;
  a.out = out;
  a.m = m;
  a.out_dim = out_dim;
  a.in_dim = in_dim;
  a.bpr = (in_dim + kQK - 1) / kQK;
  a.spr = p.nslices * (kSlicePairs / 4);
  a.spr_magic = (uint32_t)((0x100000000ull + a.spr - 1) / a.spr);
  a.scale_dw = (a.spr == a.bpr && reinterpret_cast<uintptr_t>(ws) % 4 == 0) ? 1 : 0;
  a.npairs = a.bpr * 4;
  a.nslices = p.nslices;
  a.rg_per_chunk = p.rg_per_chunk;
  a.nchunks = p.nchunks;
  a.ntasks = p.ntasks;
  a.ntasks_row = p.ntasks_row;
  a.ntasks_magic = (uint32_t)((0x100000000ull + p.ntasks_row - 1) / p.ntasks_row);
  a.wb_records = out_dim * a.bpr * block_bytes;
  a.ws_records = out_dim * a.bpr * sb_bytes;
  a.x_records = m * in_dim * (x_dtype == 0 ? 4u : 2u);
  a.plane_stride = p.plane_stride;
  a.scale_ofs = p.scale_ofs;
  a.xsc_ofs = p.xsc_ofs;
  a.xdig_ofs = p.xdig_ofs;
  a.red_ofs = p.red_ofs;
  a.wred_ofs = p.wred_ofs;
  a.flag_ofs = p.flag_ofs;
  a.w8a8 = w8a8 ? 1 : 0;
  a.gate = gate;
  return a;
}

// Code and scale bytes per block of IQ2_XS (variant 1), IQ2_S (2), IQ3_S (3).
static uint32_t variant_block_bytes(int v) {
  return v == 1 ? RowsFmtXS::kBlockBytes : (v == 2 ? RowsFmtS::kBlockBytes : RowsFmtS3::kBlockBytes);
}
static uint32_t variant_scale_bytes(int v) {
  return v == 3 ? RowsFmtS3::kScaleBytes : RowsFmtXS::kScaleBytes;
}

// IQ2_XS, IQ2_S and IQ3_S at m = 1 on the one-row kernel: 16-byte aligned rows
// of x, weight_bytes 16-byte (IQ2_XS) or 8-byte aligned and weight_scales
// 4-byte aligned, whole slices of 4 blocks per row, the format's tables, one
// chunk per workgroup and one round of digits.
static bool plan_gemv_h16(int variant, const void* x, const uint8_t* wb, const uint8_t* ws,
                          uint32_t out_dim, uint32_t in_dim, int x_dtype, int num_cus,
                          GemvPlan* p) {
  if (variant < 1 || variant > 3) return false;
  const size_t esize = x_dtype == 0 ? 4 : 2;
  const uint32_t bpr = (in_dim + kQK - 1) / kQK;
  const uint32_t block_bytes = variant_block_bytes(variant);
  const uint32_t scale_bytes = variant_scale_bytes(variant);
  if (in_dim % 8 != 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0 ||
      (size_t)in_dim * esize % 16 != 0 || reinterpret_cast<uintptr_t>(ws) % 4 != 0 ||
      reinterpret_cast<uintptr_t>(wb) % (variant == 1 ? 16 : 8) != 0 || bpr % 4 != 0)
    return false;
  if ((uint64_t)out_dim * bpr * scale_bytes > kOutOfRange - 4096) return false;
  if ((uint64_t)out_dim * bpr * block_bytes > kOutOfRange - 4096) return false;
  const uint32_t tables = variant == 1 ? RowsFmtXS::kTableBytes
                                       : (variant == 2 ? RowsFmtS::kTableBytes
                                                       : RowsFmtS3::kTableBytes);
  if (!plan_gemv(1, out_dim, in_dim, x_dtype, num_cus, p, scale_bytes, variant == 3 ? 2 : 3,
                 tables))
    return false;
  return p->wide && p->nchunks <= p->grid && p->ntasks <= kGemvThreads * p->xt;
}

bool iq_variant_gemv_fits(int variant, const void* x, const uint8_t* wb, const uint8_t* ws,
                          uint32_t out_dim, uint32_t in_dim, int x_dtype, int num_cus) {
  GemvPlan p;
  return plan_gemv_h16(variant, x, wb, ws, out_dim, in_dim, x_dtype, num_cus, &p);
}

template <int XD, int F>
static hipError_t launch_gemv_h16_xd(const GemvArgs& a, const GemvPlan& p, bool w8a8,
                                     hipStream_t stream) {
  if (w8a8)
    return p.xt <= 1 ? launch_gemv_t<XD, true, true, 1, true, false, F>(a, p, stream)
                     : launch_gemv_t<XD, true, true, 2, true, false, F>(a, p, stream);
  return p.xt <= 1 ? launch_gemv_t<XD, true, true, 1, false, false, F>(a, p, stream)
                   : launch_gemv_t<XD, true, true, 2, false, false, F>(a, p, stream);
}

template <int F>
static hipError_t launch_gemv_h16_f(const GemvArgs& a, const GemvPlan& p, int x_dtype, bool w8a8,
                                    hipStream_t stream) {
  switch (x_dtype) {
    case 0: return launch_gemv_h16_xd<0, F>(a, p, w8a8, stream);
    case 1: return launch_gemv_h16_xd<1, F>(a, p, w8a8, stream);
    default: return launch_gemv_h16_xd<2, F>(a, p, w8a8, stream);
  }
}

hipError_t launch_iq_variant_gemv(int variant, const void* x, int x_dtype, const uint8_t* wb,
                                  const uint8_t* ws, float* out, uint32_t out_dim,
                                  uint32_t in_dim, bool w8a8, int num_cus, hipStream_t stream) {
  GemvPlan p;
  if (!plan_gemv_h16(variant, x, wb, ws, out_dim, in_dim, x_dtype, num_cus, &p))
    return hipErrorInvalidValue;
  const GemvArgs a = gemv_args(x, x_dtype, 1, wb, ws, out, out_dim, in_dim, w8a8, nullptr, p,
                               variant_scale_bytes(variant), variant_block_bytes(variant));
  switch (variant) {
    case 1: return launch_gemv_h16_f<kGemvXS>(a, p, x_dtype, w8a8, stream);
    case 2: return launch_gemv_h16_f<kGemvS>(a, p, x_dtype, w8a8, stream);
    default: return launch_gemv_h16_f<kGemvS3>(a, p, x_dtype, w8a8, stream);
  }
}

// 2 to 4 activation rows on the one-row kernel (kM4): rows of x 16-byte
// aligned, every digitisation task in registers at once (m * 32 * bpr <=
// 2048), one chunk per workgroup and the LDS budget.
static bool plan_gemv4(uint32_t m, uint32_t out_dim, uint32_t in_dim, int x_dtype, bool w8a8,
                       const void* x, int num_cus, GemvPlan* p) {
  const size_t esize = x_dtype == 0 ? 4 : 2;
  if (m < 2 || m > 4 || in_dim % 8 != 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0 ||
      (size_t)in_dim * esize % 16 != 0)
    return false;
  if (!plan_gemv(m, out_dim, in_dim, x_dtype, num_cus, p, kScalesPerBlock, kScaleLoads, 0, m,
                 w8a8 ? 1 : 3))
    return false;
  return p->nchunks <= p->grid && p->ntasks <= kGemvThreads * p->xt;
}

// Where the 2-4 row launch runs instead of the multi-row kernel: where the
// latter's 32-row groups would cover at most half the CUs (out_dim <= 16 per
// CU, 4096 on 256), and for two rows (two MFMA chain pairs per tile) at any
// out_dim when K <= 4096.  Timed side by side on MI355X (graph replays, rotated
// weights, f32 x; f16 alike): N = 4096, K = 4096, m = 2 / 3 / 4: 6.20 / 6.75 /
// 7.09 against 7.45 / 8.21 / 8.45 us; N = 1024: 4.9 / 5.6 / 6.1 against 7.1 /
// 8.0 / 8.2 us; N = 4096, K = 2048: 5.0 / 5.2 / 5.5 against 6.4 / 6.6 / 6.7
// us; W8A8 within 4 % either way at these N.  At N = 14336 (K = 4096) it lost
// (m = 4: 12.0 against 10.5 us), as at N = 8192 (K = 8192, m = 2: 13.2
// against 10.8 us): the three MFMA chains per tile and the per-tile digit
// reads then outweigh the fuller grid.  Two rows, with their six (row, plane)
// pairs packed into two A operands: N = 14336, K = 4096 9.7 (f16 x 8.8, W8A8
// 10.7) against 10.3 (10.2, 12.0) us; N = 4096 5.6 against 6.1 us (6.0
// unpacked); N = 8192, K = 8192 level or 3 % slower (f32, W8A8).
static bool gemv4_pays(uint32_t m, uint32_t out_dim, uint32_t in_dim, int num_cus) {
  if (m <= 2 && in_dim <= 4096) return true;
  return (uint64_t)out_dim <= 16ull * (uint64_t)(num_cus > 0 ? num_cus : 1);
}

template <int XD, bool W, bool Q>
static hipError_t launch_gemv4_xt(const GemvArgs& a, const GemvPlan& p, hipStream_t stream) {
  return p.xt <= 1 ? launch_gemv_t<XD, true, W, 1, Q, false, kGemvXXS, true>(a, p, stream)
                   : launch_gemv_t<XD, true, W, 2, Q, false, kGemvXXS, true>(a, p, stream);
}

template <int XD>
static hipError_t launch_gemv4(const GemvArgs& a, const GemvPlan& p, hipStream_t stream) {
  if (a.w8a8)
    return p.wide ? launch_gemv4_xt<XD, true, true>(a, p, stream)
                  : launch_gemv4_xt<XD, false, true>(a, p, stream);
  return p.wide ? launch_gemv4_xt<XD, true, false>(a, p, stream)
                : launch_gemv4_xt<XD, false, false>(a, p, stream);
}

hipError_t launch_iq2xxs_gemv(const void* x, int x_dtype, uint32_t m, const uint8_t* wb,
                              const uint8_t* ws, float* out, uint32_t out_dim, uint32_t in_dim,
                              bool w8a8, int num_cus, hipStream_t stream, const float* gate,
                              void* split_ws, size_t split_ws_bytes) {
  if (m > 1 && m <= 4 && gemv4_pays(m, out_dim, in_dim, num_cus)) {
    GemvPlan p;
    if (plan_gemv4(m, out_dim, in_dim, x_dtype, w8a8, x, num_cus, &p)) {
      const GemvArgs a = gemv_args(x, x_dtype, m, wb, ws, out, out_dim, in_dim, w8a8, gate, p,
                                   kScalesPerBlock);
      switch (x_dtype) {
        case 0: return launch_gemv4<0>(a, p, stream);
        case 1: return launch_gemv4<1>(a, p, stream);
        default: return launch_gemv4<2>(a, p, stream);
      }
    }
  }
  if (m > 1) {
    // groups of up to 16 activation rows (W8A8: 32), each decoding the weights once
    const size_t esize = x_dtype == 0 ? 4 : 2;
    const uint32_t group = w8a8 ? 32 : 16;
    for (uint32_t r0 = 0; r0 < m; r0 += group) {
      const hipError_t e = launch_iq2xxs_gemv_rows(
          static_cast<const uint8_t*>(x) + (size_t)r0 * in_dim * esize, x_dtype,
          m - r0 < group ? m - r0 : group, wb, ws, out + (size_t)r0 * out_dim, out_dim, in_dim,
          w8a8, num_cus, stream, gate ? gate + (size_t)r0 * out_dim : nullptr, split_ws,
          split_ws_bytes);
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }
  GemvPlan p;
  if (!plan_gemv(m, out_dim, in_dim, x_dtype, num_cus, &p)) return hipErrorInvalidValue;
  const GemvArgs a = gemv_args(x, x_dtype, m, wb, ws, out, out_dim, in_dim, w8a8, gate, p,
                               kScalesPerBlock);
  const size_t esize = x_dtype == 0 ? 4 : 2;
  const bool vec = (in_dim % 8 == 0) && (reinterpret_cast<uintptr_t>(x) % 16 == 0) &&
                   ((size_t)in_dim * esize % 16 == 0);
  switch (x_dtype) {
    case 0: return launch_gemv_v<0>(a, p, vec, stream);
    case 1: return launch_gemv_v<1>(a, p, vec, stream);
    default: return launch_gemv_v<2>(a, p, vec, stream);
  }
}

}  // namespace cmk
