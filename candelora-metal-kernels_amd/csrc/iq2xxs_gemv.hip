// iq2xxs_gemv.hip — decode-shaped IQ2_XXS matmul (small m) for gfx950.
//
// Replaces iq2_xxs_matmul_kernel / iq2_xxs_matmul_w8a8_kernel
// (src/metal_src/iq2_matmul.metal:188-240, 436-499), which run one thread per
// output walking all of K serially with byte loads, and (for W8A8) rescan the
// whole x row per thread to find its max.
//
// Design (one launch, no scratch memory, one workgroup of up to 16 waves per
// CU for the usual shapes):
//  * Activations are turned into exact integer digits once per workgroup:
//    each 32-column chunk with max|x| < 2^e becomes v = rint(x*2^(21-e)) split
//    into three signed 8-bit digit planes (iq2xxs_device.h), held in LDS.
//  * The weights stream from HBM with 16-byte buffer loads, one pair of
//    32-weight sub-blocks per lane and row group.  Absent rows and pairs get an
//    offset past the buffer's size, so they read zeros without touching memory
//    and without a branch.
//  * Codes expand through two LDS tables (codebook bytes, sign byte-masks)
//    replicated 16 times: lane l reads copy l & 15, so the 16 lanes the LDS
//    serves together hit 16 different bank pairs whatever entries they ask for.
//    One v_perm forms each table address from a code byte.
//  * v_mfma_i32_4x4x4_16b_i8 does the dot products: in each of the 16 4x4
//    blocks, the A rows are the three digit planes (the fourth row is zero),
//    the B columns are 4 weight rows, so eight instructions give, for 4 rows,
//    the three digit sums of a 32-column sub-block.  The sub-block scale
//    d*(2s+1)/8 * 2^(e-21) is applied in fp32 when the sums are folded in.
//  * Each wave reduces its 16 blocks with a fixed butterfly; the workgroup
//    then adds the K-slices of a row in slice order.  Results are
//    deterministic.
//
// Bound: HBM.  Algorithmic bytes per weight row: ceil(K/256)*66, plus x and
// out once.
#include <atomic>

#include "iq2xxs_device.h"
#include "iq2xxs_kernels.h"

namespace cmk {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Lane roles in v_mfma_i32_4x4x4_16b_i8: lane L belongs to 4x4 block L/4; it
// supplies row L%4 of A and column L%4 of B, and receives column L%4 of C
// (rows in the four result registers).
__device__ __forceinline__ v4i mfma4x4(int a_xdigits, int b_weights, v4i c) {
  return __builtin_amdgcn_mfma_i32_4x4x4i8(a_xdigits, b_weights, c, 0, 0, 0);
}

constexpr uint32_t kGemvMaxWaves = 16;
constexpr uint32_t kGemvT = 2;     // sub-block pairs per lane per row group
constexpr uint32_t kGemvMaxR = 2;  // row groups per wave (weights held in registers)
// Digitisation tasks per thread whose activations are loaded before the
// weights (more would spill at 128 VGPRs).
template <bool kVecX>
constexpr uint32_t gemv_max_xt() {
  return kVecX ? 2 : 1;
}
constexpr uint32_t kGemvLdsLimit = 160 * 1024;
// Buffer offset past every num_records used here (weights are < 2^31 bytes).
constexpr uint32_t kOutOfRange = 0x80000000u;
// Word 3 of a gfx9 raw buffer resource (32-bit data format, no swizzle).
constexpr int kBufferWord3 = 0x00020000;

// Replicated lookup tables at LDS offset 0: row r (0..255) is 256 bytes;
// bytes [0, 128) hold 16 copies of codebook entry r (8 magnitude bytes each),
// bytes [128, 256) hold 16 copies of the sign byte-mask of ksigns(r & 127).
constexpr uint32_t kTableRowBytes = 256;
constexpr uint32_t kTableBytes = 256 * kTableRowBytes;
constexpr uint32_t kSignHalf = 128;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes,
                                           kBufferWord3);
}

// Fill the replicated tables.  Slot u < 256 is codebook row u, slot 256 + i
// the sign row i (rows 128..255 repeat rows 0..127: a sign index read as a
// byte carries one unrelated bit on top).  Lane-rotated copy order keeps the
// 16 stores of a lane group on distinct banks.
__device__ __forceinline__ void store_table_slot(uint8_t* lds, uint32_t u, uint64_t v) {
  const uint32_t base = (u & 255) * kTableRowBytes + (u >> 8) * kSignHalf;
#pragma unroll
  for (uint32_t k = 0; k < 16; ++k)
    *reinterpret_cast<uint64_t*>(lds + base + 8 * ((u + k) & 15)) = v;
}

// `code_tid` is this thread's codebook word, fetched before the weight loads
// were issued; only workgroups of fewer than 512 threads load more words here
// (in a separate loop, so the first slot never waits for the weights).
__device__ __forceinline__ void build_replicated_tables(uint8_t* lds, uint32_t tid,
                                                        uint32_t nthreads, uint32_t code_tid) {
  if (tid < 512)
    store_table_slot(lds, tid,
                     tid < 256 ? grid_entry_from_code(code_tid) : expand_sign_mask((int)(tid & 127)));
  for (uint32_t u = tid + nthreads; u < 512; u += nthreads)
    store_table_slot(lds, u, u < 256 ? expand_grid_entry((int)u) : expand_sign_mask((int)(u & 127)));
}

// Table address  256 * byte G of w + low byte of cbase  as one v_perm
// (result bytes: cbase.b0, w.bG, 0, 0).
template <int G>
__device__ __forceinline__ uint32_t table_addr(uint32_t w, uint32_t cbase) {
  return __builtin_amdgcn_perm(w, cbase, 0x0C0C0000u | ((0x04u + G) << 8));
}

// 8-byte LDS read at a byte address (the kernel's dynamic LDS starts at 0).
__device__ __forceinline__ u32x2 lds_load_u2(uint32_t addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) u32x2*>(
      static_cast<uintptr_t>(addr));
}

// Makes v look modified here (emits no instruction).  Used on the weight
// registers right before they are decoded, so the decode's address arithmetic
// cannot be hoisted out of the activation-row loop, where it would wait for
// every weight load and hold all addresses in registers at once.
// The scale stays a 16-bit value until then: widening it would be hoisted too
// (v_cvt_f32_f16 reads only the low half of the register anyway).
__device__ __forceinline__ void pin_here(u32x4& v, uint16_t& d) {
  asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w), "+v"(d));
}

// Sum of v over the 16 lanes of a wave that share lane & 3, in a fixed order.
__device__ __forceinline__ float sum_over_blocks(float v) {
  // row_ror:4 and row_ror:8 inside each 16-lane row, then across rows.
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

struct GemvArgs {
  const void* x;
  const uint8_t* wb;
  const uint8_t* ws;
  float* out;
  uint32_t m, out_dim, in_dim;
  uint32_t bpr;           // super-blocks per row
  uint32_t npairs;        // sub-block pairs per row = 4 * bpr
  uint32_t slices;        // waves that split one row group's K range
  uint32_t teams;         // wave groups; team t takes row groups t, t + teams, ...
  uint32_t rgs;           // row groups per wave (<= kGemvMaxR)
  uint32_t rg_per_wg;     // teams * rgs
  uint32_t xt;            // digitisation tasks per thread per round (<= gemv_max_xt)
  uint32_t wb_records;    // bytes of weight_bytes covering out_dim rows
  uint32_t ws_records;    // bytes of weight_scales covering out_dim rows
  uint32_t plane_stride;  // LDS bytes between the three digit planes
  int w8a8;
};

// LDS layout (dynamic): tables (64 KB) | xsc[2*npairs] f32 |
//   xdig[3][plane_stride] | red[rg_per_wg][slices][4] f32 | wave maxima[16] f32
// XD: activation dtype (0 f32, 1 f16, 2 bf16); kVecX: activations can be read
// as aligned 16-byte vectors.  All global loads are branch-free, so the
// compiler waits for a load only where its value is used, and loads complete
// in issue order: activations first, then weights.
template <int XD, bool kVecX>
__global__ __launch_bounds__(kGemvMaxWaves * 64) void iq2xxs_gemv_kernel(GemvArgs a) {
  extern __shared__ __align__(16) uint8_t lds[];
  const uint32_t nsb = a.npairs * 2;
  float* xsc = reinterpret_cast<float*>(lds + kTableBytes);
  uint8_t* xdig = reinterpret_cast<uint8_t*>(xsc + nsb);
  float* red = reinterpret_cast<float*>(xdig + 3 * a.plane_stride);
  float* s_wred = red + a.rg_per_wg * a.slices * 4;

  const uint32_t nthreads = blockDim.x;
  const uint32_t nwaves = nthreads >> 6;
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t b = lane >> 2;  // 4x4 block within the wave
  const uint32_t j = lane & 3;   // row of the 4-row group / digit plane of this lane
  const uint32_t slice = wave % a.slices;
  const uint32_t team = wave / a.slices;

  const uint32_t rg_begin = blockIdx.x * a.rg_per_wg;
  const uint32_t n_rg_total = (a.out_dim + 3) / 4;
  const uint32_t rg_end = min(rg_begin + a.rg_per_wg, n_rg_total);
  const uint32_t ntasks = nsb * 4;
  constexpr uint32_t kMaxXT = gemv_max_xt<kVecX>();

  // ---- Order of work.  The weight stream of all CUs fills the memory
  // queues for microseconds; a request issued behind it waits that long, and
  // a wave whose weight loads back up in its CU's memory pipeline stalls at
  // issue.  So everything that needs no weights comes first: the codebook
  // word and the activations of row 0 are loaded, the tables are built and
  // the activations digitised, and only then are the weights issued.
  const uint32_t grid_code = fetch_grid_code(tid);
  XOctet<XD, kVecX> xo[kMaxXT];
  auto load_x_tasks = [&](uint32_t task0, size_t xbase) {
#pragma unroll
    for (uint32_t u = 0; u < kMaxXT; ++u) {
      if (u >= a.xt) break;  // uniform
      const uint32_t task = task0 + tid + u * nthreads;
      const uint32_t c0 = (task >> 2) * 32 + (task & 3) * 8;
      xo[u].load(a.x, xbase, c0, a.in_dim, task < ntasks && c0 < a.in_dim);
    }
  };

  // Digit planes of activation row `mrow` into xdig / xsc: 4 threads per
  // 32-column chunk, 8 columns each.  The first round of activations must
  // already be in xo.
  auto digitize_row = [&](uint32_t mrow) {
    const size_t xbase = (size_t)mrow * a.in_dim;
    // W8A8 row scale (iq2_matmul.metal:86-96), reduced over the whole row.
    float inv_scale = 1.0f;
    if (a.w8a8) {
      float mx0 = 0.0f, mx1 = 0.0f;
      for (uint32_t c = tid; c < a.in_dim; c += 2 * nthreads) {
        const uint32_t c1 = c + nthreads;
        const uint32_t b0 = load_x_bits<XD>(a.x, xbase + c);
        const uint32_t b1 = load_x_bits<XD>(a.x, c1 < a.in_dim ? xbase + c1 : xbase);
        mx0 = fmaxf(mx0, fabsf(x_bits_to_float<XD>(b0)));
        mx1 = fmaxf(mx1, fabsf(x_bits_to_float<XD>(b1)));
      }
      float mx = fmaxf(mx0, mx1);
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
      if (lane == 0) s_wred[wave] = mx;
      __syncthreads();
      mx = 0.0f;
      for (uint32_t w = 0; w < nwaves; ++w) mx = fmaxf(mx, s_wred[w]);
      inv_scale = (mx < 1e-8f) ? 1.0f : 127.0f / mx;
    }
    const uint32_t round = nthreads * a.xt;
    for (uint32_t task0 = 0; task0 < ntasks; task0 += round) {
      if (task0 > 0) load_x_tasks(task0, xbase);  // activations beyond the first round
#pragma unroll
      for (uint32_t u = 0; u < kMaxXT; ++u) {
        // the 4 tasks of a chunk sit in 4 consecutive lanes: all active or none
        if (u >= a.xt || task0 + u * nthreads >= ntasks) break;
        const uint32_t task = task0 + tid + u * nthreads;
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
          *reinterpret_cast<uint2*>(xdig + a.plane_stride + c0) = make_uint2(p1[0], p1[1]);
          *reinterpret_cast<uint2*>(xdig + 2 * a.plane_stride + c0) = make_uint2(p2[0], p2[1]);
          if ((task & 3) == 0) xsc[task >> 2] = ldexpf(1.0f, e - kDigitShift - 3);
        }
        __builtin_amdgcn_sched_barrier(0);  // one task at a time: bounds register use
      }
    }
  };

  // The digit planes are complete once every wave has passed this barrier.
  // The scheduler is fenced on both sides: weight-dependent work hoisted
  // above it would make every wave wait for its weights here.
  auto digits_ready = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
  };

  load_x_tasks(0, 0);
  build_replicated_tables(lds, tid, nthreads, grid_code);
  digitize_row(0);
  digits_ready();
  // Each wave issues its weights only now and then works on them as they
  // arrive: no barrier stands between a wave's loads and its dot products,
  // so a wave whose loads queue longer in the CU's memory pipeline delays
  // no other wave.

  // ---- R row groups x T sub-block pairs of weights per lane, by buffer loads.
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(a.wb, a.wb_records);
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(a.ws, a.ws_records);
  const uint32_t pair0 = slice * (16 * kGemvT) + b;
  const uint32_t row_bytes = a.bpr * kBytesPerBlock;
  const uint32_t row0 = (rg_begin + team) * 4 + j;
  const uint32_t wofs0 = row0 * row_bytes + pair0 * 16;
  const uint32_t sofs0 = (row0 * a.bpr + (pair0 >> 2)) * kScalesPerBlock;
  const uint32_t wstep = a.teams * 4 * row_bytes;
  const uint32_t sstep = a.teams * 4 * a.bpr * kScalesPerBlock;
  uint16_t dbits[kGemvMaxR][kGemvT];
  u32x4 q[kGemvMaxR][kGemvT];
  bool present[kGemvMaxR][kGemvT];
#pragma unroll
  for (uint32_t r = 0; r < kGemvMaxR; ++r) {
    const bool rok = r < a.rgs && rg_begin + team + r * a.teams < rg_end;
#pragma unroll
    for (uint32_t t = 0; t < kGemvT; ++t) {
      present[r][t] = rok && pair0 + 16 * t < a.npairs;
      const uint32_t so = present[r][t] ? sofs0 + r * sstep + t * 8 : kOutOfRange;
      dbits[r][t] = __builtin_amdgcn_raw_buffer_load_b16(rs, so, 0, 0);
    }
  }
  // scales ahead of the codes: the first row group's wait must not cover the
  // later groups' weights
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (uint32_t r = 0; r < kGemvMaxR; ++r)
#pragma unroll
    for (uint32_t t = 0; t < kGemvT; ++t) {
      const uint32_t wo = present[r][t] ? wofs0 + r * wstep + t * 256 : kOutOfRange;
      q[r][t] = __builtin_amdgcn_raw_buffer_load_b128(rw, wo, 0, 0);
    }

  const uint32_t cg = 8 * (lane & 15);  // this lane's copy in the codebook half
  const uint32_t cs = kSignHalf + cg;   // and in the sign half

  // Dot products and output of activation row `mrow`, whose digits are in
  // LDS.  Called once for row 0 outside any loop: inside the row loop the
  // activation reloads of later rows would make the compiler's load-count
  // bookkeeping wait for every weight before the first row group.
  auto compute_row = [&](uint32_t mrow) {
    // ---- per-lane activation registers for this wave's slice.  Lane (b, j)
    // holds digit plane j (j < 3; row 3 of A is zero) of both sub-blocks of
    // pair  p = pair0 + 16 t.
    uint32_t xr[kGemvT][2][8];
    float xs[kGemvT][2];
#pragma unroll
    for (uint32_t t = 0; t < kGemvT; ++t) {
      const uint32_t pair = pair0 + 16 * t;
      const bool ok = pair < a.npairs;
#pragma unroll
      for (uint32_t h = 0; h < 2; ++h) {
        const uint32_t sb = 2 * pair + h;
        xs[t][h] = ok ? xsc[sb] : 0.0f;
        if (ok && j < 3) {
          const u32x4* src = reinterpret_cast<const u32x4*>(xdig + j * a.plane_stride + sb * 32);
          const u32x4 lo = src[0], hi = src[1];
          xr[t][h][0] = lo.x; xr[t][h][1] = lo.y; xr[t][h][2] = lo.z; xr[t][h][3] = lo.w;
          xr[t][h][4] = hi.x; xr[t][h][5] = hi.y; xr[t][h][6] = hi.z; xr[t][h][7] = hi.w;
        } else {
#pragma unroll
          for (int k = 0; k < 8; ++k) xr[t][h][k] = 0u;
        }
      }
    }

    // ---- the dot products, one 4-row group at a time.
#pragma unroll
    for (uint32_t r = 0; r < kGemvMaxR; ++r) {
      const uint32_t rg = rg_begin + team + r * a.teams;
      if (r >= a.rgs || rg >= rg_end) break;  // wave-uniform
      float acc = 0.0f;
#pragma unroll
      for (uint32_t t = 0; t < kGemvT; ++t) {
        pin_here(q[r][t], dbits[r][t]);
        const float d = half_bits_to_float(dbits[r][t]);
        const uint32_t words[4] = {q[r][t].x, q[r][t].y, q[r][t].z, q[r][t].w};
        // signed int8 weights of both sub-blocks of the pair
        uint32_t w[2][8];
#pragma unroll
        for (uint32_t h = 0; h < 2; ++h) {
          const uint32_t aux_g = words[2 * h];
          const uint32_t aux_s = words[2 * h + 1];
          // sign index g sits in byte g of aux_s << g, under one unrelated bit
          const uint32_t sa[4] = {aux_s, aux_s << 1, aux_s << 2, aux_s << 3};
          const uint32_t ga[4] = {table_addr<0>(aux_g, cg), table_addr<1>(aux_g, cg),
                                  table_addr<2>(aux_g, cg), table_addr<3>(aux_g, cg)};
          const uint32_t ma[4] = {table_addr<0>(sa[0], cs), table_addr<1>(sa[1], cs),
                                  table_addr<2>(sa[2], cs), table_addr<3>(sa[3], cs)};
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const u32x2 gv = lds_load_u2(ga[g]);
            const u32x2 sm = lds_load_u2(ma[g]);
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
      acc = sum_over_blocks(acc);
      if (lane < 4) red[((rg - rg_begin) * a.slices + slice) * 4 + j] = acc;
      // keep row groups apart: interleaving them only raises register pressure
      __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();
    // ---- the K-slices of each row, added in slice order.
    const uint32_t rows_here = (rg_end > rg_begin) ? (rg_end - rg_begin) * 4 : 0;
    for (uint32_t rr = tid; rr < rows_here; rr += nthreads) {
      const uint32_t row = rg_begin * 4 + rr;
      const float* p = red + (rr >> 2) * a.slices * 4 + (rr & 3);
      float sum = 0.0f;
      for (uint32_t sl = 0; sl < a.slices; ++sl) sum += p[sl * 4];
      if (row < a.out_dim) a.out[(size_t)mrow * a.out_dim + row] = sum;
    }
    __syncthreads();  // xdig / red are rewritten for the next activation row
  };

  compute_row(0);
  for (uint32_t mrow = 1; mrow < a.m; ++mrow) {
    load_x_tasks(0, (size_t)mrow * a.in_dim);
    digitize_row(mrow);
    digits_ready();
    compute_row(mrow);
  }
}

// ---------------------------------------------------------------------------
// Launch policy.
// ---------------------------------------------------------------------------
struct GemvPlan {
  uint32_t slices, teams, rgs, rg_per_wg, xt, grid, threads, plane_stride;
  size_t lds;
};

// Shape of the launch for out_dim x in_dim on num_cus CUs.  One workgroup per
// CU when the row groups allow: its waves are split into `slices` K-ranges of
// 32 sub-block pairs and `teams` row sets; each wave holds at most kGemvMaxR
// row groups of weights in registers.  False when the shape does not fit.
static bool plan_gemv(uint32_t out_dim, uint32_t in_dim, int num_cus, GemvPlan* p) {
  const uint64_t bpr = (in_dim + kQK - 1) / kQK;
  const uint64_t npairs = bpr * 4;
  const uint64_t nsb = bpr * 8;
  if ((uint64_t)out_dim * bpr * kBytesPerBlock > kOutOfRange - 4096) return false;
  const uint32_t slices = (uint32_t)((npairs + 16 * kGemvT - 1) / (16 * kGemvT));
  if (slices > kGemvMaxWaves) return false;
  const uint32_t teams_max = kGemvMaxWaves / slices;
  const uint32_t n_rg = (out_dim + 3) / 4;
  const uint32_t cus = num_cus > 0 ? (uint32_t)num_cus : 1;
  const uint32_t target = (n_rg + cus - 1) / cus;  // row groups per workgroup
  uint32_t rgs = (target + teams_max - 1) / teams_max;
  if (rgs < 1) rgs = 1;
  if (rgs > kGemvMaxR) rgs = kGemvMaxR;
  uint32_t teams = (target + rgs - 1) / rgs;
  if (teams > teams_max) teams = teams_max;
  if (teams < 1) teams = 1;
  p->slices = slices;
  p->teams = teams;
  p->rgs = rgs;
  p->rg_per_wg = teams * rgs;
  p->grid = (n_rg + p->rg_per_wg - 1) / p->rg_per_wg;
  p->threads = 64 * slices * teams;
  const uint64_t ntasks = nsb * 4;
  p->xt = (uint32_t)((ntasks + p->threads - 1) / p->threads);  // capped per variant at launch
  p->plane_stride = (uint32_t)(nsb * 32 + 16);
  p->lds = kTableBytes + nsb * 4 + 3 * (uint64_t)p->plane_stride +
           (uint64_t)p->rg_per_wg * slices * 16 + kGemvMaxWaves * 4;
  return p->lds <= kGemvLdsLimit;
}

bool gemv_supported(uint32_t out_dim, uint32_t in_dim) {
  GemvPlan p;
  return plan_gemv(out_dim, in_dim, 1, &p);
}

template <int XD, bool V>
static hipError_t launch_gemv_t(GemvArgs a, const GemvPlan& p, hipStream_t stream) {
  if (a.xt > gemv_max_xt<V>()) a.xt = gemv_max_xt<V>();
  // The tables alone exceed the default 64 KB of dynamic LDS: raise the
  // limit once per instantiation.
  static std::atomic<bool> attr_set{false};
  if (!attr_set.load()) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&iq2xxs_gemv_kernel<XD, V>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)kGemvLdsLimit);
    if (e != hipSuccess) return e;
    attr_set.store(true);
  }
  hipLaunchKernelGGL((iq2xxs_gemv_kernel<XD, V>), dim3(p.grid), dim3(p.threads), p.lds, stream, a);
  return hipGetLastError();
}

template <int XD>
static hipError_t launch_gemv_v(const GemvArgs& a, const GemvPlan& p, bool vec,
                                hipStream_t stream) {
  return vec ? launch_gemv_t<XD, true>(a, p, stream) : launch_gemv_t<XD, false>(a, p, stream);
}

hipError_t launch_iq2xxs_gemv(const void* x, int x_dtype, uint32_t m, const uint8_t* wb,
                              const uint8_t* ws, float* out, uint32_t out_dim, uint32_t in_dim,
                              bool w8a8, int num_cus, hipStream_t stream) {
  GemvPlan p;
  if (!plan_gemv(out_dim, in_dim, num_cus, &p)) return hipErrorInvalidValue;
  GemvArgs a;
  a.x = x;
  a.wb = wb;
  a.ws = ws;
  a.out = out;
  a.m = m;
  a.out_dim = out_dim;
  a.in_dim = in_dim;
  a.bpr = (in_dim + kQK - 1) / kQK;
  a.npairs = a.bpr * 4;
  a.slices = p.slices;
  a.teams = p.teams;
  a.rgs = p.rgs;
  a.rg_per_wg = p.rg_per_wg;
  a.xt = p.xt;
  a.wb_records = out_dim * a.bpr * kBytesPerBlock;
  a.ws_records = out_dim * a.bpr * kScalesPerBlock;
  a.plane_stride = p.plane_stride;
  a.w8a8 = w8a8 ? 1 : 0;
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
