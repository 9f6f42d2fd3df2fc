// iq2xxs_gemv_rows.hip — IQ2_XXS matmul for 2..16 activation rows (W8A8: up
// to 32), and IQ2_XS, IQ2_S and IQ3_S matmuls for up to 16 rows per launch
// (W8A8: 32), on gfx950.
//
// Replaces iq2_xxs_matmul_kernel / iq2_xxs_matmul_w8a8_kernel
// (src/metal_src/iq2_matmul.metal:188-240, 436-499) for small m > 1, and the
// IQ2_XS / IQ2_S / IQ3_S matmul kernels (:242-434, 501-699) for m <= 16 per
// launch.  The reference runs one thread per output, so every weight is
// decoded once per activation row; here a weight is decoded once per launch
// and one MFMA multiplies it against all the rows.  What differs between the
// formats (tables, loads, code expansion, sub-scales) is a policy class from
// iq_rows_formats.h; formats whose sub-scale covers 16 weights (IQ2_XS, IQ2_S)
// take two v_mfma_i32_32x32x16_i8 per sub-block instead of one
// v_mfma_i32_32x32x32_i8, with lane l supplying columns 8 (l/32) .. + 7 of
// each 16-column half.
//
// Arithmetic.  The activations become exact integer digits as in the one-row
// kernel (iq2xxs_gemv.hip): per 32-column sub-block, three signed 8-bit planes
// of rint(x * 2^(D-e)), in LDS, with D = 22 bits for IQ2_XXS (as in the
// one-row kernel) and 21 for the other formats.  The codes expand through the same
// LDS tables ({g, -g} codebook rows, 8-byte sign masks, one bit select per
// dword).  v_mfma_i32_32x32x32_i8 then takes
//   A: 32 rows = 8 activation rows x 4 digit planes (plane 3 and absent rows
//      read a zero plane), 32 columns = one sub-block (16 activation rows:
//      two such operands, each multiplied by the same decoded weights);
//   B: the same 32 columns of 32 weight rows.
// Lane l supplies A row l%32 and B column (weight row) l%32, both over columns
// 16*(l/32) .. +15 of the sub-block (so A and B agree on the k order whatever
// the hardware's byte order is), and receives C rows 8*(r/4) + 4*(l/32) + r%4
// in register r: planes 0..2 of activation rows 2t + l/32 (t = r/4) against
// weight row l%32.  The three plane sums combine exactly in int32 where they
// fit (IQ2_XXS: 256 C2 + C1 exactly, then one fp32 rounding for the last
// byte); the scale (2s+1) * 2^(e-D-3) is applied in fp32 per sub-block, d
// once per super-block.
//
// Work split.  A *unit* is 32 weight rows x half a super-block (4 sub-blocks,
// 1 KB of codes: one 16-byte load per lane).  A workgroup of 16 waves owns a
// chunk of R consecutive 32-row groups; the P = 16/R waves of a row group share
// its units.  K is processed in slices of S super-blocks whose digits fit in
// LDS next to the tables; a wave holds at most kU units per slice and
// prefetches the next slice's unit into the registers of the one it has just
// unpacked.  A slice's scale bytes (d and sub-scales) for the chunk's rows are
// loaded coalesced with the slice's activations and staged in LDS, where the
// units read them: a unit's own scale bytes are a few scattered bytes per row,
// which cost more than the unit's codes.  The waves of a row group add their
// partial sums in wave order, so results are deterministic.
//
// Split over K.  When the row groups alone would leave CUs idle (fewer 32-row
// groups than CUs: N = 4096 has 128), each row group's K range is cut into
// `kparts` parts of whole slices, one workgroup each.  A part writes its sums
// to the caller's workspace with agent-scope atomic stores, waits for them to
// complete, then counts itself in on its row group's arrival word (an
// agent-scope compare-and-swap); the part that arrives last reads every
// part's sums with agent-scope atomic loads, adds them in part order -- the
// same result whichever part is last -- and writes the outputs, the gated
// step and the non-finite fix-up.  The word needs no initial value: it holds
// (launch epoch, count), a count under another epoch counts as zero, and the
// last part clears it, so replays of a captured launch (same epoch) start from
// zero.  No workgroup waits for another.
//
// W8A8 (true int8).  The reference fake-quantises x per row (q / inv with q =
// clamp(round(x * inv), +-127), iq2_matmul.metal:85-126) and multiplies in
// fp32.  Here q itself is the A operand: one int8 plane per activation row, so
// the 32 A rows are 32 activation rows and one launch serves up to 32 rows
// (kRows 8 keeps the four result registers of rows 0..7, kRows 32 all 16).
// The sub-block sums of q times the codes are exact in int32; (2s+1) d is
// applied per sub-block in fp32 and 1 / (8 inv) once per output.  A value
// whose q / inv is not finite (an infinite x, or every x of a row that holds
// one, where inv = 0) is set aside and fixed up like a non-finite x.
//
// Bound: HBM (the same algorithmic bytes as the one-row kernel; every weight
// byte is read once, x once per workgroup from L2).
#include <atomic>
#include <type_traits>

#include "iq2xxs_device.h"
#include "iq2xxs_gemv_common.h"
#include "iq2xxs_kernels.h"
#include "iq_rows_formats.h"

namespace cmk {

typedef int v16i __attribute__((ext_vector_type(16)));

constexpr uint32_t kRowsWaves = 16;
constexpr uint32_t kRowsThreads = kRowsWaves * 64;
// Digitisation tasks (8 columns of one activation row) per thread and slice:
// one where one suffices -- up to 4 rows, W8A8 up to 4 rows -- two otherwise.
// A second slot costs a load and a digitisation per thread even when empty
// (0.4-2 us at 4 rows); one slot for 8 rows would halve their slices (slower).
constexpr uint32_t rows_tasks(uint32_t rows, bool w8a8, uint32_t m) {
  return (w8a8 ? m <= 4 : rows <= 4) ? 1 : 2;
}
// Units of the first slice issued before the set-up work (tables, digits); the
// rest are issued one per computed unit.  A CU's memory pipeline stalls a wave
// at issue while it is full, so weight requests issued ahead of a barrier
// would hold every wave at that barrier until they drain.  Two units go
// early (W8A8: 0.4 us less at 4 and 8 rows; mode Off, timed side by side:
// IQ2_XXS 0.05-0.3 us less at 4 and 8 rows, IQ3_S 0.2-0.5 us less, IQ2_XS
// level) except for IQ2_S in mode Off (three loads per unit), where two early
// units were 0.5-0.9 us slower.
template <class F, bool kW8A8>
constexpr uint32_t rows_units_early() {
  return (kW8A8 || !std::is_same<F, RowsFmtS>::value) ? 2 : 1;
}
// Flags and the W8A8 row scales.
constexpr uint32_t rows_flag_bytes(uint32_t rows) { return (16 + 4 * rows + 15) & ~15u; }

struct RowsArgs {
  const void* x;
  const uint8_t* wb;
  const uint8_t* ws;
  float* out;
  uint32_t m, out_dim, in_dim, bpr;
  uint32_t n_rg;         // 32-row groups
  uint32_t rg_shift;     // log2 of the row groups per chunk (R)
  uint32_t nchunks;
  uint32_t slice_shift;  // log2 of the super-blocks per K slice (S)
  uint32_t nslices;
  uint32_t wb_records, ws_records, x_records;  // bytes addressable by the buffer loads
  uint32_t plane_stride;                       // LDS bytes between digit planes
  uint32_t xdig_ofs, xsc_ofs, flag_ofs;        // LDS layout; partial sums reuse xdig
  uint32_t sc_ofs;  // the K slice's scale bytes for the chunk's rows: [row][block][bytes]
  // Non-null: out = silu(gate) * (x . w), the gated MLP step in the epilogue
  // (gate: [m, out_dim] f32, the gate projection's output).
  const float* gate;
  // Split over K (kparts > 1): chunk c is part c % kparts of row group
  // c / kparts, slices [part * kslices, min(nslices, (part + 1) * kslices)).
  uint32_t kparts, kslices, epoch;
  unsigned long long* arrive;  // [n_rg] (epoch << 32) | parts arrived
  uint32_t* part_special;      // [n_rg][kparts] non-finite row masks of the parts
  float* part_sums;            // [kparts][m][out_dim] raw sums of the parts
};

// Counts a part in on its row group's arrival word; true for the last of
// `parts` parts of launch `epoch`.  A count left under another epoch counts
// as zero.  Relaxed: the parts exchange their sums and masks only through
// agent-scope atomic stores and loads, which the caches do not hold back, and
// the caller waits for its own stores to complete before it arrives -- no
// fence, which would write back and invalidate the whole L2 of the XCD.
__device__ __forceinline__ bool rows_arrive_last(unsigned long long* w, uint32_t epoch,
                                                 uint32_t parts) {
  unsigned long long old = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (;;) {  // at most `parts` rounds: a failed exchange means another part got in
    const uint32_t cnt = (uint32_t)(old >> 32) == epoch ? (uint32_t)old + 1u : 1u;
    const unsigned long long nw = ((unsigned long long)epoch << 32) | cnt;
    if (__hip_atomic_compare_exchange_strong(w, &old, nw, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT))
      return cnt == parts;
  }
}

// Agent-scope relaxed store / load of a part's sum.
__device__ __forceinline__ void part_store(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float part_load(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Units a wave holds per slice: four with IQ2_XXS's 5-register units, x read
// as vectors and at most four result registers (up to 4 rows; W8A8 up to 8),
// two otherwise (the registers a 1024-thread workgroup leaves a wave: 128).
template <class F>
constexpr uint32_t rows_units(int rows, bool vec, bool w8a8) {
  return (w8a8 ? rows == 8 : rows <= 4) && vec && sizeof(typename F::Unit) <= 20 ? 4 : 2;
}

// F: the weight format (iq_rows_formats.h); XD: activation dtype (0 f32,
// 1 f16, 2 bf16); kVecX: activations can be read as aligned 16-byte vectors;
// kW8A8: int8 activations q (kRows 8 or 32); otherwise kRows is 2, 4, 8 or 16
// (the plane sums of kRows / 2 rows per lane folded in the epilogue); at
// least m.  kTasks: digitisation task slots per thread (rows_tasks).
template <class F, int XD, bool kVecX, bool kW8A8, int kRows, int kTasks>
__global__ __launch_bounds__(kRowsThreads) void iq_gemv_rows_kernel(RowsArgs a) {
  extern __shared__ __align__(16) uint8_t lds[];
  constexpr uint32_t kT = kRows / 2;  // activation rows per lane: 2t + h
  // result registers kept per lane: W8A8 the first kRows / 2 (activation rows
  // 8 (r/4) + 4 h + r % 4), otherwise the plane sums folded into kT rows
  constexpr uint32_t kAcc = kT;
  static_assert(!kW8A8 || kRows == 8 || kRows == 32, "W8A8 runs 8 or 32 rows per launch");
  // mode Off: 8 activation rows x 4 digit planes fill one A operand; 16 rows
  // take two, multiplied by the same decoded weights
  constexpr uint32_t kAOps = (!kW8A8 && kRows == 16) ? 2 : 1;
  constexpr uint32_t kTO = kT / kAOps;  // activation-row pairs per A operand
  constexpr uint32_t kU = rows_units<F>(kRows, kVecX, kW8A8);
  constexpr uint32_t kEarly = rows_units_early<F, kW8A8>();
  // scale staging: 2-byte tasks per thread (a chunk holds R * 32 rows and a
  // slice S blocks, R * S <= 8 kU)
  constexpr uint32_t kSH = F::kScaleBytes / 2;
  constexpr uint32_t kScaleTasks = (32 * 8 * kU * kSH + kRowsThreads - 1) / kRowsThreads;
  uint8_t* xdig = lds + a.xdig_ofs;
  float* xsc = reinterpret_cast<float*>(lds + a.xsc_ofs);
  float* red = reinterpret_cast<float*>(lds + a.xdig_ofs);
  uint32_t* s_kinds = reinterpret_cast<uint32_t*>(lds + a.xdig_ofs);
  uint32_t* s_special = reinterpret_cast<uint32_t*>(lds + a.flag_ofs);  // bit r: row r not finite
  float* s_inv = reinterpret_cast<float*>(lds + a.flag_ofs + 16);      // W8A8 scales

  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t h = lane >> 5;  // column half of the sub-block / activation row parity
  const uint32_t n = lane & 31;  // weight row in the group
  const uint32_t R = 1u << a.rg_shift;
  const uint32_t P = kRowsWaves >> a.rg_shift;  // waves per row group
  const uint32_t rgl = wave >> (4 - a.rg_shift);
  const uint32_t wp = wave & (P - 1);
  const uint32_t S = 1u << a.slice_shift;
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(a.x, a.x_records);
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(a.wb, a.wb_records);
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(a.ws, a.ws_records);
  auto sync = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
  };

  // ---- W8A8 row scales (iq2_matmul.metal:86-96): 127 / max|x_r|.  Wave w
  // takes rows w, w + 16: its lanes read the row as 8-element tasks, eight per
  // lane in flight (K = 4096 in one round trip), and the wave reduces them (fmaxf drops a NaN, as the
  // reference's max does).
  if constexpr (kW8A8) {
    constexpr uint32_t kBatch = 8;
    const uint32_t tpr = (a.in_dim + 7) / 8;  // tasks per row
    for (uint32_t r = wave; r < a.m; r += kRowsWaves) {
      float mx = 0.0f;
      for (uint32_t t0 = 0; t0 < tpr; t0 += 64 * kBatch) {
        XTask<XD, kVecX> xt[kBatch];
#pragma unroll
        for (uint32_t u = 0; u < kBatch; ++u) {
          const uint32_t t = t0 + u * 64 + lane;
          xt[u].load(rx, r * a.in_dim + 8 * t, 8 * t, a.in_dim, t < tpr);
        }
#pragma unroll
        for (uint32_t u = 0; u < kBatch; ++u)
#pragma unroll
          for (int k = 0; k < 8; ++k) mx = fmaxf(mx, fabsf(xt[u].get(k)));
      }
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
      if (lane == 0) s_inv[r] = (mx < 1e-8f) ? 1.0f : 127.0f / mx;
    }
    sync();
  }

  // ---- per-lane constants
  const typename F::Consts fk = F::consts(lane);
  // A row l%32 = (activation row, plane); plane 3 and absent rows read zeros.
  // W8A8: A row l%32 = activation row l%32 (its q); rows from m on read zeros.
  const uint32_t ai = lane & 31, axr = ai >> 2, ap = ai & 3;
  const uint32_t zero_plane = kW8A8 ? a.m : 3u * kRows;
  const uint32_t aplane = kW8A8 ? (ai < a.m ? ai : zero_plane)
                                : ((ap == 3 || axr >= a.m) ? zero_plane : axr * 3 + ap);
  const uint32_t a_base0 = a.xdig_ofs + aplane * a.plane_stride + (F::kHalf ? 8 : 16) * h;
  // the second operand (16 rows): activation rows 8..15
  const uint32_t aplane1 = (ap == 3 || axr + 8 >= a.m) ? zero_plane : (axr + 8) * 3 + ap;
  const uint32_t a_base[2] = {a_base0,
                              a.xdig_ofs + aplane1 * a.plane_stride + (F::kHalf ? 8 : 16) * h};
  const uint32_t xs_base = a.xsc_ofs + h * kT * 4;
  // activation scales of rows 2 tt + h for slice sub-block sub
  auto load_xs = [&](float* xs, uint32_t sub) {
    if constexpr (kT >= 4) {
#pragma unroll
      for (uint32_t q4 = 0; q4 < kT / 4; ++q4) {
        const u32x4 v = lds_u4(xs_base + sub * kRows * 4 + 16 * q4);
        xs[4 * q4] = __uint_as_float(v.x); xs[4 * q4 + 1] = __uint_as_float(v.y);
        xs[4 * q4 + 2] = __uint_as_float(v.z); xs[4 * q4 + 3] = __uint_as_float(v.w);
      }
    } else if constexpr (kT == 2) {
      const u32x2 v = lds_u2(xs_base + sub * kRows * 4);
      xs[0] = __uint_as_float(v.x); xs[1] = __uint_as_float(v.y);
    } else if constexpr (kT == 1) {
      xs[0] = *reinterpret_cast<const __attribute__((address_space(3))) float*>(
          static_cast<uintptr_t>(xs_base + sub * kRows * 4));
    }
  };

  // ---- digitisation of one K slice: task = row * (32 S) + 8-column group
  XTask<XD, kVecX> xo[kTasks];
  auto load_x = [&](uint32_t s) {
    const uint32_t sb0 = s << a.slice_shift;
    const uint32_t s_eff = min(S, a.bpr - sb0);
#pragma unroll
    for (uint32_t u = 0; u < (uint32_t)kTasks; ++u) {
      const uint32_t task = u * kRowsThreads + tid;
      const uint32_t xrow = task >> (a.slice_shift + 5);
      const uint32_t col8 = task & (32 * S - 1);
      const uint32_t c0 = sb0 * kQK + col8 * 8;
      const bool ok = s < a.nslices && xrow < a.m && col8 < 32 * s_eff && c0 < a.in_dim;
      xo[u].load(rx, xrow * a.in_dim + c0, c0, a.in_dim, ok);
    }
  };
  auto digitize = [&](uint32_t s) {
    const uint32_t sb0 = s << a.slice_shift;
    const uint32_t s_eff = min(S, a.bpr - sb0);
#pragma unroll
    for (uint32_t u = 0; u < (uint32_t)kTasks; ++u) {
      const uint32_t task = u * kRowsThreads + tid;
      const uint32_t xrow = task >> (a.slice_shift + 5);
      const uint32_t col8 = task & (32 * S - 1);
      const bool ok = xrow < a.m && col8 < 32 * s_eff;  // same on the 4 lanes of a quad
      float inv = 1.0f;
      if constexpr (kW8A8) inv = s_inv[min(xrow, kRows - 1u)];
      float xv[8], qv[8];
      uint32_t mb = 0;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        xv[k] = xo[u].get(k);
        if constexpr (kW8A8) xv[k] = qv[k] = quant_w8a8(xv[k], inv);
      }
      if constexpr (kW8A8) {
        // xv only flags values whose q / inv is not finite: for inv >= 2^-100,
        // |q / inv| <= 127 * 2^100 is finite unless q is NaN
        if (inv < 0x1p-100f) {
#pragma unroll
          for (int k = 0; k < 8; ++k) xv[k] = qv[k] / inv;
        }
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) mb = max(mb, __float_as_uint(xv[k]) & kAbsMask);
      mb = quad_max_u32(mb);
      if (mb >= kInfBits) {  // a NaN or an infinity: set aside (fixed up at the end)
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
        if (ok) atomicOr(s_special, 1u << xrow);
      }
      if constexpr (kW8A8) {
        // the row's plane: q as signed bytes
        if (ok) {
          uint32_t qb[2] = {0, 0};
#pragma unroll
          for (int k = 0; k < 8; ++k)
            qb[k >> 2] |= ((uint32_t)(int)qv[k] & 0xFFu) << (8 * (k & 3));
          *reinterpret_cast<uint2*>(xdig + xrow * a.plane_stride + col8 * 8) =
              make_uint2(qb[0], qb[1]);
        }
      } else if (ok) {
        const int e = digit_exponent(__uint_as_float(mb));
        const float scale = ldexpf(1.0f, F::kDigitShift - e);
        uint32_t dg[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) dg[k] = digitize_biased(xv[k], scale);
        uint32_t p0[2], p1[2], p2[2];
        digits_to_planes(dg[0], dg[1], dg[2], dg[3], p0[0], p1[0], p2[0]);
        digits_to_planes(dg[4], dg[5], dg[6], dg[7], p0[1], p1[1], p2[1]);
        uint8_t* dst = xdig + xrow * 3 * a.plane_stride + col8 * 8;
        *reinterpret_cast<uint2*>(dst) = make_uint2(p0[0] ^ 0x80808080u, p0[1] ^ 0x80808080u);
        *reinterpret_cast<uint2*>(dst + a.plane_stride) =
            make_uint2(p1[0] ^ 0x80808080u, p1[1] ^ 0x80808080u);
        *reinterpret_cast<uint2*>(dst + 2 * a.plane_stride) =
            make_uint2(p2[0] ^ 0x80808080u, p2[1] ^ 0x80808080u);
        if ((col8 & 3) == 0)
          xsc[(col8 >> 2) * kRows + (xrow & 1) * kT + (xrow >> 1)] =
              ldexpf(1.0f, e - F::kDigitShift - 3);
      }
    }
  };

  // ---- scale bytes of slice s for the chunk's rows, in 2-byte tasks: loaded
  // with the slice's activations (coalesced, unlike a unit's own scattered
  // scale bytes), written to LDS after its digitisation
  uint32_t crow0 = 0;  // first row of the current chunk
  uint32_t sraw[kScaleTasks];
  auto load_scales = [&](uint32_t s) {
    const uint32_t sb0 = s << a.slice_shift;
    const uint32_t per_row = kSH << a.slice_shift;  // 2-byte tasks per row and slice
#pragma unroll
    for (uint32_t k = 0; k < kScaleTasks; ++k) {
      const uint32_t i = tid + k * kRowsThreads;
      const uint32_t rl = (i >> a.slice_shift) / kSH;
      const uint32_t w = i - rl * per_row;
      const bool ok = s < a.nslices && rl < R * 32 && crow0 + rl < a.out_dim &&
                      sb0 + w / kSH < a.bpr;
      sraw[k] = __builtin_amdgcn_raw_buffer_load_b16(
          rs, ok ? ((crow0 + rl) * a.bpr + sb0) * F::kScaleBytes + 2 * w : kOutOfRange, 0, 0);
    }
  };
  auto stage_scales = [&]() {
#pragma unroll
    for (uint32_t k = 0; k < kScaleTasks; ++k) {
      const uint32_t i = tid + k * kRowsThreads;
      if (i < ((R * 32 * kSH) << a.slice_shift))
        *reinterpret_cast<uint16_t*>(lds + a.sc_ofs + 2 * i) = (uint16_t)sraw[k];
    }
  };

  // ---- weight units: this wave's t-th unit of slice s is half-super-block
  // ul = wp + P * t of the slice (super-block s * S + ul / 2, half ul % 2);
  // lane (n, h) loads its half of row n's bytes of the unit
  typename F::Unit q[kU];
  uint32_t row0 = 0;
  auto issue_unit = [&](uint32_t s, uint32_t t) {
    const uint32_t sb0 = s << a.slice_shift;
    const uint32_t ul = wp + P * t;
    const uint32_t row = row0 + n;
    const bool ok = s < a.nslices && ul < 2 * min(S, a.bpr - sb0) && row < a.out_dim;
    q[t] = F::load(rw, ok, row * a.bpr + sb0 + (ul >> 1), ul & 1, h);
  };

  float acc[kAcc];
  bool tables_ready = false;
  uint32_t* s_last = reinterpret_cast<uint32_t*>(lds + a.flag_ofs + 4);  // last part (split)
  for (uint32_t chunk = blockIdx.x; chunk < a.nchunks; chunk += gridDim.x) {
    if (chunk != blockIdx.x) sync();  // the previous chunk's flags are read
    // row group chunk (of R row groups) and K part of this chunk
    const uint32_t rgc = chunk / a.kparts, kpart = chunk - rgc * a.kparts;
    const uint32_t s_begin = kpart * a.kslices;
    const uint32_t s_end = min(a.nslices, s_begin + a.kslices);
    row0 = (rgc * R + rgl) * 32;
    crow0 = rgc * R * 32;
    const uint32_t code = !tables_ready ? F::seed(tid) : 0u;
    if (tid == 0) *s_special = 0;
    // set-up loads ahead of the weights: the first slice's activations, then a
    // barrier (which does not wait for loads), so that every wave's activation
    // requests are queued before any weight request
    load_x(s_begin);
    load_scales(s_begin);
    sync();
#pragma unroll
    for (uint32_t t = 0; t < kEarly && t < kU; ++t) issue_unit(s_begin, t);
    if (!tables_ready) {
      F::tables(lds, tid, code);
      tables_ready = true;
    }
#pragma unroll
    for (uint32_t t = 0; t < kAcc; ++t) acc[t] = 0.0f;

    // One K slice: digits of slice s (its activations are in flight), then
    // this wave's units of slice s (each prefetches the next slice's unit).
    // The first slice runs as straight-line code before the loop, so the wait
    // for its activations counts exactly the weight loads issued behind them.
    auto run_slice = [&](uint32_t s) {
      // the zero plane (its area is rewritten by the partial sums at the end)
      if (tid < 16 * S)
        *reinterpret_cast<u32x4*>(xdig + zero_plane * a.plane_stride + 16 * tid) =
            u32x4{0, 0, 0, 0};
      digitize(s);
      stage_scales();
      sync();
      const uint32_t sb0 = s << a.slice_shift;
      const uint32_t s_eff = min(S, a.bpr - sb0);
      // this lane's row of the staged scale bytes
      const uint32_t sc_row = a.sc_ofs + ((rgl * 32 + n) << a.slice_shift) * F::kScaleBytes;
#pragma unroll
      for (uint32_t t = 0; t < kU; ++t) {
        // the first slice's later units: one more in flight per unit computed
        if (s == s_begin && t + kEarly < kU) issue_unit(s_begin, t + kEarly);
        const uint32_t ul = wp + P * t;
        if (ul >= 2 * s_eff) break;  // uniform
        // the codes of the unit's 4 sub-blocks for this lane's row, and its scales
        F::fill_scales(q[t], sc_row + (ul >> 1) * F::kScaleBytes, ul & 1);
        const typename F::Words w = F::unpack(q[t]);
        const float dq = F::unit_scale(q[t]);
        // the registers are free: prefetch (none after the last slice)
        if (s + 1 < s_end) issue_unit(s + 1, t);
        float au[kT];
#pragma unroll
        for (uint32_t tt = 0; tt < kT; ++tt) au[tt] = 0.0f;
        // c: this lane's 16 results of the MFMA of A operand o; scale: the
        // sub-scale of its columns.  Digits: au += (integer plane sums of c) *
        // scale * xs, activation row 2 tt + h (tt = kTO o + i).  W8A8: acc +=
        // c * (2s+1) d, exact int32 sums of q (|c| < 2^24) times an exact scale.
        auto accumulate = [&](const v16i& c, float scale, const float* xs, uint32_t o) {
          if constexpr (kW8A8) {
            const float sd = scale * dq;
#pragma unroll
            for (uint32_t r = 0; r < kAcc; ++r) acc[r] = fmaf((float)c[r], sd, acc[r]);
          } else {
#pragma unroll
            for (uint32_t i = 0; i < kTO; ++i) {
              const uint32_t tt = kTO * o + i;
              const uint32_t hi = ((uint32_t)c[4 * i + 2] << 8) + (uint32_t)c[4 * i + 1];
              const float f = F::kSplitSum
                                  ? fmaf((float)(int)hi, 256.0f, (float)c[4 * i])
                                  : (float)(int)((hi << 8) + (uint32_t)c[4 * i]);
              au[tt] = fmaf(f, scale * xs[tt], au[tt]);
            }
          }
        };
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
          const uint32_t sub = ul * 4 + j;  // sub-block in the slice
          // (the one-operand instantiations keep their own code: written as the
          // two-operand loop with one trip, the compiler schedules them
          // differently, and W8A8 at 32 rows ran 8 % slower)
          if constexpr (!F::kHalf && kAOps == 1) {
            const v4i bw = F::pair(w, j, fk);
            const u32x4 av = lds_u4(a_base0 + sub * 32);
            const v4i aw = {(int)av.x, (int)av.y, (int)av.z, (int)av.w};
            const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(aw, bw, v16i{}, 0, 0, 0);
            float xs[kT];
            if constexpr (!kW8A8) load_xs(xs, sub);
            accumulate(c, F::pair_scale(w, j, fk), xs, 0);
          } else if constexpr (!F::kHalf) {
            const v4i bw = F::pair(w, j, fk);
            float xs[kT];
#pragma unroll
            for (uint32_t o = 0; o < kAOps; ++o) {
              const u32x4 av = lds_u4(a_base[o] + sub * 32);
              const v4i aw = {(int)av.x, (int)av.y, (int)av.z, (int)av.w};
              const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(aw, bw, v16i{}, 0, 0, 0);
              if (o == 0) {
                if constexpr (!kW8A8) load_xs(xs, sub);
              }
              accumulate(c, F::pair_scale(w, j, fk), xs, o);
            }
          } else if constexpr (kAOps == 1) {
            float xs[kT];
            if constexpr (!kW8A8) load_xs(xs, sub);
#pragma unroll
            for (uint32_t hf = 0; hf < 2; ++hf) {
              const u32x2 bw = F::group(w, j, hf, fk);
              const u32x2 av = lds_u2(a_base0 + sub * 32 + 16 * hf);
              const v16i c = __builtin_amdgcn_mfma_i32_32x32x16_i8(
                  (long)(((uint64_t)av.y << 32) | av.x), (long)(((uint64_t)bw.y << 32) | bw.x),
                  v16i{}, 0, 0, 0);
              accumulate(c, F::group_scale(w, j, hf), xs, 0);
            }
          } else {
            float xs[kT];
            if constexpr (!kW8A8) load_xs(xs, sub);
#pragma unroll
            for (uint32_t hf = 0; hf < 2; ++hf) {
              const u32x2 bw = F::group(w, j, hf, fk);
#pragma unroll
              for (uint32_t o = 0; o < kAOps; ++o) {
                const u32x2 av = lds_u2(a_base[o] + sub * 32 + 16 * hf);
                const v16i c = __builtin_amdgcn_mfma_i32_32x32x16_i8(
                    (long)(((uint64_t)av.y << 32) | av.x), (long)(((uint64_t)bw.y << 32) | bw.x),
                    v16i{}, 0, 0, 0);
                accumulate(c, F::group_scale(w, j, hf), xs, o);
              }
            }
          }
        }
        if constexpr (!kW8A8) {
#pragma unroll
          for (uint32_t tt = 0; tt < kT; ++tt) acc[tt] = fmaf(au[tt], dq, acc[tt]);
        }
      }
    };
    sync();  // tables and the cleared flag
    run_slice(s_begin);
    for (uint32_t s = s_begin + 1; s < s_end; ++s) {
      load_x(s);
      load_scales(s);
      sync();  // the previous slice's digits and scales are consumed
      run_slice(s);
    }

    // ---- the P waves of a row group add their partial sums in wave order
    // (split over K: into this part's sums in the workspace)
    const uint32_t chunk_row0 = rgc * R * 32;
    const bool split = a.kparts > 1;  // uniform
    float* const psum = split ? a.part_sums + (size_t)kpart * a.m * a.out_dim : nullptr;
    uint32_t special = 0;
    bool gated = false;
    if constexpr (kW8A8) {
      // four result registers at a time: activation rows 8 g + 4 h + i
#pragma unroll
      for (uint32_t g = 0; g < kAcc / 4; ++g) {
        if (8 * g >= a.m) break;  // uniform
        sync();
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i)
          red[((rgl * P + wp) * 4 + i) * 64 + lane] = acc[4 * g + i];
        sync();
        special = *s_special;  // uniform (final since the last digitisation)
        gated = a.gate != nullptr && special == 0;
        for (uint32_t o = tid; o < R * 4 * 64; o += kRowsThreads) {
          const uint32_t ol = o & 63, i = (o >> 6) & 3, rg = o >> 8;
          float sum = 0.0f;
          for (uint32_t w = 0; w < P; ++w) sum += red[((rg * P + w) * 4 + i) * 64 + ol];
          const uint32_t xrow = 8 * g + 4 * (ol >> 5) + i, row = chunk_row0 + rg * 32 + (ol & 31);
          if (xrow < a.m && row < a.out_dim) {
            const size_t oi = (size_t)xrow * a.out_dim + row;
            if (split) {
              part_store(psum + oi, sum);
            } else {
              const float v = sum * 0.125f / s_inv[xrow];  // q / inv, and the weights' 1/8
              a.out[oi] = gated ? silu_mul(a.gate[oi], v) : v;
            }
          }
        }
      }
    } else {
      sync();
#pragma unroll
      for (uint32_t tt = 0; tt < kT; ++tt)
        red[((rgl * P + wp) * kT + tt) * 64 + lane] = acc[tt];
      sync();
      special = *s_special;  // uniform (final since the last digitisation)
      gated = a.gate != nullptr && special == 0;
      for (uint32_t o = tid; o < R * kT * 64; o += kRowsThreads) {
        const uint32_t ol = o & 63, tt = (o >> 6) % kT, rg = (o >> 6) / kT;
        float sum = 0.0f;
        for (uint32_t w = 0; w < P; ++w) sum += red[((rg * P + w) * kT + tt) * 64 + ol];
        const uint32_t xrow = 2 * tt + (ol >> 5), row = chunk_row0 + rg * 32 + (ol & 31);
        if (xrow < a.m && row < a.out_dim) {
          const size_t i = (size_t)xrow * a.out_dim + row;
          if (split)
            part_store(psum + i, sum);
          else
            a.out[i] = gated ? silu_mul(a.gate[i], sum) : sum;
        }
      }
    }

    // ---- split over K: hand the sums over; the last part of the row group
    // to arrive adds every part's sums in part order and goes on with the
    // outputs' fix-up (R = 1 when split)
    if (split) {
      const uint32_t nrow = min(32u, a.out_dim - chunk_row0);
      if (tid == 0)
        __hip_atomic_store(a.part_special + rgc * a.kparts + kpart, special, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      // every wave's stores of the sums complete (performed at agent scope)
      // before the barrier, and the barrier before the arrival
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      sync();
      if (tid == 0) *s_last = rows_arrive_last(a.arrive + rgc, a.epoch, a.kparts) ? 1u : 0u;
      sync();
      if (*s_last == 0) continue;  // uniform: another part finishes this row group
      special = 0;
      for (uint32_t k = 0; k < a.kparts; ++k)
        special |= __hip_atomic_load(a.part_special + rgc * a.kparts + k, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
      gated = a.gate != nullptr && special == 0;
      for (uint32_t o = tid; o < a.m * nrow; o += kRowsThreads) {
        const uint32_t xrow = o / nrow, rl = o - xrow * nrow;
        const size_t i = (size_t)xrow * a.out_dim + chunk_row0 + rl;
        float sum = 0.0f;
        for (uint32_t k = 0; k < a.kparts; ++k)
          sum += part_load(a.part_sums + (size_t)k * a.m * a.out_dim + i);
        if constexpr (kW8A8) sum = sum * 0.125f / s_inv[xrow];
        a.out[i] = gated ? silu_mul(a.gate[i], sum) : sum;
      }
      if (tid == 0)
        __hip_atomic_store(a.arrive + rgc, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // ---- rows that held a NaN or an infinity: add the kind of the
    // set-aside terms x_c * w_rc to the chunk's outputs
    sync();
    if (special) {
      const uint32_t rows = min(R * 32, a.out_dim - min(chunk_row0, a.out_dim));
      for (uint32_t xrow = 0; xrow < a.m; ++xrow) {
        if (!((special >> xrow) & 1u)) continue;
        if constexpr (kW8A8) {
          // an infinite activation makes the row's max infinite and inv 0:
          // every q / inv of the row is NaN, and so is every output, as in the
          // reference (uniform branch)
          if (s_inv[xrow] == 0.0f) {
            for (uint32_t rl = tid; rl < rows; rl += kRowsThreads)
              a.out[(size_t)xrow * a.out_dim + chunk_row0 + rl] = __builtin_nanf("");
            continue;
          }
        }
        for (uint32_t rl = tid; rl < rows; rl += kRowsThreads) s_kinds[rl] = 0;
        sync();
        float inv = 1.0f;
        if constexpr (kW8A8) inv = s_inv[xrow];
        const size_t xbase = (size_t)xrow * a.in_dim;
        for (uint32_t c = tid; c < a.in_dim; c += kRowsThreads) {
          float v = x_bits_to_float<XD>(load_x_bits<XD>(a.x, xbase + c));
          if constexpr (kW8A8) v = qdq_w8a8(v, inv);
          if ((__float_as_uint(v) & kAbsMask) < kInfBits) continue;
          for (uint32_t rl = 0; rl < rows; ++rl)
            atomicOr(&s_kinds[rl],
                     special_kind(v * F::weight_at(a.wb, a.ws, chunk_row0 + rl, c, a.bpr)));
        }
        sync();
        for (uint32_t rl = tid; rl < rows; rl += kRowsThreads) {
          const uint32_t kinds = s_kinds[rl];
          float* o = a.out + (size_t)xrow * a.out_dim + chunk_row0 + rl;
          if (kinds) *o = *o + special_value(kinds);
        }
        sync();
      }
      // the gated step on the completed sums
      if (a.gate != nullptr) {
        const uint32_t rows = min(R * 32, a.out_dim - min(chunk_row0, a.out_dim));
        for (uint32_t i = tid; i < a.m * rows; i += kRowsThreads) {
          const uint32_t xrow = i / rows, rl = i - xrow * rows;
          const size_t o = (size_t)xrow * a.out_dim + chunk_row0 + rl;
          a.out[o] = silu_mul(a.gate[o], a.out[o]);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Launch policy.
// ---------------------------------------------------------------------------
struct RowsPlan {
  uint32_t rows;   // kRows
  uint32_t tasks;  // kTasks
  uint32_t rg_shift, nchunks, grid, slice_shift, nslices, plane_stride;
  uint32_t xdig_ofs, xsc_ofs, flag_ofs, sc_ofs;
  uint32_t kparts, kslices;  // split over K
  size_t lds;
};

static uint32_t align16r(uint64_t v) { return (uint32_t)((v + 15) & ~15ull); }
static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Parts the split over K may cut each 32-row group into: the largest power of
// two up to 8 that keeps the chunks within one per CU, with at least one
// super-block per part (1: no split).  A function of the shape and the CU
// count only, so the workspace query and the launch agree.
static uint32_t rows_kparts_max(uint64_t out_dim, uint64_t in_dim, uint64_t cus) {
  const uint64_t n_rg = (out_dim + 31) / 32, bpr = (in_dim + kQK - 1) / kQK;
  uint32_t k = 1;
  while (k < 8 && n_rg * (2 * k) <= cus && 2 * k <= bpr) k *= 2;
  return k;
}

// Instantiation rows for m activation rows (the kernel's kRows).
static uint32_t rows_for(uint32_t m, bool w8a8) {
  return w8a8 ? (m <= 8 ? 8 : 32) : (m <= 2 ? 2 : (m <= 4 ? 4 : (m <= 8 ? 8 : 16)));
}

// Whether splitting K in kmax parts shortens the launch.  The exchange of
// the sums costs about three memory round trips (the sums' stores, the
// arrival, the last part's loads: about 3 us at N = 4096) and more with more
// parts (the arrivals retry against each other), so the split pays where a
// workgroup's unsplit K loop is long: measured on MI355X (f32 x, mode Off and
// W8A8, M = 2..32, N = 1024..4096, K = 2048..14336), splitting won for K >=
// 12288 at any row count (N = 4096, K = 14336: 16.1 -> 13.4 us at M = 2),
// for the 16-row (W8A8: 32-row) launches at K >= 8192, and for those at
// K = 4096 with at most 4 parts (N = 4096 M = 16: 16.5 -> 13.8 us); it lost
// 1-3 us at 2-8 rows with K <= 8192 (N = 4096, M = 4: 8.7 -> 10.4 us) and at
// 8 parts with K = 4096 (N = 1024 M = 16: 16.0 -> 17.4 us).
static bool rows_split_pays(uint32_t m, bool w8a8, uint32_t in_dim, uint32_t kmax) {
  if (kmax < 2) return false;
  const bool big = w8a8 ? rows_for(m, true) == 32 : rows_for(m, false) == 16;
  return in_dim >= 12288 || (big && in_dim >= 8192) || (big && kmax <= 4 && in_dim >= 4096);
}

// Workspace of the split: arrival words, the parts' non-finite masks, then
// the parts' sums for `rows` activation rows.
static size_t rows_split_layout(uint32_t rows, uint32_t out_dim, uint32_t kmax,
                                size_t* special_ofs, size_t* sums_ofs) {
  const size_t n_rg = (out_dim + 31) / 32;
  *special_ofs = align256(n_rg * sizeof(unsigned long long));
  *sums_ofs = *special_ofs + align256(n_rg * kmax * sizeof(uint32_t));
  return *sums_ofs + (size_t)kmax * rows * out_dim * sizeof(float);
}

size_t gemv_rows_split_bytes(uint32_t m, uint32_t out_dim, uint32_t in_dim, bool w8a8,
                             int num_cus) {
  if (m < 2 || out_dim == 0 || in_dim == 0) return 0;
  const uint32_t kmax = rows_kparts_max(out_dim, in_dim, num_cus > 0 ? (uint64_t)num_cus : 1);
  // (the largest launch of the call: later ones have no more rows, and the
  // split pays for fewer rows only where it pays for more)
  const uint32_t group = w8a8 ? 32 : 16;
  const uint32_t rows = m < group ? m : group;
  if (!rows_split_pays(rows, w8a8, in_dim, kmax)) return 0;
  size_t so, mo;
  return rows_split_layout(rows, out_dim, kmax, &so, &mo);
}

// Launch shape for m (1..16; W8A8 1..32) x out_dim x in_dim on num_cus CUs
// for format F, split over K when `split` allows it; false when the shape
// does not fit (31-bit buffer offsets, LDS).
template <class F>
static bool plan_rows(uint32_t m, uint32_t out_dim, uint32_t in_dim, int x_dtype, bool vec,
                      bool w8a8, int num_cus, bool split, RowsPlan* p) {
  if (m < 1 || m > (w8a8 ? 32u : 16u) || out_dim == 0 || in_dim == 0) return false;
  const uint64_t bpr = (in_dim + kQK - 1) / kQK;
  const uint64_t esize = x_dtype == 0 ? 4 : 2;
  if ((uint64_t)out_dim * bpr * F::kBlockBytes > kOutOfRange - 4096) return false;
  if ((uint64_t)out_dim * bpr * F::kScaleBytes > kOutOfRange - 4096) return false;
  if ((uint64_t)m * in_dim * esize > kOutOfRange - 4096) return false;
  p->rows = rows_for(m, w8a8);
  p->tasks = rows_tasks(p->rows, w8a8, m);
  // activation rows digitised per slice (W8A8 digitises the m rows only)
  const uint64_t task_rows = w8a8 ? m : p->rows;
  const uint64_t n_rg = (out_dim + 31) / 32;
  const uint64_t cus = num_cus > 0 ? (uint64_t)num_cus : 1;
  uint32_t rs = 0;
  while (rs < 4 && (n_rg + (1u << rs) - 1) >> rs > cus) ++rs;
  p->rg_shift = rs;
  const uint64_t waves_per_rg = kRowsWaves >> rs;
  const uint64_t rg_chunks = (n_rg + (1u << rs) - 1) >> rs;
  // (n_rg <= cus whenever kmax > 1, so R = 1 when split)
  const uint32_t kmax = split ? rows_kparts_max(out_dim, in_dim, cus) : 1;
  // slice: a power of two of super-blocks, at most kU units per wave and two
  // digitisation tasks per thread, whose digits fit in LDS beside the tables;
  // split: at most bpr / kmax, so that every part holds at least one slice
  const uint64_t units = rows_units<F>((int)p->rows, vec, w8a8);
  uint32_t ss = 0;
  while (2 * (2ull << ss) <= units * waves_per_rg &&
         task_rows * (2ull << ss) * 32 <= p->tasks * kRowsThreads &&
         (1ull << ss) < bpr && (2ull << ss) * kmax <= bpr)
    ++ss;
  for (;; --ss) {
    const uint64_t S = 1ull << ss;
    p->slice_shift = ss;
    p->nslices = (uint32_t)((bpr + S - 1) / S);
    p->plane_stride = (uint32_t)(S * kQK + 16);
    // digit planes and the zero plane; W8A8: the rows' q and the zero plane
    const uint64_t digits = (w8a8 ? m + 1ull : 3ull * p->rows + 1) * p->plane_stride;
    const uint64_t partials = (uint64_t)kRowsWaves * (w8a8 ? 4 : p->rows / 2) * 64 * 4;
    const uint64_t kinds = (1ull << rs) * 32 * 4;
    uint64_t region = digits > partials ? digits : partials;
    region = region > kinds ? region : kinds;
    p->xdig_ofs = F::kTableBytes;
    p->xsc_ofs = p->xdig_ofs + align16r(region);
    p->flag_ofs = p->xsc_ofs + (w8a8 ? 0u : align16r(S * 8 * p->rows * 4));
    // the kernel stages the slice's scale bytes in 32 * 8 * units 2-byte
    // tasks per scale-byte pair: R * S <= 8 units (the slice growth keeps it)
    if ((1ull << rs) * S > 8 * units) return false;
    p->sc_ofs = p->flag_ofs + rows_flag_bytes(p->rows);
    p->lds = p->sc_ofs + align16r((1ull << rs) * 32 * S * F::kScaleBytes);
    if (p->lds <= kGemvLdsLimit) {
      p->kslices = (p->nslices + kmax - 1) / kmax;
      p->kparts = (p->nslices + p->kslices - 1) / p->kslices;  // every part non-empty
      const uint64_t chunks = rg_chunks * p->kparts;
      p->nchunks = (uint32_t)chunks;
      p->grid = chunks < cus ? (uint32_t)chunks : (uint32_t)cus;
      return true;
    }
    if (ss == 0) return false;
  }
}

bool gemv_rows_supported(uint32_t m, uint32_t out_dim, uint32_t in_dim, int x_dtype,
                         bool w8a8) {
  RowsPlan p;
  return plan_rows<RowsFmtXXS>(m, out_dim, in_dim, x_dtype, false, w8a8, 1, false, &p);
}

template <class F, int XD, bool V, bool Q, int ROWS, int TASKS>
static hipError_t launch_rows_t(const RowsArgs& a, const RowsPlan& p, hipStream_t stream) {
  // The tables alone exceed the default 64 KB of dynamic LDS: raise the
  // limit once per instantiation.
  static std::atomic<bool> attr_set{false};
  if (!attr_set.load()) {
    hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&iq_gemv_rows_kernel<F, XD, V, Q, ROWS, TASKS>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGemvLdsLimit);
    if (e != hipSuccess) return e;
    attr_set.store(true);
  }
  hipLaunchKernelGGL((iq_gemv_rows_kernel<F, XD, V, Q, ROWS, TASKS>), dim3(p.grid),
                     dim3(kRowsThreads), p.lds, stream, a);
  return hipGetLastError();
}

template <class F, int XD, bool V>
static hipError_t launch_rows_v(const RowsArgs& a, const RowsPlan& p, bool w8a8,
                                hipStream_t stream) {
  // (task slots as rows_tasks chose them in the plan)
  if (w8a8) {
    if (p.rows == 32) return launch_rows_t<F, XD, V, true, 32, 2>(a, p, stream);
    return p.tasks == 1 ? launch_rows_t<F, XD, V, true, 8, 1>(a, p, stream)
                        : launch_rows_t<F, XD, V, true, 8, 2>(a, p, stream);
  }
  if (p.rows == 2) return launch_rows_t<F, XD, V, false, 2, 1>(a, p, stream);
  if (p.rows == 16) return launch_rows_t<F, XD, V, false, 16, 2>(a, p, stream);
  return p.rows == 4 ? launch_rows_t<F, XD, V, false, 4, 1>(a, p, stream)
                     : launch_rows_t<F, XD, V, false, 8, 2>(a, p, stream);
}

// Launch epochs of the split over K: distinct per launch (a captured launch
// keeps its own), never 0 (a cleared arrival word).
static uint32_t next_rows_epoch() {
  static std::atomic<uint32_t> counter{0};
  for (;;) {
    const uint32_t e = (counter.fetch_add(1) + 1u) * 2654435761u;  // odd multiplier: a bijection
    if (e != 0) return e;
  }
}

// One launch for m <= 16 rows (W8A8: m <= 32); split over K when the shape
// leaves CUs idle and `split_ws` (16-byte aligned) holds split_ws_bytes >=
// gemv_rows_split_bytes(m, ...).
template <class F>
static hipError_t launch_rows_fmt(const void* x, int x_dtype, uint32_t m, const uint8_t* wb,
                                  const uint8_t* ws, float* out, uint32_t out_dim,
                                  uint32_t in_dim, bool w8a8, int num_cus, hipStream_t stream,
                                  const float* gate, void* split_ws, size_t split_ws_bytes) {
  const size_t esize = x_dtype == 0 ? 4 : 2;
  const bool vec = (in_dim % 8 == 0) && (reinterpret_cast<uintptr_t>(x) % 16 == 0) &&
                   ((size_t)in_dim * esize % 16 == 0);
  const uint32_t kmax = rows_kparts_max(out_dim, in_dim, num_cus > 0 ? (uint64_t)num_cus : 1);
  size_t special_ofs = 0, sums_ofs = 0;
  const size_t split_need = rows_split_pays(m, w8a8, in_dim, kmax)
                                ? rows_split_layout(m, out_dim, kmax, &special_ofs, &sums_ofs)
                                : 0;
  const bool split = split_need > 0 && split_ws != nullptr && split_ws_bytes >= split_need &&
                     reinterpret_cast<uintptr_t>(split_ws) % 16 == 0;
  RowsPlan p;
  if (!plan_rows<F>(m, out_dim, in_dim, x_dtype, vec, w8a8, num_cus, split, &p))
    return hipErrorInvalidValue;
  RowsArgs a;
  a.x = x;
  a.wb = wb;
  a.ws = ws;
  a.out = out;
  a.m = m;
  a.out_dim = out_dim;
  a.in_dim = in_dim;
  a.bpr = (in_dim + kQK - 1) / kQK;
  a.n_rg = (out_dim + 31) / 32;
  a.rg_shift = p.rg_shift;
  a.nchunks = p.nchunks;
  a.slice_shift = p.slice_shift;
  a.nslices = p.nslices;
  a.wb_records = out_dim * a.bpr * F::kBlockBytes;
  a.ws_records = out_dim * a.bpr * F::kScaleBytes;
  a.x_records = m * in_dim * (x_dtype == 0 ? 4u : 2u);
  a.plane_stride = p.plane_stride;
  a.xdig_ofs = p.xdig_ofs;
  a.xsc_ofs = p.xsc_ofs;
  a.flag_ofs = p.flag_ofs;
  a.sc_ofs = p.sc_ofs;
  a.gate = gate;
  a.kparts = p.kparts;
  a.kslices = p.kslices;
  a.epoch = p.kparts > 1 ? next_rows_epoch() : 0u;
  uint8_t* const wsb = static_cast<uint8_t*>(split_ws);
  a.arrive = p.kparts > 1 ? reinterpret_cast<unsigned long long*>(wsb) : nullptr;
  a.part_special = p.kparts > 1 ? reinterpret_cast<uint32_t*>(wsb + special_ofs) : nullptr;
  a.part_sums = p.kparts > 1 ? reinterpret_cast<float*>(wsb + sums_ofs) : nullptr;
  switch (x_dtype) {
    case 0: return vec ? launch_rows_v<F, 0, true>(a, p, w8a8, stream)
                       : launch_rows_v<F, 0, false>(a, p, w8a8, stream);
    case 1: return vec ? launch_rows_v<F, 1, true>(a, p, w8a8, stream)
                       : launch_rows_v<F, 1, false>(a, p, w8a8, stream);
    default: return vec ? launch_rows_v<F, 2, true>(a, p, w8a8, stream)
                        : launch_rows_v<F, 2, false>(a, p, w8a8, stream);
  }
}

hipError_t launch_iq2xxs_gemv_rows(const void* x, int x_dtype, uint32_t m, const uint8_t* wb,
                                   const uint8_t* ws, float* out, uint32_t out_dim,
                                   uint32_t in_dim, bool w8a8, int num_cus, hipStream_t stream,
                                   const float* gate, void* split_ws, size_t split_ws_bytes) {
  return launch_rows_fmt<RowsFmtXXS>(x, x_dtype, m, wb, ws, out, out_dim, in_dim, w8a8, num_cus,
                                     stream, gate, split_ws, split_ws_bytes);
}

template <class F>
static bool variant_rows_fit(uint32_t out_dim, uint32_t in_dim, int x_dtype) {
  RowsPlan p;
  return plan_rows<F>(16, out_dim, in_dim, x_dtype, false, false, 1, false, &p) &&
         plan_rows<F>(8, out_dim, in_dim, x_dtype, false, false, 1, false, &p) &&
         plan_rows<F>(4, out_dim, in_dim, x_dtype, true, false, 1, false, &p) &&
         plan_rows<F>(32, out_dim, in_dim, x_dtype, false, true, 1, false, &p);
}

bool variant_rows_supported(int variant, uint32_t out_dim, uint32_t in_dim, int x_dtype) {
  switch (variant) {
    case 1: return variant_rows_fit<RowsFmtXS>(out_dim, in_dim, x_dtype);
    case 2: return variant_rows_fit<RowsFmtS>(out_dim, in_dim, x_dtype);
    case 3: return variant_rows_fit<RowsFmtS3>(out_dim, in_dim, x_dtype);
    default: return false;
  }
}

hipError_t launch_iq_variant_rows(int variant, const void* x, int x_dtype, uint32_t m,
                                  const uint8_t* wb, const uint8_t* ws, float* out,
                                  uint32_t out_dim, uint32_t in_dim, bool w8a8, int num_cus,
                                  hipStream_t stream, void* split_ws, size_t split_ws_bytes) {
  const size_t esize = x_dtype == 0 ? 4 : 2;
  // groups of 16 activation rows (W8A8: 32), each a launch that reads every
  // weight once
  const uint32_t group = w8a8 ? 32 : 16;
  for (uint32_t r0 = 0; r0 < m; r0 += group) {
    const uint32_t mr = m - r0 < group ? m - r0 : group;
    const void* xr = static_cast<const uint8_t*>(x) + (size_t)r0 * in_dim * esize;
    float* o = out + (size_t)r0 * out_dim;
    hipError_t e;
    switch (variant) {
      case 1:
        e = launch_rows_fmt<RowsFmtXS>(xr, x_dtype, mr, wb, ws, o, out_dim, in_dim, w8a8,
                                       num_cus, stream, nullptr, split_ws,
                                       split_ws_bytes);
        break;
      case 2:
        e = launch_rows_fmt<RowsFmtS>(xr, x_dtype, mr, wb, ws, o, out_dim, in_dim, w8a8,
                                      num_cus, stream, nullptr, split_ws,
                                       split_ws_bytes);
        break;
      case 3:
        e = launch_rows_fmt<RowsFmtS3>(xr, x_dtype, mr, wb, ws, o, out_dim, in_dim, w8a8,
                                       num_cus, stream, nullptr, split_ws,
                                       split_ws_bytes);
        break;
      default:
        return hipErrorInvalidValue;
    }
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace cmk
