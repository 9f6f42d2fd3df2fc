// bench_read_floor.hip — a plain read of n bytes from HBM: the floor bench.py sets
// beside the decode GEMV (the same bytes read, no decoding, no arithmetic).
// Not part of the matmul library or its C ABI; built as libcmk_probe.so.
//
// Every 16-byte chunk is read once with a nontemporal load by a grid of
// 256-thread workgroups (grid stride).  The loads are kept alive by a store
// behind a condition the data never meets (the xor of a thread's chunks equal
// to its index), so nothing is written in practice.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void probe_read_kernel(const u32x4* __restrict__ p, size_t n16,
                                                         uint32_t* __restrict__ sink) {
  const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  u32x4 acc = {0, 0, 0, 0};
  for (size_t i = tid; i < n16; i += stride) acc ^= __builtin_nontemporal_load(p + i);
  const uint32_t v = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (v == (uint32_t)tid + 0x9E3779B9u) sink[blockIdx.x] = v;
}

}  // namespace

// Reads the first bytes / 16 * 16 bytes of buf (16-byte aligned) with `blocks`
// workgroups; sink holds `blocks` words.  Returns a hipError_t code.
extern "C" int cmk_probe_read(const void* buf, size_t bytes, uint32_t* sink, int blocks,
                              void* stream) {
  if (buf == nullptr || sink == nullptr || blocks <= 0 ||
      reinterpret_cast<uintptr_t>(buf) % 16 != 0)
    return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(probe_read_kernel, dim3(blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const u32x4*>(buf), bytes / 16,
                     sink);
  return (int)hipGetLastError();
}
