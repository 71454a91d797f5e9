// Bandwidth ceiling probe for bench.py (not part of libcgpt.so's ABI): a
// plain device copy with one 16-byte vector per thread, non-temporal loads and
// stores (the access width and streaming policy of the HBM-bound kernels), so
// a kernel's rate can be set beside what a copy of the same bytes reaches.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace cgpt_bench {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void copy16_nt_kernel(const u32x4* __restrict__ x,
                                                        u32x4* __restrict__ y, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) __builtin_nontemporal_store(__builtin_nontemporal_load(x + i), y + i);
}

}  // namespace cgpt_bench

// Copies `bytes` (a multiple of 16; x and y 16-byte aligned) from x to y on
// `stream`.  Returns 0, or -1 for bad arguments, or the HIP error code.
extern "C" int cgpt_bench_copy16(const void* x, void* y, int64_t bytes, void* stream) {
  if (x == nullptr || y == nullptr || bytes < 0 || bytes % 16 != 0 ||
      ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15))
    return -1;
  const int64_t n = bytes / 16;
  if (n == 0) return 0;
  const int64_t blocks = (n + 255) / 256;
  if (blocks > 0x7fffffff) return -1;
  hipLaunchKernelGGL(cgpt_bench::copy16_nt_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const cgpt_bench::u32x4*>(x),
                     static_cast<cgpt_bench::u32x4*>(y), n);
  return static_cast<int>(hipGetLastError());
}
