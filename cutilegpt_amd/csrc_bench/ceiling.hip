// Bandwidth ceiling probes for bench.py (not part of libcgpt.so's ABI): plain
// device copies of the same bytes an HBM-bound kernel moves, so that kernel's
// rate can be set beside the best a copy reaches at that size.
//
//   variant 0: one-shot grid, one 16-byte vector a thread, non-temporal loads
//              and stores (the access width and policy of the HBM kernels);
//   variant 1: persistent grid (blocks_per_cu blocks of 256 threads a CU),
//              grid-stride over groups of VEC 16-byte vectors a thread, all of
//              a group's loads issued before its stores, non-temporal;
//   variant 2: variant 1 with the default (cached) policy;
//   variant 3: one-shot grid, VEC consecutive vectors a thread (a thread's
//              loads cover 16 * VEC contiguous bytes), non-temporal.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace cgpt_bench {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void copy16_nt_kernel(const u32x4* __restrict__ x,
                                                        u32x4* __restrict__ y, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) __builtin_nontemporal_store(__builtin_nontemporal_load(x + i), y + i);
}

// Group g covers vectors [g * 256 * VEC, (g + 1) * 256 * VEC): thread t takes
// t, t + 256, ... so each load instruction of a wave reads 1 KiB contiguous.
template <int VEC, bool NT>
__global__ __launch_bounds__(256) void copy_persistent_kernel(const u32x4* __restrict__ x,
                                                              u32x4* __restrict__ y, int64_t n) {
  const int64_t groups = (n + 256 * VEC - 1) / (256 * VEC);
  for (int64_t g = blockIdx.x; g < groups; g += gridDim.x) {
    const int64_t base = g * 256 * VEC + threadIdx.x;
    u32x4 v[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const int64_t i = base + j * 256;
      if (i < n) v[j] = NT ? __builtin_nontemporal_load(x + i) : x[i];
    }
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const int64_t i = base + j * 256;
      if (i < n) {
        if (NT)
          __builtin_nontemporal_store(v[j], y + i);
        else
          y[i] = v[j];
      }
    }
  }
}

template <int VEC>
__global__ __launch_bounds__(256) void copy_consecutive_nt_kernel(const u32x4* __restrict__ x,
                                                                  u32x4* __restrict__ y,
                                                                  int64_t n) {
  const int64_t base = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * VEC;
  u32x4 v[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j)
    if (base + j < n) v[j] = __builtin_nontemporal_load(x + base + j);
#pragma unroll
  for (int j = 0; j < VEC; ++j)
    if (base + j < n) __builtin_nontemporal_store(v[j], y + base + j);
}

static int num_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 256;
  return cus > 0 ? cus : 256;
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

// The copy variants above (variant 0 = cgpt_bench_copy16).  vec: 16-byte
// vectors a thread, 1, 2, 4 or 8 (variants 1-3); blocks_per_cu: persistent
// blocks of 256 threads a CU, 1-32 (variants 1-2).
extern "C" int cgpt_bench_copy_variant(const void* x, void* y, int64_t bytes, int variant,
                                       int vec, int blocks_per_cu, void* stream) {
  using namespace cgpt_bench;
  if (variant == 0) return cgpt_bench_copy16(x, y, bytes, stream);
  if (x == nullptr || y == nullptr || bytes < 0 || bytes % 16 != 0 ||
      ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15))
    return -1;
  if (variant < 1 || variant > 3 || !(vec == 1 || vec == 2 || vec == 4 || vec == 8)) return -1;
  if (blocks_per_cu < 1 || blocks_per_cu > 32) return -1;
  const int64_t n = bytes / 16;
  if (n == 0) return 0;
  const auto* xs = static_cast<const u32x4*>(x);
  auto* ys = static_cast<u32x4*>(y);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (variant == 3) {
    const int64_t blocks = (n + 256 * vec - 1) / (256 * vec);
    if (blocks > 0x7fffffff) return -1;
    const dim3 grid(static_cast<unsigned>(blocks));
    switch (vec) {
      case 1: hipLaunchKernelGGL(copy_consecutive_nt_kernel<1>, grid, dim3(256), 0, s, xs, ys, n); break;
      case 2: hipLaunchKernelGGL(copy_consecutive_nt_kernel<2>, grid, dim3(256), 0, s, xs, ys, n); break;
      case 4: hipLaunchKernelGGL(copy_consecutive_nt_kernel<4>, grid, dim3(256), 0, s, xs, ys, n); break;
      default: hipLaunchKernelGGL(copy_consecutive_nt_kernel<8>, grid, dim3(256), 0, s, xs, ys, n); break;
    }
    return static_cast<int>(hipGetLastError());
  }
  const int64_t groups = (n + 256 * vec - 1) / (256 * vec);
  const int64_t want = static_cast<int64_t>(num_cus()) * blocks_per_cu;
  const dim3 grid(static_cast<unsigned>(groups < want ? groups : want));
  const bool nt = variant == 1;
#define CGPT_COPY_CASE(V)                                                                      \
  case V:                                                                                      \
    if (nt)                                                                                    \
      hipLaunchKernelGGL((copy_persistent_kernel<V, true>), grid, dim3(256), 0, s, xs, ys, n);  \
    else                                                                                       \
      hipLaunchKernelGGL((copy_persistent_kernel<V, false>), grid, dim3(256), 0, s, xs, ys, n); \
    break;
  switch (vec) {
    CGPT_COPY_CASE(1)
    CGPT_COPY_CASE(2)
    CGPT_COPY_CASE(4)
    default:
      CGPT_COPY_CASE(8)
  }
#undef CGPT_COPY_CASE
  return static_cast<int>(hipGetLastError());
}
