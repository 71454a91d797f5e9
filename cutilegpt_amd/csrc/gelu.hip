// Standalone element-wise tanh-GELU (HBM-bound streaming kernel).
//
// A block owns kGeluThreads * gelu_unroll<T>() consecutive 16-byte vectors;
// each thread issues its loads before any arithmetic, then converts and
// stores.  Loads and stores go through a buffer
// resource that starts at the block's first vector and ends at the tensor's
// last, so the final block's lanes past the end read zeros and their stores
// are dropped — no branch.  Arithmetic is fp32 whatever the storage type.
#include "common.h"

namespace cgpt {

constexpr int kGeluThreads = 256;
// 16-byte vectors per thread: 16 fp32 or 8 bf16 / fp16 elements (the fastest of 1, 2,
// 4 and 8 per type in a sweep over rotating buffers larger than the MALL).
template <typename T> constexpr int gelu_unroll() { return sizeof(T) == 4 ? 4 : 1; }
// Buffer-access cache policy: non-temporal (streamed once, marked for early
// eviction), +10-15 % over cached accesses in the same sweep.
constexpr int kStreamPolicy = 2;

template <typename T>
__device__ __forceinline__ u32x4_t gelu_vec16(const u32x4_t& raw) {
  constexpr int V = Elem<T>::kVec;
  float v[V];
  unpack_vec<T>(raw, v);
#pragma unroll
  for (int j = 0; j < V; ++j) v[j] = gelu_tanh(v[j]);
  u32x4_t out;
  if constexpr (V == 4) {
#pragma unroll
    for (int j = 0; j < 4; ++j) out[j] = __float_as_uint(v[j]);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) out[j] = pack2<T>(v[2 * j], v[2 * j + 1]);
  }
  return out;
}

template <typename T>
__global__ __launch_bounds__(kGeluThreads) void gelu_vec_kernel(const T* x,
                                                                T* y,
                                                                int64_t nvec) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int V = Elem<T>::kVec;
  constexpr int U = gelu_unroll<T>();
  constexpr int PER_BLOCK = kGeluThreads * U;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * PER_BLOCK;
  const int64_t left = nvec - first;
  const int bytes = static_cast<int>((left < PER_BLOCK ? left : PER_BLOCK) * 16);
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<T*>(x + first * V), 0, bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc(y + first * V, 0, bytes,
                                                                      0x00020000);
  u32x4_t raw[U];
#pragma unroll
  for (int u = 0; u < U; ++u)
    raw[u] = __builtin_amdgcn_raw_buffer_load_b128(rx, (u * kGeluThreads + threadIdx.x) * 16, 0,
                                                   kStreamPolicy);
#pragma unroll
  for (int u = 0; u < U; ++u)
    __builtin_amdgcn_raw_buffer_store_b128(gelu_vec16<T>(raw[u]), ry,
                                           (u * kGeluThreads + threadIdx.x) * 16, 0, kStreamPolicy);
#endif
}

// Scalar path for the ragged tail (and for unaligned tensors).
template <typename T>
__global__ __launch_bounds__(kGeluThreads) void gelu_scalar_kernel(const T* x,
                                                                   T* y,
                                                                   int64_t begin, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kGeluThreads;
  for (int64_t i = begin + static_cast<int64_t>(blockIdx.x) * kGeluThreads + threadIdx.x; i < n;
       i += stride)
    Elem<T>::store(y + i, gelu_tanh(Elem<T>::load(x + i)));
}

template <typename T>
static int launch_gelu(const void* xv, void* yv, int64_t n, hipStream_t stream) {
  const T* x = static_cast<const T*>(xv);
  T* y = static_cast<T*>(yv);
  constexpr int V = Elem<T>::kVec;
  const bool aligned = (reinterpret_cast<uintptr_t>(x) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(y) % 16 == 0);
  int64_t nvec = aligned ? n / V : 0;
  if (nvec > 0) {
    const int64_t per_block = kGeluThreads * gelu_unroll<T>();
    const int64_t blocks = (nvec + per_block - 1) / per_block;
    if (blocks > 0x7fffffff) return CGPT_ESHAPE;
    hipLaunchKernelGGL(gelu_vec_kernel<T>, dim3(static_cast<unsigned>(blocks)),
                       dim3(kGeluThreads), 0, stream, x, y, nvec);
  }
  const int64_t done = nvec * V;
  if (done < n) {
    int64_t rem = n - done;
    int64_t blocks = (rem + kGeluThreads - 1) / kGeluThreads;
    if (blocks > 2048) blocks = 2048;
    hipLaunchKernelGGL(gelu_scalar_kernel<T>, dim3(static_cast<unsigned>(blocks)),
                       dim3(kGeluThreads), 0, stream, x, y, done, n);
  }
  return hip_status(hipGetLastError());
}

}  // namespace cgpt

extern "C" int cgpt_gelu(const void* x, void* y, int64_t n, int dtype, void* stream) {
  using namespace cgpt;
  if (n < 0 || (n > 0 && (x == nullptr || y == nullptr))) return CGPT_EINVAL;
  if (n == 0) return CGPT_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == CGPT_F32) return launch_gelu<float>(x, y, n, s);
  if (dtype == CGPT_BF16) return launch_gelu<bf16_t>(x, y, n, s);
  if (dtype == CGPT_F16) return launch_gelu<f16_t>(x, y, n, s);
  return CGPT_EDTYPE;
}
