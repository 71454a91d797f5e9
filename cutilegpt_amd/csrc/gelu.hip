// Standalone element-wise tanh-GELU (HBM-bound streaming kernel).
//
// Each thread moves UNROLL 16-byte vectors per iteration and issues all of
// its loads before any arithmetic, so every wave keeps UNROLL dwordx4 loads in
// flight; the grid is sized to a few waves per CU and grid-strides over the
// tensor.  Arithmetic is fp32 whatever the storage type.
#include "common.h"

namespace cgpt {

constexpr int kGeluThreads = 256;
constexpr int kGeluUnroll = 4;

template <typename T>
__global__ __launch_bounds__(kGeluThreads) void gelu_vec_kernel(const T* __restrict__ x,
                                                                T* __restrict__ y,
                                                                int64_t nvec) {
  constexpr int V = Elem<T>::kVec;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kGeluThreads;
  int64_t i = static_cast<int64_t>(blockIdx.x) * kGeluThreads + threadIdx.x;
  for (; i + (kGeluUnroll - 1) * stride < nvec; i += kGeluUnroll * stride) {
    float v[kGeluUnroll][V];
#pragma unroll
    for (int u = 0; u < kGeluUnroll; ++u) load_vec(x + (i + u * stride) * V, v[u]);
#pragma unroll
    for (int u = 0; u < kGeluUnroll; ++u) {
#pragma unroll
      for (int j = 0; j < V; ++j) v[u][j] = gelu_tanh(v[u][j]);
      store_vec(y + (i + u * stride) * V, v[u]);
    }
  }
  for (; i < nvec; i += stride) {
    float v[V];
    load_vec(x + i * V, v);
#pragma unroll
    for (int j = 0; j < V; ++j) v[j] = gelu_tanh(v[j]);
    store_vec(y + i * V, v);
  }
}

// Scalar path for the ragged tail (and for unaligned tensors).
template <typename T>
__global__ __launch_bounds__(kGeluThreads) void gelu_scalar_kernel(const T* __restrict__ x,
                                                                   T* __restrict__ y,
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
    // 256 CUs x 8 blocks of 256 threads keeps every SIMD busy; more blocks only
    // add scheduling overhead for a streaming kernel.
    int64_t blocks = (nvec + kGeluThreads - 1) / kGeluThreads;
    if (blocks > 2048) blocks = 2048;
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
  return CGPT_EDTYPE;
}
