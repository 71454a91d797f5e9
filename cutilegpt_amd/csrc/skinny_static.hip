// cgpt_gemm_skinny_noalloc: the split-K skinny GEMM of cgpt_gemm_skinny with
// its workspace and block counters in a static device array instead of caller
// memory, for callers that cannot allocate (code under HIP graph capture,
// serving loops that forbid hipMalloc).
//
// `scratch` is one array per GPU, loaded with the code object.  In host code
// its name is only a stand-in for the device symbol: the device address is
// obtained once per device with hipGetSymbolAddress (with that device
// current) and only that address is ever handed to a kernel.  Calls on one
// GPU share the array: two calls that overlap in time on the same GPU (other
// streams, other threads) race on it.
#include <mutex>

#include "common.h"
#include "internal.h"

namespace cgpt {

// Capacity.  The skinny planner splits K only while it has fewer than 512
// column slices, with at most 16 chunks a slice, so slices * split < 1024 and
// the partial tiles of a call take at most 1023 * 4 m-tiles * 2 n-tiles * 256
// floats = 8 MiB - 8 KiB; counters: one per slice, at most 511.  The
// decode-form split is taken only when its chunk sums and counters fit the
// same capacity (else the other form runs).
constexpr int64_t kScratchWsBytes = kSkinnyMaxWsBytes;
constexpr int kScratchCounters = kSkinnyMaxCounters;
constexpr int64_t kScratchBytes = kScratchWsBytes + kScratchCounters * 4;

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the current device, looked up on the first
// call per device.
static int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e);
  if (dev < 0 || dev >= kMaxDevices) return CGPT_EINVAL;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_status(e);
    if (p == nullptr || (reinterpret_cast<uintptr_t>(p) & 255)) return CGPT_EINVAL;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return CGPT_OK;
}

// Counters start every call at zero (a fill kernel rather than a memset, so
// the call can be captured in a graph).
__global__ __launch_bounds__(1024) void zero_ints_kernel(int* p, int n) {
  const int i = static_cast<int>(blockIdx.x) * 1024 + static_cast<int>(threadIdx.x);
  if (i < n) p[i] = 0;
}

}  // namespace cgpt

extern "C" int cgpt_gemm_skinny_noalloc(const void* a, const void* w, const void* bias, void* c,
                                        int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldw,
                                        int64_t ldc, int in_dtype, int bias_dtype, int out_dtype,
                                        int epilogue, void* stream) {
  using namespace cgpt;
  int st = validate_gemm(a, w, bias, c, M, N, K, lda, ldw, ldc, in_dtype, bias_dtype, out_dtype,
                         epilogue);
  if (st != CGPT_OK || M == 0 || N == 0) return st;
  if (M > 64) return CGPT_ESHAPE;
  if (epilogue == CGPT_EPI_BIAS_RESID) return CGPT_EINVAL;  // not a skinny epilogue
  const bool bf16 = in_dtype == CGPT_BF16;
  int64_t ws_bytes = 0, n_counters = 0;
  st = skinny_workspace(static_cast<int>(M), static_cast<int>(N), static_cast<int>(K), bf16,
                        &ws_bytes, &n_counters);
  if (st != CGPT_OK) return st;
  if (ws_bytes > kScratchWsBytes || n_counters > kScratchCounters) return CGPT_ESCRATCH;
  void* base = nullptr;
  st = scratch_address(&base);
  if (st != CGPT_OK) return st;
  float* ws = static_cast<float*>(base);
  int* counters = reinterpret_cast<int*>(static_cast<uint8_t*>(base) + kScratchWsBytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (n_counters > 0) {
    hipLaunchKernelGGL(zero_ints_kernel, dim3(1), dim3(1024), 0, s, counters,
                       static_cast<int>(n_counters));
    st = hip_status(hipGetLastError());
    if (st != CGPT_OK) return st;
  }
  return launch_gemm_skinny(bf16, epilogue, a, w, bias, bias_dtype == CGPT_BF16, c,
                            out_dtype == CGPT_BF16, static_cast<int>(M), static_cast<int>(N),
                            static_cast<int>(K), lda, ldw, ldc, ws, kScratchWsBytes, counters,
                            kScratchCounters, s);
}
