// Incremental (KV-cache) decoding kernels: the pieces a greedy generation
// step needs beyond the prefill kernels.
//
//  * gemm_skinny_kernel — C[M,N] = epi(A W^T + bias) for M <= 64 (one row per
//    sequence in the batch).  Decode GEMMs are weight-streaming: every weight
//    byte is read once per step, so the kernel is built around HBM traffic,
//    not MFMA reuse: W rows go straight from global memory into MFMA fragments
//    (no LDS staging), several full cache lines per lane in flight, against
//    the (L2-resident) activation rows; K is split across the waves of a block
//    and, with a caller workspace, across blocks (deterministic fix-up by the
//    last block of each column slice).
//  * attn_decode_kernel — one block per (batch, head): appends the step's key
//    and value to the cache at position pos, then softmax(q K^T * scale) V
//    over cache rows 0..pos.  pos = pos_base + *pos_dev, read on the device so
//    one captured launch sequence serves every step.
//  * kv_store_kernel — copies a prefill's keys and values into the cache.
//  * argmax_kernel — greedy next token per row (first maximum, as argmax), also
//    recorded into a token history at column *step_dev.
#include "common.h"
#include "internal.h"

#include <limits.h>

namespace cgpt {

// --------------------------------------------------------------- skinny GEMM

constexpr int kSkWaves = 8;      // waves per block, splitting the block's K range
constexpr int kSkNT = 4;         // 16-column n-tiles per block (64 columns)
constexpr int kSkU = 2;          // double slabs in flight per wave
constexpr int kSkTargetBlocks = 512;
constexpr int kSkMaxSplit = 16;  // K chunks per column slice at most
constexpr int kCpolSc1 = 16;     // buffer cache-policy bits: sc1 (agent scope)

__device__ __forceinline__ float bias_value(const void* bias, bool bf16, int n) {
  return bf16 ? bf16_to_f32(static_cast<const bf16_t*>(bias)[n]) : static_cast<const float*>(bias)[n];
}

// Work split shared by the launcher and the workspace query: 64-column slices
// x `split` K chunks.
struct SkinnyPlan {
  int slices, dslabs, split, mt;
  int64_t ws_floats;  // per-block partial tiles, all blocks
};

static SkinnyPlan skinny_plan(int M, int N, int K, int elem_bytes, bool have_ws) {
  SkinnyPlan p;
  const int kd = 8 * (16 / elem_bytes);  // k per double slab
  p.mt = M <= 16 ? 1 : M <= 32 ? 2 : 4;
  p.slices = (N + 16 * kSkNT - 1) / (16 * kSkNT);
  p.dslabs = (K + kd - 1) / kd;
  int split = 1;
  if (have_ws) {
    // About kSkTargetBlocks blocks, but every wave of a block keeps at least
    // one double slab and at most kSkMaxSplit chunks per slice.
    split = (kSkTargetBlocks + p.slices - 1) / p.slices;
    int cap = p.dslabs / kSkWaves;
    cap = cap < kSkMaxSplit ? cap : kSkMaxSplit;
    split = split < cap ? split : cap;
    split = split > 1 ? split : 1;
  }
  p.split = split;
  p.ws_floats = split > 1 ? static_cast<int64_t>(p.slices) * split * p.mt * kSkNT * 64 * 4 : 0;
  return p;
}

// C[M,N] = epi(A W^T + bias) for M <= 16 * MT.  Block = 64 output columns
// (4 n-tiles) x one K chunk; its 8 waves split the chunk and stream W rows
// straight into MFMA fragments.  A "double slab" covers 2 * 4 * EPC k: lane
// group g loads 32 contiguous bytes of each row (k = 2g EPC .. 2g EPC + 2 EPC),
// so the 4 groups of a row read one full 128-byte line per load pair; the two
// 16-byte halves feed two MFMAs (any consistent assignment of k to MFMA slots
// gives the same sums, and A uses the same one).  Partial tiles are summed
// across waves through LDS in wave order; with split > 1 each block writes its
// sum to the workspace and the last block of a slice (counted on a device
// atomic) adds the split partials in chunk order, applies the epilogue and
// resets the counter — deterministic, and no clearing is needed between calls.
template <typename TIn, int MT, int EPI, typename TOut>
__global__ __launch_bounds__(64 * kSkWaves) void gemm_skinny_kernel(
    const TIn* __restrict__ A, const TIn* __restrict__ W, const void* __restrict__ bias,
    bool bias_bf16, TOut* __restrict__ C, int M, int N, int K, int64_t lda, int64_t ldw,
    int64_t ldc, bool vec_store, int split, int dslabs, float* __restrict__ ws,
    int* __restrict__ counters) {
  constexpr int EPC = 16 / sizeof(TIn);  // elements per 16-byte half
  constexpr int KD = 8 * EPC;            // k per double slab
  constexpr int U = kSkU;
  constexpr int NT = kSkNT;
  __shared__ f32x4_t red[kSkWaves][MT][NT][64];
  __shared__ int s_last;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nb = blockIdx.x / split, sk = blockIdx.x % split;
  const int n0 = nb * 16 * NT;
  const int r16 = lane & 15, g = lane >> 4;
  const int kl = g * 2 * EPC;  // this lane's first k inside a double slab
  // Rows past N / M are clamped (loaded, never stored).
  const TIn* wrow[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) wrow[j] = W + static_cast<int64_t>(min(n0 + 16 * j + r16, N - 1)) * ldw;
  const TIn* arow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) arow[mt] = A + static_cast<int64_t>(min(16 * mt + r16, M - 1)) * lda;

  const int per_blk = (dslabs + split - 1) / split;
  const int d0 = sk * per_blk, d1 = min(dslabs, d0 + per_blk);
  const int cnt = d1 > d0 ? d1 - d0 : 0;
  const int per_w = (cnt + kSkWaves - 1) / kSkWaves;
  const int w0 = d0 + wave * per_w, w1 = min(d1, w0 + per_w);

  f32x4_t acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[mt][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int d = w0; d < w1; d += U) {
    u32x4_t wf[U][NT][2], af[U][MT][2];
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        // Halves past K or past this wave's range load the row's first
        // chunk and are zeroed (K is a multiple of EPC).
        const int k = (d + u) * KD + kl + h * EPC;
        const bool ok = (d + u < w1) && (k < K);
        const int off = ok ? k : 0;
#pragma unroll
        for (int j = 0; j < NT; ++j) wf[u][j][h] = *reinterpret_cast<const u32x4_t*>(wrow[j] + off);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) af[u][mt][h] = *reinterpret_cast<const u32x4_t*>(arow[mt] + off);
        if (!ok) {
#pragma unroll
          for (int j = 0; j < NT; ++j) wf[u][j][h] = u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) af[u][mt][h] = u32x4_t{0u, 0u, 0u, 0u};
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int j = 0; j < NT; ++j) Mfma<TIn>::run(wf[u][j][h], af[u][mt][h], acc[mt][j]);
  }

#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < NT; ++j) red[wave][mt][j][lane] = acc[mt][j];
  __syncthreads();

  // One (m-tile, n-tile) pair per wave and pass: its sum over the waves.
  constexpr int kPairs = MT * NT;
  constexpr int kTile = kPairs * 64;  // f32x4 per block tile
  f32x4_t sum[(kPairs + kSkWaves - 1) / kSkWaves];
#pragma unroll
  for (int q = 0; q < (kPairs + kSkWaves - 1) / kSkWaves; ++q) {
    const int pr = wave + q * kSkWaves;
    if (pr < kPairs) {
      const int mt = pr / NT, j = pr % NT;
      f32x4_t t = red[0][mt][j][lane];
#pragma unroll
      for (int w = 1; w < kSkWaves; ++w) t += red[w][mt][j][lane];
      sum[q] = t;
    }
  }

  if (split > 1) {
    // Cross-block hand-off without cache-wide fences (an agent-scope fence
    // writes back and invalidates this XCD's whole L2): partials are stored
    // and loaded with agent-scope cache policy (sc1), which makes those
    // accesses coherent across the XCDs' L2s, the same encoding the memory
    // model uses for agent-scope atomic loads and stores.  The s_waitcnt
    // before the barrier completes every thread's partial stores before
    // thread 0 counts the block with a device atomic.
    const __amdgpu_buffer_rsrc_t rws = __builtin_amdgcn_make_buffer_rsrc(
        ws + static_cast<int64_t>(nb) * split * kTile * 4, 0, split * kTile * 16, 0x00020000);
#pragma unroll
    for (int q = 0; q < (kPairs + kSkWaves - 1) / kSkWaves; ++q) {
      const int pr = wave + q * kSkWaves;
      if (pr < kPairs)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, sum[q]), rws,
                                               (sk * kTile + pr * 64 + lane) * 16, 0, kCpolSc1);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
      s_last = __hip_atomic_fetch_add(&counters[nb], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               split - 1;
    __syncthreads();
    if (!s_last) return;
#pragma unroll
    for (int q = 0; q < (kPairs + kSkWaves - 1) / kSkWaves; ++q) {
      const int pr = wave + q * kSkWaves;
      if (pr < kPairs) {
        // All partials in flight at once, then summed in chunk order.
        u32x4_t part[kSkMaxSplit];
#pragma unroll
        for (int c = 0; c < kSkMaxSplit; ++c)
          if (c < split)
            part[c] = __builtin_amdgcn_raw_buffer_load_b128(rws, (c * kTile + pr * 64 + lane) * 16, 0,
                                                            kCpolSc1);
        f32x4_t t = __builtin_bit_cast(f32x4_t, part[0]);
#pragma unroll
        for (int c = 1; c < kSkMaxSplit; ++c)
          if (c < split) t += __builtin_bit_cast(f32x4_t, part[c]);
        sum[q] = t;
      }
    }
    if (threadIdx.x == 0)
      __hip_atomic_store(&counters[nb], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

#pragma unroll
  for (int q = 0; q < (kPairs + kSkWaves - 1) / kSkWaves; ++q) {
    const int pr = wave + q * kSkWaves;
    if (pr >= kPairs) continue;
    const int mt = pr / NT, j = pr % NT;
    const int m = 16 * mt + r16, n = n0 + 16 * j + 4 * g;
    float v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float x = sum[q][r];
      if (EPI != CGPT_EPI_NONE) x += n + r < N ? bias_value(bias, bias_bf16, n + r) : 0.f;
      if (EPI == CGPT_EPI_BIAS_GELU) x = gelu_tanh(x);
      v[r] = x;
    }
    if (m < M && n < N) {
      TOut* out = C + static_cast<int64_t>(m) * ldc + n;
      if (vec_store && n + 3 < N) {
        store4_out(out, v);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (n + r < N) Elem<TOut>::store(out + r, v[r]);
      }
    }
  }
}

template <typename TIn, int EPI, typename TOut>
static int launch_skinny_mt(const SkinnyPlan& p, const void* a, const void* w, const void* bias,
                            bool bias_bf16, void* c, int M, int N, int K, int64_t lda, int64_t ldw,
                            int64_t ldc, bool vec_store, float* ws, int* counters, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(p.slices * p.split)), block(64 * kSkWaves);
  const TIn* A = static_cast<const TIn*>(a);
  const TIn* W = static_cast<const TIn*>(w);
  TOut* C = static_cast<TOut*>(c);
  if (p.mt == 1)
    hipLaunchKernelGGL((gemm_skinny_kernel<TIn, 1, EPI, TOut>), grid, block, 0, s, A, W, bias,
                       bias_bf16, C, M, N, K, lda, ldw, ldc, vec_store, p.split, p.dslabs, ws, counters);
  else if (p.mt == 2)
    hipLaunchKernelGGL((gemm_skinny_kernel<TIn, 2, EPI, TOut>), grid, block, 0, s, A, W, bias,
                       bias_bf16, C, M, N, K, lda, ldw, ldc, vec_store, p.split, p.dslabs, ws, counters);
  else
    hipLaunchKernelGGL((gemm_skinny_kernel<TIn, 4, EPI, TOut>), grid, block, 0, s, A, W, bias,
                       bias_bf16, C, M, N, K, lda, ldw, ldc, vec_store, p.split, p.dslabs, ws, counters);
  return hip_status(hipGetLastError());
}

template <typename TIn, typename TOut>
static int launch_skinny_epi(const SkinnyPlan& p, int epi, const void* a, const void* w,
                             const void* bias, bool bias_bf16, void* c, int M, int N, int K,
                             int64_t lda, int64_t ldw, int64_t ldc, bool vec_store, float* ws,
                             int* counters, hipStream_t s) {
  switch (epi) {
    case CGPT_EPI_NONE:
      return launch_skinny_mt<TIn, CGPT_EPI_NONE, TOut>(p, a, w, bias, bias_bf16, c, M, N, K, lda, ldw, ldc, vec_store, ws, counters, s);
    case CGPT_EPI_BIAS:
      return launch_skinny_mt<TIn, CGPT_EPI_BIAS, TOut>(p, a, w, bias, bias_bf16, c, M, N, K, lda, ldw, ldc, vec_store, ws, counters, s);
    case CGPT_EPI_BIAS_GELU:
      return launch_skinny_mt<TIn, CGPT_EPI_BIAS_GELU, TOut>(p, a, w, bias, bias_bf16, c, M, N, K, lda, ldw, ldc, vec_store, ws, counters, s);
    default:
      return CGPT_EINVAL;
  }
}

int launch_gemm_skinny(bool bf16_in, int epilogue, const void* a, const void* w, const void* bias,
                       bool bias_bf16, void* c, bool out_bf16, int M, int N, int K, int64_t lda,
                       int64_t ldw, int64_t ldc, void* workspace, int64_t ws_bytes, int* counters,
                       int64_t n_counters, hipStream_t s) {
  if (M > 64) return CGPT_ESHAPE;
  SkinnyPlan p = skinny_plan(M, N, K, bf16_in ? 2 : 4, workspace != nullptr && counters != nullptr);
  if (p.split > 1 && (p.ws_floats * 4 > ws_bytes || p.slices > n_counters ||
                      (reinterpret_cast<uintptr_t>(workspace) & 15)))
    return CGPT_EINVAL;
  const uintptr_t oa = out_bf16 ? 7 : 15;
  const bool vec_store = ldc % 4 == 0 && (reinterpret_cast<uintptr_t>(c) & oa) == 0;
  float* ws = static_cast<float*>(workspace);
  if (bf16_in)
    return out_bf16 ? launch_skinny_epi<bf16_t, bf16_t>(p, epilogue, a, w, bias, bias_bf16, c, M, N, K, lda, ldw, ldc, vec_store, ws, counters, s)
                    : launch_skinny_epi<bf16_t, float>(p, epilogue, a, w, bias, bias_bf16, c, M, N, K, lda, ldw, ldc, vec_store, ws, counters, s);
  return out_bf16 ? launch_skinny_epi<float, bf16_t>(p, epilogue, a, w, bias, bias_bf16, c, M, N, K, lda, ldw, ldc, vec_store, ws, counters, s)
                  : launch_skinny_epi<float, float>(p, epilogue, a, w, bias, bias_bf16, c, M, N, K, lda, ldw, ldc, vec_store, ws, counters, s);
}

int skinny_workspace(int M, int N, int K, bool bf16_in, int64_t* ws_bytes, int64_t* n_counters) {
  const SkinnyPlan p = skinny_plan(M, N, K, bf16_in ? 2 : 4, true);
  *ws_bytes = p.ws_floats * 4;
  *n_counters = p.split > 1 ? p.slices : 0;
  return CGPT_OK;
}

// ------------------------------------------------------- decode attention

constexpr int kDecThreads = 256;
constexpr int kDecWaves = kDecThreads / 64;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Block-wide reduction of one value per thread (sum or max); `scr` holds
// kDecWaves floats.  Every thread returns the result.
template <bool kMax>
__device__ __forceinline__ float block_reduce(float v, float* scr) {
  v = kMax ? wave_max(v) : wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) scr[wave] = v;
  __syncthreads();
  float r = scr[0];
#pragma unroll
  for (int w = 1; w < kDecWaves; ++w) r = kMax ? fmaxf(r, scr[w]) : r + scr[w];
  return r;
}

template <typename T> __device__ __forceinline__ float round_to(float x);
template <> __device__ __forceinline__ float round_to<float>(float x) { return x; }
template <> __device__ __forceinline__ float round_to<bf16_t>(float x) { return bf16_to_f32(f32_to_bf16(x)); }

template <typename T>
__global__ __launch_bounds__(kDecThreads) void attn_decode_kernel(
    const T* __restrict__ q, const T* __restrict__ kn, const T* __restrict__ vn, T* __restrict__ kc,
    T* __restrict__ vc, T* __restrict__ o, int H, int hd, int Tmax, int pos_base,
    const int* __restrict__ pos_dev, int64_t q_sb, int64_t q_sh, int64_t kn_sb, int64_t kn_sh,
    int64_t vn_sb, int64_t vn_sh, int64_t c_sb, int64_t c_sh, int64_t c_st, int64_t o_sb,
    int64_t o_sh, float scale_log2, int* err_flag) {
  constexpr int EPV = Elem<T>::kVec;  // elements per 16-byte vector
  extern __shared__ float dsm[];
  float* qs = dsm;                     // hd
  float* sc = qs + hd;                 // Tmax scores, then probabilities
  float* part = sc + Tmax;             // kDecThreads * 8 partial outputs
  float* scr = part + kDecThreads * 8; // kDecWaves
  const int tid = threadIdx.x;
  const int b = blockIdx.x / H, h = blockIdx.x % H;
  int pos = pos_base + (pos_dev != nullptr ? *pos_dev : 0);
  if (pos < 0 || pos >= Tmax) {
    if (err_flag != nullptr && tid == 0) *err_flag = 1;
    pos = pos < 0 ? 0 : Tmax - 1;
  }
  const int Tk = pos + 1;
  T* kcb = kc + b * c_sb + h * c_sh;
  T* vcb = vc + b * c_sb + h * c_sh;
  const T* knb = kn + b * kn_sb + h * kn_sh;
  const T* vnb = vn + b * vn_sb + h * vn_sh;
  const T* qb = q + b * q_sb + h * q_sh;
  for (int d = tid; d < hd; d += kDecThreads) {
    kcb[pos * c_st + d] = knb[d];
    vcb[pos * c_st + d] = vnb[d];
    qs[d] = Elem<T>::load(qb + d);
  }
  __syncthreads();  // the appended row and q are visible to the whole block

  float mx = -INFINITY;
  for (int j = tid; j < Tk; j += kDecThreads) {
    const T* kr = kcb + j * c_st;
    float s = 0.f;
    for (int d = 0; d < hd; d += EPV) {
      float kv[EPV];
      load_vec(kr + d, kv);
#pragma unroll
      for (int e = 0; e < EPV; ++e) s = fmaf(qs[d + e], kv[e], s);
    }
    s *= scale_log2;
    sc[j] = s;
    mx = fmaxf(mx, s);
  }
  mx = block_reduce<true>(mx, scr);
  float sum = 0.f;
  for (int j = tid; j < Tk; j += kDecThreads) {
    const float p = __builtin_amdgcn_exp2f(sc[j] - mx);
    sc[j] = p;
    sum += p;
  }
  sum = block_reduce<false>(sum, scr);  // its barriers also publish sc

  // P V: key group kg = tid / TPR handles keys kg, kg + KG, ...; its TPR
  // threads each own EPV consecutive dims of the row (one 16-byte load per
  // key).  P is rounded to the storage type before the product, as in the
  // prefill kernel.  The KG group sums are then added through LDS.
  const int tpr = hd / EPV;            // threads per value row
  const int kgroups = kDecThreads / tpr;
  const int kg = tid / tpr, c0 = (tid % tpr) * EPV;
  float acc[EPV];
#pragma unroll
  for (int e = 0; e < EPV; ++e) acc[e] = 0.f;
  for (int j = kg; j < Tk; j += kgroups) {
    float vv[EPV];
    load_vec(vcb + j * c_st + c0, vv);
    const float p = round_to<T>(sc[j]);
#pragma unroll
    for (int e = 0; e < EPV; ++e) acc[e] = fmaf(p, vv[e], acc[e]);
  }
  // part holds kDecThreads * EPV floats: [group][dim]
#pragma unroll
  for (int e = 0; e < EPV; ++e) part[kg * hd + c0 + e] = acc[e];
  __syncthreads();
  if (tid < hd) {
    float t = 0.f;
    for (int k = 0; k < kgroups; ++k) t += part[k * hd + tid];
    Elem<T>::store(o + b * o_sb + h * o_sh + tid, t / sum);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void kv_store_kernel(
    const T* __restrict__ k, const T* __restrict__ v, T* __restrict__ kc, T* __restrict__ vc, int H,
    int Tn, int hd, int pos0, int64_t k_sb, int64_t k_sh, int64_t k_st, int64_t v_sb, int64_t v_sh,
    int64_t v_st, int64_t c_sb, int64_t c_sh, int64_t c_st, int64_t total_chunks) {
  constexpr int EPV = Elem<T>::kVec;
  const int cpr = hd / EPV;  // 16-byte chunks per row
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total_chunks;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int c = static_cast<int>(i % cpr);
    int64_t r = i / cpr;
    const int t = static_cast<int>(r % Tn);
    r /= Tn;
    const int h = static_cast<int>(r % H);
    const int64_t b = r / H;
    const int64_t dst = b * c_sb + h * c_sh + static_cast<int64_t>(pos0 + t) * c_st + c * EPV;
    *reinterpret_cast<u32x4_t*>(kc + dst) =
        *reinterpret_cast<const u32x4_t*>(k + b * k_sb + h * k_sh + t * k_st + c * EPV);
    *reinterpret_cast<u32x4_t*>(vc + dst) =
        *reinterpret_cast<const u32x4_t*>(v + b * v_sb + h * v_sh + t * v_st + c * EPV);
  }
}

// ------------------------------------------------------------------- argmax

constexpr int kAmThreads = 1024;
constexpr int kAmUnroll = 8;

template <typename T>
__global__ __launch_bounds__(kAmThreads) void argmax_kernel(const T* __restrict__ x, int64_t ld, int cols,
                                                            int64_t* __restrict__ ids, int64_t* __restrict__ hist,
                                                            int64_t hist_ld, const int* __restrict__ step_dev) {
  constexpr int NW = kAmThreads / 64;
  __shared__ float sv[NW];
  __shared__ int si[NW];
  const T* row = x + static_cast<int64_t>(blockIdx.x) * ld;
  float best = -INFINITY;
  int bi = INT_MAX;
  // kAmUnroll independent loads per thread in flight; each thread scans its
  // columns in ascending order, so the first maximum wins within a thread.
  for (int c0 = threadIdx.x; c0 < cols; c0 += kAmThreads * kAmUnroll) {
    float v[kAmUnroll];
#pragma unroll
    for (int u = 0; u < kAmUnroll; ++u) {
      const int c = c0 + u * kAmThreads;
      v[u] = c < cols ? Elem<T>::load(row + c) : -INFINITY;
    }
#pragma unroll
    for (int u = 0; u < kAmUnroll; ++u)
      if (v[u] > best) {
        best = v[u];
        bi = c0 + u * kAmThreads;
      }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(best, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    if (ov > best || (ov == best && oi < bi)) {
      best = ov;
      bi = oi;
    }
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = best;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < NW; ++w)
      if (sv[w] > best || (sv[w] == best && si[w] < bi)) {
        best = sv[w];
        bi = si[w];
      }
    if (bi == INT_MAX) bi = 0;  // a row of NaN or -inf only
    ids[blockIdx.x] = bi;
    if (hist != nullptr) hist[blockIdx.x * hist_ld + (step_dev != nullptr ? *step_dev : 0)] = bi;
  }
}

}  // namespace cgpt

using namespace cgpt;

extern "C" int cgpt_attention_decode(const void* q, const void* k_new, const void* v_new,
                                     void* k_cache, void* v_cache, void* o, int64_t B, int64_t H,
                                     int64_t head_dim, int64_t t_max, int64_t pos_base,
                                     const int* pos_dev, int64_t q_sb, int64_t q_sh,
                                     int64_t kn_sb, int64_t kn_sh, int64_t vn_sb, int64_t vn_sh,
                                     int64_t c_sb, int64_t c_sh, int64_t c_st, int64_t o_sb,
                                     int64_t o_sh, float scale, int dtype, int* err_flag,
                                     void* stream) {
  if (B < 0 || H <= 0 || head_dim <= 0 || t_max <= 0) return CGPT_EINVAL;
  if (B == 0) return CGPT_OK;
  if (!q || !k_new || !v_new || !k_cache || !v_cache || !o) return CGPT_EINVAL;
  if (dtype != CGPT_F32 && dtype != CGPT_BF16) return CGPT_EDTYPE;
  const int epv = dtype == CGPT_F32 ? 4 : 8;
  if (head_dim > kDecThreads || kDecThreads % head_dim != 0 || head_dim % epv != 0) return CGPT_ESHAPE;
  if (t_max > 8192 || B * H > 0x7fffffff) return CGPT_ESHAPE;  // dynamic LDS <= 64 KiB
  // Cache rows are read as 16-byte vectors.
  if (c_st % epv != 0 || c_sh % epv != 0 || c_sb % epv != 0 || c_st < head_dim) return CGPT_EINVAL;
  if ((reinterpret_cast<uintptr_t>(k_cache) & 15) || (reinterpret_cast<uintptr_t>(v_cache) & 15))
    return CGPT_EINVAL;
  if (pos_dev == nullptr && (pos_base < 0 || pos_base >= t_max)) return CGPT_EINVAL;
  const size_t smem = (static_cast<size_t>(head_dim) + t_max + kDecThreads * 8 + kDecWaves) * sizeof(float);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const float sl2 = scale * 1.4426950408889634f;
  const int hh = static_cast<int>(H), hd = static_cast<int>(head_dim), tm = static_cast<int>(t_max);
  const int pb = static_cast<int>(pos_base);
  if (dtype == CGPT_BF16)
    hipLaunchKernelGGL(attn_decode_kernel<bf16_t>, dim3(static_cast<unsigned>(B * H)), dim3(kDecThreads),
                       smem, s, static_cast<const bf16_t*>(q), static_cast<const bf16_t*>(k_new),
                       static_cast<const bf16_t*>(v_new), static_cast<bf16_t*>(k_cache),
                       static_cast<bf16_t*>(v_cache), static_cast<bf16_t*>(o), hh, hd, tm, pb, pos_dev,
                       q_sb, q_sh, kn_sb, kn_sh, vn_sb, vn_sh, c_sb, c_sh, c_st, o_sb, o_sh, sl2, err_flag);
  else
    hipLaunchKernelGGL(attn_decode_kernel<float>, dim3(static_cast<unsigned>(B * H)), dim3(kDecThreads),
                       smem, s, static_cast<const float*>(q), static_cast<const float*>(k_new),
                       static_cast<const float*>(v_new), static_cast<float*>(k_cache),
                       static_cast<float*>(v_cache), static_cast<float*>(o), hh, hd, tm, pb, pos_dev,
                       q_sb, q_sh, kn_sb, kn_sh, vn_sb, vn_sh, c_sb, c_sh, c_st, o_sb, o_sh, sl2, err_flag);
  return hip_status(hipGetLastError());
}

extern "C" int cgpt_kv_store(const void* k, const void* v, void* k_cache, void* v_cache, int64_t B,
                             int64_t H, int64_t T, int64_t head_dim, int64_t pos0, int64_t t_max,
                             int64_t k_sb, int64_t k_sh, int64_t k_st, int64_t v_sb, int64_t v_sh,
                             int64_t v_st, int64_t c_sb, int64_t c_sh, int64_t c_st, int dtype,
                             void* stream) {
  if (B < 0 || H <= 0 || T < 0 || head_dim <= 0 || pos0 < 0) return CGPT_EINVAL;
  if (B == 0 || T == 0) return CGPT_OK;
  if (!k || !v || !k_cache || !v_cache) return CGPT_EINVAL;
  if (pos0 + T > t_max) return CGPT_ESHAPE;
  if (dtype != CGPT_F32 && dtype != CGPT_BF16) return CGPT_EDTYPE;
  const int epv = dtype == CGPT_F32 ? 4 : 8;
  if (head_dim % epv != 0) return CGPT_ESHAPE;
  for (int64_t st : {k_sb, k_sh, k_st, v_sb, v_sh, v_st, c_sb, c_sh, c_st})
    if (st % epv != 0) return CGPT_EINVAL;
  for (const void* p : {k, v, static_cast<const void*>(k_cache), static_cast<const void*>(v_cache)})
    if (reinterpret_cast<uintptr_t>(p) & 15) return CGPT_EINVAL;
  const int64_t chunks = B * H * T * (head_dim / epv);
  const int64_t want = (chunks + 255) / 256;
  const unsigned grid = static_cast<unsigned>(want < 4096 ? want : 4096);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int hh = static_cast<int>(H), tt = static_cast<int>(T), hd = static_cast<int>(head_dim);
  const int p0 = static_cast<int>(pos0);
  if (dtype == CGPT_BF16)
    hipLaunchKernelGGL(kv_store_kernel<bf16_t>, dim3(grid), dim3(256), 0, s, static_cast<const bf16_t*>(k),
                       static_cast<const bf16_t*>(v), static_cast<bf16_t*>(k_cache),
                       static_cast<bf16_t*>(v_cache), hh, tt, hd, p0, k_sb, k_sh, k_st, v_sb, v_sh, v_st,
                       c_sb, c_sh, c_st, chunks);
  else
    hipLaunchKernelGGL(kv_store_kernel<float>, dim3(grid), dim3(256), 0, s, static_cast<const float*>(k),
                       static_cast<const float*>(v), static_cast<float*>(k_cache),
                       static_cast<float*>(v_cache), hh, tt, hd, p0, k_sb, k_sh, k_st, v_sb, v_sh, v_st,
                       c_sb, c_sh, c_st, chunks);
  return hip_status(hipGetLastError());
}

extern "C" int cgpt_argmax(const void* x, int64_t rows, int64_t cols, int64_t ld, int dtype,
                           int64_t* ids, int64_t* hist, int64_t hist_ld, const int* step_dev,
                           void* stream) {
  if (rows < 0 || cols <= 0 || ld < cols) return CGPT_EINVAL;
  if (rows == 0) return CGPT_OK;
  if (!x || !ids || (hist != nullptr && hist_ld <= 0)) return CGPT_EINVAL;
  if (rows > 0x7fffffff || cols > 0x7fffffff) return CGPT_ESHAPE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int c = static_cast<int>(cols);
  if (dtype == CGPT_F32)
    hipLaunchKernelGGL(argmax_kernel<float>, dim3(static_cast<unsigned>(rows)), dim3(kAmThreads), 0, s,
                       static_cast<const float*>(x), ld, c, ids, hist, hist_ld, step_dev);
  else if (dtype == CGPT_BF16)
    hipLaunchKernelGGL(argmax_kernel<bf16_t>, dim3(static_cast<unsigned>(rows)), dim3(kAmThreads), 0, s,
                       static_cast<const bf16_t*>(x), ld, c, ids, hist, hist_ld, step_dev);
  else
    return CGPT_EDTYPE;
  return hip_status(hipGetLastError());
}
