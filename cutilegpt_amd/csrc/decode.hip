// Incremental (KV-cache) decoding kernels: the pieces a greedy generation
// step needs beyond the prefill kernels (the decode-shaped GEMM is in
// skinny.hip).
//
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

// ------------------------------------------------------- decode attention

constexpr int kDecThreads = 256;
constexpr int kDecChunk = 256;  // keys per softmax chunk
constexpr int kDecWaves = kDecThreads / 64;

// Barrier for LDS traffic only: the block's LDS writes are complete, its
// global stores (the cache append) may still be in flight.  __syncthreads()
// would also wait for those stores' write acknowledgements.
__device__ __forceinline__ void lds_barrier() {
  wait_lgkm0();
  raw_barrier();
}

template <typename T> __device__ __forceinline__ float round_to(float x);
template <> __device__ __forceinline__ float round_to<float>(float x) { return x; }
template <> __device__ __forceinline__ float round_to<bf16_t>(float x) { return bf16_to_f32(f32_to_bf16(x)); }

// The step's q, k and v for one decode-attention call: T rows (direct), or
// the fused QKV GEMM's split-K partial products plus its bias — columns
// q_off / k_off / v_off + h * hd of row b, P[s] at parts + s * part_stride —
// added in chunk order and rounded to T as the GEMM's own output would be.
template <typename T>
struct DecIn {
  const T* q;
  const T* kn;
  const T* vn;
  int64_t q_sb, q_sh, kn_sb, kn_sh, vn_sb, vn_sh;
  const float* parts;
  int n_parts;
  int64_t part_stride, ldp, q_off, k_off, v_off;
  const T* bias;
};

// One block per (batch, head), keys in chunks of kDecChunk.  Thread
// (kg, cv) = (tid / NV, tid % NV) owns 16-byte column vector cv of keys
// kg, kg + KG, ... of a chunk for both K and V, so a wave's loads cover whole
// cache rows; a chunk's K and V loads are all issued before the first is
// used, through buffer resources whose record count ends at row pos (rows at
// and past pos read as zero: the new row comes from registers, and nothing is
// read back from the cache rows this block writes).  Scores are dot products
// reduced across the NV lanes of a key; softmax runs online across chunks
// (one chunk for pos < kDecChunk), two barriers a chunk.  P is rounded to T
// before the P V product, as in the prefill kernel.
template <typename T, int NV, int MAXP>
__global__ __launch_bounds__(kDecThreads, NV <= 8 ? 4 : 1) void attn_decode_kernel(
    DecIn<T> in, T* __restrict__ kc, T* __restrict__ vc, T* __restrict__ o, int H, int Tmax,
    int pos_base, const int* __restrict__ pos_dev, int64_t c_sb, int64_t c_sh, int64_t c_st,
    int64_t o_sb, int64_t o_sh, float scale_log2, int* err_flag) {
  constexpr int EPV = Elem<T>::kVec;  // elements per 16-byte vector
  constexpr int HD = NV * EPV;
  constexpr int KG = kDecThreads / NV;   // key groups
  constexpr int KPT = kDecChunk / KG;    // keys of a chunk per thread
  constexpr int SPL = kDecChunk / 64;    // scores of a chunk per lane
  constexpr int R3 = (3 * HD + kDecThreads - 1) / kDecThreads;
  static_assert(KPT >= 1, "head_dim too large for the chunk");
  __shared__ float qs[HD], kns[HD], vns[HD];
  __shared__ float sc[kDecChunk], pb[kDecChunk];
  __shared__ float part[KG][HD];
  const int tid = threadIdx.x;
  const int kg = tid / NV, cv = tid % NV;
  const int b = blockIdx.x / H, h = blockIdx.x % H;
  int pos = pos_base + (pos_dev != nullptr ? *pos_dev : 0);
  if (pos < 0 || pos >= Tmax) {
    if (err_flag != nullptr && tid == 0) *err_flag = 1;
    pos = pos < 0 ? 0 : Tmax - 1;
  }
  const int Tk = pos + 1;
  T* kcb = kc + b * c_sb + h * c_sh;
  T* vcb = vc + b * c_sb + h * c_sh;
  const int row_bytes = static_cast<int>(c_st * sizeof(T));
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(kcb, 0, pos * row_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(vcb, 0, pos * row_bytes, 0x00020000);

  // The step's q / k / v values: thread tid + r * kDecThreads holds value i of
  // the 3 * HD (q | k | v).  Their loads, then chunk 0's K and V loads, are
  // all issued before the first is used.
  float sv[R3], bv[R3];
  float pv[R3][MAXP > 0 ? MAXP : 1];
  const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(in.parts), 0, MAXP > 0 ? static_cast<int>(in.n_parts * in.part_stride * 4) : 0,
      0x00020000);
#pragma unroll
  for (int r = 0; r < R3; ++r) {
    const int i = tid + r * kDecThreads;
    const int which = i < 3 * HD ? i / HD : 0, d = i % HD;
    if (MAXP == 0) {
      const T* src = which == 0 ? in.q + b * in.q_sb + h * in.q_sh
                   : which == 1 ? in.kn + b * in.kn_sb + h * in.kn_sh
                                : in.vn + b * in.vn_sb + h * in.vn_sh;
      sv[r] = Elem<T>::load(src + d);  // threads past 3 * HD load a valid element, unused
    } else {
      // Partials past n_parts (a uniform branch: no load issued) hold +0.
      const int64_t col = (which == 0 ? in.q_off : which == 1 ? in.k_off : in.v_off) + h * HD + d;
      const uint32_t off = static_cast<uint32_t>((b * in.ldp + col) * 4);
#pragma unroll
      for (int s = 0; s < MAXP; ++s)
        pv[r][s] = s < in.n_parts ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                                        rp, off + static_cast<uint32_t>(s * in.part_stride * 4), 0, 0))
                                  : 0.f;
      bv[r] = Elem<T>::load(in.bias + col);
    }
  }
  u32x4_t kr[KPT], vr[KPT];
  auto load_chunk = [&](int c0) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const uint32_t off = static_cast<uint32_t>((c0 + kg + KG * i) * row_bytes + cv * 16);
      kr[i] = __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0);
      vr[i] = __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0);
    }
  };
  // Keep the q / k / v loads ahead of the K and V loads: vmcnt retires in
  // issue order, so their sums then wait for them alone.
  __builtin_amdgcn_sched_barrier(0);
  load_chunk(0);
  if (MAXP > 0) {
#pragma unroll
    for (int r = 0; r < R3; ++r) {
      // Slots past n_parts hold +0: adding them leaves every sum but -0 as is.
      float t = pv[r][0];
#pragma unroll
      for (int s = 1; s < MAXP; ++s) t += pv[r][s];
      sv[r] = round_to<T>(t + bv[r]);
    }
  }
  // Publish q / k / v and append k, v at row pos of the cache.
#pragma unroll
  for (int r = 0; r < R3; ++r) {
    const int i = tid + r * kDecThreads, which = i / HD, d = i % HD;
    if (i < 3 * HD) {
      if (which == 0) {
        qs[d] = sv[r];
      } else if (which == 1) {
        kns[d] = sv[r];
        Elem<T>::store(kcb + pos * c_st + d, sv[r]);
      } else {
        vns[d] = sv[r];
        Elem<T>::store(vcb + pos * c_st + d, sv[r]);
      }
    }
  }
  lds_barrier();
  float qv[EPV];
#pragma unroll
  for (int e = 0; e < EPV; ++e) qv[e] = qs[cv * EPV + e];
  const int lane = tid & 63, wave = tid >> 6;
  // The new key's score, reduced by every wave (the cache rows loaded above
  // stop before row pos).
  float sp = 0.f;
  for (int d = lane; d < HD; d += 64) sp = fmaf(qs[d], kns[d], sp);
  sp = wave_sum(sp) * scale_log2;

  float mrun = -INFINITY, lsum = 0.f;
  float acc[EPV];
#pragma unroll
  for (int e = 0; e < EPV; ++e) acc[e] = 0.f;

  // Chunk c0 covers keys [c0, c0 + kDecChunk) of 0 .. pos; the last one
  // holds the new key pos.
  int c0 = 0;
  for (;; c0 += kDecChunk) {
    if (c0 > 0) load_chunk(c0);
    // Partial dot products of this lane's column vector, then summed over the
    // NV lanes of each key (consecutive lanes).
    float s[KPT];
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      float kv[EPV];
      unpack_vec<T>(kr[i], kv);
      float t = 0.f;
#pragma unroll
      for (int e = 0; e < EPV; ++e) t = fmaf(qv[e], kv[e], t);
      s[i] = t;
    }
    if constexpr (NV <= 16) {
#pragma unroll
      for (int i = 0; i < KPT; ++i) s[i] = group_sum<NV>(s[i]);
    } else {
#pragma unroll
      for (int off = 1; off < NV; off <<= 1)
#pragma unroll
        for (int i = 0; i < KPT; ++i) s[i] += __shfl_xor(s[i], off, 64);
    }
    if (cv == 0) {
#pragma unroll
      for (int i = 0; i < KPT; ++i) {
        const int j = kg + KG * i;
        sc[j] = c0 + j == pos ? sp : s[i] * scale_log2;
      }
    }
    lds_barrier();
    // Every wave reduces the whole chunk (SPL scores a lane), so the chunk's
    // maximum and sum need no further barrier; lane l of wave w < SPL also
    // owns key 64 w + l's probability for the P V product.
    float sj[SPL];
    float cm = -INFINITY;
#pragma unroll
    for (int k = 0; k < SPL; ++k) {
      sj[k] = c0 + lane + 64 * k < Tk ? sc[lane + 64 * k] : -INFINITY;
      cm = fmaxf(cm, sj[k]);
    }
    const float mnew = fmaxf(mrun, wave_max(cm));
    const float alpha = __builtin_amdgcn_exp2f(mrun - mnew);
    float ps = 0.f, pown = 0.f;
#pragma unroll
    for (int k = 0; k < SPL; ++k) {
      const float p = c0 + lane + 64 * k < Tk ? __builtin_amdgcn_exp2f(sj[k] - mnew) : 0.f;
      ps += p;
      if (k == wave) pown = p;
    }
    lsum = lsum * alpha + wave_sum(ps);
    mrun = mnew;
    if (tid < kDecChunk) pb[tid] = round_to<T>(pown);
    lds_barrier();
#pragma unroll
    for (int e = 0; e < EPV; ++e) acc[e] *= alpha;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      float vv[EPV];
      unpack_vec<T>(vr[i], vv);  // row pos reads as zero
      const float pj = pb[kg + KG * i];
#pragma unroll
      for (int e = 0; e < EPV; ++e) acc[e] = fmaf(pj, vv[e], acc[e]);
    }
    if (c0 + kDecChunk > pos) break;
    // The next chunk's first barrier comes after this chunk's last read of
    // pb and after every wave's reads of sc.
  }
  if (kg == 0) {
    // The new value row, weighted by its probability from the last chunk.
    const float pj = pb[pos - c0];
#pragma unroll
    for (int e = 0; e < EPV; ++e) acc[e] = fmaf(pj, vns[cv * EPV + e], acc[e]);
  }
#pragma unroll
  for (int e = 0; e < EPV; ++e) part[kg][cv * EPV + e] = acc[e];
  lds_barrier();
  for (int d = tid; d < HD; d += kDecThreads) {
    float t = 0.f;
    for (int k = 0; k < KG; ++k) t += part[k][d];
    Elem<T>::store(o + b * o_sb + h * o_sh + d, t / lsum);
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

// One block per row; 56 loads a thread cover 57 344 columns, so a GPT-2
// vocabulary row is read in one memory round trip (with 8 a thread it took
// seven dependent ones).
constexpr int kAmThreads = 1024;
constexpr int kAmUnroll = 56;

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

template <typename T, int MAXP>
static void launch_dec_nv(int nv, const DecIn<T>& in, T* kc, T* vc, T* o, int64_t BH, int H, int tm,
                          int pb, const int* pos_dev, int64_t c_sb, int64_t c_sh, int64_t c_st,
                          int64_t o_sb, int64_t o_sh, float sl2, int* err, hipStream_t s) {
#define CGPT_DEC_NV(N)                                                                              \
  case N:                                                                                           \
    hipLaunchKernelGGL((attn_decode_kernel<T, N, MAXP>), dim3(static_cast<unsigned>(BH)),           \
                       dim3(kDecThreads), 0, s, in, kc, vc, o, H, tm, pb, pos_dev, c_sb, c_sh, c_st, \
                       o_sb, o_sh, sl2, err);                                                       \
    break;
  switch (nv) {
    CGPT_DEC_NV(2)
    CGPT_DEC_NV(4)
    CGPT_DEC_NV(8)
    CGPT_DEC_NV(16)
    CGPT_DEC_NV(32)
    default:
      break;
  }
#undef CGPT_DEC_NV
}

// Checks shared by both decode-attention entry points; the q / k / v sources
// are checked by each.
static int check_decode(int64_t B, int64_t H, int64_t head_dim, int64_t t_max, int64_t pos_base,
                        const int* pos_dev, const void* k_cache, const void* v_cache, const void* o,
                        int64_t c_sb, int64_t c_sh, int64_t c_st, int dtype) {
  if (B < 0 || H <= 0 || head_dim <= 0 || t_max <= 0) return CGPT_EINVAL;
  if (!k_cache || !v_cache || !o) return CGPT_EINVAL;
  if (dtype != CGPT_F32 && dtype != CGPT_BF16) return CGPT_EDTYPE;
  const int64_t es = dtype == CGPT_F32 ? 4 : 2, epv = 16 / es;
  // head_dim = NV 16-byte vectors, NV a power of two from 2 to 32.
  const int64_t nv = head_dim / epv;
  if (head_dim % epv != 0 || nv < 2 || nv > 32 || (nv & (nv - 1)) != 0) return CGPT_ESHAPE;
  if (B * H > 0x7fffffff || t_max > 0x7fffffff) return CGPT_ESHAPE;
  // Cache rows are read as 16-byte vectors through 32-bit buffer offsets.
  if (c_st % epv != 0 || c_sh % epv != 0 || c_sb % epv != 0 || c_st < head_dim) return CGPT_EINVAL;
  if (t_max * c_st * es >= (int64_t{1} << 31)) return CGPT_ESHAPE;
  if ((reinterpret_cast<uintptr_t>(k_cache) & 15) || (reinterpret_cast<uintptr_t>(v_cache) & 15))
    return CGPT_EINVAL;
  if (pos_dev == nullptr && (pos_base < 0 || pos_base >= t_max)) return CGPT_EINVAL;
  return CGPT_OK;
}

template <typename T>
static int launch_decode(const DecIn<T>& in, int maxp, void* k_cache, void* v_cache, void* o,
                         int64_t B, int64_t H, int64_t head_dim, int64_t t_max, int64_t pos_base,
                         const int* pos_dev, int64_t c_sb, int64_t c_sh, int64_t c_st, int64_t o_sb,
                         int64_t o_sh, float scale, int* err_flag, void* stream) {
  const int nv = static_cast<int>(head_dim / Elem<T>::kVec);
  T* kc = static_cast<T*>(k_cache);
  T* vc = static_cast<T*>(v_cache);
  T* op = static_cast<T*>(o);
  const float sl2 = scale * 1.4426950408889634f;
  const int hh = static_cast<int>(H), tm = static_cast<int>(t_max), pb = static_cast<int>(pos_base);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t bh = B * H;
  if (maxp == 0)
    launch_dec_nv<T, 0>(nv, in, kc, vc, op, bh, hh, tm, pb, pos_dev, c_sb, c_sh, c_st, o_sb, o_sh, sl2, err_flag, s);
  else if (maxp <= 4)
    launch_dec_nv<T, 4>(nv, in, kc, vc, op, bh, hh, tm, pb, pos_dev, c_sb, c_sh, c_st, o_sb, o_sh, sl2, err_flag, s);
  else if (maxp <= 8)
    launch_dec_nv<T, 8>(nv, in, kc, vc, op, bh, hh, tm, pb, pos_dev, c_sb, c_sh, c_st, o_sb, o_sh, sl2, err_flag, s);
  else
    launch_dec_nv<T, 16>(nv, in, kc, vc, op, bh, hh, tm, pb, pos_dev, c_sb, c_sh, c_st, o_sb, o_sh, sl2, err_flag, s);
  return hip_status(hipGetLastError());
}

// ------------------------------------------- split-K partials + bias + GELU

// out[r][c..c+3] = act(P[0] + ... + P[n-1] + bias) for one 4-column group a
// thread: the n partial vectors are all loaded before the first is added
// (slots past n, skipped by a uniform branch, hold +0; adding +0 leaves every
// sum but -0 as is, and the sum starts from P[0]), fp32 additions in
// chunk order, then the bias, the activation and one rounding — the values
// the GEMM's own bias / GELU epilogue stores.
template <int MAXP, bool BIAS_BF16, bool GELU, typename TOut>
__global__ __launch_bounds__(256) void partials_bias_act_kernel(
    const float* __restrict__ P, int n_parts, int part_stride, int ldp, const void* __restrict__ bias,
    TOut* __restrict__ out, int64_t ldo, int rows, int cols) {
  const int groups = cols / 4;
  const int i = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
  if (i >= rows * groups) return;
  const int r = i / groups, c = (i - r * groups) * 4;
  const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(P), 0, n_parts * part_stride * 4, 0x00020000);
  const uint32_t off = static_cast<uint32_t>(r * ldp + c) * 4;
  u32x4_t pv[MAXP];
#pragma unroll
  for (int s = 0; s < MAXP; ++s)
    pv[s] = s < n_parts ? __builtin_amdgcn_raw_buffer_load_b128(
                              rp, off + static_cast<uint32_t>(s * part_stride) * 4, 0, 0)
                        : u32x4_t{0u, 0u, 0u, 0u};
  float b[4];
  if constexpr (BIAS_BF16) {
    const u32x2_t w = *reinterpret_cast<const u32x2_t*>(static_cast<const bf16_t*>(bias) + c);
    b[0] = __uint_as_float(w[0] << 16);
    b[1] = __uint_as_float(w[0] & 0xffff0000u);
    b[2] = __uint_as_float(w[1] << 16);
    b[3] = __uint_as_float(w[1] & 0xffff0000u);
  } else {
    const u32x4_t w = *reinterpret_cast<const u32x4_t*>(static_cast<const float*>(bias) + c);
#pragma unroll
    for (int e = 0; e < 4; ++e) b[e] = __uint_as_float(w[e]);
  }
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float t = __uint_as_float(pv[0][e]);
#pragma unroll
    for (int s = 1; s < MAXP; ++s) t += __uint_as_float(pv[s][e]);
    t += b[e];
    v[e] = GELU ? gelu_tanh(t) : t;
  }
  store4_out(out + static_cast<int64_t>(r) * ldo + c, v);
}

template <int MAXP, bool GELU>
static int launch_pba_maxp(const float* P, int n, int ps, int ldp, const void* bias, bool bias_bf16,
                           void* out, bool out_bf16, int64_t ldo, int rows, int cols,
                           hipStream_t s) {
  const int threads = rows * (cols / 4);
  const dim3 grid(static_cast<unsigned>((threads + 255) / 256));
#define CGPT_PBA(BB, TO)                                                                           \
  hipLaunchKernelGGL((partials_bias_act_kernel<MAXP, BB, GELU, TO>), grid, dim3(256), 0, s, P, n, \
                     ps, ldp, bias, static_cast<TO*>(out), ldo, rows, cols)
  if (bias_bf16) {
    if (out_bf16) CGPT_PBA(true, bf16_t); else CGPT_PBA(true, float);
  } else {
    if (out_bf16) CGPT_PBA(false, bf16_t); else CGPT_PBA(false, float);
  }
#undef CGPT_PBA
  return hip_status(hipGetLastError());
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
  const int st = check_decode(B, H, head_dim, t_max, pos_base, pos_dev, k_cache, v_cache, o, c_sb,
                              c_sh, c_st, dtype);
  if (st != CGPT_OK || B == 0) return st;
  if (!q || !k_new || !v_new) return CGPT_EINVAL;
  if (dtype == CGPT_BF16) {
    DecIn<bf16_t> in{static_cast<const bf16_t*>(q), static_cast<const bf16_t*>(k_new),
                     static_cast<const bf16_t*>(v_new), q_sb, q_sh, kn_sb, kn_sh, vn_sb, vn_sh,
                     nullptr, 0, 0, 0, 0, 0, 0, nullptr};
    return launch_decode(in, 0, k_cache, v_cache, o, B, H, head_dim, t_max, pos_base, pos_dev, c_sb,
                         c_sh, c_st, o_sb, o_sh, scale, err_flag, stream);
  }
  DecIn<float> in{static_cast<const float*>(q), static_cast<const float*>(k_new),
                  static_cast<const float*>(v_new), q_sb, q_sh, kn_sb, kn_sh, vn_sb, vn_sh,
                  nullptr, 0, 0, 0, 0, 0, 0, nullptr};
  return launch_decode(in, 0, k_cache, v_cache, o, B, H, head_dim, t_max, pos_base, pos_dev, c_sb,
                       c_sh, c_st, o_sb, o_sh, scale, err_flag, stream);
}

extern "C" int cgpt_attention_decode_partials(
    const float* qkv_partials, int64_t n_parts, int64_t part_stride, int64_t ldp,
    const void* qkv_bias, int64_t q_off, int64_t k_off, int64_t v_off, void* k_cache,
    void* v_cache, void* o, int64_t B, int64_t H, int64_t head_dim, int64_t t_max,
    int64_t pos_base, const int* pos_dev, int64_t c_sb, int64_t c_sh, int64_t c_st, int64_t o_sb,
    int64_t o_sh, float scale, int dtype, int* err_flag, void* stream) {
  const int st = check_decode(B, H, head_dim, t_max, pos_base, pos_dev, k_cache, v_cache, o, c_sb,
                              c_sh, c_st, dtype);
  if (st != CGPT_OK || B == 0) return st;
  if (!qkv_partials || !qkv_bias) return CGPT_EINVAL;
  if (n_parts < 1 || n_parts > 16 || q_off < 0 || k_off < 0 || v_off < 0) return CGPT_EINVAL;
  const int64_t width = H * head_dim;  // columns of q, of k and of v
  const int64_t hi = (q_off > k_off ? q_off : k_off) > v_off ? (q_off > k_off ? q_off : k_off) : v_off;
  if (ldp < hi + width || part_stride < (B - 1) * ldp + hi + width) return CGPT_EINVAL;
  if (n_parts * part_stride * 4 >= (int64_t{1} << 31)) return CGPT_ESHAPE;
  if (dtype == CGPT_BF16) {
    DecIn<bf16_t> in{nullptr, nullptr, nullptr, 0, 0, 0, 0, 0, 0, qkv_partials,
                     static_cast<int>(n_parts), part_stride, ldp, q_off, k_off, v_off,
                     static_cast<const bf16_t*>(qkv_bias)};
    return launch_decode(in, static_cast<int>(n_parts), k_cache, v_cache, o, B, H, head_dim, t_max,
                         pos_base, pos_dev, c_sb, c_sh, c_st, o_sb, o_sh, scale, err_flag, stream);
  }
  DecIn<float> in{nullptr, nullptr, nullptr, 0, 0, 0, 0, 0, 0, qkv_partials,
                  static_cast<int>(n_parts), part_stride, ldp, q_off, k_off, v_off,
                  static_cast<const float*>(qkv_bias)};
  return launch_decode(in, static_cast<int>(n_parts), k_cache, v_cache, o, B, H, head_dim, t_max,
                       pos_base, pos_dev, c_sb, c_sh, c_st, o_sb, o_sh, scale, err_flag, stream);
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

extern "C" int cgpt_partials_bias_act(const float* partials, int64_t n_parts, int64_t part_stride,
                                      int64_t ldp, const void* bias, int bias_dtype, void* out,
                                      int64_t ldo, int64_t rows, int64_t cols, int epilogue,
                                      int out_dtype, void* stream) {
  if (rows < 0 || cols < 0) return CGPT_EINVAL;
  if (rows == 0 || cols == 0) return CGPT_OK;
  if (partials == nullptr || bias == nullptr || out == nullptr) return CGPT_EINVAL;
  if (epilogue != CGPT_EPI_BIAS && epilogue != CGPT_EPI_BIAS_GELU) return CGPT_EINVAL;
  if ((bias_dtype != CGPT_F32 && bias_dtype != CGPT_BF16) ||
      (out_dtype != CGPT_F32 && out_dtype != CGPT_BF16))
    return CGPT_EDTYPE;
  if (n_parts < 1 || n_parts > 16 || cols % 4 != 0 || ldp < cols || ldp % 4 != 0 ||
      part_stride % 4 != 0 || part_stride < (rows - 1) * ldp + cols || ldo < cols || ldo % 4 != 0)
    return CGPT_EINVAL;
  const uintptr_t ba = bias_dtype == CGPT_F32 ? 15 : 7, oa = out_dtype == CGPT_F32 ? 15 : 7;
  if ((reinterpret_cast<uintptr_t>(partials) & 15) || (reinterpret_cast<uintptr_t>(bias) & ba) ||
      (reinterpret_cast<uintptr_t>(out) & oa))
    return CGPT_EINVAL;
  if (n_parts * part_stride * 4 >= (int64_t{1} << 31) || rows * (cols / 4) > 0x7fffffff)
    return CGPT_ESHAPE;
  const int n = static_cast<int>(n_parts), ps = static_cast<int>(part_stride);
  const int lp = static_cast<int>(ldp), r = static_cast<int>(rows), c = static_cast<int>(cols);
  const bool bb = bias_dtype == CGPT_BF16, ob = out_dtype == CGPT_BF16;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool gelu = epilogue == CGPT_EPI_BIAS_GELU;
  if (n <= 8)
    return gelu ? launch_pba_maxp<8, true>(partials, n, ps, lp, bias, bb, out, ob, ldo, r, c, s)
                : launch_pba_maxp<8, false>(partials, n, ps, lp, bias, bb, out, ob, ldo, r, c, s);
  return gelu ? launch_pba_maxp<16, true>(partials, n, ps, lp, bias, bb, out, ob, ldo, r, c, s)
              : launch_pba_maxp<16, false>(partials, n, ps, lp, bias, bb, out, ob, ldo, r, c, s);
}
