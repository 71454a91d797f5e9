// Token + position embedding gather (HBM-bound, one wavefront per token).
//
// out[i, :] = wte[idx[i], :] (+ wpe[pos0 + i % T, :], or wpe[pos0 + *pos_dev, :]
// for every token when the position comes from device memory, as in a decode
// step replayed from one captured launch sequence); lane l of the wave moves
// columns [4(64c + l), 4(64c + l) + 4) for each 256-column chunk c, so each row
// is read and written with contiguous, fully coalesced spans.  Out-of-range
// ids/positions are clamped (no out-of-bounds read is possible) and reported
// through an optional device flag.  Widths that are not a multiple of 4, or
// rows without 4-element vector alignment, move one element a lane per step.
#include "common.h"

namespace cgpt {

constexpr int kEmbThreads = 256;
constexpr int kEmbTokensPerBlock = kEmbThreads / 64;

__device__ __forceinline__ void ld4(const float* p, float* v) { load_vec(p, v); }
__device__ __forceinline__ void ld4(const bf16_t* p, float* v) {
  u32x2_t u = *reinterpret_cast<const u32x2_t*>(p);
  v[0] = __uint_as_float(u[0] << 16);
  v[1] = __uint_as_float(u[0] & 0xffff0000u);
  v[2] = __uint_as_float(u[1] << 16);
  v[3] = __uint_as_float(u[1] & 0xffff0000u);
}
__device__ __forceinline__ void ld4(const f16_t* p, float* v) {
  u32x2_t u = *reinterpret_cast<const u32x2_t*>(p);
  v[0] = f16_lo(u[0]);
  v[1] = f16_hi(u[0]);
  v[2] = f16_lo(u[1]);
  v[3] = f16_hi(u[1]);
}
__device__ __forceinline__ void st4(f16_t* p, const float* v) {
  u32x2_t u = {pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3])};
  *reinterpret_cast<u32x2_t*>(p) = u;
}
__device__ __forceinline__ void st4(float* p, const float* v) { store_vec(p, v); }
__device__ __forceinline__ void st4(bf16_t* p, const float* v) {
  u32x2_t u = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  *reinterpret_cast<u32x2_t*>(p) = u;
}

template <typename TW, typename TO, bool VEC>
__global__ __launch_bounds__(kEmbThreads) void embedding_kernel(
    const int64_t* __restrict__ idx, const TW* __restrict__ wte, const TW* __restrict__ wpe,
    TO* __restrict__ out, int64_t n_tokens, int64_t T, int D, int64_t vocab, int64_t pos0,
    const int* __restrict__ pos_dev, int64_t n_pos, int* err_flag) {
  const int lane = threadIdx.x & 63;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kEmbTokensPerBlock + (threadIdx.x >> 6);
  if (i >= n_tokens) return;
  int64_t id = idx[i];
  bool bad = false;
  if (id < 0 || id >= vocab) {
    bad = true;
    id = id < 0 ? 0 : vocab - 1;
  }
  int64_t pos = pos0 + (pos_dev != nullptr ? static_cast<int64_t>(*pos_dev) : i % T);
  if (wpe != nullptr && (pos < 0 || pos >= n_pos)) {
    bad = true;
    pos = pos < 0 ? 0 : n_pos - 1;
  }
  if (bad && err_flag != nullptr && lane == 0) *err_flag = 1;
  const TW* trow = wte + id * D;
  const TW* prow = wpe != nullptr ? wpe + pos * D : nullptr;
  TO* orow = out + i * D;
  if constexpr (!VEC) {
    for (int col = lane; col < D; col += 64) {
      float v = Elem<TW>::load(trow + col);
      if (prow != nullptr) v += Elem<TW>::load(prow + col);
      Elem<TO>::store(orow + col, v);
    }
    return;
  }
  for (int col = lane * 4; col < D; col += 256) {
    float v[4];
    ld4(trow + col, v);
    if (prow != nullptr) {
      float p[4];
      ld4(prow + col, p);
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] += p[j];
    }
    st4(orow + col, v);
  }
}

template <typename TW, typename TO>
static int launch_emb(const int64_t* idx, const void* wte, const void* wpe, void* out,
                      int64_t n_tokens, int64_t T, int D, int64_t vocab, int64_t pos0,
                      const int* pos_dev, int64_t n_pos, int* err, bool vec, hipStream_t s) {
  const int64_t blocks = (n_tokens + kEmbTokensPerBlock - 1) / kEmbTokensPerBlock;
  if (blocks > 0x7fffffff) return CGPT_ESHAPE;
  const dim3 grid(static_cast<unsigned>(blocks));
  if (vec)
    hipLaunchKernelGGL((embedding_kernel<TW, TO, true>), grid, dim3(kEmbThreads), 0, s, idx,
                       static_cast<const TW*>(wte), static_cast<const TW*>(wpe),
                       static_cast<TO*>(out), n_tokens, T, D, vocab, pos0, pos_dev, n_pos, err);
  else
    hipLaunchKernelGGL((embedding_kernel<TW, TO, false>), grid, dim3(kEmbThreads), 0, s, idx,
                       static_cast<const TW*>(wte), static_cast<const TW*>(wpe),
                       static_cast<TO*>(out), n_tokens, T, D, vocab, pos0, pos_dev, n_pos, err);
  return hip_status(hipGetLastError());
}

}  // namespace cgpt

static int embedding_impl(const int64_t* idx, const void* wte, const void* wpe, void* out,
                          int64_t n_tokens, int64_t T, int64_t D, int64_t vocab, int64_t pos0,
                          const int* pos_dev, int64_t n_pos, int w_dtype, int out_dtype,
                          int* err_flag, void* stream) {
  using namespace cgpt;
  if (n_tokens < 0 || D <= 0 || vocab <= 0) return CGPT_EINVAL;
  if (n_tokens == 0) return CGPT_OK;
  if (idx == nullptr || wte == nullptr || out == nullptr || T <= 0) return CGPT_EINVAL;
  if (wpe != nullptr && n_pos <= 0) return CGPT_EINVAL;
  if (D > 0x7fffffff / 4) return CGPT_ESHAPE;
  // fp32 / bf16 weights take fp32 or bf16 outputs, fp16 weights fp32 or fp16.
  const bool wf16 = w_dtype == CGPT_F16;
  if (w_dtype != CGPT_F32 && w_dtype != CGPT_BF16 && !wf16) return CGPT_EDTYPE;
  if (out_dtype != CGPT_F32 && out_dtype != (wf16 ? CGPT_F16 : CGPT_BF16)) return CGPT_EDTYPE;
  const uintptr_t we = (w_dtype == CGPT_F32) ? 3 : 1, oe = (out_dtype == CGPT_F32) ? 3 : 1;
  if ((reinterpret_cast<uintptr_t>(wte) & we) || (reinterpret_cast<uintptr_t>(wpe) & we) ||
      (reinterpret_cast<uintptr_t>(out) & oe) || (reinterpret_cast<uintptr_t>(idx) & 7))
    return CGPT_EINVAL;
  // Four-element vectors: D % 4 == 0 and 16-byte (fp32) / 8-byte (16-bit)
  // aligned rows.
  const uintptr_t wa = (w_dtype == CGPT_F32) ? 15 : 7, oa = (out_dtype == CGPT_F32) ? 15 : 7;
  const bool vec = D % 4 == 0 && !(reinterpret_cast<uintptr_t>(wte) & wa) &&
                   !(reinterpret_cast<uintptr_t>(wpe) & wa) && !(reinterpret_cast<uintptr_t>(out) & oa);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int d = static_cast<int>(D);
#define CGPT_EMB(TW, TO) \
  launch_emb<TW, TO>(idx, wte, wpe, out, n_tokens, T, d, vocab, pos0, pos_dev, n_pos, err_flag, vec, s)
  if (w_dtype == CGPT_F32) return out_dtype == CGPT_F32 ? CGPT_EMB(float, float) : CGPT_EMB(float, bf16_t);
  if (w_dtype == CGPT_BF16) return out_dtype == CGPT_F32 ? CGPT_EMB(bf16_t, float) : CGPT_EMB(bf16_t, bf16_t);
  return out_dtype == CGPT_F32 ? CGPT_EMB(f16_t, float) : CGPT_EMB(f16_t, f16_t);
#undef CGPT_EMB
}

extern "C" int cgpt_embedding(const int64_t* idx, const void* wte, const void* wpe, void* out,
                              int64_t n_tokens, int64_t T, int64_t D, int64_t vocab,
                              int64_t pos0, int64_t n_pos, int w_dtype, int out_dtype,
                              int* err_flag, void* stream) {
  return embedding_impl(idx, wte, wpe, out, n_tokens, T, D, vocab, pos0, nullptr, n_pos, w_dtype,
                        out_dtype, err_flag, stream);
}

extern "C" int cgpt_embedding_at(const int64_t* idx, const void* wte, const void* wpe, void* out,
                                 int64_t n_tokens, int64_t D, int64_t vocab, int64_t pos_base,
                                 const int* pos_dev, int64_t n_pos, int w_dtype, int out_dtype,
                                 int* err_flag, void* stream) {
  if (pos_dev == nullptr) return CGPT_EINVAL;
  return embedding_impl(idx, wte, wpe, out, n_tokens, 1, D, vocab, pos_base, pos_dev, n_pos,
                        w_dtype, out_dtype, err_flag, stream);
}
