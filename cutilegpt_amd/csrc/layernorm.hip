// Fused residual add + LayerNorm (HBM-bound, rows held in registers).
//
// A 256-thread block is 4 waves; a wave normalises R consecutive rows.  Lane l
// owns columns [4(64c + l), 4(64c + l) + 4) of each row for chunk c <
// ceil(cols / 256), so every load and store of a wave covers one contiguous
// 1 KiB (fp32) or 512 B (bf16) span.  Whole rows stay in registers: mean and
// the centred variance are two wave reductions over the registers (no second
// read of x), the residual sum is written once (x_out) and the normalised row
// once (y).
#include <type_traits>

#include "common.h"

namespace cgpt {

constexpr int kLnThreads = 256;
constexpr int kLnRowsPerBlock = kLnThreads / 64;

__device__ __forceinline__ void load4(const float* p, float* v) { load_vec(p, v); }
__device__ __forceinline__ void load4(const bf16_t* p, float* v) {
  u32x2_t u = *reinterpret_cast<const u32x2_t*>(p);
  v[0] = __uint_as_float(u[0] << 16);
  v[1] = __uint_as_float(u[0] & 0xffff0000u);
  v[2] = __uint_as_float(u[1] << 16);
  v[3] = __uint_as_float(u[1] & 0xffff0000u);
}
__device__ __forceinline__ void store4(float* p, const float* v) { store_vec(p, v); }
__device__ __forceinline__ void store4(bf16_t* p, const float* v) {
  u32x2_t u = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  *reinterpret_cast<u32x2_t*>(p) = u;
}

// The same four elements through non-temporal (streaming) accesses: the
// lines are marked for early eviction instead of being kept for reuse.
__device__ __forceinline__ void load4_nt(const float* p, float* v) {
  const f32x4_t t = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(p));
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = t[j];
}
__device__ __forceinline__ void load4_nt(const bf16_t* p, float* v) {
  const u32x2_t u = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
  v[0] = __uint_as_float(u[0] << 16);
  v[1] = __uint_as_float(u[0] & 0xffff0000u);
  v[2] = __uint_as_float(u[1] << 16);
  v[3] = __uint_as_float(u[1] & 0xffff0000u);
}
__device__ __forceinline__ void store4_nt(float* p, const float* v) {
  __builtin_nontemporal_store(f32x4_t{v[0], v[1], v[2], v[3]}, reinterpret_cast<f32x4_t*>(p));
}
__device__ __forceinline__ void store4_nt(bf16_t* p, const float* v) {
  __builtin_nontemporal_store(u32x2_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])},
                              reinterpret_cast<u32x2_t*>(p));
}
__device__ __forceinline__ void load4(const f16_t* p, float* v) {
  const u32x2_t u = *reinterpret_cast<const u32x2_t*>(p);
  v[0] = f16_lo(u[0]);
  v[1] = f16_hi(u[0]);
  v[2] = f16_lo(u[1]);
  v[3] = f16_hi(u[1]);
}
__device__ __forceinline__ void store4(f16_t* p, const float* v) {
  *reinterpret_cast<u32x2_t*>(p) = u32x2_t{pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3])};
}
__device__ __forceinline__ void load4_nt(const f16_t* p, float* v) {
  const u32x2_t u = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
  v[0] = f16_lo(u[0]);
  v[1] = f16_hi(u[0]);
  v[2] = f16_lo(u[1]);
  v[3] = f16_hi(u[1]);
}
__device__ __forceinline__ void store4_nt(f16_t* p, const float* v) {
  __builtin_nontemporal_store(u32x2_t{pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3])},
                              reinterpret_cast<u32x2_t*>(p));
}
template <bool NT, typename T> __device__ __forceinline__ void load4p(const T* p, float* v) {
  if constexpr (NT) load4_nt(p, v); else load4(p, v);
}
template <bool NT, typename T> __device__ __forceinline__ void store4p(T* p, const float* v) {
  if constexpr (NT) store4_nt(p, v); else store4(p, v);
}

// gamma / beta: 16 raw bytes from the chunk's first element through a buffer
// resource (fp32: 4 values; bf16: the first 8 bytes), decoded by the uniform
// type flag after the load, so no branch separates a load from its use.
template <typename P16 = bf16_t>
__device__ __forceinline__ void decode_param(u32x4_t r, bool bf16, float* v) {
  if (bf16) {
    if constexpr (std::is_same<P16, f16_t>::value) {
      v[0] = f16_lo(r[0]);
      v[1] = f16_hi(r[0]);
      v[2] = f16_lo(r[1]);
      v[3] = f16_hi(r[1]);
    } else {
      v[0] = __uint_as_float(r[0] << 16);
      v[1] = __uint_as_float(r[0] & 0xffff0000u);
      v[2] = __uint_as_float(r[1] << 16);
      v[3] = __uint_as_float(r[1] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = __uint_as_float(r[j]);
  }
}

// R rows per wave, NCH 256-column chunks per row (the smallest count that
// covers it, so no load slot is wasted on a padded chunk); POL bit 0 makes the
// x / delta loads non-temporal, bit 1 the x_out / y stores.  Every load of the wave's rows is issued before
// any is used, with no branch around them: columns past the row load column
// 0 and rows past the last load the last row, both masked — one memory round
// trip per wave, which is what short batches (decode steps) are bound by.
template <typename TX, typename TD, typename TY, int NCH, int R, bool HASD, int POL>
__global__ __launch_bounds__(kLnThreads) void add_layernorm_kernel(
    const TX* x, const TD* __restrict__ delta, TX* x_out,
    const void* __restrict__ gamma, const void* __restrict__ beta, bool param_bf16,
    TY* __restrict__ y, int64_t rows, int cols, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * kLnRowsPerBlock + (threadIdx.x >> 6)) * R;
  if (row0 >= rows) return;
  const int pshift = param_bf16 ? 1 : 2;
  const __amdgpu_buffer_rsrc_t rg = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(gamma), 0, cols << pshift, 0x00020000);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(beta), 0, cols << pshift, 0x00020000);

  float v[R][NCH][4], dv[R][NCH][4];
  u32x4_t graw[NCH], braw[NCH];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int64_t base = min(row0 + i, rows - 1) * cols;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int col = (c * 64 + lane) * 4;
      const int cc = col < cols ? col : 0;
      load4p<(POL & 1) != 0>(x + base + cc, v[i][c]);
      if constexpr (HASD) load4p<(POL & 1) != 0>(delta + base + cc, dv[i][c]);
    }
  }
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int col = (c * 64 + lane) * 4;
    const int cc = col < cols ? col : 0;
    graw[c] = __builtin_amdgcn_raw_buffer_load_b128(rg, cc << pshift, 0, 0);
    braw[c] = __builtin_amdgcn_raw_buffer_load_b128(rb, cc << pshift, 0, 0);
  }
  // Correctly rounded divisions (not a multiply by 1/cols, which the compiler
  // may fuse into x - mean): a constant row then gives mean == x exactly and
  // y == beta.
  const float n_f = static_cast<float>(cols);
  float mean[R], rstd[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    float sum = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const bool ok = (c * 64 + lane) * 4 < cols;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float t = HASD ? v[i][c][j] + dv[i][c][j] : v[i][c][j];
        v[i][c][j] = ok ? t : 0.f;
        sum += v[i][c][j];
      }
    }
    mean[i] = wave_sum(sum) / n_f;
  }
#pragma unroll
  for (int i = 0; i < R; ++i) {
    float sq = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const bool ok = (c * 64 + lane) * 4 < cols;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float t = v[i][c][j] - mean[i];
        sq += ok ? t * t : 0.f;
      }
    }
    rstd[i] = 1.0f / sqrtf(wave_sum(sq) / n_f + eps);
  }
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    float gm[4], bt[4];
    // 16-bit parameters have the type of an fp16 row, else bf16.
    using P16 = typename std::conditional<std::is_same<TX, f16_t>::value, f16_t, bf16_t>::type;
    decode_param<P16>(graw[c], param_bf16, gm);
    decode_param<P16>(braw[c], param_bf16, bt);
    const int col = (c * 64 + lane) * 4;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      if (col < cols && row0 + i < rows) {
        const int64_t base = (row0 + i) * cols;
        if (x_out != nullptr) store4p<(POL & 2) != 0>(x_out + base + col, v[i][c]);
        float o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = (v[i][c][j] - mean[i]) * rstd[i] * gm[j] + bt[j];
        store4p<(POL & 2) != 0>(y + base + col, o);
      }
    }
  }
}

// bf16 rows in and out, no residual, bf16 gamma / beta, cols % 8 == 0 and
// cols <= 2048 (141 VGPRs a lane at 2048; 4096 would leave one wave a SIMD): a
// half-wave (32 lanes) per row so every access is 16 bytes (8 elements), the
// width at which a plain streaming copy runs fastest; with 4 elements a lane
// (8-byte accesses) the 16384 x 768 launch moved 4.1 TB/s.  Lane h of a half
// owns columns [8(32c + h), 8(32c + h) + 8) for chunk c < NCH; the sums run
// over the 32 lanes of the half (DPP rows of 16, then the two rows' results).
template <int NCH>
__global__ __launch_bounds__(kLnThreads) void layernorm_bf16_rows16_kernel(
    const bf16_t* x, const bf16_t* __restrict__ gamma, const bf16_t* __restrict__ beta,
    bf16_t* y, int64_t rows, int cols, float eps) {
  const int lane = threadIdx.x & 63, hl = lane & 31;
  const int64_t wrow = (static_cast<int64_t>(blockIdx.x) * kLnRowsPerBlock + (threadIdx.x >> 6)) * 2;
  if (wrow >= rows) return;
  const int64_t row = wrow + (lane >> 5);
  const int64_t base = (row < rows ? row : rows - 1) * cols;
  const __amdgpu_buffer_rsrc_t rg =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t*>(gamma), 0, cols * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t rb =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t*>(beta), 0, cols * 2, 0x00020000);
  u32x4_t raw[NCH], graw[NCH], braw[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int col = (c * 32 + hl) * 8;
    const int cc = col < cols ? col : 0;
    raw[c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(x + base + cc));
    graw[c] = __builtin_amdgcn_raw_buffer_load_b128(rg, cc * 2, 0, 0);
    braw[c] = __builtin_amdgcn_raw_buffer_load_b128(rb, cc * 2, 0, 0);
  }
  auto half_sum = [&](float v) {
    v = group_sum<16>(v);
    const float lo = lane_value(v, 0) + lane_value(v, 16);
    const float hi = lane_value(v, 32) + lane_value(v, 48);
    return lane < 32 ? lo : hi;
  };
  float v[NCH][8];
  float sum = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const bool ok = (c * 32 + hl) * 8 < cols;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[c][2 * j] = ok ? __uint_as_float(raw[c][j] << 16) : 0.f;
      v[c][2 * j + 1] = ok ? __uint_as_float(raw[c][j] & 0xffff0000u) : 0.f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) sum += v[c][j];
  }
  const float n_f = static_cast<float>(cols);
  const float mean = half_sum(sum) / n_f;
  float sq = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const bool ok = (c * 32 + hl) * 8 < cols;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float t = v[c][j] - mean;
      sq += ok ? t * t : 0.f;
    }
  }
  const float rstd = 1.0f / sqrtf(half_sum(sq) / n_f + eps);
  if (row >= rows) return;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int col = (c * 32 + hl) * 8;
    if (col < cols) {
      u32x4_t o;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float g0 = __uint_as_float(graw[c][j] << 16), g1 = __uint_as_float(graw[c][j] & 0xffff0000u);
        const float b0 = __uint_as_float(braw[c][j] << 16), b1 = __uint_as_float(braw[c][j] & 0xffff0000u);
        o[j] = pack_bf16x2((v[c][2 * j] - mean) * rstd * g0 + b0,
                           (v[c][2 * j + 1] - mean) * rstd * g1 + b1);
      }
      __builtin_nontemporal_store(o, reinterpret_cast<u32x4_t*>(y + base + col));
    }
  }
}

static int launch_ln_bf16_rows16(const bf16_t* x, const bf16_t* gamma, const bf16_t* beta,
                                 bf16_t* y, int64_t rows, int cols, float eps, hipStream_t s) {
  const int64_t blocks = (rows + 2 * kLnRowsPerBlock - 1) / (2 * kLnRowsPerBlock);
  if (blocks > 0x7fffffff) return CGPT_ESHAPE;
  const dim3 grid(static_cast<unsigned>(blocks));
#define CGPT_LN16(NCH)                                                                     \
  hipLaunchKernelGGL((layernorm_bf16_rows16_kernel<NCH>), grid, dim3(kLnThreads), 0, s, x, \
                     gamma, beta, y, rows, cols, eps)
  if (cols <= 256) CGPT_LN16(1);
  else if (cols <= 512) CGPT_LN16(2);
  else if (cols <= 768) CGPT_LN16(3);
  else if (cols <= 1024) CGPT_LN16(4);
  else if (cols <= 1792) CGPT_LN16(7);
  else CGPT_LN16(8);
#undef CGPT_LN16
  return hip_status(hipGetLastError());
}

template <typename TX, typename TD, typename TY, int NCH, bool HASD>
static void launch_ln_nch(const TX* x, const TD* d, TX* xo, const void* gamma, const void* beta,
                          bool pb, TY* y, int64_t rows, int cols, float eps, hipStream_t s) {
  // One row per wave: with 2 or 4 rows a wave (fewer, longer waves) the
  // 16384-row GPT-2 batch ran 4-15 % slower.  Streaming policy, from a sweep
  // over rotating buffers larger than the MALL: with a delta (the model's
  // residual add), non-temporal loads and cached stores (the next GEMM reads
  // y right away); without one, non-temporal loads and stores.
  constexpr int R = 1, POL = HASD ? 1 : 3;
  const dim3 grid(static_cast<unsigned>((rows + kLnRowsPerBlock * R - 1) / (kLnRowsPerBlock * R)));
  hipLaunchKernelGGL((add_layernorm_kernel<TX, TD, TY, NCH, R, HASD, POL>), grid, dim3(kLnThreads), 0, s,
                     x, d, xo, gamma, beta, pb, y, rows, cols, eps);
}

template <typename TX, typename TD, typename TY, bool HASD>
static void launch_ln_cols(const TX* x, const TD* d, TX* xo, const void* gamma, const void* beta,
                           bool pb, TY* y, int64_t rows, int cols, float eps, hipStream_t s) {
  if (cols <= 512)
    launch_ln_nch<TX, TD, TY, 2, HASD>(x, d, xo, gamma, beta, pb, y, rows, cols, eps, s);
  else if (cols <= 768)
    launch_ln_nch<TX, TD, TY, 3, HASD>(x, d, xo, gamma, beta, pb, y, rows, cols, eps, s);
  else if (cols <= 1024)
    launch_ln_nch<TX, TD, TY, 4, HASD>(x, d, xo, gamma, beta, pb, y, rows, cols, eps, s);
  else if (cols <= 1792)
    launch_ln_nch<TX, TD, TY, 7, HASD>(x, d, xo, gamma, beta, pb, y, rows, cols, eps, s);
  else if (cols <= 2048)
    launch_ln_nch<TX, TD, TY, 8, HASD>(x, d, xo, gamma, beta, pb, y, rows, cols, eps, s);
  else
    launch_ln_nch<TX, TD, TY, 16, HASD>(x, d, xo, gamma, beta, pb, y, rows, cols, eps, s);
}

template <typename TX, typename TD, typename TY>
static int launch_ln3(const void* x, const void* delta, void* x_out, const void* gamma,
                      const void* beta, bool param_bf16, void* y, int64_t rows, int cols,
                      float eps, hipStream_t s) {
  const TX* xp = static_cast<const TX*>(x);
  const TD* dp = static_cast<const TD*>(delta);
  TX* xo = static_cast<TX*>(x_out);
  TY* yp = static_cast<TY*>(y);
  if (dp != nullptr) {
    launch_ln_cols<TX, TD, TY, true>(xp, dp, xo, gamma, beta, param_bf16, yp, rows, cols, eps, s);
  } else if constexpr (std::is_same<TX, TD>::value) {
    // Without a delta the TD parameter is unused: only the TD = TX instance exists.
    launch_ln_cols<TX, TD, TY, false>(xp, dp, xo, gamma, beta, param_bf16, yp, rows, cols, eps, s);
  } else {
    return CGPT_EINVAL;
  }
  return hip_status(hipGetLastError());
}

// ---- token + position embedding fused with the first LayerNorm
//
// One wave per token, as add_layernorm_kernel without a delta: the gathered
// row x = wte[id] + wpe[pos] (fp32, the residual stream) is written once and
// normalised from registers, so the LayerNorm does not read it back.  The
// arithmetic (fp32 sum of the two rows, two-pass mean / centred variance,
// the same reduction order) equals the embedding kernel followed by
// add_layernorm_kernel bit for bit.  Ids / positions out of range are clamped
// and flagged as in the embedding kernel.
template <typename TW, typename TY, int NCH>
__global__ __launch_bounds__(kLnThreads) void embedding_layernorm_kernel(
    const int64_t* __restrict__ idx, const TW* __restrict__ wte, const TW* __restrict__ wpe,
    const int* __restrict__ pos_dev, float* __restrict__ x_out, const void* __restrict__ gamma,
    const void* __restrict__ beta, TY* __restrict__ y, int64_t n_tokens, int64_t T, int cols,
    int64_t vocab, int64_t pos0, int64_t n_pos, float eps, int* err_flag) {
  const int lane = threadIdx.x & 63;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kLnRowsPerBlock + (threadIdx.x >> 6);
  if (i >= n_tokens) return;
  int64_t id = idx[i];
  bool bad = false;
  if (id < 0 || id >= vocab) {
    bad = true;
    id = id < 0 ? 0 : vocab - 1;
  }
  int64_t pos = pos0 + (pos_dev != nullptr ? static_cast<int64_t>(*pos_dev) : i % T);
  if (pos < 0 || pos >= n_pos) {
    bad = true;
    pos = pos < 0 ? 0 : n_pos - 1;
  }
  if (bad && err_flag != nullptr && lane == 0) *err_flag = 1;
  constexpr bool kParamBf16 = sizeof(TW) == 2;
  const int pshift = kParamBf16 ? 1 : 2;
  const __amdgpu_buffer_rsrc_t rg = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(gamma), 0, cols << pshift, 0x00020000);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(beta), 0, cols << pshift, 0x00020000);
  const TW* trow = wte + id * cols;
  const TW* prow = wpe + pos * cols;
  float v[NCH][4], pv[NCH][4];
  u32x4_t graw[NCH], braw[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int col = (c * 64 + lane) * 4;
    const int cc = col < cols ? col : 0;
    load4(trow + cc, v[c]);
    load4(prow + cc, pv[c]);
    graw[c] = __builtin_amdgcn_raw_buffer_load_b128(rg, cc << pshift, 0, 0);
    braw[c] = __builtin_amdgcn_raw_buffer_load_b128(rb, cc << pshift, 0, 0);
  }
  const float n_f = static_cast<float>(cols);
  float sum = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const bool ok = (c * 64 + lane) * 4 < cols;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float t = v[c][j] + pv[c][j];
      v[c][j] = ok ? t : 0.f;
      sum += v[c][j];
    }
  }
  const float mean = wave_sum(sum) / n_f;
  float sq = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const bool ok = (c * 64 + lane) * 4 < cols;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float t = v[c][j] - mean;
      sq += ok ? t * t : 0.f;
    }
  }
  const float rstd = 1.0f / sqrtf(wave_sum(sq) / n_f + eps);
  const int64_t base = i * cols;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int col = (c * 64 + lane) * 4;
    if (col < cols) {
      float gm[4], bt[4];
      decode_param(graw[c], kParamBf16, gm);
      decode_param(braw[c], kParamBf16, bt);
      store4(x_out + base + col, v[c]);
      float o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = (v[c][j] - mean) * rstd * gm[j] + bt[j];
      store4(y + base + col, o);
    }
  }
}

template <typename TW, typename TY>
static int launch_emb_ln(const int64_t* idx, const void* wte, const void* wpe, const int* pos_dev,
                         float* x_out, const void* gamma, const void* beta, void* y,
                         int64_t n_tokens, int64_t T, int cols, int64_t vocab, int64_t pos0,
                         int64_t n_pos, float eps, int* err, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((n_tokens + kLnRowsPerBlock - 1) / kLnRowsPerBlock));
  const TW* tw = static_cast<const TW*>(wte);
  const TW* pw = static_cast<const TW*>(wpe);
  TY* yp = static_cast<TY*>(y);
#define CGPT_EMB_LN(NCH)                                                                        \
  hipLaunchKernelGGL((embedding_layernorm_kernel<TW, TY, NCH>), grid, dim3(kLnThreads), 0, s, idx, \
                     tw, pw, pos_dev, x_out, gamma, beta, yp, n_tokens, T, cols, vocab, pos0,   \
                     n_pos, eps, err)
  if (cols <= 512) CGPT_EMB_LN(2);
  else if (cols <= 768) CGPT_EMB_LN(3);
  else if (cols <= 1024) CGPT_EMB_LN(4);
  else if (cols <= 1792) CGPT_EMB_LN(7);
  else if (cols <= 2048) CGPT_EMB_LN(8);
  else CGPT_EMB_LN(16);
#undef CGPT_EMB_LN
  return hip_status(hipGetLastError());
}

template <typename TX, typename TD>
static int launch_ln2(int y_dtype, const void* x, const void* delta, void* x_out,
                      const void* gamma, const void* beta, bool param_bf16, void* y,
                      int64_t rows, int cols, float eps, hipStream_t s) {
  if (y_dtype == CGPT_F32)
    return launch_ln3<TX, TD, float>(x, delta, x_out, gamma, beta, param_bf16, y, rows, cols, eps, s);
  if (y_dtype == CGPT_BF16)
    return launch_ln3<TX, TD, bf16_t>(x, delta, x_out, gamma, beta, param_bf16, y, rows, cols, eps, s);
  return CGPT_EDTYPE;
}

template <typename TX>
static int launch_ln1(int delta_dtype, int y_dtype, const void* x, const void* delta, void* x_out,
                      const void* gamma, const void* beta, bool param_bf16, void* y,
                      int64_t rows, int cols, float eps, hipStream_t s) {
  // Without a delta the TD parameter is unused; reuse the TX instantiation.
  if (delta == nullptr || delta_dtype == (sizeof(TX) == 4 ? CGPT_F32 : CGPT_BF16))
    return launch_ln2<TX, TX>(y_dtype, x, delta, x_out, gamma, beta, param_bf16, y, rows, cols, eps, s);
  if (delta_dtype == CGPT_F32)
    return launch_ln2<TX, float>(y_dtype, x, delta, x_out, gamma, beta, param_bf16, y, rows, cols, eps, s);
  if (delta_dtype == CGPT_BF16)
    return launch_ln2<TX, bf16_t>(y_dtype, x, delta, x_out, gamma, beta, param_bf16, y, rows, cols, eps, s);
  return CGPT_EDTYPE;
}

// ---- residual + LayerNorm over split-K partial products (decode steps)
//
// delta[r][c] = round_to(TD, P[0][r][c] + ... + P[n-1][r][c] + bias[c]) (the
// value the GEMM would have stored), then as add_layernorm_kernel.  A row is
// short (a decode step has one row per sequence) and its partials are n times
// its size, so a 256-thread block takes one row: thread t owns columns
// [4(256c + t), +4) for chunk c, and every load of the row (x, the n partials,
// bias, gamma, beta) is issued before any is used.  Partials past n read as
// zero from past their buffer's record count.
constexpr int kLnpThreads = 256;

template <typename TD> __device__ __forceinline__ float round_delta(float v);
template <> __device__ __forceinline__ float round_delta<float>(float v) { return v; }
template <> __device__ __forceinline__ float round_delta<bf16_t>(float v) { return bf16_to_f32(f32_to_bf16(v)); }

template <typename TD, typename TY, int MAXCH, int MAXP>
__global__ __launch_bounds__(kLnpThreads) void add_layernorm_partials_kernel(
    const float* x, const float* __restrict__ parts, int n_parts, int part_stride,
    int ldp, const void* __restrict__ bias, float* x_out, const void* __restrict__ gamma,
    const void* __restrict__ beta, bool param_bf16, TY* __restrict__ y, int cols, float eps) {
  __shared__ float scr[kLnpThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row = blockIdx.x;
  const int64_t base = static_cast<int64_t>(row) * cols;
  const int pshift = param_bf16 ? 1 : 2;
  const __amdgpu_buffer_rsrc_t rg = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(gamma), 0, cols << pshift, 0x00020000);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(beta), 0, cols << pshift, 0x00020000);
  // No bias: a zero record count makes every bias load read zero.
  const __amdgpu_buffer_rsrc_t rbi = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(bias), 0, bias != nullptr ? cols << pshift : 0, 0x00020000);
  const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(parts), 0, n_parts * part_stride * 4, 0x00020000);
  float v[MAXCH][4], gm[MAXCH][4], bt[MAXCH][4], bi[MAXCH][4];
  u32x4_t praw[MAXCH][MAXP], graw[MAXCH], braw[MAXCH], biraw[MAXCH];
#pragma unroll
  for (int c = 0; c < MAXCH; ++c) {
    const int col = (c * kLnpThreads + tid) * 4;
    const int cc = col < cols ? col : 0;
    load4(x + base + cc, v[c]);
    // Slots past n_parts (a uniform branch: no load issued) hold +0.
#pragma unroll
    for (int s = 0; s < MAXP; ++s)
      praw[c][s] = s < n_parts ? __builtin_amdgcn_raw_buffer_load_b128(
                                     rp, static_cast<uint32_t>(((s * part_stride) + row * ldp + cc) * 4), 0, 0)
                               : u32x4_t{0u, 0u, 0u, 0u};
    graw[c] = __builtin_amdgcn_raw_buffer_load_b128(rg, cc << pshift, 0, 0);
    braw[c] = __builtin_amdgcn_raw_buffer_load_b128(rb, cc << pshift, 0, 0);
    biraw[c] = __builtin_amdgcn_raw_buffer_load_b128(rbi, cc << pshift, 0, 0);
  }
  float sum = 0.f;
#pragma unroll
  for (int c = 0; c < MAXCH; ++c) {
    const bool ok = (c * kLnpThreads + tid) * 4 < cols;
    decode_param(graw[c], param_bf16, gm[c]);
    decode_param(braw[c], param_bf16, bt[c]);
    decode_param(biraw[c], param_bf16, bi[c]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // Slots past n_parts hold +0: adding them leaves every sum but -0 as is.
      float d = __uint_as_float(praw[c][0][j]);
#pragma unroll
      for (int s = 1; s < MAXP; ++s) d += __uint_as_float(praw[c][s][j]);
      const float t = v[c][j] + round_delta<TD>(d + bi[c][j]);
      v[c][j] = ok ? t : 0.f;
      sum += v[c][j];
    }
  }
  // Block sums in wave order; correctly rounded divisions as the row kernel.
  const float n_f = static_cast<float>(cols);
  float ws = wave_sum(sum);
  if (lane == 0) scr[wave] = ws;
  __syncthreads();
  float tot = scr[0];
#pragma unroll
  for (int w = 1; w < kLnpThreads / 64; ++w) tot += scr[w];
  const float mean = tot / n_f;
  float sq = 0.f;
#pragma unroll
  for (int c = 0; c < MAXCH; ++c) {
    const bool ok = (c * kLnpThreads + tid) * 4 < cols;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float t = v[c][j] - mean;
      sq += ok ? t * t : 0.f;
    }
  }
  ws = wave_sum(sq);
  __syncthreads();  // every wave has read scr
  if (lane == 0) scr[wave] = ws;
  __syncthreads();
  tot = scr[0];
#pragma unroll
  for (int w = 1; w < kLnpThreads / 64; ++w) tot += scr[w];
  const float rstd = 1.0f / sqrtf(tot / n_f + eps);
#pragma unroll
  for (int c = 0; c < MAXCH; ++c) {
    const int col = (c * kLnpThreads + tid) * 4;
    if (col < cols) {
      if (x_out != nullptr) store4(x_out + base + col, v[c]);
      float o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = (v[c][j] - mean) * rstd * gm[c][j] + bt[c][j];
      store4(y + base + col, o);
    }
  }
}

template <typename TD, typename TY, int MAXCH>
static void launch_lnp_p(int maxp, const float* x, const float* parts, int n, int ps, int ldp,
                         const void* bias, float* x_out, const void* gamma, const void* beta,
                         bool pb, TY* y, int rows, int cols, float eps, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(rows)), block(kLnpThreads);
  if (maxp <= 2)
    hipLaunchKernelGGL((add_layernorm_partials_kernel<TD, TY, MAXCH, 2>), grid, block, 0, s, x, parts, n, ps, ldp, bias, x_out, gamma, beta, pb, y, cols, eps);
  else if (maxp <= 4)
    hipLaunchKernelGGL((add_layernorm_partials_kernel<TD, TY, MAXCH, 4>), grid, block, 0, s, x, parts, n, ps, ldp, bias, x_out, gamma, beta, pb, y, cols, eps);
  else if (maxp <= 8)
    hipLaunchKernelGGL((add_layernorm_partials_kernel<TD, TY, MAXCH, 8>), grid, block, 0, s, x, parts, n, ps, ldp, bias, x_out, gamma, beta, pb, y, cols, eps);
  else
    hipLaunchKernelGGL((add_layernorm_partials_kernel<TD, TY, MAXCH, 16>), grid, block, 0, s, x, parts, n, ps, ldp, bias, x_out, gamma, beta, pb, y, cols, eps);
}

template <typename TD, typename TY>
static int launch_lnp(const float* x, const float* parts, int n, int ps, int ldp, const void* bias,
                      float* x_out, const void* gamma, const void* beta, bool pb, void* y,
                      int rows, int cols, float eps, hipStream_t s) {
  TY* yp = static_cast<TY*>(y);
  if (cols <= 1024)
    launch_lnp_p<TD, TY, 1>(n, x, parts, n, ps, ldp, bias, x_out, gamma, beta, pb, yp, rows, cols, eps, s);
  else if (cols <= 2048)
    launch_lnp_p<TD, TY, 2>(n, x, parts, n, ps, ldp, bias, x_out, gamma, beta, pb, yp, rows, cols, eps, s);
  else
    launch_lnp_p<TD, TY, 4>(n, x, parts, n, ps, ldp, bias, x_out, gamma, beta, pb, yp, rows, cols, eps, s);
  return hip_status(hipGetLastError());
}

// ---- any width, any element alignment, every dtype combination
//
// One 256-thread block per row; thread t owns columns t, t + 256, ...  Three
// passes over the row: the sum of x (+ delta), the centred sum of squares,
// then x_out and y — the second and third re-read the row (from L2 for rows
// up to a few MB).  Dtypes are launch arguments (uniform branches).  Used for
// what the vector kernels above do not take: fp16, widths not a multiple of
// 4 or above 4096, rows that are not 16-byte (fp32) / 8-byte aligned.  Same
// arithmetic as those kernels (fp32 sums, mean and centred variance divided
// by cols, y = (v - mean) * rstd * gamma + beta) up to summation order.
__device__ __forceinline__ float ld_any(const void* p, int dt, int64_t i) {
  if (dt == CGPT_F32) return static_cast<const float*>(p)[i];
  if (dt == CGPT_BF16) return bf16_to_f32(static_cast<const bf16_t*>(p)[i]);
  return static_cast<float>(static_cast<const f16_t*>(p)[i]);
}
__device__ __forceinline__ void st_any(void* p, int dt, int64_t i, float v) {
  if (dt == CGPT_F32) static_cast<float*>(p)[i] = v;
  else if (dt == CGPT_BF16) static_cast<bf16_t*>(p)[i] = f32_to_bf16(v);
  else static_cast<f16_t*>(p)[i] = static_cast<f16_t>(v);
}

__device__ __forceinline__ float block_sum256(float v, float* red) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6;
  __syncthreads();  // earlier readers of red are done
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

__global__ __launch_bounds__(kLnThreads) void add_layernorm_any_kernel(
    const void* x, const void* delta, void* x_out, const void* gamma, const void* beta, void* y,
    int64_t cols, float eps, int xd, int dd, int pd, int yd) {
  __shared__ float red[kLnThreads / 64];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * cols;
  auto val = [&](int64_t c) {
    const float v = ld_any(x, xd, base + c);
    return delta != nullptr ? v + ld_any(delta, dd, base + c) : v;
  };
  const float n_f = static_cast<float>(cols);
  float sum = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += kLnThreads) sum += val(c);
  const float mean = block_sum256(sum, red) / n_f;
  float sq = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += kLnThreads) {
    const float t = val(c) - mean;
    sq += t * t;
  }
  const float rstd = 1.0f / sqrtf(block_sum256(sq, red) / n_f + eps);
  // Every element is read and then written by the same thread, so x_out or y
  // may alias x.
  for (int64_t c = threadIdx.x; c < cols; c += kLnThreads) {
    const float v = val(c);
    if (x_out != nullptr) st_any(x_out, xd, base + c, v);
    st_any(y, yd, base + c, (v - mean) * rstd * ld_any(gamma, pd, c) + ld_any(beta, pd, c));
  }
}

static bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7) == 0; }
static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
static bool dtype_ok(int d) { return d == CGPT_F32 || d == CGPT_BF16; }
static bool dtype_any_ok(int d) { return d == CGPT_F32 || d == CGPT_BF16 || d == CGPT_F16; }
static bool elem_aligned(const void* p, int dtype) {
  return (reinterpret_cast<uintptr_t>(p) & (dtype == CGPT_F32 ? 3 : 1)) == 0;
}
static bool ptr_aligned(const void* p, int dtype) {
  return p == nullptr || (dtype == CGPT_F32 ? aligned16(p) : aligned8(p));
}

}  // namespace cgpt

extern "C" int cgpt_add_layernorm(const void* x, const void* delta, void* x_out,
                                  const void* gamma, const void* beta, void* y, int64_t rows,
                                  int64_t cols, float eps, int x_dtype, int delta_dtype,
                                  int param_dtype, int y_dtype, void* stream) {
  using namespace cgpt;
  if (rows < 0 || cols <= 0) return CGPT_EINVAL;
  if (rows == 0) return CGPT_OK;
  if (x == nullptr || gamma == nullptr || beta == nullptr || y == nullptr) return CGPT_EINVAL;
  if (!dtype_any_ok(x_dtype) || !dtype_any_ok(param_dtype) || !dtype_any_ok(y_dtype) ||
      (delta != nullptr && !dtype_any_ok(delta_dtype)))
    return CGPT_EDTYPE;
  if (!elem_aligned(x, x_dtype) || (x_out != nullptr && !elem_aligned(x_out, x_dtype)) ||
      !elem_aligned(y, y_dtype) || !elem_aligned(gamma, param_dtype) ||
      !elem_aligned(beta, param_dtype) || (delta != nullptr && !elem_aligned(delta, delta_dtype)))
    return CGPT_EINVAL;
  if (!(eps >= 0.f)) return CGPT_EINVAL;
  if (cols > 0x7fffffff) return CGPT_ESHAPE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // The vector kernels: fp32 / bf16, four-element vectors per lane (rows
  // keep 4-element alignment), whole rows in registers up to 4096 columns.
  const bool vec = dtype_ok(x_dtype) && dtype_ok(param_dtype) && dtype_ok(y_dtype) &&
                   (delta == nullptr || dtype_ok(delta_dtype)) && cols % 4 == 0 && cols <= 4096 &&
                   ptr_aligned(x, x_dtype) && ptr_aligned(x_out, x_dtype) &&
                   ptr_aligned(y, y_dtype) && ptr_aligned(gamma, param_dtype) &&
                   ptr_aligned(beta, param_dtype) && (delta == nullptr || ptr_aligned(delta, delta_dtype));
  // fp16 rows (x, delta, y all fp16; fp16 or fp32 parameters) on the same
  // register-resident kernel, 8-byte aligned like bf16.
  const bool vec16 = x_dtype == CGPT_F16 && y_dtype == CGPT_F16 &&
                     (delta == nullptr || delta_dtype == CGPT_F16) &&
                     (param_dtype == CGPT_F16 || param_dtype == CGPT_F32) && cols % 4 == 0 &&
                     cols <= 4096 && aligned8(x) && (x_out == nullptr || aligned8(x_out)) &&
                     aligned8(y) && (delta == nullptr || aligned8(delta)) &&
                     ptr_aligned(gamma, param_dtype) && ptr_aligned(beta, param_dtype);
  if (vec16) {
    const f16_t* xp = static_cast<const f16_t*>(x);
    const f16_t* dp = static_cast<const f16_t*>(delta);
    f16_t* xo = static_cast<f16_t*>(x_out);
    f16_t* yp = static_cast<f16_t*>(y);
    const bool p16 = param_dtype == CGPT_F16;
    if (dp != nullptr)
      launch_ln_cols<f16_t, f16_t, f16_t, true>(xp, dp, xo, gamma, beta, p16, yp, rows,
                                                static_cast<int>(cols), eps, s);
    else
      launch_ln_cols<f16_t, f16_t, f16_t, false>(xp, dp, xo, gamma, beta, p16, yp, rows,
                                                 static_cast<int>(cols), eps, s);
    return hip_status(hipGetLastError());
  }
  if (!vec) {
    if (rows > 0x7fffffff) return CGPT_ESHAPE;
    hipLaunchKernelGGL(add_layernorm_any_kernel, dim3(static_cast<unsigned>(rows)), dim3(kLnThreads),
                       0, s, x, delta, x_out, gamma, beta, y, cols, eps, x_dtype, delta_dtype,
                       param_dtype, y_dtype);
    return hip_status(hipGetLastError());
  }
  const bool pb = param_dtype == CGPT_BF16;
  const int c = static_cast<int>(cols);
  if (x_dtype == CGPT_BF16 && y_dtype == CGPT_BF16 && pb && delta == nullptr &&
      x_out == nullptr && c % 8 == 0 && c <= 2048 &&
      ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15) == 0)
    return launch_ln_bf16_rows16(static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(gamma),
                                 static_cast<const bf16_t*>(beta), static_cast<bf16_t*>(y), rows,
                                 c, eps, s);
  if (x_dtype == CGPT_F32)
    return launch_ln1<float>(delta_dtype, y_dtype, x, delta, x_out, gamma, beta, pb, y, rows, c, eps, s);
  return launch_ln1<bf16_t>(delta_dtype, y_dtype, x, delta, x_out, gamma, beta, pb, y, rows, c, eps, s);
}

extern "C" int cgpt_add_layernorm_partials(const void* x, const float* partials, int64_t n_parts,
                                           int64_t part_stride, int64_t ldp, const void* bias,
                                           void* x_out, const void* gamma, const void* beta,
                                           void* y, int64_t rows, int64_t cols, float eps,
                                           int x_dtype, int delta_dtype, int param_dtype,
                                           int y_dtype, void* stream) {
  using namespace cgpt;
  if (rows < 0 || cols <= 0) return CGPT_EINVAL;
  if (rows == 0) return CGPT_OK;
  if (x == nullptr || partials == nullptr || gamma == nullptr || beta == nullptr || y == nullptr)
    return CGPT_EINVAL;
  if (x_dtype != CGPT_F32 || !dtype_ok(delta_dtype) || !dtype_ok(param_dtype) || !dtype_ok(y_dtype))
    return CGPT_EDTYPE;
  if (cols % 4 != 0 || cols > 4096 || rows > 0x7fffffff) return CGPT_ESHAPE;
  if (n_parts < 1 || n_parts > 16 || ldp < cols || ldp % 4 != 0 || part_stride % 4 != 0 ||
      part_stride < (rows - 1) * ldp + cols)
    return CGPT_EINVAL;
  if (n_parts * part_stride * 4 >= (int64_t{1} << 31)) return CGPT_ESHAPE;
  if (!aligned16(partials) || !ptr_aligned(x, x_dtype) || !ptr_aligned(x_out, x_dtype) ||
      !ptr_aligned(y, y_dtype) || !ptr_aligned(gamma, param_dtype) ||
      !ptr_aligned(beta, param_dtype) || !ptr_aligned(bias, param_dtype))
    return CGPT_EINVAL;
  if (!(eps >= 0.f)) return CGPT_EINVAL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool pb = param_dtype == CGPT_BF16;
  const int r = static_cast<int>(rows), c = static_cast<int>(cols), n = static_cast<int>(n_parts);
  const int ps = static_cast<int>(part_stride), lp = static_cast<int>(ldp);
  const float* xp = static_cast<const float*>(x);
  float* xo = static_cast<float*>(x_out);
  if (delta_dtype == CGPT_BF16)
    return y_dtype == CGPT_BF16
               ? launch_lnp<bf16_t, bf16_t>(xp, partials, n, ps, lp, bias, xo, gamma, beta, pb, y, r, c, eps, s)
               : launch_lnp<bf16_t, float>(xp, partials, n, ps, lp, bias, xo, gamma, beta, pb, y, r, c, eps, s);
  return y_dtype == CGPT_BF16
             ? launch_lnp<float, bf16_t>(xp, partials, n, ps, lp, bias, xo, gamma, beta, pb, y, r, c, eps, s)
             : launch_lnp<float, float>(xp, partials, n, ps, lp, bias, xo, gamma, beta, pb, y, r, c, eps, s);
}

extern "C" int cgpt_embedding_layernorm(const int64_t* idx, const void* wte, const void* wpe,
                                        const int* pos_dev, float* x_out, const void* gamma,
                                        const void* beta, void* y, int64_t n_tokens, int64_t T,
                                        int64_t D, int64_t vocab, int64_t pos0, int64_t n_pos,
                                        float eps, int w_dtype, int y_dtype, int* err_flag,
                                        void* stream) {
  using namespace cgpt;
  if (n_tokens < 0 || D <= 0 || vocab <= 0 || n_pos <= 0) return CGPT_EINVAL;
  if (n_tokens == 0) return CGPT_OK;
  if (idx == nullptr || wte == nullptr || wpe == nullptr || x_out == nullptr || gamma == nullptr ||
      beta == nullptr || y == nullptr || T <= 0)
    return CGPT_EINVAL;
  if (!dtype_ok(w_dtype) || !dtype_ok(y_dtype)) return CGPT_EDTYPE;
  if (D % 4 != 0 || D > 4096) return CGPT_ESHAPE;
  if (!ptr_aligned(wte, w_dtype) || !ptr_aligned(wpe, w_dtype) || !ptr_aligned(gamma, w_dtype) ||
      !ptr_aligned(beta, w_dtype) || !aligned16(x_out) || !ptr_aligned(y, y_dtype) ||
      (reinterpret_cast<uintptr_t>(idx) & 7))
    return CGPT_EINVAL;
  if (!(eps >= 0.f)) return CGPT_EINVAL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int c = static_cast<int>(D);
  if (w_dtype == CGPT_BF16)
    return y_dtype == CGPT_BF16
               ? launch_emb_ln<bf16_t, bf16_t>(idx, wte, wpe, pos_dev, x_out, gamma, beta, y, n_tokens, T, c, vocab, pos0, n_pos, eps, err_flag, s)
               : launch_emb_ln<bf16_t, float>(idx, wte, wpe, pos_dev, x_out, gamma, beta, y, n_tokens, T, c, vocab, pos0, n_pos, eps, err_flag, s);
  return y_dtype == CGPT_BF16
             ? launch_emb_ln<float, bf16_t>(idx, wte, wpe, pos_dev, x_out, gamma, beta, y, n_tokens, T, c, vocab, pos0, n_pos, eps, err_flag, s)
             : launch_emb_ln<float, float>(idx, wte, wpe, pos_dev, x_out, gamma, beta, y, n_tokens, T, c, vocab, pos0, n_pos, eps, err_flag, s);
}
