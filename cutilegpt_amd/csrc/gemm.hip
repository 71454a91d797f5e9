// C[M,N] = epilogue(A[M,K] W[N,K]^T + bias) on CDNA4 matrix cores.
//
// Layout and schedule
//  * A (activations, row-major) and W (nn.Linear weight, row-major (N, K)) are
//    both K-contiguous, so both tiles are staged in LDS the same way: one
//    128-byte LDS row per matrix row per K step (64 bf16 or 32 fp32), written
//    as eight 16-byte chunks whose position is XOR-swizzled with (row & 7) to
//    spread the fragment reads of 16 consecutive rows over the LDS banks.
//  * A block of WGM x WGN wavefronts owns a BM x BN output tile; each wave owns
//    a (BM/WGM) x (BN/WGN) sub-tile made of 16x16 MFMA tiles.  The MFMA is fed
//    with the W fragment as its "A" operand and the activation fragment as its
//    "B" operand, so the 16x16 accumulator is C^T: lane l holds C[m = l%16]
//    [n = 4(l/16) .. 4(l/16)+3] — four consecutive output columns of one row,
//    which makes bias, GELU and the store 4-wide.
//  * bf16: v_mfma_f32_16x16x32_bf16 (each lane supplies 8 consecutive k).
//    fp32: four v_mfma_f32_16x16x4_f32 per 16-byte fragment; lane group g
//    supplies k = 4g + j to the j-th MFMA (any consistent permutation of the
//    k axis leaves the dot product unchanged).
//  * Global -> register -> LDS double buffering: the loads of K step t+1 are in
//    flight while the MFMAs of step t run; one barrier per K step.
//  * Block ids are remapped so that tiles adjacent in the grouped (GROUP_M)
//    order run on the same XCD (the dispatcher deals block ids round-robin over
//    the 8 XCDs, each with its own L2).
#include "common.h"

namespace cgpt {

constexpr int kGroupM = 8;
constexpr int kNumXcd = 8;

template <typename T> struct Mfma;
template <> struct Mfma<bf16_t> {
  __device__ static void run(const u32x4_t& a, const u32x4_t& b, f32x4_t& c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
};
template <> struct Mfma<float> {
  __device__ static void run(const u32x4_t& a, const u32x4_t& b, f32x4_t& c) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[j]), __uint_as_float(b[j]), c, 0,
                                               0, 0);
  }
};

__device__ __forceinline__ void store4_out(float* p, const float* v) { store_vec(p, v); }
__device__ __forceinline__ void store4_out(bf16_t* p, const float* v) {
  u32x2_t u = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  *reinterpret_cast<u32x2_t*>(p) = u;
}

__device__ __forceinline__ float load_bias(const void* bias, bool bf16, int64_t n) {
  return bf16 ? bf16_to_f32(static_cast<const bf16_t*>(bias)[n]) : static_cast<const float*>(bias)[n];
}

// Map a hardware block id to (tile_m, tile_n): XCD-contiguous, then grouped.
__device__ __forceinline__ void tile_coords(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int nblocks = tiles_m * tiles_n;
  const int q = nblocks / kNumXcd, r = nblocks % kNumXcd;
  const int xcd = bid % kNumXcd;
  const int logical = xcd * q + (xcd < r ? xcd : r) + bid / kNumXcd;
  const int group = kGroupM * tiles_n;
  const int g = logical / group;
  const int first_m = g * kGroupM;
  const int gsz = min(tiles_m - first_m, kGroupM);
  const int in_group = logical % group;
  tm = first_m + in_group % gsz;
  tn = in_group / gsz;
}

template <typename TIn, int BM, int BN, int WGM, int WGN, int EPI, typename TOut>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_kernel(
    const TIn* __restrict__ A, const TIn* __restrict__ W, const void* __restrict__ bias,
    bool bias_bf16, TOut* __restrict__ C, int M, int N, int K, int64_t lda, int64_t ldw,
    int64_t ldc, int tiles_m, int tiles_n, bool vec_store) {
  constexpr int NT = 64 * WGM * WGN;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int EPC = 16 / sizeof(TIn);  // elements per 16-byte chunk
  constexpr int BK = 8 * EPC;            // elements per 128-byte LDS row
  constexpr int A_LD = BM * 8 / NT;      // 16-byte chunks per thread per stage
  constexpr int W_LD = BN * 8 / NT;
  static_assert(BM * 8 % NT == 0 && BN * 8 % NT == 0, "tile/thread mismatch");
  constexpr int STAGE = (BM + BN) * 128;
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm0 = (wave / WGN) * WM;
  const int wn0 = (wave % WGN) * WN;

  int tile_m, tile_n;
  tile_coords(blockIdx.x, tiles_m, tiles_n, tile_m, tile_n);
  const int m0 = tile_m * BM;
  const int n0 = tile_n * BN;

  u32x4_t ra[A_LD], rw[W_LD];
  // Row indices past the matrix edge are clamped to the last row (the rows are
  // loaded but never stored); the K tail past K is zero-filled.
  auto gload = [&](int kt) {
    const int kbase = kt * BK;
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const int q = tid + i * NT;
      const int r = q >> 3, kc = q & 7;
      const int64_t row = min(m0 + r, M - 1);
      const int k = kbase + kc * EPC;
      ra[i] = (k < K) ? *reinterpret_cast<const u32x4_t*>(A + row * lda + k) : u32x4_t{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < W_LD; ++i) {
      const int q = tid + i * NT;
      const int r = q >> 3, kc = q & 7;
      const int64_t row = min(n0 + r, N - 1);
      const int k = kbase + kc * EPC;
      rw[i] = (k < K) ? *reinterpret_cast<const u32x4_t*>(W + row * ldw + k) : u32x4_t{0, 0, 0, 0};
    }
  };
  auto swrite = [&](int buf) {
    uint8_t* sa = smem + buf * STAGE;
    uint8_t* sw = sa + BM * 128;
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const int q = tid + i * NT;
      const int r = q >> 3, kc = q & 7;
      *reinterpret_cast<u32x4_t*>(sa + r * 128 + ((kc ^ (r & 7)) << 4)) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < W_LD; ++i) {
      const int q = tid + i * NT;
      const int r = q >> 3, kc = q & 7;
      *reinterpret_cast<u32x4_t*>(sw + r * 128 + ((kc ^ (r & 7)) << 4)) = rw[i];
    }
  };

  f32x4_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int KT = (K + BK - 1) / BK;
  gload(0);
  swrite(0);
  __syncthreads();

  const int frow = lane & 15;   // row within a 16-row fragment
  const int fgrp = lane >> 4;   // which 16-byte chunk of the 64-byte k-slab
  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < KT) gload(kt + 1);
    const uint8_t* sa = smem + buf * STAGE;
    const uint8_t* sw = sa + BM * 128;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int c = 4 * s + fgrp;
      u32x4_t af[TM], wf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = wm0 + i * 16 + frow;
        af[i] = *reinterpret_cast<const u32x4_t*>(sa + r * 128 + ((c ^ (r & 7)) << 4));
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int r = wn0 + j * 16 + frow;
        wf[j] = *reinterpret_cast<const u32x4_t*>(sw + r * 128 + ((c ^ (r & 7)) << 4));
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) Mfma<TIn>::run(wf[j], af[i], acc[i][j]);
    }
    if (kt + 1 < KT) swrite(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: lane holds C[m][n .. n+3].
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = m0 + wm0 + i * 16 + frow;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + wn0 + j * 16 + 4 * fgrp;
      if (n >= N) continue;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float t = acc[i][j][r];
        if (EPI != CGPT_EPI_NONE && n + r < N) t += load_bias(bias, bias_bf16, n + r);
        if (EPI == CGPT_EPI_BIAS_GELU) t = gelu_tanh(t);
        v[r] = t;
      }
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

// ---------------------------------------------------------------------------
// Tile table.  Entries are (BM, BN, waves along M, waves along N); the LDS use
// is 2 * (BM + BN) * 128 bytes.

struct TileCfg {
  int bm, bn, wgm, wgn;
};

// bf16 configurations (index = tile id for CGPT_BF16).
static const TileCfg kBf16Tiles[] = {
    {256, 256, 2, 2},  // 0: 128x128 per wave, 128 KiB LDS
    {256, 128, 2, 2},  // 1: 128x64 per wave, 96 KiB LDS
    {128, 128, 2, 2},  // 2: 64x64 per wave, 64 KiB LDS
    {128, 64, 2, 2},   // 3: 64x32 per wave, 48 KiB LDS
    {64, 64, 2, 2},    // 4: 32x32 per wave, 32 KiB LDS
};
// fp32 configurations (index = tile id for CGPT_F32).
static const TileCfg kF32Tiles[] = {
    {128, 128, 2, 2},  // 0
    {64, 64, 2, 2},    // 1
};
constexpr int kNumBf16Tiles = sizeof(kBf16Tiles) / sizeof(kBf16Tiles[0]);
constexpr int kNumF32Tiles = sizeof(kF32Tiles) / sizeof(kF32Tiles[0]);

template <typename TIn, int BM, int BN, int WGM, int WGN, int EPI, typename TOut>
static int launch_cfg(const void* a, const void* w, const void* bias, bool bias_bf16, void* c,
                      int M, int N, int K, int64_t lda, int64_t ldw, int64_t ldc, bool vec_store,
                      hipStream_t s) {
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = (N + BN - 1) / BN;
  const int64_t blocks = static_cast<int64_t>(tiles_m) * tiles_n;
  if (blocks > 0x7fffffff) return CGPT_ESHAPE;
  hipLaunchKernelGGL((gemm_kernel<TIn, BM, BN, WGM, WGN, EPI, TOut>), dim3(static_cast<unsigned>(blocks)),
                     dim3(64 * WGM * WGN), 0, s, static_cast<const TIn*>(a),
                     static_cast<const TIn*>(w), bias, bias_bf16, static_cast<TOut*>(c), M, N, K,
                     lda, ldw, ldc, tiles_m, tiles_n, vec_store);
  return hip_status(hipGetLastError());
}

template <typename TIn, int EPI, typename TOut>
static int launch_tile(int tile, const void* a, const void* w, const void* bias, bool bias_bf16,
                       void* c, int M, int N, int K, int64_t lda, int64_t ldw, int64_t ldc,
                       bool vec_store, hipStream_t s) {
#define CGPT_GEMM_CASE(id, BM, BN, WGM, WGN)                                                   \
  case id:                                                                                    \
    return launch_cfg<TIn, BM, BN, WGM, WGN, EPI, TOut>(a, w, bias, bias_bf16, c, M, N, K, lda, \
                                                        ldw, ldc, vec_store, s);
  if constexpr (sizeof(TIn) == 2) {
    switch (tile) {
      CGPT_GEMM_CASE(0, 256, 256, 2, 2)
      CGPT_GEMM_CASE(1, 256, 128, 2, 2)
      CGPT_GEMM_CASE(2, 128, 128, 2, 2)
      CGPT_GEMM_CASE(3, 128, 64, 2, 2)
      CGPT_GEMM_CASE(4, 64, 64, 2, 2)
      default: return CGPT_EINVAL;
    }
  } else {
    switch (tile) {
      CGPT_GEMM_CASE(0, 128, 128, 2, 2)
      CGPT_GEMM_CASE(1, 64, 64, 2, 2)
      default: return CGPT_EINVAL;
    }
  }
#undef CGPT_GEMM_CASE
}

// Default tile choice: the largest tile whose grid still fills the 256 CUs
// about once; small problems fall back to smaller tiles.  The 256x256 bf16
// tile is only used when asked for explicitly.
static int auto_tile(bool bf16, int M, int N) {
  const TileCfg* t = bf16 ? kBf16Tiles : kF32Tiles;
  const int nt = bf16 ? kNumBf16Tiles : kNumF32Tiles;
  for (int i = bf16 ? 1 : 0; i < nt; ++i) {
    const int64_t blocks =
        static_cast<int64_t>((M + t[i].bm - 1) / t[i].bm) * ((N + t[i].bn - 1) / t[i].bn);
    if (blocks >= 256) return i;
  }
  return nt - 1;
}

template <typename TIn, typename TOut>
static int launch_epi(int epi, int tile, const void* a, const void* w, const void* bias,
                      bool bias_bf16, void* c, int M, int N, int K, int64_t lda, int64_t ldw,
                      int64_t ldc, bool vec_store, hipStream_t s) {
  switch (epi) {
    case CGPT_EPI_NONE:
      return launch_tile<TIn, CGPT_EPI_NONE, TOut>(tile, a, w, bias, bias_bf16, c, M, N, K, lda, ldw, ldc, vec_store, s);
    case CGPT_EPI_BIAS:
      return launch_tile<TIn, CGPT_EPI_BIAS, TOut>(tile, a, w, bias, bias_bf16, c, M, N, K, lda, ldw, ldc, vec_store, s);
    case CGPT_EPI_BIAS_GELU:
      return launch_tile<TIn, CGPT_EPI_BIAS_GELU, TOut>(tile, a, w, bias, bias_bf16, c, M, N, K, lda, ldw, ldc, vec_store, s);
    default:
      return CGPT_EINVAL;
  }
}

}  // namespace cgpt

extern "C" int cgpt_gemm_num_tiles(void) { return cgpt::kNumBf16Tiles; }

extern "C" int cgpt_gemm(const void* a, const void* w, const void* bias, void* c, int64_t M,
                         int64_t N, int64_t K, int64_t lda, int64_t ldw, int64_t ldc, int in_dtype,
                         int bias_dtype, int out_dtype, int epilogue, int tile, void* stream) {
  using namespace cgpt;
  if (M < 0 || N < 0 || K < 0) return CGPT_EINVAL;
  if (M == 0 || N == 0) return CGPT_OK;
  if (M > 0x7fffffff || N > 0x7fffffff || K > 0x7fffffff) return CGPT_ESHAPE;
  if (a == nullptr || w == nullptr || c == nullptr) return CGPT_EINVAL;
  if (epilogue != CGPT_EPI_NONE && epilogue != CGPT_EPI_BIAS && epilogue != CGPT_EPI_BIAS_GELU)
    return CGPT_EINVAL;
  if (epilogue != CGPT_EPI_NONE && bias == nullptr) return CGPT_EINVAL;
  if (in_dtype != CGPT_F32 && in_dtype != CGPT_BF16) return CGPT_EDTYPE;
  if (out_dtype != CGPT_F32 && out_dtype != CGPT_BF16) return CGPT_EDTYPE;
  if (epilogue != CGPT_EPI_NONE && bias_dtype != CGPT_F32 && bias_dtype != CGPT_BF16)
    return CGPT_EDTYPE;
  const bool bf16 = in_dtype == CGPT_BF16;
  const int64_t epc = bf16 ? 8 : 4;
  if (K == 0 || K % epc != 0) return CGPT_ESHAPE;
  if (lda < K || ldw < K || ldc < N) return CGPT_EINVAL;
  if (lda % epc != 0 || ldw % epc != 0) return CGPT_EINVAL;
  if ((reinterpret_cast<uintptr_t>(a) & 15) || (reinterpret_cast<uintptr_t>(w) & 15))
    return CGPT_EINVAL;
  const int nt = bf16 ? kNumBf16Tiles : kNumF32Tiles;
  if (tile == CGPT_TILE_AUTO) tile = auto_tile(bf16, static_cast<int>(M), static_cast<int>(N));
  if (tile < 0 || tile >= nt) return CGPT_EINVAL;
  const int64_t out_align = out_dtype == CGPT_F32 ? 16 : 8;
  const bool vec_store = (ldc % 4 == 0) && (reinterpret_cast<uintptr_t>(c) % out_align == 0);
  const bool bias_bf16 = bias_dtype == CGPT_BF16;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
  if (bf16 && out_dtype == CGPT_BF16)
    return launch_epi<bf16_t, bf16_t>(epilogue, tile, a, w, bias, bias_bf16, c, m, n, k, lda, ldw, ldc, vec_store, s);
  if (bf16)
    return launch_epi<bf16_t, float>(epilogue, tile, a, w, bias, bias_bf16, c, m, n, k, lda, ldw, ldc, vec_store, s);
  if (out_dtype == CGPT_F32)
    return launch_epi<float, float>(epilogue, tile, a, w, bias, bias_bf16, c, m, n, k, lda, ldw, ldc, vec_store, s);
  return launch_epi<float, bf16_t>(epilogue, tile, a, w, bias, bias_bf16, c, m, n, k, lda, ldw, ldc, vec_store, s);
}
