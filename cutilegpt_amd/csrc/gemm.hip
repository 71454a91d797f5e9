// C[M,N] = epilogue(A[M,K] W[N,K]^T + bias) on CDNA4 matrix cores.
//
// Layout shared by every kernel in this file
//  * A (activations, row-major) and W (nn.Linear weight, row-major (N, K)) are
//    both K-contiguous, so both tiles are staged in LDS the same way: one LDS
//    row per matrix row per stage (64 or 128 bytes of K), made of 16-byte chunks
//    whose position is XOR-swizzled with the row index so that the fragment
//    reads of 16 consecutive rows hit distinct LDS banks.
//  * A block of WGM x WGN wavefronts owns a BM x BN output tile; each wave owns
//    a (BM/WGM) x (BN/WGN) sub-tile made of 16x16 MFMA tiles.  The MFMA is fed
//    with the W fragment as its "A" operand and the activation fragment as its
//    "B" operand, so the 16x16 accumulator is C^T: lane l holds C[m = l%16]
//    [n = 4(l/16) .. 4(l/16)+3] — four consecutive output columns of one row,
//    which makes bias, GELU and the store 4-wide.
//  * bf16 / fp16: v_mfma_f32_16x16x32_bf16 / _f16 (each lane supplies 8
//    consecutive k); every 16-bit kernel is templated on the input type.
//    fp32: four v_mfma_f32_16x16x4_f32 per 16-byte fragment; lane group g
//    supplies k = 4g + j to the j-th MFMA (any consistent permutation of the
//    k axis leaves the dot product unchanged).
//  * Block (or tile) ids are remapped so that tiles adjacent in the grouped
//    (GROUP_M) order run on the same XCD (the dispatcher deals block ids
//    round-robin over the 8 XCDs, each with its own L2).
//
// Main loops:
//  * gemm_kernel: global -> registers -> LDS double buffering (fp32, and small
//    16-bit problems, any K multiple of 8/4; with element loads, any K, stride
//    or alignment).
//  * gemm_pipe_kernel / gemm_pipe_a3_kernel / gemm_slab_kernel: 16-bit
//    direct-to-LDS multi-stage pipelines, persistent over tiles (see the
//    comments above them).
#include <atomic>

#include "common.h"
#include "gemm_common.h"
#include "internal.h"

namespace cgpt {


#if defined(__HIP_DEVICE_COMPILE__)
// Four consecutive outputs through a buffer resource: a store whose byte
// offset lies at or past the resource's size is dropped by the hardware, so
// callers pass an out-of-range offset instead of branching around the store.
__device__ __forceinline__ void buffer_store4(__amdgpu_buffer_rsrc_t r, uint32_t off, const float* v,
                                              float*) {
  __builtin_amdgcn_raw_buffer_store_b128(
      u32x4_t{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])},
      r, off, 0, 0);
}
__device__ __forceinline__ void buffer_store4(__amdgpu_buffer_rsrc_t r, uint32_t off, const float* v,
                                              bf16_t*) {
  __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])}, r,
                                        off, 0, 0);
}
__device__ __forceinline__ void buffer_store4(__amdgpu_buffer_rsrc_t r, uint32_t off, const float* v,
                                              f16_t*) {
  __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3])}, r,
                                        off, 0, 0);
}
#endif

// The low (hi = false) or high 16-bit element of a 32-bit word as fp32, for a
// 16-bit type T (bf16 or fp16).
template <typename T>
__device__ __forceinline__ float half_word(uint32_t w, bool hi) {
  if constexpr (std::is_same<T, f16_t>::value) return hi ? f16_hi(w) : f16_lo(w);
  return __uint_as_float(hi ? (w & 0xffff0000u) : (w << 16));
}

// `half`: the bias holds 16-bit elements — fp16 when the inputs are fp16,
// bf16 otherwise — else fp32.
template <typename TIn>
__device__ __forceinline__ float load_bias(const void* bias, bool half, int64_t n) {
  if (!half) return static_cast<const float*>(bias)[n];
  if constexpr (std::is_same<TIn, f16_t>::value) return static_cast<float>(static_cast<const f16_t*>(bias)[n]);
  return bf16_to_f32(static_cast<const bf16_t*>(bias)[n]);
}




// Per-wave LDS scratch for re-mapping one 16x16 output block (17-float rows:
// conflict-free column and row accesses).
constexpr int kScrFloats = 16 * 17;

// Store a 16x16 block held in the C^T accumulator layout (lane l: row l%16,
// columns 4(l/16)..+3, values v[0..3]) when rows cannot take 16-byte stores
// (ldc not a multiple of 4, e.g. a 50257-wide vocabulary).  The block goes
// through the wave's LDS scratch so that each store instruction writes 16
// consecutive columns of 4 rows instead of 16 scattered rows.
template <typename TOut>
__device__ __forceinline__ void store_block_remap(float* scr, TOut* __restrict__ C, int64_t ldc,
                                                  int m0, int n0, int M, int N, const float* v,
                                                  int lane) {
  const int c = lane & 15, g = lane >> 4;
#pragma unroll
  for (int r = 0; r < 4; ++r) scr[c * 17 + 4 * g + r] = v[r];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = 4 * g + r;
    const float x = scr[row * 17 + c];
    const int m = m0 + row, n = n0 + c;
    if (m < M && n < N) Elem<TOut>::store(C + static_cast<int64_t>(m) * ldc + n, x);
  }
}

// ---------------------------------------------------------------------------
// Register-staged double-buffered kernel (fp32 and bf16; K % 8 (bf16) or
// K % 4 (fp32); the K tail of the last 128-byte row is zero-filled).

template <typename TIn, int BM, int BN, int WGM, int WGN, int EPI, typename TOut, bool EL = false>
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
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm0 = (wave / WGN) * WM;
  const int wn0 = (wave % WGN) * WN;

  int tile_m, tile_n;
  tile_coords(blockIdx.x, tiles_m, tiles_n, tile_m, tile_n);
  const int m0 = tile_m * BM;
  const int n0 = tile_n * BN;

  u32x4_t ra[A_LD], rw[W_LD];
  // 16 bytes of row `p` from element k: one vector load, or with EL (any K,
  // stride or alignment) element by element, elements at or past K read as 0.
  auto chunk = [&](const TIn* p, int k) -> u32x4_t {
    if constexpr (!EL) {
      return (k < K) ? *reinterpret_cast<const u32x4_t*>(p + k) : u32x4_t{0, 0, 0, 0};
    } else {
      u32x4_t v;
      if constexpr (sizeof(TIn) == 4) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = k + e < K ? reinterpret_cast<const uint32_t*>(p)[k + e] : 0u;
      } else {
        const uint16_t* h = reinterpret_cast<const uint16_t*>(p);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t lo = k + 2 * e < K ? h[k + 2 * e] : 0u;
          const uint32_t hi = k + 2 * e + 1 < K ? h[k + 2 * e + 1] : 0u;
          v[e] = lo | (hi << 16);
        }
      }
      return v;
    }
  };
  // Row indices past the matrix edge are clamped to the last row (the rows are
  // loaded but never stored); the K tail past K is zero-filled.
  auto gload = [&](int kt) {
    const int kbase = kt * BK;
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const int q = tid + i * NT;
      const int r = q >> 3, kc = q & 7;
      const int64_t row = min(m0 + r, M - 1);
      ra[i] = chunk(A + row * lda, kbase + kc * EPC);
    }
#pragma unroll
    for (int i = 0; i < W_LD; ++i) {
      const int q = tid + i * NT;
      const int r = q >> 3, kc = q & 7;
      const int64_t row = min(n0 + r, N - 1);
      rw[i] = chunk(W + row * ldw, kbase + kc * EPC);
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
        if (EPI != CGPT_EPI_NONE && n + r < N) t += load_bias<TIn>(bias, bias_bf16, n + r);
        if (EPI == CGPT_EPI_BIAS_GELU) t = gelu_tanh(t);
        if (EPI == CGPT_EPI_BIAS_RESID && n + r < N)
          t += Elem<TOut>::load(C + static_cast<int64_t>(m) * ldc + n + r);
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
// 16-bit (bf16 / fp16) direct-to-LDS pipeline, persistent over tiles.
//
// * Tiles reach LDS through `buffer_load_dwordx4 ... lds`: each lane's 16 bytes
//   land at (LDS base + lane * 16), so one wave instruction fills 1 KiB of LDS
//   rows; the XOR swizzle is applied on the global side (the lane that fills
//   physical chunk p of row r fetches logical chunk p ^ swz(r)).  No staging
//   registers and no ds_write.  Per-lane byte offsets are loop-invariant
//   within a tile; the K advance is the scalar offset.  Rows past M (or N) are
//   clamped to the last row, so every access stays inside the matrix.
// * A stage holds SPS k32 slabs (LDS rows of 64 * SPS bytes); STAGES stages
//   rotate through distinct __shared__ arrays.  Step g: raw s_barrier (every
//   wave has already waited for its own part of stage g), issue stage
//   g + STAGES - 1 into the buffer freed by step g - 1, read + MFMA the SPS
//   slabs of stage g, then wait (s_waitcnt vmcnt) until stage g + 1 has
//   landed, leaving only later stages (and the epilogue's stores, below) in
//   flight.  A full __syncthreads would add a release fence, i.e. vmcnt(0),
//   and collapse the pipeline to one stage; the empty asm statements keep the
//   compiler from moving LDS accesses across the barrier, and lgkmcnt(0) in
//   the same wait retires this step's LDS reads before the buffer is refilled.
// * Persistent: block b walks tiles b, b + grid, ...; their K stages form one
//   flattened stream, so the first stages of tile i+1 are in flight while tile
//   i finishes.  The grid holds as many blocks per CU as fit (one for the
//   8-wave tiles, two or three for the 4-wave ones).  The bias of the current tile is reloaded at every step before
//   the DMA (so it is older than anything a wait counts); the epilogue ends a
//   tile's last step.  With buffer-resource stores an epilogue issues exactly
//   TM * TN stores per wave and the following wait leaves them in flight;
//   otherwise that wait drains everything.
// Requires K % (32 * SPS) == 0.

// Wait until the stage that has `later` stages of LPS loads each issued after
// it, plus (when `stores`) ST stores, has landed: vmcnt retires loads and
// stores in issue order.  Counts past the 6-bit counter's range wait for 63
// (a stronger condition).
constexpr int vm_cap(int n) { return n < 63 ? n : 63; }
template <int LPS, int MAXLATER, int ST>
__device__ __forceinline__ void wait_stages(int later, bool stores) {
  static_assert(MAXLATER <= 4, "up to 6 stages");
  static_assert(MAXLATER * LPS < 64, "vmcnt range");
  if (stores) {
    if constexpr (MAXLATER >= 4) if (later >= 4) { wait_vmcnt<vm_cap(4 * LPS + ST)>(); return; }
    if constexpr (MAXLATER >= 3) if (later >= 3) { wait_vmcnt<vm_cap(3 * LPS + ST)>(); return; }
    if constexpr (MAXLATER >= 2) if (later >= 2) { wait_vmcnt<vm_cap(2 * LPS + ST)>(); return; }
    if constexpr (MAXLATER >= 1) if (later >= 1) { wait_vmcnt<vm_cap(1 * LPS + ST)>(); return; }
    wait_vmcnt<vm_cap(ST)>();
    return;
  }
  if constexpr (MAXLATER >= 4) if (later >= 4) { wait_vmcnt<4 * LPS>(); return; }
  if constexpr (MAXLATER >= 3) if (later >= 3) { wait_vmcnt<3 * LPS>(); return; }
  if constexpr (MAXLATER >= 2) if (later >= 2) { wait_vmcnt<2 * LPS>(); return; }
  if constexpr (MAXLATER >= 1) if (later >= 1) { wait_vmcnt<1 * LPS>(); return; }
  wait_vmcnt<0>();
}


// Output modes of gemm_pipe_kernel.  kOutWaveStagedNT is kOutWaveStaged with
// non-temporal stores: the LM head's logits (larger than the MALL, so nothing
// would still be cached for a consumer) are written 20 % faster (1.58 -> 1.31
// ms for the GPT-2 head), and c_fc + GELU runs 10 % faster (858 -> 947
// TFLOP/s in the GPT-2 forward) with the next GEMM reading its output no
// slower.
constexpr int kOutPlain = 0, kOutBuffer = 1, kOutWaveStaged = 2, kOutWaveStagedNT = 3;


// OUTM: kOutBuffer — every output store goes through a buffer resource
// (requires N % 4 == 0 and 16/8-byte aligned rows); kOutWaveStaged — the same,
// with each wave's rows staged through LDS so a store writes whole lines
// (requires rows of 16-byte multiples), and kOutWaveStagedNT the same with
// non-temporal stores; kOutPlain — plain stores behind per-lane bounds.
template <int BM, int BN, int WGM, int WGN, int SPS, int STAGES, int EPI, typename TOut, int OUTM,
          typename TIn = bf16_t>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_pipe_kernel(
    const TIn* __restrict__ A, const TIn* __restrict__ W, const void* __restrict__ bias,
    bool bias_bf16, TOut* __restrict__ C, int M, int N, int K, int64_t lda, int64_t ldw,
    int64_t ldc, int tiles_m, int tiles_n, bool vec_store) {
  // The body uses AMDGPU-only types (buffer resources); the host pass only
  // needs the kernel's signature for its launch stub.
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int NT = 64 * WGM * WGN, NW = NT / 64;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int ROWB = 64 * SPS;           // bytes of K per LDS row per stage
  constexpr int CPR = ROWB / 16;           // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;            // rows filled by one wave DMA instruction
  constexpr int STAGE = (BM + BN) * ROWB;
  constexpr int A_INS = BM / (RPI * NW);
  constexpr int W_INS = BN / (RPI * NW);
  constexpr int LPS = A_INS + W_INS;       // DMA instructions per wave per stage
  static_assert(SPS == 1 || SPS == 2, "one or two k32 slabs per stage");
  static_assert(STAGES >= 2 && STAGES <= 6, "2..6 stages");
  static_assert(BM % (RPI * NW) == 0 && BN % (RPI * NW) == 0, "tile/wave mismatch");
  static_assert((STAGES - 2) * LPS < 64, "vmcnt range");
  // Stage buffers at computed offsets in one array (the DMA writes them
  // through M0, so the compiler sees only the fragment reads).
  constexpr bool BUFST = OUTM >= kOutBuffer;
  // Wave-staged output: each wave's 16-row band of its WN columns (bias and
  // GELU applied) goes through a private LDS slot and out as whole rows.
  constexpr bool WSTAGED = OUTM == kOutWaveStaged || OUTM == kOutWaveStagedNT;
  constexpr int kStorePolicy = OUTM == kOutWaveStagedNT ? 2 : 0;  // 2: non-temporal
  constexpr int WROWB = WN * static_cast<int>(sizeof(TOut));  // bytes of a wave's row
  constexpr int WCPR = WROWB / 16;                              // 16-byte chunks per row
  constexpr int WNQ = 16 * WCPR / 64;                           // stores per 16-row band
  static_assert(!WSTAGED || (WCPR % 8 == 0 && WNQ * 64 == 16 * WCPR),
                "wave rows of whole 128-byte lines");
  static_assert(!WSTAGED || EPI != CGPT_EPI_BIAS_RESID, "no residual epilogue on staged output");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[STAGES * STAGE];
  __shared__ float escr[OUTM == kOutPlain ? NW : 1][OUTM == kOutPlain ? kScrFloats : 1];
  __shared__ __attribute__((aligned(16))) uint8_t sout[WSTAGED ? NW * 16 * WROWB : 16];

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm0 = (wave / WGN) * WM, wn0 = (wave % WGN) * WN;
  const int frow = lane & 15, fgrp = lane >> 4;
  const int lrow = lane / CPR, pchunk = lane % CPR;
  auto swz = [](int row) { return ROWB == 128 ? (row & 7) : ((row >> 1) & 3); };

  const u32x4_t ra = buffer_desc(A, static_cast<uint32_t>(static_cast<int64_t>(M) * lda * 2));
  const u32x4_t rw = buffer_desc(W, static_cast<uint32_t>(static_cast<int64_t>(N) * ldw * 2));

  const int n_tiles = tiles_m * tiles_n;
  const int KT = K / (32 * SPS);
  const int n_mine = (n_tiles - 1 - static_cast<int>(blockIdx.x)) / static_cast<int>(gridDim.x) + 1;
  const int total = n_mine * KT;

  // ---- issue side: next flattened stage to fetch and its tile's offsets
  int iss_i = 0, iss_kt = 0;
  uint32_t aoff[A_INS], woff[W_INS];
  auto set_offsets = [&](int i) {
    int tm, tn;
    tile_coords(static_cast<int>(blockIdx.x) + i * static_cast<int>(gridDim.x), tiles_m, tiles_n,
                tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
#pragma unroll
    for (int ii = 0; ii < A_INS; ++ii) {
      const int row = (ii * NW + wave) * RPI + lrow;
      const int64_t g = min(m0 + row, M - 1);
      aoff[ii] = static_cast<uint32_t>(g * lda * 2 + ((pchunk ^ swz(row)) << 4));
    }
#pragma unroll
    for (int ii = 0; ii < W_INS; ++ii) {
      const int row = (ii * NW + wave) * RPI + lrow;
      const int64_t g = min(n0 + row, N - 1);
      woff[ii] = static_cast<uint32_t>(g * ldw * 2 + ((pchunk ^ swz(row)) << 4));
    }
  };
  auto issue = [&](uint8_t* buf) {
    const int soff = iss_kt * ROWB;
#pragma unroll
    for (int ii = 0; ii < A_INS; ++ii)
      dma_lds16(ra, lds_addr(buf + (ii * NW + wave) * 1024), aoff[ii], soff);
#pragma unroll
    for (int ii = 0; ii < W_INS; ++ii)
      dma_lds16(rw, lds_addr(buf + BM * ROWB + (ii * NW + wave) * 1024), woff[ii], soff);
    if (++iss_kt == KT) {
      iss_kt = 0;
      if (++iss_i < n_mine) set_offsets(iss_i);
    }
  };

  // ---- compute side
  f32x4_t acc[TM][TN];
  auto zero_acc = [&]() {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  };
  // Byte offset of this lane's fragment row inside a stage, per slab.
  int xo[SPS];
#pragma unroll
  for (int s = 0; s < SPS; ++s) xo[s] = ((4 * s + fgrp) ^ swz(frow)) << 4;
  const int a_base = (wm0 + frow) * ROWB, w_base = BM * ROWB + (wn0 + frow) * ROWB;
  struct Frag {
    u32x4_t a[TM], w[TN];
  };
  auto read_slab = [&](const uint8_t* buf, int s, Frag& f) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
      f.a[i] = *reinterpret_cast<const u32x4_t*>(buf + a_base + i * 16 * ROWB + xo[s]);
#pragma unroll
    for (int j = 0; j < TN; ++j)
      f.w[j] = *reinterpret_cast<const u32x4_t*>(buf + w_base + j * 16 * ROWB + xo[s]);
  };
  auto mma_slab = [&](const Frag& f) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) Mfma<TIn>::run(f.w[j], f.a[i], acc[i][j]);
  };

  // Bias of a tile, loaded once per tile: tile 0's before the prologue, tile
  // i+1's right after tile i's epilogue stores (clamped to the last tile, so
  // the loads are unconditional).  The registers stay live until the next
  // epilogue, so the compiler never waits on them except before that first
  // use.  With buffer stores N % 4 == 0, so each 4-column group is one
  // aligned vector load with no branch on the bias type (groups past N read
  // the last group); otherwise each element's dword is loaded, clamped into
  // [0, N): byte (n+r)*4 (fp32) or ((n+r)*2) & ~3 (bf16, half by parity).
  uint32_t braw[TN][4];
  const int bshift = bias_bf16 ? 1 : 2;
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(bias), 0, EPI != CGPT_EPI_NONE ? N << bshift : 0, kBufferRsrcWord3);
  auto load_bias = [&](int i) {
    int tm, tn;
    tile_coords(static_cast<int>(blockIdx.x) + min(i, n_mine - 1) * static_cast<int>(gridDim.x),
                tiles_m, tiles_n, tm, tn);
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = tn * BN + wn0 + j * 16 + 4 * fgrp;
      if constexpr (BUFST) {
        // 16 bytes from the group's first element whatever the type (bf16
        // uses the first 8); bytes past the bias read as zero.
        const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rb, min(n, N - 4) << bshift, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) braw[j][r] = v[r];
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int idx = min(n + r, N - 1);
          braw[j][r] = *reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(bias) +
                                                          ((idx << bshift) & ~3));
        }
      }
    }
  };
  auto bias_at = [&](int j, int r, int n) -> float {
    if constexpr (BUFST) {
      if (!bias_bf16) return __uint_as_float(braw[j][r]);
      const uint32_t w = braw[j][r >> 1];
      return half_word<TIn>(w, (r & 1) != 0);
    } else {
      const uint32_t w = braw[j][r];
      if (!bias_bf16) return __uint_as_float(w);
      return half_word<TIn>(w, (min(n + r, N - 1) & 1) != 0);
    }
  };
  // Returns true when the tile took the buffer-store path, which issues exactly
  // TM * TN stores per wave (rows past M lie past the resource's size and
  // columns past N get an offset past it, so both are dropped), and the next
  // wait can leave them in flight.  Plain stores sit behind per-lane
  // conditions, so the next wait drains everything.
  auto epilogue = [&](int i) -> bool {
    int tm, tn;
    tile_coords(static_cast<int>(blockIdx.x) + i * static_cast<int>(gridDim.x), tiles_m, tiles_n,
                tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    if constexpr (WSTAGED) {
      // Per 16-row band: write the band (16-byte chunk c of row r at slot
      // c ^ (r & 7) of its 128-byte group), then WNQ stores of 64 consecutive
      // chunks each, i.e. 64 / WCPR whole rows of the wave's columns.  The
      // slot is private to the wave (LDS keeps one wave's accesses in order),
      // so no barrier is needed.  An opaque zero keeps the addresses inside
      // the tile loop (hoisted, they would stay live through every K step).
      int zero;
      asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
      uint8_t* sw = sout + wave * 16 * WROWB;
      auto spos = [](int r, int c) { return r * WROWB + (((c & ~7) | ((c & 7) ^ (r & 7))) << 4); };
      const int rows = min(BM, M - m0);
      const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
          C + static_cast<int64_t>(m0) * ldc, 0,
          static_cast<int>(static_cast<int64_t>(rows) * ldc * static_cast<int64_t>(sizeof(TOut))),
          kBufferRsrcWord3);
      const int lr = frow + zero, ll = lane + zero;
#pragma unroll
      for (int ii = 0; ii < TM; ++ii) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float t = acc[ii][j][r];
            if (EPI != CGPT_EPI_NONE) t += bias_at(j, r, 0);
            if (EPI == CGPT_EPI_BIAS_GELU) t = gelu_tanh(t);
            v[r] = t;
          }
          const int byte = (j * 16 + 4 * fgrp) * static_cast<int>(sizeof(TOut));
          uint8_t* dst = sw + spos(lr, byte >> 4) + (byte & 15);
          if constexpr (sizeof(TOut) == 4) {
            *reinterpret_cast<u32x4_t*>(dst) = u32x4_t{__float_as_uint(v[0]), __float_as_uint(v[1]),
                                                       __float_as_uint(v[2]), __float_as_uint(v[3])};
          } else {
            *reinterpret_cast<u32x2_t*>(dst) = u32x2_t{pack2<TOut>(v[0], v[1]), pack2<TOut>(v[2], v[3])};
          }
        }
#pragma unroll
        for (int q = 0; q < WNQ; ++q) {
          const int ch = q * 64 + ll;
          const int r = ch / WCPR, c = ch % WCPR;
          const u32x4_t d = *reinterpret_cast<const u32x4_t*>(sw + spos(r, c));
          const int col = n0 + wn0 + c * (16 / static_cast<int>(sizeof(TOut)));
          const uint32_t off =
              col < N ? static_cast<uint32_t>((static_cast<int64_t>(wm0 + ii * 16 + r) * ldc + col) *
                                              sizeof(TOut))
                      : 0x80000000u;
          __builtin_amdgcn_raw_buffer_store_b128(d, rc, off, 0, kStorePolicy);
        }
      }
      return true;
    } else if constexpr (BUFST) {
      const int rows = min(BM, M - m0);
      const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
          C + static_cast<int64_t>(m0) * ldc, 0,
          static_cast<int>(static_cast<int64_t>(rows) * ldc * static_cast<int64_t>(sizeof(TOut))),
          kBufferRsrcWord3);
      // Residual epilogue (C += A W^T + bias): every old C value of the tile
      // is loaded before the first is used (rows past M and columns past N
      // lie past the resource and read as zero; their stores are dropped).
      constexpr bool RES = EPI == CGPT_EPI_BIAS_RESID;
      static_assert(!RES || TM * TN <= 16, "residual epilogue: small tiles only");
      float cold[RES ? TM : 1][RES ? TN : 1][4];
      if constexpr (RES) {
#pragma unroll
        for (int ii = 0; ii < TM; ++ii) {
          const uint32_t roff = static_cast<uint32_t>((wm0 + ii * 16 + frow) * ldc);
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            const int n = n0 + wn0 + j * 16 + 4 * fgrp;
            const uint32_t off =
                n < N ? (roff + static_cast<uint32_t>(n)) * static_cast<uint32_t>(sizeof(TOut)) : 0x80000000u;
            if constexpr (sizeof(TOut) == 4) {
              const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rc, off, 0, 0);
#pragma unroll
              for (int r = 0; r < 4; ++r) cold[ii][j][r] = __uint_as_float(v[r]);
            } else {
              const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(rc, off, 0, 0);
              cold[ii][j][0] = half_word<TOut>(v[0], false);
              cold[ii][j][1] = half_word<TOut>(v[0], true);
              cold[ii][j][2] = half_word<TOut>(v[1], false);
              cold[ii][j][3] = half_word<TOut>(v[1], true);
            }
          }
        }
      }
#pragma unroll
      for (int ii = 0; ii < TM; ++ii) {
        const uint32_t roff = static_cast<uint32_t>((wm0 + ii * 16 + frow) * ldc);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int n = n0 + wn0 + j * 16 + 4 * fgrp;
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float t = acc[ii][j][r];
            if (EPI != CGPT_EPI_NONE) t += bias_at(j, r, n);
            if (EPI == CGPT_EPI_BIAS_GELU) t = gelu_tanh(t);
            if constexpr (RES) t += cold[ii][j][r];
            v[r] = t;
          }
          const uint32_t off =
              n < N ? (roff + static_cast<uint32_t>(n)) * static_cast<uint32_t>(sizeof(TOut)) : 0x80000000u;
          buffer_store4(rc, off, v, static_cast<TOut*>(nullptr));
        }
      }
      return true;
    }
#pragma unroll
    for (int ii = 0; ii < TM; ++ii) {
      const int mb = m0 + wm0 + ii * 16;
      const int m = mb + frow;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int nb = n0 + wn0 + j * 16;
        const int n = nb + 4 * fgrp;
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float t = acc[ii][j][r];
          if (EPI != CGPT_EPI_NONE) t += bias_at(j, r, n);
          if (EPI == CGPT_EPI_BIAS_GELU) t = gelu_tanh(t);
          if (EPI == CGPT_EPI_BIAS_RESID && m < M && n + r < N)
            t += Elem<TOut>::load(C + static_cast<int64_t>(m) * ldc + n + r);
          v[r] = t;
        }
        if (!vec_store) {
          store_block_remap(escr[wave], C, ldc, mb, nb, M, N, v, lane);
        } else if (m < M && n < N) {
          TOut* out = C + static_cast<int64_t>(m) * ldc + n;
          if (n + 3 < N) {
            store4_out(out, v);
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (n + r < N) Elem<TOut>::store(out + r, v[r]);
          }
        }
      }
    }
    return false;
  };

  Frag fr;
  // Memory operations a buffer-store epilogue issues: its stores and the next
  // tile's bias loads.
  constexpr int EPI_OPS = vm_cap((WSTAGED ? TM * WNQ : TM * TN) +
                                 (EPI != CGPT_EPI_NONE ? TN : 0));
  // Wait until stage `h` has landed: `later` stages issued after it may stay
  // in flight, and so may the exact EPI_OPS operations of a buffer-store
  // epilogue issued after them.
  auto wait_for = [&](int h, bool epi) {
    int later = total - 1 - h;
    later = later < STAGES - 2 ? later : STAGES - 2;
    wait_stages<LPS, STAGES - 2, EPI_OPS>(later, epi);
  };
  // Tile loop around a K-step loop, so the accumulators are zeroed at the top
  // of a tile and carried in place through its steps (no select between the
  // running sums and zero inside the step loop).  The DMA stream is flat:
  // step g (global over this block's tiles) reads stage buffer g % STAGES
  // and issues stage g + STAGES - 1, which may belong to the next tile.  Every
  // wave enters a step having waited for its own part of stage g; the
  // barrier makes all waves' parts visible.  After a tile's epilogue the wait
  // for the next stage runs in the same straight-line code as the stores, so
  // it can leave them in flight.
  set_offsets(0);
  if (EPI != CGPT_EPI_NONE) load_bias(0);
  int ib = 0;  // stage buffer the next issue fills
  auto next_buf = [](int b) { return b + 1 == STAGES ? 0 : b + 1; };
#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < total) {
      issue(smem + ib * STAGE);
      ib = next_buf(ib);
    }
  wait_for(0, false);
  int cb = 0, g = 0;  // stage buffer being read, flattened step
  for (int t = 0; t < n_mine; ++t) {
    zero_acc();
    for (int kt = 0; kt < KT; ++kt, ++g) {
      raw_barrier();
      if (g + STAGES - 1 < total) {
        issue(smem + ib * STAGE);
        ib = next_buf(ib);
      }
      const uint8_t* cur = smem + cb * STAGE;
#pragma unroll
      for (int s = 0; s < SPS; ++s) {
        read_slab(cur, s, fr);
        mma_slab(fr);
      }
      cb = next_buf(cb);
      if (kt + 1 < KT) wait_for(g + 1, false);
    }
    const bool buf = epilogue(t);
    if (EPI != CGPT_EPI_NONE) load_bias(t + 1);
    if (buf)
      wait_for(g, true);
    else
      wait_vmcnt<0>();
  }
#endif  // __HIP_DEVICE_COMPILE__
}

// The same persistent pipeline with the A (activation) operand fetched one
// step further ahead than W: A rotates through 3 LDS buffers, W through 2, and
// each step issues W(g+1) then A(g+2), so the A rows — most of an XCD's L2
// misses, since each A block is shared by 4 CUs of a round and each W block
// by 8 — get two steps to arrive.  k = 64 per stage (SPS 2).
template <int BM, int BN, int WGM, int WGN, int EPI, typename TOut, typename TIn = bf16_t>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_pipe_a3_kernel(
    const TIn* __restrict__ A, const TIn* __restrict__ W, const void* __restrict__ bias,
    bool bias_bf16, TOut* __restrict__ C, int M, int N, int K, int64_t lda, int64_t ldw,
    int64_t ldc, int tiles_m, int tiles_n, bool vec_store) {
  // The body uses AMDGPU-only types (buffer resources); the host pass only
  // needs the kernel's signature for its launch stub.
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int NT = 64 * WGM * WGN, NW = NT / 64;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int SPS = 2;
  constexpr int ROWB = 64 * SPS;           // bytes of K per LDS row per stage
  constexpr int CPR = ROWB / 16;           // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;            // rows filled by one wave DMA instruction
  constexpr int ABUF = BM * ROWB, WBUF = BN * ROWB;
  constexpr int A_INS = BM / (RPI * NW);
  constexpr int W_INS = BN / (RPI * NW);
  static_assert(BM % (RPI * NW) == 0 && BN % (RPI * NW) == 0, "tile/wave mismatch");
  static_assert(A_INS < 64, "vmcnt range");
  // A buffers 0..2, then W buffers 0..1 (the DMA writes them through M0, so
  // one array with computed offsets is all the compiler needs to see).
  __shared__ __attribute__((aligned(1024))) uint8_t smem[3 * ABUF + 2 * WBUF];

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm0 = (wave / WGN) * WM, wn0 = (wave % WGN) * WN;
  const int frow = lane & 15, fgrp = lane >> 4;
  const int lrow = lane / CPR, pchunk = lane % CPR;
  auto swz = [](int row) { return ROWB == 128 ? (row & 7) : ((row >> 1) & 3); };

  const u32x4_t ra = buffer_desc(A, static_cast<uint32_t>(static_cast<int64_t>(M) * lda * 2));
  const u32x4_t rw = buffer_desc(W, static_cast<uint32_t>(static_cast<int64_t>(N) * ldw * 2));

  const int n_tiles = tiles_m * tiles_n;
  const int KT = K / (32 * SPS);
  const int n_mine = (n_tiles - 1 - static_cast<int>(blockIdx.x)) / static_cast<int>(gridDim.x) + 1;
  const int total = n_mine * KT;

  // ---- issue side: one cursor per operand (A runs a stage ahead of W)
  int ia_i = 0, ia_kt = 0, iw_i = 0, iw_kt = 0;
  uint32_t aoff[A_INS], woff[W_INS];
  auto tile_of = [&](int i, int& tm, int& tn) {
    tile_coords(static_cast<int>(blockIdx.x) + i * static_cast<int>(gridDim.x), tiles_m, tiles_n,
                tm, tn);
  };
  auto set_a = [&](int i) {
    int tm, tn;
    tile_of(i, tm, tn);
#pragma unroll
    for (int ii = 0; ii < A_INS; ++ii) {
      const int row = (ii * NW + wave) * RPI + lrow;
      const int64_t g = min(tm * BM + row, M - 1);
      aoff[ii] = static_cast<uint32_t>(g * lda * 2 + ((pchunk ^ swz(row)) << 4));
    }
  };
  auto set_w = [&](int i) {
    int tm, tn;
    tile_of(i, tm, tn);
#pragma unroll
    for (int ii = 0; ii < W_INS; ++ii) {
      const int row = (ii * NW + wave) * RPI + lrow;
      const int64_t g = min(tn * BN + row, N - 1);
      woff[ii] = static_cast<uint32_t>(g * ldw * 2 + ((pchunk ^ swz(row)) << 4));
    }
  };
  auto issue_a = [&](int b) {
    uint8_t* buf = smem + b * ABUF;
#pragma unroll
    for (int ii = 0; ii < A_INS; ++ii)
      dma_lds16(ra, lds_addr(buf + (ii * NW + wave) * 1024), aoff[ii], ia_kt * ROWB);
    if (++ia_kt == KT) {
      ia_kt = 0;
      if (++ia_i < n_mine) set_a(ia_i);
    }
  };
  auto issue_w = [&](int b) {
    uint8_t* buf = smem + 3 * ABUF + b * WBUF;
#pragma unroll
    for (int ii = 0; ii < W_INS; ++ii)
      dma_lds16(rw, lds_addr(buf + (ii * NW + wave) * 1024), woff[ii], iw_kt * ROWB);
    if (++iw_kt == KT) {
      iw_kt = 0;
      if (++iw_i < n_mine) set_w(iw_i);
    }
  };

  // ---- compute side
  f32x4_t acc[TM][TN];
  auto zero_acc = [&]() {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  };
  // Byte offset of this lane's fragment row inside a stage, per slab.
  int xo[SPS];
#pragma unroll
  for (int s = 0; s < SPS; ++s) xo[s] = ((4 * s + fgrp) ^ swz(frow)) << 4;
  const int a_base = (wm0 + frow) * ROWB, w_base = (wn0 + frow) * ROWB;
  struct Frag {
    u32x4_t a[TM], w[TN];
  };
  auto read_slab = [&](const uint8_t* abuf, const uint8_t* wbuf, int s, Frag& f) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
      f.a[i] = *reinterpret_cast<const u32x4_t*>(abuf + a_base + i * 16 * ROWB + xo[s]);
#pragma unroll
    for (int j = 0; j < TN; ++j)
      f.w[j] = *reinterpret_cast<const u32x4_t*>(wbuf + w_base + j * 16 * ROWB + xo[s]);
  };
  auto mma_slab = [&](const Frag& f) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) Mfma<TIn>::run(f.w[j], f.a[i], acc[i][j]);
  };

  // Bias of a tile, loaded once per tile as in gemm_pipe_kernel (N % 4 == 0:
  // one 16-byte load per 4-column group, groups past N read the last group).
  uint32_t braw[TN][4];
  const int bshift = bias_bf16 ? 1 : 2;
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(bias), 0, EPI != CGPT_EPI_NONE ? N << bshift : 0, kBufferRsrcWord3);
  auto load_bias = [&](int i) {
    int tm, tn;
    tile_of(min(i, n_mine - 1), tm, tn);
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = tn * BN + wn0 + j * 16 + 4 * fgrp;
      const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rb, min(n, N - 4) << bshift, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) braw[j][r] = v[r];
    }
  };
  auto bias_at = [&](int j, int r) -> float {
    if (!bias_bf16) return __uint_as_float(braw[j][r]);
    const uint32_t w = braw[j][r >> 1];
    return half_word<TIn>(w, (r & 1) != 0);
  };
  // Exactly TM * TN buffer stores per wave: rows past M lie past the
  // resource's size and columns past N get an offset past it, so both are
  // dropped, and the next wait can leave the stores in flight.
  auto epilogue = [&](int i) {
    int tm, tn;
    tile_of(i, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int rows = min(BM, M - m0);
    const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
        C + static_cast<int64_t>(m0) * ldc, 0,
        static_cast<int>(static_cast<int64_t>(rows) * ldc * static_cast<int64_t>(sizeof(TOut))),
        kBufferRsrcWord3);
#pragma unroll
    for (int ii = 0; ii < TM; ++ii) {
      const uint32_t roff = static_cast<uint32_t>((wm0 + ii * 16 + frow) * ldc);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = n0 + wn0 + j * 16 + 4 * fgrp;
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float t = acc[ii][j][r];
          if (EPI != CGPT_EPI_NONE) t += bias_at(j, r);
          if (EPI == CGPT_EPI_BIAS_GELU) t = gelu_tanh(t);
          v[r] = t;
        }
        const uint32_t off =
            n < N ? (roff + static_cast<uint32_t>(n)) * static_cast<uint32_t>(sizeof(TOut)) : 0x80000000u;
        buffer_store4(rc, off, v, static_cast<TOut*>(nullptr));
      }
    }
  };

  Frag fr;
  // After step g: A(g+1) and W(g+1) must have landed; only A(g+2) (issued
  // last in step g) and the epilogue's stores and bias loads may stay in
  // flight.
  constexpr int EPI_OPS = TM * TN + (EPI != CGPT_EPI_NONE ? TN : 0);
  auto wait_next = [&](int g, bool epi) {
    wait_stages<A_INS, 1, EPI_OPS>(g + 2 < total ? 1 : 0, epi);
  };
  int ab = 0, wb = 0;  // buffers of stage g: A g % 3, W g % 2
  if (EPI != CGPT_EPI_NONE) load_bias(0);
  set_a(0);
  set_w(0);
  // Prologue: W(0), A(0), A(1); wait for W(0), A(0).
  if (total > 0) issue_w(0);
  if (total > 0) issue_a(0);
  if (total > 1) issue_a(1);
  wait_stages<A_INS, 1, EPI_OPS>(total > 1 ? 1 : 0, false);
  // Tile loop around the K-step loop (accumulators zeroed per tile, carried
  // in place), flat DMA stream as in gemm_pipe_kernel.
  int g = 0;
  for (int t = 0; t < n_mine; ++t) {
    zero_acc();
    for (int kt = 0; kt < KT; ++kt, ++g) {
      raw_barrier();
      if (g + 1 < total) issue_w(wb ^ 1);
      if (g + 2 < total) issue_a(ab == 0 ? 2 : ab - 1);
      const uint8_t* abuf = smem + ab * ABUF;
      const uint8_t* wbuf = smem + 3 * ABUF + wb * WBUF;
#pragma unroll
      for (int s = 0; s < SPS; ++s) {
        read_slab(abuf, wbuf, s, fr);
        mma_slab(fr);
      }
      ab = ab == 2 ? 0 : ab + 1;
      wb ^= 1;
      if (kt + 1 < KT) wait_next(g, false);
    }
    epilogue(t);
    if (EPI != CGPT_EPI_NONE) load_bias(t + 1);
    wait_next(g - 1, true);
  }
#endif  // __HIP_DEVICE_COMPILE__
}

// Two stages of k = 64 (2 k32 slabs each) with the LDS fragment reads
// software-pipelined one slab ahead of the MFMAs, so no MFMA waits for an LDS
// read it has just issued:
//   step g:  read slab 1 of stage g      | MFMAs of slab 0 of stage g
//            wait (own DMA of stage g+1, own reads of stage g), barrier,
//            DMA stage g+2 into stage g's buffer,
//            read slab 0 of stage g+1    | MFMAs of slab 1 of stage g
//            [last step of a tile: epilogue, next tile's bias]
// The barrier sits between the two slabs: once every wave has read all of
// stage g its buffer can be refilled.  Output rows are staged through LDS and
// stored as whole lines (requires 16-byte aligned rows and N a multiple of
// 16 bytes' worth of elements).
// Output stores are non-temporal: in the GPT-2 forward this took c_attn from
// 826 to 900 TFLOP/s and attn c_proj from 741 to 783, the attention that reads
// c_attn's output lost 7 %, and the forward gained 1.2 %.
//
// Residual epilogue (CGPT_EPI_BIAS_RESID, fp32 C: C += A W^T + bias, the
// residual stream of the model): the LDS that stages output rows otherwise
// is a ring of residual fragments instead.  Each wave owns 24 16 x 16 blocks
// of C (8 row blocks x 3 column blocks); the first 8 steps of a tile each add
// one row block's 3 blocks of C into the accumulators (zero at the tile's
// start), fetched two steps earlier by DMA in the accumulator layout (lane l's
// 16 bytes land at slot + 16 l, so a linear ds_read_b128 returns them), and
// the tile ends with direct buffer stores of the accumulators plus bias.  The
// C reads are thereby spread over the K loop instead of serialising an
// epilogue that would wait for them; requires K >= 512.
constexpr int kSlabStorePolicy = 2;
constexpr int kResidMinSteps = 8;  // k64 steps a tile needs for the residual ring

template <int BM, int BN, int WGM, int WGN, int EPI, typename TOut, typename TIn = bf16_t>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_slab_kernel(
    const TIn* __restrict__ A, const TIn* __restrict__ W, const void* __restrict__ bias,
    bool bias_bf16, TOut* __restrict__ C, int M, int N, int K, int64_t lda, int64_t ldw,
    int64_t ldc, int tiles_m, int tiles_n, bool vec_store) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int NT = 64 * WGM * WGN, NW = NT / 64;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int ROWB = 128, CPR = 8, RPI = 8;  // k = 64 per LDS row
  constexpr int STAGE = (BM + BN) * ROWB;
  constexpr int A_INS = BM / (RPI * NW), W_INS = BN / (RPI * NW);
  static_assert(BM % (RPI * NW) == 0 && BN % (RPI * NW) == 0, "tile/wave mismatch");
  // Output staging: the rest of the CU's LDS holds IIP 16-row bands of every
  // wave row (PASS_ROWS rows of the tile), written in the MFMA layout and read
  // back as consecutive 16-byte chunks of whole rows.
  constexpr int OUT_BYTES = 160 * 1024 - 2 * STAGE;
  constexpr int ROWB_O = BN * static_cast<int>(sizeof(TOut));  // bytes of one tile row
  constexpr int CPRO = ROWB_O / 16;                            // 16-byte chunks per row
  constexpr int IIP = OUT_BYTES / (WGM * 16 * ROWB_O);
  constexpr int PASS_ROWS = WGM * 16 * IIP;
  constexpr int CH_PER_T = PASS_ROWS * CPRO / NT;
  constexpr int NPASS = TM / IIP;
  static_assert(IIP >= 1 && TM % IIP == 0, "output staging bands");
  static_assert(PASS_ROWS * CPRO == CH_PER_T * NT, "whole chunks per thread");
  static_assert(CPRO % 8 == 0, "rows of whole 128-byte groups");
  constexpr bool RESID = EPI == CGPT_EPI_BIAS_RESID;
  static_assert(!RESID || (sizeof(TOut) == 4 && TM == kResidMinSteps && TN == 3 &&
                           NW * 2 * TN * 1024 <= OUT_BYTES),
                "residual ring: fp32 C, 8 x 3 blocks a wave, two slots of 3 KiB a wave");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t sout[OUT_BYTES];

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm0 = (wave / WGN) * WM, wn0 = (wave % WGN) * WN;
  const int frow = lane & 15, fgrp = lane >> 4;
  const int lrow = lane / CPR, pchunk = lane % CPR;

  const u32x4_t ra = buffer_desc(A, static_cast<uint32_t>(static_cast<int64_t>(M) * lda * 2));
  const u32x4_t rw = buffer_desc(W, static_cast<uint32_t>(static_cast<int64_t>(N) * ldw * 2));

  const int n_tiles = tiles_m * tiles_n;
  const int KT = K / 64;
  const int n_mine = (n_tiles - 1 - static_cast<int>(blockIdx.x)) / static_cast<int>(gridDim.x) + 1;
  const int total = n_mine * KT;
  auto tile_of = [&](int i, int& tm, int& tn) {
    tile_coords(static_cast<int>(blockIdx.x) + i * static_cast<int>(gridDim.x), tiles_m, tiles_n,
                tm, tn);
  };

  // ---- issue side (flat stage stream over this block's tiles)
  // Per-lane source offsets are set once and moved by a uniform delta at each
  // tile change.  Rows past M (or N) are not clamped: their offsets lie past
  // the resource's size, so the hardware returns zeros for them (such rows
  // are never stored); the launcher checks that these offsets fit 32 bits.
  int iss_i = 0, iss_kt = 0, iss_tm = 0, iss_tn = 0;
  uint32_t aoff[A_INS], woff[W_INS];
  {
    tile_of(0, iss_tm, iss_tn);
#pragma unroll
    for (int ii = 0; ii < A_INS; ++ii) {
      const int row = (ii * NW + wave) * RPI + lrow;
      aoff[ii] = static_cast<uint32_t>(static_cast<int64_t>(iss_tm * BM + row) * lda * 2 +
                                       ((pchunk ^ (row & 7)) << 4));
    }
#pragma unroll
    for (int ii = 0; ii < W_INS; ++ii) {
      const int row = (ii * NW + wave) * RPI + lrow;
      woff[ii] = static_cast<uint32_t>(static_cast<int64_t>(iss_tn * BN + row) * ldw * 2 +
                                       ((pchunk ^ (row & 7)) << 4));
    }
  }
  const uint32_t a_tile_bytes = static_cast<uint32_t>(BM * lda * 2);
  const uint32_t w_tile_bytes = static_cast<uint32_t>(BN * ldw * 2);
  auto set_offsets = [&](int i) {
    int tm, tn;
    tile_of(i, tm, tn);
    const uint32_t da = static_cast<uint32_t>(tm - iss_tm) * a_tile_bytes;
    const uint32_t dw = static_cast<uint32_t>(tn - iss_tn) * w_tile_bytes;
    iss_tm = tm;
    iss_tn = tn;
#pragma unroll
    for (int ii = 0; ii < A_INS; ++ii) aoff[ii] += da;
#pragma unroll
    for (int ii = 0; ii < W_INS; ++ii) woff[ii] += dw;
  };
  auto issue = [&](uint8_t* buf) {
    const int soff = iss_kt * ROWB;
#pragma unroll
    for (int ii = 0; ii < A_INS; ++ii)
      dma_lds16(ra, lds_addr(buf + (ii * NW + wave) * 1024), aoff[ii], soff);
#pragma unroll
    for (int ii = 0; ii < W_INS; ++ii)
      dma_lds16(rw, lds_addr(buf + BM * ROWB + (ii * NW + wave) * 1024), woff[ii], soff);
    if (++iss_kt == KT) {
      iss_kt = 0;
      if (++iss_i < n_mine) set_offsets(iss_i);
    }
  };

  // ---- residual ring (RESID): the C blocks of row block kt of a tile, for
  // the tile's step kt < TM, go to slot (flat step & 1) of this wave, fetched
  // at the middle of the step two flat steps earlier (the first two in the
  // prologue), so the wait that precedes every step's second half — which
  // leaves in flight at most an epilogue's stores and bias loads, issued after
  // them — has retired them one step before they are read.
  const u32x4_t rcres = buffer_desc(C, RESID ? static_cast<uint32_t>(
                                               static_cast<int64_t>(M) * ldc * 4) : 0u);
  uint8_t* const sres = sout + wave * (2 * TN * 1024);
  int res_t = 0, res_kt = 0;  // tile and step of the next fetch
  auto issue_res = [&]() {
    if (res_t < n_mine && res_kt < TM) {
      int tm, tn;
      tile_of(res_t, tm, tn);
      const int row = tm * BM + wm0 + res_kt * 16 + frow;
      const int col = tn * BN + wn0 + 4 * fgrp;
      const uint32_t base = static_cast<uint32_t>((static_cast<int64_t>(row) * ldc + col) * 4);
      uint8_t* slot = sres + ((res_t * KT + res_kt) & 1) * (TN * 1024);
#pragma unroll
      for (int j = 0; j < TN; ++j) dma_lds16(rcres, lds_addr(slot + j * 1024), base + j * 64, 0);
    }
    if (++res_kt == KT) {
      res_kt = 0;
      ++res_t;
    }
  };

  // ---- compute side
  f32x4_t acc[TM][TN];
  auto zero_acc = [&]() {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  };
  // Add row block kt's C blocks (slot of flat step g) into the accumulators.
  auto add_res = [&](int kt, int g) {
    if constexpr (RESID) {
      const uint8_t* slot = sres + (g & 1) * (TN * 1024) + lane * 16;
      f32x4_t r[TN];
#pragma unroll
      for (int j = 0; j < TN; ++j) r[j] = *reinterpret_cast<const f32x4_t*>(slot + j * 1024);
      switch (kt) {
#define CGPT_RES_ROW(i) \
  case i:               \
    for (int j = 0; j < TN; ++j) acc[i][j] += r[j]; \
    break;
        CGPT_RES_ROW(0) CGPT_RES_ROW(1) CGPT_RES_ROW(2) CGPT_RES_ROW(3)
        CGPT_RES_ROW(4) CGPT_RES_ROW(5) CGPT_RES_ROW(6) CGPT_RES_ROW(7)
#undef CGPT_RES_ROW
        default: break;
      }
    }
  };
  const int xo0 = (fgrp ^ (frow & 7)) << 4, xo1 = ((4 + fgrp) ^ (frow & 7)) << 4;
  const int a_base = (wm0 + frow) * ROWB, w_base = BM * ROWB + (wn0 + frow) * ROWB;
  struct Frag {
    u32x4_t a[TM], w[TN];
  };
  auto read_slab = [&](const uint8_t* buf, int xo, Frag& f) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
      f.a[i] = *reinterpret_cast<const u32x4_t*>(buf + a_base + i * 16 * ROWB + xo);
#pragma unroll
    for (int j = 0; j < TN; ++j)
      f.w[j] = *reinterpret_cast<const u32x4_t*>(buf + w_base + j * 16 * ROWB + xo);
  };
  auto mma_slab = [&](const Frag& f) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) Mfma<TIn>::run(f.w[j], f.a[i], acc[i][j]);
  };

  uint32_t braw[TN][4];
  const int bshift = bias_bf16 ? 1 : 2;
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(bias), 0, EPI != CGPT_EPI_NONE ? N << bshift : 0, kBufferRsrcWord3);
  auto load_bias = [&](int i) {
    int tm, tn;
    tile_of(min(i, n_mine - 1), tm, tn);
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = tn * BN + wn0 + j * 16 + 4 * fgrp;
      const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rb, min(n, N - 4) << bshift, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) braw[j][r] = v[r];
    }
  };
  auto bias_at = [&](int j, int r) -> float {
    if (!bias_bf16) return __uint_as_float(braw[j][r]);
    const uint32_t w = braw[j][r >> 1];
    return half_word<TIn>(w, (r & 1) != 0);
  };
  // Epilogue through LDS: each pass writes IIP row bands of every wave (bias
  // and GELU applied) into sout, barrier, then every thread stores CH_PER_T
  // consecutive 16-byte chunks of whole tile rows, so a wave's store covers
  // full 128-byte lines (the MFMA layout would give 16 rows x 32 or 64 bytes
  // per store).  16-byte chunk c of staged row r sits at slot c ^ (r & 7)
  // within its 128-byte group (conflict-free column writes and row reads).
  // Exactly NPASS * CH_PER_T stores per thread: rows past M fall outside the
  // resource, chunks past N get an offset past it.
  auto spos = [](int r, int c) { return r * ROWB_O + (((c & ~7) | ((c & 7) ^ (r & 7))) << 4); };
  const int wr = wave / WGN;
  auto epilogue = [&](int i) {
    int tm, tn;
    tile_of(i, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int rows = min(BM, M - m0);
    const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
        C + static_cast<int64_t>(m0) * ldc, 0,
        static_cast<int>(static_cast<int64_t>(rows) * ldc * static_cast<int64_t>(sizeof(TOut))),
        kBufferRsrcWord3);
    // An opaque zero defined here keeps the per-lane staging and store
    // addresses from being hoisted out of the tile loop, where they would
    // stay live (and spill) through every K step.
    int zero;
    asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
    if constexpr (RESID) {
      // Accumulators (C already added) plus bias, stored in place: exactly
      // TM * TN stores (rows past M lie past the resource, column groups past
      // N get an offset past it).
#pragma unroll
      for (int ii = 0; ii < TM; ++ii) {
        const uint32_t roff = static_cast<uint32_t>((wm0 + ii * 16 + frow + zero) * ldc);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int n = n0 + wn0 + j * 16 + 4 * fgrp;
          const u32x4_t d{__float_as_uint(acc[ii][j][0] + bias_at(j, 0)),
                          __float_as_uint(acc[ii][j][1] + bias_at(j, 1)),
                          __float_as_uint(acc[ii][j][2] + bias_at(j, 2)),
                          __float_as_uint(acc[ii][j][3] + bias_at(j, 3))};
          const uint32_t off = n < N ? (roff + static_cast<uint32_t>(n)) * 4u : 0x80000000u;
          __builtin_amdgcn_raw_buffer_store_b128(d, rc, off, 0, 0);
        }
      }
      return;
    }
    const int lt = tid + zero, lrw = frow + zero;
#pragma unroll
    for (int p = 0; p < NPASS; ++p) {
#pragma unroll
      for (int il = 0; il < IIP; ++il) {
        const int ii = p * IIP + il;
        const int r = (wr * IIP + il) * 16 + lrw;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          float v[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            float t = acc[ii][j][q];
            if (EPI != CGPT_EPI_NONE) t += bias_at(j, q);
            if (EPI == CGPT_EPI_BIAS_GELU) t = gelu_tanh(t);
            v[q] = t;
          }
          const int byte = (wn0 + j * 16 + 4 * fgrp) * static_cast<int>(sizeof(TOut));
          uint8_t* dst = sout + spos(r, byte >> 4) + (byte & 15);
          if constexpr (sizeof(TOut) == 4) {
            *reinterpret_cast<u32x4_t*>(dst) = u32x4_t{__float_as_uint(v[0]), __float_as_uint(v[1]),
                                                       __float_as_uint(v[2]), __float_as_uint(v[3])};
          } else {
            *reinterpret_cast<u32x2_t*>(dst) = u32x2_t{pack2<TOut>(v[0], v[1]), pack2<TOut>(v[2], v[3])};
          }
        }
      }
      wait_lgkm0();
      raw_barrier();
#pragma unroll
      for (int q = 0; q < CH_PER_T; ++q) {
        const int ch = lt + q * NT;
        const int r = ch / CPRO, c = ch % CPRO;
        const u32x4_t d = *reinterpret_cast<const u32x4_t*>(sout + spos(r, c));
        // Staged row r: wave row r / (16 IIP), band p * IIP + (r / 16) % IIP.
        const int grow = (r / (16 * IIP)) * WM + p * IIP * 16 + r % (16 * IIP);
        const int ncol = n0 + c * (16 / static_cast<int>(sizeof(TOut)));
        const uint32_t off = ncol < N ? static_cast<uint32_t>(
                                            (static_cast<int64_t>(grow) * ldc + ncol) * sizeof(TOut))
                                      : 0x80000000u;
        __builtin_amdgcn_raw_buffer_store_b128(d, rc, off, 0, kSlabStorePolicy);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (p + 1 < NPASS) {
        wait_lgkm0();
        raw_barrier();
      }
    }
  };

  // Memory operations an epilogue leaves in flight: its stores and the next
  // tile's bias loads (capped to the counter's range: a stronger wait).
  constexpr int EPI_OPS =
      vm_cap((RESID ? TM * TN : NPASS * CH_PER_T) + (EPI != CGPT_EPI_NONE ? TN : 0));
  Frag f0, f1;
  if (EPI != CGPT_EPI_NONE) load_bias(0);
  if (RESID) {
    issue_res();
    issue_res();
  }
  issue(smem);
  if (total > 1) {
    issue(smem + STAGE);
    wait_vmcnt<A_INS + W_INS>();
  } else {
    wait_vmcnt<0>();
  }
  raw_barrier();
  read_slab(smem, xo0, f0);
  int g = 0;
  for (int t = 0; t < n_mine; ++t) {
    zero_acc();
    for (int kt = 0; kt < KT; ++kt, ++g) {
      uint8_t* cur = smem + (g & 1) * STAGE;
      if (RESID && kt < TM) add_res(kt, g);
      read_slab(cur, xo1, f1);
      mma_slab(f0);
      if (g + 1 < total) {
        if (kt == 0 && t > 0)
          wait_vmcnt<EPI_OPS>();
        else
          wait_vmcnt<0>();
        raw_barrier();
        if (g + 2 < total) issue(cur);
        if (RESID) issue_res();
        // At a tile's last step the next slab is read after the epilogue,
        // so its fragments are not live across it.
        if (kt + 1 < KT) read_slab(smem + ((g + 1) & 1) * STAGE, xo0, f0);
      }
      mma_slab(f1);
    }
    epilogue(t);
    if (EPI != CGPT_EPI_NONE) load_bias(t + 1);
    if (g < total) read_slab(smem + (g & 1) * STAGE, xo0, f0);
  }
#endif  // __HIP_DEVICE_COMPILE__
}

// ---------------------------------------------------------------------------
// Tile tables.

struct TileCfg {
  int bm, bn, wgm, wgn;
};

// bf16 configurations (index = tile id for CGPT_BF16).
//   ids 0-4: register-staged double buffer (any K % 8), LDS 2*(BM+BN)*128 B
//   ids 5+ : direct-to-LDS pipeline, persistent (K % (32*SPS) == 0),
//            LDS STAGES*(BM+BN)*64*SPS B + 1088 B per wave
static const TileCfg kBf16Tiles[] = {
    {256, 256, 2, 2},  // 0
    {256, 128, 2, 2},  // 1
    {128, 128, 2, 2},  // 2
    {128, 64, 2, 2},   // 3
    {64, 64, 2, 2},    // 4
    {256, 256, 2, 4},  // 5: 8 waves (128x64), SPS 2, 2 stages, 128 KiB
    {256, 256, 2, 4},  // 6: 8 waves (128x64), SPS 1, 4 stages, 128 KiB
    {256, 192, 2, 4},  // 7: 8 waves (128x48), SPS 2, 2 stages, 112 KiB
    {256, 192, 4, 2},  // 8: 8 waves (64x96),  SPS 2, 2 stages, 112 KiB
    {256, 128, 4, 2},  // 9: 8 waves (64x64),  SPS 2, 3 stages, 144 KiB
    {128, 256, 2, 4},  // 10: 8 waves (64x64), SPS 2, 3 stages, 144 KiB
    {256, 128, 4, 2},  // 11: 8 waves (64x64), SPS 1, 6 stages, 144 KiB
    {256, 256, 2, 4},  // 12: 8 waves (128x64), A 3 buffers / W 2, 160 KiB
    {256, 192, 2, 4},  // 13: 8 waves (128x48), A 3 buffers / W 2, 144 KiB
    {256, 192, 2, 4},  // 14: 8 waves (128x48), fragment reads one slab ahead, 112 KiB
    {256, 256, 2, 4},  // 15: 8 waves (128x64), SPS 2, 2 stages, rows staged per wave, 160 KiB
    {256, 256, 2, 4},  // 16: 15 with non-temporal output stores
    {128, 128, 2, 2},  // 17: 4 waves (64x64),  SPS 2, 2 stages, 64 KiB
    {128, 64, 2, 2},   // 18: 4 waves (64x32),  SPS 2, 3 stages, 72 KiB
    {64, 64, 2, 2},    // 19: 4 waves (32x32),  SPS 2, 3 stages, 48 KiB
};
constexpr int kFirstPipeTile = 5;
static const int kPipeSps[] = {2, 1, 2, 2, 2, 2, 1, 2, 2, 2, 2, 2, 2, 2, 2};
// Pipelined tiles that also take the residual epilogue (few accumulators a
// lane, so the tile's old C values fit in registers beside them).
constexpr int kFirstSmallPipeTile = 17;
// fp32 configurations (index = tile id for CGPT_F32).
static const TileCfg kF32Tiles[] = {
    {128, 128, 2, 2},  // 0
    {64, 64, 2, 2},    // 1
};
constexpr int kNumBf16Tiles = sizeof(kBf16Tiles) / sizeof(kBf16Tiles[0]);
constexpr int kNumF32Tiles = sizeof(kF32Tiles) / sizeof(kF32Tiles[0]);

template <typename TIn, int BM, int BN, int WGM, int WGN, int EPI, typename TOut, bool EL = false>
static int launch_cfg(const void* a, const void* w, const void* bias, bool bias_bf16, void* c,
                      int M, int N, int K, int64_t lda, int64_t ldw, int64_t ldc, bool vec_store,
                      hipStream_t s) {
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = (N + BN - 1) / BN;
  const int64_t blocks = static_cast<int64_t>(tiles_m) * tiles_n;
  if (blocks > 0x7fffffff) return CGPT_ESHAPE;
  hipLaunchKernelGGL((gemm_kernel<TIn, BM, BN, WGM, WGN, EPI, TOut, EL>), dim3(static_cast<unsigned>(blocks)),
                     dim3(64 * WGM * WGN), 0, s, static_cast<const TIn*>(a),
                     static_cast<const TIn*>(w), bias, bias_bf16, static_cast<TOut*>(c), M, N, K,
                     lda, ldw, ldc, tiles_m, tiles_n, vec_store);
  return hip_status(hipGetLastError());
}

// Compute units of the current device (persistent grids launch as many blocks
// per CU as fit).  Cached per device id; concurrent first calls store the same
// value.
static int num_cus() {
  static std::atomic<int> cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Blocks for a persistent launch: one per tile, up to as many as fit on every
// CU at once — registers and LDS, from the runtime's occupancy query for that
// kernel, looked up on its first launch and kept in `occ`.  The 4-wave
// pipeline tiles fit two (128x128, 128x64) or three (64x64) blocks a CU, whose
// waves hide each other's memory waits (XL MLP c_proj with the residual add,
// 4096 x 1600 x 6400, 128x128 tiles: 134 -> 91 us); the 8-wave kernels fit one.
static int persistent_grid(const void* kernel, int threads, int64_t tiles, std::atomic<int>& occ) {
  int n = occ.load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, 0) != hipSuccess || n < 1)
      n = 1;
    occ.store(n, std::memory_order_relaxed);
  }
  const int64_t cap = static_cast<int64_t>(n) * num_cus();
  return static_cast<int>(tiles < cap ? tiles : cap);
}

// WSO: 0 = buffer (or plain) stores, else the wave-staged output mode to use
// where the output allows it (kOutWaveStaged or kOutWaveStagedNT).
template <int BM, int BN, int WGM, int WGN, int SPS, int STAGES, int EPI, typename TOut,
          int WSO = 0, typename TIn = bf16_t>
static int launch_pipe(const void* a, const void* w, const void* bias, bool bias_bf16, void* c,
                       int M, int N, int K, int64_t lda, int64_t ldw, int64_t ldc, bool vec_store,
                       hipStream_t s) {
  constexpr int kStages = STAGES * (BM + BN) * 64 * SPS;
  static_assert(kStages + (WGM * WGN) * kScrFloats * 4 <= 160 * 1024, "LDS budget of one CU");
  constexpr int kWaveRowB = BN / WGN * static_cast<int>(sizeof(TOut));
  static_assert(WSO == 0 || (kStages + 16 * kWaveRowB * WGM * WGN <= 160 * 1024 &&
                                 kWaveRowB % 128 == 0),
                "wave-staged output: LDS budget and whole lines per wave row");
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = (N + BN - 1) / BN;
  const int64_t tiles = static_cast<int64_t>(tiles_m) * tiles_n;
  if (tiles > 0x7fffffff) return CGPT_ESHAPE;
  constexpr int kThreads = 64 * WGM * WGN;
  // Buffer-resource stores write whole 4-column groups and address one tile's
  // rows with 31-bit byte offsets; staged stores write whole 16-byte chunks.
  const bool buf_store = vec_store && N % 4 == 0 &&
                         static_cast<int64_t>(BM) * ldc * static_cast<int64_t>(sizeof(TOut)) < 0x7fffffff;
  constexpr int EPC = 16 / static_cast<int>(sizeof(TOut));
  const bool staged = WSO != 0 && buf_store && N % EPC == 0 && ldc % EPC == 0 &&
                      reinterpret_cast<uintptr_t>(c) % 16 == 0;
  if constexpr (WSO != 0) {
    if (staged) {
      static std::atomic<int> occ{0};
      const int grid = persistent_grid(
          reinterpret_cast<const void*>(&gemm_pipe_kernel<BM, BN, WGM, WGN, SPS, STAGES, EPI, TOut, WSO, TIn>),
          kThreads, tiles, occ);
      hipLaunchKernelGGL((gemm_pipe_kernel<BM, BN, WGM, WGN, SPS, STAGES, EPI, TOut, WSO, TIn>),
                         dim3(grid), dim3(kThreads), 0, s, static_cast<const TIn*>(a),
                         static_cast<const TIn*>(w), bias, bias_bf16, static_cast<TOut*>(c), M,
                         N, K, lda, ldw, ldc, tiles_m, tiles_n, vec_store);
      return hip_status(hipGetLastError());
    }
  }
  if (buf_store) {
    static std::atomic<int> occ{0};
    const int grid = persistent_grid(
        reinterpret_cast<const void*>(&gemm_pipe_kernel<BM, BN, WGM, WGN, SPS, STAGES, EPI, TOut, kOutBuffer, TIn>),
        kThreads, tiles, occ);
    hipLaunchKernelGGL((gemm_pipe_kernel<BM, BN, WGM, WGN, SPS, STAGES, EPI, TOut, kOutBuffer, TIn>), dim3(grid),
                       dim3(kThreads), 0, s, static_cast<const TIn*>(a),
                       static_cast<const TIn*>(w), bias, bias_bf16, static_cast<TOut*>(c), M, N,
                       K, lda, ldw, ldc, tiles_m, tiles_n, vec_store);
  } else {
    static std::atomic<int> occ{0};
    const int grid = persistent_grid(
        reinterpret_cast<const void*>(&gemm_pipe_kernel<BM, BN, WGM, WGN, SPS, STAGES, EPI, TOut, kOutPlain, TIn>),
        kThreads, tiles, occ);
    hipLaunchKernelGGL((gemm_pipe_kernel<BM, BN, WGM, WGN, SPS, STAGES, EPI, TOut, kOutPlain, TIn>), dim3(grid),
                       dim3(kThreads), 0, s, static_cast<const TIn*>(a),
                       static_cast<const TIn*>(w), bias, bias_bf16, static_cast<TOut*>(c), M, N,
                       K, lda, ldw, ldc, tiles_m, tiles_n, vec_store);
  }
  return hip_status(hipGetLastError());
}

// A fetched two steps ahead (3 A buffers, 2 W buffers, k = 64 per stage).  It
// only has the buffer-store epilogue; other output layouts take the two-stage
// kernel of the same tile.
template <int BM, int BN, int WGM, int WGN, int EPI, typename TOut, typename TIn = bf16_t>
static int launch_pipe_a3(const void* a, const void* w, const void* bias, bool bias_bf16, void* c,
                          int M, int N, int K, int64_t lda, int64_t ldw, int64_t ldc,
                          bool vec_store, hipStream_t s) {
  static_assert((3 * BM + 2 * BN) * 128 <= 160 * 1024, "LDS budget of one CU");
  const bool buf_store = vec_store && N % 4 == 0 &&
                         static_cast<int64_t>(BM) * ldc * static_cast<int64_t>(sizeof(TOut)) < 0x7fffffff;
  if (!buf_store)
    return launch_pipe<BM, BN, WGM, WGN, 2, 2, EPI, TOut, 0, TIn>(a, w, bias, bias_bf16, c, M, N, K,
                                                                  lda, ldw, ldc, vec_store, s);
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = (N + BN - 1) / BN;
  const int64_t tiles = static_cast<int64_t>(tiles_m) * tiles_n;
  if (tiles > 0x7fffffff) return CGPT_ESHAPE;
  const int grid = static_cast<int>(tiles < num_cus() ? tiles : num_cus());
  hipLaunchKernelGGL((gemm_pipe_a3_kernel<BM, BN, WGM, WGN, EPI, TOut, TIn>), dim3(grid),
                     dim3(64 * WGM * WGN), 0, s, static_cast<const TIn*>(a),
                     static_cast<const TIn*>(w), bias, bias_bf16, static_cast<TOut*>(c), M, N,
                     K, lda, ldw, ldc, tiles_m, tiles_n, vec_store);
  return hip_status(hipGetLastError());
}

// Slab-pipelined kernel (whole-line staged stores only; other output layouts
// take the two-stage pipeline kernel of the same tile).  Its source offsets
// are not clamped to the last row, so a whole tile past M (or N) must still
// address below 4 GiB.
template <int BM, int BN, int WGM, int WGN, int EPI, typename TOut, typename TIn = bf16_t>
static int launch_slab(const void* a, const void* w, const void* bias, bool bias_bf16, void* c,
                       int M, int N, int K, int64_t lda, int64_t ldw, int64_t ldc, bool vec_store,
                       hipStream_t s) {
  if ((static_cast<int64_t>(M) + BM) * lda * 2 >= (int64_t{1} << 32) ||
      (static_cast<int64_t>(N) + BN) * ldw * 2 >= (int64_t{1} << 32) ||
      static_cast<int64_t>(BM) * lda * 2 >= (int64_t{1} << 31) ||
      static_cast<int64_t>(BN) * ldw * 2 >= (int64_t{1} << 31))
    return launch_pipe<BM, BN, WGM, WGN, 2, 2, EPI, TOut, 0, TIn>(a, w, bias, bias_bf16, c, M, N, K,
                                                                  lda, ldw, ldc, vec_store, s);
  static_assert(2 * (BM + BN) * 128 < 160 * 1024, "LDS budget of one CU");
  // Whole 16-byte chunks: N and ldc multiples of 16 bytes' worth of elements
  // and a 16-byte aligned C (vec_store guarantees only 8 bytes for bf16).
  constexpr int EPC = 16 / static_cast<int>(sizeof(TOut));
  const bool buf_store = vec_store && N % EPC == 0 && ldc % EPC == 0 &&
                         reinterpret_cast<uintptr_t>(c) % 16 == 0 &&
                         static_cast<int64_t>(BM) * ldc * static_cast<int64_t>(sizeof(TOut)) < 0x7fffffff;
  if (!buf_store)
    return launch_pipe<BM, BN, WGM, WGN, 2, 2, EPI, TOut, 0, TIn>(a, w, bias, bias_bf16, c, M, N, K,
                                                                  lda, ldw, ldc, vec_store, s);
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = (N + BN - 1) / BN;
  const int64_t tiles = static_cast<int64_t>(tiles_m) * tiles_n;
  if (tiles > 0x7fffffff) return CGPT_ESHAPE;
  const int grid = static_cast<int>(tiles < num_cus() ? tiles : num_cus());
  hipLaunchKernelGGL((gemm_slab_kernel<BM, BN, WGM, WGN, EPI, TOut, TIn>), dim3(grid),
                     dim3(64 * WGM * WGN), 0, s, static_cast<const TIn*>(a),
                     static_cast<const TIn*>(w), bias, bias_bf16, static_cast<TOut*>(c), M, N,
                     K, lda, ldw, ldc, tiles_m, tiles_n, vec_store);
  return hip_status(hipGetLastError());
}

// Weight prefetch.  A persistent launch whose weight matrix is much larger
// than an XCD's L2 (the LM heads: 50 257 x d_model) has every XCD sweep all
// of W once per 8 tile rows, all eight XCDs at about the same column band at
// the same time; when W has not been read recently the first touch of each
// band comes from HBM at the start of a round and stalls the two-stage
// pipeline.  Reading W once just before the GEMM leaves it in the 256 MiB
// memory-side cache (MALL), from which all later band fetches are served.
// The loads feed an empty asm so they are kept; nothing is stored.
__global__ __launch_bounds__(256) void prefetch_kernel(const uint4* __restrict__ p, int64_t n) {
  uint32_t x = 0;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride) {
    const uint4 v = p[i];
    x ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  asm volatile("" ::"v"(x));
}

constexpr int64_t kPrefetchMinBytes = int64_t{32} << 20;  // W bytes that trigger it
constexpr int kPrefetchMinTileRows = 4;                     // 256-row tile bands of A

// Reads W (rows 0..N-1 of ldw bf16 elements, 16-byte aligned) ahead of a
// persistent GEMM launch on the same stream when it is worth it.
static int maybe_prefetch_w(const void* w, int64_t M, int64_t N, int64_t K, int64_t ldw,
                            hipStream_t s) {
  const int64_t bytes = ((N - 1) * ldw + K) * 2;
  if (bytes < kPrefetchMinBytes || M < kPrefetchMinTileRows * 256 ||
      reinterpret_cast<uintptr_t>(w) % 16 != 0)
    return CGPT_OK;
  const int64_t n = bytes / 16;  // whole 16-byte vectors inside W's extent
  hipLaunchKernelGGL(prefetch_kernel, dim3(2048), dim3(256), 0, s,
                     static_cast<const uint4*>(w), n);
  return hip_status(hipGetLastError());
}

// The pipelined kernels address A and W through 32-bit buffer offsets and
// consume K in whole stages.
static bool pipe_ok(int tile, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldw) {
  const int sps = kPipeSps[tile - kFirstPipeTile];
  return K % (32 * sps) == 0 && M * lda * 2 < 0x7fffffff && N * ldw * 2 < 0x7fffffff;
}

template <typename TIn, int EPI, typename TOut>
static int launch_tile(int tile, const void* a, const void* w, const void* bias, bool bias_bf16,
                       void* c, int M, int N, int K, int64_t lda, int64_t ldw, int64_t ldc,
                       bool vec_store, hipStream_t s) {
#define CGPT_GEMM_CASE(id, BM, BN, WGM, WGN)                                                   \
  case id:                                                                                    \
    return launch_cfg<TIn, BM, BN, WGM, WGN, EPI, TOut>(a, w, bias, bias_bf16, c, M, N, K, lda, \
                                                        ldw, ldc, vec_store, s);
#define CGPT_PIPE_CASE(id, BM, BN, WGM, WGN, SPS, ST)                                           \
  case id:                                                                                      \
    return launch_pipe<BM, BN, WGM, WGN, SPS, ST, EPI, TOut, 0, TIn>(a, w, bias, bias_bf16, c, M, \
                                                                     N, K, lda, ldw, ldc,         \
                                                                     vec_store, s);
  if constexpr (sizeof(TIn) == 2) {
    switch (tile) {
      CGPT_GEMM_CASE(0, 256, 256, 2, 2)
      CGPT_GEMM_CASE(1, 256, 128, 2, 2)
      CGPT_GEMM_CASE(2, 128, 128, 2, 2)
      CGPT_GEMM_CASE(3, 128, 64, 2, 2)
      CGPT_GEMM_CASE(4, 64, 64, 2, 2)
      CGPT_PIPE_CASE(5, 256, 256, 2, 4, 2, 2)
      CGPT_PIPE_CASE(6, 256, 256, 2, 4, 1, 4)
      CGPT_PIPE_CASE(7, 256, 192, 2, 4, 2, 2)
      CGPT_PIPE_CASE(8, 256, 192, 4, 2, 2, 2)
      CGPT_PIPE_CASE(9, 256, 128, 4, 2, 2, 3)
      CGPT_PIPE_CASE(10, 128, 256, 2, 4, 2, 3)
      CGPT_PIPE_CASE(11, 256, 128, 4, 2, 1, 6)
      case 12:
        return launch_pipe_a3<256, 256, 2, 4, EPI, TOut, TIn>(a, w, bias, bias_bf16, c, M, N, K, lda,
                                                         ldw, ldc, vec_store, s);
      case 13:
        return launch_pipe_a3<256, 192, 2, 4, EPI, TOut, TIn>(a, w, bias, bias_bf16, c, M, N, K, lda,
                                                         ldw, ldc, vec_store, s);
      case 14:
        return launch_slab<256, 192, 2, 4, EPI, TOut, TIn>(a, w, bias, bias_bf16, c, M, N, K, lda, ldw,
                                                      ldc, vec_store, s);
      case 15:
        return launch_pipe<256, 256, 2, 4, 2, 2, EPI, TOut, kOutWaveStaged, TIn>(
            a, w, bias, bias_bf16, c, M, N, K, lda, ldw, ldc, vec_store, s);
      case 16:
        return launch_pipe<256, 256, 2, 4, 2, 2, EPI, TOut, kOutWaveStagedNT, TIn>(
            a, w, bias, bias_bf16, c, M, N, K, lda, ldw, ldc, vec_store, s);
      CGPT_PIPE_CASE(17, 128, 128, 2, 2, 2, 2)
      CGPT_PIPE_CASE(18, 128, 64, 2, 2, 2, 3)
      CGPT_PIPE_CASE(19, 64, 64, 2, 2, 2, 3)
      default: return CGPT_EINVAL;
    }
  } else {
    switch (tile) {
      CGPT_GEMM_CASE(0, 128, 128, 2, 2)
      CGPT_GEMM_CASE(1, 64, 64, 2, 2)
      default: return CGPT_EINVAL;
    }
  }
#undef CGPT_PIPE_CASE
#undef CGPT_GEMM_CASE
}

// The largest 4-wave pipeline tile that gives the CUs at least 1.5 tiles each
// (their blocks run two or three a CU), else 64x64; -1 when K or the offsets
// rule the pipeline out.  Residual projections measured with each: XL
// 4096 x 1600 x 6400 128x128 91 / 128x64 112 / 64x64 138 us, 4096 x 1600 x
// 1600 33 / 38 / 41 us (the slab's 144 tiles: 123 and 43 us); medium
// 4096 x 512 x 2048 26 / 20 / 17 us.
static int small_pipe_tile(int M, int N, int K, int64_t lda, int64_t ldw) {
  constexpr int kIds[3] = {17, 18, 19}, kBm[3] = {128, 128, 64}, kBn[3] = {128, 64, 64};
  const int64_t cus = num_cus();
  int fallback = -1;
  for (int i = 0; i < 3; ++i) {
    if (!pipe_ok(kIds[i], M, N, K, lda, ldw)) continue;
    const int64_t t = static_cast<int64_t>((M + kBm[i] - 1) / kBm[i]) * ((N + kBn[i] - 1) / kBn[i]);
    if (2 * t >= 3 * cus) return kIds[i];
    fallback = kIds[i];
  }
  return fallback;
}

// Default tile choice when the caller's table has no entry: the register-staged
// kernel with the largest tile that still gives every CU about two blocks
// (128x128 for long K, 128x64 otherwise), smaller tiles for small grids.
static int auto_tile(bool half, int M, int N, int K, int64_t lda, int64_t ldw, int epi) {
  // 16-bit (bf16 / fp16) problems with at least one 256x192 tile per CU: the persistent
  // direct-to-LDS pipelines — 256x256 with wave-staged non-temporal stores
  // for wide N (the LM heads) and for the GELU epilogue; 256x192 with
  // block-staged stores otherwise.  With fewer tiles than CUs, a 4-wave
  // pipeline tile (several blocks a CU; medium's 4096 x 2048 x 512 c_fc:
  // 15.7 us against 17.3 for 256x128), else the persistent 256x192, 256x128
  // or 128x256 tile whose last round leaves the fewest CUs idle (ties to the
  // larger tile), as long as it still gives half the CUs a tile; below that
  // the register-staged kernel with smaller tiles.
  if (half) {
    auto tiles = [&](int bm, int bn) {
      return static_cast<int64_t>((M + bm - 1) / bm) * ((N + bn - 1) / bn);
    };
    const int cus = num_cus();
    const int64_t t14 = tiles(256, 192);
    if (t14 >= cus) {
      const int pick = (N >= 16384 || epi == CGPT_EPI_BIAS_GELU) ? 16 : 14;
      if (pipe_ok(pick, M, N, K, lda, ldw)) return pick;
    } else {
      const int small = small_pipe_tile(M, N, K, lda, ldw);
      if (small >= 0) return small;
      const int64_t cand_t[3] = {t14, tiles(256, 128), tiles(128, 256)};
      const int cand_id[3] = {14, 9, 10};
      int best = -1;
      double best_util = 0.0;
      for (int i = 0; i < 3; ++i) {
        const int64_t rounds = (cand_t[i] + cus - 1) / cus;
        const double util = static_cast<double>(cand_t[i]) / static_cast<double>(rounds * cus);
        if (cand_t[i] * 2 >= cus && util > best_util + 1e-9 && pipe_ok(cand_id[i], M, N, K, lda, ldw)) {
          best = cand_id[i];
          best_util = util;
        }
      }
      if (best >= 0) return best;
    }
  }
  const TileCfg* t = half ? kBf16Tiles : kF32Tiles;
  const int nt = half ? kNumBf16Tiles : kNumF32Tiles;
  const int first = half ? (K >= 2048 ? 2 : 3) : 0;
  const int last = half ? kFirstPipeTile - 1 : nt - 1;
  for (int i = first; i <= last; ++i) {
    const int64_t blocks =
        static_cast<int64_t>((M + t[i].bm - 1) / t[i].bm) * ((N + t[i].bn - 1) / t[i].bn);
    if (blocks >= 512) return i;
  }
  return last;
}

// Residual epilogue (C += A W^T + bias).  `tile`: 14 = the slab kernel's
// residual ring (16-bit inputs into fp32 C, at least 8 k64 steps, whole
// 4-column groups, 32-bit offsets; otherwise as TILE_AUTO); 17-19 = that
// small pipeline tile (16-bit inputs, K % 64 == 0; otherwise as TILE_AUTO); a
// register-staged tile id (bf16 / fp16 0-4, fp32 0-1) = that tile; anything
// else = TILE_AUTO: the slab kernel when its 256x192 tiles give every CU a
// tile, else the largest 4-wave pipeline tile (128x128, 128x64, 64x64) with
// at least 1.5 tiles a CU, else 64x64 (16-bit inputs, K % 64 == 0), else the
// register-staged tile the library's heuristic gives (the largest with 512
// blocks, 64x64 below that).
template <typename TIn, int EPI, typename TOut>
static int launch_small_pipe(int tile, const void* a, const void* w, const void* bias,
                             bool bias_bf16, void* c, int M, int N, int K, int64_t lda,
                             int64_t ldw, int64_t ldc, bool vec_store, hipStream_t s) {
  switch (tile) {
    case 17:
      return launch_pipe<128, 128, 2, 2, 2, 2, EPI, TOut, 0, TIn>(a, w, bias, bias_bf16, c, M, N, K,
                                                                  lda, ldw, ldc, vec_store, s);
    case 18:
      return launch_pipe<128, 64, 2, 2, 2, 3, EPI, TOut, 0, TIn>(a, w, bias, bias_bf16, c, M, N, K,
                                                                 lda, ldw, ldc, vec_store, s);
    default:
      return launch_pipe<64, 64, 2, 2, 2, 3, EPI, TOut, 0, TIn>(a, w, bias, bias_bf16, c, M, N, K,
                                                                lda, ldw, ldc, vec_store, s);
  }
}

template <typename TIn, typename TOut>
static int launch_resid(int req_tile, const void* a, const void* w, const void* bias,
                        bool bias_bf16, void* c, int M, int N, int K, int64_t lda, int64_t ldw,
                        int64_t ldc, bool vec_store, hipStream_t s) {
  constexpr int EPI = CGPT_EPI_BIAS_RESID;
  const int last = sizeof(TIn) == 2 ? kFirstPipeTile - 1 : kNumF32Tiles - 1;
  const bool reg_tile = req_tile >= 0 && req_tile <= last;
  if constexpr (sizeof(TIn) == 2) {
    if (req_tile >= kFirstSmallPipeTile && req_tile < kNumBf16Tiles &&
        pipe_ok(req_tile, M, N, K, lda, ldw))
      return launch_small_pipe<TIn, EPI, TOut>(req_tile, a, w, bias, bias_bf16, c, M, N, K, lda,
                                               ldw, ldc, vec_store, s);
  }
  if constexpr (sizeof(TIn) == 2 && sizeof(TOut) == 4) {
    const int64_t m = M, n = N;
    const int tiles_m = (M + 255) / 256, tiles_n = (N + 191) / 192;
    const int64_t tiles = static_cast<int64_t>(tiles_m) * tiles_n;
    const bool want = req_tile == 14 || (!reg_tile && tiles >= num_cus());
    if (want && K % 64 == 0 && K / 64 >= kResidMinSteps && n % 4 == 0 && ldc % 4 == 0 &&
        reinterpret_cast<uintptr_t>(c) % 16 == 0 && (m + 256) * ldc * 4 < (int64_t{1} << 32) &&
        (m + 256) * lda * 2 < (int64_t{1} << 32) && (n + 192) * ldw * 2 < (int64_t{1} << 32) &&
        256 * ldc * 4 < 0x7fffffff) {
      if (tiles > 0x7fffffff) return CGPT_ESHAPE;
      const int grid = static_cast<int>(tiles < num_cus() ? tiles : num_cus());
      hipLaunchKernelGGL((gemm_slab_kernel<256, 192, 2, 4, EPI, float, TIn>), dim3(grid), dim3(512),
                         0, s, static_cast<const TIn*>(a), static_cast<const TIn*>(w), bias,
                         bias_bf16, static_cast<float*>(c), M, N, K, lda, ldw, ldc, tiles_m,
                         tiles_n, vec_store);
      return hip_status(hipGetLastError());
    }
  }
  // Fewer slab tiles than CUs: a 4-wave pipeline tile where K allows it
  // (medium's 4096x512 projections: 13.0 -> 7.8 and 29.2 -> 16.9 us against
  // the 64x64 register tile).
  if constexpr (sizeof(TIn) == 2) {
    const int pick = reg_tile ? -1 : small_pipe_tile(M, N, K, lda, ldw);
    if (pick >= 0)
      return launch_small_pipe<TIn, EPI, TOut>(pick, a, w, bias, bias_bf16, c, M, N, K, lda, ldw,
                                               ldc, vec_store, s);
  }
  const TileCfg* t = sizeof(TIn) == 2 ? kBf16Tiles : kF32Tiles;
  const int first = sizeof(TIn) == 2 ? (K >= 2048 ? 2 : 3) : 0;
  int tile = last;
  if (reg_tile) {
    tile = req_tile;
  } else {
    for (int i = first; i <= last; ++i) {
      if (static_cast<int64_t>((M + t[i].bm - 1) / t[i].bm) * ((N + t[i].bn - 1) / t[i].bn) >=
          512) {
        tile = i;
        break;
      }
    }
  }
#define CGPT_RES_CFG(id, BM, BN)                                                                  \
  case id:                                                                                        \
    return launch_cfg<TIn, BM, BN, 2, 2, EPI, TOut>(a, w, bias, bias_bf16, c, M, N, K, lda, ldw,  \
                                                     ldc, vec_store, s);
  if constexpr (sizeof(TIn) == 2) {
    switch (tile) {
      CGPT_RES_CFG(0, 256, 256)
      CGPT_RES_CFG(1, 256, 128)
      CGPT_RES_CFG(2, 128, 128)
      CGPT_RES_CFG(3, 128, 64)
      default: CGPT_RES_CFG(4, 64, 64)
    }
  } else {
    switch (tile) {
      CGPT_RES_CFG(0, 128, 128)
      default: CGPT_RES_CFG(1, 64, 64)
    }
  }
#undef CGPT_RES_CFG
}

template <typename TIn, typename TOut>
static int launch_epi(int epi, int tile, const void* a, const void* w, const void* bias,
                      bool bias_bf16, void* c, int M, int N, int K, int64_t lda, int64_t ldw,
                      int64_t ldc, bool vec_store, bool elem_loads, hipStream_t s) {
  if (elem_loads) {
    // Any K, stride or alignment: the register-staged 64x64 tile with element
    // loads, every epilogue (the residual one included).
#define CGPT_EL_CASE(E)                                                                         \
  case E:                                                                                       \
    return launch_cfg<TIn, 64, 64, 2, 2, E, TOut, true>(a, w, bias, bias_bf16, c, M, N, K, lda, \
                                                        ldw, ldc, vec_store, s);
    switch (epi) {
      CGPT_EL_CASE(CGPT_EPI_NONE)
      CGPT_EL_CASE(CGPT_EPI_BIAS)
      CGPT_EL_CASE(CGPT_EPI_BIAS_GELU)
      CGPT_EL_CASE(CGPT_EPI_BIAS_RESID)
      default: return CGPT_EINVAL;
    }
#undef CGPT_EL_CASE
  }
  switch (epi) {
    case CGPT_EPI_BIAS_RESID:
      return launch_resid<TIn, TOut>(tile, a, w, bias, bias_bf16, c, M, N, K, lda, ldw, ldc,
                                     vec_store, s);
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

namespace cgpt {
// Argument checks shared by the GEMM entry points: CGPT_OK when the problem is
// well formed (M == 0 or N == 0 included: nothing to launch).
int validate_gemm(const void* a, const void* w, const void* bias, const void* c, int64_t M,
                  int64_t N, int64_t K, int64_t lda, int64_t ldw, int64_t ldc, int in_dtype,
                  int bias_dtype, int out_dtype, int epilogue, bool* elem_loads) {
  if (M < 0 || N < 0 || K < 0) return CGPT_EINVAL;
  if (M == 0 || N == 0) return CGPT_OK;
  if (M > 0x7fffffff || N > 0x7fffffff || K > 0x7fffffff) return CGPT_ESHAPE;
  if (a == nullptr || w == nullptr || c == nullptr) return CGPT_EINVAL;
  if (epilogue != CGPT_EPI_NONE && epilogue != CGPT_EPI_BIAS && epilogue != CGPT_EPI_BIAS_GELU &&
      epilogue != CGPT_EPI_BIAS_RESID)
    return CGPT_EINVAL;
  if (epilogue != CGPT_EPI_NONE && bias == nullptr) return CGPT_EINVAL;
  const bool f16 = in_dtype == CGPT_F16 && elem_loads != nullptr;
  if (in_dtype != CGPT_F32 && in_dtype != CGPT_BF16 && !f16) return CGPT_EDTYPE;
  // Outputs and bias: fp32, or the 16-bit type of the inputs' family (fp16
  // with fp16 inputs, bf16 otherwise).
  const int half = f16 ? CGPT_F16 : CGPT_BF16;
  if (out_dtype != CGPT_F32 && out_dtype != half) return CGPT_EDTYPE;
  if (epilogue != CGPT_EPI_NONE && bias_dtype != CGPT_F32 && bias_dtype != half)
    return CGPT_EDTYPE;
  if (K == 0) return CGPT_ESHAPE;
  if (lda < K || ldw < K || ldc < N) return CGPT_EINVAL;
  const int64_t epc = in_dtype == CGPT_F32 ? 4 : 8;
  const int64_t ealign = in_dtype == CGPT_F32 ? 4 : 2;
  const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pw = reinterpret_cast<uintptr_t>(w);
  const uintptr_t pb = epilogue != CGPT_EPI_NONE ? reinterpret_cast<uintptr_t>(bias) : 0;
  if (elem_loads != nullptr) {
    // Element alignment is all the element-load kernel needs.
    if (pa % ealign != 0 || pw % ealign != 0 ||
        pb % (bias_dtype == CGPT_F32 ? 4 : 2) != 0 ||
        reinterpret_cast<uintptr_t>(c) % (out_dtype == CGPT_F32 ? 4 : 2) != 0)
      return CGPT_EINVAL;
    *elem_loads = K % epc != 0 || lda % epc != 0 || ldw % epc != 0 || (pa & 15) || (pw & 15) ||
                  (pb & 15);
    return CGPT_OK;
  }
  if (K % epc != 0) return CGPT_ESHAPE;
  if (lda % epc != 0 || ldw % epc != 0) return CGPT_EINVAL;
  if ((pa & 15) || (pw & 15) || (pb & 15)) return CGPT_EINVAL;
  return CGPT_OK;
}
}  // namespace cgpt

extern "C" int cgpt_gemm_skinny_workspace(int64_t M, int64_t N, int64_t K, int in_dtype,
                                          int64_t* workspace_bytes, int64_t* n_counters) {
  using namespace cgpt;
  if (!workspace_bytes || !n_counters || M <= 0 || M > 64 || N <= 0 || K <= 0) return CGPT_EINVAL;
  if (N > 0x7fffffff || K > 0x7fffffff) return CGPT_ESHAPE;
  if (in_dtype != CGPT_F32 && in_dtype != CGPT_BF16) return CGPT_EDTYPE;
  return skinny_workspace(static_cast<int>(M), static_cast<int>(N), static_cast<int>(K),
                          in_dtype == CGPT_BF16, workspace_bytes, n_counters);
}

extern "C" int cgpt_gemm_skinny(const void* a, const void* w, const void* bias, void* c, int64_t M,
                                int64_t N, int64_t K, int64_t lda, int64_t ldw, int64_t ldc,
                                int in_dtype, int bias_dtype, int out_dtype, int epilogue,
                                void* workspace, int64_t workspace_bytes, int* counters,
                                int64_t n_counters, void* stream) {
  using namespace cgpt;
  const int st = validate_gemm(a, w, bias, c, M, N, K, lda, ldw, ldc, in_dtype, bias_dtype,
                               out_dtype, epilogue);
  if (st != CGPT_OK || M == 0 || N == 0) return st;
  if (M > 64) return CGPT_ESHAPE;
  if (epilogue == CGPT_EPI_BIAS_RESID) return CGPT_EINVAL;  // not a skinny epilogue
  return launch_gemm_skinny(in_dtype == CGPT_BF16, epilogue, a, w, bias, bias_dtype == CGPT_BF16,
                            c, out_dtype == CGPT_BF16, static_cast<int>(M), static_cast<int>(N),
                            static_cast<int>(K), lda, ldw, ldc, workspace, workspace_bytes, counters,
                            n_counters, static_cast<hipStream_t>(stream));
}

extern "C" int cgpt_gemm_partials_plan(int64_t M, int64_t N, int64_t K, int in_dtype,
                                       int64_t* n_split) {
  using namespace cgpt;
  if (!n_split || M <= 0 || M > 64 || N <= 0 || K <= 0) return CGPT_EINVAL;
  if (N > 0x7fffffff || K > 0x7fffffff) return CGPT_ESHAPE;
  if (in_dtype != CGPT_F32 && in_dtype != CGPT_BF16) return CGPT_EDTYPE;
  *n_split = gemm_partials_split(static_cast<int>(M), static_cast<int>(N), static_cast<int>(K),
                                 in_dtype == CGPT_BF16);
  return CGPT_OK;
}

extern "C" int cgpt_gemm_partials(const void* a, const void* w, float* partials, int64_t M,
                                  int64_t N, int64_t K, int64_t lda, int64_t ldw, int64_t ldp,
                                  int64_t n_split, int in_dtype, void* stream) {
  using namespace cgpt;
  const int st = validate_gemm(a, w, nullptr, partials, M, N, K, lda, ldw, ldp, in_dtype, in_dtype,
                               CGPT_F32, CGPT_EPI_NONE);
  if (st != CGPT_OK || M == 0 || N == 0) return st;
  if (M > 64) return CGPT_ESHAPE;
  if (reinterpret_cast<uintptr_t>(partials) & 3) return CGPT_EINVAL;
  if (n_split < 1 || n_split > 0x7fffffff) return CGPT_EINVAL;
  return launch_gemm_partials(in_dtype == CGPT_BF16, a, w, partials, static_cast<int>(M),
                              static_cast<int>(N), static_cast<int>(K), lda, ldw, ldp,
                              static_cast<int>(n_split), static_cast<hipStream_t>(stream));
}

extern "C" int cgpt_gemm(const void* a, const void* w, const void* bias, void* c, int64_t M,
                         int64_t N, int64_t K, int64_t lda, int64_t ldw, int64_t ldc, int in_dtype,
                         int bias_dtype, int out_dtype, int epilogue, int tile, void* stream) {
  using namespace cgpt;
  bool el = false;
  const int st = validate_gemm(a, w, bias, c, M, N, K, lda, ldw, ldc, in_dtype, bias_dtype,
                               out_dtype, epilogue, &el);
  if (st != CGPT_OK || M == 0 || N == 0) return st;
  const bool bf16 = in_dtype == CGPT_BF16, f16 = in_dtype == CGPT_F16;
  const int nt = (bf16 || f16) ? kNumBf16Tiles : kNumF32Tiles;
  const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool bb = bias_dtype != CGPT_F32;
  const bool out16 = out_dtype != CGPT_F32;
  const int64_t out_align = out16 ? 8 : 16;
  const bool vec_store = (ldc % 4 == 0) && (reinterpret_cast<uintptr_t>(c) % out_align == 0);
  if (tile == CGPT_TILE_SKINNY && (el || f16)) return CGPT_EINVAL;  // vector-rule bf16 / fp32 only
  if (epilogue == CGPT_EPI_BIAS_RESID) {
    if (tile == CGPT_TILE_SKINNY) return CGPT_EINVAL;  // not a skinny epilogue
    // launch_resid picks the kernel (tile: a preference; an id it does not
    // take for these dtypes, in or out of the tile tables, means TILE_AUTO).
    if (el) {
      if (f16)
        return out16 ? launch_epi<f16_t, f16_t>(epilogue, 0, a, w, bias, bb, c, m, n, k, lda, ldw, ldc, vec_store, true, s)
                     : launch_epi<f16_t, float>(epilogue, 0, a, w, bias, bb, c, m, n, k, lda, ldw, ldc, vec_store, true, s);
      if (bf16)
        return out16 ? launch_epi<bf16_t, bf16_t>(epilogue, 0, a, w, bias, bb, c, m, n, k, lda, ldw, ldc, vec_store, true, s)
                     : launch_epi<bf16_t, float>(epilogue, 0, a, w, bias, bb, c, m, n, k, lda, ldw, ldc, vec_store, true, s);
      return out16 ? launch_epi<float, bf16_t>(epilogue, 0, a, w, bias, bb, c, m, n, k, lda, ldw, ldc, vec_store, true, s)
                   : launch_epi<float, float>(epilogue, 0, a, w, bias, bb, c, m, n, k, lda, ldw, ldc, vec_store, true, s);
    }
    if (f16)
      return out16 ? launch_resid<f16_t, f16_t>(tile, a, w, bias, bb, c, m, n, k, lda, ldw, ldc, vec_store, s)
                   : launch_resid<f16_t, float>(tile, a, w, bias, bb, c, m, n, k, lda, ldw, ldc, vec_store, s);
    if (bf16 && out16)
      return launch_resid<bf16_t, bf16_t>(tile, a, w, bias, bb, c, m, n, k, lda, ldw, ldc, vec_store, s);
    if (bf16)
      return launch_resid<bf16_t, float>(tile, a, w, bias, bb, c, m, n, k, lda, ldw, ldc, vec_store, s);
    if (!out16)
      return launch_resid<float, float>(tile, a, w, bias, bb, c, m, n, k, lda, ldw, ldc, vec_store, s);
    return launch_resid<float, bf16_t>(tile, a, w, bias, bb, c, m, n, k, lda, ldw, ldc, vec_store, s);
  }
  if (tile != CGPT_TILE_AUTO && tile != CGPT_TILE_SKINNY && (tile < 0 || tile >= nt))
    return CGPT_EINVAL;
  if (tile == CGPT_TILE_AUTO && M <= 64 && !el && !f16) tile = CGPT_TILE_SKINNY;
  if (tile == CGPT_TILE_SKINNY) {
    if (M > 64) return CGPT_ESHAPE;
    return launch_gemm_skinny(bf16, epilogue, a, w, bias, bb, c, out16, m, n, k, lda, ldw, ldc,
                              nullptr, 0, nullptr, 0, s);
  }
  if (el) tile = 0;  // the element-load kernel has one tile
  if (tile == CGPT_TILE_AUTO) tile = auto_tile(bf16 || f16, m, n, k, lda, ldw, epilogue);
  if ((bf16 || f16) && tile >= kFirstPipeTile && !pipe_ok(tile, M, N, K, lda, ldw))
    return CGPT_ESHAPE;
  if ((bf16 || f16) && tile >= kFirstPipeTile) {
    const int pst = maybe_prefetch_w(w, M, N, K, ldw, s);
    if (pst != CGPT_OK) return pst;
  }
  if (f16)
    return out16 ? launch_epi<f16_t, f16_t>(epilogue, tile, a, w, bias, bb, c, m, n, k, lda, ldw, ldc, vec_store, el, s)
                 : launch_epi<f16_t, float>(epilogue, tile, a, w, bias, bb, c, m, n, k, lda, ldw, ldc, vec_store, el, s);
  if (bf16 && out16)
    return launch_epi<bf16_t, bf16_t>(epilogue, tile, a, w, bias, bb, c, m, n, k, lda, ldw, ldc, vec_store, el, s);
  if (bf16)
    return launch_epi<bf16_t, float>(epilogue, tile, a, w, bias, bb, c, m, n, k, lda, ldw, ldc, vec_store, el, s);
  if (!out16)
    return launch_epi<float, float>(epilogue, tile, a, w, bias, bb, c, m, n, k, lda, ldw, ldc, vec_store, el, s);
  return launch_epi<float, bf16_t>(epilogue, tile, a, w, bias, bb, c, m, n, k, lda, ldw, ldc, vec_store, el, s);
}
