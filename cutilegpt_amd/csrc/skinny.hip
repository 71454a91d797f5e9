// Weight-streaming GEMM for decode shapes: C[M,N] = epi(A W^T + bias) with
// M <= 64 (one row per sequence of a decode batch).  Every weight byte is read
// once per call, so the kernel is built around memory round trips, not MFMA
// reuse:
//
//  * a block owns 16*NT output columns (NT n-tiles of W rows) and one K chunk;
//    its NW waves split the chunk's double slabs evenly;
//  * a wave issues every W and A fragment load of a round (DPW double slabs)
//    before its first MFMA, as buffer loads whose out-of-range offsets return
//    zero (k past K and slots past the wave's range need no select), so a
//    block costs one memory round trip;
//  * W rows go straight from global memory into MFMA fragments: lane group g
//    of a row loads 32 contiguous bytes (k = 2g EPC .. 2g EPC + 2 EPC), the 4
//    groups of a row one full 128-byte line per load pair; the two 16-byte
//    halves feed two MFMAs (any consistent assignment of k to MFMA slots gives
//    the same sums, and A uses the same one);
//  * partial tiles are summed across the block's waves through LDS in wave
//    order.  Across K chunks (split > 1) either
//      - the block's sum goes to a workspace and the last block of a column
//        slice (counted on a device atomic) adds the chunks in order and
//        applies the epilogue (cgpt_gemm_skinny), or
//      - the chunk sums are written as fp32 partial products for the consumer
//        to add (cgpt_gemm_partials; the decode step's attention and
//        residual+LayerNorm kernels do), which leaves the GEMM a single
//        round trip with no cross-block hand-off.
#include "common.h"
#include "internal.h"

#include <algorithm>

namespace cgpt {

// Block shapes: NT n-tiles per block, NW waves, DPW double slabs per wave and
// load round.
struct SkShape {
  int nt, nw, dpw;
};
// Shape 3 (8 n-tiles, 4 waves, 1 double slab a round) is for wide N with the
// final epilogue: 128 columns a block halve the A re-reads of shape 1 and
// its 4-wave blocks leave LDS for more of them a CU (GPT-2 XL LM head, 32
// rows: 60 -> 50 us on weights rotated past the MALL; as the partials
// shape for K = 6400 it was slower, 8.1 -> 10.2 us).
// Shape 4 (4 n-tiles, 4 waves, 1 double slab) takes the partials of long K
// (>= 64 double slabs: MLP-proj at K = 6400, 7.8-8.1 -> 7.4 us in a sweep of
// every shape over weights rotated past the MALL).
constexpr SkShape kSkShapes[] = {{2, 8, 1}, {4, 8, 2}, {2, 16, 2}, {8, 4, 1}, {4, 4, 1}};
constexpr int kSkTargetBlocks = 512;  // fix-up path: blocks to aim for
constexpr int kSkMaxSplit = 16;       // fix-up path: K chunks per column slice at most
constexpr int kCpolSc1 = 16;          // buffer cache-policy bits: sc1 (agent scope)
constexpr uint32_t kOob = 0x80000000u;  // past every record count: the load returns 0

__device__ __forceinline__ float bias_value(const void* bias, bool bf16, int n) {
  return bf16 ? bf16_to_f32(static_cast<const bf16_t*>(bias)[n]) : static_cast<const float*>(bias)[n];
}

enum SkMode { kSkFinal = 0, kSkPartials = 1 };

template <typename TIn, int MT, int NT, int NW, int DPW, int MODE, int EPI, typename TOut>
__global__ __launch_bounds__(64 * NW) void gemm_skinny_kernel(
    const TIn* __restrict__ A, const TIn* __restrict__ W, const void* __restrict__ bias,
    bool bias_bf16, TOut* __restrict__ C, int M, int N, int K, int lda, int ldw, int64_t ldc,
    bool vec_store, int split, int dslabs, float* __restrict__ ws, int* __restrict__ counters) {
  constexpr int ES = sizeof(TIn);
  constexpr int EPC = 16 / ES;  // elements per 16-byte half
  constexpr int KD = 8 * EPC;   // k per double slab
  constexpr int P = MT * NT;    // (m-tile, n-tile) pairs of the block tile
  constexpr int Q = (P + NW - 1) / NW;
  __shared__ f32x4_t red[NW][P][64];
  __shared__ int s_last;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nb = blockIdx.x / split, sk = blockIdx.x % split;
  const int n0 = nb * 16 * NT;
  const int r16 = lane & 15, g = lane >> 4;
  const int kl = g * 2 * EPC;  // this lane's first k inside a double slab

  // Record counts end at the last row's K-th element: the host keeps them
  // below 2^31, so kOob is out of range for both.
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<TIn*>(W), 0, static_cast<int>((N - 1) * ldw * ES + K * ES), 0x00020000);
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<TIn*>(A), 0, static_cast<int>((M - 1) * lda * ES + K * ES), 0x00020000);
  // Rows past N / M are clamped (loaded, never stored).
  uint32_t wro[NT], aro[MT];
#pragma unroll
  for (int j = 0; j < NT; ++j) wro[j] = static_cast<uint32_t>(min(n0 + 16 * j + r16, N - 1)) * ldw * ES;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) aro[mt] = static_cast<uint32_t>(min(16 * mt + r16, M - 1)) * lda * ES;

  const int chunk = (dslabs + split - 1) / split;
  const int d0 = sk * chunk, d1 = min(dslabs, d0 + chunk);
  const int cnt = d1 > d0 ? d1 - d0 : 0;
  const int w0 = d0 + wave * cnt / NW, w1 = d0 + (wave + 1) * cnt / NW;

  f32x4_t acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[mt][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int d = w0; d < w1; d += DPW) {
    u32x4_t wf[DPW][NT][2], af[DPW][MT][2];
#pragma unroll
    for (int u = 0; u < DPW; ++u)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int k = (d + u) * KD + kl + h * EPC;
        const uint32_t kb = (d + u < w1 && k < K) ? static_cast<uint32_t>(k) * ES : kOob;
#pragma unroll
        for (int j = 0; j < NT; ++j) wf[u][j][h] = __builtin_amdgcn_raw_buffer_load_b128(rw, wro[j] + kb, 0, 0);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) af[u][mt][h] = __builtin_amdgcn_raw_buffer_load_b128(ra, aro[mt] + kb, 0, 0);
      }
    // Keep the round's loads ahead of its MFMAs: interleaving them makes the
    // compiler wait on each load in turn.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < DPW; ++u)
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
    for (int j = 0; j < NT; ++j) red[wave][mt * NT + j][lane] = acc[mt][j];
  __syncthreads();

  // One (m-tile, n-tile) pair per wave and pass: its sum over the waves.
  f32x4_t sum[Q];
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const int pr = wave + q * NW;
    if (pr < P) {
      f32x4_t t = red[0][pr][lane];
#pragma unroll
      for (int w = 1; w < NW; ++w) t += red[w][pr][lane];
      sum[q] = t;
    }
  }

  if (MODE == kSkPartials) {
    // Chunk sk's partial products: ws[sk][m][n], rows of ldc floats.
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const int pr = wave + q * NW;
      if (pr >= P) continue;
      const int m = 16 * (pr / NT) + r16, n = n0 + 16 * (pr % NT) + 4 * g;
      if (m >= M || n >= N) continue;
      float* out = ws + (static_cast<int64_t>(sk) * M + m) * ldc + n;
      const float v[4] = {sum[q][0], sum[q][1], sum[q][2], sum[q][3]};
      if (vec_store && n + 3 < N) {
        store4_out(out, v);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (n + r < N) out[r] = v[r];
      }
    }
    return;
  }

  if (split > 1) {
    // Cross-block hand-off without cache-wide fences (an agent-scope fence
    // writes back and invalidates this XCD's whole L2): partials are stored
    // and loaded with agent-scope cache policy (sc1), which makes those
    // accesses coherent across the XCDs' L2s, the same encoding the memory
    // model uses for agent-scope atomic loads and stores.  The s_waitcnt
    // before the barrier completes every thread's partial stores before
    // thread 0 counts the block with a device atomic.
    constexpr int kTile = P * 64;  // f32x4 per block tile
    const __amdgpu_buffer_rsrc_t rws = __builtin_amdgcn_make_buffer_rsrc(
        ws + static_cast<int64_t>(nb) * split * kTile * 4, 0, split * kTile * 16, 0x00020000);
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const int pr = wave + q * NW;
      if (pr < P)
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
    for (int q = 0; q < Q; ++q) {
      const int pr = wave + q * NW;
      if (pr < P) {
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
  for (int q = 0; q < Q; ++q) {
    const int pr = wave + q * NW;
    if (pr >= P) continue;
    const int m = 16 * (pr / NT) + r16, n = n0 + 16 * (pr % NT) + 4 * g;
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

// Work split of one call: which block shape, 16*NT-column slices x `split`
// K chunks.
struct SkinnyPlan {
  int shape, mt, slices, dslabs, split;
  int64_t ws_floats;  // fix-up path: per-block partial tiles, all blocks
};

static int sk_mt(int M) { return M <= 16 ? 1 : M <= 32 ? 2 : 4; }

// Final output (fix-up split when workspace and counters are given).
static SkinnyPlan skinny_plan(int M, int N, int K, int elem_bytes, bool have_ws) {
  SkinnyPlan p;
  const int kd = 8 * (16 / elem_bytes);
  p.mt = sk_mt(M);
  p.dslabs = (K + kd - 1) / kd;
  const int slices2 = (N + 31) / 32;
  if (have_ws) {
    p.shape = 0;
  } else if (slices2 >= 1024) {
    // wide N (an LM head): fewer A re-reads per weight byte; shape 3 holds
    // 8 n-tiles of accumulators, so four m-tiles stay on shape 1
    p.shape = p.mt < 4 ? 3 : 1;
  } else {
    // 16 waves leave 128 VGPRs a lane: too few for four m-tiles' fragments.
    p.shape = p.dslabs >= 16 && p.mt < 4 ? 2 : 0;
  }
  const SkShape& s = kSkShapes[p.shape];
  p.slices = (N + 16 * s.nt - 1) / (16 * s.nt);
  int split = 1;
  if (have_ws) {
    // About kSkTargetBlocks blocks, but every wave of a block keeps at least
    // one double slab and at most kSkMaxSplit chunks per slice.
    split = (kSkTargetBlocks + p.slices - 1) / p.slices;
    int cap = p.dslabs / s.nw;
    cap = cap < kSkMaxSplit ? cap : kSkMaxSplit;
    split = split < cap ? split : cap;
    split = split > 1 ? split : 1;
  }
  p.split = split;
  p.ws_floats = split > 1 ? static_cast<int64_t>(p.slices) * split * p.mt * s.nt * 64 * 4 : 0;
  return p;
}

// Partial products: chunks of about 5 double slabs (K <= 64 slabs) or 10.
static SkinnyPlan partials_plan(int M, int N, int K, int elem_bytes, int split) {
  SkinnyPlan p;
  const int kd = 8 * (16 / elem_bytes);
  p.mt = sk_mt(M);
  p.dslabs = (K + kd - 1) / kd;
  p.shape = p.dslabs >= 64 ? 4 : 0;
  const SkShape& s = kSkShapes[p.shape];
  p.slices = (N + 16 * s.nt - 1) / (16 * s.nt);
  if (split <= 0) {
    const int target = p.shape == 4 ? 10 : 5;
    split = (p.dslabs + target - 1) / target;
  }
  p.split = split;
  p.ws_floats = 0;
  return p;
}

// Wide-N form for at most 32 rows of bf16 (the decode step's LM head, N in
// the tens of thousands): one block of kWideWaves waves a CU.  The block
// stages all of A in LDS once (rows zero-padded to 16 * MT, K to whole double
// slabs, each row padded by 16 bytes so the 16 rows a fragment read touches
// fall in different banks); each wave then owns whole 16-column slices of C
// (slice blockIdx.x + gridDim.x * (wave + kWideWaves * i)) and streams the
// slice's W rows straight from global memory into MFMA fragments, in rounds
// of kWideDpw double slabs whose loads are all issued before the round's
// MFMAs, with A's fragments read from LDS.  A slice is summed over all of K
// by one wave, so there is no cross-wave or cross-block reduction, and the
// grid's CUs take ceil or floor of slices / CUs slices each (the 128-column
// blocks of shape 3 split 393 blocks over 256 CUs, two on some and one on
// others).
constexpr int kWideWaves = 16;
constexpr int kWideDpw = 5;
constexpr int kWideKMax = 2496;  // K a row may hold: 32 rows x (2 * 2496 + 16) B fit in LDS

template <int MT, int EPI, typename TOut>
__global__ __launch_bounds__(64 * kWideWaves) void gemm_skinny_wide_kernel(
    const bf16_t* __restrict__ A, const bf16_t* W, const void* __restrict__ bias,
    bool bias_bf16, TOut* __restrict__ C, int M, int N, int K, int lda, int ldw, int64_t ldc,
    bool vec_store) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int KD = 64;  // k per double slab
  // 1 KiB past the A image: the last 64-lane DMA of the staging may run past it.
  __shared__ __attribute__((aligned(16))) uint8_t sa[MT * 16 * (2 * kWideKMax + 16) + 1024];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int kp = (K + KD - 1) / KD * KD;  // K padded to whole double slabs
  const int rs = 2 * kp + 16;             // LDS bytes per A row
  const int D = kp / KD;

  // A goes to LDS by DMA (16 bytes a lane, 64 consecutive 16-byte slots an
  // instruction; the slot after each row's last chunk is the row's padding),
  // then the first W round; the wait before the barrier leaves exactly that
  // round's kWideDpw * 2 loads outstanding, so the barrier does not wait for
  // W.  Rows past M, k past K and the padding slots load zero (an offset past
  // the record count).
  const u32x4_t ra = buffer_desc(A, static_cast<uint32_t>((M - 1) * lda * 2 + K * 2));
  const int cpr = kp / 8;  // chunks per row
  const int nslot = MT * 16 * (cpr + 1);
#pragma unroll
  for (int i = 0; i < (MT * 16 * (kWideKMax / 8 + 1) + 64 * kWideWaves - 1) / (64 * kWideWaves); ++i) {
    const int base = (i * kWideWaves + wave) * 64;
    if (base >= nslot) break;
    const int slot = base + lane;
    const int row = slot / (cpr + 1), ch = slot - row * (cpr + 1);
    const uint32_t off = (row < M && ch < cpr && ch * 8 < K)
                             ? static_cast<uint32_t>(row * lda + ch * 8) * 2 : kOob;
    dma_lds16(ra, lds_addr(sa + base * 16), off, 0);
  }
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<bf16_t*>(W), 0, static_cast<int>((N - 1) * ldw * 2 + K * 2), 0x00020000);
  const int nslices = (N + 15) / 16;
  const int stride = static_cast<int>(gridDim.x) * kWideWaves;
  int sl = static_cast<int>(blockIdx.x) + static_cast<int>(gridDim.x) * wave;
  u32x4_t wf[kWideDpw][2];
  auto load_round = [&](int s, int d) {
    const bool live = s < nslices;
    const uint32_t wro = static_cast<uint32_t>(min(s * 16 + r16, N - 1)) * ldw * 2;
#pragma unroll
    for (int u = 0; u < kWideDpw; ++u)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int k = (d + u) * KD + g * 16 + h * 8;
        const uint32_t kb = (live && d + u < D && k < K) ? static_cast<uint32_t>(k) * 2 : kOob;
        wf[u][h] = __builtin_amdgcn_raw_buffer_load_b128(rw, wro + kb, 0, 0);
      }
  };
  load_round(sl, 0);
  // W is not __restrict__ here: loads through it are then not invariant and
  // cannot move across the memory clobbers of the DMA above or of this wait,
  // so exactly the round's loads are younger than the last DMA.
  static_assert(kWideDpw * 2 == 10, "the wait below counts one W round");
  asm volatile("s_waitcnt vmcnt(10)" ::: "memory");
  raw_barrier();

  const uint8_t* abase = sa + r16 * rs + g * 32;  // this lane's fragment row, k = 16 g
  for (; sl < nslices; sl += stride) {
    f32x4_t acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int d = 0; d < D; d += kWideDpw) {
      if (d > 0) load_round(sl, d);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < kWideDpw; ++u) {
        if (d + u < D) {
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              const u32x4_t af = *reinterpret_cast<const u32x4_t*>(
                  abase + mt * 16 * rs + ((d + u) * KD + h * 8) * 2);
              Mfma<bf16_t>::run(wf[u][h], af, acc[mt]);
            }
        }
      }
    }
    // The next slice's first round goes out before this one's stores.
    const int n0 = sl * 16;
    if (sl + stride < nslices) load_round(sl + stride, 0);
    // Lane (g, r16) holds C[16 mt + r16][n0 + 4 g + i], i = 0..3.
    const int n = n0 + 4 * g;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = 16 * mt + r16;
      if (m >= M || n >= N) continue;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float x = acc[mt][r];
        if (EPI != CGPT_EPI_NONE) x += n + r < N ? bias_value(bias, bias_bf16, n + r) : 0.f;
        if (EPI == CGPT_EPI_BIAS_GELU) x = gelu_tanh(x);
        v[r] = x;
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
#endif  // __HIP_DEVICE_COMPILE__
}

// Decode-layer form for at most 32 rows of bf16 and N of a few hundred
// 16-column n-tiles (the QKV, projection and MLP GEMMs of a decode step).
// Block (group g, chunk sk) covers the 16 * NW columns of group g over the
// K chunk sk (chunk double slabs, at most KS):
//  * its waves DMA the chunk of A into LDS (16-byte slots, each row padded by
//    one slot so the 16 rows of a fragment read fall in different banks);
//  * each wave then issues all KS * 2 loads of its n-tile's W rows at once,
//    one memory round trip, and the wait before the barrier leaves exactly
//    those loads outstanding (W is not __restrict__: loads through it are not
//    invariant and cannot move across the memory clobbers of the DMA or of the
//    wait), so the barrier waits for A only;
//  * MT * 2 MFMAs per double slab with A's fragments read from LDS.
// Waves split N, not K, so there is no cross-wave reduction, and A is read
// from L2 once per block instead of once per n-tile.  The chunk sums are
// either written as fp32 partial products P[sk][m][n] (rows of ldc floats) for
// the consumer to add (kSkPartials), or, for the final output, stored to the
// workspace and added in chunk order by the last block of the column group to
// arrive (counted on a device atomic; the same sc1 hand-off as
// gemm_skinny_kernel), which applies the epilogue (kSkFinal; split == 1
// stores directly).
constexpr int kDecMaxKs = 10;  // double slabs a chunk may hold

template <int MT, int NW, int KS, int MODE, int EPI, typename TOut>
__global__ __launch_bounds__(64 * NW) void gemm_decode_kernel(
    const bf16_t* __restrict__ A, const bf16_t* W, const void* __restrict__ bias,
    bool bias_bf16, TOut* __restrict__ C, int M, int N, int K, int lda, int ldw, int64_t ldc,
    bool vec_store, int split, int chunk, float* __restrict__ ws, int* __restrict__ counters) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int KD = 64;               // k per double slab
  constexpr int SROW = KS * 8 + 1;     // 16-byte slots per A row, the last one padding
  constexpr int RS = SROW * 16;        // LDS bytes per A row
  constexpr int NSLOT = MT * 16 * SROW;
  constexpr int NINS = (NSLOT + 64 * NW - 1) / (64 * NW);  // DMA instructions a wave, at most
  // Whole 64-slot DMA instructions: the last one may run past the A image.
  __shared__ __attribute__((aligned(16))) uint8_t sa[NINS * NW * 64 * 16];
  __shared__ int s_last;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int gi = blockIdx.x / split, sk = blockIdx.x % split;
  const int dslabs = (K + KD - 1) / KD;
  const int d0 = sk * chunk;
  const int d1 = min(dslabs, d0 + chunk);  // d1 <= d0: an empty chunk, zero sums

  // A's chunk -> LDS; rows past M, k past K or past the chunk, and the padding
  // slots load zero (an offset past the record count).
  const u32x4_t ra = buffer_desc(A, static_cast<uint32_t>((M - 1) * lda * 2 + K * 2));
#pragma unroll
  for (int i = 0; i < NINS; ++i) {
    const int base = (i * NW + wave) * 64;
    if (base >= NSLOT) break;
    const int slot = base + lane;
    const int row = slot / SROW, ch = slot - row * SROW;
    const int k = d0 * KD + ch * 8;
    const bool ok = row < M && ch < KS * 8 && d0 + ch / 8 < d1 && k < K;
    dma_lds16(ra, lds_addr(sa + base * 16), ok ? static_cast<uint32_t>(row * lda + k) * 2 : kOob, 0);
  }
  // This wave's n-tile (rows past N are clamped: loaded, never stored).
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<bf16_t*>(W), 0, static_cast<int>((N - 1) * ldw * 2 + K * 2), 0x00020000);
  const int nt = gi * NW + wave;
  const bool live = nt * 16 < N;
  const uint32_t wro = static_cast<uint32_t>(min(nt * 16 + r16, N - 1)) * ldw * 2;
  u32x4_t wf[KS][2];
#pragma unroll
  for (int u = 0; u < KS; ++u)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int k = (d0 + u) * KD + g * 16 + h * 8;
      const uint32_t kb = (live && d0 + u < d1 && k < K) ? static_cast<uint32_t>(k) * 2 : kOob;
      wf[u][h] = __builtin_amdgcn_raw_buffer_load_b128(rw, wro + kb, 0, 0);
    }
  asm volatile("" ::: "memory");
  wait_vmcnt<KS * 2>();
  raw_barrier();

  f32x4_t acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const uint8_t* abase = sa + r16 * RS + g * 32;  // this lane's fragment row, k = 16 g
#pragma unroll
  for (int u = 0; u < KS; ++u) {
    if (d0 + u < d1) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const u32x4_t af =
              *reinterpret_cast<const u32x4_t*>(abase + mt * 16 * RS + (u * KD + h * 8) * 2);
          Mfma<bf16_t>::run(wf[u][h], af, acc[mt]);
        }
    }
  }
  // Lane (g, r16) holds C[16 mt + r16][16 nt + 4 g + i], i = 0..3.
  const int n = nt * 16 + 4 * g;

  if (MODE == kSkPartials) {
    if (!live) return;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = 16 * mt + r16;
      if (m >= M || n >= N) continue;
      float* out = reinterpret_cast<float*>(C) + (static_cast<int64_t>(sk) * M + m) * ldc + n;
      const float v[4] = {acc[mt][0], acc[mt][1], acc[mt][2], acc[mt][3]};
      if (vec_store && n + 3 < N) {
        store4_out(out, v);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (n + r < N) out[r] = v[r];
      }
    }
    return;
  }

  if (split > 1) {
    // Chunk sk's sums go to the group's workspace slots [sk][wave][mt][lane]
    // (f32x4) with sc1 stores; the last block to count itself on the group's
    // counter adds all chunks in order and resets the counter.
    constexpr int kTile = NW * MT * 64;  // f32x4 per chunk
    const __amdgpu_buffer_rsrc_t rws = __builtin_amdgcn_make_buffer_rsrc(
        ws + static_cast<int64_t>(gi) * split * kTile * 4, 0, split * kTile * 16, 0x00020000);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, acc[mt]), rws,
                                             ((sk * NW + wave) * MT * 64 + mt * 64 + lane) * 16, 0,
                                             kCpolSc1);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
      s_last = __hip_atomic_fetch_add(&counters[gi], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               split - 1;
    __syncthreads();
    if (!s_last) return;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      u32x4_t part[kSkMaxSplit];
#pragma unroll
      for (int c = 0; c < kSkMaxSplit; ++c)
        if (c < split)
          part[c] = __builtin_amdgcn_raw_buffer_load_b128(
              rws, ((c * NW + wave) * MT * 64 + mt * 64 + lane) * 16, 0, kCpolSc1);
      f32x4_t t = __builtin_bit_cast(f32x4_t, part[0]);
#pragma unroll
      for (int c = 1; c < kSkMaxSplit; ++c)
        if (c < split) t += __builtin_bit_cast(f32x4_t, part[c]);
      acc[mt] = t;
    }
    if (threadIdx.x == 0)
      __hip_atomic_store(&counters[gi], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (!live) return;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = 16 * mt + r16;
    if (m >= M || n >= N) continue;
    float v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float x = acc[mt][r];
      if (EPI != CGPT_EPI_NONE) x += n + r < N ? bias_value(bias, bias_bf16, n + r) : 0.f;
      if (EPI == CGPT_EPI_BIAS_GELU) x = gelu_tanh(x);
      v[r] = x;
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
#endif  // __HIP_DEVICE_COMPILE__
}

static int skinny_num_cus() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    return 256;
  return n;
}

// The wide form is taken for bf16, M <= 32, K within the LDS budget, no split
// workspace, and N wide enough that every CU gets several slices.
static bool wide_ok(bool bf16_in, bool have_ws, int M, int N, int K) {
  return bf16_in && !have_ws && M <= 32 && K <= kWideKMax && (N + 15) / 16 >= 8 * skinny_num_cus();
}

template <int EPI, typename TOut>
static void launch_wide_mt(const bf16_t* A, const bf16_t* W, const void* bias, bool bias_bf16,
                           TOut* C, int M, int N, int K, int lda, int ldw, int64_t ldc,
                           bool vec_store, hipStream_t s) {
  const int slices = (N + 15) / 16;
  const int cus = skinny_num_cus();
  const dim3 grid(static_cast<unsigned>(slices < cus ? slices : cus));
  if (M <= 16)
    hipLaunchKernelGGL((gemm_skinny_wide_kernel<1, EPI, TOut>), grid, dim3(64 * kWideWaves), 0, s, A, W,
                       bias, bias_bf16, C, M, N, K, lda, ldw, ldc, vec_store);
  else
    hipLaunchKernelGGL((gemm_skinny_wide_kernel<2, EPI, TOut>), grid, dim3(64 * kWideWaves), 0, s, A, W,
                       bias, bias_bf16, C, M, N, K, lda, ldw, ldc, vec_store);
}

template <typename TOut>
static int launch_wide(int epi, const void* a, const void* w, const void* bias, bool bias_bf16,
                       void* c, int M, int N, int K, int lda, int ldw, int64_t ldc, bool vec_store,
                       hipStream_t s) {
  const bf16_t* A = static_cast<const bf16_t*>(a);
  const bf16_t* W = static_cast<const bf16_t*>(w);
  TOut* C = static_cast<TOut*>(c);
  switch (epi) {
    case CGPT_EPI_NONE:
      launch_wide_mt<CGPT_EPI_NONE, TOut>(A, W, bias, bias_bf16, C, M, N, K, lda, ldw, ldc, vec_store, s);
      break;
    case CGPT_EPI_BIAS:
      launch_wide_mt<CGPT_EPI_BIAS, TOut>(A, W, bias, bias_bf16, C, M, N, K, lda, ldw, ldc, vec_store, s);
      break;
    case CGPT_EPI_BIAS_GELU:
      launch_wide_mt<CGPT_EPI_BIAS_GELU, TOut>(A, W, bias, bias_bf16, C, M, N, K, lda, ldw, ldc, vec_store, s);
      break;
    default:
      return CGPT_EINVAL;
  }
  return hip_status(hipGetLastError());
}

template <typename TIn, int MT, int NT, int NW, int DPW, int MODE, int EPI, typename TOut>
static void launch_one(const SkinnyPlan& p, const TIn* A, const TIn* W, const void* bias,
                       bool bias_bf16, TOut* C, int M, int N, int K, int lda, int ldw, int64_t ldc,
                       bool vec_store, float* ws, int* counters, hipStream_t s) {
  hipLaunchKernelGGL((gemm_skinny_kernel<TIn, MT, NT, NW, DPW, MODE, EPI, TOut>),
                     dim3(static_cast<unsigned>(p.slices * p.split)), dim3(64 * NW), 0, s, A, W, bias,
                     bias_bf16, C, M, N, K, lda, ldw, ldc, vec_store, p.split, p.dslabs, ws, counters);
}

template <typename TIn, int MT, int MODE, int EPI, typename TOut>
static void launch_shape(const SkinnyPlan& p, const TIn* A, const TIn* W, const void* bias,
                         bool bias_bf16, TOut* C, int M, int N, int K, int lda, int ldw, int64_t ldc,
                         bool vec_store, float* ws, int* counters, hipStream_t s) {
#define CGPT_SK_SHAPE(I)                                                                          \
  launch_one<TIn, MT, kSkShapes[I].nt, kSkShapes[I].nw, kSkShapes[I].dpw, MODE, EPI, TOut>(        \
      p, A, W, bias, bias_bf16, C, M, N, K, lda, ldw, ldc, vec_store, ws, counters, s)
  if (p.shape == 1) {
    CGPT_SK_SHAPE(1);
  } else if (p.shape == 4) {
    CGPT_SK_SHAPE(4);
  } else if constexpr (MT < 4) {  // the planners give shapes 2 and 3 at most two m-tiles
    if (p.shape == 3)
      CGPT_SK_SHAPE(3);
    else if (p.shape == 2)
      CGPT_SK_SHAPE(2);
    else
      CGPT_SK_SHAPE(0);
  } else {
    CGPT_SK_SHAPE(0);
  }
#undef CGPT_SK_SHAPE
}

template <typename TIn, int MODE, int EPI, typename TOut>
static void launch_mt(const SkinnyPlan& p, const TIn* A, const TIn* W, const void* bias,
                      bool bias_bf16, TOut* C, int M, int N, int K, int lda, int ldw, int64_t ldc,
                      bool vec_store, float* ws, int* counters, hipStream_t s) {
  if (p.mt == 1)
    launch_shape<TIn, 1, MODE, EPI, TOut>(p, A, W, bias, bias_bf16, C, M, N, K, lda, ldw, ldc, vec_store, ws, counters, s);
  else if (p.mt == 2)
    launch_shape<TIn, 2, MODE, EPI, TOut>(p, A, W, bias, bias_bf16, C, M, N, K, lda, ldw, ldc, vec_store, ws, counters, s);
  else
    launch_shape<TIn, 4, MODE, EPI, TOut>(p, A, W, bias, bias_bf16, C, M, N, K, lda, ldw, ldc, vec_store, ws, counters, s);
}

template <typename TIn, typename TOut>
static int launch_final(const SkinnyPlan& p, int epi, const void* a, const void* w, const void* bias,
                        bool bias_bf16, void* c, int M, int N, int K, int lda, int ldw, int64_t ldc,
                        bool vec_store, float* ws, int* counters, hipStream_t s) {
  const TIn* A = static_cast<const TIn*>(a);
  const TIn* W = static_cast<const TIn*>(w);
  TOut* C = static_cast<TOut*>(c);
  switch (epi) {
    case CGPT_EPI_NONE:
      launch_mt<TIn, kSkFinal, CGPT_EPI_NONE, TOut>(p, A, W, bias, bias_bf16, C, M, N, K, lda, ldw, ldc, vec_store, ws, counters, s);
      break;
    case CGPT_EPI_BIAS:
      launch_mt<TIn, kSkFinal, CGPT_EPI_BIAS, TOut>(p, A, W, bias, bias_bf16, C, M, N, K, lda, ldw, ldc, vec_store, ws, counters, s);
      break;
    case CGPT_EPI_BIAS_GELU:
      launch_mt<TIn, kSkFinal, CGPT_EPI_BIAS_GELU, TOut>(p, A, W, bias, bias_bf16, C, M, N, K, lda, ldw, ldc, vec_store, ws, counters, s);
      break;
    default:
      return CGPT_EINVAL;
  }
  return hip_status(hipGetLastError());
}

// Buffer offsets are 32-bit: A's rows, and the W rows of one launch, must end
// below 2^31 bytes.  Returns the columns per launch (a multiple of the slice
// width), or 0 when even one slice is too large.
static int cols_per_launch(int N, int K, int64_t ldw, int es, int slice_cols) {
  const int64_t lim = (int64_t{1} << 31) - static_cast<int64_t>(K) * es;
  const int64_t rows = lim / (ldw * es) + 1;  // rows r with (r - 1) * ldw * es + K * es < 2^31
  const int64_t slices = rows / slice_cols;
  if (slices <= 0) return 0;
  const int64_t cols = slices * slice_cols;
  return cols >= N ? N : static_cast<int>(cols);
}

static bool a_fits(int M, int K, int64_t lda, int es) {
  return static_cast<int64_t>(M - 1) * lda * es + static_cast<int64_t>(K) * es < (int64_t{1} << 31);
}

// Work split of a decode-form call: `nw` n-tiles (waves) a block, K chunks of
// `chunk` double slabs in a kernel instance holding `ks` >= chunk, `split`
// chunks, `groups` column groups.
struct DecodePlan {
  int mt, nw, ks, chunk, split, groups;
  int64_t ws_floats;  // final output with split > 1: every group's chunk sums
};
constexpr int kDecKs[] = {2, 3, 5, kDecMaxKs};
constexpr int kDecChunk = 5;         // double slabs a chunk at most, when the split is ours
constexpr int kDecWavesPerCu = 5;    // waves (n-tile x chunk units) to aim for a CU

// split > 0: exactly that many K chunks (a partials caller's n_split); 0: chunks
// of at most kDecChunk double slabs, and more of them while there are fewer
// than kDecWavesPerCu waves a CU, but at most kSkMaxSplit chunks (the fix-up's
// limit, and that of the decode step's partials consumers); a chunk that
// still exceeds kDecChunk takes the longest kernel instance whole.  A sweep of
// the GPT-2 XL decode shapes on rotated weights picked QKV 5 chunks,
// projection 13, MLP projection 10 of the choices within 16.  Blocks hold 8
// waves, or 4 for K of 64 double slabs or more.  nw > 0 forces the waves a
// block.  False when the shape is not one for the decode form (M > 32, chunks
// longer than kDecMaxKs, or more than kSkMaxSplit chunks of a final output).
static bool decode_plan(int M, int N, int K, int split, bool final_out, int nw, DecodePlan* p) {
  if (M < 1 || M > 32 || N < 1 || K < 1) return false;
  const int dslabs = (K + 63) / 64;
  const int tiles = (N + 15) / 16;
  if (split <= 0) {
    const int want = (kDecWavesPerCu * skinny_num_cus() + tiles - 1) / tiles;
    split = std::min({dslabs, kSkMaxSplit, std::max((dslabs + kDecChunk - 1) / kDecChunk, want)});
    int chunk = (dslabs + split - 1) / split;
    if (chunk > kDecChunk) chunk = kDecMaxKs;
    split = (dslabs + chunk - 1) / chunk;
    if (split > kSkMaxSplit) return false;
  }
  if (split > dslabs || (final_out && split > kSkMaxSplit)) return false;
  const int chunk = (dslabs + split - 1) / split;
  int ks = 0;
  for (int k : kDecKs)
    if (ks == 0 && k >= chunk) ks = k;
  if (ks == 0) return false;
  p->mt = M <= 16 ? 1 : 2;
  p->nw = nw > 0 ? nw : dslabs >= 64 ? 4 : 8;
  p->ks = ks;
  p->chunk = chunk;
  p->split = split;
  p->groups = (tiles + p->nw - 1) / p->nw;
  p->ws_floats = final_out && split > 1
                     ? static_cast<int64_t>(p->groups) * split * p->nw * p->mt * 64 * 4 : 0;
  return true;
}

// A final output in the decode form: unsplit when one chunk covers K (a single
// round trip; the cross-block hand-off costs three more), else split K with
// the last-block fix-up when there is a workspace and the split's chunk sums
// and counters fit kSkinnyMaxWsBytes / kSkinnyMaxCounters.
static bool decode_final_plan(int M, int N, int K, bool have_ws, DecodePlan* p) {
  if ((K + 63) / 64 <= kDecMaxKs) return decode_plan(M, N, K, 1, true, 0, p);
  // Beyond the scratch capacity every split plan keeps to, the other form.
  return have_ws && decode_plan(M, N, K, 0, true, 0, p) &&
         p->ws_floats * 4 <= kSkinnyMaxWsBytes && p->groups <= kSkinnyMaxCounters;
}

// Both operands' buffer offsets are 32-bit in the decode form (one launch).
static bool decode_fits(int M, int N, int K, int64_t lda, int64_t ldw) {
  return a_fits(M, K, lda, 2) && a_fits(N, K, ldw, 2);
}

template <int MT, int NW, int MODE, int EPI, typename TOut>
static int launch_decode_nw(const DecodePlan& p, const bf16_t* A, const bf16_t* W, const void* bias,
                            bool bias_bf16, TOut* C, int M, int N, int K, int lda, int ldw,
                            int64_t ldc, bool vec_store, float* ws, int* counters, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(p.groups * p.split)), block(64 * NW);
#define CGPT_DEC(KS)                                                                            \
  hipLaunchKernelGGL((gemm_decode_kernel<MT, NW, KS, MODE, EPI, TOut>), grid, block, 0, s, A, W, \
                     bias, bias_bf16, C, M, N, K, lda, ldw, ldc, vec_store, p.split, p.chunk, ws, \
                     counters)
  switch (p.ks) {
    case kDecKs[0]: CGPT_DEC(kDecKs[0]); break;
    case kDecKs[1]: CGPT_DEC(kDecKs[1]); break;
    case kDecKs[2]: CGPT_DEC(kDecKs[2]); break;
    case kDecKs[3]: CGPT_DEC(kDecKs[3]); break;
    default: return CGPT_EINVAL;
  }
#undef CGPT_DEC
  return hip_status(hipGetLastError());
}

template <int MODE, int EPI, typename TOut>
static int launch_decode(const DecodePlan& p, const void* a, const void* w, const void* bias,
                         bool bias_bf16, void* c, int M, int N, int K, int lda, int ldw, int64_t ldc,
                         bool vec_store, float* ws, int* counters, hipStream_t s) {
  const bf16_t* A = static_cast<const bf16_t*>(a);
  const bf16_t* W = static_cast<const bf16_t*>(w);
  TOut* C = static_cast<TOut*>(c);
#define CGPT_DEC_NW(MT, NW)                                                                \
  return launch_decode_nw<MT, NW, MODE, EPI, TOut>(p, A, W, bias, bias_bf16, C, M, N, K, lda, \
                                                   ldw, ldc, vec_store, ws, counters, s)
  if (p.mt == 1) {
    if (p.nw == 4) CGPT_DEC_NW(1, 4);
    if (p.nw == 8) CGPT_DEC_NW(1, 8);
  } else {
    if (p.nw == 4) CGPT_DEC_NW(2, 4);
    if (p.nw == 8) CGPT_DEC_NW(2, 8);
  }
#undef CGPT_DEC_NW
  return CGPT_EINVAL;
}

template <typename TOut>
static int launch_decode_final(const DecodePlan& p, int epi, const void* a, const void* w,
                               const void* bias, bool bias_bf16, void* c, int M, int N, int K,
                               int lda, int ldw, int64_t ldc, bool vec_store, float* ws,
                               int* counters, hipStream_t s) {
  switch (epi) {
    case CGPT_EPI_NONE:
      return launch_decode<kSkFinal, CGPT_EPI_NONE, TOut>(p, a, w, bias, bias_bf16, c, M, N, K, lda, ldw, ldc, vec_store, ws, counters, s);
    case CGPT_EPI_BIAS:
      return launch_decode<kSkFinal, CGPT_EPI_BIAS, TOut>(p, a, w, bias, bias_bf16, c, M, N, K, lda, ldw, ldc, vec_store, ws, counters, s);
    case CGPT_EPI_BIAS_GELU:
      return launch_decode<kSkFinal, CGPT_EPI_BIAS_GELU, TOut>(p, a, w, bias, bias_bf16, c, M, N, K, lda, ldw, ldc, vec_store, ws, counters, s);
    default:
      return CGPT_EINVAL;
  }
}

int launch_gemm_skinny(bool bf16_in, int epilogue, const void* a, const void* w, const void* bias,
                       bool bias_bf16, void* c, bool out_bf16, int M, int N, int K, int64_t lda,
                       int64_t ldw, int64_t ldc, void* workspace, int64_t ws_bytes, int* counters,
                       int64_t n_counters, hipStream_t s) {
  if (M > 64) return CGPT_ESHAPE;
  const int es = bf16_in ? 2 : 4;
  const bool have_ws = workspace != nullptr && counters != nullptr;
  if (wide_ok(bf16_in, have_ws, M, N, K) && a_fits(M, K, lda, es) &&
      static_cast<int64_t>(N - 1) * ldw * es + static_cast<int64_t>(K) * es < (int64_t{1} << 31)) {
    const uintptr_t oa = out_bf16 ? 7 : 15;
    const bool vec_store = ldc % 4 == 0 && (reinterpret_cast<uintptr_t>(c) & oa) == 0;
    const int li = static_cast<int>(lda), lw = static_cast<int>(ldw);
    return out_bf16 ? launch_wide<bf16_t>(epilogue, a, w, bias, bias_bf16, c, M, N, K, li, lw, ldc, vec_store, s)
                    : launch_wide<float>(epilogue, a, w, bias, bias_bf16, c, M, N, K, li, lw, ldc, vec_store, s);
  }
  // The decode form, when its split (if any) fits the workspace given.
  DecodePlan dp;
  if (bf16_in && decode_fits(M, N, K, lda, ldw) && decode_final_plan(M, N, K, have_ws, &dp) &&
      (dp.split == 1 || (dp.ws_floats * 4 <= ws_bytes && dp.groups <= n_counters &&
                         (reinterpret_cast<uintptr_t>(workspace) & 15) == 0))) {
    const uintptr_t oa = out_bf16 ? 7 : 15;
    const bool vec_store = ldc % 4 == 0 && (reinterpret_cast<uintptr_t>(c) & oa) == 0;
    const int li = static_cast<int>(lda), lw = static_cast<int>(ldw);
    float* wsf = dp.split > 1 ? static_cast<float*>(workspace) : nullptr;
    int* cnt = dp.split > 1 ? counters : nullptr;
    return out_bf16 ? launch_decode_final<bf16_t>(dp, epilogue, a, w, bias, bias_bf16, c, M, N, K, li, lw, ldc, vec_store, wsf, cnt, s)
                    : launch_decode_final<float>(dp, epilogue, a, w, bias, bias_bf16, c, M, N, K, li, lw, ldc, vec_store, wsf, cnt, s);
  }
  const SkinnyPlan p = skinny_plan(M, N, K, es, have_ws);
  const int scols = 16 * kSkShapes[p.shape].nt;
  const int step = cols_per_launch(N, K, ldw, es, scols);
  if (step == 0 || !a_fits(M, K, lda, es)) return CGPT_ESHAPE;
  if (p.split > 1 && (p.ws_floats * 4 > ws_bytes || p.slices > n_counters ||
                      (reinterpret_cast<uintptr_t>(workspace) & 15)))
    return CGPT_EINVAL;
  const uintptr_t oa = out_bf16 ? 7 : 15;
  const bool vec_store = ldc % 4 == 0 && (reinterpret_cast<uintptr_t>(c) & oa) == 0;
  const int ob = out_bf16 ? 2 : 4, bb = bias_bf16 ? 2 : 4;
  const int64_t tile_floats = static_cast<int64_t>(p.split) * p.mt * kSkShapes[p.shape].nt * 64 * 4;
  for (int c0 = 0; c0 < N; c0 += step) {
    // Column groups start on slice boundaries, so the workspace and counter
    // slots of a group are its slices' own.
    const int n = N - c0 < step ? N - c0 : step;
    SkinnyPlan pg = p;
    pg.slices = (n + scols - 1) / scols;
    const int first = c0 / scols;
    const void* wg = static_cast<const char*>(w) + static_cast<int64_t>(c0) * ldw * es;
    const void* bg = bias != nullptr ? static_cast<const char*>(bias) + static_cast<int64_t>(c0) * bb : nullptr;
    void* cg = static_cast<char*>(c) + static_cast<int64_t>(c0) * ob;
    float* wsg = have_ws ? static_cast<float*>(workspace) + first * tile_floats : nullptr;
    int* cng = have_ws ? counters + first : nullptr;
    const int li = static_cast<int>(lda), lw = static_cast<int>(ldw);
    int st;
    if (bf16_in)
      st = out_bf16 ? launch_final<bf16_t, bf16_t>(pg, epilogue, a, wg, bg, bias_bf16, cg, M, n, K, li, lw, ldc, vec_store, wsg, cng, s)
                    : launch_final<bf16_t, float>(pg, epilogue, a, wg, bg, bias_bf16, cg, M, n, K, li, lw, ldc, vec_store, wsg, cng, s);
    else
      st = out_bf16 ? launch_final<float, bf16_t>(pg, epilogue, a, wg, bg, bias_bf16, cg, M, n, K, li, lw, ldc, vec_store, wsg, cng, s)
                    : launch_final<float, float>(pg, epilogue, a, wg, bg, bias_bf16, cg, M, n, K, li, lw, ldc, vec_store, wsg, cng, s);
    if (st != CGPT_OK) return st;
  }
  return CGPT_OK;
}

// Enough for either form (the decode form runs when the workspace holds its
// split; the other split-K form otherwise).
int skinny_workspace(int M, int N, int K, bool bf16_in, int64_t* ws_bytes, int64_t* n_counters) {
  const SkinnyPlan p = skinny_plan(M, N, K, bf16_in ? 2 : 4, true);
  *ws_bytes = p.ws_floats * 4;
  *n_counters = p.split > 1 ? p.slices : 0;
  DecodePlan dp;
  if (bf16_in && decode_final_plan(M, N, K, true, &dp) && dp.split > 1) {
    *ws_bytes = std::max(*ws_bytes, dp.ws_floats * 4);
    *n_counters = std::max(*n_counters, static_cast<int64_t>(dp.groups));
  }
  return CGPT_OK;
}

// At most kSkMaxSplit chunks: the decode step's consumers add up to 16.
int gemm_partials_split(int M, int N, int K, bool bf16_in) {
  DecodePlan dp;
  if (bf16_in && decode_plan(M, N, K, 0, false, 0, &dp)) return dp.split;
  return std::min(partials_plan(M, N, K, bf16_in ? 2 : 4, 0).split, kSkMaxSplit);
}

int launch_gemm_partials(bool bf16_in, const void* a, const void* w, float* partials, int M, int N,
                         int K, int64_t lda, int64_t ldw, int64_t ldp, int split, hipStream_t s) {
  if (M > 64) return CGPT_ESHAPE;
  const int es = bf16_in ? 2 : 4;
  const SkinnyPlan p = partials_plan(M, N, K, es, split);
  if (split < 1 || split > p.dslabs) return CGPT_EINVAL;
  DecodePlan dp;
  if (bf16_in && decode_fits(M, N, K, lda, ldw) && decode_plan(M, N, K, split, false, 0, &dp)) {
    const bool vec_store = ldp % 4 == 0 && (reinterpret_cast<uintptr_t>(partials) & 15) == 0;
    return launch_decode<kSkPartials, CGPT_EPI_NONE, float>(
        dp, a, w, nullptr, false, partials, M, N, K, static_cast<int>(lda), static_cast<int>(ldw),
        ldp, vec_store, nullptr, nullptr, s);
  }
  const int scols = 16 * kSkShapes[p.shape].nt;
  const int step = cols_per_launch(N, K, ldw, es, scols);
  if (step == 0 || !a_fits(M, K, lda, es)) return CGPT_ESHAPE;
  const bool vec_store = ldp % 4 == 0 && (reinterpret_cast<uintptr_t>(partials) & 15) == 0;
  const int li = static_cast<int>(lda), lw = static_cast<int>(ldw);
  for (int c0 = 0; c0 < N; c0 += step) {
    const int n = N - c0 < step ? N - c0 : step;
    SkinnyPlan pg = p;
    pg.slices = (n + scols - 1) / scols;
    const void* wg = static_cast<const char*>(w) + static_cast<int64_t>(c0) * ldw * es;
    float* pp = partials + c0;
    if (bf16_in)
      launch_mt<bf16_t, kSkPartials, CGPT_EPI_NONE, float>(
          pg, static_cast<const bf16_t*>(a), static_cast<const bf16_t*>(wg), nullptr, false, nullptr,
          M, n, K, li, lw, ldp, vec_store, pp, nullptr, s);
    else
      launch_mt<float, kSkPartials, CGPT_EPI_NONE, float>(
          pg, static_cast<const float*>(a), static_cast<const float*>(wg), nullptr, false, nullptr,
          M, n, K, li, lw, ldp, vec_store, pp, nullptr, s);
    const int st = hip_status(hipGetLastError());
    if (st != CGPT_OK) return st;
  }
  return CGPT_OK;
}

}  // namespace cgpt
