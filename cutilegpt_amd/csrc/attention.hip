// Causal flash attention forward on CDNA4 matrix cores.
//
// Work decomposition
//  * One block = 4 wavefronts = BQ = 128 queries of one (batch, head); each wave
//    owns QT = 2 sub-tiles of 16 queries (both kernels also have a 64-query
//    form, one sub-tile a wave, for small grids).  Blocks are ordered so that the last
//    (most expensive, under the causal mask) query blocks are dispatched first.
//  * Keys/values stream through LDS in BKV = 64-row blocks, double-buffered
//    through registers (the loads of block j+1 are in flight while block j is
//    computed).  Under the causal mask the loop stops at the block holding the
//    block's last query (causal tile skip) and only blocks that straddle the
//    diagonal (or the end of the sequence) evaluate the mask.
//
// Matrix-core formulation (16x16 MFMA tiles, fp32 accumulation)
//  * S^T = K Q^T: the K fragment is the MFMA "A" operand and the Q fragment the
//    "B" operand, so lane l holds S^T[key = 4(l/16) + r][query = l%16]: every
//    lane owns exactly one query.  The row maximum then needs two cross-lane
//    shuffles (lanes l^16, l^32), and the running max, the normaliser and the
//    rescale factor are per-lane scalars.
//  * O^T = V^T P^T: V is stored transposed in LDS ([d][key], keys contiguous);
//    the P operand is taken straight from the S^T accumulator registers.  The
//    key order inside one MFMA k-slab is permuted identically on both operands
//    (lane group g, element i <-> key 4g + i of the first 16-key tile, then of
//    the second), which leaves the contraction unchanged.
//  * bf16 / fp16: v_mfma_f32_16x16x32_bf16 / _f16; P is rounded to the input
//    type before P.V while the normaliser accumulates the unrounded fp32 P.
//    fp32: v_mfma_f32_16x16x4_f32.
//  * Softmax runs in the base-2 domain with scale * log2(e) folded into one
//    multiply; fully masked rows never produce NaN (the running max is clamped
//    to 0 while it is still -inf).
#include "common.h"

namespace cgpt {

constexpr int kAttnThreads = 256;
constexpr int kAttnBKV = 64;                       // keys per LDS block

template <typename T> struct AttnMfma;
template <> struct AttnMfma<bf16_t> {
  __device__ static void run(const u32x4_t& a, const u32x4_t& b, f32x4_t& c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
};
template <> struct AttnMfma<f16_t> {
  __device__ static void run(const u32x4_t& a, const u32x4_t& b, f32x4_t& c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                               __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
};
template <> struct AttnMfma<float> {
  __device__ static void run(const u32x4_t& a, const u32x4_t& b, f32x4_t& c) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[j]), __uint_as_float(b[j]), c, 0,
                                               0, 0);
  }
};

__device__ __forceinline__ void store4_o(float* p, const float* v) { store_vec(p, v); }
__device__ __forceinline__ void store4_o(bf16_t* p, const float* v) {
  u32x2_t u = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  *reinterpret_cast<u32x2_t*>(p) = u;
}
__device__ __forceinline__ void store4_o(f16_t* p, const float* v) {
  u32x2_t u = {pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3])};
  *reinterpret_cast<u32x2_t*>(p) = u;
}

template <typename T, int HD, int QTW>
__global__ __launch_bounds__(kAttnThreads) void attn_fwd_kernel(
    const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V, T* __restrict__ O,
    int H, int Tq, int Tk, int64_t q_sb, int64_t q_sh, int64_t q_st, int64_t k_sb, int64_t k_sh,
    int64_t k_st, int64_t v_sb, int64_t v_sh, int64_t v_st, int64_t o_sb, int64_t o_sh,
    int64_t o_st, float scale_log2, int causal, int n_bh) {
  constexpr int QT = QTW, BQ = 4 * 16 * QTW, BKV = kAttnBKV;
  constexpr int EPC = 16 / sizeof(T);          // elements per 16-byte chunk
  constexpr int CPR = HD / EPC;                // 16-byte chunks per K row
  constexpr int SWZ = (CPR < 8 ? CPR : 8) - 1; // chunk swizzle mask
  constexpr int KSTEP = 4 * EPC;               // head_dim covered by one k-slab
  constexpr int NKS = (HD + KSTEP - 1) / KSTEP;
  constexpr int ND = HD / 16;                  // 16-wide d tiles of O
  constexpr int KROW = HD * static_cast<int>(sizeof(T));
  // V^T rows are padded (8 B for bf16, 16 B for fp32) so the transposing writes
  // of one wave spread over the LDS banks; reads stay 8/16-byte aligned.
  constexpr int VROW = BKV * static_cast<int>(sizeof(T)) + (sizeof(T) == 2 ? 8 : 16);
  constexpr int KBYTES = BKV * KROW;
  constexpr int STAGE = KBYTES + HD * VROW;
  constexpr int KCH = BKV * CPR;               // K chunks per block
  constexpr int KL = (KCH + kAttnThreads - 1) / kAttnThreads;
  constexpr int VCH = (BKV / 2) * CPR;         // (key pair, chunk) items per block
  constexpr int VL = (VCH + kAttnThreads - 1) / kAttnThreads;
  static_assert(HD % 16 == 0, "head_dim must be a multiple of 16");
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * STAGE];

  // readfirstlane: the wave index is uniform, so wave-level conditions below
  // become scalar branches instead of exec-masked code.
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, frow = lane & 15;

  const int n_qblk = (Tq + BQ - 1) / BQ;
  const int qb = n_qblk - 1 - static_cast<int>(blockIdx.x) / n_bh;  // heavy blocks first
  const int bh = static_cast<int>(blockIdx.x) % n_bh;
  const int b = bh / H, h = bh % H;
  const int q0 = qb * BQ;
  const int off = Tk - Tq;  // absolute position of query 0

  const T* Qb = Q + b * q_sb + h * q_sh;
  const T* Kb = K + b * k_sb + h * k_sh;
  const T* Vb = V + b * v_sb + h * v_sh;

  // Q fragments stay in registers for the whole key loop.
  u32x4_t qf[QT][NKS];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qi = q0 + wave * 16 * QT + qt * 16 + frow;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int c = 4 * ks + g;
      qf[qt][ks] = (qi < Tq && c < CPR)
                       ? *reinterpret_cast<const u32x4_t*>(Qb + qi * q_st + c * EPC)
                       : u32x4_t{0, 0, 0, 0};
    }
  }

  // Key range this block needs.
  const int last_q = min(q0 + BQ, Tq) - 1 + off;  // absolute position of the block's last query
  const int kv_end = causal ? min(last_q + 1, Tk) : Tk;
  const int n_kv = (kv_end + BKV - 1) / BKV;
  const int wave_q0 = q0 + wave * 16 * QT;
  const int wave_last = min(wave_q0 + 16 * QT, Tq) - 1 + off;  // wave's last query position
  const bool wave_live = wave_q0 < Tq;

  u32x4_t rk[KL];
  u32x4_t rv[VL][2];
  auto gload = [&](int j) {
    const int kv0 = j * BKV;
#pragma unroll
    for (int i = 0; i < KL; ++i) {
      const int item = tid + i * kAttnThreads;
      if (item < KCH) {
        const int key = min(kv0 + item / CPR, Tk - 1);
        rk[i] = *reinterpret_cast<const u32x4_t*>(Kb + key * k_st + (item % CPR) * EPC);
      }
    }
#pragma unroll
    for (int i = 0; i < VL; ++i) {
      const int item = tid + i * kAttnThreads;
      if (item < VCH) {
        const int kp = item / CPR, c = item % CPR;
        const int k0 = min(kv0 + 2 * kp, Tk - 1), k1 = min(kv0 + 2 * kp + 1, Tk - 1);
        rv[i][0] = *reinterpret_cast<const u32x4_t*>(Vb + k0 * v_st + c * EPC);
        rv[i][1] = *reinterpret_cast<const u32x4_t*>(Vb + k1 * v_st + c * EPC);
      }
    }
  };
  auto swrite = [&](int buf) {
    uint8_t* sk = smem + buf * STAGE;
    uint8_t* sv = sk + KBYTES;
#pragma unroll
    for (int i = 0; i < KL; ++i) {
      const int item = tid + i * kAttnThreads;
      if (item < KCH) {
        const int key = item / CPR, c = item % CPR;
        *reinterpret_cast<u32x4_t*>(sk + key * KROW + ((c ^ (key & SWZ)) << 4)) = rk[i];
      }
    }
#pragma unroll
    for (int i = 0; i < VL; ++i) {
      const int item = tid + i * kAttnThreads;
      if (item < VCH) {
        const int kp = item / CPR, c = item % CPR;
        if constexpr (sizeof(T) == 2) {
          // 8 head_dim values of two consecutive keys -> 8 words [d][2kp, 2kp+1].
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t a = rv[i][0][e], bb = rv[i][1][e];
            const int d = c * EPC + 2 * e;
            *reinterpret_cast<uint32_t*>(sv + d * VROW + kp * 4) = (a & 0xffffu) | (bb << 16);
            *reinterpret_cast<uint32_t*>(sv + (d + 1) * VROW + kp * 4) = (a >> 16) | (bb & 0xffff0000u);
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int d = c * EPC + e;
            *reinterpret_cast<u32x2_t*>(sv + d * VROW + kp * 8) = u32x2_t{rv[i][0][e], rv[i][1][e]};
          }
        }
      }
    }
  };

  f32x4_t o_acc[QT][ND];
  float m_run[QT], l_run[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    m_run[qt] = -INFINITY;
    l_run[qt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) o_acc[qt][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  if (n_kv > 0) {
    gload(0);
    swrite(0);
  }
  __syncthreads();
  for (int j = 0; j < n_kv; ++j) {
    const int buf = j & 1;
    const int kv0 = j * BKV;
    if (j + 1 < n_kv) gload(j + 1);
    const uint8_t* sk = smem + buf * STAGE;
    const uint8_t* sv = sk + KBYTES;
    // A wave whose queries all precede this key block has nothing to do here.
    if (wave_live && !(causal && kv0 > wave_last)) {
      f32x4_t s[QT][4];
#pragma unroll
      for (int qt = 0; qt < QT; ++qt)
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) s[qt][kt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const int c = 4 * ks + g;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
          const int key = kt * 16 + frow;
          const u32x4_t kf = (c < CPR) ? *reinterpret_cast<const u32x4_t*>(
                                             sk + key * KROW + ((c ^ (key & SWZ)) << 4))
                                       : u32x4_t{0, 0, 0, 0};
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) AttnMfma<T>::run(kf, qf[qt][ks], s[qt][kt]);
        }
      }
      // Online softmax (base 2) on raw scores: p = exp2(s * scale_log2 - m) is
      // one FMA feeding v_exp_f32.  The shift m of a row only moves when the
      // row's block maximum exceeds it by more than kLazyLog2 (so P <= 2^8):
      // softmax is invariant to the shift, and the rescale of O and l (which
      // pulls the accumulators through the VALU) then runs only on the few
      // blocks where some row's maximum jumps, instead of on every block.
      // Masking is branch-free and only on blocks that straddle the diagonal
      // or the end of the sequence.
      constexpr float kLazyLog2 = 8.0f;
      const bool need_mask = (causal && kv0 + BKV - 1 > wave_q0 + off) || (kv0 + BKV > Tk);
      // Masking is a separate pass over the scores, taken by one wave-uniform
      // branch, so blocks off the diagonal run straight-line code with no
      // per-element key arithmetic.  Key kv0 + 4g + 16kt + r survives iff
      // 16kt + r <= lim, lim being the row's last visible key relative to
      // kv0 + 4g.
      if (need_mask) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          const int qpos = wave_q0 + qt * 16 + frow + off;
          const int lim = (causal ? min(qpos, Tk - 1) : Tk - 1) - kv0 - 4 * g;
#pragma unroll
          for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              s[qt][kt][r] = (kt * 16 + r > lim) ? -INFINITY : s[qt][kt][r];
        }
      }
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        float mloc = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) mloc = fmaxf(mloc, s[qt][kt][r]);
        mloc = column_max(mloc);
        const float mblk = mloc * scale_log2;  // scale > 0: max commutes
        const bool grow = mblk > m_run[qt] + kLazyLog2;
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {
          const float m_new = grow ? mblk : m_run[qt];
          const float alpha = grow ? __builtin_amdgcn_exp2f(m_run[qt] - m_new) : 1.0f;
          m_run[qt] = m_new;
          l_run[qt] *= alpha;
#pragma unroll
          for (int dt = 0; dt < ND; ++dt)
#pragma unroll
            for (int r = 0; r < 4; ++r) o_acc[qt][dt][r] *= alpha;
        }
        // A row that has seen only masked keys keeps m = -inf; its p are 0.
        const float neg_m = m_run[qt] == -INFINITY ? 0.f : -m_run[qt];
        float lsum = 0.f;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[qt][kt][r], scale_log2, neg_m));
            s[qt][kt][r] = p;
            lsum += p;
          }
        l_run[qt] += lsum;
      }
      // O^T += V^T P^T
      if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          u32x4_t pf[QT];
#pragma unroll
          for (int qt = 0; qt < QT; ++qt)
            pf[qt] = u32x4_t{pack2<T>(s[qt][2 * c][0], s[qt][2 * c][1]),
                             pack2<T>(s[qt][2 * c][2], s[qt][2 * c][3]),
                             pack2<T>(s[qt][2 * c + 1][0], s[qt][2 * c + 1][1]),
                             pack2<T>(s[qt][2 * c + 1][2], s[qt][2 * c + 1][3])};
#pragma unroll
          for (int dt = 0; dt < ND; ++dt) {
            const uint8_t* row = sv + (dt * 16 + frow) * VROW;
            const u32x2_t lo = *reinterpret_cast<const u32x2_t*>(row + (32 * c + 4 * g) * 2);
            const u32x2_t hi = *reinterpret_cast<const u32x2_t*>(row + (32 * c + 16 + 4 * g) * 2);
            const u32x4_t vf = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) AttnMfma<T>::run(vf, pf[qt], o_acc[qt][dt]);
          }
        }
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          u32x4_t pf[QT];
#pragma unroll
          for (int qt = 0; qt < QT; ++qt)
            pf[qt] = u32x4_t{__float_as_uint(s[qt][c][0]), __float_as_uint(s[qt][c][1]),
                             __float_as_uint(s[qt][c][2]), __float_as_uint(s[qt][c][3])};
#pragma unroll
          for (int dt = 0; dt < ND; ++dt) {
            const uint8_t* row = sv + (dt * 16 + frow) * VROW;
            const u32x4_t vf = *reinterpret_cast<const u32x4_t*>(row + (16 * c + 4 * g) * 4);
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) AttnMfma<T>::run(vf, pf[qt], o_acc[qt][dt]);
          }
        }
      }
    }
    if (j + 1 < n_kv) swrite(buf ^ 1);
    __syncthreads();
  }

  // Normalise and store: lane holds O[query][dt*16 + 4g .. +3].
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qi = wave_q0 + qt * 16 + frow;
    float l = l_run[qt];
    l = column_sum(l);
    if (qi >= Tq) continue;
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    T* orow = O + b * o_sb + h * o_sh + qi * o_st;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) {
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = o_acc[qt][dt][r] * inv;
      store4_o(orow + dt * 16 + 4 * g, v);
    }
  }
}

// 16-bit (bf16 / fp16) variant with K and V streamed straight into LDS
// (head_dim 64 or 128).
// Differences from attn_fwd_kernel:
//  * Keys and values go global -> LDS by buffer_load ... lds (no staging
//    registers, no LDS writes), STAGES blocks deep: block j + STAGES - 1 is
//    issued at step j into the buffer block j - 1 has released.  As in the
//    GEMM pipeline these loads are invisible to the compiler, so each step
//    ends with an explicit s_waitcnt for this wave's part of block j + 1 and
//    starts with a barrier.
//  * V stays row-major ([key][d], like K) and the V^T operand of O^T = V^T P^T
//    is read with ds_read_b64_tr_b16: within a 16-lane group, lane k points at
//    4 consecutive d of key (4j + k/4)-th row and receives, transposed, the 4
//    keys of its own d.  Two such reads give the 8-key k-slab in the key order
//    of the P operand (keys 32c + 4g + r, then 32c + 16 + 4g + r).
//  * 16-byte chunk c of row r is stored at chunk c ^ (r & 7): the DMA lane
//    that fills a slot fetches the chunk that belongs there.
template <int HD, int STAGES, int QTW, typename T = bf16_t>
// Four waves per SIMD (VGPRs capped at 128; two 32 KiB stages per block, so
// four 128-query blocks fit a CU's LDS): 576 -> 620 TFLOP/s at 16x12x1024x64
// against three waves and three stages, bit-identical.
__global__ __launch_bounds__(kAttnThreads) __attribute__((amdgpu_waves_per_eu(4, 4))) void attn_fwd_dma_kernel(
    const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
    T* __restrict__ O, int H, int Tq, int Tk, int64_t q_sb, int64_t q_sh, int64_t q_st,
    int64_t k_sb, int64_t k_sh, int64_t k_st, int64_t v_sb, int64_t v_sh, int64_t v_st,
    int64_t o_sb, int64_t o_sh, int64_t o_st, float scale_log2, int causal, int n_bh) {
#if defined(__HIP_DEVICE_COMPILE__)
  static_assert(sizeof(T) == 2, "16-bit inputs (bf16 or fp16)");
  constexpr int QT = QTW, BQ = 4 * 16 * QTW, BKV = kAttnBKV;
  constexpr int NWAVE = kAttnThreads / 64;
  constexpr int KROW = HD * 2;                 // bytes per K / V row
  constexpr int CPR = KROW / 16;               // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;                // rows per 1 KiB DMA instruction
  constexpr int XB = BKV * KROW;               // bytes of K (or V) per block
  constexpr int INS = XB / 1024 / NWAVE;       // DMA instructions per wave per operand
  constexpr int LPS = 2 * INS;
  constexpr int STAGE = 2 * XB;
  constexpr int NKS = HD / 32;                 // k32 slabs of head_dim
  constexpr int ND = HD / 16;
  static_assert(HD == 64 || HD == 128, "head_dim 64 or 128");
  static_assert(INS * NWAVE * 1024 == XB, "whole DMA instructions per wave");
  static_assert((STAGES - 2) * LPS < 64, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[STAGES * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, frow = lane & 15;

  const int n_qblk = (Tq + BQ - 1) / BQ;
  const int qb = n_qblk - 1 - static_cast<int>(blockIdx.x) / n_bh;  // heavy blocks first
  const int bh = static_cast<int>(blockIdx.x) % n_bh;
  const int b = bh / H, h = bh % H;
  const int q0 = qb * BQ;
  const int off = Tk - Tq;

  const T* Qb = Q + b * q_sb + h * q_sh;
  const u32x4_t rk = buffer_desc(K + b * k_sb + h * k_sh,
                                 static_cast<uint32_t>((static_cast<int64_t>(Tk - 1) * k_st + HD) * 2));
  const u32x4_t rv = buffer_desc(V + b * v_sb + h * v_sh,
                                 static_cast<uint32_t>((static_cast<int64_t>(Tk - 1) * v_st + HD) * 2));

  const int last_q = min(q0 + BQ, Tq) - 1 + off;
  const int kv_end = causal ? min(last_q + 1, Tk) : Tk;
  const int n_kv = (kv_end + BKV - 1) / BKV;
  const int wave_q0 = q0 + wave * 16 * QT;
  const int wave_last = min(wave_q0 + 16 * QT, Tq) - 1 + off;
  const bool wave_live = wave_q0 < Tq;

  // DMA of block j into stage buffer `buf`: instruction ii of this wave
  // fills rows (ii * NWAVE + wave) * RPI + lane / CPR; keys past Tk re-read
  // the last key (masked later).  When K and V share a row stride (always
  // for the fused QKV output), a block wholly below Tk adds its uniform key
  // offset kv0 * stride through the instruction's SGPR offset to the lane's
  // loop-invariant row part, so issuing it takes no VALU work.
  const int lrow = lane / CPR, slot = lane % CPR;
  const bool same_st = k_st == v_st;
  uint32_t kvo[INS];
#pragma unroll
  for (int ii = 0; ii < INS; ++ii) {
    const int row = (ii * NWAVE + wave) * RPI + lrow;
    kvo[ii] = static_cast<uint32_t>(row * k_st * 2) + static_cast<uint32_t>((slot ^ (row & 7)) << 4);
  }
  auto issue = [&](int j, uint8_t* buf) {
    const int kv0 = j * BKV;
    if (same_st && kv0 + BKV <= Tk) {
      const uint32_t so = static_cast<uint32_t>(kv0 * k_st * 2);
#pragma unroll
      for (int ii = 0; ii < INS; ++ii) {
        const uint32_t lds = (ii * NWAVE + wave) * 1024;
        dma_lds16(rk, lds_addr(buf + lds), kvo[ii], so);
        dma_lds16(rv, lds_addr(buf + XB + lds), kvo[ii], so);
      }
      return;
    }
#pragma unroll
    for (int ii = 0; ii < INS; ++ii) {
      const int row = (ii * NWAVE + wave) * RPI + lrow;
      const int key = min(kv0 + row, Tk - 1);
      const uint32_t chunk = static_cast<uint32_t>((slot ^ (row & 7)) << 4);
      const uint32_t lds = (ii * NWAVE + wave) * 1024;
      dma_lds16(rk, lds_addr(buf + lds), static_cast<uint32_t>(key * k_st * 2) + chunk, 0);
      dma_lds16(rv, lds_addr(buf + XB + lds), static_cast<uint32_t>(key * v_st * 2) + chunk, 0);
    }
  };
  // This wave's part of the block `later` stages before the newest one has
  // landed (and its LDS reads are done).
  auto wait_later = [&](int later) {
    if constexpr (STAGES >= 3)
      if (later >= 1) {
        wait_vmcnt<LPS>();
        return;
      }
    wait_vmcnt<0>();
  };

  f32x4_t o_acc[QT][ND];
  // nm = minus the running maximum of a query's scaled scores, +inf while the
  // query has none; l_run = its running normaliser.  Every query sees key 0
  // (Tk >= Tq, checked by the entry point), so the first key block gives
  // every lane a finite maximum unless its scores are not finite numbers.
  float nm[QT], l_run[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    nm[qt] = INFINITY;
    l_run[qt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) o_acc[qt][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  // V^T read: lane (g, k) of the 16-lane group points at row 4g + k/4 (plus
  // the slab's base key) and d = dt*16 + 4 (k % 4).
  const int tr_row = 4 * g + (frow >> 2);
  const int tr_byte = 8 * (frow & 3);
  auto vt_read = [&](const uint8_t* sv, int row, int dt) -> u32x2_t {
    const int byte = dt * 32 + tr_byte;
    const uint8_t* p = sv + row * KROW + ((((byte >> 4) ^ (row & 7))) << 4) + (byte & 15);
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4*)((__attribute__((address_space(3))) uint8_t*)(p)));
    return __builtin_bit_cast(u32x2_t, r);
  };

  // The first stages' DMA goes out before the Q loads, so the block's first
  // two memory round trips overlap; one wait then retires both (and keeps the
  // compiler's own wait for Q, which would sit before the first MFMA inside
  // the key loop, from draining the DMA queue there).
  int ib = 0;
#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < n_kv) {
      issue(s, smem + s * STAGE);
      ib = s + 1;
    }
  u32x4_t qf[QT][NKS];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qi = q0 + wave * 16 * QT + qt * 16 + frow;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
      qf[qt][ks] = qi < Tq ? *reinterpret_cast<const u32x4_t*>(Qb + qi * q_st + (4 * ks + g) * 8)
                           : u32x4_t{0, 0, 0, 0};
  }
  wait_vmcnt<0>();
  int cb = 0;
  for (int j = 0; j < n_kv; ++j) {
    raw_barrier();
    if (j + STAGES - 1 < n_kv) {
      issue(j + STAGES - 1, smem + ib * STAGE);
      ib = ib + 1 == STAGES ? 0 : ib + 1;
    }
    const int kv0 = j * BKV;
    const uint8_t* sk = smem + cb * STAGE;
    const uint8_t* sv = sk + XB;
    cb = cb + 1 == STAGES ? 0 : cb + 1;
    if (wave_live && !(causal && kv0 > wave_last)) {
      f32x4_t s[QT][4];
#pragma unroll
      for (int qt = 0; qt < QT; ++qt)
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) s[qt][kt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const int c = 4 * ks + g;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
          const int key = kt * 16 + frow;
          const u32x4_t kf =
              *reinterpret_cast<const u32x4_t*>(sk + key * KROW + ((c ^ (key & 7)) << 4));
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) AttnMfma<T>::run(kf, qf[qt][ks], s[qt][kt]);
        }
      }
      constexpr float kLazyLog2 = 8.0f;
      const bool need_mask = (causal && kv0 + BKV - 1 > wave_q0 + off) || (kv0 + BKV > Tk);
      if (need_mask) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          const int qpos = wave_q0 + qt * 16 + frow + off;
          const int lim = (causal ? min(qpos, Tk - 1) : Tk - 1) - kv0 - 4 * g;
#pragma unroll
          for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              s[qt][kt][r] = (kt * 16 + r > lim) ? -INFINITY : s[qt][kt][r];
        }
      }
      // P against the running maximum as it stands, before the block's own
      // maximum is known.  A lane whose 16 values sum to at most 2^7 has none
      // above 2^7, i.e. its scores sit at least 1 (log2 units) below the lazy
      // threshold (running maximum + kLazyLog2), so the rule below keeps the
      // maximum for its query and these values are the final ones.  Only when
      // some lane of the wave fails that (a NaN sum fails it too, and so does
      // a query with no maximum yet) is the block maximum taken and the rule
      // applied; lanes whose maximum moves recompute their values.  The
      // results equal those of always applying the rule first, bit for bit,
      // and the common block skips the maximum.
      constexpr float kOptimisticSum = 128.0f;
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        float p[4][4];
        float lsum = 0.f;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            p[kt][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[qt][kt][r], scale_log2, nm[qt]));
            lsum += p[kt][r];
          }
        // Every active lane settled: the compare's lane mask against exec (__all
        // would take two more VALU instructions).  A query with no maximum yet
        // (nm = +inf) sums to +inf or NaN and fails the test.
        if (__builtin_amdgcn_ballot_w64(lsum <= kOptimisticSum) != __builtin_amdgcn_read_exec()) {
          const float m_old = -nm[qt];  // -inf while the query has no maximum
          float mloc = -INFINITY;
#pragma unroll
          for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) mloc = fmaxf(mloc, s[qt][kt][r]);
          mloc = column_max(mloc);
          const float mblk = mloc * scale_log2;
          const bool grow = mblk > m_old + kLazyLog2;
          if (__builtin_amdgcn_ballot_w64(grow) != 0) {
            const float m_new = grow ? mblk : m_old;
            const float alpha = grow ? __builtin_amdgcn_exp2f(m_old - m_new) : 1.0f;
            nm[qt] = m_new == -INFINITY ? INFINITY : -m_new;
            l_run[qt] *= alpha;
#pragma unroll
            for (int dt = 0; dt < ND; ++dt)
#pragma unroll
              for (int r = 0; r < 4; ++r) o_acc[qt][dt][r] *= alpha;
            if (grow) {
              lsum = 0.f;
#pragma unroll
              for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                  p[kt][r] =
                      __builtin_amdgcn_exp2f(__builtin_fmaf(s[qt][kt][r], scale_log2, nm[qt]));
                  lsum += p[kt][r];
                }
            }
          }
        }
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) s[qt][kt][r] = p[kt][r];
        l_run[qt] += lsum;
      }
      // O^T += V^T P^T, k-slab c = keys 32c .. 32c + 31.
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        u32x4_t pf[QT];
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)
          pf[qt] = u32x4_t{pack2<T>(s[qt][2 * c][0], s[qt][2 * c][1]),
                           pack2<T>(s[qt][2 * c][2], s[qt][2 * c][3]),
                           pack2<T>(s[qt][2 * c + 1][0], s[qt][2 * c + 1][1]),
                           pack2<T>(s[qt][2 * c + 1][2], s[qt][2 * c + 1][3])};
#pragma unroll
        for (int dt = 0; dt < ND; ++dt) {
          const u32x2_t lo = vt_read(sv, 32 * c + tr_row, dt);
          const u32x2_t hi = vt_read(sv, 32 * c + 16 + tr_row, dt);
          const u32x4_t vf = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) AttnMfma<T>::run(vf, pf[qt], o_acc[qt][dt]);
        }
      }
    }
    if (j + 1 < n_kv) wait_later(n_kv - 1 - (j + 1) > STAGES - 2 ? STAGES - 2 : n_kv - 1 - (j + 1));
  }

#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qi = wave_q0 + qt * 16 + frow;
    float l = l_run[qt];
    l = column_sum(l);
    if (qi >= Tq) continue;
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    T* orow = O + b * o_sb + h * o_sh + qi * o_st;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) {
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = o_acc[qt][dt][r] * inv;
      store4_o(orow + dt * 16 + 4 * g, v);
    }
  }
#endif  // __HIP_DEVICE_COMPILE__
}

// The DMA kernel addresses a (batch, head)'s keys and values through 32-bit
// buffer offsets.
static bool attn_dma_ok(int Tk, const int64_t* st) {
  return (static_cast<int64_t>(Tk) + 1) * st[5] * 2 < (int64_t{1} << 31) &&
         (static_cast<int64_t>(Tk) + 1) * st[8] * 2 < (int64_t{1} << 31);
}

// Queries per block: 128 (2 sub-tiles of 16 a wave), or 64 (1 a wave) when
// 128-query blocks would give fewer than four blocks per CU — small batches or
// short sequences, where the launch is bound by its longest block.  Measured
// (bit-identical outputs): 8x12x512 216 -> 263 TFLOP/s, 16x8x256 126 -> 154,
// GPT-2 XL prefill 32x25x128 107 -> 118; at 16x12x1024 (6 blocks per CU) 64
// queries fell from 542 to 454.
template <int HD, int STAGES, int QTW, typename T>
static int launch_attn_dma_qt(const void* q, const void* k, const void* v, void* o, int B, int H,
                              int Tq, int Tk, const int64_t* st, float scale, int causal,
                              hipStream_t s) {
  constexpr int BQ = 4 * 16 * QTW;
  const int n_bh = B * H;
  const int n_qblk = (Tq + BQ - 1) / BQ;
  const int64_t blocks = static_cast<int64_t>(n_bh) * n_qblk;
  if (blocks > 0x7fffffff) return CGPT_ESHAPE;
  const float scale_log2 = scale * 1.4426950408889634f;
  hipLaunchKernelGGL((attn_fwd_dma_kernel<HD, STAGES, QTW, T>), dim3(static_cast<unsigned>(blocks)),
                     dim3(kAttnThreads), 0, s, static_cast<const T*>(q), static_cast<const T*>(k),
                     static_cast<const T*>(v), static_cast<T*>(o), H, Tq, Tk, st[0], st[1], st[2], st[3], st[4], st[5],
                     st[6], st[7], st[8], st[9], st[10], st[11], scale_log2, causal, n_bh);
  return hip_status(hipGetLastError());
}

static int attn_num_cus() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    return 256;
  return n;
}

template <int HD, int STAGES, typename T>
static int launch_attn_dma(const void* q, const void* k, const void* v, void* o, int B, int H,
                           int Tq, int Tk, const int64_t* st, float scale, int causal,
                           hipStream_t s) {
  const int64_t blocks128 = static_cast<int64_t>(B) * H * ((Tq + 127) / 128);
  if (blocks128 < 4 * static_cast<int64_t>(attn_num_cus()))
    return launch_attn_dma_qt<HD, STAGES, 1, T>(q, k, v, o, B, H, Tq, Tk, st, scale, causal, s);
  return launch_attn_dma_qt<HD, STAGES, 2, T>(q, k, v, o, B, H, Tq, Tk, st, scale, causal, s);
}

template <typename T, int HD>
static int launch_attn(const void* q, const void* k, const void* v, void* o, int B, int H, int Tq,
                       int Tk, const int64_t* st, float scale, int causal, hipStream_t s) {
  if constexpr (sizeof(T) == 2 && (HD == 64 || HD == 128)) {
    if (attn_dma_ok(Tk, st))
      return launch_attn_dma<HD, 2, T>(q, k, v, o, B, H, Tq, Tk, st, scale, causal, s);
  }
  // 64-query blocks when 128-query ones would give fewer than four per CU, as
  // for the DMA kernel.
  const int64_t blocks128 = static_cast<int64_t>(B) * H * ((Tq + 127) / 128);
  const bool small = blocks128 < 4 * static_cast<int64_t>(attn_num_cus());
  const int bq = small ? 64 : 128;
  const int n_bh = B * H;
  const int n_qblk = (Tq + bq - 1) / bq;
  const int64_t blocks = static_cast<int64_t>(n_bh) * n_qblk;
  if (blocks > 0x7fffffff) return CGPT_ESHAPE;
  const float scale_log2 = scale * 1.4426950408889634f;
#define CGPT_ATTN_LAUNCH(QTW)                                                                     \
  hipLaunchKernelGGL((attn_fwd_kernel<T, HD, QTW>), dim3(static_cast<unsigned>(blocks)),            \
                     dim3(kAttnThreads), 0, s, static_cast<const T*>(q), static_cast<const T*>(k), \
                     static_cast<const T*>(v), static_cast<T*>(o), H, Tq, Tk, st[0], st[1], st[2], \
                     st[3], st[4], st[5], st[6], st[7], st[8], st[9], st[10], st[11], scale_log2, \
                     causal, n_bh)
  if (small)
    CGPT_ATTN_LAUNCH(1);
  else
    CGPT_ATTN_LAUNCH(2);
#undef CGPT_ATTN_LAUNCH
  return hip_status(hipGetLastError());
}

template <typename T>
static int dispatch_hd(int hd, const void* q, const void* k, const void* v, void* o, int B, int H,
                       int Tq, int Tk, const int64_t* st, float scale, int causal, hipStream_t s) {
  switch (hd) {
    case 16: return launch_attn<T, 16>(q, k, v, o, B, H, Tq, Tk, st, scale, causal, s);
    case 32: return launch_attn<T, 32>(q, k, v, o, B, H, Tq, Tk, st, scale, causal, s);
    case 64: return launch_attn<T, 64>(q, k, v, o, B, H, Tq, Tk, st, scale, causal, s);
    case 128: return launch_attn<T, 128>(q, k, v, o, B, H, Tq, Tk, st, scale, causal, s);
    default: return CGPT_ESHAPE;
  }
}

}  // namespace cgpt

extern "C" int cgpt_attention_fwd(const void* q, const void* k, const void* v, void* o, int64_t B,
                                  int64_t H, int64_t Tq, int64_t Tk, int64_t head_dim,
                                  int64_t q_sb, int64_t q_sh, int64_t q_st, int64_t k_sb,
                                  int64_t k_sh, int64_t k_st, int64_t v_sb, int64_t v_sh,
                                  int64_t v_st, int64_t o_sb, int64_t o_sh, int64_t o_st,
                                  float scale, int causal, int dtype, void* stream) {
  using namespace cgpt;
  if (B < 0 || H < 0 || Tq < 0 || Tk < 0) return CGPT_EINVAL;
  if (B == 0 || H == 0 || Tq == 0) return CGPT_OK;
  if (q == nullptr || k == nullptr || v == nullptr || o == nullptr) return CGPT_EINVAL;
  if (Tk < Tq || Tk == 0) return CGPT_EINVAL;
  if (B * H > 0x7fffffff || Tk > 0x7fffffff) return CGPT_ESHAPE;
  if (dtype != CGPT_F32 && dtype != CGPT_BF16 && dtype != CGPT_F16) return CGPT_EDTYPE;
  const int64_t epc = dtype == CGPT_F32 ? 4 : 8;
  const int64_t st[12] = {q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh, v_st, o_sb, o_sh, o_st};
  // 16-byte vector loads of Q/K/V rows and 4-element stores of O need every
  // row start to stay 16-byte (8-byte for O in bf16) aligned.
  for (int i = 0; i < 9; ++i)
    if (st[i] < 0 || st[i] % epc != 0) return CGPT_EINVAL;
  for (int i = 9; i < 12; ++i)
    if (st[i] < 0 || st[i] % 4 != 0) return CGPT_EINVAL;
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
       reinterpret_cast<uintptr_t>(v)) & 15)
    return CGPT_EINVAL;
  if (reinterpret_cast<uintptr_t>(o) & (dtype == CGPT_F32 ? 15 : 7)) return CGPT_EINVAL;
  if (!(scale > 0.f)) return CGPT_EINVAL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int b = static_cast<int>(B), h = static_cast<int>(H);
  const int tq = static_cast<int>(Tq), tk = static_cast<int>(Tk);
  const int hd = static_cast<int>(head_dim);
  if (dtype == CGPT_BF16) return dispatch_hd<bf16_t>(hd, q, k, v, o, b, h, tq, tk, st, scale, causal != 0, s);
  if (dtype == CGPT_F16) return dispatch_hd<f16_t>(hd, q, k, v, o, b, h, tq, tk, st, scale, causal != 0, s);
  return dispatch_hd<float>(hd, q, k, v, o, b, h, tq, tk, st, scale, causal != 0, s);
}
