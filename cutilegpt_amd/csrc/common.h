// Shared device helpers for the gfx950 (CDNA4) kernels of cutilegpt_amd.
//
// Conventions used by every kernel in this directory:
//  * one wavefront = 64 lanes; blocks are multiples of 64 threads;
//  * bf16 is stored as raw uint16_t bit patterns, fp16 as _Float16; both are
//    converted with round-to-nearest-even; arithmetic is always fp32;
//  * 16-byte vector accesses (dwordx4) for every streaming load/store.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/cgpt.h"

namespace cgpt {

typedef uint16_t bf16_t;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_to_f32(bf16_t v) {
  return __uint_as_float(static_cast<uint32_t>(v) << 16);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two fp32 -> packed pair of bf16 (low half = a), round to nearest even, in one
// gfx950 v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

// Round-to-nearest-even fp32 -> bf16.
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(bf16_t, static_cast<__bf16>(f));
}

// IEEE binary16 (fp16) storage; conversions from fp32 round to nearest even.
typedef _Float16 f16_t;
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, f16x2_t));
}
__device__ __forceinline__ float f16_lo(uint32_t w) {
  return static_cast<float>(__builtin_bit_cast(f16x2_t, w)[0]);
}
__device__ __forceinline__ float f16_hi(uint32_t w) {
  return static_cast<float>(__builtin_bit_cast(f16x2_t, w)[1]);
}

// Two fp32 values packed as a pair of 16-bit elements of type T (low half = a).
template <typename T> __device__ __forceinline__ uint32_t pack2(float a, float b);
template <> __device__ __forceinline__ uint32_t pack2<bf16_t>(float a, float b) { return pack_bf16x2(a, b); }
template <> __device__ __forceinline__ uint32_t pack2<f16_t>(float a, float b) { return pack_f16x2(a, b); }

// Element type traits: load/store a float from/to T storage.
template <typename T> struct Elem;
template <> struct Elem<float> {
  static constexpr int kVec = 4;  // elements per 16-byte vector
  __device__ static float load(const float* p) { return *p; }
  __device__ static void store(float* p, float v) { *p = v; }
};
template <> struct Elem<bf16_t> {
  static constexpr int kVec = 8;
  __device__ static float load(const bf16_t* p) { return bf16_to_f32(*p); }
  __device__ static void store(bf16_t* p, float v) { *p = f32_to_bf16(v); }
};
template <> struct Elem<f16_t> {
  static constexpr int kVec = 8;
  __device__ static float load(const f16_t* p) { return static_cast<float>(*p); }
  __device__ static void store(f16_t* p, float v) { *p = static_cast<f16_t>(v); }
};

// Load/store 16 bytes as kVec floats.
__device__ __forceinline__ void load_vec(const float* p, float* out) {
  f32x4_t v = *reinterpret_cast<const f32x4_t*>(p);
  out[0] = v[0]; out[1] = v[1]; out[2] = v[2]; out[3] = v[3];
}
__device__ __forceinline__ void load_vec(const bf16_t* p, float* out) {
  u32x4_t v = *reinterpret_cast<const u32x4_t*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(v[i] << 16);
    out[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ void load_vec(const f16_t* p, float* out) {
  u32x4_t v = *reinterpret_cast<const u32x4_t*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = f16_lo(v[i]);
    out[2 * i + 1] = f16_hi(v[i]);
  }
}
// The same conversions for 16 bytes already in registers.
template <typename T> __device__ __forceinline__ void unpack_vec(const u32x4_t& v, float* out);
template <> __device__ __forceinline__ void unpack_vec<float>(const u32x4_t& v, float* out) {
#pragma unroll
  for (int i = 0; i < 4; ++i) out[i] = __uint_as_float(v[i]);
}
template <> __device__ __forceinline__ void unpack_vec<bf16_t>(const u32x4_t& v, float* out) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(v[i] << 16);
    out[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
  }
}
template <> __device__ __forceinline__ void unpack_vec<f16_t>(const u32x4_t& v, float* out) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = f16_lo(v[i]);
    out[2 * i + 1] = f16_hi(v[i]);
  }
}
__device__ __forceinline__ void store_vec(float* p, const float* in) {
  f32x4_t v = {in[0], in[1], in[2], in[3]};
  *reinterpret_cast<f32x4_t*>(p) = v;
}
__device__ __forceinline__ void store_vec(bf16_t* p, const float* in) {
  u32x4_t v;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = pack_bf16x2(in[2 * i], in[2 * i + 1]);
  *reinterpret_cast<u32x4_t*>(p) = v;
}
__device__ __forceinline__ void store_vec(f16_t* p, const float* in) {
  u32x4_t v;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = pack_f16x2(in[2 * i], in[2 * i + 1]);
  *reinterpret_cast<u32x4_t*>(p) = v;
}

// Cross-lane reductions through DPP (VALU operand modifiers, no LDS round
// trip as with __shfl_xor's ds_bpermute).  kDppXor1 / kDppXor2 swap
// neighbours within quads; kDppMirror8 pairs lane i with 7 - i of its group
// of 8, kDppMirror16 with 15 - i of its row of 16 — after xor1, xor2 and
// mirror8 each lane of an 8-lane group has combined all 8.
template <int CTRL> __device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppMirror8 = 0x141, kDppMirror16 = 0x140;
__device__ __forceinline__ float lane_value(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Sum over groups of G consecutive lanes (G = 1, 2, 4, 8 or 16), in every lane.
template <int G> __device__ __forceinline__ float group_sum(float v) {
  if (G >= 2) v += dpp<kDppXor1>(v);
  if (G >= 4) v += dpp<kDppXor2>(v);
  if (G >= 8) v += dpp<kDppMirror8>(v);
  if (G >= 16) v += dpp<kDppMirror16>(v);
  return v;
}

// Max / sum over the 64 lanes: rows of 16 through DPP, then the 4 rows'
// results read back as scalars (the same value in every lane).
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<kDppXor1>(v));
  v = fmaxf(v, dpp<kDppXor2>(v));
  v = fmaxf(v, dpp<kDppMirror8>(v));
  v = fmaxf(v, dpp<kDppMirror16>(v));
  return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}
__device__ __forceinline__ float wave_sum(float v) {
  v = group_sum<16>(v);
  return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}

// Max / sum of lane i with lanes i ^ 16, i ^ 32 and i ^ 48 (one column across
// the wave's four 16-lane rows), in every lane, through gfx950's
// v_permlane16_swap / v_permlane32_swap: VALU moves between rows, no LDS round
// trip.  Given the same value as both operands, a swap leaves in each lane the
// pair {v[i], v[i ^ 16]} (resp. i ^ 32), in some order; max and + commute, so
// all four lanes of a column end with the identical result.
__device__ __forceinline__ float swap_combine16_max(float v) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float swap_combine32_max(float v) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float column_max(float v) {
  return swap_combine32_max(swap_combine16_max(v));
}
__device__ __forceinline__ float column_sum(float v) {
  auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}


// tanh-approximate GELU written through the identity
//   0.5 x (1 + tanh(u)) = x / (1 + exp(-2u)),  u = sqrt(2/pi) (x + 0.044715 x^3),
// with exp(-2u) = 2^(-2u log2 e) on the hardware exp2 and the reciprocal on the
// hardware v_rcp_f32 (1 ulp).  Saturates cleanly: u -> +inf gives x, u -> -inf
// gives -0 (rcp(inf) = 0).
// The exponent -2u log2(e) = x (k1 + k3 x^2) with the constants folded, so the
// argument costs a multiply, an FMA and a multiply (k1 = -2 sqrt(2/pi) / ln 2,
// k3 = 0.044715 k1): three VALU instructions an element fewer than the
// unfolded polynomial, in the c_fc GEMM's epilogue where the matrix cores wait
// for them.
__device__ __forceinline__ float gelu_tanh(float x) {
  constexpr float kK1 = -2.302208198144325f;
  constexpr float kK3 = -0.1029432395800235f;
  const float a = x * __builtin_fmaf(kK3, x * x, kK1);
  const float e = __builtin_amdgcn_exp2f(a);
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

// One 16x16 MFMA tile step with 16-byte operand fragments: lane l supplies
// row l % 16 and k chunk l / 16 of each operand.  bf16: one
// v_mfma_f32_16x16x32_bf16 (8 k per lane).  fp32: four v_mfma_f32_16x16x4_f32;
// lane group g supplies k = 4g + j to the j-th (a consistent permutation of the
// k axis leaves the dot product unchanged).  With operand a = 16 rows of W and
// b = 16 rows of A, lane l of c holds C[m = l % 16][n = 4(l/16) .. +3].
template <typename T> struct Mfma;
template <> struct Mfma<bf16_t> {
  __device__ static void run(const u32x4_t& a, const u32x4_t& b, f32x4_t& c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
};
template <> struct Mfma<f16_t> {
  __device__ static void run(const u32x4_t& a, const u32x4_t& b, f32x4_t& c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                               __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
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
__device__ __forceinline__ void store4_out(f16_t* p, const float* v) {
  u32x2_t u = {pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3])};
  *reinterpret_cast<u32x2_t*>(p) = u;
}


// ---- direct-to-LDS streaming (shared by the GEMM and attention pipelines)

#if defined(__HIP_DEVICE_COMPILE__)
// Raw buffer descriptor (base, no stride, `bytes` records, gfx9 raw format).
__device__ __forceinline__ u32x4_t buffer_desc(const void* p, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  return u32x4_t{static_cast<uint32_t>(a), static_cast<uint32_t>(a >> 32) & 0xffffu, bytes,
                 0x00020000u};
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const uint8_t*)(p)));
}
// Global -> LDS DMA of 16 bytes per lane: lane l's bytes land at M0 + 16 l.
// Issued from inline assembly on purpose: the compiler then
// neither counts these loads nor guards later LDS reads against them, so the
// stage pipeline's own vmcnt waits and barriers are the only synchronisation
// (the compiler cannot prove that a read of one stage buffer does not alias
// the DMA into another and would otherwise drain the queue before every
// read).  M0 needs one wait state after its write.
// M0 is on the clobber list because the statement writes it.  clang warns that
// it does not save a reserved register around an asm statement (-Winline-asm,
// once per inlined call); nothing of the compiler's own lives in M0 across one:
// in the device code of every kernel here the only instructions that name M0
// are these moves (tests/test_dma_waits.py checks the skinny kernels' code).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma_lds16(u32x4_t desc, uint32_t lds, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :: "s"(lds), "v"(voff), "s"(desc), "s"(soff) : "memory", "m0");
}
#pragma clang diagnostic pop
#endif

__device__ __forceinline__ void raw_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// s_waitcnt vmcnt(N) lgkmcnt(0) (gfx9 encoding: vmcnt[3:0], expcnt[6:4],
// lgkmcnt[11:8], vmcnt[5:4] at [15:14]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0x0 << 8) | ((N >> 4) << 14));
}

// s_waitcnt lgkmcnt(0) alone (vmcnt and expcnt at their maxima).
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Error codes shared with the C ABI (see include/cgpt.h).
__host__ __forceinline__ int hip_status(hipError_t e) {
  return e == hipSuccess ? CGPT_OK : static_cast<int>(e);
}

}  // namespace cgpt
