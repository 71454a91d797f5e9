// Entry points shared between translation units of libcgpt.so (not exported).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cgpt {

// Argument checks shared by the GEMM entry points (cgpt_gemm, the skinny
// variants): CGPT_OK when the problem is well formed, M == 0 or N == 0
// included (nothing to launch).  Without `elem_loads` (the skinny kernels)
// inputs are fp32 or bf16 and must follow the 16-byte vector rules (K, lda
// and ldw multiples of the elements in 16 bytes, A, W and bias 16-byte
// aligned).  With it (cgpt_gemm) fp16 inputs are accepted too, and
// *elem_loads tells whether the problem breaks those rules and needs the
// element-load kernel.
int validate_gemm(const void* a, const void* w, const void* bias, const void* c, int64_t M,
                  int64_t N, int64_t K, int64_t lda, int64_t ldw, int64_t ldc, int in_dtype,
                  int bias_dtype, int out_dtype, int epilogue, bool* elem_loads = nullptr);

// Skinny GEMM (M <= 64): C[M,N] = epilogue(A W^T + bias).  Column slices of
// C, K split across the block's waves and (when workspace and counters are
// given) across blocks.  Arguments as cgpt_gemm's, already validated
// (K % (16 / element size) == 0, 16-byte aligned A and W rows).
int launch_gemm_skinny(bool bf16_in, int epilogue, const void* a, const void* w, const void* bias,
                       bool bias_bf16, void* c, bool out_bf16, int M, int N, int K, int64_t lda,
                       int64_t ldw, int64_t ldc, void* workspace, int64_t ws_bytes, int* counters,
                       int64_t n_counters, hipStream_t s);

// Workspace bytes and counters the split-K skinny GEMM uses for (M, N, K).
int skinny_workspace(int M, int N, int K, bool bf16_in, int64_t* ws_bytes, int64_t* n_counters);

// Every split-K plan launch_gemm_skinny makes stays within these (the
// no-allocation entry point's static scratch has exactly this capacity).
constexpr int64_t kSkinnyMaxWsBytes = int64_t{8} << 20;
constexpr int kSkinnyMaxCounters = 1024;

// Split-K partial products P[s][m][n] (fp32, P[s] at partials + s * M * ldp)
// of the skinny GEMM, for a consumer that adds them; the split the kernel is
// tuned for, and the launch.
int gemm_partials_split(int M, int N, int K, bool bf16_in);
int launch_gemm_partials(bool bf16_in, const void* a, const void* w, float* partials, int M, int N,
                         int K, int64_t lda, int64_t ldw, int64_t ldp, int split, hipStream_t s);

}  // namespace cgpt
