// Entry points shared between translation units of libcgpt.so (not exported).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cgpt {

// Skinny GEMM (M <= 64): C[M,N] = epilogue(A W^T + bias), one 16-column slice of
// C per block, K split across the block's waves and reduced through LDS.
// Arguments as cgpt_gemm's, already validated (K % (16 / element size) == 0,
// 16-byte aligned A and W rows).
int launch_gemm_skinny(bool bf16_in, int epilogue, const void* a, const void* w, const void* bias,
                       bool bias_bf16, void* c, bool out_bf16, int M, int N, int K, int64_t lda,
                       int64_t ldw, int64_t ldc, hipStream_t s);

}  // namespace cgpt
