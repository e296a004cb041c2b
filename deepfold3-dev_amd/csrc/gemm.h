// Batched NT GEMM used inside the library (not part of the C ABI): for each batch item b,
// C[b] = A[b] B[b]^T with A [M][K] and B [N][K] (k contiguous, leading dimensions lda, ldb,
// 16-byte aligned rows), C [M][N] (leading dimension ldc) in fp32 or the operand dtype. K must
// be a multiple of kBgemmK (callers zero-pad it). Batch strides in elements; sB = 0 shares B.
#pragma once

#include "capi.h"

constexpr int kBgemmK = 64;

int bgemm_nt(const void* A, const void* B, void* C, int M, int N, int K, long lda, long ldb, long ldc, long sA,
             long sB, long sC, int batch, int tc_dtype, int out_dtype, hipStream_t s);
