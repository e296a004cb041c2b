// Batched NT GEMM used inside the library (not part of the C ABI): for each batch item b,
// C[b] = A[b] B[b]^T with A [M][K] and B [N][K] (k contiguous, leading dimensions lda, ldb,
// 16-byte aligned rows), C [M][N] (leading dimension ldc) in fp32 or the operand dtype. K must
// be a multiple of kBgemmK (callers zero-pad it). Batch strides in elements; sB = 0 shares B.
#pragma once

#include "capi.h"

constexpr int kBgemmK = 64;

int bgemm_nt(const void* A, const void* B, void* C, int M, int N, int K, long lda, long ldb, long ldc, long sA,
             long sB, long sC, int batch, int tc_dtype, int out_dtype, hipStream_t s);

// Row GEMM over many rows with the row kernels' epilogues: out[m][n] = epi(A W^T), A [M][K],
// W [Nout or 2 Nout][K], out [M][Nout], row-major. epi 0 stores, 1 adds into out, 2 is
// SwiGLU (out column j = silu(h_j) h_{Nout + j}). K must be a multiple of the k-tile (32 for
// bf16 operands, 16 for fp32). Operands bf16 with bf16 or fp32 output, or fp32 throughout.
int tile_gemm_rows(const void* A, const void* W, void* out, long M, int Nout, int K, int epi, int tc_dtype,
                   int out_dtype, hipStream_t s);
// The same GEMM (bf16 operands, epi 0 or 1) on the gated operand: out = epi((A * gate) W^T),
// gate [M][K] like A, each product rounded to bf16 before the GEMM.
int tile_gemm_rows_gated(const void* A, const void* gate, const void* W, void* out, long M, int Nout, int K,
                         int accumulate, int out_dtype, hipStream_t s);
// Rows from which the row GEMM hands over to tile_gemm_rows.
constexpr long kTileGemmMinRows = 16384;
