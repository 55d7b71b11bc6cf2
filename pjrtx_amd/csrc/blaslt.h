// Plain large GEMMs on hipBLASLt (AMD's tuned library kernels for gfx950).
//
// The planner's own MFMA kernels handle every dot_general; a plain product
// large enough to fill the GPU (no fused epilogue, 16-bit inputs) is handed
// to hipBLASLt instead when the library is present and has an algorithm for
// the shape (environment: PJRTX_BLASLT=0 keeps the own kernels). This is the
// reference's "plain library matmul" path (reference:
// src/backend/mlx_metal/api.cc:3349-3498, which calls mlx::matmul).
#pragma once

#include "kernels/dot.h"
#include "runtime.h"

namespace pjrtx {

// C[b] (M x N row-major, ldc) = A[b] (M x K row-major, lda) * B[b], with B
// stored [K][N] (N contiguous, ldb) when !b_kmajor or [N][K] (K contiguous,
// ldb) when b_kmajor; f32 accumulation, C in the input type (out_bytes 2)
// or f32 (out_bytes 4). Returns false, having launched nothing, when
// hipBLASLt is off, absent or has no algorithm for the problem.
bool blaslt_gemm(Device* dev, const GemmParams& g, const void* A, const void* B, void* C, bool f16, bool b_kmajor,
                 int out_bytes);

// True when a product of this size goes to blaslt_gemm first.
bool blaslt_wanted(const GemmParams& g);

}  // namespace pjrtx
