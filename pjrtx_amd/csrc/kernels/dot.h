// Launchers of the dot_general kernels (kernels/dot.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.h"

namespace pjrtx {

// C[b][m][n] = sum_k A[b][m][k] * B[b][k][n]; A K-contiguous (row stride lda);
// B N-contiguous ([K][N], row stride ldb) or K-contiguous ([N][K]); C row-major
// with row stride ldc and batch stride M*ldc. Strides in elements.
struct GemmParams {
  int batch = 1, M = 0, N = 0, K = 0;
  int64_t lda = 0, ldb = 0, ldc = 0;
  int64_t a_batch_stride = 0, b_batch_stride = 0;
};
void launch_mfma_gemm(hipStream_t s, const GemmParams& p, const void* A, const void* B, void* C, bool f16, bool b_kmajor,
                      int out_bytes);
// True when the 256 x 256 tile kernel applies (M, N >= 256, 16-byte aligned
// rows, K a multiple of 8 and, for an N-contiguous B, N too; enough tiles to
// fill the GPU). It takes B in either layout.
bool use_big_gemm(const GemmParams& p, bool b_kmajor);
// out[b] = transpose(in[b]) for 16-bit elements: in [rows][cols] -> out
// [cols][rows], batch strides in elements.
void launch_transpose16(hipStream_t s, const void* in, void* out, int64_t batch, int64_t rows, int64_t cols,
                        int64_t in_bs, int64_t out_bs);

// Y[b][m][n] = sum_k X[b][m][k] * W[b][.]: M in 1..8 (decode rows). W is
// [K][N] (N contiguous, row stride ldw) or, when K-major, [N][K] (K
// contiguous, row stride ldw). Strides in elements; batch strides x_bs,
// w_bs, y_bs. N-contiguous W is split over K into `ksplit` chunks of
// `kchunk` rows; `partials` then holds batch*ksplit*M*N floats.
struct GemvParams {
  int batch = 1, M = 1, N = 0, K = 0;
  int64_t ldx = 0, ldw = 0, ldy = 0;
  int64_t x_bs = 0, w_bs = 0, y_bs = 0;
  int kchunk = 0, ksplit = 1;
  int out_kind = 0;  // 0 bf16, 1 f16, 2 f32
};
// Columns per workgroup of the N-contiguous kernel (64 lanes x 8).
constexpr int kGemvCols = 512;
// Split plan for an N-contiguous GEMV: fills kchunk / ksplit so the launch
// reaches about `target_blocks` workgroups.
void plan_gemv_split(GemvParams* p, int target_blocks = 512);
void launch_gemv(hipStream_t s, const GemvParams& p, const void* X, const void* W, void* Y, float* partials, bool f16,
                 bool w_kmajor);

// Decode GEMVs sharing one X (the reference's dot group: Q/K/V projections
// of one normalized row, executable_metal_graph_lowering_fusion.zig:394-424):
// up to 4 weights W_i [K][N_i] (N contiguous, row stride ldw), outputs Y_i
// [M][N_i] (row stride ldy), optionally Y_i = add_i + round(X.W_i) with add_i
// shaped like Y_i. One launch, one pass over each W, no split-K partials.
constexpr int kMaxGemvMembers = 4;
constexpr int64_t kGemvWideMaxX = 16384;  // M * K floats staged in LDS
struct GemvMember {
  const void* W = nullptr;
  void* Y = nullptr;
  const void* add = nullptr;
  int N = 0;
  int64_t ldw = 0, ldy = 0;
  int tile0 = 0;  // first workgroup of this member (set by launch_gemv_wide)
};
struct GemvGroup {
  int count = 0, M = 1, K = 0;
  int64_t ldx = 0;
  int out_kind = 0;  // 0 bf16, 1 f16, 2 f32
  GemvMember m[kMaxGemvMembers];
};
// Columns per workgroup for a group (32 or 64; environment PJRTX_GEMV_COLS
// forces one) and the group's workgroup count at that width.
int gemv_wide_cols(const GemvGroup& g);
int gemv_wide_tiles(const GemvGroup& g);
// True when the one-pass kernel applies: M <= 4, M*K <= kGemvWideMaxX and at
// least 32 workgroups over the members (gemv_wide_tiles).
bool gemv_wide_fits(int M, int K, int total_tiles);
void launch_gemv_wide(hipStream_t s, GemvGroup g, const void* X, bool f16);

// Fallback with arbitrary element strides.
struct FmaGemmParams {
  int64_t batch = 1, M = 0, N = 0, K = 0;
  int64_t a_bs = 0, a_ms = 0, a_ks = 0;
  int64_t b_bs = 0, b_ns = 0, b_ks = 0;
};
void launch_fma_gemm(hipStream_t s, const FmaGemmParams& p, const void* A, const void* B, void* C, DType in, DType out);

}  // namespace pjrtx
