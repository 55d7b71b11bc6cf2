// dot_general kernels for gfx950.
//
//  * mfma_gemm: C[b] = A[b] (MxK) * B[b] (KxN) for bf16 / f16 inputs with f32
//    accumulation on v_mfma_f32_16x16x32_{bf16,f16}. 128x128 block tile,
//    BK = 64, 256 threads (4 waves in 2x2, 64x64 each), LDS double buffer,
//    B either N-contiguous ([K][N], transposed into LDS) or K-contiguous
//    ([N][K]). The C tile is staged through LDS and written with 16-byte
//    coalesced stores. XCD-aware tile order: the 8 XCDs each get contiguous
//    runs of tiles so neighbouring tiles share an L2.
//  * gemv: M <= 8 rows (decode), split over K with a deterministic second
//    pass; memory-bound on the weight stream.
//  * fma_gemm: scalar fallback for f32 / f64 and unaligned layouts.
//
// Replaces the reference's dot_general (reference:
// src/backend/mlx_metal/api.cc:3349-3498, mlx::matmul / tensordot) and the
// MSL dot steps (metal_graph_dot.zig:14-324, scalar FMA only).
#include <hip/hip_runtime.h>

#include "common.h"
#include "kernels/dot.h"

namespace pjrtx {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 128, BK = 64, PAD = 8, LDK = BK + PAD;  // LDS row stride in elements
constexpr int LDC = BN + PAD;

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

template <bool kF16>
__device__ __forceinline__ f32x4 mfma16(const u32x4& a, const u32x4& b, const f32x4& c) {
  if constexpr (kF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
                                                   0);
  }
}

// kBKMajor: B stored [N][K] (K contiguous). Otherwise [K][N] (N contiguous).
// kOutBytes: 2 (bf16/f16 output, same type as inputs) or 4 (f32 output).
template <bool kF16, bool kBKMajor, int kOutBytes>
__global__ void __launch_bounds__(256) mfma_gemm(GemmParams p, const uint16_t* __restrict__ A,
                                                 const uint16_t* __restrict__ B, void* __restrict__ C) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * LDK];

  // Tile index with XCD-aware remap: hardware deals consecutive workgroups to
  // the 8 XCDs in turn; give each XCD a contiguous range of tiles instead.
  const int tiles_m = (p.M + BM - 1) / BM, tiles_n = (p.N + BN - 1) / BN;
  const int per_batch = tiles_m * tiles_n;
  const int total = per_batch * p.batch;
  int bid = blockIdx.x;
  if (total % 8 == 0) bid = (bid % 8) * (total / 8) + bid / 8;
  const int b = bid / per_batch;
  const int t = bid - b * per_batch;
  // Within a batch, walk tiles in groups of 8 rows of tiles (L2 reuse of B).
  const int group = 8;
  const int gsize = group * tiles_n;
  const int g = t / gsize;
  const int first_m = g * group;
  const int gm = min(tiles_m - first_m, group);
  const int tm = first_m + (t - g * gsize) % gm;
  const int tn = (t - g * gsize) / gm;
  const int m0 = tm * BM, n0 = tn * BN;

  const uint16_t* Ab = A + (int64_t)b * p.a_batch_stride;
  const uint16_t* Bb = B + (int64_t)b * p.b_batch_stride;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;

  u32x4 ra[4], rb[4];
  const u32x4 zero = {0u, 0u, 0u, 0u};

  auto load_a = [&](int k0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = tid + 256 * j;
      const int row = c >> 3, kc = (c & 7) * 8;
      const int m = m0 + row, k = k0 + kc;
      ra[j] = (m < p.M && k + 8 <= p.K) ? *reinterpret_cast<const u32x4*>(Ab + (int64_t)m * p.lda + k) : zero;
      if (m < p.M && k < p.K && k + 8 > p.K) {  // ragged K tail
        uint16_t tmp[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) tmp[e] = (k + e < p.K) ? Ab[(int64_t)m * p.lda + k + e] : (uint16_t)0;
        ra[j] = *reinterpret_cast<u32x4*>(tmp);
      }
    }
  };
  auto load_b = [&](int k0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = tid + 256 * j;
      if constexpr (kBKMajor) {
        const int row = c >> 3, kc = (c & 7) * 8;  // row = n
        const int n = n0 + row, k = k0 + kc;
        rb[j] = (n < p.N && k + 8 <= p.K) ? *reinterpret_cast<const u32x4*>(Bb + (int64_t)n * p.ldb + k) : zero;
        if (n < p.N && k < p.K && k + 8 > p.K) {
          uint16_t tmp[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) tmp[e] = (k + e < p.K) ? Bb[(int64_t)n * p.ldb + k + e] : (uint16_t)0;
          rb[j] = *reinterpret_cast<u32x4*>(tmp);
        }
      } else {
        const int kr = c >> 4, nc = (c & 15) * 8;  // 64 k rows x 16 chunks of 8 n
        const int k = k0 + kr, n = n0 + nc;
        rb[j] = (k < p.K && n + 8 <= p.N) ? *reinterpret_cast<const u32x4*>(Bb + (int64_t)k * p.ldb + n) : zero;
        if (k < p.K && n < p.N && n + 8 > p.N) {
          uint16_t tmp[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) tmp[e] = (n + e < p.N) ? Bb[(int64_t)k * p.ldb + n + e] : (uint16_t)0;
          rb[j] = *reinterpret_cast<u32x4*>(tmp);
        }
      }
    }
  };
  auto store_lds = [&](int buf) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = tid + 256 * j;
      const int row = c >> 3, kc = (c & 7) * 8;
      *reinterpret_cast<u32x4*>(&As[buf][row * LDK + kc]) = ra[j];
      if constexpr (kBKMajor) {
        *reinterpret_cast<u32x4*>(&Bs[buf][row * LDK + kc]) = rb[j];
      } else {
        const int kr = c >> 4, nc = (c & 15) * 8;
        const uint16_t* v = reinterpret_cast<const uint16_t*>(&rb[j]);
#pragma unroll
        for (int e = 0; e < 8; ++e) Bs[buf][(nc + e) * LDK + kr] = v[e];
      }
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int kt_count = (p.K + BK - 1) / BK;
  load_a(0);
  load_b(0);
  store_lds(0);
  __syncthreads();
  for (int kt = 0; kt < kt_count; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < kt_count) {
      load_a((kt + 1) * BK);
      load_b((kt + 1) * BK);
    }
#pragma unroll
    for (int kk = 0; kk < BK; kk += 32) {
      u32x4 af[4], bfr[4];
      const int kofs = kk + (lane >> 4) * 8;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[i] = *reinterpret_cast<const u32x4*>(&As[buf][(wm * 64 + i * 16 + (lane & 15)) * LDK + kofs]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        bfr[j] = *reinterpret_cast<const u32x4*>(&Bs[buf][(wn * 64 + j * 16 + (lane & 15)) * LDK + kofs]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16<kF16>(af[i], bfr[j], acc[i][j]);
    }
    if (kt + 1 < kt_count) store_lds(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: lane holds D[(lane/16)*4 + r][lane%16] of each 16x16 subtile.
  if constexpr (kOutBytes == 2) {
    uint16_t* Cs = &As[0][0];  // 128 x LDC staging tile (fits in As)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = wm * 64 + i * 16 + (lane >> 4) * 4 + r;
          const int col = wn * 64 + j * 16 + (lane & 15);
          const float v = acc[i][j][r];
          Cs[row * LDC + col] = kF16 ? f32_to_f16_bits(v) : f32_to_bf16_rne(v);
        }
    __syncthreads();
    uint16_t* Cb = reinterpret_cast<uint16_t*>(C) + (int64_t)b * p.M * p.ldc;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int c = tid + 256 * j;  // 2048 chunks of 8
      const int row = c >> 4, nc = (c & 15) * 8;
      const int m = m0 + row, n = n0 + nc;
      if (m >= p.M) continue;
      const u32x4 v = *reinterpret_cast<const u32x4*>(&Cs[row * LDC + nc]);
      if (n + 8 <= p.N && p.ldc % 8 == 0) {
        *reinterpret_cast<u32x4*>(Cb + (int64_t)m * p.ldc + n) = v;
      } else {
        const uint16_t* e = reinterpret_cast<const uint16_t*>(&v);
        for (int q = 0; q < 8 && n + q < p.N; ++q) Cb[(int64_t)m * p.ldc + n + q] = e[q];
      }
    }
  } else {
    float* Cb = reinterpret_cast<float*>(C) + (int64_t)b * p.M * p.ldc;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + wm * 64 + i * 16 + (lane >> 4) * 4 + r;
          const int n = n0 + wn * 64 + j * 16 + (lane & 15);
          if (m < p.M && n < p.N) Cb[(int64_t)m * p.ldc + n] = acc[i][j][r];
        }
  }
}

// ------------------------------------------------------------------- GEMV
// y[m][n] = sum_k x[m][k] * W[k][n] for M <= 8, W N-contiguous ([K][N]) or
// K-contiguous ([N][K]). Pass 1: each workgroup reduces a K-chunk for 2048
// (N-contiguous) or 256 (K-contiguous) columns into f32 partials; pass 2 sums
// the chunks in order and rounds.
template <int kM, bool kF16>
__global__ void __launch_bounds__(256) gemv_nmajor(GemvParams p, const uint16_t* __restrict__ X,
                                                   const uint16_t* __restrict__ W, float* __restrict__ part) {
  const int n = (blockIdx.x * 256 + threadIdx.x) * 8;
  const int kc = blockIdx.y;
  const int k0 = kc * p.kchunk, k1 = min(p.K, k0 + p.kchunk);
  float acc[kM][8];
#pragma unroll
  for (int m = 0; m < kM; ++m)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[m][e] = 0.f;
  if (n < p.N) {
    const bool full = n + 8 <= p.N;
    for (int k = k0; k < k1; ++k) {
      uint16_t w[8];
      if (full) {
        *reinterpret_cast<u32x4*>(w) = *reinterpret_cast<const u32x4*>(W + (int64_t)k * p.ldw + n);
      } else {
        for (int e = 0; e < 8; ++e) w[e] = (n + e < p.N) ? W[(int64_t)k * p.ldw + n + e] : (uint16_t)0;
      }
#pragma unroll
      for (int m = 0; m < kM; ++m) {
        const float xv = kF16 ? f16_bits_to_f32(X[(int64_t)m * p.ldx + k]) : bf16_bits_to_f32(X[(int64_t)m * p.ldx + k]);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[m][e] += xv * (kF16 ? f16_bits_to_f32(w[e]) : bf16_bits_to_f32(w[e]));
      }
    }
#pragma unroll
    for (int m = 0; m < kM; ++m)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (n + e < p.N) part[((int64_t)kc * kM + m) * p.N + n + e] = acc[m][e];
  }
}

template <int kM, bool kF16>
__global__ void __launch_bounds__(256) gemv_kmajor(GemvParams p, const uint16_t* __restrict__ X,
                                                   const uint16_t* __restrict__ W, float* __restrict__ part) {
  // One wave per column n; lanes stride over K in 8-element chunks.
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int kc = blockIdx.y;
  const int k0 = kc * p.kchunk, k1 = min(p.K, k0 + p.kchunk);
  if (n >= p.N) return;
  float acc[kM];
#pragma unroll
  for (int m = 0; m < kM; ++m) acc[m] = 0.f;
  for (int k = k0 + lane * 8; k < k1; k += 512) {
    uint16_t w[8];
    if (k + 8 <= k1) *reinterpret_cast<u32x4*>(w) = *reinterpret_cast<const u32x4*>(W + (int64_t)n * p.ldw + k);
    else
      for (int e = 0; e < 8; ++e) w[e] = (k + e < k1) ? W[(int64_t)n * p.ldw + k + e] : (uint16_t)0;
#pragma unroll
    for (int m = 0; m < kM; ++m)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint16_t xb = (k + e < k1) ? X[(int64_t)m * p.ldx + k + e] : (uint16_t)0;
        acc[m] += (kF16 ? f16_bits_to_f32(xb) : bf16_bits_to_f32(xb)) * (kF16 ? f16_bits_to_f32(w[e]) : bf16_bits_to_f32(w[e]));
      }
  }
#pragma unroll
  for (int m = 0; m < kM; ++m) {
    float v = acc[m];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    if (lane == 0) part[((int64_t)kc * kM + m) * p.N + n] = v;
  }
}

template <int kM>
__global__ void __launch_bounds__(256) gemv_finish(GemvParams p, const float* __restrict__ part, void* __restrict__ Y,
                                                   int out_kind) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // over kM * N
  if (i >= (int64_t)kM * p.N) return;
  const int m = (int)(i / p.N), n = (int)(i - (int64_t)m * p.N);
  float s = 0.f;
  for (int kc = 0; kc < p.ksplit; ++kc) s += part[((int64_t)kc * kM + m) * p.N + n];
  if (out_kind == 0) reinterpret_cast<uint16_t*>(Y)[(int64_t)m * p.ldy + n] = f32_to_bf16_rne(s);
  else if (out_kind == 1) reinterpret_cast<uint16_t*>(Y)[(int64_t)m * p.ldy + n] = f32_to_f16_bits(s);
  else reinterpret_cast<float*>(Y)[(int64_t)m * p.ldy + n] = s;
}

// --------------------------------------------------------------- fallback
template <typename T, typename Acc>
__global__ void __launch_bounds__(256) fma_gemm(FmaGemmParams p, const T* __restrict__ A, const T* __restrict__ B,
                                                T* __restrict__ C) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)p.batch * p.M * p.N;
  if (i >= total) return;
  const int64_t b = i / ((int64_t)p.M * p.N);
  const int64_t r = i - b * p.M * p.N;
  const int64_t m = r / p.N, n = r - m * p.N;
  Acc s = 0;
  const T* a = A + b * p.a_bs + m * p.a_ms;
  const T* bb = B + b * p.b_bs + n * p.b_ns;
  for (int64_t k = 0; k < p.K; ++k) s += (Acc)a[k * p.a_ks] * (Acc)bb[k * p.b_ks];
  C[i] = (T)s;
}

// f16/bf16 storage variant of the fallback (bits in uint16_t).
__global__ void __launch_bounds__(256) fma_gemm_16(FmaGemmParams p, const uint16_t* __restrict__ A,
                                                   const uint16_t* __restrict__ B, void* __restrict__ C, int in_f16,
                                                   int out_kind) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)p.batch * p.M * p.N;
  if (i >= total) return;
  const int64_t b = i / ((int64_t)p.M * p.N);
  const int64_t r = i - b * p.M * p.N;
  const int64_t m = r / p.N, n = r - m * p.N;
  float s = 0.f;
  const uint16_t* a = A + b * p.a_bs + m * p.a_ms;
  const uint16_t* bb = B + b * p.b_bs + n * p.b_ns;
  for (int64_t k = 0; k < p.K; ++k) {
    const float x = in_f16 ? f16_bits_to_f32(a[k * p.a_ks]) : bf16_bits_to_f32(a[k * p.a_ks]);
    const float y = in_f16 ? f16_bits_to_f32(bb[k * p.b_ks]) : bf16_bits_to_f32(bb[k * p.b_ks]);
    s += x * y;
  }
  if (out_kind == 0) reinterpret_cast<uint16_t*>(C)[i] = f32_to_bf16_rne(s);
  else if (out_kind == 1) reinterpret_cast<uint16_t*>(C)[i] = f32_to_f16_bits(s);
  else reinterpret_cast<float*>(C)[i] = s;
}

void check(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) fail(Code::kInternal, strformat("%s launch failed: %s", what, hipGetErrorString(e)));
}

}  // namespace

void launch_mfma_gemm(hipStream_t s, const GemmParams& p, const void* A, const void* B, void* C, bool f16, bool b_kmajor,
                      int out_bytes) {
  const int64_t tiles = (int64_t)((p.M + BM - 1) / BM) * ((p.N + BN - 1) / BN) * p.batch;
  if (tiles == 0 || p.K == 0) fail(Code::kInternal, "mfma_gemm: empty problem must be handled by the caller");
  PJRTX_CHECK(tiles < (int64_t(1) << 31), Code::kUnimplemented, "mfma_gemm: too many tiles");
  const dim3 grid(static_cast<unsigned>(tiles)), block(256);
  const uint16_t* a = static_cast<const uint16_t*>(A);
  const uint16_t* b = static_cast<const uint16_t*>(B);
#define PJRTX_GEMM(F16, KM, OB) hipLaunchKernelGGL((mfma_gemm<F16, KM, OB>), grid, block, 0, s, p, a, b, C)
  if (out_bytes == 2) {
    if (f16) { if (b_kmajor) PJRTX_GEMM(true, true, 2); else PJRTX_GEMM(true, false, 2); }
    else { if (b_kmajor) PJRTX_GEMM(false, true, 2); else PJRTX_GEMM(false, false, 2); }
  } else {
    if (f16) { if (b_kmajor) PJRTX_GEMM(true, true, 4); else PJRTX_GEMM(true, false, 4); }
    else { if (b_kmajor) PJRTX_GEMM(false, true, 4); else PJRTX_GEMM(false, false, 4); }
  }
#undef PJRTX_GEMM
  check("mfma_gemm");
}

void launch_gemv(hipStream_t s, const GemvParams& p, const void* X, const void* W, void* Y, float* partials, bool f16,
                 bool w_kmajor, int out_kind) {
  const uint16_t* x = static_cast<const uint16_t*>(X);
  const uint16_t* w = static_cast<const uint16_t*>(W);
#define PJRTX_GEMV(M)                                                                                              \
  case M:                                                                                                          \
    if (w_kmajor) {                                                                                                \
      const dim3 g((p.N + 3) / 4, p.ksplit);                                                                       \
      if (f16) hipLaunchKernelGGL((gemv_kmajor<M, true>), g, dim3(256), 0, s, p, x, w, partials);                  \
      else hipLaunchKernelGGL((gemv_kmajor<M, false>), g, dim3(256), 0, s, p, x, w, partials);                     \
    } else {                                                                                                       \
      const dim3 g((p.N + 2047) / 2048, p.ksplit);                                                                 \
      if (f16) hipLaunchKernelGGL((gemv_nmajor<M, true>), g, dim3(256), 0, s, p, x, w, partials);                  \
      else hipLaunchKernelGGL((gemv_nmajor<M, false>), g, dim3(256), 0, s, p, x, w, partials);                     \
    }                                                                                                              \
    hipLaunchKernelGGL((gemv_finish<M>), dim3((unsigned)(((int64_t)M * p.N + 255) / 256)), dim3(256), 0, s, p,     \
                       partials, Y, out_kind);                                                                     \
    break;
  switch (p.M) {
    PJRTX_GEMV(1)
    PJRTX_GEMV(2)
    PJRTX_GEMV(3)
    PJRTX_GEMV(4)
    PJRTX_GEMV(5)
    PJRTX_GEMV(6)
    PJRTX_GEMV(7)
    PJRTX_GEMV(8)
    default: fail(Code::kInternal, "gemv: M must be 1..8");
  }
#undef PJRTX_GEMV
  check("gemv");
}

void launch_fma_gemm(hipStream_t s, const FmaGemmParams& p, const void* A, const void* B, void* C, DType in,
                     DType out) {
  const int64_t total = (int64_t)p.batch * p.M * p.N;
  if (total == 0) return;
  const dim3 grid(static_cast<unsigned>((total + 255) / 256)), block(256);
  if (in == DType::kF32 && out == DType::kF32) {
    hipLaunchKernelGGL((fma_gemm<float, float>), grid, block, 0, s, p, (const float*)A, (const float*)B, (float*)C);
  } else if (in == DType::kF64 && out == DType::kF64) {
    hipLaunchKernelGGL((fma_gemm<double, double>), grid, block, 0, s, p, (const double*)A, (const double*)B, (double*)C);
  } else if ((in == DType::kBF16 || in == DType::kF16) &&
             (out == DType::kBF16 || out == DType::kF16 || out == DType::kF32)) {
    const int ok = out == DType::kBF16 ? 0 : (out == DType::kF16 ? 1 : 2);
    hipLaunchKernelGGL(fma_gemm_16, grid, block, 0, s, p, (const uint16_t*)A, (const uint16_t*)B, C,
                       in == DType::kF16 ? 1 : 0, ok);
  } else if (in == DType::kS32 && out == DType::kS32) {
    hipLaunchKernelGGL((fma_gemm<int32_t, int32_t>), grid, block, 0, s, p, (const int32_t*)A, (const int32_t*)B,
                       (int32_t*)C);
  } else {
    fail(Code::kUnimplemented, strformat("dot_general %s -> %s is not supported", dtype_name(in), dtype_name(out)));
  }
  check("fma_gemm");
}

}  // namespace pjrtx
