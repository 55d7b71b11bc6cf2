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

#include <algorithm>
#include <type_traits>

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

// ------------------------------------------------------------- large GEMM
// gemm_nt_256: C[b] = A[b] (M x K, K contiguous) * B[b]^T (N x K, K
// contiguous) for products with enough 256 x 256 tiles to fill the GPU.
//  * 256 x 256 block tile, 64-deep k-tiles, 512 threads: 2 x 4 waves of
//    128 x 64 (4 x 2 blocks of v_mfma_f32_32x32x16, 128 f32 accumulators a
//    lane), two waves per SIMD.
//  * A and B k-tiles go from global memory straight into LDS (buffer loads
//    with the LDS destination, 16 bytes a lane, eight 128-byte row pieces per
//    instruction); two stages. Waves 0-3 issue all of the loads, so on every
//    SIMD one of the two waves never waits on a load issue.
//  * One barrier per k-tile, placed before the tile's last 16-deep slab: by
//    then every wave holds its last-slab fragments in registers and has read
//    all of the tile, so the barrier both publishes tile kt+1 (loaded during
//    tile kt) and frees tile kt's stage for tile kt+2.
//  * LDS rows are 64 elements (eight 16-byte chunks), chunk c of row r stored
//    at c ^ ((r >> 1) & 7): the fragment reads of 16 consecutive rows hit
//    distinct banks. A load places lane L's 16 bytes in slot L of its 1 KB,
//    so the swizzle is applied on the global side (the lane filling slot
//    (r, c) fetches chunk c ^ f(r)).
//  * Rows past M or N and 8-element k chunks past K read as zero: the whole
//    offset of every load is in its lane part, which the buffer range check
//    covers, and chunks past K get an offset beyond the range.
constexpr int GBM = 256, GBN = 256, GBK = 64, GTHREADS = 512;
constexpr int kGemmLoadWaves = 4;  // waves 0..3 issue the LDS loads
constexpr int kGemmLoadsPerWave = (GBM + GBN) / 8 / kGemmLoadWaves;  // 1 KB loads a load wave issues per tile

typedef __attribute__((address_space(3))) void* gemm_lds_ptr;
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ int gswz(int row, int chunk) { return row * GBK + ((chunk ^ ((row >> 1) & 7)) << 3); }
constexpr int gemm_vmcnt0() { return (7 << 4) | (15 << 8); }  // s_waitcnt vmcnt(0) alone

template <bool kF16>
__device__ __forceinline__ f32x16 mfma32(const u32x4& a, const u32x4& b, const f32x16& c) {
  if constexpr (kF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
                                                   0);
}

// kBN: B is N-contiguous ([K][N], row stride ldb) instead of K-contiguous.
// Its k-tile is then stored as 64 rows of 256 columns (512 bytes, chunk c of
// row k at c ^ 4 (k & 3): the 32 lanes of a transposing read, 4 rows x 64
// bytes, hit 64 distinct banks), and the B fragments come from transposing LDS
// reads (ds_read_b64_tr_b16: lane j of a 16-lane group gets element j & 3
// of the 8-byte pieces lanes 4 e + (j >> 2) address, e = 0..3; lanes
// addressing 4 consecutive k rows x 16 columns return 4 consecutive k of
// one column, half a fragment), so no transposed copy of B is made.
template <bool kF16, int kOutBytes, bool kBN>
__global__ void __launch_bounds__(GTHREADS, 1) gemm_nt_256(GemmParams p, const uint16_t* __restrict__ A,
                                                            const uint16_t* __restrict__ B, void* __restrict__ C) {
  constexpr int STAGE = (GBM + GBN) * GBK;  // elements per stage
  __shared__ __attribute__((aligned(1024))) uint16_t smem[2 * STAGE];

  const int tiles_m = (p.M + GBM - 1) / GBM, tiles_n = (p.N + GBN - 1) / GBN;
  const int per_batch = tiles_m * tiles_n;
  const int total = per_batch * p.batch;
  int bid = blockIdx.x;
  if (total % 8 == 0) bid = (bid % 8) * (total / 8) + bid / 8;  // contiguous tile runs per XCD
  const int b = bid / per_batch;
  const int t = bid - b * per_batch;
  const int group = 8;  // walk 8 tile-rows at a time so B k-tiles are reused from L2
  const int gsize = group * tiles_n;
  const int g = t / gsize;
  const int first_m = g * group;
  const int gm = min(tiles_m - first_m, group);
  const int tm = first_m + (t - g * gsize) % gm;
  const int tn = (t - g * gsize) / gm;
  const int m0 = tm * GBM, n0 = tn * GBN;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;

  // Buffer resources over this tile's row panels; the range ends with the
  // last valid row's K elements.
  const uint16_t* Ap = A + (int64_t)b * p.a_batch_stride + (int64_t)m0 * p.lda;
  const uint16_t* Bp = B + (int64_t)b * p.b_batch_stride + (kBN ? (int64_t)n0 : (int64_t)n0 * p.ldb);
  const int rows_a = min(GBM, p.M - m0), rows_b = min(GBN, p.N - n0);
  const __amdgpu_buffer_rsrc_t ars = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(Ap), 0, (int)(((int64_t)(rows_a - 1) * p.lda + p.K) * 2), 0x00020000);
  // N-contiguous B: the range ends with row K-1's last valid column, so k
  // rows past K read as zero; columns past N are masked per load below.
  const __amdgpu_buffer_rsrc_t brs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(Bp), 0,
      kBN ? (int)(((int64_t)(p.K - 1) * p.ldb + rows_b) * 2) : (int)(((int64_t)(rows_b - 1) * p.ldb + p.K) * 2),
      0x00020000);
  const int nk = (p.K + GBK - 1) / GBK;
  const int ktail = p.K - (nk - 1) * GBK;  // valid elements of the last k-tile

  // Load lanes: load i of load wave w fills stage rows (4 i + w) * 8 + L / 8,
  // slot L % 8; its global chunk is (L % 8) ^ f(row), and f depends only on
  // row % 16 = 8 (w % 2) + L / 8.
  const int lrow = lane >> 3, lslot = lane & 7;
  const int lchunk = lslot ^ ((((wave & 1) * 8 + lrow) >> 1) & 7);
  const uint32_t tail_oob = lchunk * 8 >= ktail ? 0x80000000u : 0u;  // beyond the range of any resource
  uint32_t aoff[kGemmLoadsPerWave / 2], boff[kGemmLoadsPerWave / 2];
#pragma unroll
  for (int i = 0; i < kGemmLoadsPerWave / 2; ++i) {
    const int row = (i * kGemmLoadWaves + wave) * 8 + lrow;
    aoff[i] = (uint32_t)(row * p.lda * 2 + lchunk * 16);
    if constexpr (kBN) {
      // Load i of load wave w fills k rows 2 (4 i + w) + L / 32, slot L % 32
      // (global chunk (L % 32) ^ 4 (k & 3)); chunks past N get an offset
      // beyond the range.
      const int krow = (i * kGemmLoadWaves + wave) * 2 + (lane >> 5);
      const int chunk = (lane & 31) ^ ((krow & 3) << 2);
      boff[i] = (uint32_t)(krow * p.ldb * 2 + chunk * 16) | (chunk * 8 >= rows_b ? 0x80000000u : 0u);
    } else {
      boff[i] = (uint32_t)(row * p.ldb * 2 + lchunk * 16);
    }
  }
  auto load_tile = [&](int kt, int stage) {
    uint16_t* st = smem + stage * STAGE;
    const uint32_t kb = (uint32_t)(kt * GBK * 2);
    const uint32_t oob = kt == nk - 1 ? tail_oob : 0u;
#pragma unroll
    for (int i = 0; i < kGemmLoadsPerWave / 2; ++i) {
      const int row = (i * kGemmLoadWaves + wave) * 8;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ars, (gemm_lds_ptr)(st + row * GBK), 16, (aoff[i] + kb) | oob, 0, 0, 0);
    }
    if constexpr (kBN) {
      const uint32_t kr = (uint32_t)(kt * GBK * p.ldb * 2);
#pragma unroll
      for (int i = 0; i < kGemmLoadsPerWave / 2; ++i) {
        const int krow = (i * kGemmLoadWaves + wave) * 2;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(brs, (gemm_lds_ptr)(st + GBM * GBK + krow * GBN), 16, boff[i] + kr, 0,
                                                 0, 0);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kGemmLoadsPerWave / 2; ++i) {
        const int row = (i * kGemmLoadWaves + wave) * 8;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(brs, (gemm_lds_ptr)(st + (GBM + row) * GBK), 16,
                                                 (boff[i] + kb) | oob, 0, 0, 0);
      }
    }
  };

  // Fragments of v_mfma_f32_32x32x16: lane L holds row L % 32 of a 32-row
  // block, k chunk 2 s + L / 32 of slab s; f(row) = f(L % 32).
  const int fr = lane & 31, fh = lane >> 5;
  int loff[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) loff[s] = gswz(fr, 2 * s + fh);
  // N-contiguous B: lane L (16-lane group g = L / 16, e = (L % 16) / 4,
  // c = L % 4) of transposing read h addresses k row 16 s + 8 (g / 2) + 4 h +
  // e, columns wn 64 + 32 j + 16 (g % 2) + 4 c .. + 3.
  int troff[4][2][2];
  if constexpr (kBN) {
    const int g4 = lane >> 4, e4 = (lane >> 2) & 3, c4 = lane & 3;
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int k = 16 * s + 8 * (g4 >> 1) + 4 * h + e4;
          const int chunk = wn * 8 + 4 * j + 2 * (g4 & 1) + (c4 >> 1);
          troff[s][h][j] = k * GBN + ((chunk ^ ((k & 3) << 2)) << 3) + 4 * (c4 & 1);
        }
  }
  u32x4 fa[2][4], fb[2][2];
  auto read_b = [&](const uint16_t* stb, int s, int j) -> u32x4 {
    if constexpr (kBN) {
      typedef short v4i16 __attribute__((ext_vector_type(4)));
      typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
      typedef __attribute__((address_space(3))) uint16_t lds_u16;
      const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)((lds_u16*)(stb + troff[s][0][j])));
      const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)((lds_u16*)(stb + troff[s][1][j])));
      typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
      const u32x2_t l2 = __builtin_bit_cast(u32x2_t, lo), h2 = __builtin_bit_cast(u32x2_t, hi);
      return u32x4{l2[0], l2[1], h2[0], h2[1]};
    } else {
      return *reinterpret_cast<const u32x4*>(stb + (wn * 64 + 32 * j) * GBK + loff[s]);
    }
  };
  auto read_slab = [&](int stage, int s, int buf) {
    const uint16_t* as = smem + stage * STAGE + (wm * 128) * GBK;
    const uint16_t* stb = smem + stage * STAGE + GBM * GBK;
    // In the order the MFMAs first use them.
    fa[buf][0] = *reinterpret_cast<const u32x4*>(as + loff[s]);
    fb[buf][0] = read_b(stb, s, 0);
    fb[buf][1] = read_b(stb, s, 1);
#pragma unroll
    for (int i = 1; i < 4; ++i) fa[buf][i] = *reinterpret_cast<const u32x4*>(as + i * 32 * GBK + loff[s]);
  };
  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  auto mma = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = mfma32<kF16>(fa[buf][i], fb[buf][j], acc[i][j]);
  };
  // One MFMA, then one fragment read, for each read of the slab; then the
  // remaining MFMAs.
  auto interleave_reads = [&]() {
    constexpr int kReads = kBN ? 8 : 6;
#pragma unroll
    for (int q = 0; q < kReads; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    if constexpr (kReads < 8) __builtin_amdgcn_sched_group_barrier(0x008, 8 - kReads, 0);
  };

  // Tile kt: slabs 0..2 read the next slab's fragments while multiplying;
  // then the barrier; then tile kt+1's first slab is read and tile kt+2's
  // loads issued while the last slab multiplies. Tile indices past the last
  // reload it into the free stage, so the load waves' counts stay uniform.
  auto tile_body = [&](int kt, bool last, auto loader) {
    constexpr bool kLoads = decltype(loader)::value;
    const int cur = kt & 1;
#pragma unroll
    for (int s = 0; s < 3; ++s) {
      read_slab(cur, s + 1, (s + 1) & 1);
      mma(s & 1);
      interleave_reads();
      __builtin_amdgcn_sched_barrier(0);
    }
    if (!last) {
      // Own loads of tile kt+1 landed and own reads of tile kt done, then
      // everyone's.
      __builtin_amdgcn_s_waitcnt(gemm_vmcnt0() & ~(15 << 8));
      __builtin_amdgcn_s_barrier();
      read_slab(cur ^ 1, 0, 0);
      if constexpr (kLoads) load_tile(min(kt + 2, nk - 1), cur);
    }
    mma(1);
    interleave_reads();
    if constexpr (kLoads) {
#pragma unroll
      for (int q = 0; q < kGemmLoadsPerWave; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  auto run = [&](auto loader) {
    constexpr bool kLoads = decltype(loader)::value;
    if constexpr (kLoads) {
      load_tile(0, 0);
      load_tile(min(1, nk - 1), 1);
      __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8) | (kGemmLoadsPerWave & 15) | ((kGemmLoadsPerWave >> 4) << 14));
    }
    __builtin_amdgcn_s_barrier();
    read_slab(0, 0, 0);
    for (int kt = 0; kt < nk - 1; ++kt) tile_body(kt, false, loader);
    tile_body(nk - 1, true, loader);
  };
  if (wave < kGemmLoadWaves) run(std::true_type{});
  else run(std::false_type{});
  __builtin_amdgcn_s_waitcnt(gemm_vmcnt0());
  __syncthreads();

  // Epilogue: lane L holds rows 8 (r / 4) + 4 (L / 32) + r % 4, column L % 32
  // of each 32 x 32 block.
  const int wrow0 = m0 + wm * 128, wcol0 = n0 + wn * 64;
  if constexpr (kOutBytes == 2) {
    uint16_t* cs = smem + wave * 128 * GBK;  // this wave's 128 x 64 staging tile
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = i * 32 + (r >> 2) * 8 + fh * 4 + (r & 3);
          const int col = j * 32 + fr;
          const float v = acc[i][j][r];
          cs[gswz(row, col >> 3) + (col & 7)] = kF16 ? f32_to_f16_bits(v) : f32_to_bf16_rne(v);
        }
    __syncthreads();
    uint16_t* Cb = reinterpret_cast<uint16_t*>(C) + (int64_t)b * p.M * p.ldc;
#pragma unroll
    for (int tt = 0; tt < 16; ++tt) {
      const int c = lane + 64 * tt;  // 1024 chunks of 8
      const int row = c >> 3, ch = c & 7;
      const int m = wrow0 + row, n = wcol0 + ch * 8;
      if (m >= p.M || n >= p.N) continue;
      const u32x4 v = *reinterpret_cast<const u32x4*>(&cs[gswz(row, ch)]);
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
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = wrow0 + i * 32 + (r >> 2) * 8 + fh * 4 + (r & 3);
          const int n = wcol0 + j * 32 + fr;
          if (m < p.M && n < p.N) Cb[(int64_t)m * p.ldc + n] = acc[i][j][r];
        }
  }
}

// out[b][c][r] = in[b][r][c] for 16-bit elements; 64 x 64 tiles through LDS.
__global__ void __launch_bounds__(256) transpose16(const uint16_t* __restrict__ in, uint16_t* __restrict__ out,
                                                   int64_t rows, int64_t cols, int64_t in_bs, int64_t out_bs) {
  __shared__ uint16_t tile[64][66];
  const int64_t b = blockIdx.z;
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const uint16_t* src = in + b * in_bs;
  uint16_t* dst = out + b * out_bs;
  const int tid = threadIdx.x;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int c = tid + 256 * j;  // 512 chunks of 8
    const int rr = c >> 3, cc = (c & 7) * 8;
    const int64_t r = r0 + rr, col = c0 + cc;
    uint16_t v[8];
    if (r < rows && col + 8 <= cols && cols % 8 == 0) {
      *reinterpret_cast<u32x4*>(v) = *reinterpret_cast<const u32x4*>(src + r * cols + col);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (r < rows && col + e < cols) ? src[r * cols + col + e] : (uint16_t)0;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) tile[rr][cc + e] = v[e];
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int c = tid + 256 * j;
    const int oc = c >> 3, orr = (c & 7) * 8;  // output row = input column
    const int64_t orow = c0 + oc, ocol = r0 + orr;
    if (orow >= cols) continue;
    uint16_t v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = tile[orr + e][oc];
    if (ocol + 8 <= rows && rows % 8 == 0) {
      *reinterpret_cast<u32x4*>(dst + orow * rows + ocol) = *reinterpret_cast<const u32x4*>(v);
    } else {
      for (int e = 0; e < 8 && ocol + e < rows; ++e) dst[orow * rows + ocol + e] = v[e];
    }
  }
}

// ------------------------------------------------------------------- GEMV
// Decode-shaped products (M <= 8) are bound by streaming W once.
//
// gemv_n (W [K][N], N contiguous): a workgroup owns 512 columns (one 16-byte
// vector per lane) and a chunk of K rows; its 4 waves take interleaved rows,
// each lane issuing 8 row loads before using them so that ~32 KB per
// workgroup is in flight. The waves' sums are combined through LDS in wave
// order. With one K chunk the result is rounded and stored directly;
// otherwise f32 partials go to gemv_reduce, which sums the chunks in a
// fixed order (deterministic).
//
// gemv_k (W [N][K], K contiguous): G lanes share a row (G*8 >= K when K <=
// 512), so one wave covers 64/G rows; the G partial sums are folded by xor
// shuffles. One pass, no partials.
constexpr int kGemvRowsPerLane = 8;

template <bool kF16>
__device__ __forceinline__ float half_to_f32(uint16_t v) {
  return kF16 ? f16_bits_to_f32(v) : bf16_bits_to_f32(v);
}

__device__ __forceinline__ void store_out(void* Y, int64_t i, float v, int out_kind) {
  if (out_kind == 0) reinterpret_cast<uint16_t*>(Y)[i] = f32_to_bf16_rne(v);
  else if (out_kind == 1) reinterpret_cast<uint16_t*>(Y)[i] = f32_to_f16_bits(v);
  else reinterpret_cast<float*>(Y)[i] = v;
}

template <int kM, bool kF16>
__global__ void __launch_bounds__(256) gemv_n(GemvParams p, const uint16_t* __restrict__ X,
                                              const uint16_t* __restrict__ W, float* __restrict__ part,
                                              void* __restrict__ Y) {
  __shared__ float red[4][kM][kGemvCols];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int b = blockIdx.z, kc = blockIdx.y;
  const int n0 = blockIdx.x * kGemvCols;
  const int n = n0 + lane * 8;
  const int k0 = kc * p.kchunk, k1 = min(p.K, k0 + p.kchunk);
  const uint16_t* Wb = W + (int64_t)b * p.w_bs;
  const uint16_t* Xb = X + (int64_t)b * p.x_bs;
  float acc[kM][8];
#pragma unroll
  for (int m = 0; m < kM; ++m)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[m][e] = 0.f;
  const bool full = n + 8 <= p.N;
  if (n < p.N) {
    for (int kb = k0 + wave; kb < k1; kb += 4 * kGemvRowsPerLane) {
      u32x4 w[kGemvRowsPerLane];
#pragma unroll
      for (int r = 0; r < kGemvRowsPerLane; ++r) {
        const int k = kb + 4 * r;
        const uint16_t* src = Wb + (int64_t)k * p.ldw + n;
        if (k < k1 && full) {
          w[r] = *reinterpret_cast<const u32x4*>(src);
        } else {
          uint16_t t[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) t[e] = (k < k1 && n + e < p.N) ? src[e] : (uint16_t)0;
          w[r] = *reinterpret_cast<const u32x4*>(t);
        }
      }
#pragma unroll
      for (int r = 0; r < kGemvRowsPerLane; ++r) {
        const int k = kb + 4 * r;
        if (k < k1) {
          const uint16_t* we = reinterpret_cast<const uint16_t*>(&w[r]);
#pragma unroll
          for (int m = 0; m < kM; ++m) {
            const float xv = m < p.M ? half_to_f32<kF16>(Xb[(int64_t)m * p.ldx + k]) : 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[m][e] += xv * half_to_f32<kF16>(we[e]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < kM; ++m) {
    float4* dst = reinterpret_cast<float4*>(&red[wave][m][lane * 8]);
    dst[0] = make_float4(acc[m][0], acc[m][1], acc[m][2], acc[m][3]);
    dst[1] = make_float4(acc[m][4], acc[m][5], acc[m][6], acc[m][7]);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < kM * kGemvCols; i += 256) {
    const int m = i / kGemvCols, c = i - m * kGemvCols;
    const int nn = n0 + c;
    if (m >= p.M || nn >= p.N) continue;
    const float v = ((red[0][m][c] + red[1][m][c]) + red[2][m][c]) + red[3][m][c];
    if (p.ksplit == 1) {
      store_out(Y, (int64_t)b * p.y_bs + (int64_t)m * p.ldy + nn, v, p.out_kind);
    } else {
      part[(((int64_t)b * p.ksplit + kc) * p.M + m) * p.N + nn] = v;
    }
  }
}

// Sums the K-chunk partials of gemv_n: 32 columns x 8 chunk groups per
// workgroup; group g adds chunks g, g+8, ... in order, then the 8 group sums
// are added in group order.
__global__ void __launch_bounds__(256) gemv_reduce(GemvParams p, const float* __restrict__ part,
                                                   void* __restrict__ Y) {
  __shared__ float s[8][33];
  const int c = threadIdx.x & 31, g = threadIdx.x >> 5;
  const int n = blockIdx.x * 32 + c, m = blockIdx.y, b = blockIdx.z;
  float v = 0.f;
  if (n < p.N) {
    const float* src = part + ((int64_t)b * p.ksplit * p.M + m) * p.N + n;
    const int64_t step = (int64_t)p.M * p.N;
#pragma unroll 4
    for (int kc = g; kc < p.ksplit; kc += 8) v += src[kc * step];
  }
  s[g][c] = v;
  __syncthreads();
  if (g == 0 && n < p.N) {
    float t = s[0][c];
#pragma unroll
    for (int j = 1; j < 8; ++j) t += s[j][c];
    store_out(Y, (int64_t)b * p.y_bs + (int64_t)m * p.ldy + n, t, p.out_kind);
  }
}

// gemv_wide (W [K][N], N contiguous, one X for up to 4 weights): a
// 1024-thread workgroup owns kCols (32 or 64) columns of one member over
// the whole K, so no partials and no second launch. kCols / 8 lanes share a
// row (16 bytes each); lane (rg, cc) reads row w*RG + rg + 16*RG*r for
// r < 8 (eight rows in flight, RG = 64 / (kCols / 8) rows per wave), X comes
// from LDS; the row groups fold by xor shuffles and the 16 waves through LDS
// in wave order (deterministic). Narrower tiles give a narrow product more
// workgroups; consecutive narrow tiles (which share cache lines) run on one
// XCD. An optional addend (a residual) is added to the rounded product and
// rounded again, as the unfused add would.
constexpr int kWideDepth = 8;

template <int kM, bool kF16, int kCols>
__global__ void __launch_bounds__(1024) gemv_wide(GemvGroup g, const uint16_t* __restrict__ X) {
  constexpr int kLanesPerRow = kCols / 8, kRowGroups = 64 / kLanesPerRow, kRowStep = 16 * kRowGroups;
  extern __shared__ float xs[];  // kM * K
  __shared__ float red[16][kM][kCols];
  int t = blockIdx.x;
  const int tiles = gridDim.x;
  // Narrow tiles share cache lines with their neighbours: keep neighbours on
  // one XCD (consecutive workgroup ids go to different XCDs).
  if (kCols < 64 && tiles % 8 == 0) t = (t % 8) * (tiles / 8) + t / 8;
  int mi = 0;
#pragma unroll
  for (int i = 1; i < kMaxGemvMembers; ++i)
    if (i < g.count && t >= g.m[i].tile0) mi = i;
  const GemvMember mb = g.m[mi];
  const int n0 = (t - mb.tile0) * kCols;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int rg = lane / kLanesPerRow, cc = lane % kLanesPerRow;
  const int n = n0 + cc * 8;
  const int K = g.K;
  for (int i = threadIdx.x; i < g.M * K; i += 1024) {
    const int m = i / K, k = i - m * K;
    xs[i] = half_to_f32<kF16>(X[(int64_t)m * g.ldx + k]);
  }
  __syncthreads();
  float acc[kM][8];
#pragma unroll
  for (int m = 0; m < kM; ++m)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[m][e] = 0.f;
  const uint16_t* W = static_cast<const uint16_t*>(mb.W);
  if (n < mb.N) {
    for (int kb = wave * kRowGroups + rg; kb < K; kb += kRowStep * kWideDepth) {
      u32x4 w[kWideDepth];
#pragma unroll
      for (int r = 0; r < kWideDepth; ++r) {
        const int k = kb + kRowStep * r;
        w[r] = k < K ? *reinterpret_cast<const u32x4*>(W + (int64_t)k * mb.ldw + n) : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int r = 0; r < kWideDepth; ++r) {
        const int k = kb + kRowStep * r;
        if (k < K) {
          const uint16_t* we = reinterpret_cast<const uint16_t*>(&w[r]);
#pragma unroll
          for (int m = 0; m < kM; ++m) {
            const float xv = m < g.M ? xs[m * K + k] : 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[m][e] += xv * half_to_f32<kF16>(we[e]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < kM; ++m)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = acc[m][e];
#pragma unroll
      for (int sh = kLanesPerRow; sh < 64; sh <<= 1) v += __shfl_xor(v, sh);
      acc[m][e] = v;
    }
  if (rg == 0) {
#pragma unroll
    for (int m = 0; m < kM; ++m)
#pragma unroll
      for (int e = 0; e < 8; ++e) red[wave][m][cc * 8 + e] = acc[m][e];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < kM * kCols; i += 1024) {
    const int m = i / kCols, c = i - m * kCols;
    const int nn = n0 + c;
    if (m >= g.M || nn >= mb.N) continue;
    float v = red[0][m][c];
#pragma unroll
    for (int w = 1; w < 16; ++w) v += red[w][m][c];
    const int64_t at = (int64_t)m * mb.ldy + nn;
    if (mb.add) {
      const float y = g.out_kind == 2 ? v : (g.out_kind == 1 ? f16_bits_to_f32(f32_to_f16_bits(v))
                                                           : bf16_bits_to_f32(f32_to_bf16_rne(v)));
      const float a = g.out_kind == 2 ? static_cast<const float*>(mb.add)[at]
                      : (g.out_kind == 1 ? f16_bits_to_f32(static_cast<const uint16_t*>(mb.add)[at])
                                         : bf16_bits_to_f32(static_cast<const uint16_t*>(mb.add)[at]));
      v = a + y;
    }
    store_out(mb.Y, at, v, g.out_kind);
  }
}

template <int kM, bool kF16, int G>
__global__ void __launch_bounds__(256) gemv_k(GemvParams p, const uint16_t* __restrict__ X,
                                              const uint16_t* __restrict__ W, void* __restrict__ Y) {
  constexpr int kRowsPerWave = 64 / G;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int sub = lane / G, gl = lane - sub * G;
  const int n = (blockIdx.x * 4 + wave) * kRowsPerWave + sub;
  const int b = blockIdx.z;
  float acc[kM];
#pragma unroll
  for (int m = 0; m < kM; ++m) acc[m] = 0.f;
  if (n < p.N) {
    const uint16_t* wr = W + (int64_t)b * p.w_bs + (int64_t)n * p.ldw;
    const uint16_t* Xb = X + (int64_t)b * p.x_bs;
#pragma unroll 4
    for (int k = gl * 8; k < p.K; k += G * 8) {  // K % 8 == 0 (checked by the caller)
      const u32x4 w = *reinterpret_cast<const u32x4*>(wr + k);
      const uint16_t* we = reinterpret_cast<const uint16_t*>(&w);
#pragma unroll
      for (int m = 0; m < kM; ++m) {
        if (m >= p.M) break;
        const u32x4 x = *reinterpret_cast<const u32x4*>(Xb + (int64_t)m * p.ldx + k);
        const uint16_t* xe = reinterpret_cast<const uint16_t*>(&x);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[m] += half_to_f32<kF16>(xe[e]) * half_to_f32<kF16>(we[e]);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < kM; ++m) {
    float v = acc[m];
#pragma unroll
    for (int o = G / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    if (gl == 0 && n < p.N && m < p.M) store_out(Y, (int64_t)b * p.y_bs + (int64_t)m * p.ldy + n, v, p.out_kind);
  }
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

bool use_big_gemm(const GemmParams& p, bool b_kmajor) {
  // Below one tile per CU the 128 x 128 kernel's 4x more tiles fill the GPU
  // better (environment: PJRTX_BIG_GEMM_MIN_TILES).
  const int64_t min_tiles = env_int("PJRTX_BIG_GEMM_MIN_TILES", 256);
  const int64_t tiles = (int64_t)((p.M + GBM - 1) / GBM) * ((p.N + GBN - 1) / GBN) * p.batch;
  // Every load offset (a 256-row panel of A, a panel or all K rows of B)
  // must stay below 2^31 bytes.
  const int64_t limit = int64_t(1) << 30;
  const bool b_ok = b_kmajor ? (p.ldb >= p.K && (int64_t)GBN * p.ldb < limit)
                             : (p.N % 8 == 0 && p.ldb >= p.N && (int64_t)p.K * p.ldb < limit);
  return p.M >= GBM && p.N >= GBN && p.K > 0 && p.K % 8 == 0 && p.lda % 8 == 0 && p.ldb % 8 == 0 &&
         p.lda >= p.K && b_ok && p.a_batch_stride % 8 == 0 && p.b_batch_stride % 8 == 0 && tiles >= min_tiles &&
         tiles < (int64_t(1) << 31) && (int64_t)GBM * p.lda < limit;
}

void launch_transpose16(hipStream_t s, const void* in, void* out, int64_t batch, int64_t rows, int64_t cols,
                        int64_t in_bs, int64_t out_bs) {
  if (batch == 0 || rows == 0 || cols == 0) return;
  const dim3 grid(static_cast<unsigned>((cols + 63) / 64), static_cast<unsigned>((rows + 63) / 64),
                  static_cast<unsigned>(batch));
  hipLaunchKernelGGL(transpose16, grid, dim3(256), 0, s, static_cast<const uint16_t*>(in), static_cast<uint16_t*>(out),
                     rows, cols, in_bs, out_bs);
  check("transpose16");
}

void launch_mfma_gemm(hipStream_t s, const GemmParams& p, const void* A, const void* B, void* C, bool f16, bool b_kmajor,
                      int out_bytes) {
  if (use_big_gemm(p, b_kmajor)) {
    const int64_t tiles = (int64_t)((p.M + GBM - 1) / GBM) * ((p.N + GBN - 1) / GBN) * p.batch;
    const dim3 grid(static_cast<unsigned>(tiles)), block(GTHREADS);
    const uint16_t* a = static_cast<const uint16_t*>(A);
    const uint16_t* b = static_cast<const uint16_t*>(B);
#define PJRTX_BIG(F16, OB, BN) hipLaunchKernelGGL((gemm_nt_256<F16, OB, BN>), grid, block, 0, s, p, a, b, C)
    if (out_bytes == 2) {
      if (f16) { if (b_kmajor) PJRTX_BIG(true, 2, false); else PJRTX_BIG(true, 2, true); }
      else { if (b_kmajor) PJRTX_BIG(false, 2, false); else PJRTX_BIG(false, 2, true); }
    } else {
      if (f16) { if (b_kmajor) PJRTX_BIG(true, 4, false); else PJRTX_BIG(true, 4, true); }
      else { if (b_kmajor) PJRTX_BIG(false, 4, false); else PJRTX_BIG(false, 4, true); }
    }
#undef PJRTX_BIG
    check("gemm_nt_256");
    return;
  }
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

void plan_gemv_split(GemvParams* p, int target_blocks) {
  const int64_t col_tiles = ((int64_t)p->N + kGemvCols - 1) / kGemvCols * p->batch;
  const int64_t min_rows = 4 * kGemvRowsPerLane;  // one full load round per wave
  int64_t ksplit = std::max<int64_t>(1, (target_blocks + col_tiles - 1) / col_tiles);
  ksplit = std::min<int64_t>(ksplit, std::max<int64_t>(1, p->K / min_rows));
  int64_t kchunk = (p->K + ksplit - 1) / ksplit;
  kchunk = (kchunk + 3) / 4 * 4;
  p->kchunk = static_cast<int>(std::max<int64_t>(kchunk, 4));
  p->ksplit = static_cast<int>((p->K + p->kchunk - 1) / p->kchunk);
}

void launch_gemv(hipStream_t s, const GemvParams& p, const void* X, const void* W, void* Y, float* partials, bool f16,
                 bool w_kmajor) {
  const uint16_t* x = static_cast<const uint16_t*>(X);
  const uint16_t* w = static_cast<const uint16_t*>(W);
  if (p.M < 1 || p.M > 8) fail(Code::kInternal, "gemv: M must be 1..8");
  if (w_kmajor) {
    int G = 8;
    while (G < 64 && G * 8 < p.K) G *= 2;
    const int rows_per_block = 4 * (64 / G);
    const dim3 g((unsigned)((p.N + rows_per_block - 1) / rows_per_block), 1, (unsigned)p.batch);
#define PJRTX_GEMV_K(KM, GG)                                                                                  \
  if (f16) hipLaunchKernelGGL((gemv_k<KM, true, GG>), g, dim3(256), 0, s, p, x, w, Y);                        \
  else hipLaunchKernelGGL((gemv_k<KM, false, GG>), g, dim3(256), 0, s, p, x, w, Y);
#define PJRTX_GEMV_KM(KM)            \
  switch (G) {                       \
    case 8: PJRTX_GEMV_K(KM, 8) break;   \
    case 16: PJRTX_GEMV_K(KM, 16) break; \
    case 32: PJRTX_GEMV_K(KM, 32) break; \
    default: PJRTX_GEMV_K(KM, 64) break; \
  }
    if (p.M == 1) { PJRTX_GEMV_KM(1) }
    else if (p.M <= 2) { PJRTX_GEMV_KM(2) }
    else if (p.M <= 4) { PJRTX_GEMV_KM(4) }
    else { PJRTX_GEMV_KM(8) }
#undef PJRTX_GEMV_KM
#undef PJRTX_GEMV_K
    check("gemv_k");
    return;
  }
  const dim3 g((unsigned)((p.N + kGemvCols - 1) / kGemvCols), (unsigned)p.ksplit, (unsigned)p.batch);
#define PJRTX_GEMV_N(KM)                                                                          \
  if (f16) hipLaunchKernelGGL((gemv_n<KM, true>), g, dim3(256), 0, s, p, x, w, partials, Y);      \
  else hipLaunchKernelGGL((gemv_n<KM, false>), g, dim3(256), 0, s, p, x, w, partials, Y);
  if (p.M == 1) { PJRTX_GEMV_N(1) }
  else if (p.M <= 2) { PJRTX_GEMV_N(2) }
  else if (p.M <= 4) { PJRTX_GEMV_N(4) }
  else { PJRTX_GEMV_N(8) }
#undef PJRTX_GEMV_N
  if (p.ksplit > 1) {
    const dim3 gr((unsigned)((p.N + 31) / 32), (unsigned)p.M, (unsigned)p.batch);
    hipLaunchKernelGGL(gemv_reduce, gr, dim3(256), 0, s, p, partials, Y);
  }
  check("gemv");
}

int gemv_wide_cols(const GemvGroup& g) {
  const int64_t forced = env_int("PJRTX_GEMV_COLS", 0);
  if (forced == 32 || forced == 64) return static_cast<int>(forced);
  // Measured per launch (M = 1): 64-column tiles for groups and wide
  // products (q/k/v 6.5 us, gate/up 11.6 us, lm_head 26 us; 32 columns cost
  // 3-30% more there); 32-column tiles when 64-column ones would leave fewer
  // than 64 workgroups (a 5632 x 2048 product: 9.7 us instead of 11.8).
  int64_t tiles64 = 0;
  for (int i = 0; i < g.count; ++i) tiles64 += (g.m[i].N + 63) / 64;
  return tiles64 >= 64 ? 64 : 32;
}

int gemv_wide_tiles(const GemvGroup& g) {
  const int cols = gemv_wide_cols(g);
  int64_t tiles = 0;
  for (int i = 0; i < g.count; ++i) tiles += (g.m[i].N + cols - 1) / cols;
  return static_cast<int>(std::min<int64_t>(tiles, int64_t(1) << 30));
}

bool gemv_wide_fits(int M, int K, int total_tiles) {
  return M >= 1 && M <= 4 && K >= 1 && (int64_t)M * K <= kGemvWideMaxX && total_tiles >= 32;
}

void launch_gemv_wide(hipStream_t s, GemvGroup g, const void* X, bool f16) {
  PJRTX_CHECK(g.count >= 1 && g.count <= kMaxGemvMembers && g.M >= 1 && g.M <= 4 && (int64_t)g.M * g.K <= kGemvWideMaxX,
              Code::kInternal, "gemv_wide: bad group");
  const int cols = gemv_wide_cols(g);
  int tiles = 0;
  for (int i = 0; i < g.count; ++i) {
    PJRTX_CHECK(g.m[i].N % 8 == 0 && g.m[i].ldw % 8 == 0, Code::kInternal, "gemv_wide: bad member layout");
    g.m[i].tile0 = tiles;
    tiles += (g.m[i].N + cols - 1) / cols;
  }
  const size_t lds = static_cast<size_t>(g.M) * g.K * sizeof(float);
  const uint16_t* x = static_cast<const uint16_t*>(X);
  const dim3 grid(static_cast<unsigned>(tiles)), block(1024);
#define PJRTX_WIDE(KM, C)                                                                  \
  if (f16) hipLaunchKernelGGL((gemv_wide<KM, true, C>), grid, block, lds, s, g, x);        \
  else hipLaunchKernelGGL((gemv_wide<KM, false, C>), grid, block, lds, s, g, x);
#define PJRTX_WIDE_M(C)             \
  if (g.M == 1) { PJRTX_WIDE(1, C) } \
  else if (g.M == 2) { PJRTX_WIDE(2, C) } \
  else { PJRTX_WIDE(4, C) }
  if (cols == 32) { PJRTX_WIDE_M(32) }
  else { PJRTX_WIDE_M(64) }
#undef PJRTX_WIDE_M
#undef PJRTX_WIDE
  check("gemv_wide");
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
