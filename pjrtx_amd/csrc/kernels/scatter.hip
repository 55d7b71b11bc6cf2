// Deterministic scatter for gfx950: sort-then-segment.
//
//  1. keys: each update row (or element) gets the operand row (element) it
//     targets; windows out of bounds get an `invalid` key and are skipped.
//  2. stable LSD radix sort of (key, update position), 8-bit digits. Inside a
//     64-lane wavefront, elements with equal digits are ranked by lane order
//     from 8 ballots (no atomics on data), and a per-digit LDS counter carries
//     the order across the wavefront's 32 chunks: the sort is stable, so each
//     target's updates stay in their original order.
//  3. segments: first/last sorted position of each target.
//  4. fold: each operand element folds its own updates sequentially, in
//     update order — the order of a sequential scatter loop, so integer
//     results are bit-exact and float sums round exactly as that loop does.
//     Rows without updates are copied through.
//
// Replaces the reference's scatter (reference: src/backend/mlx_metal/
// api.cc:3035-3246, MLX scatter_add with atomics: non-deterministic float
// order; dimension numbers as in api.cc:3158-3236).
#include <hip/hip_runtime.h>

#include "common.h"
#include "kernels/scatter.h"

namespace pjrtx {
namespace {

constexpr int kItems = 32;              // elements per lane per sort tile
constexpr int kTile = 64 * kItems;      // elements per sort workgroup (one wave)
constexpr int kScanTile = 2048;         // elements per scan workgroup (256 x 8)

__device__ __forceinline__ int64_t load_index(const void* p, int64_t i, int bytes, int is_signed) {
  if (bytes == 8) return reinterpret_cast<const int64_t*>(p)[i];
  if (bytes == 4) {
    const uint32_t u = reinterpret_cast<const uint32_t*>(p)[i];
    return is_signed ? (int64_t)(int32_t)u : (int64_t)u;
  }
  if (bytes == 2) {
    const uint16_t u = reinterpret_cast<const uint16_t*>(p)[i];
    return is_signed ? (int64_t)(int16_t)u : (int64_t)u;
  }
  const uint8_t u = reinterpret_cast<const uint8_t*>(p)[i];
  return is_signed ? (int64_t)(int8_t)u : (int64_t)u;
}

// ------------------------------------------------------------------- keys
__global__ void __launch_bounds__(256) scatter_keys(ScatterKeyParams p, const void* __restrict__ indices,
                                                    uint32_t* __restrict__ keys, uint32_t* __restrict__ vals) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= p.items) return;
  const int64_t s = t / p.window_items;
  const int64_t wpos = t - s * p.window_items;
  int64_t sc[kMaxRank];
  int64_t rem = s;
  for (int j = p.n_scatter_dims - 1; j >= 0; --j) {
    sc[j] = rem % p.scatter_dims[j];
    rem /= p.scatter_dims[j];
  }
  int64_t idx_base = 0;
  for (int j = 0; j < p.n_scatter_dims; ++j) idx_base += sc[j] * p.idx_stride[p.scatter_idx_dim[j]];
  int64_t start[kMaxRank];
  for (int d = 0; d < p.op_rank; ++d) start[d] = 0;
  for (int k = 0; k < p.n_index; ++k) {
    const int64_t off = (p.ivd < p.idx_rank) ? (int64_t)k * p.idx_stride[p.ivd] : 0;
    start[p.start_map[k]] = load_index(indices, idx_base + off, p.idx_bytes, p.idx_signed);
  }
  for (int k = 0; k < p.n_batching; ++k) start[p.op_batch_dim[k]] = sc[p.idx_batch_dim[k]];
  bool in_bounds = true;
  for (int d = 0; d < p.op_rank; ++d) in_bounds &= start[d] >= 0 && start[d] <= p.op_dims[d] - p.window[d];
  uint32_t key = p.invalid;
  uint32_t val;
  if (p.row_mode) {
    if (in_bounds) {
      int64_t lin = 0;
      for (int d = 0; d < p.op_rank; ++d) lin += start[d] * p.op_stride[d];
      key = (uint32_t)(lin / p.row_elems);
    }
    val = (uint32_t)s;
  } else {
    int64_t wc[kMaxRank];
    int64_t r2 = wpos;
    for (int j = p.n_window_dims - 1; j >= 0; --j) {
      wc[j] = r2 % p.window_extent[j];
      r2 /= p.window_extent[j];
    }
    if (in_bounds) {
      int64_t lin = 0;
      for (int d = 0; d < p.op_rank; ++d) lin += start[d] * p.op_stride[d];
      for (int j = 0; j < p.n_window_dims; ++j) lin += wc[j] * p.op_stride[p.window_op_dim[j]];
      key = (uint32_t)lin;
    }
    int64_t u = 0;
    for (int j = 0; j < p.n_scatter_dims; ++j) u += sc[j] * p.upd_stride_scatter[j];
    for (int j = 0; j < p.n_window_dims; ++j) u += wc[j] * p.upd_stride_window[j];
    val = (uint32_t)u;
  }
  keys[t] = key;
  vals[t] = val;
}

// ------------------------------------------------------------- radix sort
__global__ void __launch_bounds__(64) radix_hist(const uint32_t* __restrict__ keys, int64_t n, int shift,
                                                 uint32_t* __restrict__ hist, int nblocks) {
  __shared__ uint32_t h[256];
  const int lane = threadIdx.x;
  for (int i = lane; i < 256; i += 64) h[i] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * kTile;
#pragma unroll 4
  for (int j = 0; j < kItems; ++j) {
    const int64_t e = base + j * 64 + lane;
    if (e < n) atomicAdd(&h[(keys[e] >> shift) & 255u], 1u);
  }
  __syncthreads();
  for (int i = lane; i < 256; i += 64) hist[(int64_t)i * nblocks + blockIdx.x] = h[i];
}

__global__ void __launch_bounds__(64) radix_scatter(const uint32_t* __restrict__ kin, const uint32_t* __restrict__ vin,
                                                    uint32_t* __restrict__ kout, uint32_t* __restrict__ vout, int64_t n,
                                                    int shift, const uint32_t* __restrict__ offsets, int nblocks) {
  __shared__ uint32_t cnt[256];
  const int lane = threadIdx.x;
  for (int i = lane; i < 256; i += 64) cnt[i] = offsets[(int64_t)i * nblocks + blockIdx.x];
  __syncthreads();
  const uint64_t lt_mask = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  const int64_t base = (int64_t)blockIdx.x * kTile;
  for (int j = 0; j < kItems; ++j) {
    const int64_t e = base + j * 64 + lane;
    const bool valid = e < n;
    const uint32_t k = valid ? kin[e] : 0u;
    const uint32_t v = valid ? vin[e] : 0u;
    const uint32_t d = (k >> shift) & 255u;
    // Lanes holding the same digit: intersect the 8 per-bit ballots.
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const uint64_t m = __ballot((d >> b) & 1u);
      peers &= ((d >> b) & 1u) ? m : ~m;
    }
    const uint32_t rank = (uint32_t)__popcll(peers & lt_mask);
    const uint32_t pos = cnt[d] + rank;  // every lane reads before the leader writes
    __builtin_amdgcn_wave_barrier();
    if (valid) {
      kout[pos] = k;
      vout[pos] = v;
      if (rank == 0) cnt[d] = pos + (uint32_t)__popcll(peers);
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// ---------------------------------------------------------- exclusive scan
__global__ void __launch_bounds__(256) scan_tile_sums(const uint32_t* __restrict__ in, int64_t n,
                                                      uint32_t* __restrict__ sums) {
  __shared__ uint32_t red[256];
  const int64_t base = (int64_t)blockIdx.x * kScanTile;
  uint32_t s = 0;
  for (int j = 0; j < 8; ++j) {
    const int64_t e = base + threadIdx.x + 256 * j;
    if (e < n) s += in[e];
  }
  red[threadIdx.x] = s;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) sums[blockIdx.x] = red[0];
}

// In-place exclusive scan of up to 2048 values in one workgroup.
__global__ void __launch_bounds__(256) scan_small(uint32_t* __restrict__ a, int64_t n) {
  __shared__ uint32_t t[256];
  uint32_t v[8];
  uint32_t local = 0;
  for (int j = 0; j < 8; ++j) {
    const int64_t e = threadIdx.x * 8 + j;
    v[j] = e < n ? a[e] : 0u;
    local += v[j];
  }
  t[threadIdx.x] = local;
  __syncthreads();
  for (int o = 1; o < 256; o <<= 1) {
    const uint32_t x = threadIdx.x >= o ? t[threadIdx.x - o] : 0u;
    __syncthreads();
    t[threadIdx.x] += x;
    __syncthreads();
  }
  uint32_t run = t[threadIdx.x] - local;
  for (int j = 0; j < 8; ++j) {
    const int64_t e = threadIdx.x * 8 + j;
    if (e < n) a[e] = run;
    run += v[j];
  }
}

__global__ void __launch_bounds__(256) scan_apply(const uint32_t* __restrict__ in, uint32_t* __restrict__ out, int64_t n,
                                                  const uint32_t* __restrict__ tile_offsets) {
  __shared__ uint32_t t[256];
  const int64_t base = (int64_t)blockIdx.x * kScanTile + threadIdx.x * 8;
  uint32_t v[8];
  uint32_t local = 0;
  for (int j = 0; j < 8; ++j) {
    v[j] = base + j < n ? in[base + j] : 0u;
    local += v[j];
  }
  t[threadIdx.x] = local;
  __syncthreads();
  for (int o = 1; o < 256; o <<= 1) {
    const uint32_t x = threadIdx.x >= o ? t[threadIdx.x - o] : 0u;
    __syncthreads();
    t[threadIdx.x] += x;
    __syncthreads();
  }
  uint32_t run = tile_offsets[blockIdx.x] + t[threadIdx.x] - local;
  for (int j = 0; j < 8; ++j) {
    if (base + j < n) out[base + j] = run;
    run += v[j];
  }
}

// ---------------------------------------------------------------- segments
__global__ void __launch_bounds__(256) scatter_segments(const uint32_t* __restrict__ k, int64_t n, uint32_t invalid,
                                                        uint32_t* __restrict__ seg_start, uint32_t* __restrict__ seg_end) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const uint32_t key = k[i];
  if (key == invalid) return;
  if (i == 0 || k[i - 1] != key) seg_start[key] = (uint32_t)i;
  if (i == n - 1 || k[i + 1] != key) seg_end[key] = (uint32_t)(i + 1);
}

// -------------------------------------------------------------------- fold
template <typename S>
struct Codec;  // storage <-> compute, rounding after each op
template <> struct Codec<float> {
  typedef float C;
  static __device__ __forceinline__ C ld(float x) { return x; }
  static __device__ __forceinline__ float st(C x) { return x; }
  static __device__ __forceinline__ C rnd(C x) { return x; }
};
template <> struct Codec<double> {
  typedef double C;
  static __device__ __forceinline__ C ld(double x) { return x; }
  static __device__ __forceinline__ double st(C x) { return x; }
  static __device__ __forceinline__ C rnd(C x) { return x; }
};
struct Bf16Tag {};
struct F16Tag {};
template <> struct Codec<Bf16Tag> {
  typedef float C;
  static __device__ __forceinline__ C ld(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }
  static __device__ __forceinline__ uint16_t st(C f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
  }
  static __device__ __forceinline__ C rnd(C x) { return ld(st(x)); }
};
template <> struct Codec<F16Tag> {
  typedef float C;
  static __device__ __forceinline__ C ld(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
  static __device__ __forceinline__ uint16_t st(C f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
  static __device__ __forceinline__ C rnd(C x) { return (float)(_Float16)x; }
};
template <> struct Codec<int32_t> {
  typedef int32_t C;
  static __device__ __forceinline__ C ld(int32_t x) { return x; }
  static __device__ __forceinline__ int32_t st(C x) { return x; }
  static __device__ __forceinline__ C rnd(C x) { return x; }
};
template <> struct Codec<uint32_t> {
  typedef uint32_t C;
  static __device__ __forceinline__ C ld(uint32_t x) { return x; }
  static __device__ __forceinline__ uint32_t st(C x) { return x; }
  static __device__ __forceinline__ C rnd(C x) { return x; }
};
template <> struct Codec<int64_t> {
  typedef int64_t C;
  static __device__ __forceinline__ C ld(int64_t x) { return x; }
  static __device__ __forceinline__ int64_t st(C x) { return x; }
  static __device__ __forceinline__ C rnd(C x) { return x; }
};

template <typename Tag> struct StorageOf { typedef Tag T; };
template <> struct StorageOf<Bf16Tag> { typedef uint16_t T; };
template <> struct StorageOf<F16Tag> { typedef uint16_t T; };

template <typename C>
__device__ __forceinline__ C combine(ScatterOp op, C acc, C u) {
  switch (op) {
    case ScatterOp::kAdd: return acc + u;
    case ScatterOp::kSet: return u;
    case ScatterOp::kMul: return acc * u;
    case ScatterOp::kMax: return (acc != acc || acc >= u) ? acc : u;
    case ScatterOp::kMin: return (acc != acc || acc <= u) ? acc : u;
  }
  return acc;
}

template <typename Tag>
__global__ void __launch_bounds__(64) scatter_fold(ScatterFoldParams p, const typename StorageOf<Tag>::T* __restrict__ operand,
                                                   const typename StorageOf<Tag>::T* __restrict__ updates,
                                                   const uint32_t* __restrict__ perm, const uint32_t* __restrict__ seg_start,
                                                   const uint32_t* __restrict__ seg_end,
                                                   typename StorageOf<Tag>::T* __restrict__ out) {
  typedef Codec<Tag> K;
  typedef typename K::C C;
  const int64_t t = (int64_t)blockIdx.x * 64 + threadIdx.x;
  if (t >= p.rows * p.row_elems) return;
  const int64_t r = t / p.row_elems;
  const int64_t c = t - r * p.row_elems;
  const uint32_t lo = seg_start[r], hi = seg_end[r];
  C acc = K::ld(operand[t]);
  uint32_t i = lo;
  // Four updates in flight per step; applied strictly in order.
  for (; i + 4 <= hi; i += 4) {
    const int64_t u0 = p.row_mode ? (int64_t)perm[i] * p.row_elems + c : (int64_t)perm[i];
    const int64_t u1 = p.row_mode ? (int64_t)perm[i + 1] * p.row_elems + c : (int64_t)perm[i + 1];
    const int64_t u2 = p.row_mode ? (int64_t)perm[i + 2] * p.row_elems + c : (int64_t)perm[i + 2];
    const int64_t u3 = p.row_mode ? (int64_t)perm[i + 3] * p.row_elems + c : (int64_t)perm[i + 3];
    const C x0 = K::ld(updates[u0]), x1 = K::ld(updates[u1]), x2 = K::ld(updates[u2]), x3 = K::ld(updates[u3]);
    acc = K::rnd(combine<C>(p.op, acc, x0));
    acc = K::rnd(combine<C>(p.op, acc, x1));
    acc = K::rnd(combine<C>(p.op, acc, x2));
    acc = K::rnd(combine<C>(p.op, acc, x3));
  }
  for (; i < hi; ++i) {
    const int64_t u = p.row_mode ? (int64_t)perm[i] * p.row_elems + c : (int64_t)perm[i];
    acc = K::rnd(combine<C>(p.op, acc, K::ld(updates[u])));
  }
  out[t] = K::st(acc);
}

// ------------------------------------------------------- chunked row fold
constexpr int kFoldDepth = 16;  // update rows in flight per lane

template <typename T, int VEC>
struct alignas(sizeof(T) * VEC) VecOf {
  T v[VEC];
};

__global__ void __launch_bounds__(256) chunk_count(const uint32_t* __restrict__ seg_start,
                                                   const uint32_t* __restrict__ seg_end, int64_t rows,
                                                   uint32_t* __restrict__ cnt) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= rows) return;
  const uint32_t len = seg_end[r] - seg_start[r];
  cnt[r] = len <= (uint32_t)kScatterChunk ? 1u : (len + kScatterChunk - 1) / kScatterChunk;
}

__global__ void __launch_bounds__(256) chunk_rows(const uint32_t* __restrict__ cnt, const uint32_t* __restrict__ off,
                                                  int64_t rows, uint32_t* __restrict__ chunk_row,
                                                  uint32_t* __restrict__ total) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= rows) return;
  const uint32_t o = off[r], c = cnt[r];
  for (uint32_t q = 0; q < c; ++q) chunk_row[o + q] = (uint32_t)r;
  if (r == rows - 1) total[0] = o + c;
}

// One wave per chunk; 4 chunks per workgroup.
template <typename Tag, int VEC>
__global__ void __launch_bounds__(256) scatter_chunk_fold(
    int64_t row_elems, ScatterOp op, const typename StorageOf<Tag>::T* __restrict__ operand,
    const typename StorageOf<Tag>::T* __restrict__ updates, const uint32_t* __restrict__ perm,
    const uint32_t* __restrict__ seg_start, const uint32_t* __restrict__ seg_end, const uint32_t* __restrict__ cnt,
    const uint32_t* __restrict__ off, const uint32_t* __restrict__ chunk_row, const uint32_t* __restrict__ total,
    typename StorageOf<Tag>::T* __restrict__ partial, typename StorageOf<Tag>::T* __restrict__ out) {
  typedef Codec<Tag> K;
  typedef typename K::C C;
  typedef typename StorageOf<Tag>::T T;
  typedef VecOf<T, VEC> V;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t j = blockIdx.x * 4 + wave;
  if (j >= total[0]) return;
  const uint32_t r = chunk_row[j];
  const uint32_t q = j - off[r];
  const uint32_t lo = seg_start[r] + q * kScatterChunk;
  const uint32_t hi = min(lo + (uint32_t)kScatterChunk, seg_end[r]);
  T* dst = cnt[r] == 1 ? out + (int64_t)r * row_elems : partial + (int64_t)j * row_elems;
  for (int64_t c0 = (int64_t)lane * VEC; c0 < row_elems; c0 += 64 * VEC) {
    C acc[VEC];
    uint32_t i = lo;
    {
      const V first = q == 0 ? *reinterpret_cast<const V*>(operand + (int64_t)r * row_elems + c0)
                             : *reinterpret_cast<const V*>(updates + (int64_t)perm[lo] * row_elems + c0);
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] = K::ld(first.v[e]);
      if (q != 0) ++i;
    }
    for (; i + kFoldDepth <= hi; i += kFoldDepth) {
      V u[kFoldDepth];
#pragma unroll
      for (int d = 0; d < kFoldDepth; ++d)
        u[d] = *reinterpret_cast<const V*>(updates + (int64_t)perm[i + d] * row_elems + c0);
#pragma unroll
      for (int d = 0; d < kFoldDepth; ++d)
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] = K::rnd(combine<C>(op, acc[e], K::ld(u[d].v[e])));
    }
    for (; i < hi; ++i) {
      const V u = *reinterpret_cast<const V*>(updates + (int64_t)perm[i] * row_elems + c0);
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] = K::rnd(combine<C>(op, acc[e], K::ld(u.v[e])));
    }
    V o;
#pragma unroll
    for (int e = 0; e < VEC; ++e) o.v[e] = K::st(acc[e]);
    *reinterpret_cast<V*>(dst + c0) = o;
  }
}

// Rows with more than one chunk: fold the chunk partials in chunk order. One
// wave per row, 4 rows per workgroup.
template <typename Tag, int VEC>
__global__ void __launch_bounds__(256) scatter_chunk_combine(int64_t rows, int64_t row_elems, ScatterOp op,
                                                             const uint32_t* __restrict__ cnt,
                                                             const uint32_t* __restrict__ off,
                                                             const typename StorageOf<Tag>::T* __restrict__ partial,
                                                             typename StorageOf<Tag>::T* __restrict__ out) {
  typedef Codec<Tag> K;
  typedef typename K::C C;
  typedef typename StorageOf<Tag>::T T;
  typedef VecOf<T, VEC> V;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + wave;
  if (r >= rows) return;
  const uint32_t n = cnt[r];
  if (n <= 1) return;
  const T* src = partial + (int64_t)off[r] * row_elems;
  for (int64_t c0 = (int64_t)lane * VEC; c0 < row_elems; c0 += 64 * VEC) {
    C acc[VEC];
    const V first = *reinterpret_cast<const V*>(src + c0);
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = K::ld(first.v[e]);
    uint32_t qi = 1;
    for (; qi + kFoldDepth <= n; qi += kFoldDepth) {
      V u[kFoldDepth];
#pragma unroll
      for (int d = 0; d < kFoldDepth; ++d) u[d] = *reinterpret_cast<const V*>(src + (int64_t)(qi + d) * row_elems + c0);
#pragma unroll
      for (int d = 0; d < kFoldDepth; ++d)
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] = K::rnd(combine<C>(op, acc[e], K::ld(u[d].v[e])));
    }
    for (; qi < n; ++qi) {
      const V u = *reinterpret_cast<const V*>(src + (int64_t)qi * row_elems + c0);
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] = K::rnd(combine<C>(op, acc[e], K::ld(u.v[e])));
    }
    V o;
#pragma unroll
    for (int e = 0; e < VEC; ++e) o.v[e] = K::st(acc[e]);
    *reinterpret_cast<V*>(out + r * row_elems + c0) = o;
  }
}

__global__ void __launch_bounds__(256) zero_u32(uint32_t* __restrict__ a, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) a[i] = 0u;
}

void hcheck(hipError_t e, const char* what) {
  if (e != hipSuccess) fail(Code::kInternal, strformat("%s failed: %s", what, hipGetErrorString(e)));
}

void check(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) fail(Code::kInternal, strformat("%s launch failed: %s", what, hipGetErrorString(e)));
}

unsigned blocks(int64_t n, int per) { return static_cast<unsigned>((n + per - 1) / per); }

// Exclusive scan of n uint32 (n <= 2048 * 2048) using `tmp` (>= 2048 words).
void exclusive_scan(hipStream_t s, const uint32_t* in, uint32_t* out, int64_t n, uint32_t* tmp) {
  const int64_t tiles = (n + kScanTile - 1) / kScanTile;
  PJRTX_CHECK(tiles <= kScanTile, Code::kUnimplemented, "scan too large");
  hipLaunchKernelGGL(scan_tile_sums, dim3(blocks(n, kScanTile)), dim3(256), 0, s, in, n, tmp);
  hipLaunchKernelGGL(scan_small, dim3(1), dim3(256), 0, s, tmp, tiles);
  hipLaunchKernelGGL(scan_apply, dim3(blocks(n, kScanTile)), dim3(256), 0, s, in, out, n, tmp);
}

}  // namespace

size_t radix_sort_scratch_bytes(int64_t n) {
  const int64_t nblocks = (n + kTile - 1) / kTile;
  return static_cast<size_t>(256 * nblocks * 2 + kScanTile) * 4;
}

void launch_radix_sort(hipStream_t s, uint32_t* keys, uint32_t* vals, uint32_t* tmp_keys, uint32_t* tmp_vals,
                       void* scratch, int64_t n, int bits) {
  if (n <= 1) return;
  const int64_t nblocks = (n + kTile - 1) / kTile;
  PJRTX_CHECK(256 * nblocks <= int64_t(kScanTile) * kScanTile, Code::kUnimplemented, "radix sort: too many elements");
  uint32_t* hist = static_cast<uint32_t*>(scratch);
  uint32_t* offs = hist + 256 * nblocks;
  uint32_t* tmp = offs + 256 * nblocks;
  uint32_t *ki = keys, *vi = vals, *ko = tmp_keys, *vo = tmp_vals;
  const int passes = (bits + 7) / 8;
  for (int pass = 0; pass < passes; ++pass) {
    const int shift = pass * 8;
    hipLaunchKernelGGL(radix_hist, dim3(static_cast<unsigned>(nblocks)), dim3(64), 0, s, ki, n, shift, hist,
                       static_cast<int>(nblocks));
    exclusive_scan(s, hist, offs, 256 * nblocks, tmp);
    hipLaunchKernelGGL(radix_scatter, dim3(static_cast<unsigned>(nblocks)), dim3(64), 0, s, ki, vi, ko, vo, n, shift,
                       offs, static_cast<int>(nblocks));
    std::swap(ki, ko);
    std::swap(vi, vo);
  }
  if (ki != keys) {  // odd number of passes: copy back
    hcheck(hipMemcpyAsync(keys, ki, n * 4, hipMemcpyDeviceToDevice, s), "hipMemcpyAsync(sort keys)");
    hcheck(hipMemcpyAsync(vals, vi, n * 4, hipMemcpyDeviceToDevice, s), "hipMemcpyAsync(sort values)");
  }
  check("radix_sort");
}

void launch_scatter_keys(hipStream_t s, const ScatterKeyParams& p, const void* indices, uint32_t* keys, uint32_t* vals) {
  if (p.items == 0) return;
  hipLaunchKernelGGL(scatter_keys, dim3(blocks(p.items, 256)), dim3(256), 0, s, p, indices, keys, vals);
  check("scatter_keys");
}

void launch_scatter_segments(hipStream_t s, const uint32_t* sorted_keys, int64_t n, uint32_t invalid,
                             uint32_t* seg_start, uint32_t* seg_end, int64_t rows) {
  // Zero with a kernel (not a memset node), so the sequence stays capturable.
  hipLaunchKernelGGL(zero_u32, dim3(blocks(rows, 256)), dim3(256), 0, s, seg_start, rows);
  hipLaunchKernelGGL(zero_u32, dim3(blocks(rows, 256)), dim3(256), 0, s, seg_end, rows);
  if (n == 0) return;
  hipLaunchKernelGGL(scatter_segments, dim3(blocks(n, 256)), dim3(256), 0, s, sorted_keys, n, invalid, seg_start,
                     seg_end);
  check("scatter_segments");
}

namespace {
size_t align256(size_t b) { return (b + 255) / 256 * 256; }
int64_t max_chunks(int64_t rows, int64_t n) { return rows + (n + kScatterChunk - 1) / kScatterChunk; }
}  // namespace

size_t scatter_chunk_scratch_bytes(int64_t rows, int64_t n, int64_t row_elems, DType t) {
  const int64_t mc = max_chunks(rows, n);
  return 3 * align256(rows * 4) + align256(mc * 4) + align256(256) + align256(kScanTile * 4) +
         align256(mc * row_elems * dtype_size(t));
}

void launch_scatter_chunked(hipStream_t s, int64_t rows, int64_t row_elems, int64_t n, int op_i, DType t,
                            const void* operand, const void* updates, const uint32_t* perm,
                            const uint32_t* seg_start, const uint32_t* seg_end, void* scratch, void* out) {
  if (rows == 0 || row_elems == 0) return;
  const ScatterOp op = static_cast<ScatterOp>(op_i);
  const int64_t mc = max_chunks(rows, n);
  char* b = static_cast<char*>(scratch);
  uint32_t* cnt = reinterpret_cast<uint32_t*>(b);
  b += align256(rows * 4);
  uint32_t* off = reinterpret_cast<uint32_t*>(b);
  b += align256(rows * 4);
  b += align256(rows * 4);  // reserved
  uint32_t* chunk_row = reinterpret_cast<uint32_t*>(b);
  b += align256(mc * 4);
  uint32_t* total = reinterpret_cast<uint32_t*>(b);
  b += align256(256);
  uint32_t* scan_tmp = reinterpret_cast<uint32_t*>(b);
  b += align256(kScanTile * 4);
  void* partial = b;
  hipLaunchKernelGGL(chunk_count, dim3(blocks(rows, 256)), dim3(256), 0, s, seg_start, seg_end, rows, cnt);
  exclusive_scan(s, cnt, off, rows, scan_tmp);
  hipLaunchKernelGGL(chunk_rows, dim3(blocks(rows, 256)), dim3(256), 0, s, cnt, off, rows, chunk_row, total);
  check("scatter chunk plan");
  const size_t es = dtype_size(t);
  const bool vec = (row_elems * es) % 16 == 0 && (reinterpret_cast<uintptr_t>(operand) % 16 == 0) &&
                   (reinterpret_cast<uintptr_t>(updates) % 16 == 0) && (reinterpret_cast<uintptr_t>(out) % 16 == 0);
  const dim3 g1(blocks(mc, 4)), g2(blocks(rows, 4)), blk(256);
#define PJRTX_CHUNKED(TAG, VEC)                                                                                      \
  do {                                                                                                               \
    typedef StorageOf<TAG>::T T_;                                                                                    \
    hipLaunchKernelGGL((scatter_chunk_fold<TAG, VEC>), g1, blk, 0, s, row_elems, op, (const T_*)operand,            \
                       (const T_*)updates, perm, seg_start, seg_end, cnt, off, chunk_row, total, (T_*)partial,       \
                       (T_*)out);                                                                                    \
    hipLaunchKernelGGL((scatter_chunk_combine<TAG, VEC>), g2, blk, 0, s, rows, row_elems, op, cnt, off,             \
                       (const T_*)partial, (T_*)out);                                                                \
  } while (0)
#define PJRTX_CHUNKED_T(TAG, V16)            \
  if (vec) PJRTX_CHUNKED(TAG, V16);          \
  else PJRTX_CHUNKED(TAG, 1);
  switch (t) {
    case DType::kF32: PJRTX_CHUNKED_T(float, 4) break;
    case DType::kF64: PJRTX_CHUNKED_T(double, 2) break;
    case DType::kBF16: PJRTX_CHUNKED_T(Bf16Tag, 8) break;
    case DType::kF16: PJRTX_CHUNKED_T(F16Tag, 8) break;
    case DType::kS32: PJRTX_CHUNKED_T(int32_t, 4) break;
    case DType::kU32: PJRTX_CHUNKED_T(uint32_t, 4) break;
    case DType::kS64: PJRTX_CHUNKED_T(int64_t, 2) break;
    default: fail(Code::kUnimplemented, std::string("scatter: element type not supported: ") + dtype_name(t));
  }
#undef PJRTX_CHUNKED_T
#undef PJRTX_CHUNKED
  check("scatter_chunk_fold");
}

void launch_scatter_fold(hipStream_t s, const ScatterFoldParams& p, DType t, const void* operand, const void* updates,
                         const uint32_t* perm, const uint32_t* seg_start, const uint32_t* seg_end, void* out) {
  const int64_t n = p.rows * p.row_elems;
  if (n == 0) return;
  const dim3 g(blocks(n, 64)), b(64);
#define PJRTX_FOLD(TAG)                                                                                       \
  hipLaunchKernelGGL(scatter_fold<TAG>, g, b, 0, s, p, (const StorageOf<TAG>::T*)operand,                   \
                     (const StorageOf<TAG>::T*)updates, perm, seg_start, seg_end, (StorageOf<TAG>::T*)out)
  switch (t) {
    case DType::kF32: PJRTX_FOLD(float); break;
    case DType::kF64: PJRTX_FOLD(double); break;
    case DType::kBF16: PJRTX_FOLD(Bf16Tag); break;
    case DType::kF16: PJRTX_FOLD(F16Tag); break;
    case DType::kS32: PJRTX_FOLD(int32_t); break;
    case DType::kU32: PJRTX_FOLD(uint32_t); break;
    case DType::kS64: PJRTX_FOLD(int64_t); break;
    default: fail(Code::kUnimplemented, std::string("scatter: element type not supported: ") + dtype_name(t));
  }
#undef PJRTX_FOLD
  check("scatter_fold");
}

}  // namespace pjrtx
