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

#include <type_traits>

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
// Also zeroes zero[0 .. zero_n) (the segment bounds and counters the later
// steps fill), saving a launch.
__global__ void __launch_bounds__(256) scatter_keys(ScatterKeyParams p, const void* __restrict__ indices,
                                                    uint32_t* __restrict__ keys, uint32_t* __restrict__ vals,
                                                    uint32_t* __restrict__ keys2, uint32_t* __restrict__ zero,
                                                    int64_t zero_n) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t < zero_n) zero[t] = 0u;
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
  if (keys2) keys2[t] = key;
}

// ------------------------------------------------------------- radix sort
template <int BITS>
__global__ void __launch_bounds__(64) radix_hist(const uint32_t* __restrict__ keys, int64_t n, int shift,
                                                 uint32_t* __restrict__ hist, int nblocks) {
  constexpr uint32_t BINS = 1u << BITS;
  __shared__ uint32_t h[BINS];
  const int lane = threadIdx.x;
  for (uint32_t i = lane; i < BINS; i += 64) h[i] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * kTile;
#pragma unroll 4
  for (int j = 0; j < kItems; ++j) {
    const int64_t e = base + j * 64 + lane;
    if (e < n) atomicAdd(&h[(keys[e] >> shift) & (BINS - 1)], 1u);
  }
  __syncthreads();
  for (uint32_t i = lane; i < BINS; i += 64) hist[(int64_t)i * nblocks + blockIdx.x] = h[i];
}

template <int BITS>
__global__ void __launch_bounds__(64) radix_scatter(const uint32_t* __restrict__ kin, const uint32_t* __restrict__ vin,
                                                    uint32_t* __restrict__ kout, uint32_t* __restrict__ vout, int64_t n,
                                                    int shift, const uint32_t* __restrict__ offsets, int nblocks) {
  constexpr uint32_t BINS = 1u << BITS;
  __shared__ uint32_t cnt[BINS];
  const int lane = threadIdx.x;
  for (uint32_t i = lane; i < BINS; i += 64) cnt[i] = offsets[(int64_t)i * nblocks + blockIdx.x];
  __syncthreads();
  const uint64_t lt_mask = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  const int64_t base = (int64_t)blockIdx.x * kTile;
  for (int j = 0; j < kItems; ++j) {
    const int64_t e = base + j * 64 + lane;
    const bool valid = e < n;
    const uint32_t k = valid ? kin[e] : 0u;
    const uint32_t v = valid ? vin[e] : 0u;
    const uint32_t d = (k >> shift) & (BINS - 1);
    // Lanes holding the same digit: intersect the per-bit ballots.
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < BITS; ++b) {
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

// Exclusive scan of one tile, offset by the sum of the tile sums before it
// (at most kScanTile of them, summed by the workgroup: integers, so the
// order does not matter).
__global__ void __launch_bounds__(256) scan_apply(const uint32_t* __restrict__ in, uint32_t* __restrict__ out, int64_t n,
                                                  const uint32_t* __restrict__ tile_sums) {
  __shared__ uint32_t t[256];
  __shared__ uint32_t tile_offset;
  {
    uint32_t pre = 0;
    for (int64_t i = threadIdx.x; i < (int64_t)blockIdx.x; i += 256) pre += tile_sums[i];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) pre += __shfl_xor(pre, o);
    if ((threadIdx.x & 63) == 0) t[threadIdx.x >> 6] = pre;
    __syncthreads();
    if (threadIdx.x == 0) tile_offset = t[0] + t[1] + t[2] + t[3];
    __syncthreads();
  }
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
  uint32_t run = tile_offset + t[threadIdx.x] - local;
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

// ------------------------------------------------------------ row fold
//
// Row mode: every operand row folds its updates strictly in update order, so
// f32 results equal a sequential scatter loop bit for bit. Two kernels:
//
//  * bulk rows (segments of at most kHotMinUpdates updates, or every row when
//    the sliced path is off): one wave per row folds the whole row, 16 bytes
//    per lane, kFoldDepth update rows in flight.
//  * hot slices (longer segments, e.g. the Zipf head with ~10^5 updates):
//    a row is cut into 64-byte slices (16 f32 columns) and each slice is
//    folded by one workgroup, so a row's sequential column chains run on
//    many CUs at once. Waves 1-3 stream the slice's update rows through a
//    register ring into double-buffered LDS blocks; wave 0's lanes run the
//    column chains over each block. Hot workgroups are persistent over a
//    list of (row, slice) items ordered longest segment class first, so the
//    longest chain starts at once. This kernel runs on a second stream
//    beside the bulk kernel.
constexpr int kFoldDepth = 16;  // update rows in flight per lane (bulk rows)

template <typename T, int VEC>
struct alignas(sizeof(T) * VEC) VecOf {
  T v[VEC];
};

// A piece of an update row (16 bytes, or one element for narrow rows), which
// the fold reads once: a non-temporal load (streams faster, and leaves the memory-side cache to
// the operand rows and the keys).
template <typename V>
__device__ __forceinline__ V load_once(const V* p) {
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
  typedef uint32_t u2 __attribute__((ext_vector_type(2)));
  if constexpr (sizeof(V) == 16) return __builtin_bit_cast(V, __builtin_nontemporal_load(reinterpret_cast<const u4*>(p)));
  else if constexpr (sizeof(V) == 8) return __builtin_bit_cast(V, __builtin_nontemporal_load(reinterpret_cast<const u2*>(p)));
  else if constexpr (sizeof(V) == 4) return __builtin_bit_cast(V, __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p)));
  else return *p;
}

// True when row r is one of the early rows (folded before the sort ends).
__device__ __forceinline__ bool is_early_row(const uint32_t* __restrict__ early, int64_t r) {
  if (!early) return false;
  const uint32_t count = early[0];
  bool hit = false;
#pragma unroll
  for (int j = 0; j < kEarlyRows; ++j) hit |= (uint32_t)j < count && early[1 + j] == (uint32_t)r;
  return hit;
}

// Lists the hot rows by length class. With `init_dst` (the integer chunk
// path, which merges into the result with atomics, when the result is not
// the operand's own buffer), also fills each hot row of the result with the
// reduction's identity; the row's first chunk folds the operand row in.
__global__ void __launch_bounds__(256) scatter_hot_classify(const uint32_t* __restrict__ seg_start,
                                                            const uint32_t* __restrict__ seg_end, int64_t rows,
                                                            ScatterHotList h, uint4 identity,
                                                            uint4* __restrict__ init_dst, int64_t row_u4,
                                                            const uint32_t* __restrict__ early) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const uint32_t len = r < rows ? seg_end[r] - seg_start[r] : 0u;
  const bool hot = len > (uint32_t)kHotMinUpdates && !is_early_row(early, r);
  if (hot) {
    const int k = 31 - __clz(len);
    const uint32_t slot = atomicAdd(&h.counts[k], 1u);  // order inside a class does not change results
    h.rows[h.base[k] + slot] = (uint32_t)r;
  }
  if (!init_dst) return;
  // The wave fills its hot rows, 16 bytes a lane (stores only: nothing to
  // wait for, where copying the operand rows waited on each row's loads).
  const int lane = threadIdx.x & 63;
  uint64_t m = __ballot(hot);
  while (m) {
    const int l = __ffsll((unsigned long long)m) - 1;
    m &= m - 1;
    const int64_t rr = (int64_t)blockIdx.x * 256 + (threadIdx.x & ~63) + l;
    for (int64_t j = lane; j < row_u4; j += 64) init_dst[rr * row_u4 + j] = identity;
  }
}

// Integer add / max / min on hot rows: exact in any order, so a row's updates
// are cut into chunks of kHotChunk folded by separate workgroups (registers,
// then the 4 waves through LDS) and merged into the result with atomics.
// Chunk items of class k: rows x ceil(2^(k+1) / kHotChunk) (empty chunks of
// shorter rows exit at once); longest class first.
constexpr int kHotChunk = 512;

template <typename T, ScatterOp OP>
__device__ __forceinline__ T int_fold(T a, T b) {
  if constexpr (OP == ScatterOp::kAdd) return (T)((typename std::make_unsigned<T>::type)a + (typename std::make_unsigned<T>::type)b);
  else if constexpr (OP == ScatterOp::kMax) return a > b ? a : b;
  else return a < b ? a : b;
}

template <typename T, ScatterOp OP>
__device__ __forceinline__ void int_atomic(T* p, T v) {
  if constexpr (sizeof(T) == 4 && std::is_signed<T>::value) {
    if constexpr (OP == ScatterOp::kAdd) atomicAdd(reinterpret_cast<int*>(p), (int)v);
    else if constexpr (OP == ScatterOp::kMax) atomicMax(reinterpret_cast<int*>(p), (int)v);
    else atomicMin(reinterpret_cast<int*>(p), (int)v);
  } else if constexpr (sizeof(T) == 4) {
    if constexpr (OP == ScatterOp::kAdd) atomicAdd(reinterpret_cast<unsigned*>(p), (unsigned)v);
    else if constexpr (OP == ScatterOp::kMax) atomicMax(reinterpret_cast<unsigned*>(p), (unsigned)v);
    else atomicMin(reinterpret_cast<unsigned*>(p), (unsigned)v);
  } else {
    if constexpr (OP == ScatterOp::kAdd) atomicAdd(reinterpret_cast<unsigned long long*>(p), (unsigned long long)v);
    else if constexpr (OP == ScatterOp::kMax) atomicMax(reinterpret_cast<long long*>(p), (long long)v);
    else atomicMin(reinterpret_cast<long long*>(p), (long long)v);
  }
}

template <typename T, ScatterOp OP>
__global__ void __launch_bounds__(256) scatter_hot_chunks(int64_t row_elems, const T* __restrict__ updates,
                                                          const uint32_t* __restrict__ perm,
                                                          const uint32_t* __restrict__ seg_start,
                                                          const uint32_t* __restrict__ seg_end, ScatterHotList h,
                                                          const T* __restrict__ operand_init, T* __restrict__ out) {
  constexpr int VEC = 16 / (int)sizeof(T);
  typedef VecOf<T, VEC> V;
  __shared__ V part[3][64];
  __shared__ uint32_t pidx[kHotChunk];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  int64_t total = 0;
  for (int k = 31; k >= h.kmin; --k) total += (int64_t)h.counts[k] * (((int64_t(2) << k) + kHotChunk - 1) / kHotChunk);
  // With xcd_group, workgroup b (on XCD b % 8) takes item slot
  // (b % 8) * (grid / 8) + b / 8 of each round: a bijection on the round's
  // slots that puts consecutive items on one XCD.
  const int64_t slot = h.xcd_group && gridDim.x % 8 == 0
                           ? (int64_t)(blockIdx.x % 8) * (gridDim.x / 8) + blockIdx.x / 8
                           : (int64_t)blockIdx.x;
  for (int64_t item = slot; item < total; item += gridDim.x) {
    int64_t it = item;
    uint32_t row = 0, chunk = 0;
    for (int k = 31; k >= h.kmin; --k) {
      const int64_t cpr = ((int64_t(2) << k) + kHotChunk - 1) / kHotChunk;
      const int64_t c = (int64_t)h.counts[k] * cpr;
      if (it < c) {
        row = h.rows[h.base[k] + it / cpr];
        chunk = (uint32_t)(it % cpr);
        break;
      }
      it -= c;
    }
    const uint32_t lo = seg_start[row] + chunk * kHotChunk, hi = min(lo + (uint32_t)kHotChunk, seg_end[row]);
    if (lo >= hi) continue;  // uniform over the workgroup
    // The chunk's update indices go to LDS first (one coalesced read), so
    // the update-row loads below need no dependent index load.
    const int n = (int)(hi - lo);
    __syncthreads();  // the previous item's readers of pidx are done
    for (int t = threadIdx.x; t < n; t += 256) pidx[t] = perm[lo + t];
    __syncthreads();
    for (int64_t c0 = (int64_t)lane * VEC; c0 - lane * VEC < row_elems; c0 += 64 * VEC) {
      const bool col_ok = c0 < row_elems;
      V acc;
      bool any = false;
      // With operand_init (the result rows hold the identity), wave 0 of
      // the row's first chunk starts from the operand row.
      if (operand_init && chunk == 0 && wave == 0 && col_ok) {
        acc = *reinterpret_cast<const V*>(operand_init + (int64_t)row * row_elems + c0);
        any = true;
      }
      // Wave w folds rows w, w + 4, ...; kFoldDepth of them per batch, the
      // next batch's loads issued before the current batch is folded.
      V ua[kFoldDepth], ub[kFoldDepth];
      auto issue = [&](V (&u)[kFoldDepth], int base) {
#pragma unroll
        for (int q = 0; q < kFoldDepth; ++q) {
          const int j = min(base + 4 * q, n - 1);  // clamped: a repeat of the last row is never folded
          u[q] = col_ok ? load_once(reinterpret_cast<const V*>(updates + (int64_t)pidx[j] * row_elems + c0)) : V();
        }
      };
      auto fold = [&](const V (&u)[kFoldDepth], int base) {
#pragma unroll
        for (int q = 0; q < kFoldDepth; ++q) {
          if (base + 4 * q >= n) break;
          if (!any) {
            acc = u[q];
            any = true;
          } else {
#pragma unroll
            for (int e = 0; e < VEC; ++e) acc.v[e] = int_fold<T, OP>(acc.v[e], u[q].v[e]);
          }
        }
      };
      int base = wave;
      if (base < n) issue(ua, base);
      while (base < n) {
        const int b1 = base + 4 * kFoldDepth;
        if (b1 < n) issue(ub, b1);
        fold(ua, base);
        if (b1 >= n) break;
        const int b2 = b1 + 4 * kFoldDepth;
        if (b2 < n) issue(ua, b2);
        fold(ub, b1);
        base = b2;
      }
      // waves 1-3 hand their partials to wave 0 (a wave with no row keeps `any` false)
      __shared__ int has[3];
      if (wave > 0) {
        part[wave - 1][lane] = acc;
        if (lane == 0) has[wave - 1] = any ? 1 : 0;
      }
      __syncthreads();
      if (wave == 0 && col_ok) {
#pragma unroll
        for (int w = 0; w < 3; ++w) {
          if (!has[w]) continue;
          const V o = part[w][lane];
          if (!any) {
            acc = o;
            any = true;
          } else {
#pragma unroll
            for (int e = 0; e < VEC; ++e) acc.v[e] = int_fold<T, OP>(acc.v[e], o.v[e]);
          }
        }
        if (any)
#pragma unroll
          for (int e = 0; e < VEC; ++e) int_atomic<T, OP>(out + (int64_t)row * row_elems + c0 + e, acc.v[e]);
      }
      __syncthreads();
    }
  }
}

template <typename Tag, ScatterOp OP>
__device__ __forceinline__ typename Codec<Tag>::C fold1(typename Codec<Tag>::C acc, typename Codec<Tag>::C u) {
  return Codec<Tag>::rnd(combine<typename Codec<Tag>::C>(OP, acc, u));
}

// Shape of a hot slice's pipeline (per element size): kHotSliceBytes of a
// row per slice, 16-byte loads, update rows staged in LDS as
// [row quad][column][4 rows] so a chain lane reads four rows of its column
// with one load.
template <typename T>
struct HotShape {
  static constexpr int COLS = kHotSliceBytes / (int)sizeof(T);  // columns per slice = chain lanes
  static constexpr int EPL = 16 / (int)sizeof(T);               // elements per 16-byte lane load
  static constexpr int LPR = COLS / EPL;                        // lanes per update row of a slice
  static constexpr int RPI = 64 / LPR;                          // update rows per wave load
  static constexpr int BROWS = 192;                             // update rows per LDS block (3 loader waves x 64)
  static constexpr int NI = (BROWS / 3) / RPI;                  // loads per loader wave per block
  static constexpr int DEPTH = (int)sizeof(T) == 2 ? 8 : ((int)sizeof(T) == 4 ? 4 : 2);  // blocks in flight
  static constexpr int QS = COLS * 4 + 4 * EPL;                 // elements per row quad in LDS (padded)
  static constexpr int BUF = (BROWS / 4) * QS;                  // elements per LDS block
};

// One (row, slice) item of the hot path. Wave 0 runs the column chains;
// waves 1-3 stream the update rows through a register ring (data DEPTH
// blocks ahead, perm indices 2*DEPTH blocks ahead) into two LDS blocks.
// Both roles pass one barrier per block. The streamed arrays are not
// __restrict__ here: the barrier then orders their loads, so each stays
// issued where it is written instead of being sunk next to its use.
template <typename Tag, ScatterOp OP>
__device__ __forceinline__ void hot_slice_fold(int64_t row_elems, uint32_t row, int slice,
                                               const typename StorageOf<Tag>::T* __restrict__ operand,
                                               const typename StorageOf<Tag>::T* updates, const uint32_t* perm,
                                               uint32_t lo, uint32_t len,
                                               typename StorageOf<Tag>::T* __restrict__ out,
                                               typename StorageOf<Tag>::T* lds) {
  typedef Codec<Tag> K;
  typedef typename K::C C;
  typedef typename StorageOf<Tag>::T T;
  typedef HotShape<T> S;
  typedef VecOf<T, S::EPL> V;
  typedef VecOf<T, 4> Q;
  constexpr int D = S::DEPTH, NI = S::NI;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t c0 = (int64_t)slice * S::COLS;
  const int nb = (int)((len + S::BROWS - 1) / S::BROWS);
  const int nsteps = (nb + D - 1) / D * D;  // whole unrolled rounds: both roles pass the same barriers

  if (wave == 0) {
    // ---- chain role: lane c folds column c0 + c in update order.
    const bool chain = lane < S::COLS && c0 + lane < row_elems;
    C acc = C();
    if (chain) acc = K::ld(operand[(int64_t)row * row_elems + c0 + lane]);
    for (int b0 = 0; b0 < nsteps; b0 += 2) {
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        const int b = b0 + d;
        __syncthreads();  // block b is in LDS buffer d
        const int here = b < nb ? (int)min((uint32_t)S::BROWS, len - (uint32_t)b * S::BROWS) : 0;
        if (chain) {
          const T* src = lds + d * S::BUF + lane * 4;
          if (here == S::BROWS) {
            // Half a block of quads into registers first: the reads queue
            // back to back and the chain only waits for the oldest.
            for (int q0 = 0; q0 < S::BROWS / 4; q0 += S::BROWS / 8) {
              Q x[S::BROWS / 8];
#pragma unroll
              for (int j = 0; j < S::BROWS / 8; ++j) x[j] = *reinterpret_cast<const Q*>(src + (q0 + j) * S::QS);
#pragma unroll
              for (int j = 0; j < S::BROWS / 8; ++j) {
                acc = fold1<Tag, OP>(acc, K::ld(x[j].v[0]));
                acc = fold1<Tag, OP>(acc, K::ld(x[j].v[1]));
                acc = fold1<Tag, OP>(acc, K::ld(x[j].v[2]));
                acc = fold1<Tag, OP>(acc, K::ld(x[j].v[3]));
              }
            }
          } else {
            for (int r = 0; r < here; ++r) acc = fold1<Tag, OP>(acc, K::ld(src[(r >> 2) * S::QS + (r & 3)]));
          }
        }
      }
    }
    if (chain) out[(int64_t)row * row_elems + c0 + lane] = K::st(acc);
  } else {
    // ---- load role: waves 1..3 each own 64 rows of a block.
    const int lw = wave - 1;
    const int g = lane % S::LPR, rr = lane / S::LPR;
    // Column of this lane's 16-byte load; a group past the row end re-reads
    // the row's first group and stores it into its quad's padding.
    const bool g_ok = c0 + g * S::EPL < row_elems;
    const int64_t lc = g_ok ? c0 + g * S::EPL : 0;
    const int wcol = g_ok ? g * S::EPL * 4 : S::COLS * 4;
    const uint32_t last = len - 1;
    auto perm_of = [&](int b, int i) -> uint32_t {
      const uint32_t r = (uint32_t)b * S::BROWS + (uint32_t)(lw * 64 + i * S::RPI + rr);
      return perm[lo + (r < last ? r : last)];
    };
    uint32_t P[D][NI];  // perm of blocks b+D .. b+2D-1 (slot = block % D)
    V R[D][NI];         // update data of blocks b .. b+D-1 (slot = block % D)
    // Prologue in the loop's own issue order (per slot: perm of the block D
    // further on, then the slot's data), so the loop sees the same queue of
    // loads on entry as around its back edge.
#pragma unroll
    for (int d = 0; d < D; ++d)
#pragma unroll
      for (int i = 0; i < NI; ++i) P[d][i] = perm_of(d, i);
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const V* a[NI];
#pragma unroll
      for (int i = 0; i < NI; ++i) a[i] = reinterpret_cast<const V*>(updates + (int64_t)P[d][i] * row_elems + lc);
#pragma unroll
      for (int i = 0; i < NI; ++i) P[d][i] = perm_of(D + d, i);
      __builtin_amdgcn_sched_barrier(0);  // keep the issue order: perm, then data, slot by slot
#pragma unroll
      for (int i = 0; i < NI; ++i) R[d][i] = *a[i];
      __builtin_amdgcn_sched_barrier(0);
    }
    for (int b0 = 0; b0 < nsteps; b0 += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        const int b = b0 + d;
        T* buf = lds + (d & 1) * S::BUF;
        // block b into LDS as [quad][column][4 rows]
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          const int rho = lw * 64 + i * S::RPI + rr;
          T* dst = buf + (rho >> 2) * S::QS + wcol + (rho & 3);
#pragma unroll
          for (int e = 0; e < S::EPL; ++e) dst[e * 4] = R[d][i].v[e];
        }
        // addresses of block b+D from its perm (formed first, so the perm
        // registers are free for the new perm loads and stay the same
        // registers around the loop), then perm of b+2D, then the loads of
        // b+D (after those perm loads: waiting for this block's data later
        // also covers them)
        const V* a[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i) a[i] = reinterpret_cast<const V*>(updates + (int64_t)P[d][i] * row_elems + lc);
#pragma unroll
        for (int i = 0; i < NI; ++i) P[d][i] = perm_of(b + 2 * D, i);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < NI; ++i) R[d][i] = *a[i];
        __syncthreads();  // block b complete
      }
    }
  }
  __syncthreads();  // the next item reuses the LDS blocks
}

template <typename Tag, ScatterOp OP>
__global__ void __launch_bounds__(256) scatter_hot_fold(
    int64_t row_elems, const typename StorageOf<Tag>::T* __restrict__ operand,
    const typename StorageOf<Tag>::T* updates, const uint32_t* perm, const uint32_t* __restrict__ seg_start,
    const uint32_t* __restrict__ seg_end, ScatterHotList h, typename StorageOf<Tag>::T* __restrict__ out) {
  typedef typename StorageOf<Tag>::T T;
  typedef HotShape<T> S;
  __shared__ __align__(16) T lds[2 * S::BUF];
  const int64_t slices = (row_elems + S::COLS - 1) / S::COLS;
  int64_t total = 0;
  for (int k = 31; k >= h.kmin; --k) total += (int64_t)h.counts[k] * slices;
  // With xcd_group, workgroup b (on XCD b % 8) takes item slot
  // (b % 8) * (grid / 8) + b / 8 of each round: a bijection on the round's
  // slots that puts consecutive items on one XCD.
  const int64_t slot = h.xcd_group && gridDim.x % 8 == 0
                           ? (int64_t)(blockIdx.x % 8) * (gridDim.x / 8) + blockIdx.x / 8
                           : (int64_t)blockIdx.x;
  for (int64_t item = slot; item < total; item += gridDim.x) {
    int64_t it = item;
    uint32_t row = 0;
    int slice = 0;
    for (int k = 31; k >= h.kmin; --k) {
      const int64_t c = (int64_t)h.counts[k] * slices;
      if (it < c) {
        row = h.rows[h.base[k] + it / slices];
        slice = (int)(it % slices);
        break;
      }
      it -= c;
    }
    const uint32_t lo = seg_start[row];
    hot_slice_fold<Tag, OP>(row_elems, row, slice, operand, updates, perm, lo, seg_end[row] - lo, out, lds);
  }
}

// ---------------------------------------------------------------- early rows
// Selection: kEarlySample keys at even strides counted in an LDS hash table
// (open addressing, at most half full); every key (not the drop key) seen at
// least kEarlyMinRun times is a candidate; the kEarlyRows most frequent
// (ties: smaller row) are listed, most frequent first.
constexpr int kEarlyTable = 2 * kEarlySample;
__global__ void __launch_bounds__(1024) scatter_early_select(const uint32_t* __restrict__ keys, int64_t n,
                                                             uint32_t invalid, uint32_t* __restrict__ early) {
  __shared__ uint32_t hkey[kEarlyTable], hcnt[kEarlyTable];
  __shared__ uint32_t cand_row[kEarlySample / kEarlyMinRun + 1], cand_len[kEarlySample / kEarlyMinRun + 1];
  __shared__ uint32_t ncand;
  const int tid = threadIdx.x;
  if (tid == 0) ncand = 0;
  for (int i = tid; i < kEarlyTable; i += 1024) {
    hkey[i] = 0xffffffffu;
    hcnt[i] = 0u;
  }
  uint32_t sample[kEarlySample / 1024];
#pragma unroll
  for (int q = 0; q < kEarlySample / 1024; ++q) sample[q] = keys[(int64_t)(tid + q * 1024) * n / kEarlySample];
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kEarlySample / 1024; ++q) {
    const uint32_t k = sample[q];
    if (k == invalid || k == 0xffffffffu) continue;
    uint32_t h = (k * 2654435761u) & (kEarlyTable - 1);
    for (;;) {  // the table never fills: at most kEarlySample keys in 2 kEarlySample slots
      const uint32_t old = atomicCAS(&hkey[h], 0xffffffffu, k);
      if (old == 0xffffffffu || old == k) {
        atomicAdd(&hcnt[h], 1u);
        break;
      }
      h = (h + 1) & (kEarlyTable - 1);
    }
  }
  __syncthreads();
  for (int i = tid; i < kEarlyTable; i += 1024) {
    if (hcnt[i] >= (uint32_t)kEarlyMinRun) {
      const uint32_t slot = atomicAdd(&ncand, 1u);
      cand_row[slot] = hkey[i];
      cand_len[slot] = hcnt[i];
    }
  }
  __syncthreads();
  // Rank among the candidates: more samples first, then the smaller row.
  const uint32_t nc = ncand;
  if ((uint32_t)tid < nc) {
    const uint32_t r = cand_row[tid], l = cand_len[tid];
    uint32_t rank = 0;
    for (uint32_t c = 0; c < nc; ++c) rank += (cand_len[c] > l || (cand_len[c] == l && cand_row[c] < r)) ? 1u : 0u;
    if (rank < (uint32_t)kEarlyRows) early[1 + rank] = r;
  }
  if (tid == 0) early[0] = nc < (uint32_t)kEarlyRows ? nc : (uint32_t)kEarlyRows;
}

// Per workgroup (kEarlyBlockItems consecutive keys, 16 a thread) and early
// row j: how many keys name row j; counts[j * blocks + b]. The workgroup 0
// also zeroes the trailing entry (the total after the scan).
__global__ void __launch_bounds__(256) scatter_early_count(const uint32_t* __restrict__ keys, int64_t n,
                                                           const uint32_t* __restrict__ early,
                                                           uint32_t* __restrict__ counts, int64_t blocks) {
  __shared__ uint32_t part[4][kEarlyRows];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const uint32_t count = early[0];
  uint32_t er[kEarlyRows];
#pragma unroll
  for (int j = 0; j < kEarlyRows; ++j) er[j] = (uint32_t)j < count ? early[1 + j] : 0xffffffffu;
  uint32_t c[kEarlyRows] = {};
  const int64_t base = (int64_t)blockIdx.x * kEarlyBlockItems + (int64_t)tid * 16;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int64_t i = base + k;
    const bool in = i < n;
    const uint32_t key = in ? keys[i] : 0u;
#pragma unroll
    for (int j = 0; j < kEarlyRows; ++j) c[j] += in && (uint32_t)j < count && key == er[j] ? 1u : 0u;
  }
#pragma unroll
  for (int j = 0; j < kEarlyRows; ++j) {
    uint32_t v = c[j];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    if (lane == 0) part[wave][j] = v;
  }
  __syncthreads();
  if (tid < kEarlyRows) counts[(int64_t)tid * blocks + blockIdx.x] = part[0][tid] + part[1][tid] + part[2][tid] + part[3][tid];
  if (blockIdx.x == 0 && tid == 0) counts[(int64_t)kEarlyRows * blocks] = 0u;
}

// Writes each early row's update indices in update order: a thread's 16
// keys, its exclusive rank among the workgroup's threads (wave scans plus
// wave totals), and the workgroup's offset from the scanned counts.
// `offsets`: the exclusive scan of `counts` (row-major [row][block]), or
// null for a grid of at most kEarlyInlineBlocks workgroups, which then
// computes its own entries of that scan from `counts` (every workgroup sums
// the rows' totals and its earlier blocks' counts) and whose workgroup 0
// writes the rows' starts and the total to row_starts[0 .. kEarlyRows].
__global__ void __launch_bounds__(256) scatter_early_write(const uint32_t* __restrict__ keys, int64_t n,
                                                           const uint32_t* __restrict__ early,
                                                           const uint32_t* __restrict__ offsets,
                                                           const uint32_t* __restrict__ counts,
                                                           uint32_t* __restrict__ row_starts, int64_t blocks,
                                                           uint32_t* __restrict__ list) {
  __shared__ uint32_t wtot[4][kEarlyRows];
  __shared__ uint32_t wpre[4][2 * kEarlyRows];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const uint32_t count = early[0];
  uint32_t start[kEarlyRows];  // scan entry (j, this block)
  if (offsets) {
#pragma unroll
    for (int j = 0; j < kEarlyRows; ++j) start[j] = offsets[(int64_t)j * blocks + blockIdx.x];
  } else {
    // tot[j]: row j's total; pre[j]: row j's counts in blocks before this one
    uint32_t tot[kEarlyRows] = {}, pre[kEarlyRows] = {};
    for (int64_t b = tid; b < blocks; b += 256) {
#pragma unroll
      for (int j = 0; j < kEarlyRows; ++j) {
        const uint32_t c = counts[(int64_t)j * blocks + b];
        tot[j] += c;
        pre[j] += b < (int64_t)blockIdx.x ? c : 0u;
      }
    }
#pragma unroll
    for (int j = 0; j < kEarlyRows; ++j) {
      uint32_t t = tot[j], q = pre[j];
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        t += __shfl_xor(t, o);
        q += __shfl_xor(q, o);
      }
      if (lane == 0) {
        wpre[wave][j] = t;
        wpre[wave][kEarlyRows + j] = q;
      }
    }
    __syncthreads();
    uint32_t row0 = 0;
#pragma unroll
    for (int j = 0; j < kEarlyRows; ++j) {
      const uint32_t t = wpre[0][j] + wpre[1][j] + wpre[2][j] + wpre[3][j];
      start[j] = row0 + wpre[0][kEarlyRows + j] + wpre[1][kEarlyRows + j] + wpre[2][kEarlyRows + j] +
                 wpre[3][kEarlyRows + j];
      if (blockIdx.x == 0 && tid == 0) row_starts[j] = row0;
      row0 += t;
    }
    if (blockIdx.x == 0 && tid == 0) row_starts[kEarlyRows] = row0;
  }
  uint32_t er[kEarlyRows];
#pragma unroll
  for (int j = 0; j < kEarlyRows; ++j) er[j] = (uint32_t)j < count ? early[1 + j] : 0xffffffffu;
  const int64_t base = (int64_t)blockIdx.x * kEarlyBlockItems + (int64_t)tid * 16;
  // match[k]: the early row (index + 1) key k names, 0 for none.
  uint32_t match[16];
  uint32_t c[kEarlyRows] = {};
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int64_t i = base + k;
    const uint32_t key = i < n ? keys[i] : 0u;
    match[k] = 0u;
#pragma unroll
    for (int j = 0; j < kEarlyRows; ++j)
      if (i < n && (uint32_t)j < count && key == er[j]) {
        match[k] = (uint32_t)j + 1u;
        c[j] += 1u;
      }
  }
  uint32_t incl[kEarlyRows];
#pragma unroll
  for (int j = 0; j < kEarlyRows; ++j) {
    uint32_t v = c[j];
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t u = __shfl_up(v, o);
      if (lane >= o) v += u;
    }
    incl[j] = v;
    if (lane == 63) wtot[wave][j] = v;
  }
  __syncthreads();
  uint32_t pos[kEarlyRows];
#pragma unroll
  for (int j = 0; j < kEarlyRows; ++j) {
    uint32_t wb = 0;
    for (int w = 0; w < wave; ++w) wb += wtot[w][j];
    pos[j] = start[j] + wb + incl[j] - c[j];
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) {
#pragma unroll
    for (int j = 0; j < kEarlyRows; ++j)
      if (match[k] == (uint32_t)j + 1u) list[pos[j]++] = (uint32_t)(base + k);
  }
}

// Early row j's slices: workgroup j * slices + slice.
template <typename Tag, ScatterOp OP>
__global__ void __launch_bounds__(256) scatter_early_fold(int64_t row_elems,
                                                          const typename StorageOf<Tag>::T* __restrict__ operand,
                                                          const typename StorageOf<Tag>::T* updates,
                                                          const uint32_t* __restrict__ early,
                                                          const uint32_t* __restrict__ row_starts, int64_t stride,
                                                          const uint32_t* list, typename StorageOf<Tag>::T* __restrict__ out,
                                                          int xcd_group) {
  typedef typename StorageOf<Tag>::T T;
  typedef HotShape<T> S;
  __shared__ __align__(16) T lds[2 * S::BUF];
  const int64_t slices = (row_elems + S::COLS - 1) / S::COLS;
  // xcd_group: workgroup b (XCD b % 8) takes slot (b % 8) * (grid / 8) + b / 8,
  // so one row's slices share an XCD (ScatterHotList::xcd_group).
  const int64_t b = xcd_group && gridDim.x % 8 == 0 ? (int64_t)(blockIdx.x % 8) * (gridDim.x / 8) + blockIdx.x / 8
                                                     : (int64_t)blockIdx.x;
  const uint32_t j = (uint32_t)(b / slices);
  const int slice = (int)(b % slices);
  if (j >= early[0]) return;
  const uint32_t lo = row_starts[(int64_t)j * stride], hi = row_starts[(int64_t)(j + 1) * stride];
  if (hi <= lo) return;  // a selected row appears in the sample, so never empty
  hot_slice_fold<Tag, OP>(row_elems, early[1 + j], slice, operand, updates, list, lo, hi - lo, out, lds);
}

template <typename Tag, ScatterOp OP, int VEC>
__global__ void __launch_bounds__(256) scatter_rows_fold(
    ScatterRowsParams p, const typename StorageOf<Tag>::T* __restrict__ operand,
    const typename StorageOf<Tag>::T* __restrict__ updates, const uint32_t* __restrict__ perm,
    const uint32_t* __restrict__ seg_start, const uint32_t* __restrict__ seg_end,
    typename StorageOf<Tag>::T* __restrict__ out, const uint32_t* __restrict__ early) {
  typedef Codec<Tag> K;
  typedef typename K::C C;
  typedef typename StorageOf<Tag>::T T;
  typedef VecOf<T, VEC> V;
  // One wave per row, 4 rows per workgroup.
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + wave;
  if (r >= p.rows) return;
  if (is_early_row(early, r)) return;  // folded by the early path
  const uint32_t lo = seg_start[r], hi = seg_end[r];
  if (p.hot_wgs > 0 && hi - lo > (uint32_t)kHotMinUpdates) return;  // a hot row: folded by slices
  const T* xr = operand + r * p.row_elems;
  T* dst = out + r * p.row_elems;
  if (lo == hi) {
    if (operand != out)
      for (int64_t c0 = (int64_t)lane * VEC; c0 < p.row_elems; c0 += 64 * VEC)
        *reinterpret_cast<V*>(dst + c0) = *reinterpret_cast<const V*>(xr + c0);
    return;
  }
  for (int64_t c0 = (int64_t)lane * VEC; c0 < p.row_elems; c0 += 64 * VEC) {
    C acc[VEC];
    const V first = *reinterpret_cast<const V*>(xr + c0);
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = K::ld(first.v[e]);
    uint32_t i = lo;
    for (; i + kFoldDepth <= hi; i += kFoldDepth) {
      V u[kFoldDepth];
#pragma unroll
      for (int d = 0; d < kFoldDepth; ++d)
        u[d] = load_once(reinterpret_cast<const V*>(updates + (int64_t)perm[i + d] * p.row_elems + c0));
#pragma unroll
      for (int d = 0; d < kFoldDepth; ++d)
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] = fold1<Tag, OP>(acc[e], K::ld(u[d].v[e]));
    }
    for (; i < hi; ++i) {
      const V u = load_once(reinterpret_cast<const V*>(updates + (int64_t)perm[i] * p.row_elems + c0));
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] = fold1<Tag, OP>(acc[e], K::ld(u.v[e]));
    }
    V o;
#pragma unroll
    for (int e = 0; e < VEC; ++e) o.v[e] = K::st(acc[e]);
    *reinterpret_cast<V*>(dst + c0) = o;
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
  hipLaunchKernelGGL(scan_apply, dim3(blocks(n, kScanTile)), dim3(256), 0, s, in, out, n, tmp);
}

}  // namespace

size_t radix_sort_scratch_bytes(int64_t n) {
  const int64_t nblocks = (n + kTile - 1) / kTile;
  return static_cast<size_t>(512 * nblocks * 2 + kScanTile) * 4;
}

void launch_radix_sort(hipStream_t s, uint32_t* keys, uint32_t* vals, uint32_t* tmp_keys, uint32_t* tmp_vals,
                       void* scratch, int64_t n, int bits) {
  if (n <= 1) return;
  const int64_t nblocks = (n + kTile - 1) / kTile;
  PJRTX_CHECK(256 * nblocks <= int64_t(kScanTile) * kScanTile, Code::kUnimplemented, "radix sort: too many elements");
  // 9-bit digits when that saves a pass (17 or 18 key bits: two passes
  // instead of three, and no copy back), 8-bit ones otherwise.
  const bool nine = (bits + 8) / 9 < (bits + 7) / 8 && 512 * nblocks <= int64_t(kScanTile) * kScanTile;
  const int width = nine ? 9 : 8;
  const int64_t bins = int64_t(1) << width;
  uint32_t* hist = static_cast<uint32_t*>(scratch);
  uint32_t* offs = hist + bins * nblocks;
  uint32_t* tmp = offs + bins * nblocks;
  uint32_t *ki = keys, *vi = vals, *ko = tmp_keys, *vo = tmp_vals;
  const int passes = (bits + width - 1) / width;
  for (int pass = 0; pass < passes; ++pass) {
    const int shift = pass * width;
    if (nine)
      hipLaunchKernelGGL(radix_hist<9>, dim3(static_cast<unsigned>(nblocks)), dim3(64), 0, s, ki, n, shift, hist,
                         static_cast<int>(nblocks));
    else
      hipLaunchKernelGGL(radix_hist<8>, dim3(static_cast<unsigned>(nblocks)), dim3(64), 0, s, ki, n, shift, hist,
                         static_cast<int>(nblocks));
    exclusive_scan(s, hist, offs, bins * nblocks, tmp);
    if (nine)
      hipLaunchKernelGGL(radix_scatter<9>, dim3(static_cast<unsigned>(nblocks)), dim3(64), 0, s, ki, vi, ko, vo, n,
                         shift, offs, static_cast<int>(nblocks));
    else
      hipLaunchKernelGGL(radix_scatter<8>, dim3(static_cast<unsigned>(nblocks)), dim3(64), 0, s, ki, vi, ko, vo, n,
                         shift, offs, static_cast<int>(nblocks));
    std::swap(ki, ko);
    std::swap(vi, vo);
  }
  if (ki != keys) {  // odd number of passes: copy back
    hcheck(hipMemcpyAsync(keys, ki, n * 4, hipMemcpyDeviceToDevice, s), "hipMemcpyAsync(sort keys)");
    hcheck(hipMemcpyAsync(vals, vi, n * 4, hipMemcpyDeviceToDevice, s), "hipMemcpyAsync(sort values)");
  }
  check("radix_sort");
}

void launch_scatter_keys(hipStream_t s, const ScatterKeyParams& p, const void* indices, uint32_t* keys, uint32_t* vals,
                         uint32_t* keys2, uint32_t* zero, int64_t zero_n) {
  if (p.items == 0 && zero_n == 0) return;
  hipLaunchKernelGGL(scatter_keys, dim3(blocks(std::max<int64_t>(p.items, zero_n), 256)), dim3(256), 0, s, p, indices,
                     keys, vals, keys2, zero, zero_n);
  check("scatter_keys");
}

void launch_scatter_segments(hipStream_t s, const uint32_t* sorted_keys, int64_t n, uint32_t invalid,
                             uint32_t* seg_start, uint32_t* seg_end, int64_t rows, int64_t extra_zero, bool zeroed) {
  // Zero with a kernel (not a memset node), so the sequence stays capturable.
  if (zeroed) {
  } else if (seg_end == seg_start + rows) {
    hipLaunchKernelGGL(zero_u32, dim3(blocks(2 * rows + extra_zero, 256)), dim3(256), 0, s, seg_start,
                       2 * rows + extra_zero);
  } else {
    hipLaunchKernelGGL(zero_u32, dim3(blocks(rows, 256)), dim3(256), 0, s, seg_start, rows);
    hipLaunchKernelGGL(zero_u32, dim3(blocks(rows + extra_zero, 256)), dim3(256), 0, s, seg_end, rows + extra_zero);
  }
  if (n == 0) return;
  hipLaunchKernelGGL(scatter_segments, dim3(blocks(n, 256)), dim3(256), 0, s, sorted_keys, n, invalid, seg_start,
                     seg_end);
  check("scatter_segments");
}



ScatterHotList scatter_hot_list(int64_t n, uint32_t* counts, uint32_t* rows_list) {
  ScatterHotList h;
  h.counts = counts;
  h.rows = rows_list;
  h.kmin = 0;
  while ((int64_t(1) << (h.kmin + 1)) <= kHotMinUpdates + 1) ++h.kmin;  // 2^kmin <= kHotMinUpdates + 1
  int64_t base = 0;
  for (int k = 31; k >= 0; --k) {
    h.base[k] = base;
    if (k >= h.kmin) base += n >> k;  // a class-k row holds at least 2^k updates
  }
  return h;
}

size_t scatter_hot_list_words(int64_t n) {
  const ScatterHotList h = scatter_hot_list(n, nullptr, nullptr);
  return static_cast<size_t>(h.base[h.kmin] + (n >> h.kmin));
}

void launch_scatter_rows(hipStream_t s, hipStream_t aux, hipEvent_t fork, hipEvent_t join, int64_t rows,
                         int64_t row_elems, int op_i, DType t, const void* operand, const void* updates,
                         const uint32_t* perm, const uint32_t* seg_start, const uint32_t* seg_end,
                         const ScatterHotList& h, int64_t hot_wgs, void* out, const uint32_t* early_rows) {
  if (rows == 0 || row_elems == 0) return;
  const ScatterOp op = static_cast<ScatterOp>(op_i);
  const size_t es = dtype_size(t);
  const bool vec = (row_elems * es) % 16 == 0 && (reinterpret_cast<uintptr_t>(operand) % 16 == 0) &&
                   (reinterpret_cast<uintptr_t>(updates) % 16 == 0) && (reinterpret_cast<uintptr_t>(out) % 16 == 0);
  ScatterRowsParams p;
  p.rows = rows;
  p.row_elems = row_elems;
  p.hot_wgs = vec && aux ? hot_wgs : 0;
  // Integer add / max / min: order-free, so hot rows fold in parallel
  // chunks merged with atomics instead of sequential column chains.
  const bool int_type = t == DType::kS32 || t == DType::kU32 || t == DType::kS64;
  const bool chunked = int_type && (op == ScatterOp::kAdd || op == ScatterOp::kMax || op == ScatterOp::kMin);
  const bool init = chunked && operand != out;
  if (p.hot_wgs > 0) {
    // The identity of the chunks' reduction, as 16 bytes of the element type.
    uint4 identity = {0u, 0u, 0u, 0u};
    if (op != ScatterOp::kAdd) {
      const bool mx = op == ScatterOp::kMax;
      uint32_t w[4];
      if (t == DType::kS32) w[0] = w[1] = w[2] = w[3] = mx ? 0x80000000u : 0x7fffffffu;
      else if (t == DType::kU32) w[0] = w[1] = w[2] = w[3] = mx ? 0u : 0xffffffffu;
      else w[0] = w[2] = mx ? 0u : 0xffffffffu, w[1] = w[3] = mx ? 0x80000000u : 0x7fffffffu;  // s64, little-endian
      identity = uint4{w[0], w[1], w[2], w[3]};
    }
    hipLaunchKernelGGL(scatter_hot_classify, dim3(blocks(rows, 256)), dim3(256), 0, s, seg_start, seg_end, rows, h,
                       identity, init ? static_cast<uint4*>(out) : nullptr, row_elems * static_cast<int64_t>(es) / 16,
                       early_rows);
    check("scatter_hot_classify");
  }
  // The hot rows and the bulk rows fold at once on two streams: the hot
  // rows on the second stream, the bulk rows on `s` (PJRTX_SCATTER_HOT_MAIN=1
  // swaps them, so the hot rows start first: slower, measured).
  hipStream_t hot_s = aux, bulk_s = s;
  if (p.hot_wgs > 0) {
    hcheck(hipEventRecord(fork, s), "hipEventRecord(scatter fork)");
    hcheck(hipStreamWaitEvent(aux, fork, 0), "hipStreamWaitEvent(scatter fork)");
    if (env_int("PJRTX_SCATTER_HOT_MAIN", 0) != 0) {
      hot_s = s;
      bulk_s = aux;
    }
  }
  const dim3 gh(static_cast<unsigned>(p.hot_wgs)), gb(static_cast<unsigned>(blocks(rows, 4))), blk(256);
#define PJRTX_HOT_OP(TAG, OPV)                                                                                        \
  hipLaunchKernelGGL((scatter_hot_fold<TAG, OPV>), gh, blk, 0, hot_s, row_elems, (const StorageOf<TAG>::T*)operand, \
                     (const StorageOf<TAG>::T*)updates, perm, seg_start, seg_end, h, (StorageOf<TAG>::T*)out)
#define PJRTX_CHUNK_OP(TAG, OPV)                                                                                      \
  do {                                                                                                                \
    if constexpr (std::is_integral<StorageOf<TAG>::T>::value && OPV != ScatterOp::kSet && OPV != ScatterOp::kMul)     \
      hipLaunchKernelGGL((scatter_hot_chunks<StorageOf<TAG>::T, OPV>), gh, blk, 0, hot_s, row_elems,                  \
                         (const StorageOf<TAG>::T*)updates, perm, seg_start, seg_end, h,                              \
                         init ? (const StorageOf<TAG>::T*)operand : nullptr, (StorageOf<TAG>::T*)out);               \
  } while (0)
#define PJRTX_ROWS_OP(TAG, V, OPV)                                                                                    \
  do {                                                                                                                \
    if (V * sizeof(StorageOf<TAG>::T) == 16 && p.hot_wgs > 0) {                                                      \
      if (chunked) PJRTX_CHUNK_OP(TAG, OPV);                                                                         \
      else PJRTX_HOT_OP(TAG, OPV);                                                                                    \
    }                                                                                                                 \
    hipLaunchKernelGGL((scatter_rows_fold<TAG, OPV, V>), gb, blk, 0, p.hot_wgs > 0 ? bulk_s : s, p,                  \
                       (const StorageOf<TAG>::T*)operand,                                                            \
                       (const StorageOf<TAG>::T*)updates, perm, seg_start, seg_end, (StorageOf<TAG>::T*)out,         \
                       early_rows);                                                                                   \
  } while (0)
#define PJRTX_ROWS_V(TAG, V)                                              \
  switch (op) {                                                           \
    case ScatterOp::kAdd: PJRTX_ROWS_OP(TAG, V, ScatterOp::kAdd); break;  \
    case ScatterOp::kSet: PJRTX_ROWS_OP(TAG, V, ScatterOp::kSet); break;  \
    case ScatterOp::kMax: PJRTX_ROWS_OP(TAG, V, ScatterOp::kMax); break;  \
    case ScatterOp::kMin: PJRTX_ROWS_OP(TAG, V, ScatterOp::kMin); break;  \
    case ScatterOp::kMul: PJRTX_ROWS_OP(TAG, V, ScatterOp::kMul); break;  \
  }
#define PJRTX_ROWS_T(TAG, V16)  \
  if (vec) {                    \
    PJRTX_ROWS_V(TAG, V16)      \
  } else {                      \
    PJRTX_ROWS_V(TAG, 1)        \
  }
  switch (t) {
    case DType::kF32: PJRTX_ROWS_T(float, 4) break;
    case DType::kF64: PJRTX_ROWS_T(double, 2) break;
    case DType::kBF16: PJRTX_ROWS_T(Bf16Tag, 8) break;
    case DType::kF16: PJRTX_ROWS_T(F16Tag, 8) break;
    case DType::kS32: PJRTX_ROWS_T(int32_t, 4) break;
    case DType::kU32: PJRTX_ROWS_T(uint32_t, 4) break;
    case DType::kS64: PJRTX_ROWS_T(int64_t, 2) break;
    default: fail(Code::kUnimplemented, std::string("scatter: element type not supported: ") + dtype_name(t));
  }
#undef PJRTX_ROWS_T
#undef PJRTX_ROWS_V
#undef PJRTX_ROWS_OP
#undef PJRTX_HOT_OP
#undef PJRTX_CHUNK_OP
  check("scatter_rows_fold");
  if (p.hot_wgs > 0) {
    hcheck(hipEventRecord(join, aux), "hipEventRecord(scatter join)");
    hcheck(hipStreamWaitEvent(s, join, 0), "hipStreamWaitEvent(scatter join)");
  }
}

void launch_scatter_early(hipStream_t aux, hipEvent_t selected, const ScatterEarly& e, const uint32_t* keys, int64_t n,
                          uint32_t invalid, int64_t row_elems, int op_i, DType t, const void* operand,
                          const void* updates, void* out) {
  PJRTX_CHECK(n >= kEarlySample && e.blocks == scatter_early_blocks(n), Code::kInternal, "scatter early: bad sizes");
  const ScatterOp op = static_cast<ScatterOp>(op_i);
  hipLaunchKernelGGL(scatter_early_select, dim3(1), dim3(1024), 0, aux, keys, n, invalid, e.rows);
  check("scatter_early_select");
  hcheck(hipEventRecord(selected, aux), "hipEventRecord(scatter early selected)");
  const dim3 gb(static_cast<unsigned>(e.blocks)), blk(256);
  hipLaunchKernelGGL(scatter_early_count, gb, blk, 0, aux, keys, n, e.rows, e.counts, e.blocks);
  // Up to kEarlyInlineBlocks workgroups compute their own offsets (no scan
  // launches on the early path); the fold then reads the rows' starts.
  const bool inline_scan = e.blocks <= kEarlyInlineBlocks;
  if (!inline_scan) exclusive_scan(aux, e.counts, e.offsets, kEarlyRows * e.blocks + 1, e.scan_tmp);
  hipLaunchKernelGGL(scatter_early_write, gb, blk, 0, aux, keys, n, e.rows, inline_scan ? nullptr : e.offsets,
                     e.counts, e.offsets, e.blocks, e.list);
  const int64_t stride = inline_scan ? 1 : e.blocks;
  const size_t es = dtype_size(t);
  const int64_t cols = kHotSliceBytes / static_cast<int64_t>(es);
  const dim3 gf(static_cast<unsigned>(kEarlyRows * ((row_elems + cols - 1) / cols)));
#define PJRTX_EARLY(TAG, OPV)                                                                                        \
  hipLaunchKernelGGL((scatter_early_fold<TAG, OPV>), gf, blk, 0, aux, row_elems, (const StorageOf<TAG>::T*)operand, \
                     (const StorageOf<TAG>::T*)updates, e.rows, e.offsets, stride, e.list, (StorageOf<TAG>::T*)out,       \
                     e.xcd_group)
#define PJRTX_EARLY_T(TAG)                                          \
  switch (op) {                                                     \
    case ScatterOp::kAdd: PJRTX_EARLY(TAG, ScatterOp::kAdd); break; \
    case ScatterOp::kSet: PJRTX_EARLY(TAG, ScatterOp::kSet); break; \
    case ScatterOp::kMax: PJRTX_EARLY(TAG, ScatterOp::kMax); break; \
    case ScatterOp::kMin: PJRTX_EARLY(TAG, ScatterOp::kMin); break; \
    case ScatterOp::kMul: PJRTX_EARLY(TAG, ScatterOp::kMul); break; \
  }
  switch (t) {
    case DType::kF32: PJRTX_EARLY_T(float) break;
    case DType::kF64: PJRTX_EARLY_T(double) break;
    case DType::kBF16: PJRTX_EARLY_T(Bf16Tag) break;
    case DType::kF16: PJRTX_EARLY_T(F16Tag) break;
    case DType::kS32: PJRTX_EARLY_T(int32_t) break;
    case DType::kU32: PJRTX_EARLY_T(uint32_t) break;
    case DType::kS64: PJRTX_EARLY_T(int64_t) break;
    default: fail(Code::kUnimplemented, std::string("scatter: element type not supported: ") + dtype_name(t));
  }
#undef PJRTX_EARLY_T
#undef PJRTX_EARLY
  check("scatter_early_fold");
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
