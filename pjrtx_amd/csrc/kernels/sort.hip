// Row sorts for stablehlo.sort and chlo.top_k on gfx950.
//
// Replaces the reference's MLX sort / argsort / take_along_axis chain
// (reference: src/backend/mlx_metal/api.cc:3248-3347, dispatched from
// execution_node_indexing.zig:83-88 and execution_node_indexing_order.zig:
// 12-72, which sorts ascending and reverses for GT comparators). Here a
// descending order is an ascending sort of the inverted key image, so equal
// keys keep their positions' order in both directions (a stable sort, as
// StableHLO's is_stable and XLA's TopK ask).
//
// Three kernels:
//  * sort_local: one workgroup sorts up to kSortBlock words of a row in LDS
//    (a bitonic network; 512 threads, each doing 4 compare-exchanges per
//    stage) and either keeps the first `keep` words or writes the results.
//  * bitonic_global: one compare-exchange stage with partner distance of
//    at least kSortBlock, for rows longer than one LDS block.
//  * sort_write: gathers the results of words held in HBM.
// top_k with k <= kSortBlock / 2 reduces instead of sorting the whole row:
// each block keeps its first k' = pow2 >= k words (every word of the row's
// top k is among its block's top k'), and the survivors are sorted again
// until one block holds them all. At [64, 128256] that is two LDS passes.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.h"
#include "kernels/sort.h"

namespace pjrtx {
namespace {

constexpr uint64_t kSentinel = ~0ull;  // sorts after every word (positions are < 2^31)
constexpr int kLocalThreads = 512;

struct LocalPass {
  // Source: raw keys of operand 0 (list == nullptr) or a list of words.
  const void* keys = nullptr;
  SortRows r;
  const uint64_t* list = nullptr;
  int64_t list_len = 0, list_stride = 0;
  int block = 0;              // words per workgroup, a power of two <= kSortBlock
  int64_t blocks_per_row = 1;
  int64_t k_first = 2, k_last = 2, j_first = 1;
  int global_dir = 0;         // direction from the word's row position (global network) or block position
  // Destination: the first `keep` words of each block, or the results.
  uint64_t* dst = nullptr;
  int64_t keep = 0, dst_stride = 0;
  int write_out = 0;
  int filter = 0;             // sort only the words that can be among the first `keep` (or out_n)
  SortGather g;
};

__device__ __forceinline__ uint32_t load_key(const void* keys, int64_t e, int bits) {
  if (bits == 32) return static_cast<const uint32_t*>(keys)[e];
  if (bits == 16) return static_cast<const uint16_t*>(keys)[e];
  return static_cast<const uint8_t*>(keys)[e];
}

// Order-preserving image of a key (ascending), inverted for descending.
__device__ __forceinline__ uint32_t key_image(uint32_t raw, const SortRows& r) {
  const uint32_t mask = r.key_bits == 32 ? 0xffffffffu : ((1u << r.key_bits) - 1u);
  const uint32_t sign = 1u << (r.key_bits - 1);
  uint32_t v = raw & mask, img;
  if (r.key_class == kSortKeySigned) {
    img = v ^ sign;
  } else if (r.key_class == kSortKeyUnsigned) {
    img = v;
  } else {
    const uint32_t mag = v & ~sign;
    if (r.key_class == kSortKeyFloat && mag > r.inf_bits) {
      img = mask;  // every NaN: one class, after +inf
    } else {
      if (r.key_class == kSortKeyFloat && mag == 0) v = 0;  // -0 == +0
      img = (v & sign) ? (~v & mask) : (v | sign);
    }
  }
  return r.descending ? (~img & mask) : img;
}

// Minimum over the wave's 64 lanes, in every lane (a butterfly of lane swaps).
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
  for (int d = 1; d < 64; d <<= 1) {
    const uint64_t o = __shfl_xor(v, d, 64);
    v = o < v ? o : v;
  }
  return v;
}

template <typename T>
__device__ __forceinline__ void copy_elem(const void* src, void* dst, int64_t s, int64_t d) {
  static_cast<T*>(dst)[d] = static_cast<const T*>(src)[s];
}

// Result i of `row` comes from position `pos` of the same row.
__device__ __forceinline__ void gather_one(const SortGather& g, const SortRows& r, int64_t row, int64_t i,
                                           int64_t pos) {
  const int64_t outer = row / r.inner, j = row - outer * r.inner;
  const int64_t s = (outer * r.n + pos) * r.inner + j;
  const int64_t d = (outer * g.out_n + i) * r.inner + j;
  for (int o = 0; o < g.count; ++o) {
    switch (g.elem_bytes[o]) {
      case 1: copy_elem<uint8_t>(g.src[o], g.dst[o], s, d); break;
      case 2: copy_elem<uint16_t>(g.src[o], g.dst[o], s, d); break;
      case 4: copy_elem<uint32_t>(g.src[o], g.dst[o], s, d); break;
      default: copy_elem<uint64_t>(g.src[o], g.dst[o], s, d); break;
    }
  }
  if (g.index_dst) static_cast<int32_t*>(g.index_dst)[d] = static_cast<int32_t>(pos);
}

__global__ void __launch_bounds__(kLocalThreads) sort_local_kernel(LocalPass p) {
  __shared__ uint64_t s[kSortBlock];
  const int64_t row = blockIdx.x / p.blocks_per_row;
  const int64_t blk = blockIdx.x - row * p.blocks_per_row;
  const int B = p.block;
  const int64_t base = blk * B;
  // Loads in batches of kBatch per thread, all issued before any is used
  // (one outstanding load per thread would leave the kernel latency-bound).
  constexpr int kBatch = 8;
  const int bd = static_cast<int>(blockDim.x);
  if (p.list) {
    const uint64_t* src = p.list + row * p.list_stride;
    for (int i0 = 0; i0 < B; i0 += kBatch * bd) {
      uint64_t w[kBatch];
#pragma unroll
      for (int q = 0; q < kBatch; ++q) {
        const int i = i0 + q * bd + static_cast<int>(threadIdx.x);
        const int64_t idx = base + i;
        w[q] = (i < B && idx < p.list_len) ? src[idx] : kSentinel;
      }
#pragma unroll
      for (int q = 0; q < kBatch; ++q) {
        const int i = i0 + q * bd + static_cast<int>(threadIdx.x);
        if (i < B) s[i] = w[q];
      }
    }
  } else {
    const int64_t outer = row / p.r.inner, j = row - outer * p.r.inner;
    const int64_t row0 = outer * p.r.n * p.r.inner + j;
    for (int i0 = 0; i0 < B; i0 += kBatch * bd) {
      uint32_t raw[kBatch];
#pragma unroll
      for (int q = 0; q < kBatch; ++q) {
        const int i = i0 + q * bd + static_cast<int>(threadIdx.x);
        const int64_t idx = base + i;
        raw[q] = (i < B && idx < p.r.n) ? load_key(p.keys, row0 + idx * p.r.inner, p.r.key_bits) : 0u;
      }
#pragma unroll
      for (int q = 0; q < kBatch; ++q) {
        const int i = i0 + q * bd + static_cast<int>(threadIdx.x);
        const int64_t idx = base + i;
        if (i < B)
          s[i] = idx < p.r.n ? ((static_cast<uint64_t>(key_image(raw[q], p.r)) << 32) | static_cast<uint64_t>(idx))
                             : kSentinel;
      }
    }
  }
  __syncthreads();
  int M = B;  // words the network sorts
  if (p.filter) {
    // Only the first `need` words are wanted. Each wave takes the r-th
    // smallest of its lanes' minima (r = need / waves, rounded up): the wave
    // then holds r distinct words at or below it, so the largest of the
    // waves' values, T, has at least `need` words at or below it, and every
    // word below the need-th is <= T. Only the words <= T are sorted.
    __shared__ uint64_t wave_t[kLocalThreads / 64];
    __shared__ uint32_t cnt;
    const int need = static_cast<int>(p.write_out ? p.g.out_n : p.keep);
    const int waves = bd / 64, wv = static_cast<int>(threadIdx.x) / 64;
    const int r = (need + waves - 1) / waves;
    // B is a multiple of the workgroup size (both powers of two, B >= 256),
    // so `q < nm` is uniform across the workgroup.
    constexpr int kMine = kSortBlock / kLocalThreads;
    const int nm = B / bd;
    uint64_t mine[kMine];
    uint64_t lo = kSentinel;
#pragma unroll
    for (int q = 0; q < kMine; ++q) {
      if (q < nm) {
        mine[q] = s[threadIdx.x + q * bd];
        lo = mine[q] < lo ? mine[q] : lo;
      }
    }
    if (threadIdx.x == 0) cnt = 0;
    uint64_t t = kSentinel, v = lo;
    for (int round = 0; round < r; ++round) {
      t = wave_min_u64(v);
      const uint64_t owner = __ballot(v == t);  // words are distinct: one lane, or none once all are sentinels
      if (static_cast<int>(__lane_id()) == __ffsll(static_cast<unsigned long long>(owner)) - 1) v = kSentinel;
    }
    if (__lane_id() == 0) wave_t[wv] = t;
    __syncthreads();
    uint64_t T = 0;
    for (int w = 0; w < waves; ++w) T = wave_t[w] > T ? wave_t[w] : T;
#pragma unroll
    for (int q = 0; q < kMine; ++q) {
      if (q >= nm) break;
      // One LDS atomic per wave: the wave's slots, then each lane's rank.
      const bool take = mine[q] <= T;
      const uint64_t mask = __ballot(take);
      if (mask) {
        uint32_t base = 0;
        if (__lane_id() == 0) base = atomicAdd(&cnt, static_cast<uint32_t>(__popcll(mask)));
        base = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(base)));
        const uint32_t rank = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                                        __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
        if (take) s[base + rank] = mine[q];
      }
    }
    __syncthreads();
    const int m = static_cast<int>(cnt);
    M = 2;
    while (M < m) M <<= 1;
    for (int i = m + threadIdx.x; i < M; i += bd) s[i] = kSentinel;
    __syncthreads();
  }
  for (int64_t k = p.k_first; k <= (p.filter ? M : p.k_last); k <<= 1) {
    // Within a block only bit log2(k) of the row position matters: it is the
    // block's (base & k) when k >= B, else the position's own bit.
    const bool block_up = !p.global_dir || k < B || (base & k) == 0;
    const int kb = k < B ? static_cast<int>(k) : 0;
    for (int64_t jj = (k == p.k_first ? p.j_first : k >> 1); jj > 0; jj >>= 1) {
      const int j = static_cast<int>(jj);
      for (int t = threadIdx.x; t < M / 2; t += blockDim.x) {
        const int i = ((t & ~(j - 1)) << 1) | (t & (j - 1));
        const int l = i | j;
        const bool up = block_up == ((i & kb) == 0);
        const uint64_t a = s[i], b = s[l];
        if ((a > b) == up) {
          s[i] = b;
          s[l] = a;
        }
      }
      __syncthreads();
    }
  }
  if (p.write_out) {
    for (int i = threadIdx.x; i < p.g.out_n; i += blockDim.x)
      gather_one(p.g, p.r, row, i, static_cast<int64_t>(s[i] & 0xffffffffu));
  } else {
    uint64_t* dst = p.dst + row * p.dst_stride + blk * p.keep;
    for (int i = threadIdx.x; i < p.keep; i += blockDim.x) dst[i] = s[i];
  }
}

__global__ void bitonic_global_kernel(uint64_t* a, int64_t rows, int64_t p, int64_t k, int64_t j) {
  const int64_t half = p >> 1;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= rows * half) return;
  const int64_t row = t / half, tt = t - row * half;
  const int64_t i = ((tt & ~(j - 1)) << 1) | (tt & (j - 1));
  const int64_t l = i | j;
  const bool up = (i & k) == 0;
  uint64_t* r = a + row * p;
  const uint64_t x = r[i], y = r[l];
  if ((x > y) == up) {
    r[i] = y;
    r[l] = x;
  }
}

__global__ void sort_write_kernel(const uint64_t* list, int64_t list_stride, SortRows r, SortGather g) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= r.rows * g.out_n) return;
  const int64_t row = t / g.out_n, i = t - row * g.out_n;
  gather_one(g, r, row, i, static_cast<int64_t>(list[row * list_stride + i] & 0xffffffffu));
}

int64_t pow2_at_least(int64_t v) {
  int64_t p = 1;
  while (p < v) p <<= 1;
  return p;
}

void check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) fail(Code::kInternal, strformat("%s launch failed: %s", what, hipGetErrorString(e)));
}

void local(hipStream_t s, const LocalPass& p, int64_t rows) {
  const int64_t grid = rows * p.blocks_per_row;
  PJRTX_CHECK(grid > 0 && grid < (int64_t{1} << 31), Code::kUnimplemented, "sort: too many rows");
  const int threads = static_cast<int>(std::min<int64_t>(kLocalThreads, std::max<int64_t>(64, p.block / 2)));
  hipLaunchKernelGGL(sort_local_kernel, dim3(static_cast<unsigned>(grid)), dim3(threads), 0, s, p);
  check_launch("sort_local");
}

// Words of scratch for each path (0 when one LDS block holds a row).
struct Layout {
  int path = 0;                // 0: one block; 1: top-k reduction; 2: full bitonic
  int64_t kp = 0, len1 = 0;    // top-k: words kept per block, list length after round one
  int64_t p = 0;               // full: padded row length
};

Layout layout_of(const SortRows& r, int64_t out_n) {
  Layout L;
  if (r.n <= kSortBlock) return L;
  L.kp = pow2_at_least(std::max<int64_t>(out_n, 1));
  if (out_n < r.n && L.kp <= kSortBlock / 2) {
    L.path = 1;
    L.len1 = (r.n + kSortBlock - 1) / kSortBlock * L.kp;
  } else {
    L.path = 2;
    L.p = pow2_at_least(r.n);
  }
  return L;
}

}  // namespace

size_t sort_scratch_bytes(const SortRows& r, int64_t out_n) {
  const Layout L = layout_of(r, out_n);
  if (L.path == 1) return static_cast<size_t>(2 * r.rows * L.len1) * 8;
  if (L.path == 2) return static_cast<size_t>(r.rows * L.p) * 8;
  return 0;
}

void sort_rows(hipStream_t s, const SortRows& r, const void* keys, const SortGather& g, void* scratch) {
  if (r.rows == 0 || r.n == 0 || g.out_n == 0) return;
  PJRTX_CHECK(r.n < (int64_t{1} << 31) && g.out_n <= r.n, Code::kInvalidArgument, "sort: row length out of range");
  PJRTX_CHECK(r.key_bits == 8 || r.key_bits == 16 || r.key_bits == 32, Code::kUnimplemented,
              "sort: keys wider than 32 bits are not supported");
  const Layout L = layout_of(r, g.out_n);
  LocalPass p;
  p.keys = keys;
  p.r = r;
  p.g = g;
  if (L.path == 0) {
    p.block = static_cast<int>(pow2_at_least(std::max<int64_t>(r.n, 2)));
    p.k_first = 2, p.k_last = p.block, p.j_first = 1;
    p.write_out = 1;
    p.filter = 8 * g.out_n <= p.block && p.block >= 256;
    local(s, p, r.rows);
    return;
  }
  uint64_t* buf = static_cast<uint64_t*>(scratch);
  if (L.path == 1) {
    // Round one from the keys, then rounds over the kept words.
    uint64_t* a = buf;
    uint64_t* b = buf + r.rows * L.len1;
    p.block = kSortBlock;
    p.blocks_per_row = (r.n + kSortBlock - 1) / kSortBlock;
    p.k_first = 2, p.k_last = kSortBlock, p.j_first = 1;
    p.keep = L.kp;
    p.filter = 8 * L.kp <= kSortBlock;
    p.dst = a;
    p.dst_stride = L.len1;
    local(s, p, r.rows);
    int64_t len = L.len1, stride = L.len1;
    while (len > kSortBlock) {
      LocalPass q = p;
      q.keys = nullptr;
      q.list = a, q.list_len = len, q.list_stride = stride;
      q.blocks_per_row = (len + kSortBlock - 1) / kSortBlock;
      q.dst = b;
      q.dst_stride = q.blocks_per_row * L.kp;
      local(s, q, r.rows);
      len = q.dst_stride, stride = q.dst_stride;
      std::swap(a, b);
    }
    LocalPass f = p;
    f.keys = nullptr;
    f.list = a, f.list_len = len, f.list_stride = stride;
    f.block = static_cast<int>(pow2_at_least(std::max<int64_t>(len, 2)));
    f.blocks_per_row = 1;
    f.k_first = 2, f.k_last = f.block, f.j_first = 1;
    f.dst = nullptr;
    f.write_out = 1;
    f.filter = 8 * g.out_n <= f.block && f.block >= 256;
    local(s, f, r.rows);
    return;
  }
  // Full bitonic network over p words per row: LDS passes for partner
  // distances below kSortBlock, global passes for the rest.
  p.block = kSortBlock;
  p.blocks_per_row = L.p / kSortBlock;
  p.k_first = 2, p.k_last = kSortBlock, p.j_first = 1;
  p.global_dir = 1;
  p.keep = kSortBlock;
  p.dst = buf;
  p.dst_stride = L.p;
  local(s, p, r.rows);
  const int64_t pairs = r.rows * (L.p / 2);
  PJRTX_CHECK((pairs + 255) / 256 < (int64_t{1} << 31), Code::kUnimplemented, "sort: too large");
  for (int64_t k = 2 * kSortBlock; k <= L.p; k <<= 1) {
    for (int64_t j = k >> 1; j >= kSortBlock; j >>= 1) {
      hipLaunchKernelGGL(bitonic_global_kernel, dim3(static_cast<unsigned>((pairs + 255) / 256)), dim3(256), 0, s, buf,
                         r.rows, L.p, k, j);
      check_launch("bitonic_global");
    }
    LocalPass m = p;
    m.keys = nullptr;
    m.list = buf, m.list_len = L.p, m.list_stride = L.p;
    m.k_first = k, m.k_last = k, m.j_first = kSortBlock / 2;
    local(s, m, r.rows);
  }
  const int64_t outs = r.rows * g.out_n;
  hipLaunchKernelGGL(sort_write_kernel, dim3(static_cast<unsigned>((outs + 255) / 256)), dim3(256), 0, s, buf, L.p, r,
                     g);
  check_launch("sort_write");
}

}  // namespace pjrtx
