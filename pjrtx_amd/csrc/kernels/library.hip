// Precompiled library kernels: N-d box copy (slices, dynamic slices,
// dynamic-update-slice, concatenate, pad), fill, and StableHLO gather.
//
// Every kernel moves data in "units": whole elements, or 16-byte vectors
// when the innermost dimension is contiguous and aligned on both sides.
// One thread handles one unit; consecutive threads touch consecutive units
// along the innermost dimension, so accesses coalesce.
//
// Replaces the reference's slice / gather steps (reference:
// src/backend/mlx_metal/executable_metal_graph_slice.zig:8-380 incl. the
// clamped DUS starts at :293-299, executable_metal_graph_gather.zig:13-92
// with clamped indices at :61-65, executable_metal_graph_structural.zig,
// executable_metal_graph_generation.zig:8-135 concatenate).
#include <hip/hip_runtime.h>

#include <vector>

#include <cstring>

#include "common.h"
#include "kernels/library.h"

namespace pjrtx {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int B> struct Unit;
template <> struct Unit<1> { typedef uint8_t T; };
template <> struct Unit<2> { typedef uint16_t T; };
template <> struct Unit<4> { typedef uint32_t T; };
template <> struct Unit<8> { typedef uint64_t T; };
template <> struct Unit<16> { typedef u32x4 T; };

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

// A gather start index after JAX's negative-index normalization folded into
// the gather: i < 0 reads as i + wrap, the add wrapping in the index type's
// width as the program's own add does; then sign-extended as before.
__device__ __forceinline__ int64_t wrap_index(int64_t i, int64_t wrap, int bytes) {
  if (wrap == 0 || i >= 0) return i;
  const uint64_t s = (uint64_t)i + (uint64_t)wrap;
  if (bytes == 8) return (int64_t)s;
  if (bytes == 4) return (int64_t)(int32_t)(uint32_t)s;
  if (bytes == 2) return (int64_t)(int16_t)(uint16_t)s;
  return (int64_t)(int8_t)(uint8_t)s;
}

__device__ __forceinline__ int64_t clamp64(int64_t v, int64_t lo, int64_t hi) { return v < lo ? lo : (v > hi ? hi : v); }

// Box copy in units. `p` dims/strides/offsets are in units; dyn starts are in
// elements of the dynamically indexed tensor and are scaled by `dyn_scale`
// (element strides in units, per dim).
struct BoxUnits {
  BoxCopy b;
  int64_t total;
  int64_t dyn_scale[kMaxRank];
};

template <typename T>
__global__ void __launch_bounds__(256) box_copy_kernel(BoxUnits p, const T* __restrict__ src, T* __restrict__ dst) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= p.total) return;
  int64_t rem = i, so = p.b.src_off, d_o = p.b.dst_off;
  for (int d = p.b.rank - 1; d >= 0; --d) {
    const int64_t D = p.b.dims[d];
    const int64_t c = rem % D;
    rem /= D;
    so += c * p.b.src_stride[d];
    d_o += c * p.b.dst_stride[d];
  }
  // Dynamic starts: same value for every thread (uniform scalar loads).
  for (int d = 0; d < p.b.rank; ++d) {
    if (!p.b.dyn_start[d]) continue;
    int64_t st = load_index(p.b.dyn_start[d], 0, p.b.dyn_start_bytes, p.b.dyn_start_signed);
    st = clamp64(st, 0, p.b.dyn_limit[d] - p.b.dims[d]);
    if (p.b.dyn_on_dst) d_o += st * p.dyn_scale[d];
    else so += st * p.dyn_scale[d];
  }
  dst[d_o] = src[so];
}

template <typename T>
__global__ void __launch_bounds__(256) fill_kernel(T* __restrict__ dst, const T* __restrict__ value, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) dst[i] = value[0];
}

__global__ void __launch_bounds__(256) zero_bytes_kernel(uint8_t* __restrict__ dst, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) dst[i] = 0;
}

struct GatherUnits {
  GatherParams g;
  int64_t total;          // output units
  int64_t unit_elems;     // elements per unit along the innermost output dim
  int vector_inner;       // 1: innermost output dim is a full contiguous operand row
};

template <typename T>
__global__ void __launch_bounds__(256) gather_kernel(GatherUnits p, const T* __restrict__ operand,
                                                     const void* __restrict__ indices, T* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= p.total) return;
  const GatherParams& g = p.g;
  int64_t coord[kMaxRank];
  int64_t rem = i;
  for (int d = g.out_rank - 1; d >= 0; --d) {
    const int64_t D = (d == g.out_rank - 1) ? g.out_dims[d] / p.unit_elems : g.out_dims[d];
    coord[d] = rem % D;
    rem /= D;
  }
  if (g.out_rank > 0) coord[g.out_rank - 1] *= p.unit_elems;
  // Position of this output's index vector inside start_indices.
  int64_t idx_base = 0;
  int64_t batch_coord[kMaxRank];
  for (int k = 0; k < kMaxRank; ++k) batch_coord[k] = 0;
  for (int d = 0; d < g.out_rank; ++d) {
    if (g.out_map[d] >= 0) {
      idx_base += coord[d] * g.idx_stride[g.out_map[d]];
      batch_coord[g.out_map[d]] = coord[d];
    }
  }
  int64_t start[kMaxRank];
  for (int d = 0; d < g.op_rank; ++d) start[d] = 0;
  for (int k = 0; k < g.n_index; ++k) {
    const int64_t off = (g.ivd < g.idx_rank) ? (int64_t)k * g.idx_stride[g.ivd] : 0;
    start[g.start_map[k]] = wrap_index(load_index(indices, idx_base + off, g.idx_bytes, g.idx_signed), g.wrap, g.idx_bytes);
  }
  for (int k = 0; k < g.n_batching; ++k) start[g.op_batch_dim[k]] = batch_coord[g.idx_batch_dim[k]];
  int64_t src = 0;
  for (int d = 0; d < g.op_rank; ++d) {
    const int64_t s = clamp64(start[d], 0, g.op_dims[d] - g.slice[d]);
    src += s * g.op_stride[d];
  }
  for (int d = 0; d < g.out_rank; ++d)
    if (g.out_map[d] < 0) src += coord[d] * g.op_stride[-g.out_map[d] - 1];
  out[i] = operand[src / p.unit_elems];
}

// Row gather (take along axis 0 of whole rows, JAX's embedding lookup): a
// workgroup copies up to 1024 16-byte units of one output row; the row index
// is read once per thread and clamped as StableHLO clamps gather starts.
constexpr int64_t kGatherRowChunk = 1024;

__global__ void __launch_bounds__(256) gather_rows_kernel(const u32x4* __restrict__ operand,
                                                          const void* __restrict__ indices, int idx_bytes,
                                                          int idx_signed, int64_t wrap, int64_t op_rows,
                                                          int64_t units_per_row, int64_t nchunks,
                                                          u32x4* __restrict__ out) {
  const int64_t bid = blockIdx.x;
  const int64_t r = bid / nchunks, chunk = bid - r * nchunks;
  const int64_t src = clamp64(wrap_index(load_index(indices, r, idx_bytes, idx_signed), wrap, idx_bytes), 0, op_rows - 1);
  const u32x4* srow = operand + src * units_per_row;
  u32x4* drow = out + r * units_per_row;
  const int64_t u0 = chunk * kGatherRowChunk + threadIdx.x;
  u32x4 v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (u0 + 256 * j < units_per_row) v[j] = srow[u0 + 256 * j];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (u0 + 256 * j < units_per_row) drow[u0 + 256 * j] = v[j];
}

int64_t blocks_for(int64_t n) { return (n + 255) / 256; }

__device__ __forceinline__ float bf16f(uint16_t v) { return __builtin_bit_cast(float, (uint32_t)v << 16); }

__global__ void __launch_bounds__(256) add_kernel(const void* __restrict__ a, const void* __restrict__ y,
                                                  void* __restrict__ out, int64_t n, int kind) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  if (kind == 2) {
    static_cast<float*>(out)[i] = static_cast<const float*>(a)[i] + static_cast<const float*>(y)[i];
  } else if (kind == 1) {
    const float v = (float)static_cast<const _Float16*>(a)[i] + (float)static_cast<const _Float16*>(y)[i];
    static_cast<_Float16*>(out)[i] = (_Float16)v;
  } else {
    const float v = bf16f(static_cast<const uint16_t*>(a)[i]) + bf16f(static_cast<const uint16_t*>(y)[i]);
    static_cast<uint16_t*>(out)[i] = __builtin_bit_cast(uint16_t, (__bf16)v);
  }
}

void check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) fail(Code::kInternal, strformat("%s launch failed: %s", what, hipGetErrorString(e)));
}

}  // namespace

void launch_box_copy(hipStream_t s, const BoxCopy& in, const void* src, void* dst, int elem_bytes) {
  BoxUnits p;
  p.b = in;
  int64_t total = 1;
  for (int d = 0; d < in.rank; ++d) total *= in.dims[d];
  if (total == 0) return;
  for (int d = 0; d < in.rank; ++d) p.dyn_scale[d] = in.dyn_on_dst ? in.dst_stride[d] : in.src_stride[d];
  // 16-byte units when the innermost dim is contiguous on both sides and
  // every offset / stride stays 16-byte aligned.
  int unit = elem_bytes;
  const int r = in.rank;
  if (r > 0 && in.src_stride[r - 1] == 1 && in.dst_stride[r - 1] == 1 && elem_bytes < 16) {
    const int64_t per = 16 / elem_bytes;
    bool ok = in.dims[r - 1] % per == 0 && in.src_off % per == 0 && in.dst_off % per == 0 &&
              reinterpret_cast<uintptr_t>(src) % 16 == 0 && reinterpret_cast<uintptr_t>(dst) % 16 == 0;
    for (int d = 0; d + 1 < r && ok; ++d) ok = in.src_stride[d] % per == 0 && in.dst_stride[d] % per == 0;
    if (ok && in.dyn_start[r - 1]) ok = false;
    if (ok) unit = 16;
  }
  if (unit != elem_bytes) {
    const int64_t per = unit / elem_bytes;
    p.b.dims[r - 1] /= per;
    for (int d = 0; d + 1 < r; ++d) {
      p.b.src_stride[d] /= per;
      p.b.dst_stride[d] /= per;
      p.dyn_scale[d] /= per;
    }
    p.b.src_off /= per;
    p.b.dst_off /= per;
    total /= per;
  }
  p.total = total;
  const dim3 grid(static_cast<unsigned>(blocks_for(total)));
  switch (unit) {
    case 1: hipLaunchKernelGGL(box_copy_kernel<uint8_t>, grid, dim3(256), 0, s, p, (const uint8_t*)src, (uint8_t*)dst); break;
    case 2: hipLaunchKernelGGL(box_copy_kernel<uint16_t>, grid, dim3(256), 0, s, p, (const uint16_t*)src, (uint16_t*)dst); break;
    case 4: hipLaunchKernelGGL(box_copy_kernel<uint32_t>, grid, dim3(256), 0, s, p, (const uint32_t*)src, (uint32_t*)dst); break;
    case 8: hipLaunchKernelGGL(box_copy_kernel<uint64_t>, grid, dim3(256), 0, s, p, (const uint64_t*)src, (uint64_t*)dst); break;
    case 16: hipLaunchKernelGGL(box_copy_kernel<u32x4>, grid, dim3(256), 0, s, p, (const u32x4*)src, (u32x4*)dst); break;
    default: fail(Code::kInternal, "box copy: bad element size");
  }
  check_launch("box_copy");
}

void launch_fill(hipStream_t s, void* dst, const void* value, int64_t n, int elem_bytes) {
  if (n == 0) return;
  const dim3 grid(static_cast<unsigned>(blocks_for(n)));
  switch (elem_bytes) {
    case 1: hipLaunchKernelGGL(fill_kernel<uint8_t>, grid, dim3(256), 0, s, (uint8_t*)dst, (const uint8_t*)value, n); break;
    case 2: hipLaunchKernelGGL(fill_kernel<uint16_t>, grid, dim3(256), 0, s, (uint16_t*)dst, (const uint16_t*)value, n); break;
    case 4: hipLaunchKernelGGL(fill_kernel<uint32_t>, grid, dim3(256), 0, s, (uint32_t*)dst, (const uint32_t*)value, n); break;
    case 8: hipLaunchKernelGGL(fill_kernel<uint64_t>, grid, dim3(256), 0, s, (uint64_t*)dst, (const uint64_t*)value, n); break;
    default: fail(Code::kInternal, "fill: bad element size");
  }
  check_launch("fill");
}

void launch_zero(hipStream_t s, void* dst, int64_t bytes) {
  if (bytes == 0) return;
  hipLaunchKernelGGL(zero_bytes_kernel, dim3(static_cast<unsigned>(blocks_for(bytes))), dim3(256), 0, s,
                     (uint8_t*)dst, bytes);
  check_launch("zero");
}

void launch_add(hipStream_t s, const void* a, const void* y, void* out, int64_t n, DType t) {
  if (n == 0) return;
  const int kind = t == DType::kF32 ? 2 : (t == DType::kF16 ? 1 : 0);
  PJRTX_CHECK(t == DType::kF32 || t == DType::kF16 || t == DType::kBF16, Code::kInternal, "add: element type");
  hipLaunchKernelGGL(add_kernel, dim3(static_cast<unsigned>(blocks_for(n))), dim3(256), 0, s, a, y, out, n, kind);
  check_launch("add");
}

void launch_gather(hipStream_t s, const GatherParams& g, const void* operand, const void* indices, void* out,
                   int elem_bytes) {
  GatherUnits p;
  p.g = g;
  int64_t total = 1;
  for (int d = 0; d < g.out_rank; ++d) total *= g.out_dims[d];
  if (total == 0) return;
  // Whole rows of a row-major operand selected by one index per output row.
  {
    const int nwin = g.op_rank - 1;
    const int nbatch = g.out_rank - nwin;
    bool rows = g.op_rank >= 1 && g.n_index == 1 && g.start_map[0] == 0 && g.n_batching == 0 && g.slice[0] == 1 &&
                nbatch >= 0 && (g.ivd == g.idx_rank || g.ivd == g.idx_rank - 1);
    for (int d = 1; d < g.op_rank && rows; ++d) rows = g.slice[d] == g.op_dims[d] && g.out_map[nbatch + d - 1] == -d - 1;
    for (int d = 0; d < nbatch && rows; ++d) rows = g.out_map[d] == d && d != g.ivd;
    int64_t row_elems = 1;
    for (int d = 1; d < g.op_rank; ++d) row_elems *= g.op_dims[d];
    rows = rows && (row_elems * elem_bytes) % 16 == 0 && reinterpret_cast<uintptr_t>(operand) % 16 == 0 &&
           reinterpret_cast<uintptr_t>(out) % 16 == 0;
    if (rows) {
      const int64_t upr = row_elems * elem_bytes / 16;
      const int64_t out_rows = total / row_elems;
      const int64_t nchunks = (upr + kGatherRowChunk - 1) / kGatherRowChunk;
      PJRTX_CHECK(out_rows * nchunks < (int64_t(1) << 31), Code::kUnimplemented, "gather: too many rows");
      hipLaunchKernelGGL(gather_rows_kernel, dim3(static_cast<unsigned>(out_rows * nchunks)), dim3(256), 0, s,
                         static_cast<const u32x4*>(operand), indices, g.idx_bytes, g.idx_signed, g.wrap, g.op_dims[0], upr,
                         nchunks, static_cast<u32x4*>(out));
      check_launch("gather_rows");
      return;
    }
  }
  p.unit_elems = 1;
  p.vector_inner = 0;
  // Rows of the operand's innermost dim copied whole: 16-byte units.
  const int r = g.out_rank;
  if (r > 0 && g.out_map[r - 1] == -(g.op_rank - 1) - 1 && g.op_stride[g.op_rank - 1] == 1 &&
      g.slice[g.op_rank - 1] == g.op_dims[g.op_rank - 1] && elem_bytes < 16) {
    const int64_t per = 16 / elem_bytes;
    bool ok = g.out_dims[r - 1] % per == 0 && reinterpret_cast<uintptr_t>(operand) % 16 == 0 &&
              reinterpret_cast<uintptr_t>(out) % 16 == 0;
    for (int d = 0; d + 1 < g.op_rank && ok; ++d) ok = g.op_stride[d] % per == 0;
    if (ok) {
      p.unit_elems = per;
      p.vector_inner = 1;
    }
  }
  p.total = total / p.unit_elems;
  const dim3 grid(static_cast<unsigned>(blocks_for(p.total)));
  if (p.unit_elems > 1) {
    hipLaunchKernelGGL(gather_kernel<u32x4>, grid, dim3(256), 0, s, p, (const u32x4*)operand, indices, (u32x4*)out);
  } else {
    switch (elem_bytes) {
      case 1: hipLaunchKernelGGL(gather_kernel<uint8_t>, grid, dim3(256), 0, s, p, (const uint8_t*)operand, indices, (uint8_t*)out); break;
      case 2: hipLaunchKernelGGL(gather_kernel<uint16_t>, grid, dim3(256), 0, s, p, (const uint16_t*)operand, indices, (uint16_t*)out); break;
      case 4: hipLaunchKernelGGL(gather_kernel<uint32_t>, grid, dim3(256), 0, s, p, (const uint32_t*)operand, indices, (uint32_t*)out); break;
      case 8: hipLaunchKernelGGL(gather_kernel<uint64_t>, grid, dim3(256), 0, s, p, (const uint64_t*)operand, indices, (uint64_t*)out); break;
      default: fail(Code::kInternal, "gather: bad element size");
    }
  }
  check_launch("gather");
}

namespace {
__global__ void __launch_bounds__(256) copy_segments_kernel(CopySegments c) {
  const int seg = blockIdx.y;
  if (seg >= c.n) return;
  const int64_t nb = c.bytes[seg];
  const char* src = static_cast<const char*>(c.src[seg]);
  char* dst = static_cast<char*>(c.dst[seg]);
  const int64_t stride = (int64_t)gridDim.x * 256;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (reinterpret_cast<uintptr_t>(src) % 16 == 0 && reinterpret_cast<uintptr_t>(dst) % 16 == 0) {
    typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
    const int64_t n16 = nb / 16;
    for (int64_t i = t; i < n16; i += stride)
      reinterpret_cast<u32x4_t*>(dst)[i] = reinterpret_cast<const u32x4_t*>(src)[i];
    for (int64_t i = n16 * 16 + t; i < nb; i += stride) dst[i] = src[i];
  } else {
    for (int64_t i = t; i < nb; i += stride) dst[i] = src[i];
  }
}
}  // namespace

namespace {
// Records the XCD (hardware register XCC_ID) each workgroup runs on.
__global__ void __launch_bounds__(64) xcc_probe_kernel(uint32_t* __restrict__ out) {
  if (threadIdx.x == 0) {
    uint32_t x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    out[blockIdx.x] = x & 0xfu;
  }
}
}  // namespace

bool probe_xcd_round_robin(hipStream_t s) {
  constexpr int kProbeBlocks = 1024;
  uint32_t* d = nullptr;
  if (hipMalloc(&d, kProbeBlocks * sizeof(uint32_t)) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  hipLaunchKernelGGL(xcc_probe_kernel, dim3(kProbeBlocks), dim3(64), 0, s, d);
  std::vector<uint32_t> h(kProbeBlocks, 0xffffffffu);
  bool ok = hipGetLastError() == hipSuccess &&
            hipMemcpyAsync(h.data(), d, kProbeBlocks * sizeof(uint32_t), hipMemcpyDeviceToHost, s) == hipSuccess &&
            hipStreamSynchronize(s) == hipSuccess;
  (void)hipFree(d);
  (void)hipGetLastError();
  // Workgroups b and b % 8 must share an XCD (one XCD: trivially).
  for (int b = 0; ok && b < kProbeBlocks; ++b) ok = h[b] == h[b % 8];
  return ok;
}

void launch_copy_segments(hipStream_t s, const CopySegments& c) {
  if (c.n <= 0) return;
  int64_t mx = 0;
  for (int i = 0; i < c.n; ++i) mx = c.bytes[i] > mx ? c.bytes[i] : mx;
  if (mx == 0) return;
  const int64_t blocks = (mx / 16 + 255) / 256;
  const dim3 grid(static_cast<unsigned>(blocks < 1 ? 1 : (blocks > 1024 ? 1024 : blocks)), static_cast<unsigned>(c.n));
  hipLaunchKernelGGL(copy_segments_kernel, grid, dim3(256), 0, s, c);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) fail(Code::kInternal, strformat("copy_segments launch failed: %s", hipGetErrorString(e)));
}

}  // namespace pjrtx
