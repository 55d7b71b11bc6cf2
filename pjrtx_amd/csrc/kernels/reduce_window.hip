// stablehlo.reduce_window: one thread per output element folds its window in
// row-major window order, starting from the init value, with padding
// positions and base-dilation holes contributing the init value (StableHLO's
// padded, dilated-input definition). Float windows fold sequentially in
// that order, the order a sequential CPU evaluation uses, so f32 sums equal
// it bit for bit; 16-bit floats accumulate in f32 and round once. The
// two-operand (value, index) form folds with the argmax / argmin pair rule,
// a selection, so its result does not depend on the order.
//
// Replaces the reference's pjrtx_mlx_metal_buffer_reduce_window
// (reference: src/backend/mlx_metal/api.cc:4324-4435: sum or max over a
// strided window view of the padded input, base dilation 1) and
// pjrtx_mlx_metal_buffer_reduce_window_max_with_indices (api.cc:4437-4620:
// the (max, index) pair of each window, found there by an argsort of the
// window's values).
#include <hip/hip_runtime.h>

#include <cmath>
#include <type_traits>

#include "common.h"
#include "kernels/reduce_window.h"

namespace pjrtx {
namespace {

template <typename T>
struct Acc {
  typedef T type;
  static __device__ T in(T v) { return v; }
  static __device__ T out(T v) { return v; }
};
template <>
struct Acc<__bf16> {
  typedef float type;
  static __device__ float in(__bf16 v) { return (float)v; }
  static __device__ __bf16 out(float v) { return (__bf16)v; }
};
template <>
struct Acc<_Float16> {
  typedef float type;
  static __device__ float in(_Float16 v) { return (float)v; }
  static __device__ _Float16 out(float v) { return (_Float16)v; }
};

// max / min propagate NaN (stablehlo.maximum / minimum).
template <typename A>
__device__ __forceinline__ A fold(int op, A a, A b) {
  if constexpr (std::is_floating_point_v<A>) {
    if (op == 2) return (a != a || b != b) ? (a != a ? a : b) : (a > b ? a : b);
    if (op == 3) return (a != a || b != b) ? (a != a ? a : b) : (a < b ? a : b);
  } else {
    if (op == 2) return a > b ? a : b;
    if (op == 3) return a < b ? a : b;
  }
  if constexpr (std::is_integral_v<A>) {  // two's-complement wraparound
    typedef std::make_unsigned_t<A> U;
    return (A)(op == 1 ? (U)a * (U)b : (U)a + (U)b);
  } else {
    return op == 1 ? a * b : a + b;
  }
}

// Output o's coordinates.
__device__ __forceinline__ void out_coords(const ReduceWindowParams& p, int64_t o, int64_t* oc) {
  for (int d = p.rank - 1; d >= 0; --d) {
    oc[d] = o % p.out_dims[d];
    o /= p.out_dims[d];
  }
}

// Input element read by window position w of the output at oc, or -1 for a
// padding position or a base-dilation hole.
__device__ __forceinline__ int64_t window_source(const ReduceWindowParams& p, const int64_t* oc, int64_t w) {
  int64_t wc[kReduceWindowMaxRank];
  for (int d = p.rank - 1; d >= 0; --d) {
    wc[d] = w % p.window[d];
    w /= p.window[d];
  }
  int64_t lin = 0;
  bool inside = true;
  for (int d = 0; d < p.rank; ++d) {
    const int64_t c = oc[d] * p.stride[d] + wc[d] * p.dilation[d] - p.pad_low[d];
    const int64_t b = p.base_dilation[d];
    const int64_t q = c >= 0 ? c / b : -1;
    inside &= c >= 0 && q * b == c && q < p.in_dims[d];
    lin = lin * p.in_dims[d] + (q >= 0 ? q : 0);
  }
  return inside ? lin : -1;
}

template <typename T>
__global__ void __launch_bounds__(256) reduce_window_kernel(ReduceWindowParams p, const T* __restrict__ in,
                                                            const T* __restrict__ init, T* __restrict__ out,
                                                            int64_t n_out, int64_t n_win) {
  typedef typename Acc<T>::type A;
  const int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (o >= n_out) return;
  int64_t oc[kReduceWindowMaxRank];
  out_coords(p, o, oc);
  const A iv = Acc<T>::in(init[0]);
  A acc = iv;
  for (int64_t w = 0; w < n_win; ++w) {
    const int64_t src = window_source(p, oc, w);
    acc = fold<A>(p.op, acc, src >= 0 ? Acc<T>::in(in[src]) : iv);
  }
  out[o] = Acc<T>::out(acc);
}

// (value, index) candidate x replaces the running pair a under the argmax
// (kMax) or argmin rule: NaN first, then the larger (smaller) value, ties to
// the lower index. Values compare as floats (so -0 == +0).
template <bool kMax, typename A, typename I>
__device__ __forceinline__ bool arg_takes(A xv, I xi, A av, I ai) {
  const bool xn = xv != xv, an = av != av;
  if (xn || an) return xn && (!an || xi < ai);
  if (xv == av) return xi < ai;
  return kMax ? xv > av : xv < av;
}

template <typename T, typename I, bool kMax>
__global__ void __launch_bounds__(256) reduce_window_arg_kernel(ReduceWindowParams p, const T* __restrict__ vals,
                                                                const I* __restrict__ idx, const T* __restrict__ init_v,
                                                                const I* __restrict__ init_i, T* __restrict__ out_v,
                                                                I* __restrict__ out_i, int64_t n_out, int64_t n_win) {
  typedef typename Acc<T>::type A;
  const int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (o >= n_out) return;
  int64_t oc[kReduceWindowMaxRank];
  out_coords(p, o, oc);
  const T ivb = init_v[0];
  const I ii = init_i[0];
  T bv = ivb;  // the winner's own bits
  A av = Acc<T>::in(ivb);
  I ai = ii;
  for (int64_t w = 0; w < n_win; ++w) {
    const int64_t src = window_source(p, oc, w);
    const T xb = src >= 0 ? vals[src] : ivb;
    const I xi = src >= 0 ? idx[src] : ii;
    const A xv = Acc<T>::in(xb);
    if (arg_takes<kMax>(xv, xi, av, ai)) {
      bv = xb;
      av = xv;
      ai = xi;
    }
  }
  out_v[o] = bv;
  out_i[o] = ai;
}

template <typename T, typename I>
void launch_arg_typed(hipStream_t s, const ReduceWindowParams& p, const void* v, const void* i, const void* iv,
                      const void* ii, void* ov, void* oi, int64_t n_out, int64_t n_win) {
  const dim3 grid(static_cast<uint32_t>((n_out + 255) / 256)), block(256);
  if (p.op == 4)
    hipLaunchKernelGGL((reduce_window_arg_kernel<T, I, true>), grid, block, 0, s, p, (const T*)v, (const I*)i,
                       (const T*)iv, (const I*)ii, (T*)ov, (I*)oi, n_out, n_win);
  else
    hipLaunchKernelGGL((reduce_window_arg_kernel<T, I, false>), grid, block, 0, s, p, (const T*)v, (const I*)i,
                       (const T*)iv, (const I*)ii, (T*)ov, (I*)oi, n_out, n_win);
}

template <typename T>
void launch_arg_index(hipStream_t s, const ReduceWindowParams& p, DType it, const void* v, const void* i,
                      const void* iv, const void* ii, void* ov, void* oi, int64_t n_out, int64_t n_win) {
  switch (it) {
    case DType::kS32: launch_arg_typed<T, int32_t>(s, p, v, i, iv, ii, ov, oi, n_out, n_win); break;
    case DType::kU32: launch_arg_typed<T, uint32_t>(s, p, v, i, iv, ii, ov, oi, n_out, n_win); break;
    case DType::kS64: launch_arg_typed<T, int64_t>(s, p, v, i, iv, ii, ov, oi, n_out, n_win); break;
    default:
      fail(Code::kUnimplemented, std::string("reduce_window: index type ") + dtype_name(it) + " is not supported");
  }
}

}  // namespace

void launch_reduce_window(hipStream_t s, const ReduceWindowParams& p, DType t, const void* in, const void* init,
                          void* out) {
  PJRTX_CHECK(p.rank >= 1 && p.rank <= kReduceWindowMaxRank, Code::kUnimplemented, "reduce_window: rank 1..8");
  int64_t n_out = 1, n_win = 1;
  for (int d = 0; d < p.rank; ++d) {
    n_out *= p.out_dims[d];
    n_win *= p.window[d];
  }
  if (n_out == 0) return;
  const dim3 grid(static_cast<uint32_t>((n_out + 255) / 256)), block(256);
  switch (t) {
    case DType::kF32:
      hipLaunchKernelGGL(reduce_window_kernel<float>, grid, block, 0, s, p, (const float*)in, (const float*)init,
                         (float*)out, n_out, n_win);
      break;
    case DType::kF64:
      hipLaunchKernelGGL(reduce_window_kernel<double>, grid, block, 0, s, p, (const double*)in, (const double*)init,
                         (double*)out, n_out, n_win);
      break;
    case DType::kBF16:
      hipLaunchKernelGGL(reduce_window_kernel<__bf16>, grid, block, 0, s, p, (const __bf16*)in, (const __bf16*)init,
                         (__bf16*)out, n_out, n_win);
      break;
    case DType::kF16:
      hipLaunchKernelGGL(reduce_window_kernel<_Float16>, grid, block, 0, s, p, (const _Float16*)in,
                         (const _Float16*)init, (_Float16*)out, n_out, n_win);
      break;
    case DType::kS32:
      hipLaunchKernelGGL(reduce_window_kernel<int32_t>, grid, block, 0, s, p, (const int32_t*)in, (const int32_t*)init,
                         (int32_t*)out, n_out, n_win);
      break;
    case DType::kS64:
      hipLaunchKernelGGL(reduce_window_kernel<int64_t>, grid, block, 0, s, p, (const int64_t*)in, (const int64_t*)init,
                         (int64_t*)out, n_out, n_win);
      break;
    default:
      fail(Code::kUnimplemented, std::string("reduce_window: element type ") + dtype_name(t) + " is not supported");
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) fail(Code::kInternal, strformat("reduce_window launch failed: %s", hipGetErrorString(e)));
}

void launch_reduce_window_arg(hipStream_t s, const ReduceWindowParams& p, DType vt, DType it, const void* values,
                              const void* indices, const void* init_value, const void* init_index, void* out_values,
                              void* out_indices) {
  PJRTX_CHECK(p.rank >= 1 && p.rank <= kReduceWindowMaxRank, Code::kUnimplemented, "reduce_window: rank 1..8");
  PJRTX_CHECK(p.op == 4 || p.op == 5, Code::kInternal, "reduce_window: two-operand form needs argmax or argmin");
  int64_t n_out = 1, n_win = 1;
  for (int d = 0; d < p.rank; ++d) {
    n_out *= p.out_dims[d];
    n_win *= p.window[d];
  }
  if (n_out == 0) return;
  switch (vt) {
    case DType::kF32:
      launch_arg_index<float>(s, p, it, values, indices, init_value, init_index, out_values, out_indices, n_out, n_win);
      break;
    case DType::kF64:
      launch_arg_index<double>(s, p, it, values, indices, init_value, init_index, out_values, out_indices, n_out, n_win);
      break;
    case DType::kBF16:
      launch_arg_index<__bf16>(s, p, it, values, indices, init_value, init_index, out_values, out_indices, n_out, n_win);
      break;
    case DType::kF16:
      launch_arg_index<_Float16>(s, p, it, values, indices, init_value, init_index, out_values, out_indices, n_out,
                                 n_win);
      break;
    default:
      fail(Code::kUnimplemented, std::string("reduce_window: value type ") + dtype_name(vt) + " is not supported");
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) fail(Code::kInternal, strformat("reduce_window launch failed: %s", hipGetErrorString(e)));
}

}  // namespace pjrtx
