// stablehlo.reduce_window: one thread per output element folds its window in
// row-major window order, starting from the init value, with padding
// positions contributing the init value (StableHLO's padded-input
// definition). Float windows fold sequentially in that order, the order a
// sequential CPU evaluation uses, so f32 sums equal it bit for bit; 16-bit
// floats accumulate in f32 and round once.
//
// Replaces the reference's pjrtx_mlx_metal_buffer_reduce_window
// (reference: src/backend/mlx_metal/api.cc:4324-4437: sum or max over a
// strided window view of the padded input, base dilation 1).
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

template <typename T>
__global__ void __launch_bounds__(256) reduce_window_kernel(ReduceWindowParams p, const T* __restrict__ in,
                                                            const T* __restrict__ init, T* __restrict__ out,
                                                            int64_t n_out, int64_t n_win) {
  typedef typename Acc<T>::type A;
  const int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (o >= n_out) return;
  int64_t oc[kReduceWindowMaxRank];
  {
    int64_t r = o;
    for (int d = p.rank - 1; d >= 0; --d) {
      oc[d] = r % p.out_dims[d];
      r /= p.out_dims[d];
    }
  }
  const A iv = Acc<T>::in(init[0]);
  A acc = iv;
  for (int64_t w = 0; w < n_win; ++w) {
    int64_t r = w, lin = 0;
    bool inside = true;
    int64_t wc[kReduceWindowMaxRank];
    for (int d = p.rank - 1; d >= 0; --d) {
      wc[d] = r % p.window[d];
      r /= p.window[d];
    }
    for (int d = 0; d < p.rank; ++d) {
      const int64_t c = oc[d] * p.stride[d] + wc[d] * p.dilation[d] - p.pad_low[d];
      inside &= c >= 0 && c < p.in_dims[d];
      lin = lin * p.in_dims[d] + c;
    }
    acc = fold<A>(p.op, acc, inside ? Acc<T>::in(in[lin]) : iv);
  }
  out[o] = Acc<T>::out(acc);
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

}  // namespace pjrtx
