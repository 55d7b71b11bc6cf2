// Windowed reductions (stablehlo.reduce_window) on the GPU.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.h"

namespace pjrtx {

constexpr int kReduceWindowMaxRank = 8;

// out[o] = init (+) in[window of o] in row-major window order. Window
// position w of output o is at coordinate c = o * stride + w * dilation -
// pad_low of the padded, base-dilated input (StableHLO: the input with
// base_dilation - 1 holes between neighbours, then padded; pad_low may be
// negative); c reads input element c / base_dilation when c is a multiple
// of base_dilation inside the dilated input, and contributes `init`
// otherwise (padding and holes). (+) is the reducer `op`: 0 sum, 1 product,
// 2 max, 3 min; 4 argmax and 5 argmin for the two-operand (value, index)
// form.
struct ReduceWindowParams {
  int rank = 0;
  int op = 0;
  int64_t in_dims[kReduceWindowMaxRank] = {};
  int64_t out_dims[kReduceWindowMaxRank] = {};
  int64_t window[kReduceWindowMaxRank] = {};
  int64_t stride[kReduceWindowMaxRank] = {};
  int64_t dilation[kReduceWindowMaxRank] = {};
  int64_t base_dilation[kReduceWindowMaxRank] = {};
  int64_t pad_low[kReduceWindowMaxRank] = {};
};

// `init` is a device scalar of the element type. Element types: f32, f64,
// bf16, f16 (16-bit floats accumulate in f32, rounded once at the end), s32,
// s64.
void launch_reduce_window(hipStream_t s, const ReduceWindowParams& p, DType t, const void* in, const void* init,
                          void* out);

// Two-operand windows over (values, indices) with the argmax (op 4) or
// argmin (op 5) pair rule of jnp.argmax: a NaN value wins (the lowest index
// among NaNs), then the larger (argmin: smaller) value, ties to the lower
// index; the winner's own value bits and index are written. Padding and
// holes contribute (init_value, init_index). Values f32, f64, bf16, f16;
// indices s32, u32, s64.
void launch_reduce_window_arg(hipStream_t s, const ReduceWindowParams& p, DType vt, DType it, const void* values,
                              const void* indices, const void* init_value, const void* init_index, void* out_values,
                              void* out_indices);

}  // namespace pjrtx
