// Launchers of the fused attention kernels (kernels/attention.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.h"

namespace pjrtx {

// out[b, h, q, :] = softmax_k(s[q, k]) . V[b, h / (Hq / Hkv), k, :] with
// s[q, k] = scale * round?(Q[b, h, q, :] . K[b, h / (Hq / Hkv), k, :]) over
// the allowed keys: k < Skv and, when `causal`, k <= q_coef * q + offset
// (+ the integer scalar at `offset_ptr` when set). A row with no allowed key
// gives NaN (0 / 0), as the unfused softmax does. The head dimension is
// contiguous; the other strides are in elements, per tensor.
struct AttnParams {
  int B = 1, Hq = 1, Hkv = 1, Sq = 0, Skv = 0, D = 0;
  int64_t q_b = 0, q_h = 0, q_s = 0;
  int64_t k_b = 0, k_h = 0, k_s = 0;
  int64_t v_b = 0, v_h = 0, v_s = 0;
  int64_t o_b = 0, o_h = 0, o_s = 0;
  float scale = 1.f;
  int causal = 0;
  int q_coef = 1;
  int64_t offset = 0;
  const void* offset_ptr = nullptr;  // device integer scalar added to offset
  int offset_bytes = 4;
  int offset_signed = 1;
  int offset_as_s32 = 0;  // truncate the operand to int32 first (the custom call casts it)
  // Round q.k to the input element type before scaling (the unfused graph's
  // dot_general returns the input type).
  int round_scores = 0;
};

// True when the MFMA tile kernel takes the problem (16-bit types, head dim
// 64 or 128, 16-byte aligned rows, Sq >= 16, scale > 0).
bool attention_uses_tiles(const AttnParams& p, DType t);

// Kernel choice: MFMA tiles; the split-key decode kernel (head dim a
// power-of-two count of 16-byte chunks from 4 to 32, aligned rows); or the
// generic row kernel.
enum class AttnPath { kTiles, kDecode, kRows };
AttnPath attention_path(const AttnParams& p, DType t, int* nsplit, int* keys_per_split);
// Device scratch the launch needs (split-key partials), 0 if none.
size_t attention_scratch_bytes(const AttnParams& p, DType t);
// Launches the kernels for element type t (bf16, f16 or f32; Q, K, V and out
// share it). `scratch` holds attention_scratch_bytes(p, t) bytes. The split
// decode kernel merges its splits in the same launch when `xcd_local` (the
// device runs workgroup b on XCD b % 8) and `counters` (arrival counters, one
// per 128 bytes, zero on entry and left zero) covers the query rows (at most
// kAttnCounterRows); otherwise a second kernel merges them.
//
// `partials_out` (split decode path only, attention_scratch_bytes > 0): `out`
// receives the split partials instead of the output rows, as floats [row]
// [split][m, l, D unnormalized outputs] with l = -1 for a split past the
// row's last allowed key, for a reader that merges them itself (a decode
// GEMV whose input is this output); `scratch` is not used.
constexpr int64_t kAttnCounterRows = 8192;
void launch_attention(hipStream_t s, const AttnParams& p, DType t, const void* Q, const void* K, const void* V,
                      void* out, float* scratch, uint32_t* counters, bool xcd_local, bool partials_out = false);

}  // namespace pjrtx
