// Program IR produced by the StableHLO text importer and consumed by the
// fusion planner.
//
// It plays the role of the reference's ExecutablePlan / PlanInstruction /
// Value (reference: src/compiler/executable_plan.zig:9-140,
// src/compiler/plan_instruction.zig:10-93): SSA values with a tensor type, and
// instructions that carry the StableHLO attributes the backend needs
// (dimensions, reduce dimensions, dot / gather / scatter dimension numbers,
// comparison direction, literal bytes). Functions called with `call` are
// inlined at import, as the reference's MLIR inliner does
// (reference: src/compiler/mlir_session.zig:206-234).
#pragma once

#include <map>
#include <string>
#include <vector>

#include "common.h"

namespace pjrtx {

enum class OpKind {
  kParameter,  // function argument (not an instruction in the body)
  kConstant,
  // elementwise unary
  kAbs, kNegate, kExp, kExpm1, kLog, kLog1p, kLogistic, kSqrt, kRsqrt, kCbrt,
  kTanh, kSine, kCosine, kTan, kFloor, kCeil, kRoundAfz, kRoundEven, kSign,
  kNot, kIsFinite, kPopcnt, kClz, kConvert, kBitcastConvert,
  // rounds to `mantissa_bits` / clamps to `exponent_bits` in the same type
  kReducePrecision,
  // elementwise binary
  kAdd, kSubtract, kMultiply, kDivide, kRemainder, kPower, kMaximum, kMinimum,
  kAnd, kOr, kXor, kShiftLeft, kShiftRightArithmetic, kShiftRightLogical,
  kAtan2, kCompare,
  // elementwise ternary
  kSelect, kClamp,
  // index-remapping views
  kBroadcastInDim, kReshape, kTranspose, kSlice, kIota, kReverse,
  // materializing structural ops
  kConcatenate, kPad, kDynamicSlice, kDynamicUpdateSlice,
  // reductions and library ops
  kReduce, kDotGeneral, kGather, kScatter,
  // windowed reduction: regions[0] the reducer; window in `sizes`, strides in
  // `strides`, dilations in base_dilations / window_dilations, padding in
  // pad_low / pad_high
  kReduceWindow,
  // control flow: regions[0] = cond (state -> pred), regions[1] = body
  // (state -> state); operands = initial state, results = final state
  kWhile,
  // stablehlo.sort: operands sorted together along `dim` by the comparator
  // in regions[0]; chlo.top_k: the k largest along the last dim (k in
  // `sizes[0]`), results (values, s32 indices)
  kSort, kTopK,
  // stablehlo.custom_call (only known targets pass validation), and the
  // fused attention op that the program rewrite produces from a
  // scaled-dot-product-attention custom call or the unfused pattern.
  kCustomCall, kAttention,
  kReturn,
};

const char* op_kind_name(OpKind k);
bool op_is_elementwise(OpKind k);
bool op_is_view(OpKind k);  // broadcast/reshape/transpose/slice/iota/reverse

enum class CmpDir { kEQ, kNE, kLT, kLE, kGT, kGE };
enum class CmpType { kNotSet, kFloat, kTotalOrder, kSigned, kUnsigned };

// Nested computation of reduce / scatter (its own parameters, ops, return).
struct Region;

// kAttention: out = softmax_k(scale * round?(q.k) over allowed keys) . v per
// (batch, head, query). Operands (q, k, v[, offset scalar]). Allowed keys:
// k < kv_len and, when causal, k <= q_coef * q + offset (+ the offset
// operand when present).
struct AttentionAttrs {
  // Operand layouts: 0 = [B, H, S, D] (the unfused dot_general form),
  // 1 = [B, S, H, D], 2 = [S, H, D] (the custom call's rank 4 / rank 3).
  int layout = 0;
  double scale = 1.0;
  bool causal = false;
  int q_coef = 1;
  int64_t offset = 0;
  bool has_offset_operand = false;
  bool round_scores = false;
};

struct Op {
  OpKind kind = OpKind::kReturn;
  std::string name;              // "stablehlo.add"
  std::vector<int> operands;     // value ids
  std::vector<int> results;      // value ids

  // broadcast_in_dim dims, transpose permutation, reduce dimensions,
  // reverse dims
  Dims dims;
  int64_t dim = -1;  // iota / concatenate dimension
  CmpDir cmp_dir = CmpDir::kEQ;
  CmpType cmp_type = CmpType::kNotSet;

  // slice
  Dims start, limit, strides;
  // pad
  Dims pad_low, pad_high, pad_interior;
  // dynamic_slice sizes / gather slice_sizes
  Dims sizes;

  // reduce_precision
  int64_t exponent_bits = -1, mantissa_bits = -1;
  // reduce_window dilations
  Dims base_dilations, window_dilations;
  // dot_general dimension numbers
  Dims lhs_batch, rhs_batch, lhs_contract, rhs_contract;

  // gather dimension numbers
  Dims offset_dims, collapsed_slice_dims, start_index_map;
  Dims operand_batching_dims, start_indices_batching_dims;
  int64_t index_vector_dim = -1;
  // scatter dimension numbers
  Dims update_window_dims, inserted_window_dims, scatter_dims_to_operand_dims;
  Dims input_batching_dims, scatter_indices_batching_dims;
  bool indices_are_sorted = false;
  bool unique_indices = false;
  // gather: a negative start index i is read as i + index_wrap (in the
  // index type's width, wrapping) before the clamp: JAX's negative-index
  // normalization (select(i < 0, i + N, i)) folded into the gather by
  // fold_gather_index_wrap. 0: indices are read as they are.
  int64_t index_wrap = 0;

  // constant literal: raw little-endian element bytes of the result type,
  // or one element when `splat`.
  std::vector<uint8_t> literal;
  bool splat = false;

  // reduce / scatter body
  std::vector<Region> regions;

  // custom_call target name; kAttention attributes
  std::string target;
  AttentionAttrs attn;
};

struct Region {
  std::vector<int> params;   // value ids of block arguments
  std::vector<Op> ops;       // body ops, last is kReturn
};

struct Value {
  TensorType type;
  std::string name;  // SSA name in the source text, for diagnostics
};

// One function after inlining: the program entry.
struct Program {
  std::string module_name;
  std::vector<Value> values;     // indexed by value id
  std::vector<int> params;       // value ids of entry parameters
  std::vector<Op> ops;           // entry body, topologically ordered
  std::vector<int> results;      // value ids returned by the entry
  // Per entry parameter: the result index it is donated to
  // (`tf.aliasing_output = N`), -2 for a donor with no fixed result
  // (`jax.buffer_donor = true`), -1 when not donated.
  std::vector<int> param_alias;
  int num_partitions = 1;
  int num_replicas = 1;
  int64_t mesh_devices = 1;  // largest `sdy.mesh` declared (shardings are ignored)

  const TensorType& type(int v) const { return values.at(v).type; }
  std::string describe() const;  // one line per op, for diagnostics
};

// Parses MLIR text holding a StableHLO module (JAX's `lowered.as_text()`
// form: pretty-printed stablehlo ops, func.func / call / return). Inlines
// private functions into `@main`. Throws Error(kInvalidArgument) with a line
// number on malformed input and Error(kUnimplemented) for ops outside the
// supported set (fail closed, as reference lowering_rules.zig:106 does).
Program parse_stablehlo(const std::string& text);

// Host-side helpers for literals.
uint16_t f32_to_bf16_bits(float f);  // round to nearest even
uint16_t f32_to_f16_bits(float f);   // round to nearest even
float bf16_bits_to_f32(uint16_t b);
float f16_bits_to_f32(uint16_t h);

}  // namespace pjrtx
