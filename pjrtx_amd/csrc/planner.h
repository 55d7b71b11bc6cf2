// Fusion planner: Program -> Plan (an ordered list of steps, one GPU kernel
// launch or library call per step, with liveness releases).
//
// Replaces the reference's backend program model and fusion planner
// (reference: src/backend/mlx_metal/program.zig:21-286 Program/Node/
// FusionGroup/ScheduleItem, program_build.zig:10-207,224-263,
// program_fusion.zig:8-70, program_schedule_build.zig:6-51,
// program_liveness.zig:10, program_validation.zig:11) and its per-group
// lowering (executable_metal_graph_lowering.zig:177-424). Where the reference
// only groups contiguous view/elementwise runs and materializes every
// reduction input, this planner also fuses:
//   * the elementwise/view prologue of a reduction into the reduction kernel,
//   * sibling reductions over the same operand shape (multi-output),
//   * elementwise epilogues on a reduction's output (e.g. f32->f16 convert),
//   * the iota index operand of a two-output argmax (synthesized, not read),
//   * splat constants as literals (never materialized).
#pragma once

#include <map>
#include <set>
#include <string>
#include <vector>

#include "ir.h"

namespace pjrtx {

enum class ReducerKind { kSum, kProd, kMax, kMin, kAnd, kOr, kArgMax, kArgMin };
const char* reducer_name(ReducerKind k);

// Classifies a reduce region (reference: stablehlo_operation_attrs.zig:222-245
// reduceKindFromRegion). Two-result regions with compare+select become
// argmax/argmin with JAX's comparator semantics; unknown regions fail closed.
ReducerKind classify_reducer(const Program& prog, const Op& reduce_op);

struct ReduceSpec {
  int op_index = -1;
  ReducerKind kind = ReducerKind::kSum;
  std::vector<int> inputs;   // reduced operands (argmax: values, indices)
  std::vector<int> inits;    // init values
  std::vector<int> results;  // result values
};

// kRowFused: a chain of row reductions over the same trailing dims plus the
// elementwise pass that consumes them, as one kernel with one workgroup per
// row (softmax, RMSNorm, layer norm). `phases` holds the fused steps in
// order; earlier phases' results are per-row scalars in later phases.
//
// kGemv: decode-shaped dot_generals ([M, K] x [K, N_i], M <= 4, 16-bit)
// sharing one LHS, as one generated kernel that streams each weight once,
// split over K with the partials folded by the last workgroup of each
// column segment. It may absorb the row-fused step that produces its LHS
// (e.g. RMSNorm: recomputed per workgroup into LDS) and one elementwise
// loop step over its results (e.g. SwiGLU, RoPE with the KV-row writes),
// evaluated segment by segment by those last workgroups.
enum class StepKind { kLoop, kReduce, kAlias, kLibrary, kRowFused, kGemv };

enum class LibKind {
  kCopy, kDot, kGather, kScatter, kDynamicSlice, kDynamicUpdateSlice, kConcatenate, kPad, kAttention, kDotGroup, kWhile, kSort,
  kReduceWindow
};
const char* lib_kind_name(LibKind k);

struct Step;

// Geometry and members of a kGemv step.
struct GemvSpec {
  int x = -1;               // LHS value [M, K]
  int M = 1;
  int64_t K = 0;
  std::vector<int> dots;    // member dot_general ops
  std::vector<int> result;  // per member: value holding its final value
  std::vector<int> add;     // per member: residual addend (result = add + round(dot)) or -1
  std::vector<bool> store;  // per member: the result is written to memory
  int cols = 64;            // columns per tile (8 lanes of 8 elements per row at 64)
  int depth = 4;            // weight rows in flight per lane
  int64_t ksplit = 1;       // K chunks (workgroups per tile)
  int64_t kchunk = 0;       // rows per K chunk
  // Segments: the unit whose last workgroup folds the partials. Joint
  // segments span the same `seg_cols` columns of every member (an epilogue
  // reads several members); otherwise a segment is one tile of one member.
  bool joint = false;
  int64_t seg_cols = 0, nseg = 0, wps = 0;  // wps: workgroups per segment
  int64_t root_per_seg = 0;                 // epilogue loop elements per segment
  bool direct = false;                      // ksplit 1, no epilogue: tiles store their results
  size_t partial_bytes = 0;                 // partial slots before the counters in scratch
  int64_t wgs = 0;                          // workgroups launched (8 per XCD round)
  bool stage_all_x = false;                 // whole X in LDS (else each workgroup's one chunk)
  bool weights_nt = true;                   // weights read with non-temporal loads
  // x is a split decode attention's partials output (M == 1, one query
  // row per head): element k is head k / attn_dim, column k % attn_dim,
  // merged over attn_splits splits while X is staged. 0: x is read as is.
  int attn_splits = 0;
  int attn_dim = 0;
};

struct Step {
  StepKind kind = StepKind::kLoop;
  std::string name;          // generated kernel symbol
  std::vector<int> ops;      // fused program ops (prologue/body), topological
  std::vector<int> inputs;   // materialized values read
  std::vector<int> outputs;  // materialized values written

  // kLoop
  Dims loop_shape;
  int vec = 1;

  // kReduce
  std::vector<ReduceSpec> reduces;
  std::vector<int> epilogue_ops;
  Dims reduce_operand_shape;
  Dims reduce_dims;          // sorted
  bool row_schedule = true;  // reduced dims are the trailing dims
  int64_t rows = 1;          // row schedule: product of kept dims
  int64_t row_len = 1;       // row schedule: product of reduced dims
  int64_t splits = 1;        // workgroups per row
  int64_t chunk = 0;         // elements per split
  int unroll = 1;            // 256*vec-element sub-chunks loaded together per thread
  size_t scratch_bytes = 0;  // partial accumulators (splits > 1)
  uint32_t combine_grid = 0; // splits > 1: workgroups of `<name>_combine` (4 rows each)
  // splits > 1 and no combine launch: the last workgroup of a row to finish
  // folds the row's partials (per-row arrival counters after the slots).
  bool fused_combine = false;
  size_t counter_offset = 0; // fused_combine: byte offset of the counters in scratch

  // kLibrary / kAlias
  LibKind lib = LibKind::kCopy;
  int lib_op = -1;
  // dynamic_update_slice whose operand dies here: the update is written into
  // the operand's buffer, which becomes the result (no copy).
  bool in_place = false;
  // kAttention on the split decode path whose only reader is a kGemv that
  // merges the splits: the output buffer holds the split partials
  // (attention_partials_bytes), not the output rows.
  bool attn_partials = false;

  // launch geometry of generated kernels
  uint32_t grid = 1;
  uint32_t block = 256;

  std::vector<int> release_after;  // intermediate values dead after this step

  // kRowFused
  std::vector<Step> phases;
  bool wave_per_row = false;  // one wave per row (4 rows per workgroup), else one workgroup per row

  // kDotGroup: the dot_general ops (program order) sharing one LHS
  std::vector<int> group_ops;
  // kDot: value added to the rounded product (a residual add merged into the
  // dot); the step's output is then the sum, not the dot's own result.
  int dot_add = -1;
  // kWhile: the iteration count when constants fix it (a counter from a
  // constant start, compared with a constant bound, advanced by a constant
  // step), else -1 (the predicate is read every iteration).
  int64_t while_trips = -1;

  // kLoop: outputs that are dynamic_update_slice results written in place.
  // Output `outputs[k]` shares the buffer of `operand`; the kernel stores
  // the update (the value `update`, computed in the kernel or read from
  // `update` when it is one of the step's inputs) into the window at the
  // clamped `starts` (scalar values; steps' inputs unless splat constants).
  struct WindowWrite {
    int operand = -1;
    int update = -1;
    std::vector<int> starts;
  };
  std::map<int, WindowWrite> window_out;  // output position -> window write

  // kGemv
  GemvSpec gemv;
  std::vector<Step> prologue;       // 0 or 1 kRowFused step producing gemv.x
  std::vector<Step> epilogue_loop;  // 0 or 1 kLoop step over member results
};

struct Plan {
  std::vector<Step> steps;
  std::set<int> materialized;
  std::vector<int> constants;        // materialized non-splat constant values
  // Entry parameter positions whose buffer a step writes in place (donated
  // arguments only). The runtime copies such an argument first when the
  // caller does not donate it.
  std::vector<int> written_params;
  std::map<int, int> producer;       // value -> op index
  std::string kernel_source;         // hiprtc source for all generated steps
  int64_t nt_min_bytes = 0;          // PlanOptions::nt_min_bytes
  int num_fusion_kernels = 0;
  std::string describe(const Program& prog) const;  // JSON summary
};

struct PlanOptions {
  // Multi-use elementwise values are recomputed in each consumer while their
  // inlined cost stays at or below this many ops.
  int recompute_limit = 24;
  // Target number of workgroups a reduction launch should reach.
  // (environment: PJRTX_REDUCE_TARGET_BLOCKS)
  int64_t reduce_target_blocks = env_int("PJRTX_REDUCE_TARGET_BLOCKS", 512);
  // Threads per workgroup of the row-schedule reduce kernels (256, 512 or
  // 1024).
  int reduce_block = env_int("PJRTX_REDUCE_BLOCK", 256);
  // Split reductions fold their partials in the last workgroup of each row
  // instead of a second launch (environment: PJRTX_REDUCE_FUSED_COMBINE,
  // default 1). The fold needs no device-scope fence: every split of a row
  // runs on one XCD (when the device places workgroups round-robin over the
  // XCDs; otherwise the runtime launches the `_combine` kernel instead).
  bool reduce_fused_combine = env_int("PJRTX_REDUCE_FUSED_COMBINE", 1) != 0;
  // Inputs of reduce kernels of at least this many bytes are read with
  // non-temporal loads (environment: PJRTX_NT_MIN_BYTES; 0 never). C2's
  // 16 MB logits stay below it (non-temporal: 5.06 -> 5.11 us).
  int64_t nt_min_bytes = env_int("PJRTX_NT_MIN_BYTES", 32 << 20);
  bool fuse_siblings = true;
  bool fuse_epilogues = true;
  // Row chains (reduce -> reduce/loop over the same rows) become one kernel
  // when a row has at most this many elements (environment:
  // PJRTX_ROW_FUSE_MAX, 0 disables).
  int64_t row_fuse_max = env_int("PJRTX_ROW_FUSE_MAX", 16384);
  // Decode-shaped dots that share their LHS (Q/K/V, gate/up projections)
  // become one step (environment: PJRTX_DOT_GROUPS, 0 disables).
  bool group_dots = env_int("PJRTX_DOT_GROUPS", 1) != 0;
  // A decode-shaped dot whose only reader is `add(dot, x)` writes the sum
  // itself (environment: PJRTX_DOT_RESIDUAL, 0 disables).
  bool dot_residual = env_int("PJRTX_DOT_RESIDUAL", 1) != 0;
  // Decode-shaped dots become generated split-K GEMV kernels with fused
  // prologues and epilogues (environment: PJRTX_GEMV_FUSION, 0 keeps the
  // library GEMV steps).
  bool gemv_fusion = env_int("PJRTX_GEMV_FUSION", 1) != 0;
  // Target workgroups per GEMV launch (environment: PJRTX_GEMV_WGS).
  int64_t gemv_target_wgs = env_int("PJRTX_GEMV_WGS", 768);
  // GEMV weights read with plain loads, smallest first, up to this many MB
  // per program; the rest use non-temporal loads (environment:
  // PJRTX_GEMV_MALL_MB). Plain-loaded weights may stay in the memory-side
  // cache (MALL, 256 MB) from one execute to the next. C5 decode, tokens/s:
  // 0 MB 2581, 64 MB 2594, 100 MB 2598, 160 MB 2553, 200 MB 2545.
  int64_t gemv_mall_mb = env_int("PJRTX_GEMV_MALL_MB", 96);
  // A decode GEMV whose input is a split decode attention's output merges
  // the attention's splits itself while staging its input, so the attention
  // launch ends after its partial stores (environment:
  // PJRTX_ATTN_MERGE_GEMV, 0 keeps the merge in the attention launch).
  bool attn_merge_in_gemv = env_int("PJRTX_ATTN_MERGE_GEMV", 1) != 0;
};

Plan make_plan(const Program& prog, const PlanOptions& opts = PlanOptions());

// Program rewrites before planning (attention.cc): lowers supported
// custom calls, fuses the softmax-attention pattern into one kAttention op
// (unless PJRTX_FUSED_ATTENTION=0) and drops ops left without users.
// Unsupported custom-call targets fail with kUnimplemented.
void rewrite_program(Program* prog);

// Folds JAX's negative-index normalization of gather indices into the
// gathers (library.cc); true when a gather changed.
bool fold_gather_index_wrap(Program* prog);

// Turns decode-shaped dot and dot-group library steps into kGemv steps and
// absorbs their row-fused prologues and elementwise epilogues
// (gemv_fusion.cc). Runs on a finished plan (after liveness); recomputes the
// releases. `outputs` are the program's result values.
void fuse_gemv_steps(const Program& prog, Plan* plan, const std::set<int>& outputs, const PlanOptions& opts);

// Bytes of the split partials a kAttention op writes on the split decode
// path (0 on the other paths) (attention.cc).
size_t attention_partials_bytes(const Program& prog, const Op& op);

// Emits the HIP source of every generated step (codegen.cc).
std::string generate_kernels(const Program& prog, Plan& plan);

}  // namespace pjrtx
