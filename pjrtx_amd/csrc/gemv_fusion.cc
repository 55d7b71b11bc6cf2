// Decode GEMV fusion: decode-shaped dot_general steps (one LHS row block
// [M, K], M <= 4, times weights [K, N]) become generated kernels that
//   * stream each weight exactly once over many workgroups (split over K,
//     the partial sums folded in a fixed order by the last workgroup of each
//     column segment, so the result is deterministic);
//   * compute their LHS in the kernel when a row-fused step produces it
//     (RMSNorm: every workgroup recomputes the row's sum of squares and the
//     normalized row into LDS, which costs a 4 KB read instead of a launch);
//   * evaluate one elementwise loop step over their results in the same
//     launch (SwiGLU over the gate/up pair; RoPE of q and k with the KV-row
//     writes into the caches), segment by segment.
// The reference lowers the same chain as separate Metal dispatches of its
// dot group and elementwise fusions (reference:
// executable_metal_graph_lowering_fusion.zig:394-424 dot groups,
// metal_graph_dot.zig:70-152 the GEMV dispatch); here it is one launch.
#include <algorithm>
#include <functional>
#include <map>
#include <set>

#include "planner.h"
#include "kernels/attention.h"

namespace pjrtx {

AttnParams attention_params(const Program& prog, const Op& op);  // attention.cc

namespace {

std::map<int, int> producers_of(const std::vector<Step>& steps) {
  std::map<int, int> m;
  for (size_t i = 0; i < steps.size(); ++i)
    for (int v : steps[i].outputs) m[v] = static_cast<int>(i);
  return m;
}

std::vector<int64_t> unravel(int64_t lin, const Dims& shape) {
  std::vector<int64_t> idx(shape.size());
  for (int d = static_cast<int>(shape.size()) - 1; d >= 0; --d) {
    const int64_t D = std::max<int64_t>(shape[d], 1);
    idx[d] = lin % D;
    lin /= D;
  }
  return idx;
}

int64_t ravel(const std::vector<int64_t>& idx, const Dims& shape) {
  int64_t lin = 0;
  for (size_t d = 0; d < shape.size(); ++d) lin = lin * shape[d] + idx[d];
  return lin;
}

// Calls visit(value, linear index) for every element of a materialized value
// (one of `inputs`) that the generated code reads to evaluate value `v` at
// multi-index `idx`, following the fused ops the way the kernel writer does:
// views remap the index, elementwise ops read their operands at the same
// index (rank-0 operands at the scalar), and a concatenate reads every
// operand at its clamped coordinate. Returns false for an op the writer does
// not fuse (the caller then does not absorb the step).
class ReadTracer {
 public:
  ReadTracer(const Program& prog, const std::set<int>& inputs) : prog_(prog), inputs_(inputs) {
    for (size_t i = 0; i < prog.ops.size(); ++i)
      for (int r : prog.ops[i].results) producer_[r] = static_cast<int>(i);
  }

  bool trace(int v, const std::vector<int64_t>& idx, const std::function<void(int, int64_t)>& visit) {
    seen_.clear();
    return walk(v, idx, visit);
  }

 private:
  const Program& prog_;
  const std::set<int>& inputs_;
  std::map<int, int> producer_;
  std::set<std::pair<int, int64_t>> seen_;

  bool walk(int v, const std::vector<int64_t>& idx, const std::function<void(int, int64_t)>& visit) {
    const TensorType& t = prog_.type(v);
    const int64_t lin = ravel(idx, t.dims);
    if (!seen_.insert({v, lin}).second) return true;
    if (inputs_.count(v)) {
      visit(v, lin);
      return true;
    }
    auto p = producer_.find(v);
    if (p == producer_.end()) return false;
    const Op& op = prog_.ops[p->second];
    switch (op.kind) {
      case OpKind::kConstant:
      case OpKind::kIota:
        return true;
      case OpKind::kReshape: {
        const Dims& od = prog_.type(op.operands[0]).dims;
        return walk(op.operands[0], unravel(lin, od), visit);
      }
      case OpKind::kBroadcastInDim: {
        const Dims& od = prog_.type(op.operands[0]).dims;
        std::vector<int64_t> oi(od.size());
        for (size_t k = 0; k < od.size(); ++k) oi[k] = (od[k] == 1) ? 0 : idx[op.dims[k]];
        return walk(op.operands[0], oi, visit);
      }
      case OpKind::kTranspose: {
        const Dims& od = prog_.type(op.operands[0]).dims;
        std::vector<int64_t> oi(od.size());
        for (size_t k = 0; k < op.dims.size(); ++k) oi[op.dims[k]] = idx[k];
        return walk(op.operands[0], oi, visit);
      }
      case OpKind::kSlice: {
        std::vector<int64_t> oi(idx.size());
        for (size_t k = 0; k < idx.size(); ++k)
          oi[k] = op.start[k] + idx[k] * (op.strides.empty() ? 1 : op.strides[k]);
        return walk(op.operands[0], oi, visit);
      }
      case OpKind::kReverse: {
        const Dims& od = prog_.type(op.operands[0]).dims;
        std::vector<int64_t> oi = idx;
        for (int64_t d : op.dims) oi[d] = od[d] - 1 - idx[d];
        return walk(op.operands[0], oi, visit);
      }
      case OpKind::kConcatenate: {
        const int64_t cd = op.dim;
        int64_t off = 0;
        for (int u : op.operands) {
          const Dims& od = prog_.type(u).dims;
          const int64_t sz = od[cd];
          if (sz == 0) continue;
          std::vector<int64_t> oi = idx;
          const int64_t c = idx[cd] - off;
          oi[cd] = c < 0 ? 0 : (c > sz - 1 ? sz - 1 : c);
          if (!walk(u, oi, visit)) return false;
          off += sz;
        }
        return true;
      }
      default:
        break;
    }
    if (!op_is_elementwise(op.kind)) return false;
    for (int u : op.operands) {
      if (prog_.type(u).rank() == 0 && t.rank() > 0) {
        if (!walk(u, {}, visit)) return false;
      } else if (!walk(u, idx, visit)) {
        return false;
      }
    }
    return true;
  }
};

// One decode-shaped dot: [M, K] x [K, N] -> [M, N], 16-bit operands.
bool gemv_dot(const Program& prog, const Op& op) {
  if (op.kind != OpKind::kDotGeneral || op.operands.size() != 2) return false;
  const TensorType& l = prog.type(op.operands[0]);
  const TensorType& r = prog.type(op.operands[1]);
  const TensorType& o = prog.type(op.results[0]);
  if (l.rank() != 2 || r.rank() != 2 || !op.lhs_batch.empty() || !op.rhs_batch.empty() ||
      op.lhs_contract != Dims{1} || op.rhs_contract != Dims{0} || l.dtype != r.dtype ||
      (l.dtype != DType::kBF16 && l.dtype != DType::kF16))
    return false;
  if (o.dtype != DType::kBF16 && o.dtype != DType::kF16 && o.dtype != DType::kF32) return false;
  const int64_t M = l.dims[0], K = l.dims[1], N = r.dims[1];
  return M >= 1 && M <= 4 && K >= 8 && K % 8 == 0 && N >= 8 && N % 8 == 0 && N < (int64_t(1) << 28) &&
         M * K <= (int64_t(1) << 24);
}

// Writes in place into `v` between steps a and b (exclusive)?
bool written_between(const Program& prog, const std::vector<Step>& steps, size_t a, size_t b, int v) {
  for (size_t k = a + 1; k < b; ++k) {
    const Step& s = steps[k];
    for (auto& [pos, ww] : s.window_out)
      if (ww.operand == v) return true;
    if (s.kind == StepKind::kLibrary && s.in_place && prog.ops[s.lib_op].operands[0] == v) return true;
  }
  return false;
}

bool read_between(const std::vector<Step>& steps, size_t a, size_t b, int v) {
  for (size_t k = a + 1; k < b; ++k)
    for (int u : steps[k].inputs)
      if (u == v) return true;
  return false;
}

constexpr int64_t kMaxLdsFloats = 12288;  // LHS staged in LDS (48 KB)

class GemvFuser {
 public:
  GemvFuser(const Program& prog, Plan* plan, const std::set<int>& outputs, const PlanOptions& opts)
      : prog_(prog), plan_(*plan), steps_(plan->steps), outputs_(outputs), opts_(opts) {}

  void run() {
    bool any = false;
    for (size_t i = 0; i < steps_.size(); ++i) any |= convert(i);
    if (!any) return;
    for (size_t i = 0; i < steps_.size(); ++i) {
      if (steps_[i].kind != StepKind::kGemv) continue;
      absorb_prologue(&i);
    }
    for (size_t i = 0; i < steps_.size(); ++i) {
      if (steps_[i].kind != StepKind::kGemv) continue;
      absorb_epilogue(i);
    }
    int id = 0;
    for (Step& s : steps_) {
      if (s.kind != StepKind::kGemv) continue;
      shape(&s);
      s.name = strformat("pjrtx_gemv_%d", id++);
    }
    plan_.num_fusion_kernels += id;
    if (opts_.attn_merge_in_gemv) {
      for (Step& s : steps_)
        if (s.kind == StepKind::kGemv) merge_attention_splits(&s);
    }
    keep_weights_in_mall();
    releases();
  }

 private:
  const Program& prog_;
  Plan& plan_;
  std::vector<Step>& steps_;
  const std::set<int>& outputs_;
  const PlanOptions& opts_;

  int readers(int v) const {
    int n = 0;
    for (const Step& s : steps_)
      for (int u : s.inputs) n += u == v;
    return n;
  }

  bool convert(size_t i) {
    Step& D = steps_[i];
    if (D.kind != StepKind::kLibrary || (D.lib != LibKind::kDot && D.lib != LibKind::kDotGroup)) return false;
    const std::vector<int> dots = D.lib == LibKind::kDot ? std::vector<int>{D.lib_op} : D.group_ops;
    for (int d : dots)
      if (!gemv_dot(prog_, prog_.ops[d])) return false;
    Step G;
    G.kind = StepKind::kGemv;
    GemvSpec& g = G.gemv;
    g.x = prog_.ops[dots[0]].operands[0];
    g.M = static_cast<int>(prog_.type(g.x).dims[0]);
    g.K = prog_.type(g.x).dims[1];
    g.dots = dots;
    G.inputs.push_back(g.x);
    for (size_t m = 0; m < dots.size(); ++m) {
      const Op& op = prog_.ops[dots[m]];
      G.inputs.push_back(op.operands[1]);
      const bool with_add = D.lib == LibKind::kDot && D.dot_add >= 0;
      g.result.push_back(with_add ? D.outputs[0] : op.results[0]);
      g.add.push_back(with_add ? D.dot_add : -1);
      g.store.push_back(true);
      if (with_add) G.inputs.push_back(D.dot_add);
    }
    G.outputs = g.result;
    steps_[i] = std::move(G);
    return true;
  }

  // The row-fused step that produces the LHS, when every reader of the LHS
  // is this step: its phases run in the kernel, the row lands in LDS.
  void absorb_prologue(size_t* pi) {
    const size_t i = *pi;
    Step& G = steps_[i];
    const int x = G.gemv.x;
    auto v2s = producers_of(steps_);
    auto it = v2s.find(x);
    if (it == v2s.end() || outputs_.count(x) || readers(x) != 1) return;
    const size_t p = static_cast<size_t>(it->second);
    const Step& P = steps_[p];
    if (P.kind != StepKind::kRowFused || P.outputs != std::vector<int>{x} || !P.window_out.empty()) return;
    if (P.rows != G.gemv.M || P.row_len != G.gemv.K || G.gemv.M * G.gemv.K > kMaxLdsFloats) return;
    if (P.reduce_operand_shape != prog_.type(x).dims) return;
    for (int v : P.inputs)
      if (written_between(prog_, steps_, p, i, v)) return;
    Step moved = P;
    G.prologue.push_back(std::move(moved));
    std::vector<int> ins;
    for (int v : G.prologue[0].inputs) ins.push_back(v);
    for (int v : G.inputs)
      if (v != x && std::find(ins.begin(), ins.end(), v) == ins.end()) ins.push_back(v);
    G.inputs = ins;
    plan_.materialized.erase(x);
    steps_.erase(steps_.begin() + p);
    *pi = i - 1;
  }

  bool is_result(const Step& G, int v, int* member) const {
    for (size_t m = 0; m < G.gemv.result.size(); ++m)
      if (G.gemv.result[m] == v) {
        if (member) *member = static_cast<int>(m);
        return true;
      }
    return false;
  }

  // Smallest segment width (a multiple of the tile width dividing N) whose
  // segments close the loop's reads: root elements [s*R, (s+1)*R) read
  // member results only inside columns [s*S, (s+1)*S). 0 when none does.
  int64_t segment_width(const Step& G, const Step& L, int64_t N, int cols) {
    const int64_t root = num_elements(L.loop_shape);
    std::set<int> ins(L.inputs.begin(), L.inputs.end());
    ReadTracer tr(prog_, ins);
    std::vector<int> roots;
    for (size_t o = 0; o < L.outputs.size(); ++o) {
      auto ww = L.window_out.find(static_cast<int>(o));
      roots.push_back(ww == L.window_out.end() ? L.outputs[o] : ww->second.update);
    }
    // Column range of member reads per root element.
    std::vector<int64_t> lo(root, INT64_MAX), hi(root, -1);
    for (int64_t r = 0; r < root; ++r) {
      const std::vector<int64_t> idx = unravel(r, L.loop_shape);
      for (int v : roots) {
        bool ok;
        if (ins.count(v)) {
          // The output is an input value copied at the root index.
          if (prog_.type(v).elements() != root) return 0;
          ok = tr.trace(v, unravel(r, prog_.type(v).dims), [&](int u, int64_t lin) {
            if (!is_result(G, u, nullptr)) return;
            const int64_t c = lin % N;
            lo[r] = std::min(lo[r], c);
            hi[r] = std::max(hi[r], c);
          });
        } else {
          ok = tr.trace(v, idx, [&](int u, int64_t lin) {
            if (!is_result(G, u, nullptr)) return;
            const int64_t c = lin % N;
            lo[r] = std::min(lo[r], c);
            hi[r] = std::max(hi[r], c);
          });
        }
        if (!ok) return 0;
      }
    }
    // At least 8 segments when the product has 8 tiles, so that every XCD
    // gets work.
    const int64_t max_s = N / cols >= 8 ? N / 8 : N;
    for (int64_t S = cols; S <= max_s; S *= 2) {
      if (N % S != 0) continue;
      const int64_t nseg = N / S;
      if (root % nseg != 0) continue;
      const int64_t R = root / nseg;
      bool fits = true;
      for (int64_t r = 0; r < root && fits; ++r) {
        if (hi[r] < 0) continue;
        const int64_t s = r / R;
        fits = lo[r] >= s * S && hi[r] < (s + 1) * S;
      }
      if (fits) return S;
    }
    return 0;
  }

  // The first loop step after G that reads one of its results, when it can
  // run inside G: its other inputs exist before G and are not overwritten
  // in between, its cache writes can move up to G, and its reads of the
  // results stay within column segments.
  void absorb_epilogue(size_t i) {
    Step& G = steps_[i];
    auto v2s = producers_of(steps_);
    size_t l = 0;
    for (size_t k = i + 1; k < steps_.size() && !l; ++k) {
      for (int v : steps_[k].inputs)
        if (is_result(G, v, nullptr)) l = k;
    }
    if (!l) return;
    const Step& L = steps_[l];
    if (L.kind != StepKind::kLoop || num_elements(L.loop_shape) == 0) return;
    int64_t N = -1;
    for (int d : G.gemv.dots) {
      const int64_t n = prog_.type(prog_.ops[d].results[0]).dims[1];
      if (N >= 0 && n != N) return;
      N = n;
    }
    if (G.gemv.M != 1) return;  // epilogues only for single-row products (decode)
    for (int v : L.inputs) {
      if (is_result(G, v, nullptr)) continue;
      auto it = v2s.find(v);
      if (it != v2s.end() && it->second >= static_cast<int>(i)) return;
      if (written_between(prog_, steps_, i, l, v)) return;
    }
    for (auto& [pos, ww] : L.window_out) {
      const int r = L.outputs[pos];
      if (read_between(steps_, i, l, ww.operand) || read_between(steps_, i, l, r) ||
          written_between(prog_, steps_, i, l, ww.operand))
        return;
    }
    const int cols = tile_cols(N * static_cast<int64_t>(G.gemv.dots.size()));
    if (N % cols != 0) return;
    const int64_t S = segment_width(G, L, N, cols);
    if (S == 0) return;
    const int64_t lds_floats = static_cast<int64_t>(G.gemv.dots.size()) * G.gemv.M * S;
    if (lds_floats > 4096) return;
    // Results only the loop reads are no longer written to memory.
    for (size_t m = 0; m < G.gemv.result.size(); ++m) {
      const int v = G.gemv.result[m];
      int other = 0;
      for (size_t k = 0; k < steps_.size(); ++k)
        if (k != l)
          for (int u : steps_[k].inputs) other += u == v && k != i;
      G.gemv.store[m] = other > 0 || outputs_.count(v);
    }
    G.gemv.joint = true;
    G.gemv.seg_cols = S;
    G.gemv.root_per_seg = num_elements(L.loop_shape) / (N / S);
    std::vector<int> outs;
    for (size_t m = 0; m < G.gemv.result.size(); ++m) {
      if (G.gemv.store[m]) {
        outs.push_back(G.gemv.result[m]);
      } else {
        plan_.materialized.erase(G.gemv.result[m]);
      }
    }
    const int base = static_cast<int>(outs.size());
    Step loop = L;
    G.window_out.clear();
    for (auto& [pos, ww] : loop.window_out) G.window_out[base + pos] = ww;
    for (int v : loop.outputs) outs.push_back(v);
    G.outputs = outs;
    for (int v : loop.inputs)
      if (!is_result(G, v, nullptr) && std::find(G.inputs.begin(), G.inputs.end(), v) == G.inputs.end())
        G.inputs.push_back(v);
    G.epilogue_loop.push_back(std::move(loop));
    steps_.erase(steps_.begin() + l);
  }

  // Tile width: PJRTX_GEMV_COLS (32, 64 or 128) when set, else 128 columns
  // for wide products (8192 columns and more over the members) and 64 for the
  // rest (measured on cold weights: 128 is 4-8% faster on the 5632 x 2 gate/up
  // and 32000-column lm_head products, slower on 2048-column ones).
  int tile_cols(int64_t total_n = 0) const {
    const int64_t c = env_int("PJRTX_GEMV_COLS", 0);
    if (c == 32 || c == 64 || c == 128) return static_cast<int>(c);
    return total_n >= 8192 ? 128 : 64;
  }

  void shape(Step* s) {
    GemvSpec& g = s->gemv;
    int64_t total_n = 0;
    for (int dd : g.dots) total_n += prog_.type(prog_.ops[dd].results[0]).dims[1];
    // Joint segments were sized for the tile width chosen when the epilogue
    // was absorbed; keep tiles within a segment.
    g.cols = tile_cols(total_n);
    if (g.joint) {
      while (g.cols > 32 && g.seg_cols % g.cols != 0) g.cols /= 2;
    }
    // Weight rows in flight per lane: 4, 8 or 16 (PJRTX_GEMV_DEPTH); by
    // default 4, or 8 below when that puts a whole K chunk of a GEMV without
    // prologue in flight at once.
    const int64_t d = env_int("PJRTX_GEMV_DEPTH", 0);
    g.depth = (d == 8 || d == 16) ? static_cast<int>(d) : 4;
    const int64_t rows_per_step = 4 * (64 / (g.cols / 8));  // 256 threads
    const int members = static_cast<int>(g.dots.size());
    int64_t tiles = 0;
    if (g.joint) {
      const int64_t N = prog_.type(g.result[0]).dims[1];
      g.nseg = N / g.seg_cols;
      tiles = g.nseg * members * (g.seg_cols / g.cols);
    } else {
      g.seg_cols = g.cols;
      for (int dd : g.dots) {
        const int64_t N = prog_.type(prog_.ops[dd].results[0]).dims[1];
        g.nseg += (N + g.cols - 1) / g.cols;
      }
      tiles = g.nseg;
    }
    // One item per workgroup, the K split aiming at PJRTX_GEMV_WGS workgroups
    // (768). With PJRTX_GEMV_PERSIST=1, one batch of `depth` rows per lane is
    // one item and PJRTX_GEMV_PWGS workgroups (512) walk the items,
    // prefetching the next while folding the last: slower on this GPU (the
    // wait for a partial's stores before its arrival count also waits for the
    // prefetched loads, which complete in order), so off by default.
    const bool persist = env_int("PJRTX_GEMV_PERSIST", 0) != 0 && g.M * g.K <= kMaxLdsFloats;
    int64_t kchunk;
    if (persist) {
      kchunk = rows_per_step * g.depth;
    } else {
      const int64_t target = std::max<int64_t>(opts_.gemv_target_wgs, 1);
      int64_t ksplit = std::max<int64_t>(1, (target + tiles / 2) / tiles);
      ksplit = std::min<int64_t>(ksplit, std::max<int64_t>(1, g.K / rows_per_step));
      kchunk = (g.K + ksplit - 1) / ksplit;
      kchunk = (kchunk + rows_per_step - 1) / rows_per_step * rows_per_step;
    }
    // A workgroup that stages only its chunk of X keeps it within the LDS cap.
    const int64_t xs_cap = kMaxLdsFloats / g.M / rows_per_step * rows_per_step;
    if (s->prologue.empty()) kchunk = std::min(kchunk, xs_cap);
    g.kchunk = kchunk;
    // Depth 8 when it makes the chunk one batch and there is no prologue to
    // wait for first (C5 down projection, K 5632: 7.47 -> 6.72 us per call;
    // GEMVs with an RMSNorm prologue were slower at 8).
    if (d == 0 && !persist && s->prologue.empty() && kchunk > rows_per_step * 4 && kchunk <= rows_per_step * 8)
      g.depth = 8;
    g.ksplit = (g.K + kchunk - 1) / kchunk;
    g.wps = (g.joint ? members * (g.seg_cols / g.cols) : 1) * g.ksplit;
    g.direct = g.ksplit == 1 && !g.joint;
    const int64_t items_x = (g.nseg + 7) / 8 * g.wps;  // items of the busiest XCD
    int64_t per_xcd = items_x;
    if (persist) per_xcd = std::min<int64_t>(items_x, std::max<int64_t>(1, env_int("PJRTX_GEMV_PWGS", 512) / 8));
    g.wgs = 8 * per_xcd;
    g.stage_all_x = !s->prologue.empty() || per_xcd < items_x;
    g.partial_bytes = g.direct ? 0 : static_cast<size_t>(g.nseg * g.wps * g.M * g.cols) * 4;
    g.partial_bytes = (g.partial_bytes + 255) / 256 * 256;
    if (!g.direct) {
      s->fused_combine = true;
      s->counter_offset = g.partial_bytes;
      s->scratch_bytes = g.partial_bytes + static_cast<size_t>(g.nseg) * 128;
    }
    s->grid = static_cast<uint32_t>(g.wgs);
    s->block = 256;
  }

  // A GEMV without prologue whose LHS is, through layout-preserving aliases
  // only, the output of a split decode attention with one query row per head
  // (the o-projection of a decode step), and the only reader of each value on
  // the way: the attention writes its split partials instead of the rows and
  // the GEMV merges them while staging X. The attention launch then ends with
  // its partial stores (no arrival count, no merge round trips), and the
  // GEMV's X reads, issued before its weight rows as before, fetch the
  // partials instead. Up to 16 splits (the merge keeps each split's m, l and
  // value in registers).
  void merge_attention_splits(Step* G) {
    GemvSpec& g = G->gemv;
    if (!G->prologue.empty() || g.M != 1) return;
    auto v2s = producers_of(steps_);
    int v = g.x;
    for (;;) {
      auto it = v2s.find(v);
      if (it == v2s.end() || outputs_.count(v) || readers(v) != 1) return;
      const Step& P = steps_[it->second];
      if (P.kind == StepKind::kAlias) {
        v = P.inputs[0];
        continue;
      }
      if (P.kind != StepKind::kLibrary || P.lib != LibKind::kAttention || P.outputs != std::vector<int>{v}) return;
      const Op& op = prog_.ops[P.lib_op];
      const AttnParams ap = attention_params(prog_, op);
      const DType t = prog_.type(op.operands[0]).dtype;
      int nsplit = 1, per = 0;
      if (attention_path(ap, t, &nsplit, &per) != AttnPath::kDecode || nsplit < 2 || nsplit > 16) return;
      // Row r = head r (one batch, one query); X's flat element k is output
      // element (head k / D, column k % D), the rows D apart.
      if (ap.B != 1 || ap.Sq != 1 || ap.o_h != ap.D || static_cast<int64_t>(ap.Hq) * ap.D != g.K) return;
      if (prog_.type(op.results[0]).dtype != prog_.type(g.x).dtype) return;
      if (t != DType::kBF16 && t != DType::kF16) return;
      steps_[it->second].attn_partials = true;
      g.attn_splits = nsplit;
      g.attn_dim = ap.D;
      return;
    }
  }

  // The smallest GEMV weights, up to opts_.gemv_mall_mb in all, keep plain
  // loads (they may stay in the MALL between executes); the others stream
  // with non-temporal loads, which do not displace them.
  void keep_weights_in_mall() {
    const int64_t budget = opts_.gemv_mall_mb << 20;
    if (budget <= 0) return;
    std::vector<std::pair<int64_t, size_t>> by_size;
    for (size_t i = 0; i < steps_.size(); ++i) {
      if (steps_[i].kind != StepKind::kGemv) continue;
      int64_t bytes = 0;
      for (int d : steps_[i].gemv.dots) bytes += prog_.type(prog_.ops[d].operands[1]).bytes();
      by_size.push_back({bytes, i});
    }
    std::stable_sort(by_size.begin(), by_size.end(), [](const auto& a, const auto& b) { return a.first < b.first; });
    int64_t used = 0;
    for (auto& [bytes, i] : by_size) {
      if (used + bytes > budget) break;
      used += bytes;
      steps_[i].gemv.weights_nt = false;
    }
  }

  void releases() {
    for (Step& s : steps_) s.release_after.clear();
    std::set<int> persistent(prog_.params.begin(), prog_.params.end());
    for (int c : plan_.constants) persistent.insert(c);
    std::map<int, int> last_use;
    for (size_t i = 0; i < steps_.size(); ++i)
      for (int v : steps_[i].inputs) last_use[v] = static_cast<int>(i);
    for (auto& [v, i] : last_use) {
      if (persistent.count(v) || outputs_.count(v)) continue;
      steps_[i].release_after.push_back(v);
    }
  }
};

}  // namespace

void fuse_gemv_steps(const Program& prog, Plan* plan, const std::set<int>& outputs, const PlanOptions& opts) {
  if (!opts.gemv_fusion) return;
  GemvFuser(prog, plan, outputs, opts).run();
}

}  // namespace pjrtx
