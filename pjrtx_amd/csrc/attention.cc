// Fused attention: lowering of the scaled-dot-product-attention custom call,
// the rewrite of the unfused softmax-attention pattern into one kAttention
// op, and its dispatch.
//
// Custom call: reference src/backend/mlx_metal/custom_call.zig:119-150
// (target "pjrtx.mlx_metal.scaled_dot_product_attention", operands q, k, v,
// token_index) with the legality rules of lowering_custom_call.zig:216-300
// and the semantics of api.cc:4928-5062 (layouts [b,q,h,hd] / [q,h,hd],
// grouped heads, scale 1/sqrt(hd), key allowed iff key <= token + query,
// api.cc:937-950).
//
// Pattern: dot_general(q, k) -> [convert, scale, causal select] -> f32
// softmax over the key axis -> convert -> dot_general(p, v), the form
// jax.nn.softmax attention lowers to (and the reference executes as separate
// MLX steps, api.cc:3349-3498 and 3982-4044). The fused op keeps the
// unfused graph's roundings where they are cheap to keep (scores rounded to
// the dot output type before scaling) and otherwise differs only in where
// the probabilities are rounded to the input type (before, not after, the
// division by the row sum): within the 16-bit tolerance of the outputs.
// PJRTX_FUSED_ATTENTION=0 keeps the pattern unfused.
#include <cmath>
#include <cstring>
#include <map>
#include <set>

#include "custom_call.h"
#include "kernels/attention.h"
#include "planner.h"
#include "runtime.h"

namespace pjrtx {

namespace {

constexpr const char* kSdpaTarget = "pjrtx.mlx_metal.scaled_dot_product_attention";

bool is_attention_float(DType t) { return t == DType::kF32 || t == DType::kF16 || t == DType::kBF16; }

void lower_custom_call(Program* prog, Op* op) {
  if (op->target != kSdpaTarget) {
    // Registered identity / unary / binary targets (custom_call.cc).
    lower_registered_custom_call(*prog, op);
    return;
  }
  // reference: lowering_custom_call.zig:216-300
  PJRTX_CHECK(op->operands.size() == 4 && op->results.size() == 1, Code::kInvalidArgument,
              "scaled-dot-product-attention custom_call requires q, k, v, and token_index inputs with one output");
  const TensorType& q = prog->type(op->operands[0]);
  const TensorType& k = prog->type(op->operands[1]);
  const TensorType& v = prog->type(op->operands[2]);
  const TensorType& t = prog->type(op->operands[3]);
  const TensorType& out = prog->type(op->results[0]);
  PJRTX_CHECK(is_attention_float(q.dtype) && q.dtype == k.dtype && q.dtype == v.dtype && out.dtype == q.dtype,
              Code::kInvalidArgument, "attention custom_call requires matching f16/bf16/f32 q/k/v/output dtypes");
  PJRTX_CHECK(q.rank() == 3 || q.rank() == 4, Code::kInvalidArgument,
              "attention custom_call supports rank-3 [q,h,hd] or rank-4 [b,q,h,hd] q tensors");
  PJRTX_CHECK(k.rank() == q.rank() && v.rank() == q.rank() && k.dims == v.dims && q.dims == out.dims,
              Code::kInvalidArgument,
              "attention custom_call requires k/v cache tensors with matching shape and output shape matching q");
  const int qa = q.rank() == 4 ? 1 : 0, ha = qa + 1, da = qa + 2;
  PJRTX_CHECK(q.dims[da] == k.dims[da] && q.dims[ha] > 0 && k.dims[ha] > 0 && q.dims[ha] % k.dims[ha] == 0 &&
                  q.dims[qa] > 0 && k.dims[qa] > 0,
              Code::kInvalidArgument,
              "attention custom_call requires positive q/k lengths, equal head_dim, and q_heads divisible by kv_heads");
  PJRTX_CHECK(q.rank() == 3 || q.dims[0] == k.dims[0], Code::kInvalidArgument,
              "attention custom_call requires q and k batch dimensions to match");
  PJRTX_CHECK(!dtype_is_float(t.dtype) && t.dtype != DType::kPred && (t.rank() == 0 || (t.rank() == 1 && t.dims[0] == 1)),
              Code::kInvalidArgument, "attention custom_call token_index must be an integer scalar or length-1 tensor");
  op->kind = OpKind::kAttention;
  op->name = "pjrtx.attention";
  op->attn = AttentionAttrs();
  op->attn.layout = q.rank() == 4 ? 1 : 2;
  op->attn.scale = 1.0f / std::sqrt(static_cast<float>(q.dims[da]));
  op->attn.causal = true;
  op->attn.q_coef = 1;
  op->attn.offset = 0;
  op->attn.has_offset_operand = true;
  op->attn.round_scores = false;
}

// ------------------------------------------------------------- matching

class Matcher {
 public:
  explicit Matcher(Program* prog) : prog_(*prog) {
    for (size_t i = 0; i < prog_.ops.size(); ++i) {
      for (int r : prog_.ops[i].results) producer_[r] = static_cast<int>(i);
      for (int u : prog_.ops[i].operands) users_[u]++;
    }
    for (int r : prog_.results) results_.insert(r);
  }

  // Rewrites dot_general op `i` (the p.v product) when it closes the pattern.
  bool try_rewrite(int i) {
    Op& d2 = prog_.ops[i];
    if (d2.kind != OpKind::kDotGeneral || d2.operands.size() != 2) return false;
    if (d2.lhs_batch != Dims{0, 1} || d2.rhs_batch != Dims{0, 1} || d2.lhs_contract != Dims{3} ||
        d2.rhs_contract != Dims{2})
      return false;
    const int P = d2.operands[0], V = d2.operands[1];
    const TensorType& pt = prog_.type(P);
    const TensorType& vt = prog_.type(V);
    const DType T = vt.dtype;
    if (pt.rank() != 4 || vt.rank() != 4 || (T != DType::kBF16 && T != DType::kF16) || pt.dtype != T ||
        prog_.type(d2.results[0]).dtype != T)
      return false;
    // P = convert(E / broadcast(sum(E)))
    const Op* cv = only_use_producer(P, OpKind::kConvert);
    if (!cv || prog_.type(cv->operands[0]).dtype != DType::kF32) return false;
    const int pdiv = cv->operands[0];
    const Op* dv = only_use_producer(pdiv, OpKind::kDivide);
    if (!dv) return false;
    const int E = dv->operands[0];
    const int Z = row_broadcast_source(dv->operands[1]);
    if (Z < 0 || !single_use(dv->operands[1])) return false;
    const Op* zr = only_use_producer(Z, OpKind::kReduce);
    if (!zr || !row_reduce(*zr, E, ReducerKind::kSum, 0.0)) return false;
    // E = exp(X - broadcast(max(X)))
    if (users_[E] != 2 || results_.count(E)) return false;
    const Op* ex = producer(E, OpKind::kExp);
    if (!ex || !single_use(ex->operands[0])) return false;
    const Op* sub = producer(ex->operands[0], OpKind::kSubtract);
    if (!sub) return false;
    const int X = sub->operands[0];
    const int M = row_broadcast_source(sub->operands[1]);
    if (M < 0 || !single_use(sub->operands[1])) return false;
    const Op* mr = only_use_producer(M, OpKind::kReduce);
    if (!mr || !row_reduce(*mr, X, ReducerKind::kMax, -INFINITY)) return false;
    if (users_[X] != 2 || results_.count(X) || prog_.type(X).dtype != DType::kF32) return false;
    // X = [convert, scale, select] chain over S = dot_general(q, k).
    AttentionAttrs a;
    a.layout = 0;
    a.round_scores = true;
    int cur = X, pred = -1;
    bool pred_negated = false, converted = false;
    int S = -1;
    while (S < 0) {
      if (cur != X && !single_use(cur)) return false;
      auto it = producer_.find(cur);
      if (it == producer_.end()) return false;
      const Op& op = prog_.ops[it->second];
      double c = 0;
      if (op.kind == OpKind::kConvert) {
        if (converted || prog_.type(cur).dtype != DType::kF32 || prog_.type(op.operands[0]).dtype != T) return false;
        converted = true;
        cur = op.operands[0];
      } else if (op.kind == OpKind::kMultiply && !converted &&
                 (splat_float(op.operands[1], &c) || splat_float(op.operands[0], &c))) {
        a.scale *= c;
        cur = splat_float(op.operands[1], &c) ? op.operands[0] : op.operands[1];
      } else if (op.kind == OpKind::kDivide && !converted && splat_float(op.operands[1], &c)) {
        a.scale /= c;
        cur = op.operands[0];
      } else if (op.kind == OpKind::kSelect && pred < 0) {
        double c1 = 0, c2 = 0;
        if (splat_float(op.operands[2], &c2) && c2 == -INFINITY) {
          pred = op.operands[0];
          cur = op.operands[1];
        } else if (splat_float(op.operands[1], &c1) && c1 == -INFINITY) {
          pred = op.operands[0];
          pred_negated = true;
          cur = op.operands[2];
        } else {
          return false;
        }
      } else if (op.kind == OpKind::kDotGeneral) {
        S = cur;
      } else {
        return false;
      }
    }
    if (!converted || (cur != X && !single_use(S))) return false;
    const Op& d1 = prog_.ops[producer_.at(S)];
    if (d1.lhs_batch != Dims{0, 1} || d1.rhs_batch != Dims{0, 1} || d1.lhs_contract != Dims{3} ||
        d1.rhs_contract != Dims{3})
      return false;
    const int Q = d1.operands[0], K = d1.operands[1];
    const TensorType& qt = prog_.type(Q);
    const TensorType& kt = prog_.type(K);
    if (qt.dtype != T || kt.dtype != T || prog_.type(S).dtype != T || qt.rank() != 4 || kt.rank() != 4) return false;
    if (kt.dims[0] != qt.dims[0] || kt.dims[1] != qt.dims[1] || kt.dims[3] != qt.dims[3]) return false;
    if (vt.dims[0] != qt.dims[0] || vt.dims[1] != qt.dims[1] || vt.dims[2] != kt.dims[2]) return false;
    if (qt.dims[2] < kMinQueries) return false;
    int dev = -1;
    if (pred >= 0) {
      if (!causal_mask(pred, pred_negated, &a, &dev)) return false;
    }
    Op& out = prog_.ops[i];
    out.kind = OpKind::kAttention;
    out.name = "pjrtx.attention";
    out.operands = {Q, K, V};
    if (dev >= 0) out.operands.push_back(dev);
    out.attn = a;
    out.lhs_batch.clear();
    out.rhs_batch.clear();
    out.lhs_contract.clear();
    out.rhs_contract.clear();
    return true;
  }

  // Fewest queries per (batch, head) worth fusing.
  static constexpr int64_t kMinQueries = 1;

 private:
  Program& prog_;
  std::map<int, int> producer_;
  std::map<int, int> users_;
  std::set<int> results_;

  bool single_use(int v) { return users_[v] == 1 && !results_.count(v); }
  const Op* producer(int v, OpKind k) {
    auto it = producer_.find(v);
    if (it == producer_.end()) return nullptr;
    const Op& op = prog_.ops[it->second];
    return op.kind == k ? &op : nullptr;
  }
  const Op* only_use_producer(int v, OpKind k) { return single_use(v) ? producer(v, k) : nullptr; }

  // v = broadcast_in_dim(r, dims {0, 1, 2}) of a [B, H, S] row value.
  int row_broadcast_source(int v) {
    const Op* b = producer(v, OpKind::kBroadcastInDim);
    if (!b || b->dims != Dims{0, 1, 2}) return -1;
    const TensorType& rt = prog_.type(b->operands[0]);
    const TensorType& vt = prog_.type(v);
    if (rt.rank() != 3 || vt.rank() != 4) return -1;
    for (int d = 0; d < 3; ++d)
      if (rt.dims[d] != vt.dims[d]) return -1;
    return b->operands[0];
  }

  bool row_reduce(const Op& r, int input, ReducerKind kind, double init) {
    if (r.operands.size() != 2 || r.results.size() != 1 || r.operands[0] != input || r.dims != Dims{3}) return false;
    if (classify_reducer(prog_, r) != kind) return false;
    double c = 0;
    return splat_float(r.operands[1], &c) && c == init;
  }

  // A floating splat constant, through broadcasts, reshapes and converts.
  bool splat_float(int v, double* out) {
    auto it = producer_.find(v);
    if (it == producer_.end()) return false;
    const Op& op = prog_.ops[it->second];
    if (op.kind == OpKind::kBroadcastInDim || op.kind == OpKind::kReshape ||
        (op.kind == OpKind::kConvert && dtype_is_float(prog_.type(op.operands[0]).dtype)))
      return splat_float(op.operands[0], out);
    if (op.kind != OpKind::kConstant || !(op.splat || prog_.type(v).elements() == 1) || op.literal.empty()) return false;
    const DType t = prog_.type(v).dtype;
    const uint8_t* b = op.literal.data();
    if (t == DType::kF32) {
      float f;
      std::memcpy(&f, b, 4);
      *out = f;
    } else if (t == DType::kF64) {
      std::memcpy(out, b, 8);
    } else if (t == DType::kBF16 || t == DType::kF16) {
      uint16_t h;
      std::memcpy(&h, b, 2);
      *out = t == DType::kBF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
    } else {
      return false;
    }
    return true;
  }

  // Integer affine form over the score index space (q = dim 2, k = dim 3)
  // plus at most one device scalar.
  struct Affine {
    int64_t cq = 0, ck = 0, c = 0;
    int dev = -1;
    int64_t dev_coef = 0;
  };

  bool splat_int(int v, int64_t* out) {
    auto it = producer_.find(v);
    if (it == producer_.end()) return false;
    const Op& op = prog_.ops[it->second];
    if (op.kind == OpKind::kBroadcastInDim || op.kind == OpKind::kReshape) return splat_int(op.operands[0], out);
    if (op.kind != OpKind::kConstant || !(op.splat || prog_.type(v).elements() == 1) || op.literal.empty()) return false;
    const DType t = prog_.type(v).dtype;
    if (!dtype_is_signed_int(t) && !dtype_is_unsigned_int(t)) return false;
    int64_t x = 0;
    const size_t n = dtype_size(t);
    std::memcpy(&x, op.literal.data(), n);
    if (dtype_is_signed_int(t) && n < 8) x = (x << (64 - 8 * n)) >> (64 - 8 * n);
    *out = x;
    return true;
  }

  // `map[d]` names the score dimension that dim d of v follows (2 = query,
  // 3 = key, 0/1 = batch/head, -1 = a size-1 dim read at index 0).
  bool affine(int v, const std::vector<int>& map, Affine* a, int depth = 0) {
    if (depth > 16) return false;
    const TensorType& t = prog_.type(v);
    if (!dtype_is_signed_int(t.dtype)) return false;
    int64_t c = 0;
    if (splat_int(v, &c)) {
      *a = Affine();
      a->c = c;
      return true;
    }
    bool all_fixed = true;
    for (size_t d = 0; d < map.size(); ++d) all_fixed &= map[d] == -1;
    auto it = producer_.find(v);
    const Op* op = it == producer_.end() ? nullptr : &prog_.ops[it->second];
    if (op && op->kind == OpKind::kIota) {
      *a = Affine();
      const int m = map[op->dim];
      if (m == 2) a->cq = 1;
      else if (m == 3) a->ck = 1;
      else if (m != -1) return false;
      return true;
    }
    if (op && op->kind == OpKind::kBroadcastInDim) {
      const Dims& od = prog_.type(op->operands[0]).dims;
      std::vector<int> om(od.size());
      for (size_t k = 0; k < od.size(); ++k) om[k] = od[k] == 1 ? -1 : map[op->dims[k]];
      return affine(op->operands[0], om, a, depth + 1);
    }
    if (op && op->kind == OpKind::kConvert) return affine(op->operands[0], map, a, depth + 1);
    if (op && (op->kind == OpKind::kAdd || op->kind == OpKind::kSubtract)) {
      Affine x, y;
      if (!affine(op->operands[0], map, &x, depth + 1) || !affine(op->operands[1], map, &y, depth + 1)) return false;
      const int64_t s = op->kind == OpKind::kAdd ? 1 : -1;
      if (x.dev >= 0 && y.dev >= 0 && x.dev != y.dev) return false;
      a->cq = x.cq + s * y.cq;
      a->ck = x.ck + s * y.ck;
      a->c = x.c + s * y.c;
      a->dev = x.dev >= 0 ? x.dev : y.dev;
      a->dev_coef = x.dev_coef + s * y.dev_coef;
      return true;
    }
    if (all_fixed && t.elements() == 1) {  // one runtime integer: read by the kernel
      *a = Affine();
      a->dev = v;
      a->dev_coef = 1;
      return true;
    }
    if (op && op->kind == OpKind::kReshape && prog_.type(op->operands[0]).elements() == 1) {
      const std::vector<int> om(prog_.type(op->operands[0]).rank(), -1);
      return affine(op->operands[0], om, a, depth + 1);
    }
    return false;
  }

  // pred (or its negation) must read "key <= q_coef * query + offset [+ dev]".
  bool causal_mask(int pred, bool negated, AttentionAttrs* a, int* dev) {
    std::vector<int> map = {0, 1, 2, 3};
    int v = pred;
    for (int guard = 0; guard < 8; ++guard) {
      const Op* b = producer(v, OpKind::kBroadcastInDim);
      if (!b) break;
      const Dims& od = prog_.type(b->operands[0]).dims;
      std::vector<int> om(od.size());
      for (size_t k = 0; k < od.size(); ++k) om[k] = od[k] == 1 ? -1 : map[b->dims[k]];
      map = om;
      v = b->operands[0];
    }
    const Op* cmp = producer(v, OpKind::kCompare);
    if (!cmp || cmp->cmp_type == CmpType::kUnsigned || cmp->cmp_type == CmpType::kFloat) return false;
    Affine x, y;
    if (!affine(cmp->operands[0], map, &x) || !affine(cmp->operands[1], map, &y)) return false;
    if (x.dev >= 0 && y.dev >= 0 && x.dev != y.dev) return false;
    // L = x - y; the predicate is "L <dir> 0".
    Affine L;
    L.cq = x.cq - y.cq;
    L.ck = x.ck - y.ck;
    L.c = x.c - y.c;
    L.dev = x.dev >= 0 ? x.dev : y.dev;
    L.dev_coef = x.dev_coef - y.dev_coef;
    CmpDir dir = cmp->cmp_dir;
    if (negated) {
      switch (dir) {
        case CmpDir::kLE: dir = CmpDir::kGT; break;
        case CmpDir::kLT: dir = CmpDir::kGE; break;
        case CmpDir::kGE: dir = CmpDir::kLT; break;
        case CmpDir::kGT: dir = CmpDir::kLE; break;
        default: return false;
      }
    }
    // Bring to "L' <= 0" with integer L'.
    if (dir == CmpDir::kGE || dir == CmpDir::kGT) {
      L.cq = -L.cq, L.ck = -L.ck, L.c = -L.c, L.dev_coef = -L.dev_coef;
      dir = dir == CmpDir::kGE ? CmpDir::kLE : CmpDir::kLT;
    }
    if (dir == CmpDir::kLT) L.c += 1;  // L < 0  <=>  L + 1 <= 0
    else if (dir != CmpDir::kLE) return false;
    // k + cq*q + c + dev_coef*dev <= 0  <=>  k <= -cq*q - c - dev_coef*dev
    if (L.ck != 1 || (L.cq != 0 && L.cq != -1) || (L.dev_coef != 0 && L.dev_coef != -1)) return false;
    if (L.dev_coef == 0) L.dev = -1;
    a->causal = true;
    a->q_coef = static_cast<int>(-L.cq);
    a->offset = -L.c;
    a->has_offset_operand = L.dev >= 0;
    *dev = L.dev;
    return true;
  }
};

void remove_dead_ops(Program* prog) {
  std::set<int> live(prog->results.begin(), prog->results.end());
  std::vector<bool> keep(prog->ops.size(), false);
  for (int i = static_cast<int>(prog->ops.size()) - 1; i >= 0; --i) {
    const Op& op = prog->ops[i];
    bool used = op.kind == OpKind::kReturn;
    for (int r : op.results) used |= live.count(r) > 0;
    if (!used) continue;
    keep[i] = true;
    for (int u : op.operands) live.insert(u);
  }
  std::vector<Op> ops;
  for (size_t i = 0; i < prog->ops.size(); ++i)
    if (keep[i]) ops.push_back(std::move(prog->ops[i]));
  prog->ops = std::move(ops);
}

}  // namespace

void rewrite_program(Program* prog) {
  bool changed = false;
  for (Op& op : prog->ops) {
    if (op.kind == OpKind::kCustomCall) {
      lower_custom_call(prog, &op);
      changed = true;
    }
  }
  changed |= fold_gather_index_wrap(prog);
  const char* env = std::getenv("PJRTX_FUSED_ATTENTION");
  if (!(env && std::string(env) == "0")) {
    remove_dead_ops(prog);  // use counts below must not see dead users
    for (size_t i = 0; i < prog->ops.size(); ++i) {
      Matcher m(prog);  // rebuilt per rewrite: use counts change
      if (m.try_rewrite(static_cast<int>(i))) changed = true;
    }
  }
  if (changed) remove_dead_ops(prog);
}

namespace {

void strides_of(const AttentionAttrs& a, const Dims& d, int64_t* sb, int64_t* sh, int64_t* ss) {
  if (a.layout == 0) {  // [B, H, S, D]
    *ss = d[3];
    *sh = d[2] * d[3];
    *sb = d[1] * d[2] * d[3];
  } else if (a.layout == 1) {  // [B, S, H, D]
    *sh = d[3];
    *ss = d[2] * d[3];
    *sb = d[1] * d[2] * d[3];
  } else {  // [S, H, D]
    *sh = d[2];
    *ss = d[1] * d[2];
    *sb = 0;
  }
}

}  // namespace

AttnParams attention_params(const Program& prog, const Op& op) {
  const AttentionAttrs& a = op.attn;
  const Dims& q = prog.type(op.operands[0]).dims;
  const Dims& k = prog.type(op.operands[1]).dims;
  AttnParams p;
  const int sa = a.layout == 0 ? 2 : a.layout == 1 ? 1 : 0;
  const int ha = a.layout == 0 ? 1 : a.layout == 1 ? 2 : 1;
  const int64_t B = a.layout == 2 ? 1 : q[0];
  const int64_t lim = int64_t(1) << 31;
  PJRTX_CHECK(B < lim && q[ha] < lim && q[sa] < lim && k[sa] < lim && q.back() < lim, Code::kUnimplemented,
              "attention: dimension too large");
  p.B = static_cast<int>(B);
  p.Hq = static_cast<int>(q[ha]);
  p.Hkv = static_cast<int>(k[ha]);
  p.Sq = static_cast<int>(q[sa]);
  p.Skv = static_cast<int>(k[sa]);
  p.D = static_cast<int>(q.back());
  strides_of(a, q, &p.q_b, &p.q_h, &p.q_s);
  strides_of(a, k, &p.k_b, &p.k_h, &p.k_s);
  strides_of(a, prog.type(op.operands[2]).dims, &p.v_b, &p.v_h, &p.v_s);
  strides_of(a, prog.type(op.results[0]).dims, &p.o_b, &p.o_h, &p.o_s);
  p.scale = static_cast<float>(a.scale);
  p.causal = a.causal ? 1 : 0;
  p.q_coef = a.q_coef;
  p.offset = a.offset;
  p.round_scores = a.round_scores ? 1 : 0;
  if (a.has_offset_operand) {
    const DType t = prog.type(op.operands[3]).dtype;
    p.offset_bytes = static_cast<int>(dtype_size(t));
    p.offset_signed = dtype_is_signed_int(t) ? 1 : 0;
    p.offset_as_s32 = a.layout != 0 ? 1 : 0;  // the custom call casts its token index to s32
  }
  return p;
}

static_assert(Device::kArrivalCounterBytes / 128 >= kAttnCounterRows, "one counter line per decode query row");

size_t attention_partials_bytes(const Program& prog, const Op& op) {
  return attention_scratch_bytes(attention_params(prog, op), prog.type(op.operands[0]).dtype);
}

void run_attention(Device* dev, const Program& prog, const Op& op, std::vector<MemRef>& vals, bool partials_out) {
  AttnParams p = attention_params(prog, op);
  auto ptr = [&](int v) -> void* { return vals[v] ? vals[v]->ptr : nullptr; };
  if (op.attn.has_offset_operand) p.offset_ptr = ptr(op.operands[3]);
  const DType t = prog.type(op.operands[0]).dtype;
  const size_t scratch_bytes = partials_out ? 0 : attention_scratch_bytes(p, t);
  if (partials_out) {
    PJRTX_CHECK(vals[op.results[0]] && vals[op.results[0]]->bytes >= attention_scratch_bytes(p, t), Code::kInternal,
                "attention: partials output buffer too small");
  }
  MemRef scratch = scratch_bytes ? dev->allocate(scratch_bytes) : nullptr;
  launch_attention(dev->stream(), p, t, ptr(op.operands[0]), ptr(op.operands[1]), ptr(op.operands[2]),
                   ptr(op.results[0]), scratch ? static_cast<float*>(scratch->ptr) : nullptr, dev->arrival_counters(),
                   dev->xcd_round_robin(), partials_out);
}

}  // namespace pjrtx
