// dot_general: StableHLO dimension numbers -> batched GEMM / GEMV launch.
//
// Output dims follow StableHLO (batch..., lhs free..., rhs free...), the same
// order the reference produces (reference: src/backend/mlx_metal/api.cc:
// 1562-1577, 3429-3492). Each operand is viewed as [batch][rows][K] or
// [batch][K][cols] with uniform strides when its dimension groups can be
// merged; otherwise it is first copied into that canonical layout.
#include <algorithm>

#include "blaslt.h"
#include "kernels/dot.h"
#include "kernels/library.h"
#include "runtime.h"

namespace pjrtx {

namespace {

struct OperandView {
  int64_t batch = 1, free = 1, k = 1;
  int64_t bs = 0, fs = 0, ks = 0;  // strides (elements); 0 when the group is empty
  bool ok = true;                  // groups mergeable into single strides
};

// Merges a group of dims (in the given order) into one (size, stride).
bool merge(const Dims& dims, const int64_t* strides, const std::vector<int64_t>& group, int64_t* size, int64_t* stride) {
  *size = 1;
  *stride = 0;
  if (group.empty()) return true;
  for (size_t i = 0; i < group.size(); ++i) {
    const int64_t d = group[i];
    if (i + 1 < group.size()) {
      const int64_t nd = group[i + 1];
      if (dims[nd] != 1 && dims[d] != 1 && strides[d] != strides[nd] * dims[nd]) return false;
    }
    *size *= dims[d];
  }
  // stride of the innermost non-unit dim of the group
  *stride = strides[group.back()];
  for (auto it = group.rbegin(); it != group.rend(); ++it)
    if (dims[*it] != 1) {
      *stride = strides[*it];
      break;
    }
  return true;
}

OperandView view_of(const TensorType& t, const Dims& batch, const Dims& contract) {
  int64_t st[kMaxRank];
  int64_t s = 1;
  for (int i = t.rank() - 1; i >= 0; --i) {
    st[i] = s;
    s *= t.dims[i];
  }
  std::vector<int64_t> b(batch.begin(), batch.end()), c(contract.begin(), contract.end()), f;
  for (int d = 0; d < t.rank(); ++d)
    if (std::find(b.begin(), b.end(), d) == b.end() && std::find(c.begin(), c.end(), d) == c.end()) f.push_back(d);
  OperandView v;
  v.ok = merge(t.dims, st, b, &v.batch, &v.bs) && merge(t.dims, st, f, &v.free, &v.fs) &&
         merge(t.dims, st, c, &v.k, &v.ks);
  return v;
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

// Copies `t` into a canonical [batch][free][k] (or [batch][k][free] when
// k_inner is false) row-major buffer.
MemRef canonicalize(Device* dev, const TensorType& t, const Dims& batch, const Dims& contract, const void* src,
                    bool k_inner) {
  int64_t st[kMaxRank];
  int64_t s = 1;
  for (int i = t.rank() - 1; i >= 0; --i) {
    st[i] = s;
    s *= t.dims[i];
  }
  std::vector<int64_t> order(batch.begin(), batch.end()), f;
  for (int d = 0; d < t.rank(); ++d)
    if (std::find(batch.begin(), batch.end(), d) == batch.end() &&
        std::find(contract.begin(), contract.end(), d) == contract.end())
      f.push_back(d);
  if (k_inner) {
    order.insert(order.end(), f.begin(), f.end());
    order.insert(order.end(), contract.begin(), contract.end());
  } else {
    order.insert(order.end(), contract.begin(), contract.end());
    order.insert(order.end(), f.begin(), f.end());
  }
  BoxCopy b;
  b.rank = t.rank();
  int64_t ds = 1;
  for (int i = b.rank - 1; i >= 0; --i) {
    const int64_t d = order[i];
    b.dims[i] = t.dims[d];
    b.src_stride[i] = st[d];
    b.dst_stride[i] = ds;
    ds *= t.dims[d];
  }
  MemRef out = dev->allocate(t.bytes());
  launch_box_copy(dev->stream(), b, src, out->ptr, static_cast<int>(dtype_size(t.dtype)));
  return out;
}

}  // namespace

// Workgroups of the one-pass GEMV for a single product with N columns.
int single_wide_tiles(int64_t N) {
  GemvGroup one;
  one.count = 1;
  one.m[0].N = static_cast<int>(N);
  return gemv_wide_tiles(one);
}

void run_dot_general(Device* dev, const Program& prog, const Op& op, std::vector<MemRef>& vals) {
  const TensorType& lt = prog.type(op.operands[0]);
  const TensorType& rt = prog.type(op.operands[1]);
  const TensorType& ot = prog.type(op.results[0]);
  PJRTX_CHECK(lt.rank() <= kMaxRank && rt.rank() <= kMaxRank, Code::kUnimplemented, "dot_general: rank too large");
  PJRTX_CHECK(op.lhs_batch.size() == op.rhs_batch.size() && op.lhs_contract.size() == op.rhs_contract.size(),
              Code::kInvalidArgument, "dot_general: dimension numbers do not pair up");
  for (size_t i = 0; i < op.lhs_batch.size(); ++i)
    PJRTX_CHECK(lt.dims[op.lhs_batch[i]] == rt.dims[op.rhs_batch[i]], Code::kInvalidArgument, "dot_general: batch size mismatch");
  for (size_t i = 0; i < op.lhs_contract.size(); ++i)
    PJRTX_CHECK(lt.dims[op.lhs_contract[i]] == rt.dims[op.rhs_contract[i]], Code::kInvalidArgument,
                "dot_general: contracting size mismatch");
  PJRTX_CHECK(lt.dtype == rt.dtype, Code::kUnimplemented, "dot_general: mixed operand types");

  OperandView a = view_of(lt, op.lhs_batch, op.lhs_contract);
  OperandView b = view_of(rt, op.rhs_batch, op.rhs_contract);
  const int64_t batch = a.batch, M = a.free, N = b.free, K = a.k;
  void* out = vals[op.results[0]]->ptr;
  if (ot.elements() == 0) return;
  const void* A = vals[op.operands[0]]->ptr;
  const void* B = vals[op.operands[1]]->ptr;
  const bool low_precision = lt.dtype == DType::kBF16 || lt.dtype == DType::kF16;
  const bool out_ok = ot.dtype == lt.dtype || ot.dtype == DType::kF32;
  if (K == 0) {  // empty contraction: zeros
    launch_zero(dev->stream(), out, ot.elements() * static_cast<int64_t>(dtype_size(ot.dtype)));
    return;
  }
  if (low_precision && out_ok) {
    const bool f16 = lt.dtype == DType::kF16;
    const int out_kind = ot.dtype == DType::kBF16 ? 0 : (ot.dtype == DType::kF16 ? 1 : 2);
    MemRef a_copy, b_copy;
    // LHS must be K-contiguous with 16-byte aligned rows.
    const bool a_fast = a.ok && (a.ks == 1 || K == 1) && (M == 1 || a.fs % 8 == 0) && (batch == 1 || a.bs % 8 == 0) &&
                        aligned16(A) && K % 8 == 0;
    if (!a_fast && K % 8 == 0) {
      a_copy = canonicalize(dev, lt, op.lhs_batch, op.lhs_contract, A, true);
      A = a_copy->ptr;
      a = OperandView{batch, M, K, M * K, K, 1, true};
    }
    // RHS: N-contiguous ([K][N]) or K-contiguous ([N][K]).
    bool b_kmajor = b.ok && (b.ks == 1 || K == 1) && (N == 1 || b.fs % 8 == 0) && (batch == 1 || b.bs % 8 == 0) &&
                    aligned16(B) && K % 8 == 0;
    bool b_nmajor = b.ok && (b.fs == 1 || N == 1) && (K == 1 || b.ks % 8 == 0) && (batch == 1 || b.bs % 8 == 0) &&
                    aligned16(B) && N % 8 == 0;
    if (b_nmajor && N != 1) b_kmajor = false;
    if (!b_kmajor && !b_nmajor && K % 8 == 0) {
      b_copy = canonicalize(dev, rt, op.rhs_batch, op.rhs_contract, B, true);  // [batch][N][K]
      B = b_copy->ptr;
      b = OperandView{batch, N, K, N * K, K, 1, true};
      b_kmajor = true;
    }
    if ((a_fast || a_copy) && (b_kmajor || b_nmajor) && K % 8 == 0) {
      if (M <= 8 && batch == 1 && !b_kmajor && !a_copy && N < (int64_t(1) << 30) &&
          gemv_wide_fits(static_cast<int>(M), static_cast<int>(K), single_wide_tiles(N)) && N % 8 == 0 &&
          (K == 1 || b.ks % 8 == 0)) {
        GemvGroup g;
        g.count = 1;
        g.M = static_cast<int>(M);
        g.K = static_cast<int>(K);
        g.ldx = a.fs ? a.fs : K;
        g.out_kind = out_kind;
        g.m[0].W = B;
        g.m[0].Y = out;
        g.m[0].N = static_cast<int>(N);
        g.m[0].ldw = b.ks ? b.ks : N;
        g.m[0].ldy = N;
        launch_gemv_wide(dev->stream(), g, A, f16);
        return;
      }
      if (M <= 8) {
        GemvParams g;
        g.batch = static_cast<int>(batch);
        g.M = static_cast<int>(M);
        g.N = static_cast<int>(N);
        g.K = static_cast<int>(K);
        g.ldx = a.fs ? a.fs : K;
        g.ldw = b_kmajor ? (b.fs ? b.fs : K) : (b.ks ? b.ks : N);
        g.ldy = N;
        g.x_bs = a.bs;
        g.w_bs = b.bs;
        g.y_bs = M * N;
        g.out_kind = out_kind;
        MemRef part;
        if (!b_kmajor) {
          plan_gemv_split(&g);
          if (g.ksplit > 1) part = dev->allocate(static_cast<size_t>(batch * g.ksplit * M * N) * 4);
        }
        launch_gemv(dev->stream(), g, A, B, out, part ? static_cast<float*>(part->ptr) : nullptr, f16, b_kmajor);
        return;
      }
      GemmParams g;
      g.batch = static_cast<int>(batch);
      g.M = static_cast<int>(M);
      g.N = static_cast<int>(N);
      g.K = static_cast<int>(K);
      g.lda = a.fs ? a.fs : K;
      g.ldb = b_kmajor ? (b.fs ? b.fs : K) : (b.ks ? b.ks : N);
      g.ldc = N;
      g.a_batch_stride = a.bs;
      g.b_batch_stride = b.bs;
      if (batch * M * N * K > 0 && blaslt_wanted(g) &&
          blaslt_gemm(dev, g, A, B, out, f16, b_kmajor, out_kind == 2 ? 4 : 2))
        return;
      MemRef bt;
      if (!b_kmajor && !use_big_gemm(g, false)) {
        // The large-tile kernel reads an N-contiguous B directly when its
        // rows allow (N a multiple of 8); otherwise transpose B ([K][N] per
        // batch) once, at HBM speed, when the kernel applies to the result.
        GemmParams t = g;
        t.ldb = K;
        t.b_batch_stride = N * K;
        if (use_big_gemm(t, true) && g.ldb == N && (batch == 1 || b.bs == K * N)) {
          bt = dev->allocate(static_cast<size_t>(batch * N * K) * 2);
          launch_transpose16(dev->stream(), B, bt->ptr, batch, K, N, K * N, N * K);
          B = bt->ptr;
          g = t;
          b_kmajor = true;
        }
      }
      launch_mfma_gemm(dev->stream(), g, A, B, out, f16, b_kmajor, out_kind == 2 ? 4 : 2);
      return;
    }
  }
  // Scalar fallback with general strides.
  if (!a.ok) {
    MemRef c = canonicalize(dev, lt, op.lhs_batch, op.lhs_contract, A, true);
    vals.push_back(c);  // keep alive until the step ends
    A = c->ptr;
    a = OperandView{batch, M, K, M * K, K, 1, true};
  }
  if (!b.ok) {
    MemRef c = canonicalize(dev, rt, op.rhs_batch, op.rhs_contract, B, true);
    vals.push_back(c);
    B = c->ptr;
    b = OperandView{batch, N, K, N * K, K, 1, true};
  }
  FmaGemmParams f;
  f.batch = batch;
  f.M = M;
  f.N = N;
  f.K = K;
  f.a_bs = a.bs;
  f.a_ms = a.fs;
  f.a_ks = a.ks;
  f.b_bs = b.bs;
  f.b_ns = b.fs;
  f.b_ks = b.ks;
  launch_fma_gemm(dev->stream(), f, A, B, out, lt.dtype, ot.dtype);
}

// A dot whose result only feeds `add(dot, x)`: out = x + round(dot) as the
// one-pass GEMV's epilogue, or, when that kernel does not apply to these
// buffers, the dot into a temporary followed by the elementwise add.
void run_dot_residual(Device* dev, const Program& prog, const Op& op, std::vector<MemRef>& vals, int add, int out) {
  const TensorType& lt = prog.type(op.operands[0]);
  const TensorType& rt = prog.type(op.operands[1]);
  const TensorType& ot = prog.type(op.results[0]);
  const void* A = vals[op.operands[0]]->ptr;
  const void* W = vals[op.operands[1]]->ptr;
  const bool ok = lt.rank() == 2 && rt.rank() == 2 && op.lhs_batch.empty() && op.lhs_contract == Dims{1} &&
                  op.rhs_contract == Dims{0} && (lt.dtype == DType::kBF16 || lt.dtype == DType::kF16) &&
                  rt.dtype == lt.dtype && ot.dtype == lt.dtype && lt.dims[1] % 8 == 0 && rt.dims[1] % 8 == 0 &&
                  aligned16(W) && rt.dims[1] < (int64_t(1) << 30) &&
                  gemv_wide_fits(static_cast<int>(lt.dims[0]), static_cast<int>(lt.dims[1]), single_wide_tiles(rt.dims[1]));
  if (ok) {
    GemvGroup g;
    g.count = 1;
    g.M = static_cast<int>(lt.dims[0]);
    g.K = static_cast<int>(lt.dims[1]);
    g.ldx = lt.dims[1];
    g.out_kind = lt.dtype == DType::kF16 ? 1 : 0;
    g.m[0].W = W;
    g.m[0].Y = vals[out]->ptr;
    g.m[0].add = vals[add]->ptr;
    g.m[0].N = static_cast<int>(rt.dims[1]);
    g.m[0].ldw = rt.dims[1];
    g.m[0].ldy = rt.dims[1];
    launch_gemv_wide(dev->stream(), g, A, lt.dtype == DType::kF16);
    return;
  }
  vals[op.results[0]] = dev->allocate(ot.bytes());
  run_dot_general(dev, prog, op, vals);
  launch_add(dev->stream(), vals[add]->ptr, vals[op.results[0]]->ptr, vals[out]->ptr, ot.elements(), ot.dtype);
  vals[op.results[0]].reset();
}

// A dot group (planner: dots sharing one LHS): one gemv_wide launch when
// every member is a decode-shaped product over the same X with an
// N-contiguous weight; otherwise the members run one by one.
void run_dot_group(Device* dev, const Program& prog, const std::vector<int>& ops, std::vector<MemRef>& vals) {
  GemvGroup g;
  bool ok = ops.size() >= 1 && ops.size() <= static_cast<size_t>(kMaxGemvMembers);
  const void* X = nullptr;
  DType in_t = DType::kInvalid;
  int tiles = 0;
  for (size_t i = 0; i < ops.size() && ok; ++i) {
    const Op& op = prog.ops.at(ops[i]);
    const TensorType& lt = prog.type(op.operands[0]);
    const TensorType& rt = prog.type(op.operands[1]);
    const TensorType& ot = prog.type(op.results[0]);
    ok = op.kind == OpKind::kDotGeneral && lt.rank() == 2 && rt.rank() == 2 && op.lhs_batch.empty() &&
         op.lhs_contract == Dims{1} && op.rhs_contract == Dims{0} && (lt.dtype == DType::kBF16 || lt.dtype == DType::kF16) &&
         rt.dtype == lt.dtype && (ot.dtype == lt.dtype || ot.dtype == DType::kF32);
    if (!ok) break;
    const int64_t M = lt.dims[0], K = lt.dims[1], N = rt.dims[1];
    const int out_kind = ot.dtype == DType::kBF16 ? 0 : (ot.dtype == DType::kF16 ? 1 : 2);
    const void* A = vals[op.operands[0]]->ptr;
    const void* W = vals[op.operands[1]]->ptr;
    ok = M >= 1 && M <= 4 && K % 8 == 0 && N % 8 == 0 && aligned16(A) && aligned16(W) && N < (int64_t(1) << 30) &&
         M * K <= kGemvWideMaxX;
    if (i == 0) {
      X = A;
      in_t = lt.dtype;
      g.M = static_cast<int>(M);
      g.K = static_cast<int>(K);
      g.ldx = K;
      g.out_kind = out_kind;
    } else {
      ok = ok && A == X && lt.dtype == in_t && g.M == M && g.K == K && g.out_kind == out_kind;
    }
    if (!ok) break;
    GemvMember& m = g.m[i];
    m.W = W;
    m.Y = vals[op.results[0]]->ptr;
    m.N = static_cast<int>(N);
    m.ldw = N;
    m.ldy = N;
  }
  if (ok) {
    g.count = static_cast<int>(ops.size());
    tiles = gemv_wide_tiles(g);
  }
  if (ok && gemv_wide_fits(g.M, g.K, tiles)) {
    launch_gemv_wide(dev->stream(), g, X, in_t == DType::kF16);
    return;
  }
  for (int oi : ops) run_dot_general(dev, prog, prog.ops.at(oi), vals);
}

}  // namespace pjrtx
