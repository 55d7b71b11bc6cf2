// stablehlo.sort and chlo.top_k as library steps (kernels/sort.hip).
//
// The reference lowers sort with one operand (keys) or two (keys, values)
// and an LT/LE/GT/GE comparator on the keys (reference:
// src/backend/mlx_metal/lowering_indexing.zig:290-320), and top_k with a
// static k along the last dimension (:323-356). Here a sort takes up to
// kSortMaxOperands operands, all permuted by the order of operand 0; the
// comparator must be one compare of operand 0's block arguments. FLOAT
// compares order every NaN after +inf and -0 with +0; TOTALORDER compares
// use IEEE totalOrder. top_k orders floats by totalOrder, largest first,
// equal values by position (XLA's TopK).
#include "sort_op.h"

#include "kernels/sort.h"
#include "runtime.h"

namespace pjrtx {

namespace {

struct SortSpec {
  SortRows rows;
  int64_t out_n = 0;
};

void key_class_of(DType t, CmpType ct, SortRows* r) {
  const size_t bytes = dtype_size(t);
  PJRTX_CHECK(bytes == 1 || bytes == 2 || bytes == 4, Code::kUnimplemented,
              std::string("sort: keys of type ") + dtype_name(t) + " are not supported (8, 16 or 32 bits only)");
  r->key_bits = static_cast<int>(bytes * 8);
  if (dtype_is_float(t)) {
    PJRTX_CHECK(t == DType::kF32 || t == DType::kF16 || t == DType::kBF16, Code::kUnimplemented,
                std::string("sort: float keys of type ") + dtype_name(t) + " are not supported");
    r->key_class = ct == CmpType::kTotalOrder ? kSortKeyTotal : kSortKeyFloat;
    r->inf_bits = t == DType::kF32 ? 0x7f800000u : (t == DType::kF16 ? 0x7c00u : 0x7f80u);
  } else if (dtype_is_signed_int(t)) {
    r->key_class = ct == CmpType::kUnsigned ? kSortKeyUnsigned : kSortKeySigned;
  } else {
    r->key_class = kSortKeyUnsigned;
  }
}

SortSpec spec_of(const Program& prog, const Op& op) {
  SortSpec sp;
  const TensorType& x = prog.type(op.operands.at(0));
  PJRTX_CHECK(x.rank() >= 1, Code::kInvalidArgument, "sort: operand must have rank >= 1");
  if (op.kind == OpKind::kTopK) {
    PJRTX_CHECK(op.operands.size() == 1 && op.results.size() == 2 && !op.sizes.empty(), Code::kInvalidArgument,
                "top_k: one operand, two results and a static k");
    const int64_t k = op.sizes[0];
    PJRTX_CHECK(k >= 0 && k <= x.dims.back(), Code::kInvalidArgument, "top_k: k outside [0, last dim]");
    PJRTX_CHECK(prog.type(op.results[1]).dtype == DType::kS32, Code::kUnimplemented, "top_k: indices must be s32");
    key_class_of(x.dtype, dtype_is_float(x.dtype) ? CmpType::kTotalOrder : CmpType::kNotSet, &sp.rows);
    sp.rows.descending = 1;
    sp.rows.n = x.dims.back();
    sp.rows.inner = 1;
    sp.rows.rows = x.elements() / std::max<int64_t>(sp.rows.n, 1);
    if (sp.rows.n == 0) sp.rows.rows = 0;
    sp.out_n = k;
    return sp;
  }
  const size_t n_ops = op.operands.size();
  PJRTX_CHECK(n_ops >= 1 && n_ops <= static_cast<size_t>(kSortMaxOperands) && op.results.size() == n_ops,
              Code::kUnimplemented, strformat("sort: %zu operands (1 to %d supported)", n_ops, kSortMaxOperands));
  for (size_t i = 1; i < n_ops; ++i)
    PJRTX_CHECK(prog.type(op.operands[i]).dims == x.dims, Code::kInvalidArgument, "sort: operand shapes differ");
  const int64_t dim = op.dim < 0 ? x.rank() - 1 : op.dim;
  PJRTX_CHECK(dim >= 0 && dim < x.rank(), Code::kInvalidArgument, "sort: dimension out of range");
  // Comparator: return compare(dir, lhs_0, rhs_0) (or with the two swapped).
  PJRTX_CHECK(op.regions.size() == 1, Code::kInvalidArgument, "sort: expected one comparator region");
  const Region& r = op.regions[0];
  PJRTX_CHECK(r.params.size() == 2 * n_ops, Code::kInvalidArgument, "sort: comparator takes two arguments per operand");
  const Op* cmp = nullptr;
  for (const Op& b : r.ops) {
    if (b.kind == OpKind::kReturn) {
      PJRTX_CHECK(cmp && b.operands.size() == 1 && b.operands[0] == cmp->results[0], Code::kUnimplemented,
                  "sort: comparator must return one compare of operand 0's arguments");
    } else {
      PJRTX_CHECK(b.kind == OpKind::kCompare && !cmp, Code::kUnimplemented,
                  std::string("sort: unsupported comparator op ") + op_kind_name(b.kind) +
                      " (one compare of the first operand's arguments is supported)");
      cmp = &b;
    }
  }
  PJRTX_CHECK(cmp != nullptr, Code::kUnimplemented, "sort: empty comparator");
  const int a = r.params[0], bb = r.params[1];
  bool swapped;
  if (cmp->operands == std::vector<int>{a, bb}) swapped = false;
  else if (cmp->operands == std::vector<int>{bb, a}) swapped = true;
  else fail(Code::kUnimplemented, "sort: the comparator must compare the first operand's two arguments");
  bool desc;
  switch (cmp->cmp_dir) {
    case CmpDir::kLT: case CmpDir::kLE: desc = false; break;
    case CmpDir::kGT: case CmpDir::kGE: desc = true; break;
    default: fail(Code::kUnimplemented, "sort: comparator direction must be LT, LE, GT or GE");
  }
  key_class_of(x.dtype, cmp->cmp_type, &sp.rows);
  sp.rows.descending = desc != swapped;
  int64_t outer = 1, inner = 1;
  for (int64_t d = 0; d < dim; ++d) outer *= x.dims[d];
  for (int64_t d = dim + 1; d < x.rank(); ++d) inner *= x.dims[d];
  sp.rows.n = x.dims[dim];
  sp.rows.inner = inner;
  sp.rows.rows = sp.rows.n == 0 ? 0 : outer * inner;
  sp.out_n = sp.rows.n;
  return sp;
}

}  // namespace

void check_sort_supported(const Program& prog, const Op& op) { (void)spec_of(prog, op); }

void run_sort(Device* dev, const Program& prog, const Op& op, std::vector<MemRef>& vals) {
  const SortSpec sp = spec_of(prog, op);
  SortGather g;
  g.out_n = sp.out_n;
  if (op.kind == OpKind::kTopK) {
    g.count = 1;
    g.src[0] = vals[op.operands[0]]->ptr;
    g.dst[0] = vals[op.results[0]]->ptr;
    g.elem_bytes[0] = static_cast<int>(dtype_size(prog.type(op.operands[0]).dtype));
    g.index_dst = vals[op.results[1]]->ptr;
  } else {
    g.count = static_cast<int>(op.operands.size());
    for (int i = 0; i < g.count; ++i) {
      g.src[i] = vals[op.operands[i]]->ptr;
      g.dst[i] = vals[op.results[i]]->ptr;
      g.elem_bytes[i] = static_cast<int>(dtype_size(prog.type(op.operands[i]).dtype));
    }
  }
  const size_t scratch_bytes = sort_scratch_bytes(sp.rows, sp.out_n);
  MemRef scratch = scratch_bytes ? dev->allocate(scratch_bytes) : MemRef();
  sort_rows(dev->stream(), sp.rows, vals[op.operands[0]]->ptr, g, scratch ? scratch->ptr : nullptr);
}

}  // namespace pjrtx
