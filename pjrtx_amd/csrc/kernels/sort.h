// Row sorts for stablehlo.sort and chlo.top_k (launchers of kernels/sort.hip).
//
// Every element of a row becomes one 64-bit sort word: an order-preserving
// 32-bit image of its key in the high half and its position in the row in
// the low half. All words of a row are distinct, so sorting them ascending
// gives the one order a stable sort gives (equal keys keep their positions'
// order), whatever network sorts them. Bitonic networks do: in LDS for rows
// up to kSortBlock words, with global compare-exchange passes between LDS
// passes above that. A row's results are gathered from the operands by the
// positions in the sorted words, so keys and payloads come back bit for bit.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace pjrtx {

constexpr int kSortBlock = 4096;       // words sorted per LDS pass (32 KiB)
constexpr int kSortMaxOperands = 8;    // operands gathered by one output launch

// How operand 0's bits map to the ascending 32-bit image.
enum SortKeyClass : int {
  kSortKeyUnsigned = 0,   // unsigned ints and pred
  kSortKeySigned = 1,     // two's complement ints
  kSortKeyTotal = 2,      // IEEE totalOrder: -NaN < -inf < ... < -0 < +0 < ... < +inf < +NaN
  kSortKeyFloat = 3,      // FLOAT compare: -0 == +0, every NaN equal and after +inf
};

// A set of rows: row r = outer * inner + j holds the elements at
// outer * n * inner + i * inner + j for i in [0, n).
struct SortRows {
  int64_t rows = 0;
  int64_t n = 0;
  int64_t inner = 1;
  int key_bits = 32;      // 8, 16 or 32
  int key_class = kSortKeyTotal;
  int descending = 0;     // image inverted: largest key first, ties still in position order
  uint32_t inf_bits = 0;  // float keys: the bits of +inf (a larger magnitude is a NaN)
};

// Results: out_j[outer, i, j] = operand_j[outer, pos_i, j] for i < out_n.
struct SortGather {
  int count = 0;
  const void* src[kSortMaxOperands] = {};
  void* dst[kSortMaxOperands] = {};
  int elem_bytes[kSortMaxOperands] = {};
  int64_t out_n = 0;      // n for sort, k for top_k
  void* index_dst = nullptr;  // optional s32 output of the positions (top_k indices)
};

// Bytes of device scratch sort_rows needs for these rows and out_n.
size_t sort_scratch_bytes(const SortRows& r, int64_t out_n);

// Sorts every row of operand 0 (`keys`) and writes the first `g.out_n`
// positions of each row's order through `g`. out_n == n is a full sort;
// a smaller out_n keeps only the row's first out_n (top_k with
// descending = 1). `scratch` holds sort_scratch_bytes bytes.
void sort_rows(hipStream_t s, const SortRows& r, const void* keys, const SortGather& g, void* scratch);

}  // namespace pjrtx
