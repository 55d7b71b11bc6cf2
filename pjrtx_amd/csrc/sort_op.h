// stablehlo.sort / chlo.top_k library steps.
#pragma once

#include <vector>

#include "ir.h"
#include "runtime.h"

namespace pjrtx {

// Fails with UNIMPLEMENTED / INVALID_ARGUMENT when the op (its comparator,
// operand count, key type or k) is outside what run_sort handles.
void check_sort_supported(const Program& prog, const Op& op);

// Writes the op's results (allocated by the caller) on the device's stream.
void run_sort(Device* dev, const Program& prog, const Op& op, std::vector<MemRef>& vals);

}  // namespace pjrtx
