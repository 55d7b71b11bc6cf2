// Fixed per-GPU device block of the allocation-free execute
// (kernels/noalloc.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>

namespace pjrtx {

// Size of the block every GPU holds for the allocation-free execute; a call
// whose intermediates and scratch need more fails with RESOURCE_EXHAUSTED.
constexpr size_t kNoallocScratchBytes = size_t(64) << 20;

// Device address of the block on `device`, looked up on the first call for
// that device (which must be current) and kept afterwards.
void* noalloc_scratch(int device);

// Zero-fills `bytes` (a multiple of 16) at 16-byte aligned `p` with a kernel
// on stream `s` (not a memset node, so the call stays capturable).
void launch_noalloc_zero(hipStream_t s, void* p, size_t bytes);

}  // namespace pjrtx
