// Device memory of the allocation-free execute (pjrtx_executable_execute_noalloc):
// one fixed block per GPU, a file-scope __device__ array, from which that
// entry point carves every intermediate value and every kernel scratch
// block (split-reduction partials, split-K partials, sort keys, scatter
// segments) instead of the caching allocator.
//
// The array's host-side name is not a device address. Its address on a GPU
// is looked up once per device with hipGetSymbolAddress (with that device
// current) and only that address is handed to kernels and copies.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>

#include "common.h"
#include "kernels/noalloc.h"

namespace pjrtx {

namespace {

static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

__global__ void __launch_bounds__(256) noalloc_zero(uint4* __restrict__ p, size_t n16) {
  const size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n16) p[i] = make_uint4(0u, 0u, 0u, 0u);
}

std::mutex g_mu;
std::map<int, void*> g_ptr;  // device ordinal -> address of `scratch` on it

}  // namespace

void* noalloc_scratch(int device) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_ptr.find(device);
  if (it != g_ptr.end()) return it->second;
  int cur = -1;
  PJRTX_CHECK(hipGetDevice(&cur) == hipSuccess && cur == device, Code::kInternal,
              "noalloc_scratch: the device must be current");
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || ptr == nullptr) {
    (void)hipGetLastError();
    fail(Code::kInternal, strformat("hipGetSymbolAddress(noalloc scratch) failed on device %d: %s", device,
                                    hipGetErrorString(e)));
  }
  g_ptr[device] = ptr;
  return ptr;
}

void launch_noalloc_zero(hipStream_t s, void* p, size_t bytes) {
  PJRTX_CHECK(reinterpret_cast<uintptr_t>(p) % 16 == 0 && bytes % 16 == 0, Code::kInternal,
              "noalloc zero: block must be 16-byte aligned and sized");
  const size_t n16 = bytes / 16;
  if (n16 == 0) return;
  hipLaunchKernelGGL(noalloc_zero, dim3(static_cast<unsigned>((n16 + 255) / 256)), dim3(256), 0, s,
                     static_cast<uint4*>(p), n16);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) fail(Code::kInternal, strformat("noalloc_zero launch failed: %s", hipGetErrorString(e)));
}

}  // namespace pjrtx
