// Calibration kernels: the matrix-core throughput this GPU sustains, so that
// MFMA-bound roofline fractions can be quoted against a measured peak beside
// the published one. Not part of any plan.
#include <hip/hip_runtime.h>

#include "library.h"

namespace pjrtx {
namespace {

typedef __bf16 cal_bf16x8 __attribute__((ext_vector_type(8)));
typedef float cal_f32x4 __attribute__((ext_vector_type(4)));
typedef float cal_f32x16 __attribute__((ext_vector_type(16)));

// Every wave issues `iters` rounds of kChains independent MFMAs (enough in
// flight to cover the instruction's latency); the accumulators are summed
// and stored so that none of the work is dead.
template <int kShape>
__global__ void __launch_bounds__(256) mfma_peak_kernel(int iters, float* __restrict__ out) {
  cal_bf16x8 a, b;
  for (int i = 0; i < 8; ++i) {
    a[i] = static_cast<__bf16>(0.001f * static_cast<float>((threadIdx.x + i) & 7));
    b[i] = static_cast<__bf16>(0.002f * static_cast<float>((threadIdx.x * 3 + i) & 7));
  }
  float s = 0.f;
  if constexpr (kShape == 0) {  // v_mfma_f32_16x16x32_bf16, eight named chains
    cal_f32x4 c0{}, c1{}, c2{}, c3{}, c4{}, c5{}, c6{}, c7{};
    for (int it = 0; it < iters; ++it) {
      c0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c0, 0, 0, 0);
      c1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c1, 0, 0, 0);
      c2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c2, 0, 0, 0);
      c3 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c3, 0, 0, 0);
      c4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c4, 0, 0, 0);
      c5 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c5, 0, 0, 0);
      c6 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c6, 0, 0, 0);
      c7 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c7, 0, 0, 0);
    }
    const cal_f32x4 t = c0 + c1 + c2 + c3 + c4 + c5 + c6 + c7;
    s = t[0] + t[1] + t[2] + t[3];
  } else {  // v_mfma_f32_32x32x16_bf16
    constexpr int kChains = 4;
    cal_f32x16 acc[kChains];
    for (int c = 0; c < kChains; ++c)
      for (int e = 0; e < 16; ++e) acc[c][e] = 0.f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int c = 0; c < kChains; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[c], 0, 0, 0);
    }
    for (int c = 0; c < kChains; ++c)
      for (int e = 0; e < 16; ++e) s += acc[c][e];
  }
  out[static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x] = s;
}

void cal_check(hipError_t e, const char* what) {
  if (e != hipSuccess) fail(Code::kInternal, strformat("%s failed: %s", what, hipGetErrorString(e)));
}

}  // namespace

double measure_mfma_peak_tflops(hipStream_t s, int shape, int compute_units) {
  PJRTX_CHECK(shape == 0 || shape == 1, Code::kInvalidArgument, "mfma peak: shape is 0 (16x16x32) or 1 (32x32x16)");
  PJRTX_CHECK(compute_units > 0 && compute_units <= 4096, Code::kInvalidArgument, "mfma peak: bad CU count");
  // Two workgroups of four waves per CU: two waves per SIMD.
  const int blocks = compute_units * 2;
  const int iters = 8192;
  const double flops_per_wave = shape == 0 ? 8.0 * iters * (2.0 * 16 * 16 * 32) : 4.0 * iters * (2.0 * 32 * 32 * 16);
  const double flops = flops_per_wave * blocks * 4;
  float* out = nullptr;
  cal_check(hipMalloc(&out, static_cast<size_t>(blocks) * 256 * sizeof(float)), "hipMalloc(mfma peak)");
  hipEvent_t e0 = nullptr, e1 = nullptr;
  double best_ms = 1e30;
  hipError_t err = hipEventCreate(&e0);
  if (err == hipSuccess) err = hipEventCreate(&e1);
  for (int rep = 0; rep < 6 && err == hipSuccess; ++rep) {
    err = hipEventRecord(e0, s);
    if (shape == 0)
      hipLaunchKernelGGL(mfma_peak_kernel<0>, dim3(blocks), dim3(256), 0, s, iters, out);
    else
      hipLaunchKernelGGL(mfma_peak_kernel<1>, dim3(blocks), dim3(256), 0, s, iters, out);
    if (err == hipSuccess) err = hipGetLastError();
    if (err == hipSuccess) err = hipEventRecord(e1, s);
    if (err == hipSuccess) err = hipEventSynchronize(e1);
    float ms = 0.f;
    if (err == hipSuccess) err = hipEventElapsedTime(&ms, e0, e1);
    if (err == hipSuccess && rep > 0 && ms < best_ms) best_ms = ms;  // the first run warms up
  }
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  (void)hipFree(out);
  cal_check(err, "mfma peak run");
  return flops / (best_ms * 1e-3) / 1e12;
}

}  // namespace pjrtx
