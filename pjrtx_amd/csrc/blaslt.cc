// Plain large GEMMs on hipBLASLt. Row-major C = A * B is the column-major
// product C^T = B^T * A^T, so hipBLASLt's "A" is this build's B and its "B"
// is this build's A. Algorithms are restricted to ones needing no
// workspace: those launch no memset and no split-K reduction, so a call
// captures cleanly into a hipGraph, and every one measured here returns the
// same bits on every call. The heuristic's first choice is cached per
// problem (shape, strides, types).
#include "blaslt.h"

#include <hipblaslt/hipblaslt.h>

#include <map>
#include <memory>
#include <mutex>
#include <vector>

#include "common.h"

namespace pjrtx {
namespace {

struct LtPlan {
  hipblasLtMatmulDesc_t op = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  bool ok = false;
};

struct State {
  std::mutex mu;
  hipblasLtHandle_t handle = nullptr;
  bool unavailable = false;
  std::map<std::vector<int64_t>, LtPlan> plans;
};

State& state_for(int ordinal) {
  static std::mutex mu;
  static std::map<int, std::unique_ptr<State>> states;
  std::lock_guard<std::mutex> lk(mu);
  auto& s = states[ordinal];
  if (!s) s = std::make_unique<State>();
  return *s;
}

bool ok(hipblasStatus_t s) { return s == HIPBLAS_STATUS_SUCCESS; }

bool layout(hipblasLtMatrixLayout_t* l, hipDataType t, int64_t rows, int64_t cols, int64_t ld, int batch, int64_t stride) {
  if (!ok(hipblasLtMatrixLayoutCreate(l, t, static_cast<uint64_t>(rows), static_cast<uint64_t>(cols), ld))) return false;
  if (batch == 1) return true;
  const int32_t n = batch;
  return ok(hipblasLtMatrixLayoutSetAttribute(*l, HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT, &n, sizeof(n))) &&
         ok(hipblasLtMatrixLayoutSetAttribute(*l, HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET, &stride, sizeof(stride)));
}

LtPlan make_plan(hipblasLtHandle_t h, const GemmParams& g, bool f16, bool b_kmajor, int out_bytes) {
  LtPlan p;
  const hipDataType in = f16 ? HIP_R_16F : HIP_R_16BF;
  const hipDataType out = out_bytes == 4 ? HIP_R_32F : in;
  if (!ok(hipblasLtMatmulDescCreate(&p.op, HIPBLAS_COMPUTE_32F, HIP_R_32F))) return p;
  const hipblasOperation_t ta = b_kmajor ? HIPBLAS_OP_T : HIPBLAS_OP_N, tb = HIPBLAS_OP_N;
  if (!ok(hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta))) ||
      !ok(hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb))))
    return p;
  // hipBLASLt A = this B: [K][N] row-major is column-major N x K; [N][K]
  // row-major is column-major K x N, used transposed.
  const bool la_ok = b_kmajor ? layout(&p.la, in, g.K, g.N, g.ldb, g.batch, g.b_batch_stride)
                              : layout(&p.la, in, g.N, g.K, g.ldb, g.batch, g.b_batch_stride);
  if (!la_ok || !layout(&p.lb, in, g.K, g.M, g.lda, g.batch, g.a_batch_stride) ||
      !layout(&p.lc, out, g.N, g.M, g.ldc, g.batch, static_cast<int64_t>(g.M) * g.ldc))
    return p;
  hipblasLtMatmulPreference_t pref = nullptr;
  if (!ok(hipblasLtMatmulPreferenceCreate(&pref))) return p;
  const uint64_t no_workspace = 0;
  hipblasLtMatmulHeuristicResult_t res[1];
  int n = 0;
  const bool found =
      ok(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &no_workspace,
                                               sizeof(no_workspace))) &&
      ok(hipblasLtMatmulAlgoGetHeuristic(h, p.op, p.la, p.lb, p.lc, p.lc, pref, 1, res, &n)) && n >= 1 &&
      ok(res[0].state) && res[0].workspaceSize == 0;
  (void)hipblasLtMatmulPreferenceDestroy(pref);
  if (found) {
    p.algo = res[0].algo;
    p.ok = true;
  }
  return p;
}

}  // namespace

bool blaslt_wanted(const GemmParams& g) {
  // Opt-in (PJRTX_BLASLT=1): by default every product runs on the own MFMA
  // kernels; the library route stays for A/B measurements.
  if (env_int("PJRTX_BLASLT", 0) == 0) return false;
  // The allocation-free execute never enters the library (its handle and
  // heuristics allocate).
  if (thread_arena()) return false;
  // Products that fill the GPU with 256 x 256 tiles: the size where the
  // library's tuned kernels were measured ahead of the own ones.
  const int64_t tiles = static_cast<int64_t>((g.M + 255) / 256) * ((g.N + 255) / 256) * g.batch;
  return g.M >= 256 && g.N >= 256 && g.K >= 256 && tiles >= 256;
}

bool blaslt_gemm(Device* dev, const GemmParams& g, const void* A, const void* B, void* C, bool f16, bool b_kmajor,
                 int out_bytes) {
  State& st = state_for(dev->ordinal());
  std::lock_guard<std::mutex> lk(st.mu);
  if (st.unavailable) return false;
  dev->make_current();
  if (!st.handle && !ok(hipblasLtCreate(&st.handle))) {
    st.unavailable = true;
    return false;
  }
  const std::vector<int64_t> key = {g.batch, g.M,  g.N,       g.K,      g.lda,    g.ldb, g.ldc, g.a_batch_stride,
                                    g.b_batch_stride, f16 ? 1 : 0, b_kmajor ? 1 : 0, out_bytes};
  auto it = st.plans.find(key);
  if (it == st.plans.end()) it = st.plans.emplace(key, make_plan(st.handle, g, f16, b_kmajor, out_bytes)).first;
  const LtPlan& p = it->second;
  if (!p.ok) return false;
  const float alpha = 1.f, beta = 0.f;
  return ok(hipblasLtMatmul(st.handle, p.op, &alpha, B, p.la, A, p.lb, &beta, C, p.lc, C, p.lc, &p.algo, nullptr, 0,
                            dev->stream()));
}

}  // namespace pjrtx
