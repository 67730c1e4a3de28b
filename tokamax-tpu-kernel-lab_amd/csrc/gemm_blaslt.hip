// Plain dense projections of the layer (x @ W with W stored (N, K), no ragged
// groups, no fused epilogue: the down- and up-projection GEMMs of
// ref.py:634-655 / ref.py:430) on hipBLASLt, the ROCm library GEMM.  The
// grouped expert GEMMs, the MXFP4 paths and every fused epilogue stay on the
// hand-written kernels.
//
// Row-major out (M, N) = x (M, K) @ W^T is the column-major product
// out^T (N x M) = W (N x K, i.e. col-major K x N transposed) * x^T (col-major
// K x M): A = W with op T, B = x with op N, D ld = N.  f32 accumulation and
// scale; no workspace (the heuristic is asked only for algorithms that need
// none), so the call allocates nothing.  One handle per device and one plan
// (descriptors + heuristic algorithm) per shape / dtype combination, created
// on first use and kept until the process ends.
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "lmoe_common.h"

namespace lmoe {
namespace blaslt {
namespace {

struct Plan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
  hipblasLtMatmulAlgo_t algo{};
};

using Key = std::tuple<int, int64_t, int64_t, int64_t, int, int, int>;  // dev, M, N, K, x, w, out dtypes

std::mutex g_mu;
std::map<int, hipblasLtHandle_t> g_handles;
std::map<Key, Plan> g_plans;

hipDataType dt_of(int dtype) { return dtype == LMOE_BF16 ? HIP_R_16BF : HIP_R_32F; }

// Returns 0 and the plan, or a negative status with the message set.
int get_plan(const Key& key, hipblasLtHandle_t* handle, const Plan** plan) {
  std::lock_guard<std::mutex> lock(g_mu);
  const int dev = std::get<0>(key);
  auto hit = g_handles.find(dev);
  if (hit == g_handles.end()) {
    hipblasLtHandle_t h = nullptr;
    if (hipblasLtCreate(&h) != HIPBLAS_STATUS_SUCCESS) return fail(LMOE_ERR_HIP, "dense_blaslt: hipblasLtCreate failed");
    hit = g_handles.emplace(dev, h).first;
  }
  *handle = hit->second;
  auto pit = g_plans.find(key);
  if (pit != g_plans.end()) {
    *plan = &pit->second;
    return LMOE_OK;
  }
  const int64_t M = std::get<1>(key), N = std::get<2>(key), K = std::get<3>(key);
  Plan p;
  bool ok = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS;
  const hipblasOperation_t opT = HIPBLAS_OP_T, opN = HIPBLAS_OP_N;
  ok = ok && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opT, sizeof(opT)) ==
                 HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opN, sizeof(opN)) ==
                 HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatrixLayoutCreate(&p.a, dt_of(std::get<5>(key)), K, N, K) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatrixLayoutCreate(&p.b, dt_of(std::get<4>(key)), K, M, K) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatrixLayoutCreate(&p.d, dt_of(std::get<6>(key)), N, M, N) == HIPBLAS_STATUS_SUCCESS;
  hipblasLtMatmulPreference_t pref = nullptr;
  ok = ok && hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS;
  const uint64_t no_ws = 0;
  ok = ok && hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &no_ws,
                                                   sizeof(no_ws)) == HIPBLAS_STATUS_SUCCESS;
  // Always the heuristic's first candidate: it measured fastest among the
  // first nine at the layer's shapes, and a later candidate at those shapes
  // faulted the GPU, so no override is offered.
  constexpr int kMaxAlgos = 16;
  hipblasLtMatmulHeuristicResult_t res[kMaxAlgos] = {};
  int found = 0;
  ok = ok && hipblasLtMatmulAlgoGetHeuristic(*handle, p.desc, p.a, p.b, p.d, p.d, pref, kMaxAlgos, res, &found) ==
                 HIPBLAS_STATUS_SUCCESS;
  if (pref) hipblasLtMatmulPreferenceDestroy(pref);
  const int pick = 0;
  if (!ok || found < 1 || res[pick].state != HIPBLAS_STATUS_SUCCESS) {
    if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
    for (auto l : {p.a, p.b, p.d})
      if (l) hipblasLtMatrixLayoutDestroy(l);
    return fail(LMOE_ERR_UNSUPPORTED, "dense_blaslt: no hipBLASLt algorithm for M=%lld N=%lld K=%lld",
                (long long)M, (long long)N, (long long)K);
  }
  p.algo = res[pick].algo;
  *plan = &g_plans.emplace(key, p).first->second;
  return LMOE_OK;
}

}  // namespace
}  // namespace blaslt
}  // namespace lmoe

extern "C" int lmoe_dense_blaslt(const void* x, int x_dtype, const void* w_nk, int w_dtype, int64_t M, int64_t K,
                                 int64_t N, void* out, int out_dtype, void* stream) {
  using namespace lmoe;
  LMOE_CHECK_ARG(M >= 0 && K > 0 && N > 0, "dense_blaslt: bad sizes M=%lld K=%lld N=%lld", (long long)M,
                 (long long)K, (long long)N);
  LMOE_CHECK_ARG(valid_dtype(x_dtype) && valid_dtype(w_dtype) && valid_dtype(out_dtype), "dense_blaslt: bad dtype");
  LMOE_CHECK_SUPPORTED(x_dtype == w_dtype, "dense_blaslt: x and W dtypes differ");
  LMOE_CHECK_SUPPORTED(extent_ok({M, K}) && extent_ok({N, K}) && extent_ok({M, N}),
                       "dense_blaslt: sizes beyond device memory");
  if (M == 0) return LMOE_OK;
  LMOE_CHECK_ARG(x && w_nk && out, "dense_blaslt: null pointer");
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(LMOE_ERR_HIP, "dense_blaslt: hipGetDevice");
  hipblasLtHandle_t handle = nullptr;
  const blaslt::Plan* plan = nullptr;
  const int rc = blaslt::get_plan(blaslt::Key{dev, M, N, K, x_dtype, w_dtype, out_dtype}, &handle, &plan);
  if (rc != LMOE_OK) return rc;
  const float alpha = 1.0f, beta = 0.0f;
  const hipblasStatus_t st =
      hipblasLtMatmul(handle, plan->desc, &alpha, w_nk, plan->a, x, plan->b, &beta, out, plan->d, out, plan->d,
                      &plan->algo, nullptr, 0, static_cast<hipStream_t>(stream));
  if (st != HIPBLAS_STATUS_SUCCESS) return fail(LMOE_ERR_HIP, "dense_blaslt: hipblasLtMatmul status %d", (int)st);
  return LMOE_OK;
}
