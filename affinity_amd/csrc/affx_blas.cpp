// Plain bf16 GEMMs through hipBLASLt, for the shared expert's batch form (affx_shared.hip): the
// one place in the library where the work is an ordinary dense GEMM on operands already widened to
// bf16, which the vendor library runs faster than a hand-written kernel would.
//
// Row-major operands map onto the library's column-major convention without copies: A [M][K] with
// row stride lda is the column-major K x M matrix with leading dimension lda taken transposed; B
// [N][K] is the column-major K x N matrix untransposed; D [N][M] (row stride ldd) is the column-
// major M x N result. So D[n][m] = sum_k A[m][k] B[n][k], accumulated in f32.
//
// One library handle per device (created on that device's first call) and one plan per (device,
// shape, strides, beta): the matmul descriptor, the three layouts and the algorithm the library's
// heuristic ranks first among those that need no workspace. The first call for a shape queries the
// heuristic on the host; later calls only enqueue the GEMM on the caller's stream.
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "affx_common.h"

namespace {

struct Plan {
  hipblasLtMatmulDesc_t op = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  bool ok = false;
};

using Key = std::tuple<int, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, int>;

std::mutex g_mu;
std::map<int, hipblasLtHandle_t> g_handles;
std::map<Key, Plan> g_plans;

// (under g_mu) the plan for a shape, resolved on first sight; ok == false when the library has no
// algorithm for it (remembered, so the heuristic is asked once)
Plan* plan_for(const Key& k, hipblasLtHandle_t h) {
  auto it = g_plans.find(k);
  if (it != g_plans.end()) return &it->second;
  Plan p;
  const uint32_t M = std::get<1>(k), N = std::get<2>(k), K = std::get<3>(k);
  const uint32_t lda = std::get<4>(k), ldb = std::get<5>(k), ldd = std::get<6>(k);
  hipblasLtMatmulPreference_t pref = nullptr;
  bool good = hipblasLtMatmulDescCreate(&p.op, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS;
  if (good) {
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    good = hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) ==
               HIPBLAS_STATUS_SUCCESS &&
           hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) ==
               HIPBLAS_STATUS_SUCCESS;
  }
  good = good && hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16BF, K, M, lda) == HIPBLAS_STATUS_SUCCESS;
  good = good && hipblasLtMatrixLayoutCreate(&p.b, HIP_R_16BF, K, N, ldb) == HIPBLAS_STATUS_SUCCESS;
  good = good && hipblasLtMatrixLayoutCreate(&p.d, HIP_R_32F, M, N, ldd) == HIPBLAS_STATUS_SUCCESS;
  good = good && hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS;
  if (good) {
    uint64_t no_ws = 0;
    good = hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &no_ws,
                                                 sizeof(no_ws)) == HIPBLAS_STATUS_SUCCESS;
  }
  if (good) {
    hipblasLtMatmulHeuristicResult_t res{};
    int n = 0;
    good = hipblasLtMatmulAlgoGetHeuristic(h, p.op, p.a, p.b, p.d, p.d, pref, 1, &res, &n) ==
               HIPBLAS_STATUS_SUCCESS &&
           n > 0 && res.state == HIPBLAS_STATUS_SUCCESS && res.workspaceSize == 0;
    if (good) p.algo = res.algo;
  }
  if (pref) hipblasLtMatmulPreferenceDestroy(pref);
  p.ok = good;
  return &g_plans.emplace(k, p).first->second;
}

}  // namespace

namespace affx {

int blas_gemm_bf16_nt(uint32_t M, uint32_t N, uint32_t K, const void* A, uint32_t lda, const void* B, uint32_t ldb,
                      float* D, uint32_t ldd, int beta_one, hipStream_t stream) {
  if (M == 0 || N == 0 || K == 0 || M > 0x7FFFFFFFu || N > 0x7FFFFFFFu || K > 0x7FFFFFFFu || lda < K || ldb < K ||
      ldd < M)
    return set_error(AFFX_ERR_ARG, "blas_gemm_bf16_nt: bad shape");
  int dev = 0;
  int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (rc) return rc;
  hipblasLtHandle_t h = nullptr;
  Plan* p = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_mu);
    auto it = g_handles.find(dev);
    if (it == g_handles.end()) {
      if (hipblasLtCreate(&h) != HIPBLAS_STATUS_SUCCESS)
        return set_error(AFFX_DECLINED, "blas_gemm_bf16_nt: hipblasLtCreate failed on device %d", dev);
      g_handles.emplace(dev, h);
    } else {
      h = it->second;
    }
    p = plan_for(Key(dev, M, N, K, lda, ldb, ldd, beta_one ? 1 : 0), h);
  }
  if (!p->ok)
    return set_error(AFFX_DECLINED, "blas_gemm_bf16_nt: no library algorithm for %u x %u x %u", M, N, K);
  const float alpha = 1.0f, beta = beta_one ? 1.0f : 0.0f;
  const hipblasStatus_t st =
      hipblasLtMatmul(h, p->op, &alpha, A, p->a, B, p->b, &beta, D, p->d, D, p->d, &p->algo, nullptr, 0, stream);
  if (st != HIPBLAS_STATUS_SUCCESS)
    return set_error(AFFX_ERR_HIP, "blas_gemm_bf16_nt: hipblasLtMatmul failed (status %d)", (int)st);
  return check_launch("hipblasLtMatmul");
}

}  // namespace affx
