// Dense fp16 GEMMs through hipBLASLt with the per-problem setup done once.
//
// The step's dense GEMMs (the frozen projections forward and their input gradients) stay on
// hipBLASLt, as the reference keeps them on the vendor BLAS (solution/nf4.py:108-127,
// solution/mlp.py:80-113 through torch.matmul).  What this entry point removes is the host
// cost around each call: torch's path builds the matmul descriptor and four layouts and asks
// for the algorithm on every call (about 19 us of host time per GEMM on the MI355X box, as
// long as the o projection's GEMM runs on the GPU); here the descriptor, the layouts and the
// algorithm of a problem are built on its first call and kept, and a call is one
// hipblasLtMatmul (about 6 us).  The algorithm is the hipBLASLt solution the caller names by
// index (the tuned table's choice), checked against the problem, else hipBLASLt's first
// heuristic choice: with the same solution the result is the one torch.matmul gives, bit for
// bit.
#include <hipblaslt/hipblaslt-ext.hpp>
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>
#include <vector>

#include "soupk_common.hpp"

namespace soupk {
namespace {

// hipBLASLt returned an error (no solution for the problem, or the call failed).
constexpr int kBlasFailed = hipErrorLaunchFailure;

using PlanKey = std::tuple<int, int, int, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t,
                           int64_t, int64_t, int64_t, int, int, int, int, int64_t, int>;

struct LtPlan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  int index = -1;
};

constexpr size_t kMaxPlans = 4096;            // problems kept (all dropped when full)
std::mutex g_mu;                              // guards the maps and a plan's bias attribute
std::map<int, hipblasLtHandle_t> g_handles;   // per device
std::map<PlanKey, LtPlan> g_plans;

hipblasLtMatrixLayout_t make_layout(hipDataType t, int64_t rows, int64_t cols, int64_t ld,
                                    int batch, int64_t stride) {
  hipblasLtMatrixLayout_t l = nullptr;
  if (hipblasLtMatrixLayoutCreate(&l, t, rows, cols, ld) != HIPBLAS_STATUS_SUCCESS) return nullptr;
  if (batch > 1) {
    const int32_t bc = batch;
    if (hipblasLtMatrixLayoutSetAttribute(l, HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT, &bc,
                                          sizeof(bc)) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutSetAttribute(l, HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET,
                                          &stride, sizeof(stride)) != HIPBLAS_STATUS_SUCCESS) {
      hipblasLtMatrixLayoutDestroy(l);
      return nullptr;
    }
  }
  return l;
}

void destroy(LtPlan& p) {
  if (p.a) hipblasLtMatrixLayoutDestroy(p.a);
  if (p.b) hipblasLtMatrixLayoutDestroy(p.b);
  if (p.d) hipblasLtMatrixLayoutDestroy(p.d);
  if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
  p = LtPlan{};
}

// Descriptor, layouts and algorithm of one problem (g_mu held).
int build_plan(hipblasLtHandle_t h, int ta, int tb, int64_t m, int64_t n, int64_t k,
               int64_t lda, int64_t sa, int64_t ldb, int64_t sb, int64_t ldd, int64_t sd,
               int d_f32, int batch, bool bias, bool accumulate, int algo_index,
               int64_t ws_bytes, LtPlan& p) {
  if (hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS)
    return kBlasFailed;
  const hipblasOperation_t oa = ta ? HIPBLAS_OP_T : HIPBLAS_OP_N;
  const hipblasOperation_t ob = tb ? HIPBLAS_OP_T : HIPBLAS_OP_N;
  if (hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &oa, sizeof(oa)) ||
      hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &ob, sizeof(ob)))
    return kBlasFailed;
  if (bias) {
    const hipblasLtEpilogue_t ep = HIPBLASLT_EPILOGUE_BIAS;
    const int32_t bt = HIP_R_16F;
    if (hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &ep, sizeof(ep)) ||
        hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt,
                                        sizeof(bt)))
      return kBlasFailed;
  }
  const hipDataType dt = d_f32 ? HIP_R_32F : HIP_R_16F;
  p.a = make_layout(HIP_R_16F, ta ? k : m, ta ? m : k, lda, batch, sa);
  p.b = make_layout(HIP_R_16F, tb ? n : k, tb ? k : n, ldb, batch, sb);
  p.d = make_layout(dt, m, n, ldd, batch, sd);
  if (!p.a || !p.b || !p.d) return kBlasFailed;
  const float one = 1.f, beta = accumulate ? 1.f : 0.f;
  if (algo_index >= 0) {
    std::vector<int> idx{algo_index};
    std::vector<hipblasLtMatmulHeuristicResult_t> res;
    size_t need = 0;
    if (hipblaslt_ext::getAlgosFromIndex(h, idx, res) == HIPBLAS_STATUS_SUCCESS && !res.empty() &&
        hipblaslt_ext::matmulIsAlgoSupported(h, p.desc, &one, p.a, p.b, &beta, p.d, p.d,
                                             res[0].algo, need) == HIPBLAS_STATUS_SUCCESS &&
        static_cast<int64_t>(need) <= ws_bytes) {
      p.algo = res[0].algo;
      p.index = algo_index;
      return kOk;
    }
  }
  hipblasLtMatmulPreference_t pref = nullptr;
  if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return kBlasFailed;
  const uint64_t max_ws = static_cast<uint64_t>(ws_bytes);
  hipblasLtMatmulHeuristicResult_t hr[1];
  int cnt = 0;
  const bool ok =
      hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                            &max_ws, sizeof(max_ws)) == HIPBLAS_STATUS_SUCCESS &&
      hipblasLtMatmulAlgoGetHeuristic(h, p.desc, p.a, p.b, p.d, p.d, pref, 1, hr, &cnt) ==
          HIPBLAS_STATUS_SUCCESS &&
      cnt > 0;
  hipblasLtMatmulPreferenceDestroy(pref);
  if (!ok) return kBlasFailed;
  p.algo = hr[0].algo;
  p.index = hipblaslt_ext::getIndexFromAlgo(p.algo);
  return kOk;
}

}  // namespace
}  // namespace soupk

using namespace soupk;

extern "C" __attribute__((visibility("default"))) int soupk_gemm_lt(
    int32_t trans_a, int32_t trans_b, int64_t m, int64_t n, int64_t k, const uint16_t* A,
    int64_t lda, int64_t stride_a, const uint16_t* B, int64_t ldb, int64_t stride_b, void* D,
    int64_t ldd, int64_t stride_d, int32_t d_f32, int32_t batch, int32_t accumulate,
    const uint16_t* bias, int32_t algo_index, void* workspace, int64_t workspace_bytes,
    void* stream) {
  if ((trans_a | trans_b | d_f32 | accumulate) & ~1) return kInvalid;
  if (m < 0 || n < 0 || k <= 0 || batch < 1 || workspace_bytes < 0) return kInvalid;
  if (lda < (trans_a ? k : m) || ldb < (trans_b ? n : k) || ldd < m || lda < 1 || ldb < 1 ||
      ldd < 1)
    return kInvalid;
  if (batch > 1 && (stride_a < 0 || stride_b < 0 || stride_d < ldd * n)) return kInvalid;
  if (bias != nullptr && (batch > 1 || d_f32)) return kInvalid;   // bias: one fp16 problem
  if (m == 0 || n == 0) return kOk;
  if (!A || !B || !D || (workspace_bytes > 0 && !workspace)) return kInvalid;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return kBlasFailed;
  std::lock_guard<std::mutex> lock(g_mu);
  hipblasLtHandle_t& h = g_handles[dev];
  if (h == nullptr && hipblasLtCreate(&h) != HIPBLAS_STATUS_SUCCESS) {
    h = nullptr;
    return kBlasFailed;
  }
  const PlanKey key{dev,      trans_a, trans_b,         m,         n,          k,
                    lda,      stride_a, ldb,            stride_b,  ldd,        stride_d,
                    d_f32,    batch,   bias != nullptr, accumulate, workspace_bytes, algo_index};
  auto it = g_plans.find(key);
  if (it == g_plans.end()) {
    // a bounded cache: a training run whose batches vary in tokens meets a new M each step
    if (g_plans.size() >= kMaxPlans) {
      for (auto& kv : g_plans) destroy(kv.second);
      g_plans.clear();
    }
    LtPlan p;
    const int rc = build_plan(h, trans_a, trans_b, m, n, k, lda, stride_a, ldb, stride_b, ldd,
                              stride_d, d_f32, batch, bias != nullptr, accumulate, algo_index,
                              workspace_bytes, p);
    if (rc != kOk) {
      destroy(p);
      return rc;
    }
    it = g_plans.emplace(key, p).first;
  }
  const LtPlan& p = it->second;
  if (bias != nullptr &&
      hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias,
                                      sizeof(bias)) != HIPBLAS_STATUS_SUCCESS)
    return kBlasFailed;
  const float alpha = 1.f, beta = accumulate ? 1.f : 0.f;
  const hipblasStatus_t st =
      hipblasLtMatmul(h, p.desc, &alpha, A, p.a, B, p.b, &beta, D, p.d, D, p.d, &p.algo,
                      workspace, static_cast<size_t>(workspace_bytes),
                      static_cast<hipStream_t>(stream));
  return st == HIPBLAS_STATUS_SUCCESS ? kOk : kBlasFailed;
}

// The hipBLASLt solution index a problem runs with (after its first call), or -1.
extern "C" __attribute__((visibility("default"))) int soupk_gemm_lt_index(
    int32_t trans_a, int32_t trans_b, int64_t m, int64_t n, int64_t k, int64_t lda,
    int64_t stride_a, int64_t ldb, int64_t stride_b, int64_t ldd, int64_t stride_d, int32_t d_f32,
    int32_t batch, int32_t has_bias, int32_t accumulate, int32_t algo_index,
    int64_t workspace_bytes) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  std::lock_guard<std::mutex> lock(g_mu);
  const PlanKey key{dev,      trans_a, trans_b,      m,          n,          k,
                    lda,      stride_a, ldb,         stride_b,   ldd,        stride_d,
                    d_f32,    batch,   has_bias != 0, accumulate, workspace_bytes, algo_index};
  const auto it = g_plans.find(key);
  return it == g_plans.end() ? -1 : it->second.index;
}
