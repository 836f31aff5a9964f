// Plain projections of many rows (a prompt's prefill) through hipBLASLt:
// y[M, N] = bf16(x[M, K] W[N, K]^T), fp32 accumulation, bf16 output rounded
// once -- the rounding boundary of the tiled kernels' store epilogue. The
// prefill's residual adds, RMSNorms and SwiGLU stay in this library's
// row-wise kernels (same bf16 boundaries); only the plain product goes to the
// vendor GEMM, whose gfx950 tiles run the 8B prefill shapes 1.4-1.5x faster
// than gemm_tiles.hip's (2048 rows: 89 / 69 / 291 / 184 us against
// 136 / 87 / 443 / 253 us for QKV, O, gate/up and down, weights rotated over
// 8 layers so none stays in the Infinity Cache).
//
// hipBLASLt is column-major: the row-major x [M, K] (row stride x_stride) is
// the column-major K x M matrix B, the row-major W [N, K] the column-major
// K x N matrix A taken transposed, and the row-major y [M, N] the
// column-major N x M result D = A^T B.
#include "common.h"

#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

namespace htn {
namespace {

constexpr int kLtDevices = 64;
constexpr long kLtWorkspace = 32L << 20;

struct LtPlan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  size_t workspace = 0;
  bool ok = false;
};

std::mutex lt_mutex;
hipblasLtHandle_t lt_handle[kLtDevices] = {};
// Plans by (device, n, k, rows, x_stride, y_stride); kept for the process.
std::map<std::tuple<int, long, long, long, long, long>, LtPlan> lt_plans;

LtPlan make_plan(hipblasLtHandle_t h, long n, long k, long rows, long xs, long ys) {
  LtPlan p;
  if (hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS)
    return p;
  const int32_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta));
  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb));
  if (hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16BF, k, n, k) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&p.b, HIP_R_16BF, k, rows, xs) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&p.d, HIP_R_16BF, n, rows, ys) != HIPBLAS_STATUS_SUCCESS)
    return p;
  hipblasLtMatmulPreference_t pref = nullptr;
  if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return p;
  const uint64_t ws = kLtWorkspace;
  hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws,
                                        sizeof(ws));
  hipblasLtMatmulHeuristicResult_t result[1];
  int found = 0;
  const hipblasStatus_t st = hipblasLtMatmulAlgoGetHeuristic(h, p.desc, p.a, p.b, p.d, p.d, pref,
                                                             1, result, &found);
  hipblasLtMatmulPreferenceDestroy(pref);
  if (st != HIPBLAS_STATUS_SUCCESS || found < 1 || result[0].state != HIPBLAS_STATUS_SUCCESS)
    return p;
  p.algo = result[0].algo;
  p.workspace = result[0].workspaceSize;
  p.ok = p.workspace <= static_cast<size_t>(kLtWorkspace);
  return p;
}

}  // namespace
}  // namespace htn

using namespace htn;

extern "C" int64_t htn_gemm_library_workspace_bytes() { return kLtWorkspace; }

extern "C" int htn_gemm_library(const void* x, int64_t x_stride, const void* w, int64_t n,
                                int64_t k, int64_t rows, void* y, int64_t y_stride,
                                void* workspace, htn_stream_t stream) {
  if (!x || !w || !y || !workspace || n <= 0 || k <= 0 || rows <= 0 || x_stride < k ||
      y_stride < n)
    return HTN_EINVAL;
  if (!aligned16(x) || !aligned16(w) || !aligned16(y) || !aligned16(workspace) || k % 8 ||
      x_stride % 8 || y_stride % 8)
    return HTN_EUNSUPPORTED;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kLtDevices) return HTN_EINVAL;
  const LtPlan* plan = nullptr;
  hipblasLtHandle_t handle = nullptr;
  {
    std::lock_guard<std::mutex> lock(lt_mutex);
    if (!lt_handle[dev] && hipblasLtCreate(&lt_handle[dev]) != HIPBLAS_STATUS_SUCCESS) {
      lt_handle[dev] = nullptr;
      return HTN_EUNSUPPORTED;
    }
    handle = lt_handle[dev];
    const auto key = std::make_tuple(dev, static_cast<long>(n), static_cast<long>(k),
                                     static_cast<long>(rows), static_cast<long>(x_stride),
                                     static_cast<long>(y_stride));
    auto it = lt_plans.find(key);
    if (it == lt_plans.end())
      it = lt_plans.emplace(key, make_plan(handle, n, k, rows, x_stride, y_stride)).first;
    plan = &it->second;
  }
  if (!plan->ok) return HTN_EUNSUPPORTED;
  const float alpha = 1.0f, beta = 0.0f;
  const hipblasStatus_t st =
      hipblasLtMatmul(handle, plan->desc, &alpha, w, plan->a, x, plan->b, &beta, y, plan->d, y,
                      plan->d, &plan->algo, workspace, kLtWorkspace,
                      static_cast<hipStream_t>(stream));
  return st == HIPBLAS_STATUS_SUCCESS ? HTN_OK : HTN_ELAUNCH;
}
