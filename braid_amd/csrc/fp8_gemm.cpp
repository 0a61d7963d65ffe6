// FP8 (e4m3fn) W8A8 GEMM with per-tensor dequant scales: decode shapes on
// the hand-written streaming kernel (fp8_gemm_stream.hip), the rest through
// hipBLASLt.
//
// Reference behaviour: braid/model/quant.py:232-241 (`fp8_matmul`), which calls
//   torch._scaled_mm(xq, w.data.t(), scale_a=sx, scale_b=w.scale, out_dtype)
//   out[M, N] = (xq[M, K] * sx) @ (w[N, K] * sw)^T
// with fp32 accumulation. At decode shapes (M = the batch, at most 64; N x K =
// a projection's weight) the GEMM is weight-streaming bound, and the
// streaming kernel reads the weight at a higher rate than the library's
// tiles (its coalesced loads and one column block per CU over the whole of
// K); larger M is a plain library GEMM.
//
// hipBLASLt is column-major. The row-major operands read column-major are
// w^T [K, N] and xq^T [K, M]; with op(A) = T on A = w and op(B) = N on B = xq,
// D = op(A) op(B) = w xq^T is [N, M] column-major, which is out [M, N]
// row-major. The scales are device pointers (A = w's, B = x's), so a call
// never reads them on the host and can be captured in a graph.
//
// Plans (descriptors, layouts and the heuristic's algorithm) are cached per
// (device, M, N, K, output type); the first call for a shape runs the
// heuristic query on the host, so callers warm each shape up before capturing.
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "capi_common.h"
#include "fp8_gemm_stream.h"

namespace braid {
namespace {

constexpr size_t kWorkspaceBytes = 32u << 20;

struct Plan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  size_t workspace = 0;
};

std::mutex g_mu;
std::map<int, hipblasLtHandle_t> g_handles;
std::map<std::tuple<int, int64_t, int64_t, int64_t, int>, Plan> g_plans;

int lt_status(hipblasStatus_t s, const char* what) {
  if (s == HIPBLAS_STATUS_SUCCESS) return BRAID_OK;
  return fail(BRAID_EHIP, std::string(what) + " failed (hipblasStatus " + std::to_string((int)s) +
                              ")");
}

hipDataType out_type(int dt) {
  return dt == BRAID_F32 ? HIP_R_32F : (dt == BRAID_F16 ? HIP_R_16F : HIP_R_16BF);
}

// Builds (once) the plan for this shape. Called with g_mu held.
int get_plan(int dev, hipblasLtHandle_t h, int64_t M, int64_t N, int64_t K, int out_dtype,
             const float* sw, const float* sx, Plan** out) {
  const auto key = std::make_tuple(dev, M, N, K, out_dtype);
  auto it = g_plans.find(key);
  if (it != g_plans.end()) {
    *out = &it->second;
    return BRAID_OK;
  }
  Plan p;
  int st;
  if ((st = lt_status(hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F),
                      "hipblasLtMatmulDescCreate")))
    return st;
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta));
  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb));
  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_A_SCALE_POINTER, &sw, sizeof(sw));
  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_B_SCALE_POINTER, &sx, sizeof(sx));
  if ((st = lt_status(hipblasLtMatrixLayoutCreate(&p.a, HIP_R_8F_E4M3, K, N, K),
                      "hipblasLtMatrixLayoutCreate(A)")) ||
      (st = lt_status(hipblasLtMatrixLayoutCreate(&p.b, HIP_R_8F_E4M3, K, M, K),
                      "hipblasLtMatrixLayoutCreate(B)")) ||
      (st = lt_status(hipblasLtMatrixLayoutCreate(&p.d, out_type(out_dtype), N, M, N),
                      "hipblasLtMatrixLayoutCreate(D)")))
    return st;
  hipblasLtMatmulPreference_t pref;
  if ((st = lt_status(hipblasLtMatmulPreferenceCreate(&pref), "hipblasLtMatmulPreferenceCreate")))
    return st;
  const uint64_t ws = kWorkspaceBytes;
  hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws,
                                        sizeof(ws));
  hipblasLtMatmulHeuristicResult_t res[1];
  int n = 0;
  const hipblasStatus_t hs =
      hipblasLtMatmulAlgoGetHeuristic(h, p.desc, p.a, p.b, p.d, p.d, pref, 1, res, &n);
  hipblasLtMatmulPreferenceDestroy(pref);
  if ((st = lt_status(hs, "hipblasLtMatmulAlgoGetHeuristic"))) return st;
  if (n < 1 || res[0].state != HIPBLAS_STATUS_SUCCESS)
    return fail(BRAID_EINVAL, "hipBLASLt has no FP8 algorithm for M=" + std::to_string(M) +
                                  " N=" + std::to_string(N) + " K=" + std::to_string(K));
  p.algo = res[0].algo;
  p.workspace = res[0].workspaceSize;
  *out = &(g_plans[key] = p);
  return BRAID_OK;
}

}  // namespace
}  // namespace braid

using namespace braid;

extern "C" size_t braid_fp8_gemm_workspace(void) { return kWorkspaceBytes; }

extern "C" int braid_fp8_gemm(const uint8_t* x, const float* x_scale, const uint8_t* w,
                              const float* w_scale, void* out, int out_dtype, int64_t M,
                              int64_t N, int64_t K, void* workspace, size_t workspace_bytes,
                              void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  if (M <= 0 || N <= 0 || K <= 0) return fail(BRAID_EINVAL, "M, N and K must be positive");
  if (N % 16 || K % 16)
    return fail(BRAID_EINVAL, "_scaled_mm needs both weight dims to be multiples of 16; got [" +
                                  std::to_string(N) + ", " + std::to_string(K) + "]");
  if (out_dtype != BRAID_BF16 && out_dtype != BRAID_F16 && out_dtype != BRAID_F32)
    return fail(BRAID_EINVAL, "out dtype must be bf16, fp16 or fp32");
  if (!x || !x_scale || !w || !w_scale || !out || !workspace)
    return fail(BRAID_EINVAL, "x/x_scale/w/w_scale/out/workspace must be non-null");
  if (!aligned16(x) || !aligned16(w) || !aligned16(out) || !aligned16(workspace))
    return fail(BRAID_EINVAL, "x, w, out and workspace must be 16-byte aligned");
  // Decode shapes (M <= 64) stream the weight through the hand-written
  // kernel; the rest, and BRAID_FP8_GEMM=0, go to hipBLASLt.
  if (launch_knob(BRAID_KNOB_FP8_GEMM) != 0 && fp8_gemm_stream_fits(M, N, K)) {
    const int st = fp8_gemm_stream(x, x_scale, w, w_scale, out, out_dtype, M, N, K, stream);
    return st ? st : ok();
  }
  int dev = 0;
  int st;
  if ((st = hip_status(hipGetDevice(&dev), "hipGetDevice"))) return st;

  std::lock_guard<std::mutex> lock(g_mu);
  hipblasLtHandle_t& h = g_handles[dev];
  if (h == nullptr && (st = lt_status(hipblasLtCreate(&h), "hipblasLtCreate"))) {
    h = nullptr;
    return st;
  }
  Plan* p = nullptr;
  if ((st = get_plan(dev, h, M, N, K, out_dtype, w_scale, x_scale, &p))) return st;
  if (workspace_bytes < p->workspace)
    return fail(BRAID_EINVAL, "workspace of " + std::to_string(workspace_bytes) +
                                  " bytes is smaller than the " + std::to_string(p->workspace) +
                                  " the algorithm needs");
  hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_A_SCALE_POINTER, &w_scale,
                                  sizeof(w_scale));
  hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_B_SCALE_POINTER, &x_scale,
                                  sizeof(x_scale));
  const float alpha = 1.f, beta = 0.f;
  if ((st = lt_status(hipblasLtMatmul(h, p->desc, &alpha, w, p->a, x, p->b, &beta, out, p->d, out,
                                      p->d, &p->algo, workspace, workspace_bytes, stream),
                      "hipblasLtMatmul")))
    return st;
  return ok();
}
