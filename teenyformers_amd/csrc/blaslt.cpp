// Prompt-size bf16 linear layers through hipBLASLt, the vendor GEMM library.
//
// y[M, N] = x[M, K] . w[N, K]^T, fp32 accumulation, y rounded to bf16 once:
// the same product as gemm_bf16.hip.  At the Llama shapes the library picks
// kernels with 128 x 128 wavefront tiles (one wavefront per SIMD) that keep
// the matrix cores busier than this library's own GEMM (0.80 against 0.65 of
// the cycles, measured), so teeny_linear_bf16 hands its plain products of
// more than 16 rows here and keeps its own kernel as the fallback (and for
// the fused SwiGLU product, which hipBLASLt has no epilogue for).
//
// In hipBLASLt's column-major terms y^T [N, M] = W [N, K] . x^T [K, M]: A is
// the weight's memory read as a K x N column-major matrix and transposed, B
// the activations' memory as a K x M column-major matrix, D y's memory as an
// N x M column-major matrix.  Plans (descriptors and the heuristic's first
// algorithm) are cached per (device, M, N, K); each (device, stream) gets
// its own workspace, so products on different streams never share one.  The
// handle, plans and workspaces live until the process ends.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <cstdint>
#include <map>
#include <mutex>
#include <tuple>

namespace {

constexpr size_t kWorkspace = 64u << 20;  // bytes per (device, stream)

struct Plan {
  bool ok = false;
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
  hipblasLtMatmulAlgo_t algo{};
};

struct Device {
  bool tried = false;
  hipblasLtHandle_t handle = nullptr;
  std::map<std::tuple<int, int, int>, Plan> plans;
  std::map<hipStream_t, void*> workspace;
};

std::mutex mu;
std::map<int, Device> devices;

Plan make_plan(hipblasLtHandle_t h, int M, int N, int K) {
  Plan p;
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  if (hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS)
    return p;
  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof ta);
  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof tb);
  if (hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16BF, K, N, K) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&p.b, HIP_R_16BF, K, M, K) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&p.d, HIP_R_16BF, N, M, N) != HIPBLAS_STATUS_SUCCESS)
    return p;
  hipblasLtMatmulPreference_t pref = nullptr;
  if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return p;
  const uint64_t max_ws = kWorkspace;
  hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &max_ws,
                                        sizeof max_ws);
  hipblasLtMatmulHeuristicResult_t res[1];
  int n = 0;
  const hipblasStatus_t s =
      hipblasLtMatmulAlgoGetHeuristic(h, p.desc, p.a, p.b, p.d, p.d, pref, 1, res, &n);
  hipblasLtMatmulPreferenceDestroy(pref);
  if (s != HIPBLAS_STATUS_SUCCESS || n < 1 || res[0].state != HIPBLAS_STATUS_SUCCESS) return p;
  if (res[0].workspaceSize > kWorkspace) return p;
  p.algo = res[0].algo;
  p.ok = true;
  return p;
}

}  // namespace

// 0: y written (launched on `stream`); -1: hipBLASLt is not available for
// this device or shape, nothing was launched (the caller uses its own GEMM).
extern "C" __attribute__((visibility("hidden"))) int teeny_lt_gemm_bf16(
    const void* x, const void* w, void* y, int M, int N, int K, hipStream_t stream) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  // under stream capture nothing is created (handle, plan, workspace): a
  // shape met first inside a capture runs the caller's own GEMM
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cap) != hipSuccess) return -1;
  const bool capturing = cap != hipStreamCaptureStatusNone;
  std::lock_guard<std::mutex> lock(mu);
  Device& d = devices[dev];
  if (!d.tried) {
    if (capturing) return -1;
    d.tried = true;
    if (hipblasLtCreate(&d.handle) != HIPBLAS_STATUS_SUCCESS) d.handle = nullptr;
  }
  if (!d.handle) return -1;
  auto key = std::make_tuple(M, N, K);
  auto it = d.plans.find(key);
  if (it == d.plans.end()) {
    if (capturing) return -1;
    it = d.plans.emplace(key, make_plan(d.handle, M, N, K)).first;
  }
  const Plan& p = it->second;
  if (!p.ok) return -1;
  // the whole workspace goes with every call (the heuristic chose its
  // algorithm under that limit)
  auto wi = d.workspace.find(stream);
  if (wi == d.workspace.end()) {
    if (capturing) return -1;
    void* buf = nullptr;
    if (hipMalloc(&buf, kWorkspace) != hipSuccess) return -1;
    wi = d.workspace.emplace(stream, buf).first;
  }
  const float alpha = 1.0f, beta = 0.0f;
  const hipblasStatus_t s = hipblasLtMatmul(d.handle, p.desc, &alpha, w, p.a, x, p.b, &beta, y,
                                            p.d, y, p.d, &p.algo, wi->second, kWorkspace, stream);
  return s == HIPBLAS_STATUS_SUCCESS ? 0 : -1;
}
