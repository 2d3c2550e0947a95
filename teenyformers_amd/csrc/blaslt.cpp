// Prompt-size linear layers through hipBLASLt, the vendor GEMM library.
//
// y[M, N] = x[M, K] . w[N, K]^T with fp32 accumulation, y stored once in the
// operands' type (bf16 or fp32): the same product as gemm_bf16.hip /
// gemm_f32.hip.  At the Llama shapes the library picks kernels with
// 128 x 128 wavefront tiles (one wavefront per SIMD) that keep the matrix
// cores busier than this library's own GEMM (0.80 against 0.65 of the
// cycles, measured), so teeny_linear_bf16 hands its plain products of more
// than 16 rows here and keeps its own kernel as the fallback (and for the
// fused SwiGLU product, which hipBLASLt has no epilogue for).
//
// In hipBLASLt's column-major terms y^T [N, M] = W [N, K] . x^T [K, M]: A is
// the weight's memory read as a K x N column-major matrix and transposed, B
// the activations' memory as a K x M column-major matrix, D y's memory as an
// N x M column-major matrix.
//
// No workspace: the heuristic is asked for algorithms that need none (at the
// Llama prompt shapes they run within 1 % of those it picks under a 64 MiB
// limit, measured), so a product never allocates device memory and products
// on different streams or threads share nothing but the read-only plan.
// Plans (descriptors and the heuristic's first algorithm) are built once per
// (device, dtype, M, N, K, ldy) under a lock and never freed; the matmul
// itself is enqueued outside the lock.  Where the heuristic has no algorithm
// for a wide product (the 128256-row lm_head at 8192 rows), the product runs
// as column blocks of at most 32768 features (y's rows keep their stride),
// each its own plan: the same sums per output, since no algorithm here splits
// K.  Under stream capture nothing is built or run
// here (the caller's own GEMM runs instead), so which GEMM a captured graph
// holds does not depend on what ran before the capture.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <cstdint>
#include <map>
#include <mutex>
#include <tuple>

namespace {

struct Plan {
  bool ok = false;
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
  hipblasLtMatmulAlgo_t algo{};
};

struct Device {
  bool tried = false;
  hipblasLtHandle_t handle = nullptr;
  // std::map: a plan's address stays valid while other plans are added
  std::map<std::tuple<int, int, int, int, int>, Plan> plans;
};

std::mutex mu;
std::map<int, Device> devices;

Plan make_plan(hipblasLtHandle_t h, hipDataType t, int M, int N, int K, int ldy) {
  Plan p;
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  if (hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS)
    return p;
  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof ta);
  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof tb);
  if (hipblasLtMatrixLayoutCreate(&p.a, t, K, N, K) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&p.b, t, K, M, K) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&p.d, t, N, M, ldy) != HIPBLAS_STATUS_SUCCESS)
    return p;
  hipblasLtMatmulPreference_t pref = nullptr;
  if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return p;
  const uint64_t max_ws = 0;
  hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &max_ws,
                                        sizeof max_ws);
  hipblasLtMatmulHeuristicResult_t res[1];
  int n = 0;
  const hipblasStatus_t s =
      hipblasLtMatmulAlgoGetHeuristic(h, p.desc, p.a, p.b, p.d, p.d, pref, 1, res, &n);
  hipblasLtMatmulPreferenceDestroy(pref);
  if (s != HIPBLAS_STATUS_SUCCESS || n < 1 || res[0].state != HIPBLAS_STATUS_SUCCESS) return p;
  if (res[0].workspaceSize != 0) return p;
  p.algo = res[0].algo;
  p.ok = true;
  return p;
}

constexpr int kMaxBlocks = 8;
constexpr int kBlockN = 32768;  // widest column block of a split product

// the plan of (t, M, n, K) with y's row stride ldy, built on first use;
// nullptr: no algorithm.  Called with mu held.
const Plan* plan_of(Device& d, hipDataType t, int M, int n, int K, int ldy) {
  auto key = std::make_tuple((int)t, M, n, K, ldy);
  auto it = d.plans.find(key);
  if (it == d.plans.end()) it = d.plans.emplace(key, make_plan(d.handle, t, M, n, K, ldy)).first;
  return it->second.ok ? &it->second : nullptr;
}

// 0: y written (launched on `stream`); -1: hipBLASLt is not used for this
// device, shape or stream state, and y is left to the caller's own GEMM.
int lt_gemm(hipDataType t, const void* x, const void* w, void* y, int M, int N, int K,
            hipStream_t stream) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone)
    return -1;
  hipblasLtHandle_t handle = nullptr;
  const Plan* plans[kMaxBlocks] = {};
  int nblk = 1, bn = N;
  {
    std::lock_guard<std::mutex> lock(mu);
    Device& d = devices[dev];
    if (!d.tried) {
      d.tried = true;
      if (hipblasLtCreate(&d.handle) != HIPBLAS_STATUS_SUCCESS) d.handle = nullptr;
    }
    if (!d.handle) return -1;
    plans[0] = plan_of(d, t, M, N, K, N);
    if (!plans[0]) {
      // column blocks: equal widths (multiples of 64), the last one narrower
      nblk = (N + kBlockN - 1) / kBlockN;
      if (nblk < 2 || nblk > kMaxBlocks) return -1;
      bn = ((N + nblk - 1) / nblk + 63) / 64 * 64;
      nblk = (N + bn - 1) / bn;
      for (int i = 0; i < nblk; ++i)
        if (!(plans[i] = plan_of(d, t, M, std::min(bn, N - i * bn), K, N))) return -1;
    }
    handle = d.handle;
  }
  const size_t esz = t == HIP_R_16BF ? 2 : 4;
  const float alpha = 1.0f, beta = 0.0f;
  for (int i = 0; i < nblk; ++i) {
    const Plan* plan = plans[i];
    const void* wi = static_cast<const char*>(w) + (size_t)i * bn * K * esz;
    void* yi = static_cast<char*>(y) + (size_t)i * bn * esz;
    const hipblasStatus_t s = hipblasLtMatmul(handle, plan->desc, &alpha, wi, plan->a, x,
                                              plan->b, &beta, yi, plan->d, yi, plan->d,
                                              &plan->algo, nullptr, 0, stream);
    // after a failed block the caller's own GEMM rewrites the whole of y,
    // in stream order after the blocks already enqueued
    if (s != HIPBLAS_STATUS_SUCCESS) return -1;
  }
  return 0;
}

}  // namespace

extern "C" __attribute__((visibility("hidden"))) int teeny_lt_gemm_bf16(
    const void* x, const void* w, void* y, int M, int N, int K, hipStream_t stream) {
  return lt_gemm(HIP_R_16BF, x, w, y, M, N, K, stream);
}

extern "C" __attribute__((visibility("hidden"))) int teeny_lt_gemm_f32(
    const void* x, const void* w, void* y, int M, int N, int K, hipStream_t stream) {
  return lt_gemm(HIP_R_32F, x, w, y, M, N, K, stream);
}
