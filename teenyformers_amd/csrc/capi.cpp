// C-ABI host library: validates arguments, picks the kernel instance and
// launches it with hipModuleLaunchKernel on the caller's stream.
//
// The gfx950 code objects (one per kernel source file, built with
// `hipcc --genco`) are embedded in this shared library and loaded with
// hipModuleLoadData once per device, on first use or from teeny_init().
// This plays the role of the reference's compile-to-PTX + load_program +
// device.launch sequence (tests/kernel_execution.rs:81-99), without any
// runtime compilation.
#include "teeny_hip.h"

#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

// ---------------------------------------------------------------------------
// Embedded code objects (symbols defined by the generated co_blob.S)
// ---------------------------------------------------------------------------
#define TEENY_CO_LIST(X) \
  X(transpose)           \
  X(rope)                \
  X(norm)                \
  X(swiglu)              \
  X(embed)               \
  X(fa2_f32)             \
  X(fa2_fwd_bf16)        \
  X(fa2_bwd_bf16)        \
  X(llama)               \
  X(decode_bf16)         \
  X(linear_bf16)         \
  X(gemm_bf16)           \
  X(gemm_f32)

// noalloc.hip: the current device's address of its static scratch array
extern "C" __attribute__((visibility("hidden"))) int teeny_scratch_setup(void** out);
// blaslt.cpp: a product through hipBLASLt (0), or -1 to fall back
extern "C" __attribute__((visibility("hidden"))) int teeny_lt_gemm_bf16(
    const void* x, const void* w, void* y, int M, int N, int K, hipStream_t stream);
extern "C" __attribute__((visibility("hidden"))) int teeny_lt_gemm_f32(
    const void* x, const void* w, void* y, int M, int N, int K, hipStream_t stream);

#define TEENY_CO_DECL(n) \
  extern "C" const unsigned char teeny_co_##n[]; \
  extern "C" const unsigned char teeny_co_##n##_end[];
TEENY_CO_LIST(TEENY_CO_DECL)

namespace {

struct CodeObject {
  const char* name;
  const unsigned char* begin;
  const unsigned char* end;
};

#define TEENY_CO_ENTRY(n) {#n, teeny_co_##n, teeny_co_##n##_end},
const CodeObject kCodeObjects[] = {TEENY_CO_LIST(TEENY_CO_ENTRY)};
constexpr int kNumCodeObjects = sizeof(kCodeObjects) / sizeof(kCodeObjects[0]);
constexpr int kMaxDevices = 64;

struct DeviceState {
  hipModule_t mods[kNumCodeObjects] = {};
  std::unordered_map<std::string, hipFunction_t> fns;
  std::unordered_map<std::string, int> resident;  // resident_groups' answers
};

std::mutex g_mu;
DeviceState* g_dev[kMaxDevices] = {};
thread_local int g_last_hip = 0;

int hip_fail(hipError_t e) {
  g_last_hip = (int)e;
  return TEENY_ERR_HIP;
}

// Loads every code object on the current device (caller holds g_mu).
int load_device_locked(int dev, DeviceState** out) {
  if (g_dev[dev]) {
    *out = g_dev[dev];
    return TEENY_OK;
  }
  DeviceState* st = new DeviceState();
  for (int i = 0; i < kNumCodeObjects; ++i) {
    hipError_t e = hipModuleLoadData(&st->mods[i], kCodeObjects[i].begin);
    if (e != hipSuccess) {
      g_last_hip = (int)e;
      for (int j = 0; j < i; ++j) (void)hipModuleUnload(st->mods[j]);
      delete st;
      return TEENY_ERR_MODULE;
    }
  }
  g_dev[dev] = st;
  *out = st;
  return TEENY_OK;
}

// Whether the current device's code objects are loaded (loads nothing).
bool device_ready() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
  std::lock_guard<std::mutex> lk(g_mu);
  return g_dev[dev] != nullptr;
}

int get_function(const char* name, hipFunction_t* fn) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e);
  if (dev < 0 || dev >= kMaxDevices) return TEENY_ERR_HIP;
  std::lock_guard<std::mutex> lk(g_mu);
  DeviceState* st = nullptr;
  int rc = load_device_locked(dev, &st);
  if (rc) return rc;
  auto it = st->fns.find(name);
  if (it != st->fns.end()) {
    *fn = it->second;
    return TEENY_OK;
  }
  for (int i = 0; i < kNumCodeObjects; ++i) {
    hipFunction_t f = nullptr;
    if (hipModuleGetFunction(&f, st->mods[i], name) == hipSuccess && f) {
      st->fns.emplace(name, f);
      *fn = f;
      return TEENY_OK;
    }
    // A miss sets the thread's sticky "last error"; clear it so the caller's
    // next HIP call (e.g. torch's launch check) does not report it.
    (void)hipGetLastError();
  }
  return TEENY_ERR_MODULE;
}

// Workgroups of `threads` threads of kernel `name` that the current device
// holds at once (the occupancy the kernel's registers and LDS allow, times
// the CUs), asked once per (device, kernel); `fallback` if the runtime
// cannot say.
int device_cus();
int resident_groups(const char* name, int threads, int fallback) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return fallback;
  hipFunction_t f = nullptr;
  if (get_function(name, &f)) return fallback;
  std::lock_guard<std::mutex> lk(g_mu);
  DeviceState* st = g_dev[dev];
  auto it = st->resident.find(name);
  if (it != st->resident.end()) return it->second;
  int per_cu = 0;
  int groups = fallback;
  if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, threads, 0) == hipSuccess &&
      per_cu > 0)
    groups = per_cu * device_cus();
  else
    (void)hipGetLastError();
  st->resident.emplace(name, groups);
  return groups;
}

// ---------------------------------------------------------------------------
// Opt-in launch profiler: while enabled, every launch is bracketed by two
// hipEvents recorded on its own stream; durations are read (synchronising on
// the events) only when stats are requested.
// ---------------------------------------------------------------------------
struct ProfRecord {
  std::string name;
  hipEvent_t start, stop;
};
std::mutex g_prof_mu;
bool g_prof_on = false;
std::vector<ProfRecord> g_prof;
std::vector<hipEvent_t> g_event_pool;

hipEvent_t pool_event() {
  if (!g_event_pool.empty()) {
    hipEvent_t e = g_event_pool.back();
    g_event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

void prof_clear_locked() {
  for (auto& r : g_prof) {
    g_event_pool.push_back(r.start);
    g_event_pool.push_back(r.stop);
  }
  g_prof.clear();
}

int launch(const char* name, dim3 grid, dim3 block, unsigned shmem, hipStream_t stream,
           void** args) {
  if (grid.x == 0 || grid.y == 0 || grid.z == 0) return TEENY_OK;  // nothing to do
  hipFunction_t f = nullptr;
  int rc = get_function(name, &f);
  if (rc) return rc;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    if (g_prof_on) {
      ev0 = pool_event();
      ev1 = pool_event();
    }
  }
  if (ev0 && ev1) (void)hipEventRecord(ev0, stream);
  hipError_t e = hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z,
                                       shmem, stream, args, nullptr);
  if (ev0 && ev1) {
    (void)hipEventRecord(ev1, stream);
    std::lock_guard<std::mutex> lk(g_prof_mu);
    g_prof.push_back({name, ev0, ev1});
  }
  if (e != hipSuccess) return hip_fail(e);
  return TEENY_OK;
}

const char* dtype_tag(int dtype) { return dtype == TEENY_BF16 ? "bf16" : "f32"; }
size_t dtype_size(int dtype) { return dtype == TEENY_BF16 ? 2 : 4; }
bool dtype_ok(int dtype) { return dtype == TEENY_F32 || dtype == TEENY_BF16; }
size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

constexpr long kMaxElems = 1L << 31;  // kernels index rows with 32-bit ints where safe

// ---------------------------------------------------------------------------
// Flash attention
// ---------------------------------------------------------------------------
bool fa2_head_dim_ok(int head_dim, int dtype) {
  if (dtype == TEENY_BF16) return head_dim == 64 || head_dim == 128;
  return head_dim == 8 || head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128;
}

int fa2_check(const void* q, const void* k, const void* v, int n_ctx_q, int n_ctx_k, int batch,
              int hq, int hkv, int head_dim, int dtype) {
  if (!q || !k || !v) return TEENY_ERR_NULL_POINTER;
  if (!dtype_ok(dtype)) return TEENY_ERR_UNSUPPORTED;
  if (n_ctx_q <= 0 || n_ctx_k <= 0 || batch <= 0 || hq <= 0 || hkv <= 0 || hq % hkv != 0)
    return TEENY_ERR_INVALID_SHAPE;
  if ((long)batch * hq * n_ctx_q * head_dim >= kMaxElems ||
      (long)batch * hkv * n_ctx_k * head_dim >= kMaxElems)
    return TEENY_ERR_INVALID_SHAPE;
  if (!fa2_head_dim_ok(head_dim, dtype)) return TEENY_ERR_UNSUPPORTED;
  // bf16 kernels address one head's rows through buffer descriptors whose
  // byte ranges and tile offsets are signed 32-bit values: K / V in every
  // kernel, Q and dO in the dK/dV kernel
  if (dtype == TEENY_BF16 &&
      ((long)n_ctx_k * head_dim * 2 >= kMaxElems || (long)n_ctx_q * head_dim * 2 >= kMaxElems))
    return TEENY_ERR_INVALID_SHAPE;
  return TEENY_OK;
}

// The fp32 kernels take any finite scale (they scale, then mask, as the
// reference does).  The bf16 kernels fold the scale into the exponent after
// masking raw scores to -inf, which needs scale > 0 (-inf * 0 is NaN and a
// negative scale would turn masked scores into +inf).
bool scale_ok(float scale, int dtype) {
  if (!std::isfinite(scale)) return false;
  return dtype != TEENY_BF16 || scale > 0.0f;
}

int fa2_fwd(bool causal, const void* q, const void* k, const void* v, void* o, float* l,
            int n_ctx_q, int n_ctx_k, float scale, float neg_inf, int batch, int hq, int hkv,
            int head_dim, int dtype, hipStream_t stream, int o_merged = 0,
            const float* rope_cs = nullptr) {
  int rc = fa2_check(q, k, v, n_ctx_q, n_ctx_k, batch, hq, hkv, head_dim, dtype);
  if (rc) return rc;
  if (!o || !l) return TEENY_ERR_NULL_POINTER;
  if (!(std::isinf(neg_inf) && neg_inf < 0)) return TEENY_ERR_INVALID_VALUE;
  if (!scale_ok(scale, dtype)) return TEENY_ERR_INVALID_VALUE;
  char name[64];
  const char* cz = causal ? "c" : "n";
  if (dtype == TEENY_BF16) {
    // one workgroup of 4 wavefronts per 128 query rows of a (b, head); long
    // GQA sequences at D = 128: 8 wavefronts per 256 rows share each K/V
    // tile (measured 3-6 % faster there, 1-4 % slower at 4096-8192 rows
    // without GQA and at D = 64; the outputs are the same bits).  Causal GQA
    // groups of 4 (8 at D = 128) below that length: one workgroup per
    // (b, kv head, 32 rows), a wavefront per q head of the group (measured
    // 4-18 % faster: no wavefront idles through its block's diagonal tiles;
    // 4-5 % slower than the 8-wavefront form at 8000+ rows)
    const int group = hq / hkv;
    const bool w8 = head_dim == 128 && n_ctx_q >= 8000 && group >= 2;
    const int pack = !causal || w8                      ? 0
                     : group == 4                          ? 4
                     : group == 8 && head_dim == 128       ? 8
                                                           : 0;
    const int bm = pack ? 32 : w8 ? 256 : 128;
    int nmb = (n_ctx_q + bm - 1) / bm;
    long total = (long)nmb * batch * (pack ? hkv : hq);
    if (total >= (1L << 31)) return TEENY_ERR_INVALID_SHAPE;
    int tot = (int)total;
    snprintf(name, sizeof name, "teeny_fa2_fwd_bf16_d%d_%s%s", head_dim, cz,
             pack == 4 ? "_g4" : pack == 8 ? "_g8" : w8 ? "_w8" : "");
    void* args[] = {&q, &k, &v, &o, &l, &n_ctx_q, &n_ctx_k, &scale, &hq, &hkv, &nmb, &tot,
                    &o_merged, &rope_cs};
    const int threads = pack ? 64 * pack : 2 * bm;
    return launch(name, dim3(tot), dim3(threads), 0, stream, args);
  }
  if (o_merged || rope_cs) return TEENY_ERR_UNSUPPORTED;
  snprintf(name, sizeof name, "teeny_fa2_fwd_f32_d%d_%s", head_dim, cz);
  void* args[] = {&q, &k, &v, &o, &l, &n_ctx_q, &n_ctx_k, &scale, &hq, &hkv};
  return launch(name, dim3((n_ctx_q + 63) / 64, batch * hq), dim3(64), 0, stream, args);
}

// bf16: per (b, q head) and block of 32 query rows, 32 values of -LSE/scale
// then 32 of -Delta (fp32; the last block padded).  fp32: Delta [B*Hq, n_ctx_q].
constexpr int kLdRows = 32;
size_t fa2_bwd_ws(int n_ctx_q, int batch, int hq, int head_dim, int dtype) {
  (void)head_dim;
  if (dtype == TEENY_BF16) {
    const size_t nq_pad = (size_t)(n_ctx_q + kLdRows - 1) / kLdRows * kLdRows;
    return align256((size_t)batch * hq * nq_pad * 2 * sizeof(float));
  }
  return align256((size_t)batch * hq * n_ctx_q * sizeof(float));
}

// CUs of the current device, asked once per device (256, MI355X's count,
// when it cannot be asked).  Concurrent first calls store the same value.
int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (dev >= 0 && dev < 64) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    return 256;
  if (dev >= 0 && dev < 64) cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

// bf16 dK/dV: how each GQA group's q heads are shared out.  A workgroup
// owns 128 keys of a (b, kv head) and walks the query blocks of its q heads
// (causal: key block nb sees n_ctx_q / 128 - nb of them), so with few key
// blocks the heaviest walks set the time.  Two ways to shorten them:
//   groups = 2: the workgroup is two groups of 4 wavefronts on the same
//     keys, each walking half of the q heads, their sums added through LDS
//     (one workgroup per CU);
//   split > 1: the q heads are split over `split` workgroups whose fp32
//     partial sums a merge kernel adds in a fixed order (needs the larger
//     workspace).
// Measured (MI355X, causal, Hq/Hkv 4 and 8, D 64 and 128, same-box A/B of
// every combination): two groups are 1.02-1.45x the plain kernel from 2048
// to 8191 query rows and at least as fast as any split there; from 12288
// rows of one sequence the 4-way split is 1.05-1.13x and the two groups
// 0.98-1.05x; at 512 and 1024 rows, for the bidirectional kernel and with
// many key-block workgroups (B2 S8192) the plain kernel is fastest.
struct DkdvPlan {
  int groups, split;
};
DkdvPlan dkdv_plan(bool causal, int n_ctx_q, int n_ctx_k, int batch, int hq, int hkv,
                   int dtype) {
  DkdvPlan p{1, 1};
  const int group = hq / hkv;
  if (dtype != TEENY_BF16 || !causal || group % 2 != 0 || n_ctx_q < 2048) return p;
  const long wgs = (long)((n_ctx_k + 127) / 128) * batch * hkv;
  if (n_ctx_q >= 12288 && wgs <= 4L * device_cus())
    p.split = group % 4 == 0 ? 4 : 2;
  else
    p.groups = 2;
  return p;
}

size_t dkdv_split_bytes(int n_ctx_k, int batch, int hkv, int head_dim, int split) {
  if (split <= 1) return 0;
  return align256(2 * (size_t)split * batch * hkv * n_ctx_k * head_dim * sizeof(float));
}

int fa2_bwd(bool causal, const void* q, const void* k, const void* v, const void* o,
            const void* dout, const float* l, void* dq, void* dk, void* dv, int n_ctx_q,
            int n_ctx_k, float scale, int batch, int hq, int hkv, int head_dim, int dtype,
            void* workspace, size_t workspace_bytes, hipStream_t stream) {
  // TEENY_GRAD_F32: fp32 dq/dk/dv from the bf16 kernels (the fp32 path's
  // gradients are fp32 anyway)
  const bool g32 = (dtype & TEENY_GRAD_F32) != 0;
  dtype &= ~TEENY_GRAD_F32;
  const char* gsfx = g32 && dtype == TEENY_BF16 ? "_g32" : "";
  int rc = fa2_check(q, k, v, n_ctx_q, n_ctx_k, batch, hq, hkv, head_dim, dtype);
  if (rc) return rc;
  if (!o || !dout || !l || !dq || !dk || !dv) return TEENY_ERR_NULL_POINTER;
  if (!scale_ok(scale, dtype)) return TEENY_ERR_INVALID_VALUE;
  if (!workspace || workspace_bytes < fa2_bwd_ws(n_ctx_q, batch, hq, head_dim, dtype))
    return TEENY_ERR_WORKSPACE;
  const long rows = (long)batch * hq * n_ctx_q;
  float* delta = (float*)workspace;
  const char* cz = causal ? "c" : "n";
  char name[64];
  if (dtype == TEENY_BF16) {
    float* ld = (float*)workspace;
    // dQ first: one workgroup per 128 query rows of a (b, q head), or, for
    // causal GQA groups of 4, per (b, kv head, 32 rows) with a wavefront per
    // q head as in the forward; it also writes -LSE/scale and -Delta of its
    // rows to ld for the dK/dV kernel
    const bool pack = causal && hq == 4 * hkv;
    int nmb = pack ? (n_ctx_q + 31) / 32 : (n_ctx_q + 127) / 128;
    long total = (long)nmb * batch * (pack ? hkv : hq);
    if (total >= (1L << 31)) return TEENY_ERR_INVALID_SHAPE;
    int tot = (int)total;
    snprintf(name, sizeof name, "teeny_fa2_bwd_dq_bf16_d%d_%s%s%s", head_dim, cz,
             pack ? "_g4" : "", gsfx);
    void* a2[] = {&q,       &k,       &v,     &o,  &dout, &l,   &ld,  &dq,
                  &n_ctx_q, &n_ctx_k, &scale, &hq, &hkv,  &nmb, &tot};
    rc = launch(name, dim3(tot), dim3(256), 0, stream, a2);
    if (rc) return rc;
    // dK, dV: one workgroup per 128 keys of a (b, kv head) and share of the
    // group's q heads (a split needs the larger workspace; without it the
    // two-group kernel runs instead, the group being even)
    DkdvPlan plan = dkdv_plan(causal, n_ctx_q, n_ctx_k, batch, hq, hkv, dtype);
    const size_t base = fa2_bwd_ws(n_ctx_q, batch, hq, head_dim, dtype);
    if (plan.split > 1 &&
        workspace_bytes < base + dkdv_split_bytes(n_ctx_k, batch, hkv, head_dim, plan.split))
      plan = DkdvPlan{2, 1};
    int hsplit = plan.split;
    float* part = hsplit > 1 ? (float*)((char*)workspace + base) : nullptr;
    int nnb = (n_ctx_k + 127) / 128;
    total = (long)nnb * batch * hkv * hsplit;
    if (total >= (1L << 31)) return TEENY_ERR_INVALID_SHAPE;
    tot = (int)total;
    snprintf(name, sizeof name, "teeny_fa2_bwd_dkdv_bf16_d%d_%s%s%s", head_dim, cz,
             plan.groups == 2 ? "_hg2" : "", gsfx);
    // causal blocks all resident at once, two per CU: pair heavy key blocks
    // with light ones on each CU (same-box A/B, same bits: B16 Hq32 Hkv8 S512
    // 1.12x, B8 S1024 1.24x); the kernel's order needs whole heads and an
    // even number of key blocks in each XCD's share
    const int cus = device_cus();
    int cu_pairs = causal && plan.groups == 1 && hsplit == 1 && tot > cus && tot <= 2 * cus &&
                   tot % 8 == 0 && (tot / 8) % nnb == 0 && nnb % 2 == 0;
    void* a1[] = {&q,       &k,       &v,     &dout, &ld,  &dk,  &dv,  &n_ctx_q,
                  &n_ctx_k, &scale,   &hq,    &hkv,  &nnb, &tot, &hsplit, &part, &cu_pairs};
    rc = launch(name, dim3(tot), dim3(256 * plan.groups), 0, stream, a1);
    if (rc || hsplit == 1) return rc;
    long n = (long)batch * hkv * n_ctx_k * head_dim;  // a multiple of 8
    void* a3[] = {&part, &dk, &dv, &n, &hsplit, &scale};
    return launch(*gsfx ? "teeny_fa2_dkdv_merge_bf16_g32" : "teeny_fa2_dkdv_merge_bf16", dim3((unsigned)((n / 8 + 255) / 256)), dim3(256),
                  0, stream, a3);
  }
  snprintf(name, sizeof name, "teeny_fa2_bwd_pre_f32_d%d", head_dim);
  void* a0[] = {&o, &dout, &delta, (void*)&rows};
  rc = launch(name, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, stream, a0);
  if (rc) return rc;
  snprintf(name, sizeof name, "teeny_fa2_bwd_dq_f32_d%d_%s", head_dim, cz);
  void* a1[] = {&q, &k, &v, &dout, &l, &delta, &dq, &n_ctx_q, &n_ctx_k, &scale, &hq, &hkv};
  rc = launch(name, dim3((n_ctx_q + 63) / 64, batch * hq), dim3(64), 0, stream, a1);
  if (rc) return rc;
  snprintf(name, sizeof name, "teeny_fa2_bwd_dkdv_f32_d%d_%s", head_dim, cz);
  void* a2[] = {&q,  &k,  &v,       &dout,    &l,     &delta, &dk,
                &dv, &n_ctx_q, &n_ctx_k, &scale, &hq,    &hkv};
  return launch(name, dim3((n_ctx_k + 63) / 64, batch * hkv), dim3(64), 0, stream, a2);
}

// ---------------------------------------------------------------------------
// Row-wise norms
// ---------------------------------------------------------------------------
// Picks (VEC, CH) so one wavefront covers a row of N elements.
bool norm_shape(int N, int dtype, int* vec, int* ch) {
  const int v16 = dtype == TEENY_BF16 ? 8 : 4;
  int v = (N % v16 == 0) ? v16 : 1;
  int need = (N + 64 * v - 1) / (64 * v);
  int c = 1;
  while (c < need) c <<= 1;
  if (c > 16) return false;
  *vec = v;
  *ch = c;
  return true;
}

constexpr int kNormBwdMaxParts = 256;

int norm_bwd_parts(int M) {
  int p = (M + 3) / 4;
  return p < kNormBwdMaxParts ? p : kNormBwdMaxParts;
}

}  // namespace

// ===========================================================================
// Exported entry points
// ===========================================================================
extern "C" {

int teeny_abi_version(void) { return TEENY_ABI_VERSION; }

int teeny_last_hip_error(void) { return g_last_hip; }

const char* teeny_strerror(int code) {
  switch (code) {
    case TEENY_OK: return "ok";
    case TEENY_ERR_NULL_POINTER: return "null pointer";
    case TEENY_ERR_INVALID_SHAPE: return "invalid shape";
    case TEENY_ERR_UNSUPPORTED: return "unsupported dtype or head_dim";
    case TEENY_ERR_WORKSPACE: return "workspace missing or too small";
    case TEENY_ERR_HIP: return "HIP runtime error";
    case TEENY_ERR_MODULE: return "code object or kernel could not be loaded";
    case TEENY_ERR_INVALID_VALUE: return "invalid scalar argument";
    case TEENY_ERR_SCRATCH: return "problem needs more than the library's static scratch array";
    case TEENY_ERR_NOT_INITIALIZED: return "teeny_init has not run on the current device";
    default: return "unknown error";
  }
}

int teeny_init(void) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e);
  if (dev < 0 || dev >= kMaxDevices) return TEENY_ERR_HIP;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    DeviceState* st = nullptr;
    int rc = load_device_locked(dev, &st);
    if (rc) return rc;
  }
  // this device's address of the no-allocation entry point's scratch array,
  // asked here once so that entry point never loads or looks anything up
  return teeny_scratch_setup(nullptr);
}

__attribute__((visibility("hidden"))) void teeny_set_last_hip_error(int e) { g_last_hip = e; }
__attribute__((visibility("hidden"))) int teeny_device_ready(void) { return device_ready(); }

int teeny_profile_enable(int on) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  g_prof_on = on != 0;
  if (g_prof_on) prof_clear_locked();
  return TEENY_OK;
}

int teeny_profile_kernel_stats(const char* name, int* launches, double* total_ms) {
  if (!name || !launches || !total_ms) return TEENY_ERR_NULL_POINTER;
  std::lock_guard<std::mutex> lk(g_prof_mu);
  int n = 0;
  double tot = 0.0;
  for (auto& r : g_prof) {
    if (r.name != name) continue;
    hipError_t e = hipEventSynchronize(r.stop);
    if (e != hipSuccess) return hip_fail(e);
    float ms = 0.0f;
    e = hipEventElapsedTime(&ms, r.start, r.stop);
    if (e != hipSuccess) return hip_fail(e);
    ++n;
    tot += ms;
  }
  *launches = n;
  *total_ms = tot;
  return TEENY_OK;
}

int teeny_profile_kernel_names(char* buf, size_t buf_bytes) {
  if (!buf || buf_bytes == 0) return TEENY_ERR_NULL_POINTER;
  std::lock_guard<std::mutex> lk(g_prof_mu);
  std::string out;
  for (auto& r : g_prof) {
    std::string key = r.name + "\n";
    if (out.find(key) == std::string::npos) out += key;
  }
  if (out.size() + 1 > buf_bytes) return TEENY_ERR_INVALID_SHAPE;
  memcpy(buf, out.c_str(), out.size() + 1);
  return TEENY_OK;
}

int teeny_causal_flash_attn2_fwd(const void* q, const void* k, const void* v, void* o, float* l,
                                 int n_ctx_q, int n_ctx_k, float softmax_scale, float neg_inf,
                                 int batch, int n_heads_q, int n_heads_kv, int head_dim,
                                 int dtype, hipStream_t stream) {
  return fa2_fwd(true, q, k, v, o, l, n_ctx_q, n_ctx_k, softmax_scale, neg_inf, batch, n_heads_q,
                 n_heads_kv, head_dim, dtype, stream);
}

int teeny_flash_attn2_fwd(const void* q, const void* k, const void* v, void* o, float* l,
                          int n_ctx_q, int n_ctx_k, float softmax_scale, float neg_inf,
                          int batch, int n_heads_q, int n_heads_kv, int head_dim, int dtype,
                          hipStream_t stream) {
  return fa2_fwd(false, q, k, v, o, l, n_ctx_q, n_ctx_k, softmax_scale, neg_inf, batch,
                 n_heads_q, n_heads_kv, head_dim, dtype, stream);
}

int teeny_flash_attn2_fwd_merged(const void* q, const void* k, const void* v, void* o, float* l,
                                 int n_ctx_q, int n_ctx_k, float softmax_scale, float neg_inf,
                                 int batch, int n_heads_q, int n_heads_kv, int head_dim,
                                 int dtype, int causal, hipStream_t stream) {
  if (dtype != TEENY_BF16) return TEENY_ERR_UNSUPPORTED;  // the bf16 kernels only
  return fa2_fwd(causal != 0, q, k, v, o, l, n_ctx_q, n_ctx_k, softmax_scale, neg_inf, batch,
                 n_heads_q, n_heads_kv, head_dim, dtype, stream, 1);
}

int teeny_flash_attn2_fwd_qkv(const void* qkv, const float* rope_cs, const void* k, const void* v,
                              void* o, float* l, int n_ctx_q, int n_ctx_k, float softmax_scale,
                              float neg_inf, int batch, int n_heads_q, int n_heads_kv,
                              int head_dim, int dtype, int causal, hipStream_t stream) {
  if (dtype != TEENY_BF16) return TEENY_ERR_UNSUPPORTED;  // the bf16 kernels only
  if (!rope_cs) return TEENY_ERR_NULL_POINTER;
  if (reinterpret_cast<uintptr_t>(rope_cs) % 16 != 0) return TEENY_ERR_INVALID_VALUE;
  if (n_heads_q > 0 && n_heads_kv > 0 && n_ctx_q > 0 && batch > 0 &&
      (long)batch * n_ctx_q * (n_heads_q + 2 * n_heads_kv) * head_dim >= kMaxElems)
    return TEENY_ERR_INVALID_SHAPE;
  return fa2_fwd(causal != 0, qkv, k, v, o, l, n_ctx_q, n_ctx_k, softmax_scale, neg_inf, batch,
                 n_heads_q, n_heads_kv, head_dim, dtype, stream, 1, rope_cs);
}

int teeny_rope_table(float* cs, int n_pos, int head_dim, float ln_rope_base,
                     hipStream_t stream) {
  if (!cs) return TEENY_ERR_NULL_POINTER;
  if (n_pos <= 0 || n_pos % 32 != 0 || head_dim <= 0 || head_dim % 16 != 0 ||
      (long)n_pos * head_dim >= kMaxElems)
    return TEENY_ERR_INVALID_SHAPE;
  if (!std::isfinite(ln_rope_base)) return TEENY_ERR_INVALID_VALUE;
  const long n = (long)n_pos * (head_dim / 2);
  void* args[] = {&cs, &n_pos, &head_dim, &ln_rope_base};
  return launch("teeny_rope_table_f32", dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                args);
}

int teeny_causal_flash_attn2_bwd(const void* q, const void* k, const void* v, const void* o,
                                 const void* dout, const float* l, void* dq, void* dk, void* dv,
                                 int n_ctx_q, int n_ctx_k, float softmax_scale, int batch,
                                 int n_heads_q, int n_heads_kv, int head_dim, int dtype,
                                 void* workspace, size_t workspace_bytes, hipStream_t stream) {
  return fa2_bwd(true, q, k, v, o, dout, l, dq, dk, dv, n_ctx_q, n_ctx_k, softmax_scale, batch,
                 n_heads_q, n_heads_kv, head_dim, dtype, workspace, workspace_bytes, stream);
}

int teeny_flash_attn2_bwd(const void* q, const void* k, const void* v, const void* o,
                          const void* dout, const float* l, void* dq, void* dk, void* dv,
                          int n_ctx_q, int n_ctx_k, float softmax_scale, int batch, int n_heads_q,
                          int n_heads_kv, int head_dim, int dtype, void* workspace,
                          size_t workspace_bytes, hipStream_t stream) {
  return fa2_bwd(false, q, k, v, o, dout, l, dq, dk, dv, n_ctx_q, n_ctx_k, softmax_scale, batch,
                 n_heads_q, n_heads_kv, head_dim, dtype, workspace, workspace_bytes, stream);
}

size_t teeny_flash_attn2_bwd_workspace_bytes(int n_ctx_q, int batch, int n_heads_q, int head_dim,
                                             int dtype) {
  if (n_ctx_q <= 0 || batch <= 0 || n_heads_q <= 0 || head_dim <= 0) return 0;
  dtype &= ~TEENY_GRAD_F32;
  return fa2_bwd_ws(n_ctx_q, batch, n_heads_q, head_dim, dtype);
}

size_t teeny_flash_attn2_bwd_workspace_bytes_gqa(int n_ctx_q, int n_ctx_k, int batch,
                                                 int n_heads_q, int n_heads_kv, int head_dim,
                                                 int dtype) {
  if (n_ctx_q <= 0 || n_ctx_k <= 0 || batch <= 0 || n_heads_q <= 0 || n_heads_kv <= 0 ||
      head_dim <= 0 || n_heads_q % n_heads_kv != 0)
    return 0;
  dtype &= ~TEENY_GRAD_F32;
  // the split is planned only for the causal backward
  const int split =
      dkdv_plan(true, n_ctx_q, n_ctx_k, batch, n_heads_q, n_heads_kv, dtype).split;
  return fa2_bwd_ws(n_ctx_q, batch, n_heads_q, head_dim, dtype) +
         dkdv_split_bytes(n_ctx_k, batch, n_heads_kv, head_dim, split);
}

static int rope_impl(const void* x, void* y, int n_ctx, float ln_base, int bh, int head_dim,
                     int dtype, int backward, hipStream_t stream) {
  if (!x || !y) return TEENY_ERR_NULL_POINTER;
  if (!dtype_ok(dtype)) return TEENY_ERR_UNSUPPORTED;
  if (n_ctx <= 0 || bh <= 0 || head_dim <= 0 || (long)bh * n_ctx * head_dim >= kMaxElems)
    return TEENY_ERR_INVALID_SHAPE;
  const int vn = dtype == TEENY_BF16 ? 8 : 4;
  // D a power of two, as the reference requires (src/kernels/rope.rs:56)
  if (head_dim % vn != 0 || (head_dim & (head_dim - 1)) != 0) return TEENY_ERR_UNSUPPORTED;
  if (!std::isfinite(ln_base)) return TEENY_ERR_INVALID_VALUE;
  char name[32];
  snprintf(name, sizeof name, "teeny_rope_%s", dtype_tag(dtype));
  void* args[] = {&x, &y, &bh, &n_ctx, &head_dim, &ln_base, &backward};
  // a thread per (position, 16-byte vector) of 8 rows; head_dim / vn vectors per row
  const int ppw = 256 / (head_dim / vn);  // positions per workgroup
  if (ppw < 1) return TEENY_ERR_UNSUPPORTED;
  if ((bh + 7) / 8 > 65535) return TEENY_ERR_INVALID_SHAPE;
  return launch(name, dim3((n_ctx + ppw - 1) / ppw, (bh + 7) / 8), dim3(256), 0, stream, args);
}

int teeny_rope_fwd(const void* x, void* y, int n_ctx, float ln_rope_base, int bh, int head_dim,
                   int dtype, hipStream_t stream) {
  return rope_impl(x, y, n_ctx, ln_rope_base, bh, head_dim, dtype, 0, stream);
}

int teeny_rope_bwd(const void* dy, void* dx, int n_ctx, float ln_rope_base, int bh, int head_dim,
                   int dtype, hipStream_t stream) {
  return rope_impl(dy, dx, n_ctx, ln_rope_base, bh, head_dim, dtype, 1, stream);
}

static int transpose_impl(const void* src, void* dst, int seq, int heads, int batch,
                          int head_dim, int dtype, int merge, hipStream_t stream) {
  if (!src || !dst) return TEENY_ERR_NULL_POINTER;
  if (!dtype_ok(dtype)) return TEENY_ERR_UNSUPPORTED;
  if (seq <= 0 || heads <= 0 || batch <= 0 || head_dim <= 0 || batch * heads > 65535 ||
      (long)batch * heads * seq * head_dim >= kMaxElems)
    return TEENY_ERR_INVALID_SHAPE;
  if (src == dst) return TEENY_ERR_INVALID_VALUE;  // not an in-place permutation
  int row_bytes = head_dim * (int)dtype_size(dtype);
  if (row_bytes % 4 != 0) return TEENY_ERR_UNSUPPORTED;
  const bool v16 = row_bytes % 16 == 0;
  const int vb = v16 ? 16 : 4;
  long per_slice = (long)seq * (row_bytes / vb);
  unsigned gx = (unsigned)((per_slice + 1023) / 1024);
  void* args[] = {&src, &dst, &seq, &heads, &row_bytes, &merge};
  return launch(v16 ? "teeny_transpose_heads_v16" : "teeny_transpose_heads_v4",
                dim3(gx, batch * heads), dim3(256), 0, stream, args);
}

int teeny_transpose_heads(const void* src, void* dst, int seq_len, int n_heads, int batch,
                          int head_dim, int dtype, hipStream_t stream) {
  return transpose_impl(src, dst, seq_len, n_heads, batch, head_dim, dtype, 0, stream);
}

int teeny_merge_heads(const void* src, void* dst, int seq_len, int n_heads, int batch,
                      int head_dim, int dtype, hipStream_t stream) {
  return transpose_impl(src, dst, seq_len, n_heads, batch, head_dim, dtype, 1, stream);
}

static int norm_fwd_impl(const void* x, const void* res, void* y, void* h, float* rstd,
                         const void* w, int M, int N, float eps, int dtype, hipStream_t stream) {
  if (!x || !y || !w) return TEENY_ERR_NULL_POINTER;
  if (!dtype_ok(dtype)) return TEENY_ERR_UNSUPPORTED;
  if (M <= 0 || N <= 0 || (long)M * N >= kMaxElems) return TEENY_ERR_INVALID_SHAPE;
  if (!(eps >= 0.0f) || !std::isfinite(eps)) return TEENY_ERR_INVALID_VALUE;
  int vec, ch;
  if (!norm_shape(N, dtype, &vec, &ch)) return TEENY_ERR_UNSUPPORTED;
  char name[64];
  void* args[] = {&x, &res, &y, &h, &rstd, &w, &M, &N, &eps};
  // Fewer rows than CUs: a workgroup per row (4 wavefronts share a row)
  // when the row is vectorised and fits 256 threads x 4 vectors.
  if (M < 256 && vec > 1 && ch <= 16) {
    if (dtype == TEENY_BF16 && ch == 8)  // rows of 4096: 512 threads, one vector each
      return launch("teeny_rmsnorm_fwd_wg_bf16_v8_c1_t512", dim3(M), dim3(512), 0, stream, args);
    snprintf(name, sizeof name, "teeny_rmsnorm_fwd_wg_%s_v%d_c%d", dtype_tag(dtype), vec,
             ch <= 4 ? 1 : ch / 4);
    return launch(name, dim3(M), dim3(256), 0, stream, args);
  }
  // rows strided over the workgroups of 4 wavefronts the device holds at
  // once, each wavefront loading its next row while it stores the current
  // one (8192 x 2048 bf16: 1024 workgroups 11.2 us, 512 11.4, one row per
  // wavefront 11.7-13.4, measured)
  // rows of exactly ch chunks of 64 lanes x vec elements need no bounds tests
  snprintf(name, sizeof name, "teeny_%s_fwd_%s_v%d_c%d%s", res ? "addnorm" : "rmsnorm",
           dtype_tag(dtype), vec, ch, N == ch * 64 * vec ? "_full" : "");
  const int rows4 = (M + 3) / 4;
  const int cap = resident_groups(name, 256, 1024);
  return launch(name, dim3(rows4 < cap ? rows4 : cap), dim3(256), 0, stream, args);
}

int teeny_fused_add_rmsnorm_partials_fwd(const float* parts, int n_parts, const void* residual,
                                         void* y, void* h, float* rstd, const void* weight,
                                         int M, int N, float eps, int dtype,
                                         hipStream_t stream) {
  if (!parts || !residual || !y || !h || !weight) return TEENY_ERR_NULL_POINTER;
  if (!dtype_ok(dtype)) return TEENY_ERR_UNSUPPORTED;
  if (M <= 0 || N <= 0 || n_parts <= 0 || (long)n_parts * M * N >= kMaxElems)
    return TEENY_ERR_INVALID_SHAPE;
  if (!(eps >= 0.0f) || !std::isfinite(eps)) return TEENY_ERR_INVALID_VALUE;
  int vec, ch;
  if (!norm_shape(N, dtype, &vec, &ch) || vec == 1) return TEENY_ERR_UNSUPPORTED;
  char name[64];
  void* args[] = {&parts, &n_parts, &residual, &y, &h, &rstd, &weight, &M, &N, &eps};
  if (dtype == TEENY_BF16 && ch == 8)  // as the unsplit rows of 4096: 512 threads
    return launch("teeny_addnorm_parts_fwd_bf16_v8_c1_t512", dim3(M), dim3(512), 0, stream, args);
  snprintf(name, sizeof name, "teeny_addnorm_parts_fwd_%s_v%d_c%d", dtype_tag(dtype), vec,
           ch <= 4 ? 1 : ch / 4);
  return launch(name, dim3(M), dim3(256), 0, stream, args);
}

int teeny_fused_add_rmsnorm_fwd(const void* x, const void* residual, void* y, void* h,
                                float* rstd, const void* weight, int M, int N, float eps,
                                int dtype, hipStream_t stream) {
  if (!residual || !h || !rstd) return TEENY_ERR_NULL_POINTER;
  return norm_fwd_impl(x, residual, y, h, rstd, weight, M, N, eps, dtype, stream);
}

int teeny_rmsnorm_fwd(const void* x, void* y, float* rstd, const void* weight, int M, int N,
                      float eps, int dtype, hipStream_t stream) {
  return norm_fwd_impl(x, nullptr, y, nullptr, rstd, weight, M, N, eps, dtype, stream);
}

size_t teeny_fused_add_rmsnorm_bwd_workspace_bytes(int M, int N) {
  if (M <= 0 || N <= 0) return 0;
  return align256((size_t)norm_bwd_parts(M) * N * sizeof(float));
}

static int norm_bwd_impl(bool ref_formula, const void* dy, const void* h, void* dx,
                         void* dresidual, void* dweight, const void* weight, const float* rstd,
                         int M, int N, int dtype, void* workspace, size_t workspace_bytes,
                         hipStream_t stream) {
  if (!dy || !h || !dx || !dweight || !weight || !rstd) return TEENY_ERR_NULL_POINTER;
  if (!dtype_ok(dtype)) return TEENY_ERR_UNSUPPORTED;
  if (M <= 0 || N <= 0 || (long)M * N >= kMaxElems) return TEENY_ERR_INVALID_SHAPE;
  int vec, ch;
  if (!norm_shape(N, dtype, &vec, &ch)) return TEENY_ERR_UNSUPPORTED;
  if (!workspace || workspace_bytes < teeny_fused_add_rmsnorm_bwd_workspace_bytes(M, N))
    return TEENY_ERR_WORKSPACE;
  int parts = norm_bwd_parts(M);
  float* part = (float*)workspace;
  char name[64];
  snprintf(name, sizeof name, "teeny_%s_bwd_%s_v%d_c%d", ref_formula ? "addnorm" : "rmsnorm",
           dtype_tag(dtype), vec, ch);
  void* a0[] = {&dy, &h, &dx, &dresidual, &part, &weight, &rstd, &M, &N};
  int rc = launch(name, dim3(parts), dim3(256), 0, stream, a0);
  if (rc) return rc;
  snprintf(name, sizeof name, "teeny_rmsnorm_dw_reduce_%s", dtype_tag(dtype));
  void* a1[] = {&part, &dweight, &parts, &N};
  return launch(name, dim3((N + 255) / 256), dim3(256), 0, stream, a1);
}

int teeny_fused_add_rmsnorm_bwd(const void* dy, const void* h, void* dx, void* dresidual,
                                void* dweight, const void* weight, const float* rstd, int M,
                                int N, int dtype, void* workspace, size_t workspace_bytes,
                                hipStream_t stream) {
  return norm_bwd_impl(true, dy, h, dx, dresidual, dweight, weight, rstd, M, N, dtype, workspace,
                       workspace_bytes, stream);
}

int teeny_rmsnorm_bwd(const void* dy, const void* x, void* dx, void* dweight, const void* weight,
                      const float* rstd, int M, int N, int dtype, void* workspace,
                      size_t workspace_bytes, hipStream_t stream) {
  return norm_bwd_impl(false, dy, x, dx, nullptr, dweight, weight, rstd, M, N, dtype, workspace,
                       workspace_bytes, stream);
}

static int swiglu_impl(bool bwd, const void* grad, const void* z, void* out, int M, int d_ff,
                       int dtype, hipStream_t stream) {
  if (!z || !out || (bwd && !grad)) return TEENY_ERR_NULL_POINTER;
  if (!dtype_ok(dtype)) return TEENY_ERR_UNSUPPORTED;
  if (M <= 0 || d_ff <= 0 || M > 65535 * 64 || (long)M * 2 * d_ff >= kMaxElems)
    return TEENY_ERR_INVALID_SHAPE;
  const int v16 = dtype == TEENY_BF16 ? 8 : 4;
  const int vec = d_ff % v16 == 0 ? v16 : 1;
  if (M > 65535) return TEENY_ERR_INVALID_SHAPE;
  char name[48];
  snprintf(name, sizeof name, "teeny_swiglu_%s_%s_v%d", bwd ? "bwd" : "fwd", dtype_tag(dtype),
           vec);
  dim3 grid((d_ff / vec + 255) / 256, M);
  if (bwd) {
    void* args[] = {&grad, &z, &out, &M, &d_ff};
    return launch(name, grid, dim3(256), 0, stream, args);
  }
  void* args[] = {&z, &out, &M, &d_ff};
  return launch(name, grid, dim3(256), 0, stream, args);
}

int teeny_swiglu_fwd(const void* z, void* out, int M, int d_ff, int dtype, hipStream_t stream) {
  return swiglu_impl(false, nullptr, z, out, M, d_ff, dtype, stream);
}

int teeny_swiglu_bwd(const void* grad, const void* z, void* dz, int M, int d_ff, int dtype,
                     hipStream_t stream) {
  return swiglu_impl(true, grad, z, dz, M, d_ff, dtype, stream);
}

int teeny_add(const void* a, const void* b, void* y, long n, int dtype, hipStream_t stream) {
  if (!a || !b || !y) return TEENY_ERR_NULL_POINTER;
  if (!dtype_ok(dtype)) return TEENY_ERR_UNSUPPORTED;
  if (n <= 0 || n >= (1L << 40)) return TEENY_ERR_INVALID_SHAPE;
  // whole 16-byte vectors: every pointer 16-byte aligned
  if (((uintptr_t)a | (uintptr_t)b | (uintptr_t)y) % 16 != 0) return TEENY_ERR_INVALID_VALUE;
  char name[32];
  snprintf(name, sizeof name, "teeny_add_%s", dtype_tag(dtype));
  void* args[] = {&a, &b, &y, &n};
  const long blocks = (n + 8L * 256 - 1) / (8L * 256);
  return launch(name, dim3((unsigned)blocks), dim3(256), 0, stream, args);
}

static int qkv_rope_split_check(const void* qkv, const void* q_out, const void* k_cache,
                                const void* v_cache, int batch, int seq_len, int pos0,
                                int cache_len, int n_heads_q, int n_heads_kv, int head_dim,
                                float ln_rope_base, int dtype) {
  if (!qkv || !k_cache || !v_cache) return TEENY_ERR_NULL_POINTER;
  if (!dtype_ok(dtype)) return TEENY_ERR_UNSUPPORTED;
  if (batch <= 0 || seq_len <= 0 || pos0 < 0 || n_heads_q <= 0 || n_heads_kv <= 0 ||
      n_heads_q % n_heads_kv != 0 || head_dim <= 0 || cache_len < pos0 + seq_len ||
      (long)batch * seq_len * (n_heads_q + 2 * n_heads_kv) * head_dim >= kMaxElems ||
      (long)batch * n_heads_kv * cache_len * head_dim >= kMaxElems)
    return TEENY_ERR_INVALID_SHAPE;
  const int vn = dtype == TEENY_BF16 ? 8 : 4;
  if (head_dim % vn != 0 || head_dim % 2 != 0) return TEENY_ERR_UNSUPPORTED;
  if (!std::isfinite(ln_rope_base)) return TEENY_ERR_INVALID_VALUE;
  // row kernel: one thread per 16-byte vector of a head row, 8 head rows each
  if (head_dim / vn > 256) return TEENY_ERR_UNSUPPORTED;
  if ((long)batch * ((n_heads_q + 2 * n_heads_kv + 7) / 8) > 65535 ||
      (long)batch * ((n_heads_q + 2 * n_heads_kv + 3) / 4) > 65535)
    return TEENY_ERR_INVALID_SHAPE;
  return TEENY_OK;
}

static int qkv_rope_split_impl(const void* qkv, void* q_out, void* k_cache, void* v_cache,
                               int batch, int seq_len, const int32_t* pos_dev, int pos0,
                               int cache_len, int n_heads_q, int n_heads_kv, int head_dim,
                               float ln_rope_base, int dtype, hipStream_t stream) {
  int rc = qkv_rope_split_check(qkv, q_out, k_cache, v_cache, batch, seq_len, pos0, cache_len,
                                n_heads_q, n_heads_kv, head_dim, ln_rope_base, dtype);
  if (rc) return rc;
  // 256 threads: (256 / vectors per row) positions x 8 head rows each; no
  // q_out: the K and V head rows only
  const int rows = q_out ? n_heads_q + 2 * n_heads_kv : 2 * n_heads_kv;
  const long gy = (long)batch * ((rows + 7) / 8);
  const int ppw = 256 / (head_dim / (dtype == TEENY_BF16 ? 8 : 4));
  char name[48];
  snprintf(name, sizeof name, "teeny_qkv_rope_split_%s", dtype_tag(dtype));
  void* args[] = {&qkv,      &q_out,     &k_cache,   &v_cache,    &seq_len,   &pos_dev,
                  &pos0,     &cache_len, &n_heads_q, &n_heads_kv, &head_dim,  &ln_rope_base};
  return launch(name, dim3((seq_len + ppw - 1) / ppw, (unsigned)gy), dim3(256), 0, stream, args);
}

int teeny_qkv_rope_split(const void* qkv, void* q_out, void* k_cache, void* v_cache, int batch,
                         int seq_len, int pos0, int cache_len, int n_heads_q, int n_heads_kv,
                         int head_dim, float ln_rope_base, int dtype, hipStream_t stream) {
  return qkv_rope_split_impl(qkv, q_out, k_cache, v_cache, batch, seq_len, nullptr, pos0,
                             cache_len, n_heads_q, n_heads_kv, head_dim, ln_rope_base, dtype,
                             stream);
}

int teeny_qkv_rope_split_dev(const void* qkv, void* q_out, void* k_cache, void* v_cache,
                             int batch, int seq_len, const int32_t* pos0, int cache_len,
                             int n_heads_q, int n_heads_kv, int head_dim, float ln_rope_base,
                             int dtype, hipStream_t stream) {
  if (!pos0) return TEENY_ERR_NULL_POINTER;
  return qkv_rope_split_impl(qkv, q_out, k_cache, v_cache, batch, seq_len, pos0, 0, cache_len,
                             n_heads_q, n_heads_kv, head_dim, ln_rope_base, dtype, stream);
}

int teeny_qkv_rope_split_partials_dev(const float* parts, int n_parts, void* q_out,
                                      void* k_cache, void* v_cache, int batch, int seq_len,
                                      const int32_t* pos0, int cache_len, int n_heads_q,
                                      int n_heads_kv, int head_dim, float ln_rope_base,
                                      int dtype, hipStream_t stream) {
  if (!parts || !pos0 || !q_out) return TEENY_ERR_NULL_POINTER;
  if (n_parts <= 0) return TEENY_ERR_INVALID_SHAPE;
  // shape checks on a stand-in qkv pointer, then the partial-input kernel
  int rc = qkv_rope_split_check(parts, q_out, k_cache, v_cache, batch, seq_len, 0, cache_len,
                                n_heads_q, n_heads_kv, head_dim, ln_rope_base, dtype);
  if (rc) return rc;
  const int htot = n_heads_q + 2 * n_heads_kv;
  long part_stride = (long)batch * seq_len * htot * head_dim;
  if (part_stride * n_parts >= kMaxElems || (long)batch * ((htot + 3) / 4) > 65535)
    return TEENY_ERR_INVALID_SHAPE;
  char name[48];
  snprintf(name, sizeof name, "teeny_qkv_parts_rope_split_%s", dtype_tag(dtype));
  int pos_imm = 0;
  void* args[] = {&parts,     &n_parts,   &part_stride, &q_out,      &k_cache,
                  &v_cache,   &seq_len,   &pos0,        &pos_imm,    &cache_len,
                  &n_heads_q, &n_heads_kv, &head_dim,   &ln_rope_base};
  // 4 head rows x 4 positions per workgroup (the partial-input kernel's tile)
  unsigned shmem = 4u * (unsigned)(head_dim / 2) * 8u;
  return launch(name, dim3((seq_len + 3) / 4, (unsigned)((long)batch * ((htot + 3) / 4))),
                dim3(256), shmem, stream, args);
}

int teeny_decode_qkv_attention_dev(const float* parts, int n_parts, void* k_cache,
                                   void* v_cache, void* o, int batch, int n_heads_q,
                                   int n_heads_kv, int head_dim, int cache_len,
                                   const int32_t* n_past, float ln_rope_base,
                                   float softmax_scale, int dtype, hipStream_t stream) {
  if (!parts || !k_cache || !v_cache || !o || !n_past) return TEENY_ERR_NULL_POINTER;
  if (dtype != TEENY_BF16 || (head_dim != 64 && head_dim != 128)) return TEENY_ERR_UNSUPPORTED;
  if (n_parts <= 0 || batch <= 0 || n_heads_q <= 0 || n_heads_kv <= 0 || cache_len <= 0 ||
      n_heads_q % n_heads_kv != 0)
    return TEENY_ERR_INVALID_SHAPE;
  // the group's q rows are the 32 rows of one matrix product
  if (n_heads_q / n_heads_kv > 32) return TEENY_ERR_UNSUPPORTED;
  const int htot = n_heads_q + 2 * n_heads_kv;
  long part_stride = (long)batch * htot * head_dim;
  // the kernel addresses one (b, kv head) cache slab with 32-bit byte offsets
  if (part_stride * n_parts >= kMaxElems ||
      (long)batch * n_heads_kv * cache_len * head_dim >= kMaxElems ||
      (long)cache_len * head_dim * 2 >= kMaxElems)
    return TEENY_ERR_INVALID_SHAPE;
  if (!std::isfinite(ln_rope_base) || !scale_ok(softmax_scale, dtype))
    return TEENY_ERR_INVALID_VALUE;
  char name[48];
  snprintf(name, sizeof name, "teeny_decode_qkv_attn_bf16_d%d", head_dim);
  void* args[] = {&parts,      &n_parts,   &part_stride, &k_cache,      &v_cache,
                  &o,          &n_heads_q, &n_heads_kv,  &n_past,       &cache_len,
                  &ln_rope_base, &softmax_scale};
  return launch(name, dim3((unsigned)(batch * n_heads_kv)), dim3(512), 0, stream, args);
}

static int decode_chunks(int n_keys) { return (n_keys + 255) / 256; }  // fp32 kernel

// bf16 matrix-core kernel: keys per wavefront chosen so that one step runs
// about 1024 wavefronts (a multiple of the 32-key tile, 64 .. 1024).  At the
// Llama-8B decode shape (B16, 8 kv heads, 640 cached rows) that is 96 keys
// per wavefront: attention + combine 11.3-12.1 us per layer, against
// 13.1-14.4 us at 2048 wavefronts (64 keys) and 11.6-12.0 us at 512 (measured).
static int decode_keys_per_split(int n_keys, int batch, int n_heads_kv) {
  long per = ((long)n_keys * batch * n_heads_kv + 1023) / 1024;
  per = (per + 31) / 32 * 32;
  if (per < 64) per = 64;
  if (per > 1024) per = 1024;
  return (int)per;
}

size_t teeny_decode_attention_workspace_bytes(int batch, int n_heads_q, int n_keys,
                                              int head_dim) {
  if (batch <= 0 || n_heads_q <= 0 || n_keys <= 0 || head_dim <= 0) return 0;
  // the finest split either kernel uses: 64 keys
  size_t rows = (size_t)batch * n_heads_q * ((n_keys + 63) / 64);
  return 2 * align256(rows * sizeof(float)) + align256(rows * head_dim * sizeof(float));
}

// n_keys: the keys attended (host value), or with n_past the grid's capacity
// and the kernel attends *n_past + 1 of them.
static int decode_attention_impl(const void* q, const void* k_cache, const void* v_cache,
                                 void* o, int batch, int n_heads_q, int n_heads_kv,
                                 const int32_t* n_past, int n_keys, int cache_len, int head_dim,
                                 float softmax_scale, int dtype, void* workspace,
                                 size_t workspace_bytes, hipStream_t stream) {
  if (!q || !k_cache || !v_cache || !o) return TEENY_ERR_NULL_POINTER;
  if (!dtype_ok(dtype)) return TEENY_ERR_UNSUPPORTED;
  if (batch <= 0 || n_heads_q <= 0 || n_heads_kv <= 0 || n_heads_q % n_heads_kv != 0 ||
      n_keys <= 0 || cache_len < n_keys || batch * n_heads_kv > 65535 ||
      (long)batch * n_heads_kv * cache_len * head_dim >= kMaxElems)
    return TEENY_ERR_INVALID_SHAPE;
  if (n_heads_q / n_heads_kv > 16) return TEENY_ERR_UNSUPPORTED;
  if (head_dim < 8 || head_dim > 128 || (head_dim & (head_dim - 1)) != 0)
    return TEENY_ERR_UNSUPPORTED;
  if (!std::isfinite(softmax_scale) || softmax_scale <= 0.0f) return TEENY_ERR_INVALID_VALUE;
  if (!workspace ||
      workspace_bytes < teeny_decode_attention_workspace_bytes(batch, n_heads_q, n_keys, head_dim))
    return TEENY_ERR_WORKSPACE;
  // the matrix-core kernel addresses one (b, kv head) cache slab with 32-bit
  // byte offsets
  const bool mfma = dtype == TEENY_BF16 && (head_dim == 64 || head_dim == 128) &&
                    (long)cache_len * head_dim * 2 < (1L << 31);
  const int per = mfma ? decode_keys_per_split(n_keys, batch, n_heads_kv) : 256;
  int n_chunks = mfma ? (n_keys + per - 1) / per : decode_chunks(n_keys);
  size_t rows = (size_t)batch * n_heads_q * n_chunks;
  float* pm = (float*)workspace;
  float* pl = (float*)((char*)workspace + align256(rows * sizeof(float)));
  float* po = (float*)((char*)workspace + 2 * align256(rows * sizeof(float)));
  char name[48];
  int rc;
  if (mfma) {
    snprintf(name, sizeof name, "teeny_decode_mfma_bf16_d%d", head_dim);
    int per_split = per;
    void* a0[] = {&q,  &k_cache, &v_cache, &pm,        &pl,        &po,           &n_heads_q,
                  &n_heads_kv, &n_past,  &n_keys,   &cache_len, &per_split, &softmax_scale};
    rc = launch(name, dim3(n_chunks, batch * n_heads_kv), dim3(64), 0, stream, a0);
  } else {
    snprintf(name, sizeof name, "teeny_decode_attn_partial_%s", dtype_tag(dtype));
    void* a0[] = {&q,      &k_cache, &v_cache,   &pm,       &pl,           &po, &n_heads_q,
                  &n_heads_kv, &n_past, &n_keys, &cache_len, &head_dim, &softmax_scale};
    rc = launch(name, dim3(n_chunks, batch * n_heads_kv), dim3(256), 0, stream, a0);
  }
  if (rc) return rc;
  snprintf(name, sizeof name, "teeny_decode_attn_combine_%s", dtype_tag(dtype));
  void* a1[] = {&pm, &pl, &po, &o, &n_chunks, &head_dim};
  return launch(name, dim3(batch * n_heads_q), dim3(head_dim), 0, stream, a1);
}

int teeny_decode_attention(const void* q, const void* k_cache, const void* v_cache, void* o,
                           int batch, int n_heads_q, int n_heads_kv, int n_keys, int cache_len,
                           int head_dim, float softmax_scale, int dtype, void* workspace,
                           size_t workspace_bytes, hipStream_t stream) {
  return decode_attention_impl(q, k_cache, v_cache, o, batch, n_heads_q, n_heads_kv, nullptr,
                               n_keys, cache_len, head_dim, softmax_scale, dtype, workspace,
                               workspace_bytes, stream);
}

int teeny_decode_attention_dev(const void* q, const void* k_cache, const void* v_cache, void* o,
                               int batch, int n_heads_q, int n_heads_kv, const int32_t* n_past,
                               int max_keys, int cache_len, int head_dim, float softmax_scale,
                               int dtype, void* workspace, size_t workspace_bytes,
                               hipStream_t stream) {
  if (!n_past) return TEENY_ERR_NULL_POINTER;
  return decode_attention_impl(q, k_cache, v_cache, o, batch, n_heads_q, n_heads_kv, n_past,
                               max_keys, cache_len, head_dim, softmax_scale, dtype, workspace,
                               workspace_bytes, stream);
}

int teeny_argmax_rows(const void* x, int64_t* out, int rows, int cols, int dtype,
                      hipStream_t stream) {
  if (!x || !out) return TEENY_ERR_NULL_POINTER;
  if (!dtype_ok(dtype)) return TEENY_ERR_UNSUPPORTED;
  if (rows <= 0 || cols <= 0 || (long)rows * cols >= kMaxElems * 2)
    return TEENY_ERR_INVALID_SHAPE;
  char name[48];
  snprintf(name, sizeof name, "teeny_argmax_rows_%s", dtype_tag(dtype));
  void* args[] = {&x, &out, &cols};
  return launch(name, dim3(rows), dim3(1024), 0, stream, args);
}

// Decode-step linear layers (linear_bf16.hip): 512 threads, 128 W rows per
// workgroup (64 gate + 64 up rows for SwiGLU), x staged in 512-wide K chunks.
static int linear_sk_check(const void* x, const void* w, const void* y, int M, int N, int K,
                           long w_rows, int row_tile) {
  if (!x || !w || !y) return TEENY_ERR_NULL_POINTER;
  if (M <= 0 || N <= 0 || K <= 0 || w_rows * K >= kMaxElems * 2) return TEENY_ERR_INVALID_SHAPE;
  if (M > 16 || N % row_tile != 0 || K % 128 != 0) return TEENY_ERR_UNSUPPORTED;
  return TEENY_OK;
}

// This library's matrix-core GEMM (gemm_bf16.hip: 256 x 256 tiles of y, 512
// threads), any M; N and K multiples of 64.
int teeny_gemm_bf16(const void* x, const void* w, void* y, int M, int N, int K,
                    hipStream_t stream) {
  if (!x || !w || !y) return TEENY_ERR_NULL_POINTER;
  if (M <= 0 || N <= 0 || K <= 0 || (long)N * K >= kMaxElems * 2) return TEENY_ERR_INVALID_SHAPE;
  if (N % 64 != 0 || K % 64 != 0) return TEENY_ERR_UNSUPPORTED;
  // a workgroup addresses its 256 rows of x and of w with 32-bit byte offsets
  if ((long)K * 2 * 256 >= (1L << 31)) return TEENY_ERR_INVALID_SHAPE;
  int tiles_m = (M + 255) / 256, tiles_n = (N + 255) / 256;
  if ((long)tiles_m * tiles_n >= (1L << 31)) return TEENY_ERR_INVALID_SHAPE;
  void* args[] = {&x, &w, &y, &M, &N, &K, &tiles_m, &tiles_n};
  return launch("teeny_gemm_bf16_nt", dim3(tiles_m * tiles_n), dim3(512), 0, stream, args);
}

// Any M: up to 16 rows (a decode step) stream the weight through
// linear_bf16.hip's kernels when N and K are multiples of 128; more rows go
// to hipBLASLt (blaslt.cpp), or to teeny_gemm_bf16 where hipBLASLt is not
// available for the device or shape.
int teeny_linear_bf16(const void* x, const void* w, void* y, int M, int N, int K,
                      hipStream_t stream) {
  if (!x || !w || !y) return TEENY_ERR_NULL_POINTER;
  if (M <= 0 || N <= 0 || K <= 0 || (long)N * K >= kMaxElems * 2) return TEENY_ERR_INVALID_SHAPE;
  if (M <= 16 && N % 128 == 0 && K % 128 == 0) {
    void* args[] = {&x, &w, &y, &M, &N, &K};
    return launch("teeny_linear_sk_bf16", dim3(N / 128), dim3(512), 0, stream, args);
  }
  if (N % 64 != 0 || K % 64 != 0) return TEENY_ERR_UNSUPPORTED;
  if ((long)K * 2 * 256 >= (1L << 31)) return TEENY_ERR_INVALID_SHAPE;
  if (M > 16 && teeny_lt_gemm_bf16(x, w, y, M, N, K, stream) == 0) return TEENY_OK;
  return teeny_gemm_bf16(x, w, y, M, N, K, stream);
}

// fp32 products (the reference's precision): this library's fp32 GEMM
// (gemm_f32.hip: 128 x 128 tiles of y, 256 threads), any M and N, K a
// multiple of 4, 16-byte aligned x and w.
static int gemm_f32_check(const void* x, const void* w, const void* y, int M, int N, int K) {
  if (!x || !w || !y) return TEENY_ERR_NULL_POINTER;
  if (M <= 0 || N <= 0 || K <= 0 || (long)N * K >= kMaxElems * 2 ||
      (long)M * K >= kMaxElems * 2 || (long)M * N >= kMaxElems * 2)
    return TEENY_ERR_INVALID_SHAPE;
  if (K % 4 != 0) return TEENY_ERR_UNSUPPORTED;
  if (((uintptr_t)x | (uintptr_t)w) % 16 != 0) return TEENY_ERR_INVALID_VALUE;
  if ((M + 127) / 128 > 65535) return TEENY_ERR_INVALID_SHAPE;
  return TEENY_OK;
}

int teeny_gemm_f32(const void* x, const void* w, void* y, int M, int N, int K,
                   hipStream_t stream) {
  int rc = gemm_f32_check(x, w, y, M, N, K);
  if (rc) return rc;
  void* args[] = {&x, &w, &y, &M, &N, &K};
  return launch("teeny_gemm_f32_nt", dim3((N + 127) / 128, (M + 127) / 128), dim3(256), 0, stream,
                args);
}

// hipBLASLt's fp32 GEMM (no workspace), or teeny_gemm_f32 where hipBLASLt
// does not take the device or shape, or the stream is capturing.
int teeny_linear_f32(const void* x, const void* w, void* y, int M, int N, int K,
                     hipStream_t stream) {
  int rc = gemm_f32_check(x, w, y, M, N, K);
  if (rc) return rc;
  if (teeny_lt_gemm_f32(x, w, y, M, N, K, stream) == 0) return TEENY_OK;
  return teeny_gemm_f32(x, w, y, M, N, K, stream);
}

// Any M, as teeny_linear_bf16: up to 16 rows through linear_bf16.hip's
// weight-streaming kernel when F % 64 and K % 128 are 0; otherwise the GEMM
// with the SwiGLU epilogue (256 rows x 128 features per workgroup).
int teeny_linear_swiglu_bf16(const void* x, const void* w, void* y, int M, int F, int K,
                             hipStream_t stream) {
  if (!x || !w || !y) return TEENY_ERR_NULL_POINTER;
  if (M <= 0 || F <= 0 || K <= 0 || 2L * F * K >= kMaxElems * 2) return TEENY_ERR_INVALID_SHAPE;
  if (M <= 16 && F % 64 == 0 && K % 128 == 0) {
    void* args[] = {&x, &w, &y, &M, &F, &K};
    return launch("teeny_linear_sk_swiglu_bf16", dim3(F / 64), dim3(512), 0, stream, args);
  }
  if (F % 32 != 0 || K % 64 != 0) return TEENY_ERR_UNSUPPORTED;
  if ((long)K * 2 * 256 >= (1L << 31)) return TEENY_ERR_INVALID_SHAPE;
  int tiles_m = (M + 255) / 256, tiles_n = (F + 127) / 128;
  if ((long)tiles_m * tiles_n >= (1L << 31)) return TEENY_ERR_INVALID_SHAPE;
  void* args[] = {&x, &w, &y, &M, &F, &K, &tiles_m, &tiles_n};
  return launch("teeny_gemm_swiglu_bf16_nt", dim3(tiles_m * tiles_n), dim3(512), 0, stream, args);
}

int teeny_linear_partials_count(int K, int k_split) {
  if (K <= 0 || k_split <= 0) return 0;
  if (k_split >= K) return 1;
  return (K + k_split - 1) / k_split;
}

int teeny_linear_partials_bf16(const void* x, const void* w, float* parts, int M, int N, int K,
                               int k_split, hipStream_t stream) {
  int rc = linear_sk_check(x, w, parts, M, N, K, N, 128);
  if (rc) return rc;
  if (k_split <= 0) return TEENY_ERR_INVALID_VALUE;
  if (k_split >= K) k_split = K;
  else if (k_split % 128 != 0) return TEENY_ERR_INVALID_VALUE;  // whole 128-wide K steps
  const int n = teeny_linear_partials_count(K, k_split);
  if (n > 65535) return TEENY_ERR_INVALID_SHAPE;
  void* args[] = {&x, &w, &parts, &M, &N, &K, &k_split};
  return launch("teeny_linear_sk_part_bf16", dim3(N / 128, n), dim3(512), 0, stream, args);
}

// The streaming layout of a decode weight (linear_bf16.hip): a copy of W in
// the order the decode kernels' wavefronts load it, 16-byte pieces, 256
// threads per workgroup.
int teeny_linear_stream_layout_bf16(const void* w, void* w_s, int N, int K, hipStream_t stream) {
  if (!w || !w_s) return TEENY_ERR_NULL_POINTER;
  if (N <= 0 || K <= 0 || (long)N * K >= kMaxElems * 2) return TEENY_ERR_INVALID_SHAPE;
  if (N % 16 != 0 || K % 128 != 0) return TEENY_ERR_UNSUPPORTED;
  const char *a = (const char*)w, *b = (const char*)w_s;
  const long bytes = (long)N * K * 2;
  if (a < b + bytes && b < a + bytes) return TEENY_ERR_INVALID_VALUE;  // in place or overlapping
  long n_pieces = (long)N * K / 8;
  void* args[] = {&w, &w_s, &N, &K, &n_pieces};
  return launch("teeny_linear_stream_layout_bf16", dim3((unsigned)((n_pieces + 255) / 256)),
                dim3(256), 0, stream, args);
}

// teeny_linear_bf16, teeny_linear_swiglu_bf16 and teeny_linear_partials_bf16
// at up to 16 rows with the weight in the streaming layout: the same kernels
// reading the layout, the same outputs.
int teeny_linear_sl_bf16(const void* x, const void* w_s, void* y, int M, int N, int K,
                         hipStream_t stream) {
  int rc = linear_sk_check(x, w_s, y, M, N, K, N, 128);
  if (rc) return rc;
  void* args[] = {&x, &w_s, &y, &M, &N, &K};
  return launch("teeny_linear_sl_bf16", dim3(N / 128), dim3(512), 0, stream, args);
}

int teeny_linear_swiglu_sl_bf16(const void* x, const void* w_s, void* y, int M, int F, int K,
                                hipStream_t stream) {
  int rc = linear_sk_check(x, w_s, y, M, F, K, 2L * F, 64);
  if (rc) return rc;
  void* args[] = {&x, &w_s, &y, &M, &F, &K};
  return launch("teeny_linear_sl_swiglu_bf16", dim3(F / 64), dim3(512), 0, stream, args);
}

int teeny_linear_partials_sl_bf16(const void* x, const void* w_s, float* parts, int M, int N,
                                  int K, int k_split, hipStream_t stream) {
  int rc = linear_sk_check(x, w_s, parts, M, N, K, N, 128);
  if (rc) return rc;
  if (k_split <= 0) return TEENY_ERR_INVALID_VALUE;
  if (k_split >= K) k_split = K;
  else if (k_split % 128 != 0) return TEENY_ERR_INVALID_VALUE;  // whole 128-wide K steps
  const int n = teeny_linear_partials_count(K, k_split);
  if (n > 65535) return TEENY_ERR_INVALID_SHAPE;
  void* args[] = {&x, &w_s, &parts, &M, &N, &K, &k_split};
  return launch("teeny_linear_sl_part_bf16", dim3(N / 128, n), dim3(512), 0, stream, args);
}

int teeny_token_embed_fwd(const void* ids, const void* weight, void* out, int seq_len,
                          int d_model, int vocab_size, int ids_dtype, int dtype,
                          hipStream_t stream) {
  if (!ids || !weight || !out) return TEENY_ERR_NULL_POINTER;
  if (!dtype_ok(dtype) || (ids_dtype != TEENY_F32 && ids_dtype != TEENY_I32))
    return TEENY_ERR_UNSUPPORTED;
  if (seq_len <= 0 || d_model <= 0 || vocab_size <= 0 || seq_len > 65535 ||
      (long)vocab_size * d_model >= kMaxElems * 2)
    return TEENY_ERR_INVALID_SHAPE;
  int row_bytes = d_model * (int)dtype_size(dtype);
  if (row_bytes % 4 != 0) return TEENY_ERR_UNSUPPORTED;
  const bool v16 = row_bytes % 16 == 0;
  const int vb = v16 ? 16 : 4;
  char name[48];
  snprintf(name, sizeof name, "teeny_embed_%sids_v%d", ids_dtype == TEENY_I32 ? "i32" : "f32",
           vb);
  void* args[] = {&ids, &weight, &out, &row_bytes, &vocab_size};
  dim3 grid((row_bytes / vb + 255) / 256, seq_len);
  return launch(name, grid, dim3(256), 0, stream, args);
}

}  // extern "C"
