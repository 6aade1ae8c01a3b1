// The plain fp32 score GEMM S = X W^T through hipBLASLt (a TN sgemm in its
// column-major terms: S^T (m x n) = W (d x m)^T X (d x n), every leading
// dimension the row length).  The evaluation pass's score GEMM is a plain
// GEMM - the epilogue runs as its own kernel - and the library's
// Tensile kernels (persistent, 1 wave per SIMD, 64-deep k) keep the MFMA
// pipe busier than the hand-written tile kernel at the benchmark shapes:
// 92.9 % of the fp32 MFMA peak at n = 1e5, m = 1000, d = 4096 against
// 78-84 %, 80.7 % against 69 % at the C5 shape.  The algorithm is the
// library heuristic's first choice within the workspace the caller passes
// (its stream's own scratch, so concurrent streams never share it; the
// heuristic's pick for the C4 shape takes 8 MB); the library handle is one
// per device, created on first use and kept.  Any status other than
// success (no algorithm for the shape, a launch error) returns false and
// the caller runs its MFMA kernel instead; every element of S is written
// either way.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <mutex>
#include <stdint.h>

#include "eval_launch.hpp"

namespace sdca_gpu {

namespace {

constexpr int kMaxDevices = 64;
constexpr int kCacheSlots = 16;

struct AlgoSlot {
  int device = -1;
  int64_t n = 0, m = 0, d = 0;
  size_t ws_max = 0;  // the workspace the heuristic was allowed
  size_t ws = 0;      // the workspace the algorithm needs
  bool ok = false;  // an algorithm exists for the shape
  hipblasLtMatmulAlgo_t algo;
};

std::mutex g_mutex;
hipblasLtHandle_t g_handle[kMaxDevices] = {};
AlgoSlot g_cache[kCacheSlots];
int g_next = 0;

struct Descs {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  ~Descs() {
    if (lc) hipblasLtMatrixLayoutDestroy(lc);
    if (lb) hipblasLtMatrixLayoutDestroy(lb);
    if (la) hipblasLtMatrixLayoutDestroy(la);
    if (desc) hipblasLtMatmulDescDestroy(desc);
  }
  bool make(int64_t n, int64_t m, int64_t d) {
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    return hipblasLtMatmulDescCreate(&desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) ==
               HIPBLAS_STATUS_SUCCESS &&
           hipblasLtMatmulDescSetAttribute(desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) ==
               HIPBLAS_STATUS_SUCCESS &&
           hipblasLtMatmulDescSetAttribute(desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) ==
               HIPBLAS_STATUS_SUCCESS &&
           hipblasLtMatrixLayoutCreate(&la, HIP_R_32F, static_cast<uint64_t>(d),
                                       static_cast<uint64_t>(m), d) == HIPBLAS_STATUS_SUCCESS &&
           hipblasLtMatrixLayoutCreate(&lb, HIP_R_32F, static_cast<uint64_t>(d),
                                       static_cast<uint64_t>(n), d) == HIPBLAS_STATUS_SUCCESS &&
           hipblasLtMatrixLayoutCreate(&lc, HIP_R_32F, static_cast<uint64_t>(m),
                                       static_cast<uint64_t>(n), m) == HIPBLAS_STATUS_SUCCESS;
  }
};

// The device's handle and the algorithm for (n, m, d) within ws_max bytes
// of workspace, looked up or chosen by the library's heuristic under the
// lock.
bool lookup(int dev, int64_t n, int64_t m, int64_t d, size_t ws_max, const Descs& ds,
            hipblasLtHandle_t* h, hipblasLtMatmulAlgo_t* algo) {
  std::lock_guard<std::mutex> lock(g_mutex);
  if (dev < 0 || dev >= kMaxDevices) return false;
  if (!g_handle[dev]) {
    // A failed creation (e.g. under stream capture, where it cannot
    // allocate) is tried again on the next call.
    if (hipblasLtCreate(&g_handle[dev]) != HIPBLAS_STATUS_SUCCESS) {
      g_handle[dev] = nullptr;
      return false;
    }
  }
  *h = g_handle[dev];
  for (const AlgoSlot& s : g_cache) {
    if (s.device == dev && s.n == n && s.m == m && s.d == d && s.ws_max == ws_max) {
      if (s.ok) *algo = s.algo;
      return s.ok;
    }
  }
  AlgoSlot& s = g_cache[g_next];
  g_next = (g_next + 1) % kCacheSlots;
  s.device = dev;
  s.n = n;
  s.m = m;
  s.d = d;
  s.ws_max = ws_max;
  s.ok = false;
  hipblasLtMatmulPreference_t pref = nullptr;
  if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return false;
  const uint64_t max_bytes = ws_max;
  // The first of the heuristic's ranked list (asked for several: asked
  // for one, it ranked differently at the C5 shape).
  hipblasLtMatmulHeuristicResult_t res[8];
  int count = 0;
  if (hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                            &max_bytes, sizeof(max_bytes)) ==
          HIPBLAS_STATUS_SUCCESS &&
      hipblasLtMatmulAlgoGetHeuristic(*h, ds.desc, ds.la, ds.lb, ds.lc, ds.lc, pref, 8, res,
                                      &count) == HIPBLAS_STATUS_SUCCESS &&
      count > 0 && res[0].state == HIPBLAS_STATUS_SUCCESS && res[0].workspaceSize <= ws_max) {
    s.algo = res[0].algo;
    s.ws = res[0].workspaceSize;
    s.ok = true;
    *algo = s.algo;
  }
  hipblasLtMatmulPreferenceDestroy(pref);
  return s.ok;
}

}  // namespace

bool blas_scores_gemm(const float* X, const float* W, float* S, int64_t n, int64_t m, int64_t d,
                      hipStream_t stream, void* ws, size_t ws_bytes) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  if (!ws) ws_bytes = 0;
  Descs ds;
  if (!ds.make(n, m, d)) return false;
  hipblasLtHandle_t h = nullptr;
  hipblasLtMatmulAlgo_t algo;
  if (!lookup(dev, n, m, d, ws_bytes, ds, &h, &algo)) return false;
  const float alpha = 1.0f, beta = 0.0f;
  return hipblasLtMatmul(h, ds.desc, &alpha, W, ds.la, X, ds.lb, &beta, S, ds.lc, S, ds.lc, &algo,
                         ws, ws_bytes, stream) == HIPBLAS_STATUS_SUCCESS;
}

}  // namespace sdca_gpu
