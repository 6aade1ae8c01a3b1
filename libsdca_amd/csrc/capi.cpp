// C ABI of the MI355X batched prox + evaluation path (include/sdca_hip.h):
// argument validation with the Matlab front end's rules
// (src/matlab/mex_prox.cpp:132-136), host staging for SDCA_HOST_PTR, the
// per-(device, stream) workspace cache and the kernel dispatch.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "../../include/sdca_hip.h"
#include "prox_launch.hpp"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation)
    return fail(SDCA_ERR_OUT_OF_MEMORY, "%s: %s", what, hipGetErrorString(e));
  return fail(SDCA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define SDCA_HIP_TRY(expr, what)                \
  do {                                          \
    hipError_t e_ = (expr);                     \
    if (e_ != hipSuccess) return hip_fail(e_, what); \
  } while (0)

size_t dtype_size(int dt) { return dt == SDCA_F32 ? 4 : 8; }

// Device scratch, one set per (device, stream) so that concurrent streams
// never share it.  Buffers only grow; growth frees the old buffer after the
// device is idle (hipFree synchronises).
struct Workspace {
  void* ptr[4] = {nullptr, nullptr, nullptr, nullptr};
  size_t cap[4] = {0, 0, 0, 0};
};

std::mutex g_ws_mutex;
std::map<std::pair<int, hipStream_t>, Workspace> g_ws;

// Returns slot `slot` of the calling stream's workspace with at least `bytes`.
int workspace(hipStream_t stream, int slot, size_t bytes, void** out) {
  int dev = 0;
  SDCA_HIP_TRY(hipGetDevice(&dev), "hipGetDevice");
  std::lock_guard<std::mutex> lock(g_ws_mutex);
  Workspace& w = g_ws[std::make_pair(dev, stream)];
  if (w.cap[slot] < bytes) {
    if (w.ptr[slot]) {
      SDCA_HIP_TRY(hipStreamSynchronize(stream), "hipStreamSynchronize");
      SDCA_HIP_TRY(hipFree(w.ptr[slot]), "hipFree");
      w.ptr[slot] = nullptr;
      w.cap[slot] = 0;
    }
    size_t want = bytes + bytes / 4 + 256;
    SDCA_HIP_TRY(hipMalloc(&w.ptr[slot], want), "hipMalloc(workspace)");
    w.cap[slot] = want;
  }
  *out = w.ptr[slot];
  return SDCA_OK;
}

// Host staging: a device copy of a host array, freed with the guard.
struct DeviceBuffer {
  void* ptr = nullptr;
  ~DeviceBuffer() {
    if (ptr) (void)hipFree(ptr);
  }
};

int stage_in(const void* host, size_t bytes, DeviceBuffer& buf, hipStream_t stream) {
  if (!host || bytes == 0) return SDCA_OK;
  SDCA_HIP_TRY(hipMalloc(&buf.ptr, bytes), "hipMalloc(staging)");
  SDCA_HIP_TRY(hipMemcpyAsync(buf.ptr, host, bytes, hipMemcpyHostToDevice, stream),
               "hipMemcpyAsync(H2D)");
  return SDCA_OK;
}

int check_dtypes(int data, int result) {
  if (data == SDCA_LONG_DOUBLE || result == SDCA_LONG_DOUBLE)
    return fail(SDCA_ERR_NOT_IMPLEMENTED, "long double precision is not supported on the GPU");
  if ((data != SDCA_F32 && data != SDCA_F64) || (result != SDCA_F32 && result != SDCA_F64))
    return fail(SDCA_ERR_PRECISION, "unknown precision (data %d, result %d)", data, result);
  if (data == SDCA_F64 && result == SDCA_F32)
    return fail(SDCA_ERR_NOT_IMPLEMENTED, "double data with single precision result is not supported");
  return SDCA_OK;
}

}  // namespace

extern "C" {

int sdca_abi_version(void) { return SDCA_HIP_ABI_VERSION; }

const char* sdca_last_error(void) { return g_last_error.c_str(); }

void sdca_prox_params_default(sdca_prox_params* p) {
  if (!p) return;
  p->lo = 0;
  p->hi = 1;
  p->rhs = 1;
  p->rho = 1;
  p->alpha = 1;
  p->k = 1;
  p->p = 1;
}

int sdca_prox(sdca_prox_op op, sdca_dtype data, sdca_dtype result, int64_t m, int64_t n,
              const void* in, void* out, const sdca_prox_params* params, const int64_t* col_p,
              sdca_thresholds* thresholds, unsigned flags, void* stream_ptr) {
  using namespace sdca_gpu;
  g_last_error.clear();
  sdca_prox_params p;
  if (params) p = *params;
  else sdca_prox_params_default(&p);
  if (static_cast<int>(op) < 0 || op > SDCA_PROX_TWO_SIMPLEX_SORT)
    return fail(SDCA_ERR_PROX, "unknown prox operator %d", static_cast<int>(op));
  if (op > SDCA_PROX_LAMBERT_W_EXP)
    return fail(SDCA_ERR_NOT_IMPLEMENTED, "prox operator %d is not implemented on the GPU",
                static_cast<int>(op));
  int rc = check_dtypes(data, result);
  if (rc) return rc;
  if (m < 1) return fail(SDCA_ERR_ARG_RANGE, "m must be >= 1 (got %lld)", (long long)m);
  if (n < 0) return fail(SDCA_ERR_ARG_RANGE, "n must be >= 0 (got %lld)", (long long)n);
  if (m > INT32_MAX / 2 || n > INT32_MAX)
    return fail(SDCA_ERR_ARG_RANGE, "matrix too large (m %lld, n %lld)", (long long)m, (long long)n);
  // mex_prox.cpp:132-136
  if (!(p.rhs >= 0)) return fail(SDCA_ERR_ARG_RANGE, "rhs must be >= 0 (got %g)", p.rhs);
  if (!(p.rho >= 0)) return fail(SDCA_ERR_ARG_RANGE, "rho must be >= 0 (got %g)", p.rho);
  if (!(p.alpha > 0)) return fail(SDCA_ERR_ARG_RANGE, "alpha must be > 0 (got %g)", p.alpha);
  const bool uses_k = op == SDCA_PROX_TOPK_SIMPLEX || op == SDCA_PROX_TOPK_CONE ||
                      op == SDCA_PROX_TOPK_ENTROPY;
  if (uses_k && (p.k < 1 || p.k > m))
    return fail(SDCA_ERR_ARG_RANGE, "k must be in [1, %lld] (got %lld)", (long long)m, (long long)p.k);
  if (op == SDCA_PROX_TWO_SIMPLEX) {
    if (m < 2) return fail(SDCA_ERR_ARG_RANGE, "two_simplex needs m >= 2");
    if (!col_p && (p.p < 1 || p.p > m - 1))
      return fail(SDCA_ERR_ARG_RANGE, "p must be in [1, %lld] (got %lld)", (long long)(m - 1), (long long)p.p);
    if (!(p.rhs > 0)) return fail(SDCA_ERR_ARG_RANGE, "two_simplex needs rhs > 0 (got %g)", p.rhs);
    if (col_p && (flags & SDCA_HOST_PTR)) {
      for (int64_t j = 0; j < n; ++j)
        if (col_p[j] < 1 || col_p[j] > m - 1)
          return fail(SDCA_ERR_ARG_RANGE, "col_p[%lld] = %lld outside [1, %lld]", (long long)j,
                      (long long)col_p[j], (long long)(m - 1));
    }
  }
  if ((op == SDCA_PROX_ENTROPY || op == SDCA_PROX_ENTROPY_NORM) && (!(p.hi > 0) || !(p.rhs > 0)))
    return fail(SDCA_ERR_ARG_RANGE, "entropic projections need hi > 0 and rhs > 0");
  if (n == 0) return SDCA_OK;
  if (!in || !out) return fail(SDCA_ERR_ARG_NULL, "in and out must not be NULL");

  const bool reg_ok = m <= kRegMaxM;
  const bool topk = op == SDCA_PROX_TOPK_SIMPLEX || op == SDCA_PROX_TOPK_CONE;
  const bool knap = op == SDCA_PROX_KNAPSACK_EQ || op == SDCA_PROX_KNAPSACK_LE;
  if (!reg_ok && !(topk || knap) && op != SDCA_PROX_LAMBERT_W_EXP)
    return fail(SDCA_ERR_NOT_IMPLEMENTED, "operator %d supports m <= %lld on the GPU (got %lld)",
                static_cast<int>(op), (long long)kRegMaxM, (long long)m);
  if ((topk || knap) && m > slow_max_m(data) && (!reg_ok || (topk && p.k > kTopkMaxK)))
    return fail(SDCA_ERR_NOT_IMPLEMENTED, "m = %lld is above the supported %lld for this operator",
                (long long)m, (long long)slow_max_m(data));

  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  const size_t bytes = static_cast<size_t>(m) * static_cast<size_t>(n) * dtype_size(data);
  const bool host = (flags & SDCA_HOST_PTR) != 0;
  const int64_t nthr = (op == SDCA_PROX_TWO_SIMPLEX) ? 2 * n : n;
  DeviceBuffer din, dout, dcolp, dthr;
  const void* d_in = in;
  void* d_out = out;
  const int64_t* d_colp = col_p;
  sdca_thresholds* d_thr = thresholds;
  if (host) {
    rc = stage_in(in, bytes, din, stream);
    if (rc) return rc;
    d_in = din.ptr;
    if (out == in) {
      d_out = din.ptr;
    } else {
      SDCA_HIP_TRY(hipMalloc(&dout.ptr, bytes), "hipMalloc(staging)");
      d_out = dout.ptr;
    }
    if (col_p && op == SDCA_PROX_TWO_SIMPLEX) {
      rc = stage_in(col_p, static_cast<size_t>(n) * sizeof(int64_t), dcolp, stream);
      if (rc) return rc;
      d_colp = static_cast<const int64_t*>(dcolp.ptr);
    }
    if (thresholds) {
      SDCA_HIP_TRY(hipMalloc(&dthr.ptr, static_cast<size_t>(nthr) * sizeof(sdca_thresholds)),
                   "hipMalloc(staging)");
      d_thr = static_cast<sdca_thresholds*>(dthr.ptr);
    }
  }
  if (op != SDCA_PROX_TWO_SIMPLEX) d_colp = nullptr;

  ProxLaunch a;
  a.op = op;
  a.data = data;
  a.result = result;
  a.m = m;
  a.n = n;
  a.in = d_in;
  a.out = d_out;
  a.lo = p.lo;
  a.hi = p.hi;
  a.rhs = p.rhs;
  a.k = p.k;
  a.p = p.p;
  a.col_p = d_colp;
  a.thr = d_thr;
  a.slow = nullptr;
  a.stream = stream;

  if (op == SDCA_PROX_LAMBERT_W_EXP) {
    SDCA_HIP_TRY(launch_lambert(a), "lambert_w_exp kernel");
  } else if ((topk || knap) && (!reg_ok || (topk && p.k > kTopkMaxK))) {
    SDCA_HIP_TRY(launch_slow(a, true), "prox kernel (workgroup per column)");
  } else {
    if (topk) {
      void* ws = nullptr;
      rc = workspace(stream, 0, static_cast<size_t>(n + 1) * sizeof(int), &ws);
      if (rc) return rc;
      a.slow = static_cast<int*>(ws);
      SDCA_HIP_TRY(launch_clear(a.slow, 1, stream), "clear kernel");
    }
    hipError_t e = hipSuccess;
    switch (op) {
      case SDCA_PROX_KNAPSACK_EQ:
      case SDCA_PROX_KNAPSACK_LE: e = launch_knap(a); break;
      case SDCA_PROX_TOPK_SIMPLEX:
      case SDCA_PROX_TOPK_CONE: e = launch_topk(a); break;
      case SDCA_PROX_ENTROPY:
      case SDCA_PROX_ENTROPY_NORM: e = launch_ent(a); break;
      case SDCA_PROX_TOPK_ENTROPY: e = launch_topkent(a); break;
      case SDCA_PROX_TWO_SIMPLEX: e = launch_two(a); break;
      default: break;
    }
    SDCA_HIP_TRY(e, "prox kernel");
    if (topk) SDCA_HIP_TRY(launch_slow(a, false), "prox kernel (deferred columns)");
  }

  if (host) {
    SDCA_HIP_TRY(hipMemcpyAsync(out, d_out, bytes, hipMemcpyDeviceToHost, stream), "hipMemcpyAsync(D2H)");
    if (thresholds)
      SDCA_HIP_TRY(hipMemcpyAsync(thresholds, d_thr, static_cast<size_t>(nthr) * sizeof(sdca_thresholds),
                                  hipMemcpyDeviceToHost, stream), "hipMemcpyAsync(D2H)");
    SDCA_HIP_TRY(hipStreamSynchronize(stream), "hipStreamSynchronize");
  }
  return SDCA_OK;
}

}  // extern "C"
