// C ABI of the MI355X batched prox + evaluation path (include/sdca_hip.h):
// argument validation with the Matlab front end's rules
// (src/matlab/mex_prox.cpp:132-136), host staging for SDCA_HOST_PTR, the
// per-(device, stream, host thread) workspace cache and the kernel dispatch.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <numeric>
#include <random>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <tuple>
#include <utility>
#include <vector>

#include "../../include/sdca_hip.h"
#include "epoch_launch.hpp"
#include "eval_launch.hpp"
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

// Device scratch, one set per (device, stream, host thread): concurrent
// streams never share it, and neither do host threads that enqueue on the
// same stream (growing a shared set could free a buffer that another
// thread's call has taken but not yet launched on).  Buffers only grow;
// growth frees the old buffer after the stream is idle.  A stream under
// graph capture cannot grow it (the wait and the allocation are not
// capturable): warm the stream up with one call of the same size first.
struct Workspace {
  // Slots: 0 deferred-column list, 1 scores, 2 evaluation scratch,
  // 3 transposes, 4 epoch, 5 the library GEMM's workspace, 6 the column
  // slices of the prox beyond the LDS copy.
  void* ptr[7] = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
  size_t cap[7] = {0, 0, 0, 0, 0, 0, 0};
  // Pinned host block for the evaluation's results: copies into it are
  // asynchronous, so the call waits once for all of them.
  void* host = nullptr;
  size_t host_cap = 0;
  // The deferred-column list's two counters are zero (the deferred-column
  // kernel of the last call on this stream was launched and resets them).
  bool list_zeroed = false;
};

std::mutex g_ws_mutex;
std::map<std::tuple<int, hipStream_t, std::thread::id>, Workspace> g_ws;

// Returns slot `slot` of the calling stream's workspace with at least `bytes`
// (and, with `ws`, the stream's workspace record).
int workspace(hipStream_t stream, int slot, size_t bytes, void** out, Workspace** ws = nullptr) {
  int dev = 0;
  SDCA_HIP_TRY(hipGetDevice(&dev), "hipGetDevice");
  std::lock_guard<std::mutex> lock(g_ws_mutex);
  Workspace& w = g_ws[std::make_tuple(dev, stream, std::this_thread::get_id())];
  if (ws) *ws = &w;
  if (w.cap[slot] < bytes) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    SDCA_HIP_TRY(hipStreamIsCapturing(stream, &cs), "hipStreamIsCapturing");
    if (cs != hipStreamCaptureStatusNone)
      return fail(SDCA_ERR_HIP,
                  "the stream is being captured and its scratch must grow to %zu bytes: run the "
                  "call once on this stream before the capture", bytes);
    if (slot == 0) w.list_zeroed = false;
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

// The library GEMM's workspace (slot 5) for an fp32 score GEMM of n m d:
// none below the library's threshold, and under graph capture only one the
// stream already has (the GEMM then takes an algorithm within it, or the
// MFMA kernel).
int gemm_workspace(hipStream_t stream, int64_t n, int64_t m, int64_t d, void** ws,
                   size_t* bytes) {
  using sdca_gpu::blas_shape;
  using sdca_gpu::kBlasWorkspaceBytes;
  *ws = nullptr;
  *bytes = 0;
  if (!blas_shape(n, m, d)) return SDCA_OK;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  SDCA_HIP_TRY(hipStreamIsCapturing(stream, &cs), "hipStreamIsCapturing");
  if (cs != hipStreamCaptureStatusNone) {
    int dev = 0;
    SDCA_HIP_TRY(hipGetDevice(&dev), "hipGetDevice");
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    Workspace& w = g_ws[std::make_tuple(dev, stream, std::this_thread::get_id())];
    if (w.cap[5] >= kBlasWorkspaceBytes) {
      *ws = w.ptr[5];
      *bytes = kBlasWorkspaceBytes;
    }
    return SDCA_OK;
  }
  const int rc = workspace(stream, 5, kBlasWorkspaceBytes, ws);
  if (rc) return rc;
  *bytes = kBlasWorkspaceBytes;
  return SDCA_OK;
}

// The calling stream's pinned host block of at least `bytes` (grown like
// the device slots).
int host_block(hipStream_t stream, size_t bytes, void** out) {
  int dev = 0;
  SDCA_HIP_TRY(hipGetDevice(&dev), "hipGetDevice");
  std::lock_guard<std::mutex> lock(g_ws_mutex);
  Workspace& w = g_ws[std::make_tuple(dev, stream, std::this_thread::get_id())];
  if (w.host_cap < bytes) {
    if (w.host) {
      SDCA_HIP_TRY(hipStreamSynchronize(stream), "hipStreamSynchronize");
      SDCA_HIP_TRY(hipHostFree(w.host), "hipHostFree");
      w.host = nullptr;
      w.host_cap = 0;
    }
    const size_t want = bytes + bytes / 4 + 256;
    SDCA_HIP_TRY(hipHostMalloc(&w.host, want, hipHostMallocDefault), "hipHostMalloc");
    w.host_cap = want;
  }
  *out = w.host;
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

// The prox operators take every (data, result) pair of the Matlab front
// end's precision dispatch (mex_prox.cpp:179-201) except long double; the
// evaluation pass takes (f32, f32), (f32, f64) and (f64, f64).
int check_dtypes(int data, int result, bool prox = false) {
  if (data == SDCA_LONG_DOUBLE || result == SDCA_LONG_DOUBLE)
    return fail(SDCA_ERR_NOT_IMPLEMENTED, "long double precision is not supported on the GPU");
  if ((data != SDCA_F32 && data != SDCA_F64) || (result != SDCA_F32 && result != SDCA_F64))
    return fail(SDCA_ERR_PRECISION, "unknown precision (data %d, result %d)", data, result);
  if (!prox && data == SDCA_F64 && result == SDCA_F32)
    return fail(SDCA_ERR_NOT_IMPLEMENTED,
                "the evaluation pass takes no double data with a single precision result");
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
  return sdca_gpu::prox_entry(op, data, result, m, n, in, out, params, col_p, thresholds, flags,
                              stream_ptr, nullptr, 0);
}

int sdca_prox_with_sets(sdca_prox_op op, sdca_dtype data, sdca_dtype result, int64_t m,
                        int64_t n, const void* in, void* out, const sdca_prox_params* params,
                        const int64_t* col_p, sdca_thresholds* thresholds, sdca_prox_sets* sets,
                        unsigned flags, void* stream_ptr) {
  return sdca_gpu::prox_entry(op, data, result, m, n, in, out, params, col_p, thresholds, flags,
                              stream_ptr, nullptr, 0, sets);
}

}  // extern "C"

namespace sdca_gpu {

int set_error(int code, const char* message) { return fail(code, "%s", message); }

int prox_entry(int op_in, int data_in, int result_in, int64_t m, int64_t n, const void* in,
               void* out, const sdca_prox_params* params, const int64_t* col_p,
               sdca_thresholds* thresholds, unsigned flags, void* stream_ptr, int* fixed_list,
               int64_t fixed_list_ints, sdca_prox_sets* sets) {
  const sdca_prox_op op = static_cast<sdca_prox_op>(op_in);
  const sdca_dtype data = static_cast<sdca_dtype>(data_in);
  const sdca_dtype result = static_cast<sdca_dtype>(result_in);
  g_last_error.clear();
  sdca_prox_params p;
  if (params) p = *params;
  else sdca_prox_params_default(&p);
  if (static_cast<int>(op) < 0 || op > SDCA_PROX_TWO_ENTROPY)
    return fail(SDCA_ERR_PROX, "unknown prox operator %d", static_cast<int>(op));
  int rc = check_dtypes(data, result, true);
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
                      op == SDCA_PROX_TOPK_ENTROPY || op == SDCA_PROX_TOPK_SIMPLEX_BIASED ||
                      op == SDCA_PROX_TOPK_CONE_BIASED || op == SDCA_PROX_TOPK_ENTROPY_BIASED;
  if (uses_k && (p.k < 1 || p.k > m))
    return fail(SDCA_ERR_ARG_RANGE, "k must be in [1, %lld] (got %lld)", (long long)m, (long long)p.k);
  const bool two = op == SDCA_PROX_TWO_SIMPLEX || op == SDCA_PROX_TWO_SIMPLEX_SORT ||
                   op == SDCA_PROX_TWO_ENTROPY;
  if (two) {
    if (m < 2) return fail(SDCA_ERR_ARG_RANGE, "two_simplex needs m >= 2");
    if (!col_p && (p.p < 1 || p.p > m - 1))
      return fail(SDCA_ERR_ARG_RANGE, "p must be in [1, %lld] (got %lld)", (long long)(m - 1), (long long)p.p);
    if (op != SDCA_PROX_TWO_ENTROPY && !(p.rhs > 0))
      return fail(SDCA_ERR_ARG_RANGE, "two_simplex needs rhs > 0 (got %g)", p.rhs);
    if (col_p && (flags & SDCA_HOST_PTR)) {
      for (int64_t j = 0; j < n; ++j)
        if (col_p[j] < 1 || col_p[j] > m - 1)
          return fail(SDCA_ERR_ARG_RANGE, "col_p[%lld] = %lld outside [1, %lld]", (long long)j,
                      (long long)col_p[j], (long long)(m - 1));
    }
  }
  if ((op == SDCA_PROX_ENTROPY || op == SDCA_PROX_ENTROPY_NORM) && (!(p.hi > 0) || !(p.rhs > 0)))
    return fail(SDCA_ERR_ARG_RANGE, "entropic projections need hi > 0 and rhs > 0");
  if (sets && op == SDCA_PROX_LAMBERT_W_EXP)
    return fail(SDCA_ERR_ARG_RANGE, "lambert_w_exp has no threshold records (sets must be NULL)");
  if (n == 0) return SDCA_OK;
  if (!in || !out) return fail(SDCA_ERR_ARG_NULL, "in and out must not be NULL");

  const bool reg_ok = m <= kRegMaxM;
  const bool topk = op == SDCA_PROX_TOPK_SIMPLEX || op == SDCA_PROX_TOPK_CONE;
  const bool knap = op == SDCA_PROX_KNAPSACK_EQ || op == SDCA_PROX_KNAPSACK_LE;
  // The biased simplex, cone and knapsack run in the register kernel;
  // columns whose search needs more of the sorted column are deferred to the
  // workgroup-per-column kernel through the column list.
  const bool reg_biased = op == SDCA_PROX_TOPK_SIMPLEX_BIASED ||
                          op == SDCA_PROX_TOPK_CONE_BIASED || op == SDCA_PROX_KNAPSACK_LE_BIASED;
  const bool topk_like =
      topk || op == SDCA_PROX_TOPK_SIMPLEX_BIASED || op == SDCA_PROX_TOPK_CONE_BIASED;
  const bool listed = topk || reg_biased || op == SDCA_PROX_TWO_SIMPLEX_SORT;
  // The Lambert-map operators solved one wave per column (prox_entbias.hip).
  const bool ent_biased = op == SDCA_PROX_TOPK_ENTROPY_BIASED || op == SDCA_PROX_TWO_ENTROPY;
  // Above kRegMaxM rows a column is held by one workgroup, in LDS (the
  // sorted-column, wave-per-column and workgroup-per-column kernels).
  // Above that, the knapsack and entropic operators stream the column from
  // global memory, the top-k, biased-knapsack and two-block simplex
  // operators work on the column in device memory (sorted in a scratch
  // slice, or read in place); the Lambert-map entropic ones refuse.
  const bool wide = m > max_rows(data);
  const bool streamed = wide && stream_supported(op);
  const bool global_sorted = wide && (topk || reg_biased);
  const bool global_two = wide && (op == SDCA_PROX_TWO_SIMPLEX || op == SDCA_PROX_TWO_SIMPLEX_SORT);
  const bool global_wave = wide && ent_biased;
  const bool global_topkent = wide && op == SDCA_PROX_TOPK_ENTROPY;
  if (fixed_list && (global_sorted || global_wave || global_topkent ||
                     op == SDCA_PROX_TWO_SIMPLEX_SORT) && wide)
    return fail(SDCA_ERR_ARG_RANGE,
                "sdca_prox_noalloc: m = %lld is above %lld rows, where this operator needs "
                "allocated scratch", (long long)m, (long long)max_rows(data));

  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  const size_t bytes = static_cast<size_t>(m) * static_cast<size_t>(n) * dtype_size(data);
  const bool host = (flags & SDCA_HOST_PTR) != 0;
  const int64_t nthr = two ? 2 * n : n;
  if (fixed_list) {
    // The entry point without allocation: device pointers only (host
    // staging allocates), and the deferred-column list [count, done,
    // column ids] must fit the caller-provided scratch.
    if (host)
      return fail(SDCA_ERR_ARG_RANGE,
                  "sdca_prox_noalloc takes device pointers only (SDCA_HOST_PTR stages through "
                  "allocated device buffers)");
    if (listed && n + 2 > fixed_list_ints)
      return fail(SDCA_ERR_ARG_RANGE,
                  "sdca_prox_noalloc: n = %lld columns exceed its fixed scratch of %lld columns "
                  "for this operator", (long long)n, (long long)(fixed_list_ints - 2));
  }
  DeviceBuffer din, dout, dcolp, dthr, dsets;
  const void* d_in = in;
  void* d_out = out;
  const int64_t* d_colp = col_p;
  sdca_thresholds* d_thr = thresholds;
  sdca_prox_sets* d_sets = sets;
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
    if (col_p && two) {
      rc = stage_in(col_p, static_cast<size_t>(n) * sizeof(int64_t), dcolp, stream);
      if (rc) return rc;
      d_colp = static_cast<const int64_t*>(dcolp.ptr);
    }
    if (thresholds) {
      SDCA_HIP_TRY(hipMalloc(&dthr.ptr, static_cast<size_t>(nthr) * sizeof(sdca_thresholds)),
                   "hipMalloc(staging)");
      d_thr = static_cast<sdca_thresholds*>(dthr.ptr);
    }
    if (sets) {
      SDCA_HIP_TRY(hipMalloc(&dsets.ptr, static_cast<size_t>(nthr) * sizeof(sdca_prox_sets)),
                   "hipMalloc(staging)");
      d_sets = static_cast<sdca_prox_sets*>(dsets.ptr);
    }
  }
  if (!two) d_colp = nullptr;

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
  a.rho = p.rho;
  a.alpha = p.alpha;
  a.k = p.k;
  a.p = p.p;
  a.col_p = d_colp;
  a.thr = d_thr;
  a.sets = d_sets;
  a.slow = nullptr;
  a.stream = stream;

  if (op == SDCA_PROX_LAMBERT_W_EXP) {
    SDCA_HIP_TRY(launch_lambert(a), "lambert_w_exp kernel");
  } else if (global_sorted || global_wave || global_topkent ||
             (global_two && op == SDCA_PROX_TWO_SIMPLEX_SORT)) {
    // One column slice per workgroup (per wave for the wave kernels, in
    // whole workgroups of four), as many slices as fit 512 MiB (at least
    // one workgroup's), at most one per column and 4096.
    size_t slice = static_cast<size_t>(m) * dtype_size(data);
    if (global_wave) slice = static_cast<size_t>((m + 3) & ~int64_t(3)) * dtype_size(data);
    if (global_sorted) {
      size_t pow2 = 1;
      while (pow2 < static_cast<size_t>(m)) pow2 <<= 1;
      slice = pow2 * dtype_size(data);
    }
    int64_t slices = static_cast<int64_t>((size_t(512) << 20) / slice);
    if (slices > n) slices = n;
    if (slices > 4096) slices = 4096;
    if (global_wave) slices = (slices + 3) & ~int64_t(3);  // whole workgroups of four waves
    if (slices < (global_wave ? 4 : 1)) slices = global_wave ? 4 : 1;
    void* scratch = nullptr;
    rc = workspace(stream, 6, static_cast<size_t>(slices) * slice, &scratch);
    if (rc) return rc;
    const size_t bytes_s = static_cast<size_t>(slices) * slice;
    if (global_sorted)
      SDCA_HIP_TRY(launch_slow_global(a, scratch, bytes_s),
                   "prox kernel (workgroup per column, column in device memory)");
    else if (op == SDCA_PROX_TWO_ENTROPY)
      SDCA_HIP_TRY(launch_two_ent_global(a, scratch, bytes_s),
                   "two_entropy kernel (column in device memory)");
    else if (op == SDCA_PROX_TOPK_ENTROPY_BIASED)
      SDCA_HIP_TRY(launch_ent_biased_global(a, scratch, bytes_s),
                   "topk_entropy_biased kernel (column in device memory)");
    else if (global_topkent)
      SDCA_HIP_TRY(launch_topkent_global(a, scratch, bytes_s),
                   "topk_entropy kernel (column in device memory)");
    else
      SDCA_HIP_TRY(launch_two_sort_global(a, scratch, bytes_s),
                   "two_simplex_sort kernel (column in device memory)");
  } else if (global_two) {
    SDCA_HIP_TRY(launch_two_global(a), "two_simplex kernel (column in device memory)");
  } else if (streamed) {
    SDCA_HIP_TRY(launch_stream(a), "prox kernel (column streamed from global memory)");
  } else if (op == SDCA_PROX_TWO_SIMPLEX_SORT && !reg_ok) {
    SDCA_HIP_TRY(launch_two_sort(a, true), "two_simplex_sort kernel (workgroup per column)");
  } else if (op == SDCA_PROX_TWO_ENTROPY) {
    SDCA_HIP_TRY(launch_two_ent(a), "two_entropy kernel (wave per column)");
  } else if (ent_biased) {
    SDCA_HIP_TRY(launch_ent_biased(a), "topk_entropy_biased kernel (wave per column)");
  } else if ((topk || knap || reg_biased) && (!reg_ok || (topk_like && p.k > kTopkMaxK))) {
    // Columns beyond the register kernel: one workgroup per sorted column.
    SDCA_HIP_TRY(launch_slow(a, true), "prox kernel (workgroup per column)");
  } else {
    // Deferred-column list: [count, done, column ids...].  The deferred-column
    // kernel zeroes both counters when its last workgroup finishes, so a
    // clear is launched only for a new list or after a call that did not
    // reach that kernel.
    Workspace* wsr = nullptr;
    Workspace fixed_ws;  // the fixed scratch's stand-in record (its state is not kept)
    if (listed && fixed_list) {
      // The fixed scratch is shared by every call on the device: its two
      // counters are cleared by a kernel on this stream before each use.
      a.slow = fixed_list;
      wsr = &fixed_ws;
      SDCA_HIP_TRY(launch_clear(a.slow, 2, stream), "clear kernel");
    } else if (listed) {
      void* ws = nullptr;
      rc = workspace(stream, 0, static_cast<size_t>(n + 2) * sizeof(int), &ws, &wsr);
      if (rc) return rc;
      a.slow = static_cast<int*>(ws);
      if (!wsr->list_zeroed) SDCA_HIP_TRY(launch_clear(a.slow, 2, stream), "clear kernel");
      wsr->list_zeroed = false;
    }
    hipError_t e = hipSuccess;
    switch (op) {
      case SDCA_PROX_KNAPSACK_EQ:
      case SDCA_PROX_KNAPSACK_LE:
      case SDCA_PROX_KNAPSACK_LE_BIASED: e = launch_knap(a); break;
      case SDCA_PROX_TOPK_SIMPLEX:
      case SDCA_PROX_TOPK_CONE:
      case SDCA_PROX_TOPK_SIMPLEX_BIASED:
      case SDCA_PROX_TOPK_CONE_BIASED: e = launch_topk(a); break;
      case SDCA_PROX_ENTROPY:
      case SDCA_PROX_ENTROPY_NORM: e = launch_ent(a); break;
      case SDCA_PROX_TOPK_ENTROPY: e = launch_topkent(a); break;
      case SDCA_PROX_TWO_SIMPLEX:
      case SDCA_PROX_TWO_SIMPLEX_SORT: e = launch_two(a); break;
      default: break;
    }
    SDCA_HIP_TRY(e, "prox kernel");
    if (op == SDCA_PROX_TWO_SIMPLEX_SORT) {
      SDCA_HIP_TRY(launch_two_sort(a, false), "two_simplex_sort kernel (deferred columns)");
      wsr->list_zeroed = true;
    } else if (listed) {
      SDCA_HIP_TRY(launch_slow(a, false), "prox kernel (deferred columns)");
      wsr->list_zeroed = true;
    }
  }

  if (host) {
    SDCA_HIP_TRY(hipMemcpyAsync(out, d_out, bytes, hipMemcpyDeviceToHost, stream), "hipMemcpyAsync(D2H)");
    if (thresholds)
      SDCA_HIP_TRY(hipMemcpyAsync(thresholds, d_thr, static_cast<size_t>(nthr) * sizeof(sdca_thresholds),
                                  hipMemcpyDeviceToHost, stream), "hipMemcpyAsync(D2H)");
    if (sets)
      SDCA_HIP_TRY(hipMemcpyAsync(sets, d_sets, static_cast<size_t>(nthr) * sizeof(sdca_prox_sets),
                                  hipMemcpyDeviceToHost, stream), "hipMemcpyAsync(D2H)");
    SDCA_HIP_TRY(hipStreamSynchronize(stream), "hipStreamSynchronize");
  }
  return SDCA_OK;
}

}  // namespace sdca_gpu

namespace {

bool is_multilabel(int kind) { return kind >= SDCA_OBJ_MULTILABEL_HINGE; }
bool uses_k(int kind) {
  return kind == SDCA_OBJ_HINGE_TOPK || kind == SDCA_OBJ_HINGE_TOPK_SMOOTH ||
         kind == SDCA_OBJ_TOPK_HINGE || kind == SDCA_OBJ_TOPK_HINGE_SMOOTH ||
         kind == SDCA_OBJ_ENTROPY_TOPK;
}
bool uses_gamma(int kind) {
  return kind == SDCA_OBJ_HINGE_TOPK_SMOOTH || kind == SDCA_OBJ_TOPK_HINGE_SMOOTH ||
         kind == SDCA_OBJ_MULTILABEL_HINGE_SMOOTH;
}
// objective_base::coeff_primal_loss of each objective (objective/*.h).
double loss_coeff(const sdca_objective& o) {
  switch (o.kind) {
    case SDCA_OBJ_HINGE_TOPK:
    case SDCA_OBJ_TOPK_HINGE: return o.c / static_cast<double>(o.k);
    case SDCA_OBJ_HINGE_TOPK_SMOOTH:
    case SDCA_OBJ_TOPK_HINGE_SMOOTH:
    case SDCA_OBJ_MULTILABEL_HINGE_SMOOTH: return o.c / o.gamma;
    default: return o.c;
  }
}

int check_objectives(const sdca_objective* objs, int n_obj, int64_t m, bool multilabel) {
  if (!objs) return fail(SDCA_ERR_ARG_NULL, "objectives must not be NULL");
  if (n_obj < 1 || n_obj > sdca_gpu::kMaxObjectives)
    return fail(SDCA_ERR_ARG_RANGE, "n_obj must be in [1, %d] (got %d)", sdca_gpu::kMaxObjectives, n_obj);
  for (int o = 0; o < n_obj; ++o) {
    const sdca_objective& ob = objs[o];
    if (ob.kind < SDCA_OBJ_HINGE_TOPK || ob.kind > SDCA_OBJ_MULTILABEL_ENTROPY)
      return fail(SDCA_ERR_ARG_RANGE, "unknown objective kind %d", ob.kind);
    if (is_multilabel(ob.kind) != multilabel)
      return fail(SDCA_ERR_ARG_RANGE, "objective %d does not match the %s labels", o,
                  multilabel ? "multilabel" : "multiclass");
    if (!(ob.c > 0)) return fail(SDCA_ERR_ARG_RANGE, "c must be > 0 (got %g)", ob.c);
    if (uses_gamma(ob.kind) && !(ob.gamma > 0))
      return fail(SDCA_ERR_ARG_RANGE, "gamma must be > 0 (got %g)", ob.gamma);
    if (uses_k(ob.kind)) {
      if (ob.k < 1 || ob.k > m - 1)
        return fail(SDCA_ERR_ARG_RANGE, "k must be in [1, %lld] (got %lld)", (long long)(m - 1),
                    (long long)ob.k);
    }
  }
  return SDCA_OK;
}

// Host-side label checks (data/output.h:169-208), when labels are host memory.
int check_labels(const int64_t* labels, const int64_t* offsets, int64_t m, int64_t n) {
  if (!offsets) {
    for (int64_t i = 0; i < n; ++i)
      if (labels[i] < 0 || labels[i] >= m)
        return fail(SDCA_ERR_LABELS, "label %lld of example %lld is outside [0, %lld)",
                    (long long)labels[i], (long long)i, (long long)m);
    return SDCA_OK;
  }
  if (offsets[0] != 0) return fail(SDCA_ERR_LABELS, "The first offset must be 0.");
  for (int64_t i = 0; i < n; ++i) {
    const int64_t p = offsets[i + 1] - offsets[i];
    if (p < 1 || p >= m)
      return fail(SDCA_ERR_LABELS, "Each example must have between 1 and num_classes - 1 labels.");
    for (int64_t q = offsets[i]; q < offsets[i + 1]; ++q) {
      if (labels[q] < 0 || labels[q] >= m)
        return fail(SDCA_ERR_LABELS, "label %lld is outside [0, %lld)", (long long)labels[q], (long long)m);
      if (q > offsets[i] && !(labels[q - 1] < labels[q]))
        return fail(SDCA_ERR_LABELS, "All labels for every example must be distinct and sorted.");
    }
  }
  return SDCA_OK;
}

// The shared part of sdca_eval_scores / sdca_eval_features: epilogue,
// reductions and eval_end (eval/core.h:43-95) on device pointers.
//   dA_reg: non-NULL for the kernel-input training evaluation: the dual
//           regularizer sum_i 0.5 <a_i, s_i> of A (m x n) and the scores;
//   test:   eval_test records (primal loss, accuracy / rank loss only).
int eval_on_device(const sdca_objective* objs, int n_obj, int data, int result, int64_t m,
                   int64_t n, const void* dS, const void* dA, const int64_t* dlabels,
                   const int64_t* doffsets, const void* dW, const void* dW0, int64_t dm,
                   const void* dA_reg, bool test, double preg_in, double dreg_in,
                   sdca_eval_record* records, double* accuracy, double* per_example,
                   bool per_example_host, hipStream_t stream, const float* fused_X = nullptr,
                   const float* fused_W = nullptr, int64_t fused_d = 0) {
  using namespace sdca_gpu;
  const bool multilabel = doffsets != nullptr;
  if (test) {
    dA = nullptr;
    dW = nullptr;
    dA_reg = nullptr;
  }
  // Scratch layout: per-example losses, counts, rank, slow list, sums, hist, reg.
  const size_t pe_bytes = static_cast<size_t>(n) * n_obj * 2 * sizeof(double);
  const size_t cnt_bytes = static_cast<size_t>(n) * sizeof(int);
  const size_t rank_bytes = static_cast<size_t>(n) * sizeof(double);
  // [label-check flag, deferred count, (example, objective) pairs]
  const size_t slow_bytes = (2 + 2 * static_cast<size_t>(n) * n_obj) * sizeof(int);
  const size_t sums_bytes = (2 * kMaxObjectives + 2) * sizeof(double);
  const size_t hist_bytes = static_cast<size_t>(m) * sizeof(unsigned long long);
  const size_t reg_bytes = (2 * 512 + 2) * sizeof(double);
  const size_t dreg_bytes = dA_reg ? (static_cast<size_t>(n) + 1) * sizeof(double) : 0;
  const size_t red_bytes = static_cast<size_t>(eval_reduce_scratch(n_obj)) * sizeof(double);
  auto align = [](size_t b) { return (b + 255) / 256 * 256; };
  const size_t total = align(pe_bytes) + align(cnt_bytes) + align(rank_bytes) + align(slow_bytes) +
                       align(sums_bytes) + align(hist_bytes) + align(reg_bytes) + align(dreg_bytes) +
                       align(red_bytes);
  void* ws = nullptr;
  int rc = workspace(stream, 2, total, &ws);
  if (rc) return rc;
  char* p = static_cast<char*>(ws);
  double* d_pe = reinterpret_cast<double*>(p); p += align(pe_bytes);
  int* d_cnt = reinterpret_cast<int*>(p); p += align(cnt_bytes);
  double* d_rank = reinterpret_cast<double*>(p); p += align(rank_bytes);
  int* d_bad = reinterpret_cast<int*>(p);  // label check of the epilogue kernels
  int* d_slow = d_bad + 1;
  p += align(slow_bytes);
  double* d_sums = reinterpret_cast<double*>(p); p += align(sums_bytes);
  unsigned long long* d_hist = reinterpret_cast<unsigned long long*>(p); p += align(hist_bytes);
  double* d_reg = reinterpret_cast<double*>(p); p += align(reg_bytes);
  double* d_dreg = reinterpret_cast<double*>(p);  // n per-example terms, then the sum
  p += align(dreg_bytes);
  double* d_red = reinterpret_cast<double*>(p);

  EvalLaunch a;
  a.data = data;
  a.result = result;
  a.m = m;
  a.n = n;
  a.S = dS;
  a.A = dA;
  a.labels = dlabels;
  a.offsets = doffsets;
  a.objs.n = n_obj;
  for (int o = 0; o < n_obj; ++o) {
    a.objs.o[o].kind = objs[o].kind;
    a.objs.o[o].k = static_cast<int>(objs[o].k);
    a.objs.o[o].c = objs[o].c;
    a.objs.o[o].gamma = objs[o].gamma;
  }
  a.per_example = d_pe;
  a.counts = multilabel ? nullptr : d_cnt;
  a.rank = multilabel ? d_rank : nullptr;
  a.slow = d_slow;
  a.bad = d_bad;
  a.stream = stream;
  SDCA_HIP_TRY(launch_clear(d_bad, 2, stream), "clear kernel");  // flag and deferred count
  if (fused_X) {
    // Scores and epilogue in one kernel; dS receives only the rows of
    // deferred examples, which the deferred-example kernel reads.
    SDCA_HIP_TRY(launch_eval_fused(fused_X, fused_W, a, fused_d,
                                   static_cast<float*>(const_cast<void*>(dS))),
                 "fused evaluation kernel");
  } else {
    SDCA_HIP_TRY(launch_eval_epilogue(a), "evaluation epilogue kernel");
  }
  if (!multilabel) SDCA_HIP_TRY(launch_eval_slow(a), "evaluation epilogue (deferred examples)");
  SDCA_HIP_TRY(launch_eval_reduce(a, d_sums, multilabel ? d_sums + 2 * kMaxObjectives : nullptr,
                                  multilabel ? nullptr : d_hist, d_red),
               "evaluation reduction kernels");
  if (dW) SDCA_HIP_TRY(launch_regularizer(data, dW, dW0, dm, d_reg + 2, d_reg, stream),
                       "regularizer kernel");
  if (dA_reg)
    SDCA_HIP_TRY(launch_dual_regularizer(data, result, dA_reg, dS, m, n, d_dreg, d_dreg + n, stream),
                 "dual regularizer kernel");

  // The small results go to the stream's pinned block (asynchronous
  // copies, one wait): [sums | reg (2) | dual_reg | bad label flag | hist].
  void* hb = nullptr;
  if ((rc = host_block(stream, sums_bytes + 4 * sizeof(double) + hist_bytes, &hb))) return rc;
  double* h_sums = static_cast<double*>(hb);
  double* h_reg = h_sums + (2 * kMaxObjectives + 2);
  double* h_dual_reg = h_reg + 2;
  int* h_bad = reinterpret_cast<int*>(h_dual_reg + 1);
  unsigned long long* h_hist = reinterpret_cast<unsigned long long*>(h_dual_reg + 2);
  h_reg[0] = h_reg[1] = 0;
  *h_dual_reg = 0;
  SDCA_HIP_TRY(hipMemcpyAsync(h_sums, d_sums, sums_bytes, hipMemcpyDeviceToHost, stream),
               "hipMemcpyAsync(D2H)");
  if (!multilabel && accuracy)
    SDCA_HIP_TRY(hipMemcpyAsync(h_hist, d_hist, hist_bytes, hipMemcpyDeviceToHost, stream),
                 "hipMemcpyAsync(D2H)");
  if (dW) SDCA_HIP_TRY(hipMemcpyAsync(h_reg, d_reg, 2 * sizeof(double), hipMemcpyDeviceToHost,
                                      stream), "hipMemcpyAsync(D2H)");
  SDCA_HIP_TRY(hipMemcpyAsync(h_bad, d_bad, sizeof(int), hipMemcpyDeviceToHost, stream),
               "hipMemcpyAsync(D2H)");
  if (dA_reg) SDCA_HIP_TRY(hipMemcpyAsync(h_dual_reg, d_dreg + n, sizeof(double),
                                          hipMemcpyDeviceToHost, stream), "hipMemcpyAsync(D2H)");
  if (per_example) {
    SDCA_HIP_TRY(hipMemcpyAsync(per_example, d_pe, pe_bytes,
                                per_example_host ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice,
                                stream), "hipMemcpyAsync(per_example)");
  }
  SDCA_HIP_TRY(hipStreamSynchronize(stream), "hipStreamSynchronize");
  const std::vector<double> sums(h_sums, h_sums + 2 * kMaxObjectives + 2);
  const std::vector<double> reg(h_reg, h_reg + 2);
  std::vector<unsigned long long> hist(static_cast<size_t>(m), 0ull);
  if (!multilabel && accuracy) hist.assign(h_hist, h_hist + m);
  const int bad_labels = *h_bad;
  const double dual_reg = *h_dual_reg;
  if (bad_labels)
    return fail(SDCA_ERR_LABELS,
                multilabel ? "invalid labels or offsets: the first offset must be 0, and every "
                             "example needs 1 to m - 1 distinct, sorted labels in [0, m)"
                           : "a label is outside [0, m)");

  // eval_end: primal_loss *= coeff; primal = loss + reg; dual = loss - reg;
  // accuracy = partial_sum(hist) / n; rank_loss /= n (eval/core.h:43-95).
  double preg = preg_in, dreg = dreg_in;
  if (dW) {
    preg = reg[0] - (dW0 ? reg[1] : 0.0);
    dreg = reg[0];
  }
  if (dA_reg) {  // regularizers_dual adds the same term to both (objective_base.h:92-105)
    preg = dual_reg;
    dreg = dual_reg;
  }
  for (int o = 0; o < n_obj; ++o) {
    sdca_eval_record& r = records[o];
    r.primal_loss = loss_coeff(objs[o]) * sums[2 * o];
    r.rank_loss = multilabel ? sums[2 * kMaxObjectives] / static_cast<double>(n) : 0.0;
    if (test) {
      // eval_test holds the primal loss and the accuracy / rank loss only.
      r.dual_loss = r.primal_regularizer = r.dual_regularizer = r.dual = 0.0;
      r.primal = r.primal_loss;
      continue;
    }
    r.dual_loss = sums[2 * o + 1];
    r.primal_regularizer = preg;
    r.dual_regularizer = dreg;
    r.primal = r.primal_loss + preg;
    r.dual = r.dual_loss - dreg;
  }
  if (!multilabel && accuracy) {
    // eval_end: partial_sum of the counts, then scaled by coeff = 1 / n, both
    // in the Result type (eval/core.h:65-68), so the fractions are the
    // reference's to the last bit.
    unsigned long long run = 0;
    const double coeff_d = 1.0 / static_cast<double>(n);
    const float coeff_f = 1.0f / static_cast<float>(n);
    for (int64_t j = 0; j < m; ++j) {
      run += hist[j];
      accuracy[j] = result == SDCA_F32
                        ? static_cast<double>(static_cast<float>(run) * coeff_f)
                        : static_cast<double>(run) * coeff_d;
    }
  }
  return SDCA_OK;
}

}  // namespace

extern "C" {

int sdca_scores(sdca_dtype data, int64_t d, int64_t m, int64_t n, const void* X, const void* W,
                void* S, unsigned flags, void* stream_ptr) {
  using namespace sdca_gpu;
  g_last_error.clear();
  int rc = check_dtypes(data, data);
  if (rc) return rc;
  if (d < 1 || m < 1 || n < 0) return fail(SDCA_ERR_ARG_RANGE, "need d >= 1, m >= 1, n >= 0");
  if (n == 0) return SDCA_OK;
  if (!X || !W || !S) return fail(SDCA_ERR_ARG_NULL, "X, W and S must not be NULL");
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  const size_t es = dtype_size(data);
  DeviceBuffer dx, dw, ds;
  const void* pX = X;
  const void* pW = W;
  void* pS = S;
  if (flags & SDCA_HOST_PTR) {
    if ((rc = stage_in(X, es * d * n, dx, stream))) return rc;
    if ((rc = stage_in(W, es * d * m, dw, stream))) return rc;
    SDCA_HIP_TRY(hipMalloc(&ds.ptr, es * m * n), "hipMalloc(staging)");
    pX = dx.ptr;
    pW = dw.ptr;
    pS = ds.ptr;
  }
  if (data == SDCA_F32) {
    void* gws = nullptr;
    size_t gws_bytes = 0;
    if ((rc = gemm_workspace(stream, n, m, d, &gws, &gws_bytes))) return rc;
    SDCA_HIP_TRY(launch_scores_gemm(static_cast<const float*>(pX), static_cast<const float*>(pW),
                                    static_cast<float*>(pS), n, m, d, stream, gws, gws_bytes),
                 "scores kernel");
  } else
    SDCA_HIP_TRY(launch_scores_gemm_f64(static_cast<const double*>(pX), static_cast<const double*>(pW),
                                        static_cast<double*>(pS), n, m, d, stream), "scores kernel");
  if (flags & SDCA_HOST_PTR) {
    SDCA_HIP_TRY(hipMemcpyAsync(S, pS, es * m * n, hipMemcpyDeviceToHost, stream), "hipMemcpyAsync(D2H)");
    SDCA_HIP_TRY(hipStreamSynchronize(stream), "hipStreamSynchronize");
  }
  return SDCA_OK;
}

// Feature input (X, W), kernel input (kernel: X = K, W = A, d = n_train) or
// given scores (S).
int sdca_recompute_primal(sdca_dtype data, int64_t d, int64_t m, int64_t n, const void* X,
                          const void* A, const void* W0, void* W, unsigned flags, void* stream_ptr) {
  using namespace sdca_gpu;
  g_last_error.clear();
  int rc = check_dtypes(data, data);
  if (rc) return rc;
  if (d < 1 || m < 1 || n < 1) return fail(SDCA_ERR_ARG_RANGE, "need d, m, n >= 1");
  if (!X || !A || !W) return fail(SDCA_ERR_ARG_NULL, "X, A and W must not be NULL");
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  const size_t es = dtype_size(data);
  DeviceBuffer dx, da, dw0, dw;
  const void* pX = X;
  const void* pA = A;
  const void* pW0 = W0;
  void* pW = W;
  if (flags & SDCA_HOST_PTR) {
    if ((rc = stage_in(X, es * d * n, dx, stream))) return rc;
    if ((rc = stage_in(A, es * m * n, da, stream))) return rc;
    if (W0 && (rc = stage_in(W0, es * d * m, dw0, stream))) return rc;
    SDCA_HIP_TRY(hipMalloc(&dw.ptr, es * d * m), "hipMalloc(staging)");
    pX = dx.ptr;
    pA = da.ptr;
    pW0 = W0 ? dw0.ptr : nullptr;
    pW = dw.ptr;
  }
  // W (m x d row-major) = A' (m x n) X (n x d): the score GEMM with both
  // operands transposed once so that the contraction over n runs along rows.
  void* ws = nullptr;
  if ((rc = workspace(stream, 3, es * static_cast<size_t>(n) * static_cast<size_t>(m + d), &ws)))
    return rc;
  void* At = ws;
  void* Xt = static_cast<char*>(ws) + es * static_cast<size_t>(n) * static_cast<size_t>(m);
  SDCA_HIP_TRY(launch_transpose(data, pA, At, n, m, stream), "transpose kernel");
  SDCA_HIP_TRY(launch_transpose(data, pX, Xt, n, d, stream), "transpose kernel");
  if (data == SDCA_F32) {
    void* gws = nullptr;
    size_t gws_bytes = 0;
    if ((rc = gemm_workspace(stream, m, d, n, &gws, &gws_bytes))) return rc;
    SDCA_HIP_TRY(launch_scores_gemm(static_cast<const float*>(At), static_cast<const float*>(Xt),
                                    static_cast<float*>(pW), m, d, n, stream, gws, gws_bytes),
                 "GEMM kernel");
  } else
    SDCA_HIP_TRY(launch_scores_gemm_f64(static_cast<const double*>(At),
                                        static_cast<const double*>(Xt), static_cast<double*>(pW),
                                        m, d, n, stream), "GEMM kernel");
  if (pW0) SDCA_HIP_TRY(launch_add(data, pW, pW0, d * m, stream), "add kernel");
  if (flags & SDCA_HOST_PTR) {
    SDCA_HIP_TRY(hipMemcpyAsync(W, pW, es * d * m, hipMemcpyDeviceToHost, stream), "hipMemcpyAsync(D2H)");
    SDCA_HIP_TRY(hipStreamSynchronize(stream), "hipStreamSynchronize");
  }
  return SDCA_OK;
}

static int eval_common(const sdca_objective* objs, int n_obj, sdca_dtype data, sdca_dtype result,
                       int64_t d, int64_t m, int64_t n, const void* X, const void* W,
                       const void* S, const void* A, const void* W0, const int64_t* labels,
                       const int64_t* offsets, double preg, double dreg,
                       sdca_eval_record* records, double* accuracy, double* per_example,
                       unsigned flags, void* stream_ptr, bool kernel = false) {
  using namespace sdca_gpu;
  g_last_error.clear();
  int rc = check_dtypes(data, result);
  if (rc) return rc;
  if (m < 2) return fail(SDCA_ERR_ARG_RANGE, "m must be >= 2 (got %lld)", (long long)m);
  if (n < 1) return fail(SDCA_ERR_ARG_RANGE, "n must be >= 1 (got %lld)", (long long)n);
  if (m > max_rows(data))
    return fail(SDCA_ERR_NOT_IMPLEMENTED,
                "the evaluation supports m <= %lld for this element type on the GPU",
                (long long)max_rows(data));
  if (n > INT32_MAX / 2) return fail(SDCA_ERR_ARG_RANGE, "n too large");
  const bool multilabel = offsets != nullptr;
  if ((rc = check_objectives(objs, n_obj, m, multilabel))) return rc;
  if (!records) return fail(SDCA_ERR_ARG_NULL, "records must not be NULL");
  if (!labels) return fail(SDCA_ERR_ARG_NULL, "labels must not be NULL");
  const bool host = (flags & SDCA_HOST_PTR) != 0;
  if (host && (rc = check_labels(labels, offsets, m, n))) return rc;
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  const size_t es = dtype_size(data);
  DeviceBuffer dx, dw, ds, da, dw0, dl, doff;
  const void* pX = X;
  const void* pW = W;
  const void* pS = S;
  const void* pA = A;
  const void* pW0 = W0;
  const int64_t* pl = labels;
  const int64_t* poff = offsets;
  if (host) {
    const int64_t nlab = multilabel ? offsets[n] : n;
    if (X && (rc = stage_in(X, es * d * n, dx, stream))) return rc;
    if (W && (rc = stage_in(W, es * d * m, dw, stream))) return rc;
    if (S && (rc = stage_in(S, es * m * n, ds, stream))) return rc;
    if (A && (rc = stage_in(A, es * m * (kernel ? d : n), da, stream))) return rc;
    if (W0 && (rc = stage_in(W0, es * d * m, dw0, stream))) return rc;
    if ((rc = stage_in(labels, sizeof(int64_t) * nlab, dl, stream))) return rc;
    if (offsets && (rc = stage_in(offsets, sizeof(int64_t) * (n + 1), doff, stream))) return rc;
    pX = X ? dx.ptr : nullptr;
    pW = W ? dw.ptr : nullptr;
    pS = S ? ds.ptr : nullptr;
    pA = A ? da.ptr : nullptr;
    pW0 = W0 ? dw0.ptr : nullptr;
    pl = static_cast<const int64_t*>(dl.ptr);
    poff = offsets ? static_cast<const int64_t*>(doff.ptr) : nullptr;
  }
  const bool test = (flags & SDCA_EVAL_TEST) != 0;
  if (kernel) {
    // scores_i = A K_i (eval/scores.h:30-47) as W' X with W = A' (n_train x m,
    // column-major), transposed once into the stream's workspace.
    void* wt = nullptr;
    if ((rc = workspace(stream, 3, es * static_cast<size_t>(m) * static_cast<size_t>(d), &wt))) return rc;
    SDCA_HIP_TRY(launch_transpose(data, pA, wt, d, m, stream), "transpose kernel");
    pW = wt;
  }
  bool fused = false;
  if (!pS && !kernel && data == SDCA_F32 && (flags & SDCA_EVAL_FUSED)) {
    EvalLaunch probe;
    probe.data = data;
    probe.result = result;
    probe.m = m;
    probe.n = n;
    probe.A = test ? nullptr : pA;
    probe.offsets = poff;
    probe.objs.n = n_obj;
    for (int o = 0; o < n_obj; ++o) {
      probe.objs.o[o].kind = objs[o].kind;
      probe.objs.o[o].k = static_cast<int>(objs[o].k);
    }
    fused = eval_fused_supported(probe, d);
  }
  if (fused) {
    // The fused kernel's buffer for the score rows of deferred examples.
    void* sbuf = nullptr;
    if ((rc = workspace(stream, 1, es * static_cast<size_t>(m) * static_cast<size_t>(n), &sbuf))) return rc;
    return eval_on_device(objs, n_obj, data, result, m, n, sbuf, pA, pl, poff, pW, pW0, d * m,
                          nullptr, test, preg, dreg, records, accuracy, per_example, host, stream,
                          static_cast<const float*>(pX), static_cast<const float*>(pW), d);
  }
  if (!pS) {
    // scores = W' X into the stream's workspace
    void* sbuf = nullptr;
    if ((rc = workspace(stream, 1, es * static_cast<size_t>(m) * static_cast<size_t>(n), &sbuf))) return rc;
    if (data == SDCA_F32) {
      void* gws = nullptr;
      size_t gws_bytes = 0;
      if ((rc = gemm_workspace(stream, n, m, d, &gws, &gws_bytes))) return rc;
      SDCA_HIP_TRY(launch_scores_gemm(static_cast<const float*>(pX), static_cast<const float*>(pW),
                                      static_cast<float*>(sbuf), n, m, d, stream, gws, gws_bytes),
                   "scores kernel");
    } else
      SDCA_HIP_TRY(launch_scores_gemm_f64(static_cast<const double*>(pX),
                                          static_cast<const double*>(pW), static_cast<double*>(sbuf),
                                          n, m, d, stream), "scores kernel");
    pS = sbuf;
  }
  return eval_on_device(objs, n_obj, data, result, m, n, pS, pA, pl, poff,
                        (X && !kernel) ? pW : nullptr, (X && !kernel) ? pW0 : nullptr, d * m,
                        kernel ? pA : nullptr, test, preg, dreg, records, accuracy, per_example,
                        host, stream);
}

int sdca_eval_features(const sdca_objective* objs, int n_obj, sdca_dtype data, sdca_dtype result,
                       int64_t d, int64_t m, int64_t n, const void* X, const void* W,
                       const void* A, const void* W0, const int64_t* labels,
                       const int64_t* offsets, sdca_eval_record* records, double* accuracy,
                       double* per_example, unsigned flags, void* stream) {
  if (!X || !W) return fail(SDCA_ERR_ARG_NULL, "X and W must not be NULL");
  if (d < 1) return fail(SDCA_ERR_ARG_RANGE, "d must be >= 1 (got %lld)", (long long)d);
  return eval_common(objs, n_obj, data, result, d, m, n, X, W, nullptr, A, W0, labels, offsets,
                     0.0, 0.0, records, accuracy, per_example, flags, stream);
}

int sdca_eval_kernel(const sdca_objective* objs, int n_obj, sdca_dtype data, sdca_dtype result,
                     int64_t n_train, int64_t m, int64_t n, const void* K, const void* A,
                     const int64_t* labels, const int64_t* offsets, sdca_eval_record* records,
                     double* accuracy, double* per_example, unsigned flags, void* stream) {
  if (!K || !A) return fail(SDCA_ERR_ARG_NULL, "K and A must not be NULL");
  if (n_train < 1) return fail(SDCA_ERR_ARG_RANGE, "n_train must be >= 1 (got %lld)", (long long)n_train);
  if (!(flags & SDCA_EVAL_TEST) && n != n_train)
    return fail(SDCA_ERR_ARG_RANGE,
                "a training set's kernel is n_train x n_train (got n_train %lld, n %lld)",
                (long long)n_train, (long long)n);
  return eval_common(objs, n_obj, data, result, n_train, m, n, K, nullptr, nullptr, A, nullptr,
                     labels, offsets, 0.0, 0.0, records, accuracy, per_example, flags, stream,
                     true);
}

int sdca_eval_scores(const sdca_objective* objs, int n_obj, sdca_dtype data, sdca_dtype result,
                     int64_t m, int64_t n, const void* S, const void* A, const int64_t* labels,
                     const int64_t* offsets, double primal_regularizer, double dual_regularizer,
                     sdca_eval_record* records, double* accuracy, double* per_example,
                     unsigned flags, void* stream) {
  if (!S) return fail(SDCA_ERR_ARG_NULL, "S must not be NULL");
  return eval_common(objs, n_obj, data, result, 0, m, n, nullptr, nullptr, S, A, nullptr, labels,
                     offsets, primal_regularizer, dual_regularizer, records, accuracy, per_example,
                     flags, stream);
}

int sdca_epoch_order(int64_t n, int64_t epoch, int64_t* order) {
  g_last_error.clear();
  if (n < 0 || epoch < 0) return fail(SDCA_ERR_ARG_RANGE, "n and epoch must be >= 0");
  if (n > 0 && !order) return fail(SDCA_ERR_ARG_NULL, "order must not be NULL");
  // solver.h:75-92: a default-seeded minstd_rand at the start of the solve,
  // the examples 0..n-1, one std::shuffle per epoch (solver.h:108-112).
  std::minstd_rand generator;
  generator.seed();
  std::vector<int64_t> examples(static_cast<size_t>(n));
  std::iota(examples.begin(), examples.end(), int64_t(0));
  for (int64_t e = 0; e <= epoch; ++e) std::shuffle(examples.begin(), examples.end(), generator);
  std::copy(examples.begin(), examples.end(), order);
  return SDCA_OK;
}

}  // extern "C"

namespace {

// The epoch on feature input (X: n x d, W: m x d) or, with `kernel`, on
// kernel input (X: the n x n kernel matrix, d = n, W and norms unused).
int epoch_common(const sdca_objective* obj, sdca_dtype data, sdca_dtype result, int64_t d,
                 int64_t m, int64_t n, const void* X, void* W, void* A, const int64_t* labels,
                 const int64_t* offsets, const int64_t* order, int64_t count, const void* norms,
                 unsigned flags, void* stream_ptr, bool kernel) {
  using namespace sdca_gpu;
  if (!obj) return fail(SDCA_ERR_ARG_NULL, "obj must not be NULL");
  if (obj->kind < SDCA_OBJ_HINGE_TOPK || obj->kind > SDCA_OBJ_MULTILABEL_ENTROPY)
    return fail(SDCA_ERR_NOT_IMPLEMENTED, "unknown objective kind %d",
                static_cast<int>(obj->kind));
  const bool multilabel = obj->kind >= SDCA_OBJ_MULTILABEL_HINGE;
  if (multilabel && !offsets)
    return fail(SDCA_ERR_ARG_NULL, "the multilabel objectives need label offsets");
  if (!((data == SDCA_F32 && (result == SDCA_F32 || result == SDCA_F64)) ||
        (data == SDCA_F64 && result == SDCA_F64)))
    return fail(SDCA_ERR_PRECISION,
                "the epoch takes (float, float), (float, double) or (double, double)");
  if (d < 1 || m < 2 || n < 1 || count < 0)
    return fail(SDCA_ERR_ARG_RANGE, "need d >= 1, m >= 2, n >= 1, count >= 0");
  if (m > epoch_max_m(data, obj->kind))
    return fail(SDCA_ERR_NOT_IMPLEMENTED,
                "the epoch supports m <= %lld for this element type and objective",
                (long long)epoch_max_m(data, obj->kind));
  if (n > INT32_MAX || d > INT32_MAX) return fail(SDCA_ERR_ARG_RANGE, "matrix too large");
  if (!order && count > n)
    return fail(SDCA_ERR_ARG_RANGE, "count (%lld) > n (%lld) without an order",
                (long long)count, (long long)n);
  int rc = check_objectives(obj, 1, m, multilabel);
  if (rc) return rc;
  if (!X || (!W && !kernel) || !A || !labels)
    return fail(SDCA_ERR_ARG_NULL,
                kernel ? "K, A and labels must not be NULL" : "X, W, A and labels must not be NULL");
  if (kernel) norms = nullptr;
  if (count == 0) return SDCA_OK;
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  const bool host = (flags & SDCA_HOST_PTR) != 0;
  const size_t es = dtype_size(data);
  DeviceBuffer dx, dw, da, dl, doff, dord, dnorm;
  if (host && multilabel) {
    // The CSR structure bounds the labels staged below (offsets[n] of them);
    // the labels' values are checked per example on the device.
    if (offsets[0] != 0) return fail(SDCA_ERR_LABELS, "The first offset must be 0.");
    for (int64_t i = 0; i < n; ++i)
      if (offsets[i + 1] < offsets[i])
        return fail(SDCA_ERR_LABELS, "offsets decrease at example %lld", (long long)i);
  }
  if (host) {
    if ((rc = stage_in(X, es * d * n, dx, stream))) return rc;
    if (!kernel && (rc = stage_in(W, es * d * m, dw, stream))) return rc;
    if ((rc = stage_in(A, es * m * n, da, stream))) return rc;
    const int64_t nlab = multilabel ? offsets[n] : n;
    if ((rc = stage_in(labels, sizeof(int64_t) * nlab, dl, stream))) return rc;
    if (multilabel && (rc = stage_in(offsets, sizeof(int64_t) * (n + 1), doff, stream))) return rc;
    if (order && (rc = stage_in(order, sizeof(int64_t) * count, dord, stream))) return rc;
    if (norms && (rc = stage_in(norms, es * n, dnorm, stream))) return rc;
  }
  void* ws = nullptr;
  if ((rc = workspace(stream, 4, epoch_workspace_bytes(data, d, m, n, norms != nullptr, kernel),
                      &ws)))
    return rc;
  EpochLaunch a;
  a.data = data;
  a.result = result;
  a.kind = obj->kind;
  a.c = obj->c;
  a.gamma = obj->gamma;
  a.k = static_cast<int>(obj->k);
  a.d = d;
  a.m = m;
  a.n = n;
  a.X = host ? dx.ptr : X;
  a.W = kernel ? nullptr : host ? dw.ptr : W;
  a.A = host ? da.ptr : A;
  a.labels = host ? static_cast<const int64_t*>(dl.ptr) : labels;
  a.offsets = !multilabel ? nullptr : host ? static_cast<const int64_t*>(doff.ptr) : offsets;
  a.order = host && order ? static_cast<const int64_t*>(dord.ptr) : order;
  a.count = count;
  a.norms = host && norms ? dnorm.ptr : norms;
  a.kernel = kernel;
  a.ws = ws;
  a.stream = stream;
  int* flag = nullptr;
  SDCA_HIP_TRY(launch_epoch(a, &flag), "SDCA epoch kernels");
  if (host) {
    if (!kernel)
      SDCA_HIP_TRY(hipMemcpyAsync(W, dw.ptr, es * d * m, hipMemcpyDeviceToHost, stream),
                   "hipMemcpyAsync(D2H)");
    SDCA_HIP_TRY(hipMemcpyAsync(A, da.ptr, es * m * n, hipMemcpyDeviceToHost, stream),
                 "hipMemcpyAsync(D2H)");
  }
  int bad = 0;
  SDCA_HIP_TRY(hipMemcpyAsync(&bad, flag, sizeof(int), hipMemcpyDeviceToHost, stream),
               "hipMemcpyAsync(D2H)");
  SDCA_HIP_TRY(hipStreamSynchronize(stream), "hipStreamSynchronize");
  if (bad)
    return fail(SDCA_ERR_LABELS,
                "an example index outside [0, n), a label outside [0, m) (read as 0), or a "
                "multilabel example whose labels are not 1..m-1 distinct sorted ones (skipped)");
  return SDCA_OK;
}

}  // namespace

extern "C" {

int sdca_epoch_features(const sdca_objective* obj, sdca_dtype data, sdca_dtype result, int64_t d,
                        int64_t m, int64_t n, const void* X, void* W, void* A,
                        const int64_t* labels, const int64_t* offsets, const int64_t* order,
                        int64_t count, const void* norms, unsigned flags, void* stream_ptr) {
  g_last_error.clear();
  return epoch_common(obj, data, result, d, m, n, X, W, A, labels, offsets, order, count, norms,
                      flags, stream_ptr, false);
}

int sdca_epoch_kernel(const sdca_objective* obj, sdca_dtype data, sdca_dtype result, int64_t m,
                      int64_t n, const void* K, void* A, const int64_t* labels,
                      const int64_t* offsets, const int64_t* order, int64_t count,
                      unsigned flags, void* stream_ptr) {
  g_last_error.clear();
  return epoch_common(obj, data, result, n, m, n, K, nullptr, A, labels, offsets, order, count,
                      nullptr, flags, stream_ptr, true);
}

}  // extern "C"
