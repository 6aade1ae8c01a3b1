// Host-side launch interface of the evaluation kernels (internal).
#ifndef SDCA_HIP_EVAL_LAUNCH_HPP
#define SDCA_HIP_EVAL_LAUNCH_HPP

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/sdca_hip.h"

namespace sdca_gpu {

constexpr int kMaxObjectives = 8;
// Top-k objectives keep a register list of the k + 1 largest for
// k <= kEvalMaxK; larger k takes k + 1 passes of a group argmax.
constexpr int64_t kEvalMaxK = 8;

// One objective as the kernels see it.
struct EvalObj {
  int kind;
  int k;
  double c, gamma;
};

struct EvalObjs {
  int n;
  EvalObj o[kMaxObjectives];
};

struct EvalLaunch {
  int data, result;
  int64_t m, n;
  const void* S;           // n x m scores (device)
  const void* A;           // n x m dual variables or NULL (device)
  const int64_t* labels;   // device
  const int64_t* offsets;  // device, multilabel CSR or NULL
  EvalObjs objs;
  double* per_example;     // device: n x n_obj x 2 (primal, dual) before the coefficient
  int* counts;             // device: n (multiclass top-k counts), or NULL
  double* rank;            // device: n (multilabel rank loss per example), or NULL
  int* slow;               // device: [0] = count, then (example, objective) pairs
  int* bad;                // device: set to 1 by an example with invalid labels
  hipStream_t stream;
};

// S = X W^T for fp32 on the matrix cores; X: n x d, W: m x d, S: n x m (row-major).
// From kBlasMinMacs multiply-adds (n m d) and kBlasMinClasses classes on,
// through hipBLASLt when it has an algorithm for the shape within the
// caller's workspace (blas_ws, at most kBlasWorkspaceBytes; none: only
// algorithms without one), else the hand-written MFMA kernel.  (At m = 200,
// d = 1024, n = 5e5 the library's pick took 1.90-1.94 ms against the MFMA
// kernel's 224-wide tiles at 1.84-1.88 ms.)
constexpr int64_t kBlasMinMacs = int64_t(1) << 32;
constexpr int64_t kBlasMinClasses = 512;
constexpr size_t kBlasWorkspaceBytes = size_t(32) << 20;
inline bool blas_shape(int64_t n, int64_t m, int64_t d) {
  return n > 0 && m >= kBlasMinClasses && d > 0 && n * m >= kBlasMinMacs / d;
}
hipError_t launch_scores_gemm(const float* X, const float* W, float* S, int64_t n, int64_t m,
                              int64_t d, hipStream_t stream, void* blas_ws = nullptr,
                              size_t blas_ws_bytes = 0);
// The hand-written MFMA kernel alone (the fused pass's k order).
hipError_t launch_scores_gemm_mfma(const float* X, const float* W, float* S, int64_t n,
                                   int64_t m, int64_t d, hipStream_t stream);
// The same product through hipBLASLt; false (S untouched or to be
// overwritten) when the library declines the shape or fails.
bool blas_scores_gemm(const float* X, const float* W, float* S, int64_t n, int64_t m, int64_t d,
                      hipStream_t stream, void* ws, size_t ws_bytes);
// The same contraction in double on the matrix cores (v_mfma_f64_16x16x4f64).
hipError_t launch_scores_gemm_f64(const double* X, const double* W, double* S, int64_t n,
                                  int64_t m, int64_t d, hipStream_t stream);
// The fused pass (scores on the matrix cores and the multiclass epilogue in
// one kernel, scores not stored): fp32 feature input, m <= 1024.  Deferred
// examples get their score row written to s_deferred (n x m) for
// launch_eval_slow, which then reads it as S.
bool eval_fused_supported(const EvalLaunch& a, int64_t d);
hipError_t launch_eval_fused(const float* X, const float* W, const EvalLaunch& a, int64_t d,
                             float* s_deferred);
// Per-example epilogue (losses, counts, rank loss) and its deferred examples.
hipError_t launch_eval_epilogue(const EvalLaunch& a);
hipError_t launch_eval_slow(const EvalLaunch& a);
// Deterministic reductions: sums[o*2+{0,1}] = sum_i per_example; rank sum;
// hist[c] = #{i: counts[i] == c}.  `partials` holds eval_reduce_scratch(n_obj)
// doubles.
int64_t eval_reduce_scratch(int n_obj);
hipError_t launch_eval_reduce(const EvalLaunch& a, double* sums, double* rank_sum,
                              unsigned long long* hist, double* partials);
// 0.5 <W, W> and <W0, W> in double (out[0], out[1]); `partials` holds 1024 doubles.
hipError_t launch_regularizer(int data, const void* W, const void* W0, int64_t count,
                              double* partials, double* out, hipStream_t stream);

// out (cols x rows) = in (rows x cols)^T, both row-major.
hipError_t launch_transpose(int data, const void* in, void* out, int64_t rows, int64_t cols,
                            hipStream_t stream);
// y[i] = x[i] + y[i].
hipError_t launch_add(int data, void* y, const void* x, int64_t count, hipStream_t stream);
// *out = sum_i static_cast<Result>(dot(A_i, S_i)) / 2 over n examples of m
// entries; `per_example` holds n doubles.
hipError_t launch_dual_regularizer(int data, int result, const void* A, const void* S, int64_t m,
                                   int64_t n, double* per_example, double* out,
                                   hipStream_t stream);

}  // namespace sdca_gpu

#endif
