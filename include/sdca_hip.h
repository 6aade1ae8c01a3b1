/*
 * sdca_hip.h - C ABI of the MI355X (gfx950) batched prox + evaluation path.
 *
 * Plain C: pointers, sizes and enums only.  Every entry point replaces one
 * loop of libsdca v0.3.1 (header-only C++11); the reference interface each
 * one stands in for is cited beside it.  The C++ drop-in overloads with the
 * reference's own names and signatures live in sdca_hip.hpp.
 *
 * Memory: by default every pointer argument is a device pointer
 * (hipMalloc'ed or torch CUDA memory) and the work is enqueued on `stream`
 * (a hipStream_t, NULL = the default stream) without a host synchronisation.
 * With SDCA_HOST_PTR the arrays are host memory: the library stages them
 * through device buffers and returns after the results are copied back.
 *
 * Errors: every function returns an sdca_status; the message of the last
 * failure on the calling thread is returned by sdca_last_error().  Nothing
 * aborts.  Argument checks mirror the Matlab front end
 * (src/matlab/mex_prox.cpp:132-136): rhs >= 0, rho >= 0, alpha > 0,
 * 1 <= k <= m, 1 <= p <= m - 1 (p only for the two-block operator).
 */
#ifndef SDCA_HIP_H
#define SDCA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SDCA_HIP_ABI_VERSION 1

typedef enum sdca_status {
  SDCA_OK = 0,
  SDCA_ERR_ARG_NULL = 1,        /* a required pointer is NULL */
  SDCA_ERR_ARG_RANGE = 2,       /* LIBSDCA:outOfRange (mex_util.h) */
  SDCA_ERR_PRECISION = 3,       /* LIBSDCA:precision: unknown dtype */
  SDCA_ERR_NOT_IMPLEMENTED = 4, /* e.g. long double, or an op not on this path */
  SDCA_ERR_OUT_OF_MEMORY = 5,
  SDCA_ERR_HIP = 6,             /* a HIP runtime call failed */
  SDCA_ERR_PROX = 7,            /* LIBSDCA:prox: unknown operator */
  SDCA_ERR_LABELS = 8           /* invalid labels / offsets (output.h:169-208) */
} sdca_status;

typedef enum sdca_dtype {
  SDCA_F32 = 0,
  SDCA_F64 = 1,
  SDCA_LONG_DOUBLE = 2 /* valid in the reference (mex_prox.cpp:195); not on the GPU */
} sdca_dtype;

/* Operators of the Matlab prox front end (mex_prox.cpp:145-172). */
typedef enum sdca_prox_op {
  SDCA_PROX_KNAPSACK_EQ = 0,   /* knapsack_eq.h:143-157 */
  SDCA_PROX_KNAPSACK_LE = 1,   /* knapsack_le.h:78-92 */
  SDCA_PROX_TOPK_SIMPLEX = 2,  /* topk_simplex.h:100-113 */
  SDCA_PROX_TOPK_CONE = 3,     /* topk_cone.h:187-199 */
  SDCA_PROX_ENTROPY = 4,       /* entropy.h:85-98 */
  SDCA_PROX_ENTROPY_NORM = 5,  /* entropy_norm.h:213-226 */
  SDCA_PROX_TOPK_ENTROPY = 6,  /* topk_entropy.h:106-118 */
  SDCA_PROX_TWO_SIMPLEX = 7,   /* two_simplex.h:183-196 */
  SDCA_PROX_LAMBERT_W_EXP = 8, /* apply(dim, ..., lambert_w_exp_map), proxdef.h:386-400 */
  SDCA_PROX_KNAPSACK_LE_BIASED = 9,   /* knapsack_le_biased.h:165-180 (uses rho) */
  SDCA_PROX_TOPK_SIMPLEX_BIASED = 10, /* topk_simplex_biased.h:105-119 (uses rho) */
  SDCA_PROX_TOPK_CONE_BIASED = 11,    /* topk_cone_biased.h:145-158 (uses rho) */
  SDCA_PROX_TOPK_ENTROPY_BIASED = 12, /* topk_entropy_biased.h:302-315 (uses k, alpha) */
  SDCA_PROX_TWO_SIMPLEX_SORT = 13,    /* two_simplex_sort.h:175-190 (uses p / col_p) */
  SDCA_PROX_TWO_ENTROPY = 14          /* prox_two_entropy(p, first, last, aux, alpha),
                                         two_entropy.h:280-292, batched (uses p / col_p, alpha) */
} sdca_prox_op;

/* Operator parameters; defaults as in mex_prox.cpp:121-127. */
typedef struct sdca_prox_params {
  double lo, hi, rhs, rho, alpha;
  int64_t k, p;
} sdca_prox_params;

/* Per-column threshold record (proxdef.h:29-67): x <- clamp(map(x - t), lo, hi).
 * For the two-block operator, two records per column (block a, then b). */
typedef struct sdca_thresholds {
  double t, lo, hi;
} sdca_thresholds;

/* Which return of the operator's threshold function produced a record. */
typedef enum sdca_prox_branch {
  /* the operator's own solve: knapsack_eq's variable fixing
     (knapsack_eq.h:25-109), the entropy and Lambert solves (entropy.h:30-52,
     entropy_norm.h:157-180, two_entropy.h:131-231); for the two-block
     simplex, common sum rhs (two_simplex.h:44-67 phase 1;
     two_simplex_sort.h:84-87) */
  SDCA_BRANCH_SEARCH = 0,
  /* knapsack_le: the clamp at t = 0 meets the sum (knapsack_le.h:40-43) */
  SDCA_BRANCH_INACTIVE = 1,
  /* top-k: the k largest sum to <= 16 eps, all zero (topk_cone.h:34-41) */
  SDCA_BRANCH_ZERO = 2,
  /* top-k: the k largest at hi, nothing free (topk_cone.h:43-52,
     topk_simplex.h:53-58) */
  SDCA_BRANCH_CONSTANT = 3,
  /* the equality knapsack's solution reached from another operator:
     knapsack_le active (knapsack_le.h:39-40), the top-k simplex with
     hi = rhs / k (topk_simplex.h:55-65), knapsack_le_biased's equality
     solution (knapsack_le_biased.h:117-120) */
  SDCA_BRANCH_KNAPSACK = 4,
  /* a U/M scan accepted a partition: topk_cone_search (topk_cone.h:104),
     the biased cone (topk_cone_biased.h:57), knapsack_le_biased's search
     (knapsack_le_biased.h:62) */
  SDCA_BRANCH_SCAN = 5,
  /* a U/M scan accepted nothing: the default zero record (topk_cone.h:131,
     topk_cone_biased.h:85, knapsack_le_biased.h:89) */
  SDCA_BRANCH_DEFAULT = 6,
  /* top-k entropy: U empty (topk_entropy.h:38-41; biased:
     topk_entropy_biased.h:219-233) */
  SDCA_BRANCH_U_EMPTY = 7,
  /* top-k entropy: U grown (topk_entropy.h:43-75; biased:
     topk_entropy_biased.h:235-269) */
  SDCA_BRANCH_U_GROWN = 8,
  /* two-block simplex: common sum below rhs (two_simplex.h:69-117 phase 2;
     two_simplex_sort.h:78-81) */
  SDCA_BRANCH_BELOW_RHS = 9
} sdca_prox_branch;

/* The sets of a record: the reference's record carries iterators first and
 * last over its permuted copy of the column (proxdef.h:29-67), [begin,
 * first) at hi, [first, last) free, [last, end) at lo; n_hi = first - begin,
 * n_mid = last - first, as the reference's own threshold function leaves
 * them (for example (k, 0) when the k largest are at hi, (0, m) for the top-k
 * entropy with U empty and for every biased top-k entropy record, (0, |kept|)
 * for the two-block simplex).  branch: an sdca_prox_branch. */
typedef struct sdca_prox_sets {
  int64_t n_hi;
  int64_t n_mid;
  int32_t branch;
  int32_t reserved;
} sdca_prox_sets;

#define SDCA_DEVICE_PTR 0u
#define SDCA_HOST_PTR 1u

/* Fills the defaults lo=0, hi=1, rhs=1, rho=1, alpha=1, k=1, p=1. */
void sdca_prox_params_default(sdca_prox_params* params);

/*
 * Batched prox over the n contiguous columns of an m x n column-major
 * matrix: replaces the loop prox(dim, first, last, aux, compute, params...)
 * (proxdef.h:279-298) and its two-block form (proxdef.h:301-324).
 *   data:   element type of in/out;
 *   result: the reference's Result template argument (internal precision);
 *   in/out: m*n elements each; out == in works in place like the reference;
 *   col_p:  for the two-block operators, optional per-column split p (n int64
 *           values in [1, m-1]); NULL uses params->p for every column.  Host
 *           values (SDCA_HOST_PTR) outside that range are rejected with
 *           SDCA_ERR_ARG_RANGE; device values are not read back by the host
 *           (the call stays asynchronous): the kernels bring an out-of-range
 *           value into [1, m-1], so no access leaves the column, and that
 *           column's result is the projection for the clamped split;
 *   thresholds: optional, n records (2n for the two-block operator) with the
 *           computed thresholds, in double.
 * The reference's `aux` scratch has no counterpart: scratch lives in
 * registers and LDS.  A column is held by one workgroup, in LDS up to 32768
 * rows of fp32 data and 16384 of fp64 (128 KiB of column).  Beyond that the
 * KNAPSACK_EQ, KNAPSACK_LE, ENTROPY and ENTROPY_NORM operators stream the
 * column from global memory and the others work on it in device memory
 * (sorted in, copied to or read from it, in a scratch of up to 512 MiB per
 * stream): every operator takes any m.
 */
int sdca_prox(sdca_prox_op op, sdca_dtype data, sdca_dtype result,
              int64_t m, int64_t n, const void* in, void* out,
              const sdca_prox_params* params, const int64_t* col_p,
              sdca_thresholds* thresholds, unsigned flags, void* stream);

/*
 * sdca_prox that also returns each record's sets and branch (the
 * reference's first / last, proxdef.h:29-67): sets holds n records (2n for
 * the two-block operators, block a then b), host or device memory as the
 * other arrays; NULL gives sdca_prox.  Not for SDCA_PROX_LAMBERT_W_EXP (no
 * records).  The sets are the GPU's own partition; next to the reference
 * they can differ only by entries tied with a threshold at rounding level,
 * and the branch only where the reference's own epsilon tests are decided at
 * rounding level.
 */
int sdca_prox_with_sets(sdca_prox_op op, sdca_dtype data, sdca_dtype result,
                        int64_t m, int64_t n, const void* in, void* out,
                        const sdca_prox_params* params, const int64_t* col_p,
                        sdca_thresholds* thresholds, sdca_prox_sets* sets,
                        unsigned flags, void* stream);

/*
 * sdca_prox without any device allocation.  No counterpart in the reference:
 * it is for callers that cannot allocate (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc).  Same arguments and
 * results as sdca_prox with device pointers (there is no flags argument:
 * host staging would allocate).  The deferred-column list of the top-k,
 * biased and sort-based two-simplex operators lives in a fixed device array
 * of the library, one per device, held until the process ends: those
 * operators take at most sdca_prox_noalloc_max_columns() columns (4,194,304)
 * per call and return SDCA_ERR_ARG_RANGE beyond; the other operators use no
 * scratch and take any n.  Every call on a device shares that array: calls
 * that overlap on one device (concurrent streams or host threads) race.
 */
int sdca_prox_noalloc(sdca_prox_op op, sdca_dtype data, sdca_dtype result,
                      int64_t m, int64_t n, const void* in, void* out,
                      const sdca_prox_params* params, const int64_t* col_p,
                      sdca_thresholds* thresholds, void* stream);

/* Largest n that sdca_prox_noalloc takes for the listed operators. */
int64_t sdca_prox_noalloc_max_columns(void);

/* Objectives of the evaluation pass (objective.h:55-160). */
typedef enum sdca_objective_kind {
  SDCA_OBJ_HINGE_TOPK = 0,             /* l2_hinge_topk.h:11-88 */
  SDCA_OBJ_HINGE_TOPK_SMOOTH = 1,      /* l2_hinge_topk.h:90-194 */
  SDCA_OBJ_TOPK_HINGE = 2,             /* l2_topk_hinge.h:10-88 */
  SDCA_OBJ_TOPK_HINGE_SMOOTH = 3,      /* l2_topk_hinge.h:90-198 */
  SDCA_OBJ_ENTROPY = 4,                /* l2_entropy.h:15-116 */
  SDCA_OBJ_ENTROPY_TOPK = 5,           /* l2_entropy_topk.h:11-109 */
  SDCA_OBJ_MULTILABEL_HINGE = 6,       /* l2_multilabel_hinge.h:10-98 */
  SDCA_OBJ_MULTILABEL_HINGE_SMOOTH = 7,/* l2_multilabel_hinge.h:100-210 */
  SDCA_OBJ_MULTILABEL_ENTROPY = 8      /* l2_multilabel_entropy.h:10-111 */
} sdca_objective_kind;

typedef struct sdca_objective {
  int32_t kind;   /* sdca_objective_kind */
  int32_t reserved;
  double c;       /* loss weight c = 1 / (lambda n) */
  double gamma;   /* smoothing (smooth objectives) */
  int64_t k;      /* top-k (top-k objectives) */
} sdca_objective;

/* One eval record (eval/types.h:12-20, 84-125) without the timing fields. */
typedef struct sdca_eval_record {
  double primal, dual;
  double primal_loss, dual_loss;
  double primal_regularizer, dual_regularizer;
  double rank_loss;   /* multilabel only (eval/types.h:110-125) */
} sdca_eval_record;

/*
 * Whole-dataset evaluation for feature input: replaces evaluate_dataset
 * (eval.h:15-51) for feature_input with multiclass or multilabel output.
 * Computes scores = W' X (W: d x m, X: d x n, both column-major), then per
 * example the dual loss, the top-k count histogram (multiclass) or rank loss
 * (multilabel) and the primal loss of each of the n_obj objectives, and
 * finishes each record as eval_end does (eval/core.h:43-95).
 *   A:       m x n dual variables, or NULL for all zeros;
 *   W0:      d x m initial primal variables (prox mode), or NULL;
 *   labels:  multiclass: n labels in [0, m); multilabel: CSR labels;
 *   offsets: NULL for multiclass; n+1 CSR offsets for multilabel;
 *   records: n_obj host records;
 *   accuracy: optional host array of m: top-(i+1) accuracy (after
 *           partial_sum and 1/n, eval/core.h:65-68), multiclass only;
 *   per_example: optional, n * n_obj * 2 doubles: (primal, dual) loss of
 *           each example and objective before the loss coefficient.
 * The objectives must all be multiclass or all multilabel.  m is at most
 * 32768 for fp32 data and 16384 for fp64 (an example's scores are held by
 * one workgroup); larger m returns SDCA_ERR_NOT_IMPLEMENTED.
 */
int sdca_eval_features(const sdca_objective* objs, int n_obj,
                       sdca_dtype data, sdca_dtype result,
                       int64_t d, int64_t m, int64_t n,
                       const void* X, const void* W, const void* A,
                       const void* W0, const int64_t* labels,
                       const int64_t* offsets, sdca_eval_record* records,
                       double* accuracy, double* per_example,
                       unsigned flags, void* stream);

/*
 * The same evaluation from precomputed scores S (m x n column-major), with
 * the primal regularizer 0.5 <W, W> (- <W0, W>) supplied by the caller:
 * the per-example part of evaluate_dataset (eval.h:36-47).  Used to check
 * the epilogue bit for bit on identical scores.
 */
int sdca_eval_scores(const sdca_objective* objs, int n_obj,
                     sdca_dtype data, sdca_dtype result,
                     int64_t m, int64_t n, const void* S, const void* A,
                     const int64_t* labels, const int64_t* offsets,
                     double primal_regularizer, double dual_regularizer,
                     sdca_eval_record* records, double* accuracy,
                     double* per_example, unsigned flags, void* stream);

/*
 * flags bit of the evaluation calls: evaluate a test set (eval_test,
 * eval/types.h:128-172, finished as eval/core.h:98-132): only the primal loss
 * (times the loss coefficient), the top-k accuracy or the rank loss are
 * computed; the dual variables of the examples, W0 and the regularizers are
 * not used, and the other record fields are 0.
 */
#define SDCA_EVAL_TEST 2u

/*
 * flags bit of sdca_eval_features: the fused form where it applies (fp32
 * data, multiclass, m <= 1024, the smooth top-k hinge and / or the softmax
 * cross-entropy, no dual variables): one kernel computes the scores on the
 * matrix cores and evaluates the examples from LDS without storing the
 * scores, instead of the default two-kernel form (scores written to a
 * device buffer by the GEMM, then the per-example kernel).  Below 2^32
 * multiply-adds (n m d) or 512 classes both forms give bit-identical
 * records; from there on the two-kernel form takes its scores from
 * hipBLASLt, whose summation order differs, and the records agree to the
 * rounding of the scores.
 * The default is the two-kernel form: on MI355X it
 * is the faster (the fused kernel holds 32 examples x all classes per
 * workgroup, is limited to 2 waves per SIMD by its registers and re-reads W
 * per 32 examples).
 */
#define SDCA_EVAL_FUSED 4u

/*
 * Whole-dataset evaluation for kernel input: evaluate_dataset (eval.h:15-51)
 * with kernel_input (data/input.h:44-76).  scores_i = A K_i
 * (eval/scores.h:30-47) for all i at once on the matrix cores, with
 *   K: n_train x n kernel matrix, column-major;
 *   A: m x n_train dual variables, column-major.
 * A training set (n == n_train) also gets each example's dual loss from its
 * column of A and the dual regularizer sum_i 0.5 <a_i, s_i>
 * (eval/regularizer.h:81-98, objective_base.h:92-105) in both regularizer
 * terms; there is no primal regularizer.  With SDCA_EVAL_TEST, the records
 * of a test set (K is n_train x n_test).  Other arguments as in
 * sdca_eval_features.
 */
int sdca_eval_kernel(const sdca_objective* objs, int n_obj,
                     sdca_dtype data, sdca_dtype result,
                     int64_t n_train, int64_t m, int64_t n,
                     const void* K, const void* A, const int64_t* labels,
                     const int64_t* offsets, sdca_eval_record* records,
                     double* accuracy, double* per_example,
                     unsigned flags, void* stream);

/*
 * One epoch of the SDCA solver on feature input (replaces one pass of the
 * example loop of solver::solve, solver.h:44-47: update_variables for each
 * example, update.h:52-85, with the objective's update_dual_variables) for
 * the nine objectives: the six multiclass ones (kind 0..5) and the three
 * multilabel ones (kind 6..8).  Per example i in `order`: scores W' x_i,
 * the dual update of a_i, and W -= x_i (a_old - a_new)' when
 * sum |a_old - a_new| exceeds epsilon.  The examples run in blocks whose
 * scores come from the matrix cores; the updates are the sequential loop's
 * (results equal up to the rounding of the scores' sums).
 *   X: d x n features, W: d x m primal and A: m x n dual variables, all
 *      column-major (each example's / class's values contiguous); W and A
 *      are updated in place;
 *   labels: n labels in [0, m) (multiclass, offsets NULL), or CSR labels
 *      with offsets (n + 1 row starts; multilabel: 1..m-1 distinct sorted
 *      labels per example, output.h:184-206);
 *   order: count example indices in [0, n), or NULL for 0..count-1;
 *   norms: n values ||x_i||^2 in the data type, or NULL (computed,
 *      scratch.h:27-41).
 * Device pointers on `stream` (flags 0), or host arrays with SDCA_HOST_PTR
 * (staged through device memory for the call, W and A copied back); (data,
 * result) one of (F32, F32), (F32, F64), (F64, F64); m at most 524280 (larger
 * m: SDCA_ERR_NOT_IMPLEMENTED before anything is enqueued; the example's
 * vectors stay in LDS up to 16384 (fp32) / 8192 (fp64) classes, 12200 /
 * 7268 multilabel, and move to device memory beyond).  Returns SDCA_ERR_LABELS
 * (after the epoch) for an index or multiclass label out of range (read as
 * 0) or a multilabel example whose labels break those rules (skipped).
 */
int sdca_epoch_features(const sdca_objective* obj, sdca_dtype data, sdca_dtype result,
                        int64_t d, int64_t m, int64_t n, const void* X, void* W, void* A,
                        const int64_t* labels, const int64_t* offsets, const int64_t* order,
                        int64_t count, const void* norms, unsigned flags, void* stream);

/*
 * One epoch of the SDCA solver on kernel input (replaces one pass of the
 * example loop of solver::solve, solver.h:44-47, with the kernel form of
 * update_variables, update.h:88-107): per example i in `order`, norm2 =
 * K_ii (no update when it is <= 0), scores A k_i over the current dual
 * variables of all examples (eval_scores, solver/eval/scores.h:28-45), and the
 * objective's dual update of a_i.  Every update reaches the later
 * examples' scores (there is no primal matrix and no epsilon test).  The
 * examples run in blocks whose scores come from the matrix cores and whose
 * Gram matrix is read from K; results equal the sequential loop's up to
 * the rounding of the scores' sums.
 *   K: the n x n training kernel matrix (symmetric; column i = k_i);
 *   A: m x n dual variables, column-major, updated in place;
 *   labels, offsets, order, count, flags, stream, (data, result) and the
 *   limits on m and the SDCA_ERR_LABELS return: as sdca_epoch_features.
 */
int sdca_epoch_kernel(const sdca_objective* obj, sdca_dtype data, sdca_dtype result,
                      int64_t m, int64_t n, const void* K, void* A,
                      const int64_t* labels, const int64_t* offsets, const int64_t* order,
                      int64_t count, unsigned flags, void* stream);

/*
 * The reference solver's example order for epoch `epoch` (0-based) of a
 * solve over n examples (solver.h:59, 75-79, 96-100: a default-seeded
 * std::minstd_rand, std::shuffle of 0..n-1 once per epoch): n indices into
 * the host array `order`.  Host only.
 */
int sdca_epoch_order(int64_t n, int64_t epoch, int64_t* order);

/*
 * W = W0 + X A' (W = X A' when W0 is NULL) on the matrix cores: the primal
 * recomputation of eval_recompute_primal (eval/core.h:148-182), which the
 * reference runs before each evaluation when built with SDCA_ACCURATE_MATH.
 *   X: d x n features, A: m x n dual variables, W0, W: d x m, column-major.
 */
int sdca_recompute_primal(sdca_dtype data, int64_t d, int64_t m, int64_t n,
                          const void* X, const void* A, const void* W0, void* W,
                          unsigned flags, void* stream);

/* scores = W' X on the matrix cores (eval/scores.h:21-26 for all i at once). */
int sdca_scores(sdca_dtype data, int64_t d, int64_t m, int64_t n,
                const void* X, const void* W, void* S,
                unsigned flags, void* stream);

/* Message of the last failure on this thread ("" if none). */
const char* sdca_last_error(void);

/* ABI version (SDCA_HIP_ABI_VERSION). */
int sdca_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* SDCA_HIP_H */
