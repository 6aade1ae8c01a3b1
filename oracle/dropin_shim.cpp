// The C++ drop-in (include/sdca_hip.hpp) exercised next to the reference it
// replaces (TEST INFRASTRUCTURE ONLY).  Compiled with -I/root/reference/include
// by oracle/Makefile (target `dropin`) into oracle/_ref/, never committed.
// Each entry point builds the reference's own objects (solver_context,
// dataset, objective; solver/context.h, solver/data.h, solver/objective.h),
// runs the reference call on one copy of the data and the sdca::hip call of
// the same name and arguments on another, and returns both results, so that
// a GPU test can compare the drop-in with the reference through ctypes.
#include <cstdint>
#include <cstring>
#include <vector>

#include "sdca/prox.h"
#include "sdca/solver.h"

#include "../include/sdca_hip.hpp"

namespace {

template <class Ev>
void put_train(const Ev& e, double* rec) {
  rec[0] = static_cast<double>(e.primal);
  rec[1] = static_cast<double>(e.dual);
  rec[2] = static_cast<double>(e.primal_loss);
  rec[3] = static_cast<double>(e.dual_loss);
  rec[4] = static_cast<double>(e.primal_regularizer);
  rec[5] = static_cast<double>(e.dual_regularizer);
}
template <class R>
void put(const sdca::eval_train<R, sdca::multiclass_output>& e, double* rec, double* acc) {
  put_train(e, rec);
  rec[6] = 0;
  for (size_t j = 0; j < e.accuracy.size(); ++j) acc[j] = static_cast<double>(e.accuracy[j]);
}
template <class R>
void put(const sdca::eval_train<R, sdca::multilabel_output>& e, double* rec, double*) {
  put_train(e, rec);
  rec[6] = static_cast<double>(e.rank_loss);
}
template <class R>
void put(const sdca::eval_test<R, sdca::multiclass_output>& e, double* rec, double* acc) {
  for (int i = 0; i < 7; ++i) rec[i] = 0;
  rec[2] = static_cast<double>(e.primal_loss);
  for (size_t j = 0; j < e.accuracy.size(); ++j) acc[j] = static_cast<double>(e.accuracy[j]);
}
template <class R>
void put(const sdca::eval_test<R, sdca::multilabel_output>& e, double* rec, double*) {
  for (int i = 0; i < 7; ++i) rec[i] = 0;
  rec[2] = static_cast<double>(e.primal_loss);
  rec[6] = static_cast<double>(e.rank_loss);
}

sdca::multiclass_output output(std::false_type, int64_t m, const int64_t* labels,
                               const int64_t*, int64_t n) {
  std::vector<sdca::size_type> lab(labels, labels + n);
  return sdca::multiclass_output(static_cast<sdca::size_type>(m), lab);
}
sdca::multilabel_output output(std::true_type, int64_t m, const int64_t* labels,
                               const int64_t* offsets, int64_t n) {
  std::vector<sdca::size_type> lab(labels, labels + offsets[n]);
  std::vector<sdca::size_type> off(offsets, offsets + n + 1);
  return sdca::multilabel_output(static_cast<sdca::size_type>(m), lab, off);
}

// One objective over a feature input: the reference's evaluate_dataset
// (solver/eval.h:15-51) on ctx_ref, sdca::hip::evaluate_dataset on ctx_gpu;
// the training set, then the same examples as a test set of each context.
template <class Out, template <class, class> class Obj>
int run_features(const Obj<float, double>& obj, int64_t d, int64_t m, int64_t n,
                 const float* X, const float* W, const float* W0, const float* A,
                 const int64_t* labels, const int64_t* offsets, double* rec_gpu,
                 double* acc_gpu, double* rec_ref, double* acc_ref) {
  typedef std::integral_constant<bool, std::is_same<Out, sdca::multilabel_output>::value> ML;
  std::vector<float> Wr(W, W + d * m), Wg(W, W + d * m);
  std::vector<float> Ar(A, A + m * n), Ag(A, A + m * n);
  typedef sdca::solver_context<float, double, sdca::feature_input, Out, Obj> Ctx;
  Ctx ctx_ref(sdca::make_dataset_train<double>(
                  sdca::make_input_feature(static_cast<sdca::size_type>(d),
                                           static_cast<sdca::size_type>(n), X),
                  output(ML(), m, labels, offsets, n)),
              Obj<float, double>(obj), Ar.data(), Wr.data(), W0);
  Ctx ctx_gpu(sdca::make_dataset_train<double>(
                  sdca::make_input_feature(static_cast<sdca::size_type>(d),
                                           static_cast<sdca::size_type>(n), X),
                  output(ML(), m, labels, offsets, n)),
              Obj<float, double>(obj), Ag.data(), Wg.data(), W0);
  for (Ctx* c : {&ctx_ref, &ctx_gpu}) {
    c->test.push_back(sdca::make_dataset_test<double>(
        sdca::make_input_feature(static_cast<sdca::size_type>(d),
                                 static_cast<sdca::size_type>(n), X),
        output(ML(), m, labels, offsets, n)));
  }
  sdca::solver_scratch<float, sdca::feature_input> scratch;
  scratch.scores.resize(static_cast<size_t>(m));
  sdca::evaluate_dataset(ctx_ref, ctx_ref.train, scratch);
  sdca::evaluate_dataset(ctx_ref, ctx_ref.test[0], scratch, 1);
  try {
    sdca::hip::evaluate_dataset(ctx_gpu, ctx_gpu.train, scratch);
    sdca::hip::evaluate_dataset(ctx_gpu, ctx_gpu.test[0], scratch, 1);
  } catch (const sdca::hip::error& e) {
    return e.status();
  }
  if (ctx_gpu.train.evals.size() != 1 || ctx_gpu.test[0].evals.size() != 1) return -1;
  put(ctx_ref.train.evals.back(), rec_ref, acc_ref);
  put(ctx_gpu.train.evals.back(), rec_gpu, acc_gpu);
  put(ctx_ref.test[0].evals.back(), rec_ref + 7, acc_ref + m);
  put(ctx_gpu.test[0].evals.back(), rec_gpu + 7, acc_gpu + m);
  return 0;
}

// One epoch over `order` with one objective: the reference's own loop of
// update_variables (solver.h:43-47, solver/update.h:52-85) on ctx_ref,
// sdca::hip::update_epoch on ctx_gpu, both from the given W and A.
template <class Out, template <class, class> class Obj>
int run_epoch(const Obj<float, double>& obj, int64_t d, int64_t m, int64_t n, const float* X,
              const int64_t* labels, const int64_t* offsets, const int64_t* order,
              int64_t count, float* W_gpu, float* A_gpu, float* W_ref, float* A_ref) {
  typedef std::integral_constant<bool, std::is_same<Out, sdca::multilabel_output>::value> ML;
  typedef sdca::solver_context<float, double, sdca::feature_input, Out, Obj> Ctx;
  auto make = [&](float* A, float* W) {
    return Ctx(sdca::make_dataset_train<double>(
                   sdca::make_input_feature(static_cast<sdca::size_type>(d),
                                            static_cast<sdca::size_type>(n), X),
                   output(ML(), m, labels, offsets, n)),
               Obj<float, double>(obj), A, W, nullptr);
  };
  Ctx ctx_ref = make(A_ref, W_ref);
  Ctx ctx_gpu = make(A_gpu, W_gpu);
  sdca::solver_scratch<float, sdca::feature_input> scratch;
  scratch.init(ctx_ref.train);
  std::vector<sdca::size_type> examples(order, order + count);
  for (auto i : examples) sdca::update_variables(i, ctx_ref, scratch);
  try {
    sdca::hip::update_epoch(ctx_gpu, scratch, examples.begin(), examples.end());
  } catch (const sdca::hip::error& e) {
    return e.status();
  }
  return 0;
}

// The same on kernel input (solver/update.h:88-107): K n x n, A updated.
template <class Out, template <class, class> class Obj>
int run_epoch_kernel(const Obj<float, double>& obj, int64_t m, int64_t n, const float* K,
                     const int64_t* labels, const int64_t* offsets, const int64_t* order,
                     int64_t count, float* A_gpu, float* A_ref) {
  typedef std::integral_constant<bool, std::is_same<Out, sdca::multilabel_output>::value> ML;
  typedef sdca::solver_context<float, double, sdca::kernel_input, Out, Obj> Ctx;
  auto make = [&](float* A) {
    typename Ctx::train_set_type set(
        sdca::kernel_input<float>(static_cast<sdca::size_type>(n),
                                  static_cast<sdca::size_type>(n), K),
        output(ML(), m, labels, offsets, n));
    return Ctx(std::move(set), Obj<float, double>(obj), A);
  };
  Ctx ctx_ref = make(A_ref);
  Ctx ctx_gpu = make(A_gpu);
  sdca::solver_scratch<float, sdca::kernel_input> scratch;
  scratch.init(ctx_ref.train);
  std::vector<sdca::size_type> examples(order, order + count);
  for (auto i : examples) sdca::update_variables(i, ctx_ref, scratch);
  try {
    sdca::hip::update_epoch(ctx_gpu, scratch, examples.begin(), examples.end());
  } catch (const sdca::hip::error& e) {
    return e.status();
  }
  return 0;
}

}  // namespace

extern "C" {

// dropin_update_epoch on kernel input: K (n x n) in place of X, no W.
int dropin_update_epoch_kernel(int kind, double c, double gamma, int64_t k, int64_t m, int64_t n,
                               const float* K, const int64_t* labels, const int64_t* offsets,
                               const int64_t* order, int64_t count, float* A_gpu, float* A_ref) {
  typedef sdca::multiclass_output MC;
  typedef sdca::multilabel_output ML;
  const sdca::size_type kk = static_cast<sdca::size_type>(k);
  switch (kind) {
    case SDCA_OBJ_MULTILABEL_HINGE:
      return run_epoch_kernel<ML>(sdca::l2_multilabel_hinge<float, double>(c), m, n, K, labels,
                                  offsets, order, count, A_gpu, A_ref);
    case SDCA_OBJ_MULTILABEL_HINGE_SMOOTH:
      return run_epoch_kernel<ML>(sdca::l2_multilabel_hinge_smooth<float, double>(c, gamma), m,
                                  n, K, labels, offsets, order, count, A_gpu, A_ref);
    case SDCA_OBJ_MULTILABEL_ENTROPY:
      return run_epoch_kernel<ML>(sdca::l2_multilabel_entropy<float, double>(c), m, n, K, labels,
                                  offsets, order, count, A_gpu, A_ref);
    case SDCA_OBJ_HINGE_TOPK:
      return run_epoch_kernel<MC>(sdca::l2_hinge_topk<float, double>(c, kk), m, n, K, labels,
                                  nullptr, order, count, A_gpu, A_ref);
    case SDCA_OBJ_HINGE_TOPK_SMOOTH:
      return run_epoch_kernel<MC>(sdca::l2_hinge_topk_smooth<float, double>(c, gamma, kk), m, n,
                                  K, labels, nullptr, order, count, A_gpu, A_ref);
    case SDCA_OBJ_TOPK_HINGE:
      return run_epoch_kernel<MC>(sdca::l2_topk_hinge<float, double>(c, kk), m, n, K, labels,
                                  nullptr, order, count, A_gpu, A_ref);
    case SDCA_OBJ_TOPK_HINGE_SMOOTH:
      return run_epoch_kernel<MC>(sdca::l2_topk_hinge_smooth<float, double>(c, gamma, kk), m, n,
                                  K, labels, nullptr, order, count, A_gpu, A_ref);
    case SDCA_OBJ_ENTROPY:
      return run_epoch_kernel<MC>(sdca::l2_entropy<float, double>(c), m, n, K, labels, nullptr,
                                  order, count, A_gpu, A_ref);
    case SDCA_OBJ_ENTROPY_TOPK:
      return run_epoch_kernel<MC>(sdca::l2_entropy_topk<float, double>(c, kk), m, n, K, labels,
                                  nullptr, order, count, A_gpu, A_ref);
    default:
      return -2;
  }
}

// kind: an sdca_objective_kind (multilabel ones with offsets, n + 1 CSR row
// starts).  W_* (m x d) and A_* (n x m) hold the starting point and receive
// each side's result.  Returns 0, or the
// drop-in's error status.
int dropin_update_epoch(int kind, double c, double gamma, int64_t k, int64_t d, int64_t m,
                        int64_t n, const float* X, const int64_t* labels,
                        const int64_t* offsets, const int64_t* order, int64_t count,
                        float* W_gpu, float* A_gpu, float* W_ref, float* A_ref) {
  typedef sdca::multiclass_output MC;
  typedef sdca::multilabel_output ML;
  const sdca::size_type kk = static_cast<sdca::size_type>(k);
  switch (kind) {
    case SDCA_OBJ_MULTILABEL_HINGE:
      return run_epoch<ML>(sdca::l2_multilabel_hinge<float, double>(c), d, m, n, X, labels,
                           offsets, order, count, W_gpu, A_gpu, W_ref, A_ref);
    case SDCA_OBJ_MULTILABEL_HINGE_SMOOTH:
      return run_epoch<ML>(sdca::l2_multilabel_hinge_smooth<float, double>(c, gamma), d, m, n, X,
                           labels, offsets, order, count, W_gpu, A_gpu, W_ref, A_ref);
    case SDCA_OBJ_MULTILABEL_ENTROPY:
      return run_epoch<ML>(sdca::l2_multilabel_entropy<float, double>(c), d, m, n, X, labels,
                           offsets, order, count, W_gpu, A_gpu, W_ref, A_ref);
    case SDCA_OBJ_HINGE_TOPK:
      return run_epoch<MC>(sdca::l2_hinge_topk<float, double>(c, kk), d, m, n, X,
                           labels, nullptr, order, count, W_gpu, A_gpu, W_ref, A_ref);
    case SDCA_OBJ_HINGE_TOPK_SMOOTH:
      return run_epoch<MC>(sdca::l2_hinge_topk_smooth<float, double>(c, gamma, kk), d, m, n, X,
                           labels, nullptr, order, count, W_gpu, A_gpu, W_ref, A_ref);
    case SDCA_OBJ_TOPK_HINGE:
      return run_epoch<MC>(sdca::l2_topk_hinge<float, double>(c, kk), d, m, n, X,
                           labels, nullptr, order, count, W_gpu, A_gpu, W_ref, A_ref);
    case SDCA_OBJ_TOPK_HINGE_SMOOTH:
      return run_epoch<MC>(sdca::l2_topk_hinge_smooth<float, double>(c, gamma, kk), d, m, n, X,
                           labels, nullptr, order, count, W_gpu, A_gpu, W_ref, A_ref);
    case SDCA_OBJ_ENTROPY:
      return run_epoch<MC>(sdca::l2_entropy<float, double>(c), d, m, n, X,
                           labels, nullptr, order, count, W_gpu, A_gpu, W_ref, A_ref);
    case SDCA_OBJ_ENTROPY_TOPK:
      return run_epoch<MC>(sdca::l2_entropy_topk<float, double>(c, kk), d, m, n, X,
                           labels, nullptr, order, count, W_gpu, A_gpu, W_ref, A_ref);
    default:
      return -2;
  }
}


// kind: sdca_objective_kind; multilabel when offsets != NULL.  rec_*: 14
// doubles (training record, then test record: primal, dual, primal_loss,
// dual_loss, primal_regularizer, dual_regularizer, rank_loss); acc_*: 2 m
// (training then test accuracy, multiclass).  A must be m x n (zeros for a
// cold start); W0 may be NULL.  Returns 0, or the drop-in's error status.
int dropin_evaluate_features(int kind, double c, double gamma, int64_t k, int64_t d, int64_t m,
                             int64_t n, const float* X, const float* W, const float* W0,
                             const float* A, const int64_t* labels, const int64_t* offsets,
                             double* rec_gpu, double* acc_gpu, double* rec_ref,
                             double* acc_ref) {
  typedef sdca::multiclass_output MC;
  typedef sdca::multilabel_output ML;
  const sdca::size_type kk = static_cast<sdca::size_type>(k);
  switch (kind) {
    case SDCA_OBJ_HINGE_TOPK:
      return run_features<MC>(sdca::l2_hinge_topk<float, double>(c, kk), d, m, n, X, W, W0, A,
                              labels, offsets, rec_gpu, acc_gpu, rec_ref, acc_ref);
    case SDCA_OBJ_HINGE_TOPK_SMOOTH:
      return run_features<MC>(sdca::l2_hinge_topk_smooth<float, double>(c, gamma, kk), d, m, n,
                              X, W, W0, A, labels, offsets, rec_gpu, acc_gpu, rec_ref, acc_ref);
    case SDCA_OBJ_TOPK_HINGE:
      return run_features<MC>(sdca::l2_topk_hinge<float, double>(c, kk), d, m, n, X, W, W0, A,
                              labels, offsets, rec_gpu, acc_gpu, rec_ref, acc_ref);
    case SDCA_OBJ_TOPK_HINGE_SMOOTH:
      return run_features<MC>(sdca::l2_topk_hinge_smooth<float, double>(c, gamma, kk), d, m, n,
                              X, W, W0, A, labels, offsets, rec_gpu, acc_gpu, rec_ref, acc_ref);
    case SDCA_OBJ_ENTROPY:
      return run_features<MC>(sdca::l2_entropy<float, double>(c), d, m, n, X, W, W0, A, labels,
                              offsets, rec_gpu, acc_gpu, rec_ref, acc_ref);
    case SDCA_OBJ_ENTROPY_TOPK:
      return run_features<MC>(sdca::l2_entropy_topk<float, double>(c, kk), d, m, n, X, W, W0, A,
                              labels, offsets, rec_gpu, acc_gpu, rec_ref, acc_ref);
    case SDCA_OBJ_MULTILABEL_HINGE:
      return run_features<ML>(sdca::l2_multilabel_hinge<float, double>(c), d, m, n, X, W, W0, A,
                              labels, offsets, rec_gpu, acc_gpu, rec_ref, acc_ref);
    case SDCA_OBJ_MULTILABEL_HINGE_SMOOTH:
      return run_features<ML>(sdca::l2_multilabel_hinge_smooth<float, double>(c, gamma), d, m, n,
                              X, W, W0, A, labels, offsets, rec_gpu, acc_gpu, rec_ref, acc_ref);
    case SDCA_OBJ_MULTILABEL_ENTROPY:
      return run_features<ML>(sdca::l2_multilabel_entropy<float, double>(c), d, m, n, X, W, W0,
                              A, labels, offsets, rec_gpu, acc_gpu, rec_ref, acc_ref);
    default:
      return -2;
  }
}

// A batched prox through sdca::hip next to the reference's own batched call
// (the same name in namespace sdca): x_gpu and x_ref are two copies of the
// m x n input, projected in place.  op: 0 knapsack_eq (double, lo 0, hi 1,
// rhs 1), 1 topk_simplex (float, k, rhs 1), 2 entropy_norm (double),
// 3 two_simplex (float, split p, rhs 1), 4 topk_cone (float, k, Result
// double by default).
int dropin_prox(int op, int64_t m, int64_t n, int64_t k, void* x_gpu, void* x_ref) {
  try {
    switch (op) {
      case 0: {
        double* g = static_cast<double*>(x_gpu);
        double* r = static_cast<double*>(x_ref);
        std::vector<double> aux(static_cast<size_t>(m));
        sdca::prox_knapsack_eq(m, r, r + m * n, aux.data(), 0.0, 1.0, 1.0);
        sdca::hip::prox_knapsack_eq(m, g, g + m * n, aux.data(), 0.0, 1.0, 1.0);
        return 0;
      }
      case 1: {
        float* g = static_cast<float*>(x_gpu);
        float* r = static_cast<float*>(x_ref);
        std::vector<float> aux(static_cast<size_t>(m));
        sdca::prox_topk_simplex(m, r, r + m * n, aux.data(), k, 1.0f);
        sdca::hip::prox_topk_simplex(m, g, g + m * n, aux.data(), k, 1.0f);
        return 0;
      }
      case 2: {
        double* g = static_cast<double*>(x_gpu);
        double* r = static_cast<double*>(x_ref);
        std::vector<double> aux(static_cast<size_t>(m));
        sdca::prox_entropy_norm(m, r, r + m * n, aux.data(), 1.0, 1.0);
        sdca::hip::prox_entropy_norm(m, g, g + m * n, aux.data(), 1.0, 1.0);
        return 0;
      }
      case 3: {
        float* g = static_cast<float*>(x_gpu);
        float* r = static_cast<float*>(x_ref);
        std::vector<float> aux(static_cast<size_t>(m));
        sdca::prox_two_simplex(m, k, r, r + m * n, aux.data(), 1.0f);
        sdca::hip::prox_two_simplex(m, k, g, g + m * n, aux.data(), 1.0f);
        return 0;
      }
      case 4: {
        float* g = static_cast<float*>(x_gpu);
        float* r = static_cast<float*>(x_ref);
        std::vector<float> aux(static_cast<size_t>(m));
        sdca::prox_topk_cone(m, r, r + m * n, aux.data(), k);
        sdca::hip::prox_topk_cone(m, g, g + m * n, aux.data(), k);
        return 0;
      }
      default:
        return -2;
    }
  } catch (const sdca::hip::error& e) {
    return e.status();
  }
}

}  // extern "C"
