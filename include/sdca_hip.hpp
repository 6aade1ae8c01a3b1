// sdca_hip.hpp - C++11 drop-in overloads for libsdca's batched prox calls and
// the feature-input evaluation pass, running on the MI355X through the C ABI
// of sdca_hip.h.
//
// The names, template parameters, argument order and defaults are those of
// the reference's batched (`dim`) overloads, so a caller switches by
// replacing `sdca::` with `sdca::hip::`:
//
//   sdca::prox_topk_simplex(m, A, A + m * n, aux, k, rhs);        // reference
//   sdca::hip::prox_topk_simplex(m, A, A + m * n, aux, k, rhs);   // MI355X
//
// As in the reference, Result is deduced from the floating parameter (lo,
// hi, rhs) or defaults to double where there is none (prox_topk_cone,
// prox_topk_entropy).  Iterators must be float* or double* to contiguous
// host memory; the batch is staged through device memory and updated in
// place.  `aux` (the reference's m-element scratch) is accepted and unused.
// For device-resident data call the C ABI (sdca_prox) directly.  Errors throw
// sdca::hip::error (the reference asserts instead).
#ifndef SDCA_HIP_HPP
#define SDCA_HIP_HPP

#include <cstddef>
#include <cstdint>
#include <iterator>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <vector>

#include "sdca_hip.h"

namespace sdca {
namespace hip {

class error : public std::runtime_error {
 public:
  error(int status, const std::string& what) : std::runtime_error(what), status_(status) {}
  int status() const { return status_; }

 private:
  int status_;
};

namespace detail {

template <typename T> struct dtype;
template <> struct dtype<float> { static const sdca_dtype value = SDCA_F32; };
template <> struct dtype<double> { static const sdca_dtype value = SDCA_F64; };
template <> struct dtype<long double> { static const sdca_dtype value = SDCA_LONG_DOUBLE; };

inline void check(int rc) {
  if (rc != SDCA_OK) throw error(rc, sdca_last_error());
}

template <typename Result, typename Data>
inline void run(sdca_prox_op op, std::ptrdiff_t dim, Data* first, Data* last,
                const sdca_prox_params& p, const int64_t* col_p = nullptr) {
  static_assert(std::is_same<Data, float>::value || std::is_same<Data, double>::value,
                "sdca::hip works on float* or double* ranges");
  if (dim <= 0) throw error(SDCA_ERR_ARG_RANGE, "dim must be positive");
  const std::ptrdiff_t total = last - first;
  if (total % dim != 0) throw error(SDCA_ERR_ARG_RANGE, "range is not a whole number of columns");
  check(sdca_prox(op, dtype<Data>::value, dtype<Result>::value, dim, total / dim, first, first,
                  &p, col_p, nullptr, SDCA_HOST_PTR, nullptr));
}

inline sdca_prox_params params() {
  sdca_prox_params p;
  sdca_prox_params_default(&p);
  return p;
}

}  // namespace detail

// knapsack_eq.h:143-157
template <typename Result = double, typename Data>
inline void prox_knapsack_eq(std::ptrdiff_t dim, Data* first, Data* last, Data* /*aux*/,
                             const Result lo = 0, const Result hi = 1, const Result rhs = 1) {
  sdca_prox_params p = detail::params();
  p.lo = static_cast<double>(lo);
  p.hi = static_cast<double>(hi);
  p.rhs = static_cast<double>(rhs);
  detail::run<Result>(SDCA_PROX_KNAPSACK_EQ, dim, first, last, p);
}

// knapsack_le.h:78-92
template <typename Result = double, typename Data>
inline void prox_knapsack_le(std::ptrdiff_t dim, Data* first, Data* last, Data* /*aux*/,
                             const Result lo = 0, const Result hi = 1, const Result rhs = 1) {
  sdca_prox_params p = detail::params();
  p.lo = static_cast<double>(lo);
  p.hi = static_cast<double>(hi);
  p.rhs = static_cast<double>(rhs);
  detail::run<Result>(SDCA_PROX_KNAPSACK_LE, dim, first, last, p);
}

// topk_simplex.h:100-113
template <typename Result = double, typename Data>
inline void prox_topk_simplex(std::ptrdiff_t dim, Data* first, Data* last, Data* /*aux*/,
                              const std::ptrdiff_t k = 1, const Result rhs = 1) {
  sdca_prox_params p = detail::params();
  p.k = k;
  p.rhs = static_cast<double>(rhs);
  detail::run<Result>(SDCA_PROX_TOPK_SIMPLEX, dim, first, last, p);
}

// topk_cone.h:187-199 (Result is not deducible: double by default)
template <typename Result = double, typename Data>
inline void prox_topk_cone(std::ptrdiff_t dim, Data* first, Data* last, Data* /*aux*/,
                           const std::ptrdiff_t k = 1) {
  sdca_prox_params p = detail::params();
  p.k = k;
  detail::run<Result>(SDCA_PROX_TOPK_CONE, dim, first, last, p);
}

// entropy.h:85-98
template <typename Result = double, typename Data>
inline void prox_entropy(std::ptrdiff_t dim, Data* first, Data* last, Data* /*aux*/,
                         const Result hi = 1, const Result rhs = 1) {
  sdca_prox_params p = detail::params();
  p.hi = static_cast<double>(hi);
  p.rhs = static_cast<double>(rhs);
  detail::run<Result>(SDCA_PROX_ENTROPY, dim, first, last, p);
}

// entropy_norm.h:213-226
template <typename Result = double, typename Data>
inline void prox_entropy_norm(std::ptrdiff_t dim, Data* first, Data* last, Data* /*aux*/,
                              const Result hi = 1, const Result rhs = 1) {
  sdca_prox_params p = detail::params();
  p.hi = static_cast<double>(hi);
  p.rhs = static_cast<double>(rhs);
  detail::run<Result>(SDCA_PROX_ENTROPY_NORM, dim, first, last, p);
}

// topk_entropy.h:106-118 (Result is not deducible: double by default)
template <typename Result = double, typename Data>
inline void prox_topk_entropy(std::ptrdiff_t dim, Data* first, Data* last, Data* /*aux*/,
                              const std::ptrdiff_t k = 1) {
  sdca_prox_params p = detail::params();
  p.k = k;
  detail::run<Result>(SDCA_PROX_TOPK_ENTROPY, dim, first, last, p);
}

// two_simplex.h:183-196
template <typename Result = double, typename Data>
inline void prox_two_simplex(std::ptrdiff_t dim, std::ptrdiff_t p_split, Data* first, Data* last,
                             Data* /*aux*/, const Result rhs = 1) {
  sdca_prox_params p = detail::params();
  p.p = p_split;
  p.rhs = static_cast<double>(rhs);
  detail::run<Result>(SDCA_PROX_TWO_SIMPLEX, dim, first, last, p);
}

// knapsack_le_biased.h:165-180
template <typename Result = double, typename Data>
inline void prox_knapsack_le_biased(std::ptrdiff_t dim, Data* first, Data* last, Data* /*aux*/,
                                    const Result lo = 0, const Result hi = 1,
                                    const Result rhs = 1, const Result rho = 1) {
  sdca_prox_params p = detail::params();
  p.lo = static_cast<double>(lo);
  p.hi = static_cast<double>(hi);
  p.rhs = static_cast<double>(rhs);
  p.rho = static_cast<double>(rho);
  detail::run<Result>(SDCA_PROX_KNAPSACK_LE_BIASED, dim, first, last, p);
}

// topk_simplex_biased.h:105-119
template <typename Result = double, typename Data>
inline void prox_topk_simplex_biased(std::ptrdiff_t dim, Data* first, Data* last, Data* /*aux*/,
                                     const std::ptrdiff_t k = 1, const Result rhs = 1,
                                     const Result rho = 1) {
  sdca_prox_params p = detail::params();
  p.k = k;
  p.rhs = static_cast<double>(rhs);
  p.rho = static_cast<double>(rho);
  detail::run<Result>(SDCA_PROX_TOPK_SIMPLEX_BIASED, dim, first, last, p);
}

// topk_cone_biased.h:145-158
template <typename Result = double, typename Data>
inline void prox_topk_cone_biased(std::ptrdiff_t dim, Data* first, Data* last, Data* /*aux*/,
                                  const std::ptrdiff_t k = 1, const Result rho = 1) {
  sdca_prox_params p = detail::params();
  p.k = k;
  p.rho = static_cast<double>(rho);
  detail::run<Result>(SDCA_PROX_TOPK_CONE_BIASED, dim, first, last, p);
}

// topk_entropy_biased.h:302-315 (Result is deduced from alpha, as in the
// reference)
template <typename Result = double, typename Data>
inline void prox_topk_entropy_biased(std::ptrdiff_t dim, Data* first, Data* last,
                                     Data* /*aux*/, const std::ptrdiff_t k = 1,
                                     const Result alpha = 1) {
  sdca_prox_params p = detail::params();
  p.k = k;
  p.alpha = static_cast<double>(alpha);
  detail::run<Result>(SDCA_PROX_TOPK_ENTROPY_BIASED, dim, first, last, p);
}

// two_simplex_sort.h:175-190
template <typename Result = double, typename Data>
inline void prox_two_simplex_sort(std::ptrdiff_t dim, std::ptrdiff_t p_split, Data* first,
                                  Data* last, Data* /*aux*/, const Result rhs = 1) {
  sdca_prox_params p = detail::params();
  p.p = p_split;
  p.rhs = static_cast<double>(rhs);
  detail::run<Result>(SDCA_PROX_TWO_SIMPLEX_SORT, dim, first, last, p);
}

// prox_two_entropy(p, first, last, aux, alpha) (two_entropy.h:280-292) over
// the dim-sized columns of [first, last); the reference has the per-column
// form only, this is its batch in the argument order of prox_two_simplex.
template <typename Result = double, typename Data>
inline void prox_two_entropy(std::ptrdiff_t dim, std::ptrdiff_t p_split, Data* first, Data* last,
                             Data* /*aux*/, const Result alpha = 1) {
  sdca_prox_params p = detail::params();
  p.p = p_split;
  p.alpha = static_cast<double>(alpha);
  detail::run<Result>(SDCA_PROX_TWO_ENTROPY, dim, first, last, p);
}

// apply(dim, first, last, lambert_w_exp_map<Data>()) (proxdef.h:386-400)
template <typename Data>
inline void apply_lambert_w_exp(std::ptrdiff_t dim, Data* first, Data* last) {
  detail::run<Data>(SDCA_PROX_LAMBERT_W_EXP, dim, first, last, detail::params());
}

// One evaluation record (eval/types.h:12-20, 84-125) without the timing fields.
struct eval_record {
  double primal, dual, primal_loss, dual_loss, primal_regularizer, dual_regularizer;
  double rank_loss;            // multilabel
  std::vector<double> accuracy;  // multiclass: top-(i+1) accuracy after partial_sum / n
};

namespace detail {
inline std::vector<eval_record> records(const std::vector<sdca_eval_record>& recs,
                                        const std::vector<double>& acc, bool multiclass) {
  std::vector<eval_record> out(recs.size());
  for (size_t i = 0; i < recs.size(); ++i) {
    out[i].primal = recs[i].primal;
    out[i].dual = recs[i].dual;
    out[i].primal_loss = recs[i].primal_loss;
    out[i].dual_loss = recs[i].dual_loss;
    out[i].primal_regularizer = recs[i].primal_regularizer;
    out[i].dual_regularizer = recs[i].dual_regularizer;
    out[i].rank_loss = recs[i].rank_loss;
    if (multiclass) out[i].accuracy = acc;
  }
  return out;
}
}  // namespace detail

// evaluate_dataset (eval.h:15-51) for feature_input: X is d x n and W is
// d x m, column-major (num_dimensions fastest), labels 0-based; offsets is
// empty for multiclass and holds the n + 1 CSR offsets for multilabel.
// A (m x n dual variables) and W0 (prox mode) may be null.  test = true
// evaluates a test set (eval_test: primal loss and accuracy / rank loss).
template <typename Data, typename Result = double>
inline std::vector<eval_record> evaluate_features(
    const std::vector<sdca_objective>& objectives, std::int64_t d, std::int64_t m,
    std::int64_t n, const Data* X, const Data* W, const std::vector<std::int64_t>& labels,
    const std::vector<std::int64_t>& offsets = std::vector<std::int64_t>(),
    const Data* A = nullptr, const Data* W0 = nullptr, bool test = false) {
  std::vector<sdca_eval_record> recs(objectives.size());
  std::vector<double> acc(static_cast<size_t>(m), 0.0);
  detail::check(sdca_eval_features(
      objectives.data(), static_cast<int>(objectives.size()), detail::dtype<Data>::value,
      detail::dtype<Result>::value, d, m, n, X, W, A, W0, labels.data(),
      offsets.empty() ? nullptr : offsets.data(), recs.data(),
      offsets.empty() ? acc.data() : nullptr, nullptr,
      SDCA_HOST_PTR | (test ? SDCA_EVAL_TEST : 0u), nullptr));
  return detail::records(recs, acc, offsets.empty());
}

// evaluate_dataset for kernel_input (data/input.h:44-76): K is n_train x n
// and A (the dual variables) m x n_train, column-major; scores_i = A K_i
// (eval/scores.h:30-47).  A training set has n == n_train.
template <typename Data, typename Result = double>
inline std::vector<eval_record> evaluate_kernel(
    const std::vector<sdca_objective>& objectives, std::int64_t n_train, std::int64_t m,
    std::int64_t n, const Data* K, const Data* A, const std::vector<std::int64_t>& labels,
    const std::vector<std::int64_t>& offsets = std::vector<std::int64_t>(), bool test = false) {
  std::vector<sdca_eval_record> recs(objectives.size());
  std::vector<double> acc(static_cast<size_t>(m), 0.0);
  detail::check(sdca_eval_kernel(
      objectives.data(), static_cast<int>(objectives.size()), detail::dtype<Data>::value,
      detail::dtype<Result>::value, n_train, m, n, K, A, labels.data(),
      offsets.empty() ? nullptr : offsets.data(), recs.data(),
      offsets.empty() ? acc.data() : nullptr, nullptr,
      SDCA_HOST_PTR | (test ? SDCA_EVAL_TEST : 0u), nullptr));
  return detail::records(recs, acc, offsets.empty());
}

// ---------------------------------------------------------------------------
// evaluate_dataset with the reference's own signature (solver/eval.h:15-51):
// the same template parameters and arguments, reading the reference's
// solver_context (ctx.primal_variables, ctx.dual_variables,
// ctx.primal_initial, ctx.objective; context.h:32-37) and dataset (d.in,
// d.out, d.evals), and appending the record eval_end would (eval/core.h:43-132).
// The reference's types are only declared here: this header is included
// next to the reference's solver headers, which define them.
// ---------------------------------------------------------------------------
}  // namespace hip

template <typename Data> struct feature_input;
template <typename Data> struct kernel_input;
struct multiclass_output;
struct multilabel_output;
template <typename Result, typename Output> struct eval_train;
template <typename Result, typename Output> struct eval_test;
template <typename Data, template <typename> class Input> struct solver_scratch;
template <typename Data, typename Result> struct l2_hinge_topk;
template <typename Data, typename Result> struct l2_hinge_topk_smooth;
template <typename Data, typename Result> struct l2_topk_hinge;
template <typename Data, typename Result> struct l2_topk_hinge_smooth;
template <typename Data, typename Result> struct l2_entropy;
template <typename Data, typename Result> struct l2_entropy_topk;
template <typename Data, typename Result> struct l2_multilabel_hinge;
template <typename Data, typename Result> struct l2_multilabel_hinge_smooth;
template <typename Data, typename Result> struct l2_multilabel_entropy;

namespace hip {
namespace detail {

inline sdca_objective make_objective(int kind, double c, double gamma, std::size_t k) {
  sdca_objective o;
  o.kind = kind;
  o.reserved = 0;
  o.c = c;
  o.gamma = gamma;
  o.k = static_cast<std::int64_t>(k);
  return o;
}

// The C ABI's description of each reference objective (its public c,
// gamma, k members; objective/*.h).
template <typename Objective> struct objective_of {
  static_assert(sizeof(Objective) == 0,
                "sdca::hip::evaluate_dataset: objective not on the GPU evaluation path");
};
template <typename D, typename R> struct objective_of<sdca::l2_hinge_topk<D, R>> {
  template <typename O> static sdca_objective get(const O& o) {
    return make_objective(SDCA_OBJ_HINGE_TOPK, static_cast<double>(o.c), 1.0, o.k);
  }
};
template <typename D, typename R> struct objective_of<sdca::l2_hinge_topk_smooth<D, R>> {
  template <typename O> static sdca_objective get(const O& o) {
    return make_objective(SDCA_OBJ_HINGE_TOPK_SMOOTH, static_cast<double>(o.c),
                          static_cast<double>(o.gamma), o.k);
  }
};
template <typename D, typename R> struct objective_of<sdca::l2_topk_hinge<D, R>> {
  template <typename O> static sdca_objective get(const O& o) {
    return make_objective(SDCA_OBJ_TOPK_HINGE, static_cast<double>(o.c), 1.0, o.k);
  }
};
template <typename D, typename R> struct objective_of<sdca::l2_topk_hinge_smooth<D, R>> {
  template <typename O> static sdca_objective get(const O& o) {
    return make_objective(SDCA_OBJ_TOPK_HINGE_SMOOTH, static_cast<double>(o.c),
                          static_cast<double>(o.gamma), o.k);
  }
};
template <typename D, typename R> struct objective_of<sdca::l2_entropy<D, R>> {
  template <typename O> static sdca_objective get(const O& o) {
    return make_objective(SDCA_OBJ_ENTROPY, static_cast<double>(o.c), 1.0, 1);
  }
};
template <typename D, typename R> struct objective_of<sdca::l2_entropy_topk<D, R>> {
  template <typename O> static sdca_objective get(const O& o) {
    return make_objective(SDCA_OBJ_ENTROPY_TOPK, static_cast<double>(o.c), 1.0, o.k);
  }
};
template <typename D, typename R> struct objective_of<sdca::l2_multilabel_hinge<D, R>> {
  template <typename O> static sdca_objective get(const O& o) {
    return make_objective(SDCA_OBJ_MULTILABEL_HINGE, static_cast<double>(o.c), 1.0, 1);
  }
};
template <typename D, typename R> struct objective_of<sdca::l2_multilabel_hinge_smooth<D, R>> {
  template <typename O> static sdca_objective get(const O& o) {
    return make_objective(SDCA_OBJ_MULTILABEL_HINGE_SMOOTH, static_cast<double>(o.c),
                          static_cast<double>(o.gamma), 1);
  }
};
template <typename D, typename R> struct objective_of<sdca::l2_multilabel_entropy<D, R>> {
  template <typename O> static sdca_objective get(const O& o) {
    return make_objective(SDCA_OBJ_MULTILABEL_ENTROPY, static_cast<double>(o.c), 1.0, 1);
  }
};

// Labels of the reference's outputs (data/output.h:15-166) as int64 arrays.
template <typename Output>
inline void labels_of(const Output& out, std::vector<std::int64_t>& labels,
                      std::vector<std::int64_t>& offsets, std::true_type /*multilabel*/) {
  labels.assign(out.labels.begin(), out.labels.end());
  offsets.assign(out.offsets.begin(), out.offsets.end());
}
template <typename Output>
inline void labels_of(const Output& out, std::vector<std::int64_t>& labels,
                      std::vector<std::int64_t>& offsets, std::false_type) {
  labels.assign(out.labels.begin(), out.labels.end());
  offsets.clear();
}

// The C ABI call for a feature input (scores W' x_i) or a kernel input
// (scores A K_i).
template <typename Data, typename Context>
inline int eval_call(const sdca::feature_input<Data>& in, const Context& ctx,
                     const sdca_objective& ob, sdca_dtype result, std::int64_t m,
                     std::int64_t n, const std::vector<std::int64_t>& labels,
                     const std::vector<std::int64_t>& offsets, sdca_eval_record* rec,
                     double* acc, bool test) {
  return sdca_eval_features(&ob, 1, dtype<Data>::value, result,
                            static_cast<std::int64_t>(in.num_dimensions), m, n, in.features,
                            ctx.primal_variables, test ? nullptr : ctx.dual_variables,
                            test ? nullptr : ctx.primal_initial, labels.data(),
                            offsets.empty() ? nullptr : offsets.data(), rec, acc, nullptr,
                            SDCA_HOST_PTR | (test ? SDCA_EVAL_TEST : 0u), nullptr);
}
template <typename Data, typename Context>
inline int eval_call(const sdca::kernel_input<Data>& in, const Context& ctx,
                     const sdca_objective& ob, sdca_dtype result, std::int64_t m,
                     std::int64_t n, const std::vector<std::int64_t>& labels,
                     const std::vector<std::int64_t>& offsets, sdca_eval_record* rec,
                     double* acc, bool test) {
  return sdca_eval_kernel(&ob, 1, dtype<Data>::value, result,
                          static_cast<std::int64_t>(in.num_train_examples), m, n, in.kernel,
                          ctx.dual_variables, labels.data(),
                          offsets.empty() ? nullptr : offsets.data(), rec, acc, nullptr,
                          SDCA_HOST_PTR | (test ? SDCA_EVAL_TEST : 0u), nullptr);
}

// The fields eval_end sets on a training record (eval/core.h:43-95):
// epoch and timings from the context, then the objective's terms.
template <typename Eval, typename Context>
inline void fill_train(Eval& e, const Context& ctx, const sdca_eval_record& r) {
  typedef typename Context::result_type Result;
  e.epoch = ctx.epoch;
  e.solve_time_cpu = ctx.solve_time.cpu.elapsed_now();
  e.solve_time_wall = ctx.solve_time.wall.elapsed_now();
  e.eval_time_cpu = ctx.eval_time.cpu.elapsed_now();
  e.eval_time_wall = ctx.eval_time.wall.elapsed_now();
  e.primal = static_cast<Result>(r.primal);
  e.dual = static_cast<Result>(r.dual);
  e.primal_loss = static_cast<Result>(r.primal_loss);
  e.dual_loss = static_cast<Result>(r.dual_loss);
  e.primal_regularizer = static_cast<Result>(r.primal_regularizer);
  e.dual_regularizer = static_cast<Result>(r.dual_regularizer);
}

// Filling the appended record as eval_end does (eval/core.h:43-132).
template <typename Result, typename Context>
inline void fill(sdca::eval_train<Result, sdca::multiclass_output>& e, const Context& ctx,
                 const sdca_eval_record& r, const std::vector<double>& acc) {
  fill_train(e, ctx, r);
  e.accuracy.assign(acc.begin(), acc.end());
}
template <typename Result, typename Context>
inline void fill(sdca::eval_train<Result, sdca::multilabel_output>& e, const Context& ctx,
                 const sdca_eval_record& r, const std::vector<double>&) {
  fill_train(e, ctx, r);
  e.rank_loss = static_cast<Result>(r.rank_loss);
}
template <typename Result, typename Context>
inline void fill(sdca::eval_test<Result, sdca::multiclass_output>& e, const Context&,
                 const sdca_eval_record& r, const std::vector<double>& acc) {
  e.primal_loss = static_cast<Result>(r.primal_loss);
  e.accuracy.assign(acc.begin(), acc.end());
}
template <typename Result, typename Context>
inline void fill(sdca::eval_test<Result, sdca::multilabel_output>& e, const Context&,
                 const sdca_eval_record& r, const std::vector<double>&) {
  e.primal_loss = static_cast<Result>(r.primal_loss);
  e.rank_loss = static_cast<Result>(r.rank_loss);
}
template <typename Eval> struct is_test : std::false_type {};
template <typename R, typename O> struct is_test<sdca::eval_test<R, O>> : std::true_type {};

}  // namespace detail

// evaluate_dataset (solver/eval.h:15-51) on the GPU: feature or kernel
// input, multiclass or multilabel output, training set (eval_train) or test
// set (eval_test), with the objective of ctx.  Host arrays are staged
// through device memory.  The reference's logging of the record
// (reporting::eval_created) and its SDCA_ACCURATE_MATH primal
// recomputation are not done here (recompute_primal does the latter).
template <typename Data, template <typename> class Input, typename Dataset, typename Context>
inline void evaluate_dataset(const Context& ctx, Dataset& d,
                             sdca::solver_scratch<Data, Input>& /*scratch*/,
                             std::size_t /*id*/ = 0) {
  typedef typename Context::result_type Result;
  typedef typename Dataset::eval_type Eval;
  typedef typename Dataset::output_type Output;
  const bool test = detail::is_test<Eval>::value;
  const std::int64_t m = static_cast<std::int64_t>(d.num_classes());
  const std::int64_t n = static_cast<std::int64_t>(d.num_examples());
  std::vector<std::int64_t> labels, offsets;
  detail::labels_of(d.out, labels, offsets,
                    std::integral_constant<bool, std::is_same<Output, sdca::multilabel_output>::value>());
  const sdca_objective ob = detail::objective_of<typename Context::objective_type>::get(ctx.objective);
  sdca_eval_record rec;
  std::vector<double> acc(static_cast<std::size_t>(m), 0.0);
  detail::check(detail::eval_call(d.in, ctx, ob, detail::dtype<Result>::value, m, n, labels,
                                  offsets, &rec, offsets.empty() ? acc.data() : nullptr, test));
  d.evals.resize(d.evals.size() + 1);
  detail::fill(d.evals.back(), ctx, rec, acc);
}

// One epoch of solve()'s example loop (solver.h:43-47) on the GPU:
// update_variables (solver/update.h:52-85) for each example index in
// [first, last) - the solver's examples_ after begin_epoch's shuffle - for a
// feature input with multiclass or multilabel output and its objective.
// ctx.primal_variables and ctx.dual_variables are updated in place, through
// host staging per call; scratch.norms (scratch.h:27-41) are used when
// filled.  The maintainer's switch in solve():
//   begin_epoch();
//   sdca::hip::update_epoch(ctx_, scratch_, examples_.begin(), examples_.end());
//   end_epoch();
template <typename Data, typename Context, typename Iterator>
inline void update_epoch(Context& ctx, sdca::solver_scratch<Data, sdca::feature_input>& scratch,
                         Iterator first, Iterator last) {
  typedef typename Context::result_type Result;
  const auto& d = ctx.train;
  const std::int64_t m = static_cast<std::int64_t>(d.num_classes());
  const std::int64_t n = static_cast<std::int64_t>(d.num_examples());
  const std::int64_t dim = static_cast<std::int64_t>(d.in.num_dimensions);
  typedef typename Context::output_type Output;
  std::vector<std::int64_t> labels, offsets;
  detail::labels_of(d.out, labels, offsets,
                    std::integral_constant<bool, std::is_same<Output, sdca::multilabel_output>::value>());
  std::vector<std::int64_t> order;
  for (Iterator it = first; it != last; ++it) order.push_back(static_cast<std::int64_t>(*it));
  const sdca_objective ob = detail::objective_of<typename Context::objective_type>::get(ctx.objective);
  const Data* norms = scratch.norms.size() == static_cast<std::size_t>(n) ? scratch.norms.data()
                                                                         : nullptr;
  detail::check(sdca_epoch_features(&ob, detail::dtype<Data>::value, detail::dtype<Result>::value,
                                    dim, m, n, d.in.features, ctx.primal_variables,
                                    ctx.dual_variables, labels.data(),
                                    offsets.empty() ? nullptr : offsets.data(), order.data(),
                                    static_cast<std::int64_t>(order.size()), norms,
                                    SDCA_HOST_PTR, nullptr));
}

// The same epoch for a kernel input: update_variables' kernel form
// (solver/update.h:88-107) for each example index in [first, last);
// ctx.dual_variables is updated in place.
template <typename Data, typename Context, typename Iterator>
inline void update_epoch(Context& ctx, sdca::solver_scratch<Data, sdca::kernel_input>&,
                         Iterator first, Iterator last) {
  typedef typename Context::result_type Result;
  const auto& d = ctx.train;
  const std::int64_t m = static_cast<std::int64_t>(d.num_classes());
  const std::int64_t n = static_cast<std::int64_t>(d.num_examples());
  typedef typename Context::output_type Output;
  std::vector<std::int64_t> labels, offsets;
  detail::labels_of(d.out, labels, offsets,
                    std::integral_constant<bool, std::is_same<Output, sdca::multilabel_output>::value>());
  std::vector<std::int64_t> order;
  for (Iterator it = first; it != last; ++it) order.push_back(static_cast<std::int64_t>(*it));
  const sdca_objective ob = detail::objective_of<typename Context::objective_type>::get(ctx.objective);
  detail::check(sdca_epoch_kernel(&ob, detail::dtype<Data>::value, detail::dtype<Result>::value, m,
                                  n, d.in.kernel, ctx.dual_variables, labels.data(),
                                  offsets.empty() ? nullptr : offsets.data(), order.data(),
                                  static_cast<std::int64_t>(order.size()), SDCA_HOST_PTR,
                                  nullptr));
}

// W = W0 + X A' (eval_recompute_primal, eval/core.h:148-182): X is d x n,
// A m x n, W0 (may be null) and W d x m, column-major.
template <typename Data>
inline void recompute_primal(std::int64_t d, std::int64_t m, std::int64_t n, const Data* X,
                             const Data* A, const Data* W0, Data* W) {
  detail::check(sdca_recompute_primal(detail::dtype<Data>::value, d, m, n, X, A, W0, W,
                                      SDCA_HOST_PTR, nullptr));
}

}  // namespace hip
}  // namespace sdca

#endif  // SDCA_HIP_HPP
