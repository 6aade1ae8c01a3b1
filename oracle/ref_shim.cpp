// C entry points over the reference headers themselves (TEST INFRASTRUCTURE
// ONLY).  This file is our own wrapper; it is compiled with
// -I/root/reference/include by oracle/Makefile into oracle/_ref/, which is
// never committed.  It exists to pin the oracle restatement and to time the
// reference CPU path for the bench's cpu_baseline.
//
// The BLAS-backed parts of the evaluation (the scores gemv, the regularizer
// dot products and the smooth objectives' dual losses, math/blas.h:191-319)
// go through the reference's own CBLAS prototypes (include/cblas.h, selected
// by -DBLAS_DEFAULT_LOCAL_HEADER, blas.h:15-16) to Intel MKL's single dynamic
// library (libmkl_rt, LP64: blas_int = int as blas.h:29-30 expects), the
// reference's first-choice BLAS (cmake/SelectBLAS.cmake:34-89).  MKL runs
// with its sequential threading layer: the reference's evaluation is
// single-threaded, and the harness-parallel timing splits examples over
// std::threads instead.
#include <cmath>
#include <cstdint>
#include <limits>
#include <thread>
#include <vector>

#include "sdca/prox.h"
#include "sdca/solver/context.h"
#include "sdca/solver.h"
#include "sdca/solver/eval.h"
#include "sdca/solver/eval/dual.h"
#include "sdca/solver/eval/primal.h"
#include "sdca/solver/eval/types.h"
#include "sdca/solver/objective/l2_entropy.h"
#include "sdca/solver/objective/l2_entropy_topk.h"
#include "sdca/solver/objective/l2_hinge_topk.h"
#include "sdca/solver/objective/l2_multilabel_entropy.h"
#include "sdca/solver/objective/l2_multilabel_hinge.h"
#include "sdca/solver/objective/l2_topk_hinge.h"

#include "../include/sdca_hip.h"

namespace {

template <class F>
void parallel_for(int64_t n, int nthreads, F f) {
  if (nthreads <= 1 || n < 2 * nthreads) {
    f(static_cast<int64_t>(0), n);
    return;
  }
  std::vector<std::thread> pool;
  int64_t chunk = (n + nthreads - 1) / nthreads;
  for (int w = 0; w < nthreads; ++w) {
    int64_t b = w * chunk, e = std::min(n, b + chunk);
    if (b >= e) break;
    pool.emplace_back(f, b, e);
  }
  for (auto& t : pool) t.join();
}

template <class T>
void put(sdca_thresholds* out, int64_t j, const T& th) {
  out[j].t = static_cast<double>(th.t);
  out[j].lo = static_cast<double>(th.lo);
  out[j].hi = static_cast<double>(th.hi);
}

// The record's sets as the reference leaves them (proxdef.h:29-67): first
// and last over the block's scratch copy starting at `begin`.  The branch is
// not part of the reference's record (-1).
template <class T, class D>
void put_sets(sdca_prox_sets* out, int64_t j, const T& th, const D* begin) {
  if (!out) return;
  out[j].n_hi = static_cast<int64_t>(th.first - begin);
  out[j].n_mid = static_cast<int64_t>(th.last - th.first);
  out[j].branch = -1;
  out[j].reserved = 0;
}

// The reference's own batched entry points (the Matlab dispatch,
// src/matlab/mex_prox.cpp:145-172), on columns [b, e).
template <class D, class R>
void batched(int op, int64_t m, D* first, D* last, D* aux, const sdca_prox_params* p,
             const int64_t* col_p) {
  const R lo = static_cast<R>(p->lo), hi = static_cast<R>(p->hi), rhs = static_cast<R>(p->rhs);
  const R rho = static_cast<R>(p->rho);
  const std::ptrdiff_t k = static_cast<std::ptrdiff_t>(p->k);
  switch (op) {
    case SDCA_PROX_KNAPSACK_EQ: sdca::prox_knapsack_eq(m, first, last, aux, lo, hi, rhs); break;
    case SDCA_PROX_KNAPSACK_LE: sdca::prox_knapsack_le(m, first, last, aux, lo, hi, rhs); break;
    case SDCA_PROX_TOPK_SIMPLEX: sdca::prox_topk_simplex(m, first, last, aux, k, rhs); break;
    case SDCA_PROX_TOPK_CONE: sdca::prox_topk_cone<R>(m, first, last, aux, k); break;
    case SDCA_PROX_ENTROPY: sdca::prox_entropy(m, first, last, aux, hi, rhs); break;
    case SDCA_PROX_ENTROPY_NORM: sdca::prox_entropy_norm(m, first, last, aux, hi, rhs); break;
    case SDCA_PROX_TOPK_ENTROPY: sdca::prox_topk_entropy<R>(m, first, last, aux, k); break;
    case SDCA_PROX_TWO_SIMPLEX:
      if (!col_p) {
        sdca::prox_two_simplex(m, static_cast<std::ptrdiff_t>(p->p), first, last, aux, rhs);
      } else {
        // Per-column split: one batch call per column.
        for (int64_t j = 0; first + j * m < last; ++j)
          sdca::prox_two_simplex(m, static_cast<std::ptrdiff_t>(col_p[j]), first + j * m,
                                 first + (j + 1) * m, aux, rhs);
      }
      break;
    case SDCA_PROX_LAMBERT_W_EXP: sdca::apply(m, first, last, sdca::lambert_w_exp_map<D>()); break;
    case SDCA_PROX_KNAPSACK_LE_BIASED:
      sdca::prox_knapsack_le_biased(m, first, last, aux, lo, hi, rhs, rho); break;
    case SDCA_PROX_TOPK_SIMPLEX_BIASED:
      sdca::prox_topk_simplex_biased(m, first, last, aux, k, rhs, rho); break;
    case SDCA_PROX_TOPK_CONE_BIASED: sdca::prox_topk_cone_biased(m, first, last, aux, k, rho); break;
    case SDCA_PROX_TOPK_ENTROPY_BIASED:
      sdca::prox_topk_entropy_biased(m, first, last, aux, k, static_cast<R>(p->alpha)); break;
    case SDCA_PROX_TWO_ENTROPY:
      // The reference has the per-column form only (two_entropy.h:280-292).
      for (int64_t j = 0; first + j * m < last; ++j)
        sdca::prox_two_entropy(col_p ? static_cast<std::ptrdiff_t>(col_p[j])
                                     : static_cast<std::ptrdiff_t>(p->p),
                               first + j * m, first + (j + 1) * m, aux,
                               static_cast<R>(p->alpha));
      break;
    case SDCA_PROX_TWO_SIMPLEX_SORT:
      if (!col_p) {
        sdca::prox_two_simplex_sort(m, static_cast<std::ptrdiff_t>(p->p), first, last, aux, rhs);
      } else {
        for (int64_t j = 0; first + j * m < last; ++j)
          sdca::prox_two_simplex_sort(m, static_cast<std::ptrdiff_t>(col_p[j]), first + j * m,
                                      first + (j + 1) * m, aux, rhs);
      }
      break;
    default: break;
  }
}

// Per-column loop with the threshold records (same steps as proxdef.h:279-298).
template <class D, class R>
void with_thresholds(int op, int64_t m, int64_t b, int64_t e, D* x, D* aux,
                     const sdca_prox_params* p, const int64_t* col_p, sdca_thresholds* out,
                     sdca_prox_sets* sets) {
  const R lo = static_cast<R>(p->lo), hi = static_cast<R>(p->hi), rhs = static_cast<R>(p->rhs);
  const R rho = static_cast<R>(p->rho);
  const std::ptrdiff_t k = static_cast<std::ptrdiff_t>(p->k);
  for (int64_t j = b; j < e; ++j) {
    D* col = x + j * m;
    std::copy(col, col + m, aux);
    D* al = aux + m;
    switch (op) {
      case SDCA_PROX_KNAPSACK_EQ: {
        auto t = sdca::thresholds_knapsack_eq(aux, al, lo, hi, rhs);
        sdca::prox(t, col, col + m); put(out, j, t); put_sets(sets, j, t, aux); break;
      }
      case SDCA_PROX_KNAPSACK_LE: {
        auto t = sdca::thresholds_knapsack_le(aux, al, lo, hi, rhs);
        sdca::prox(t, col, col + m); put(out, j, t); put_sets(sets, j, t, aux); break;
      }
      case SDCA_PROX_TOPK_SIMPLEX: {
        auto t = sdca::thresholds_topk_simplex(aux, al, k, rhs);
        sdca::prox(t, col, col + m); put(out, j, t); put_sets(sets, j, t, aux); break;
      }
      case SDCA_PROX_TOPK_CONE: {
        auto t = sdca::thresholds_topk_cone<R>(aux, al, k);
        sdca::prox(t, col, col + m); put(out, j, t); put_sets(sets, j, t, aux); break;
      }
      case SDCA_PROX_ENTROPY: {
        auto t = sdca::thresholds_entropy(aux, al, hi, rhs);
        sdca::prox(t, col, col + m); put(out, j, t); put_sets(sets, j, t, aux); break;
      }
      case SDCA_PROX_ENTROPY_NORM: {
        auto t = sdca::thresholds_entropy_norm(aux, al, hi, rhs);
        sdca::prox(t, col, col + m); put(out, j, t); put_sets(sets, j, t, aux); break;
      }
      case SDCA_PROX_TOPK_ENTROPY: {
        auto t = sdca::thresholds_topk_entropy<R>(aux, al, k);
        sdca::prox(t, col, col + m); put(out, j, t); put_sets(sets, j, t, aux); break;
      }
      case SDCA_PROX_TWO_SIMPLEX: {
        std::ptrdiff_t pj = col_p ? static_cast<std::ptrdiff_t>(col_p[j])
                                  : static_cast<std::ptrdiff_t>(p->p);
        auto t = sdca::thresholds_two_simplex(aux, aux + pj, aux + pj, al, rhs);
        sdca::prox(t.first, col, col + pj);
        sdca::prox(t.second, col + pj, col + m);
        put(out, 2 * j, t.first);
        put(out, 2 * j + 1, t.second);
        put_sets(sets, 2 * j, t.first, aux);
        put_sets(sets, 2 * j + 1, t.second, aux + pj);
        break;
      }
      case SDCA_PROX_TOPK_ENTROPY_BIASED: {
        auto t = sdca::thresholds_topk_entropy_biased(aux, al, k, static_cast<R>(p->alpha));
        sdca::prox(t, col, col + m); put(out, j, t); put_sets(sets, j, t, aux); break;
      }
      case SDCA_PROX_TWO_ENTROPY: {
        std::ptrdiff_t pj = col_p ? static_cast<std::ptrdiff_t>(col_p[j])
                                  : static_cast<std::ptrdiff_t>(p->p);
        auto t = sdca::thresholds_two_entropy(aux, aux + pj, aux + pj, al,
                                              static_cast<R>(p->alpha));
        sdca::prox(t.first, col, col + pj);
        sdca::prox(t.second, col + pj, col + m);
        put(out, 2 * j, t.first);
        put(out, 2 * j + 1, t.second);
        put_sets(sets, 2 * j, t.first, aux);
        put_sets(sets, 2 * j + 1, t.second, aux + pj);
        break;
      }
      case SDCA_PROX_TWO_SIMPLEX_SORT: {
        std::ptrdiff_t pj = col_p ? static_cast<std::ptrdiff_t>(col_p[j])
                                  : static_cast<std::ptrdiff_t>(p->p);
        auto t = sdca::thresholds_two_simplex_sort(aux, aux + pj, aux + pj, al, rhs);
        sdca::prox(t.first, col, col + pj);
        sdca::prox(t.second, col + pj, col + m);
        put(out, 2 * j, t.first);
        put(out, 2 * j + 1, t.second);
        put_sets(sets, 2 * j, t.first, aux);
        put_sets(sets, 2 * j + 1, t.second, aux + pj);
        break;
      }
      case SDCA_PROX_KNAPSACK_LE_BIASED: {
        auto t = sdca::thresholds_knapsack_le_biased(aux, al, lo, hi, rhs, rho);
        sdca::prox(t, col, col + m); put(out, j, t); put_sets(sets, j, t, aux); break;
      }
      case SDCA_PROX_TOPK_SIMPLEX_BIASED: {
        auto t = sdca::thresholds_topk_simplex_biased(aux, al, k, rhs, rho);
        sdca::prox(t, col, col + m); put(out, j, t); put_sets(sets, j, t, aux); break;
      }
      case SDCA_PROX_TOPK_CONE_BIASED: {
        auto t = sdca::thresholds_topk_cone_biased(aux, al, k, rho);
        sdca::prox(t, col, col + m); put(out, j, t); put_sets(sets, j, t, aux); break;
      }
      default: break;
    }
  }
}

template <class D, class R>
int prox_impl(int op, int64_t m, int64_t n, D* x, const sdca_prox_params* p,
              const int64_t* col_p, sdca_thresholds* out, int nthreads,
              sdca_prox_sets* sets = nullptr) {
  if (op == SDCA_PROX_LAMBERT_W_EXP) {
    parallel_for(n, nthreads, [&](int64_t b, int64_t e) {
      batched<D, R>(op, m, x + b * m, x + e * m, nullptr, p, nullptr);
    });
    return 0;
  }
  parallel_for(n, nthreads, [&](int64_t b, int64_t e) {
    std::vector<D> aux(static_cast<size_t>(m));
    if (out) {
      with_thresholds<D, R>(op, m, b, e, x, aux.data(), p, col_p, out, sets);
    } else {
      batched<D, R>(op, m, x + b * m, x + e * m, aux.data(), p, col_p ? col_p + b : nullptr);
    }
  });
  return 0;
}

template <class R>
void init_record(sdca::eval_train<R, sdca::multiclass_output>& e, int64_t m) {
  e.accuracy.assign(static_cast<size_t>(m), 0);
}
template <class R>
void init_record(sdca::eval_train<R, sdca::multilabel_output>&, int64_t) {}
template <class R>
void merge_record(sdca::eval_train<R, sdca::multiclass_output>& e,
                  const sdca::eval_train<R, sdca::multiclass_output>& one) {
  for (size_t j = 0; j < e.accuracy.size(); ++j) e.accuracy[j] += one.accuracy[j];
}
template <class R>
void merge_record(sdca::eval_train<R, sdca::multilabel_output>& e,
                  const sdca::eval_train<R, sdca::multilabel_output>& one) {
  e.rank_loss += one.rank_loss;
}

// Per-example evaluation with the reference's eval_primal_loss /
// eval_dual_loss (eval/primal.h, eval/dual.h) for one objective.  When
// per-example values are requested, each example runs on a fresh record whose
// loss fields are then added to the running totals: the same single
// additions the reference makes, so the totals are unchanged.
template <class Obj, class Out, class Ev, bool HasDual>
void eval_loop(const Obj& obj, const Out& out, Ev& ev, int64_t m, int64_t n,
               const typename Obj::data_type* S, const typename Obj::data_type* A,
               int o, int no, double* per_example) {
  typedef typename Obj::data_type D;
  std::vector<D> s(static_cast<size_t>(m)), v(static_cast<size_t>(m));
  for (int64_t i = 0; i < n; ++i) {
    std::copy(S + i * m, S + (i + 1) * m, s.begin());
    if (A) std::copy(A + i * m, A + (i + 1) * m, v.begin());
    else std::fill(v.begin(), v.end(), static_cast<D>(0));
    const sdca::size_type ii = static_cast<sdca::size_type>(i);
    if (!per_example) {
      if (HasDual) sdca::eval_dual_loss(ii, out, obj, v.data(), ev);
      sdca::eval_primal_loss(ii, out, obj, s.data(), ev);
      continue;
    }
    Ev one;
    init_record(one, m);
    if (HasDual) sdca::eval_dual_loss(ii, out, obj, v.data(), one);
    sdca::eval_primal_loss(ii, out, obj, s.data(), one);
    per_example[(i * no + o) * 2] = static_cast<double>(one.primal_loss);
    per_example[(i * no + o) * 2 + 1] =
        HasDual ? static_cast<double>(one.dual_loss) : std::numeric_limits<double>::quiet_NaN();
    ev.primal_loss += one.primal_loss;
    ev.dual_loss += one.dual_loss;
    merge_record(ev, one);
  }
}

template <class Obj, class D, class R, bool HasDual>
void eval_one(std::false_type, const Obj& obj, int64_t m, int64_t n, const D* S,
              const D* A, const int64_t* labels, const int64_t*, int o, int no,
              sdca_eval_record* rec, std::vector<R>* hist, double* per_example) {
  std::vector<sdca::size_type> lab(labels, labels + n);
  sdca::multiclass_output out(static_cast<sdca::size_type>(m), lab);
  sdca::eval_train<R, sdca::multiclass_output> ev;
  init_record(ev, m);
  eval_loop<Obj, sdca::multiclass_output, decltype(ev), HasDual>(
      obj, out, ev, m, n, S, A, o, no, per_example);
  obj.update_primal_loss(ev.primal_loss);
  rec[o].primal_loss = static_cast<double>(ev.primal_loss);
  rec[o].dual_loss = HasDual ? static_cast<double>(ev.dual_loss)
                             : std::numeric_limits<double>::quiet_NaN();
  rec[o].rank_loss = 0;
  if (hist) *hist = ev.accuracy;
}

template <class Obj, class D, class R, bool HasDual>
void eval_one(std::true_type, const Obj& obj, int64_t m, int64_t n, const D* S,
              const D* A, const int64_t* labels, const int64_t* offsets, int o, int no,
              sdca_eval_record* rec, std::vector<R>*, double* per_example) {
  std::vector<sdca::size_type> lab(labels, labels + offsets[n]);
  std::vector<sdca::size_type> off(offsets, offsets + n + 1);
  sdca::multilabel_output out(static_cast<sdca::size_type>(m), lab, off);
  sdca::eval_train<R, sdca::multilabel_output> ev;
  eval_loop<Obj, sdca::multilabel_output, decltype(ev), HasDual>(
      obj, out, ev, m, n, S, A, o, no, per_example);
  obj.update_primal_loss(ev.primal_loss);
  rec[o].primal_loss = static_cast<double>(ev.primal_loss);
  rec[o].dual_loss = HasDual ? static_cast<double>(ev.dual_loss)
                             : std::numeric_limits<double>::quiet_NaN();
  rec[o].rank_loss = static_cast<double>(ev.rank_loss / static_cast<R>(n));
}

#define SDCA_REF_EVAL(ML, HASDUAL, OBJ)                                              \
  eval_one<decltype(OBJ), D, R, HASDUAL>(std::integral_constant<bool, ML>(), OBJ, m, n, \
                                         S, A, labels, offsets, o, n_obj, rec, h,     \
                                         per_example)

template <class D, class R>
int eval_impl(const sdca_objective* objs, int n_obj, int64_t m, int64_t n, const D* S,
              const D* A, const int64_t* labels, const int64_t* offsets, double preg,
              double dreg, sdca_eval_record* rec, double* accuracy, double* per_example) {
  std::vector<R> hist;
  for (int o = 0; o < n_obj; ++o) {
    const sdca_objective& ob = objs[o];
    const R c = static_cast<R>(ob.c), g = static_cast<R>(ob.gamma);
    const sdca::size_type k = static_cast<sdca::size_type>(ob.k);
    std::vector<R>* h = (o == 0 && accuracy && !offsets) ? &hist : nullptr;
    rec[o].rank_loss = 0;
    switch (ob.kind) {
      case SDCA_OBJ_HINGE_TOPK:
        SDCA_REF_EVAL(false, true, (sdca::l2_hinge_topk<D, R>(c, k))); break;
      case SDCA_OBJ_HINGE_TOPK_SMOOTH:
        SDCA_REF_EVAL(false, true, (sdca::l2_hinge_topk_smooth<D, R>(c, g, k))); break;
      case SDCA_OBJ_TOPK_HINGE:
        SDCA_REF_EVAL(false, true, (sdca::l2_topk_hinge<D, R>(c, k))); break;
      case SDCA_OBJ_TOPK_HINGE_SMOOTH:
        SDCA_REF_EVAL(false, true, (sdca::l2_topk_hinge_smooth<D, R>(c, g, k))); break;
      case SDCA_OBJ_ENTROPY:
        SDCA_REF_EVAL(false, true, (sdca::l2_entropy<D, R>(c))); break;
      case SDCA_OBJ_ENTROPY_TOPK:
        SDCA_REF_EVAL(false, true, (sdca::l2_entropy_topk<D, R>(c, k))); break;
      case SDCA_OBJ_MULTILABEL_HINGE:
        SDCA_REF_EVAL(true, true, (sdca::l2_multilabel_hinge<D, R>(c))); break;
      case SDCA_OBJ_MULTILABEL_HINGE_SMOOTH:
        SDCA_REF_EVAL(true, true, (sdca::l2_multilabel_hinge_smooth<D, R>(c, g))); break;
      case SDCA_OBJ_MULTILABEL_ENTROPY:
        SDCA_REF_EVAL(true, true, (sdca::l2_multilabel_entropy<D, R>(c))); break;
      default: return SDCA_ERR_ARG_RANGE;
    }
    // objective_base::update_all (objective_base.h:116-128)
    rec[o].primal_regularizer = preg;
    rec[o].dual_regularizer = dreg;
    rec[o].primal = static_cast<double>(static_cast<R>(rec[o].primal_loss) + static_cast<R>(preg));
    rec[o].dual = static_cast<double>(static_cast<R>(rec[o].dual_loss) - static_cast<R>(dreg));
  }
  if (accuracy && !offsets && !hist.empty()) {
    // eval_end: partial_sum and scaling by 1/n (eval/core.h:65-68)
    std::partial_sum(hist.begin(), hist.end(), hist.begin());
    R coeff(1 / static_cast<R>(n));
    for (int64_t j = 0; j < m; ++j) accuracy[j] = static_cast<double>(hist[j] * coeff);
  }
  return 0;
}


// MKL's threading layer is chosen before its first call: sequential, so that
// one reference evaluation runs on one core as the shipped solver does.
extern "C" int MKL_Set_Threading_Layer(int);
struct MklSequential {
  MklSequential() { MKL_Set_Threading_Layer(1 /* MKL_THREADING_SEQUENTIAL */); }
} g_mkl_sequential;

// One eval_train record of the reference, in double.
template <class Ev>
void record_out(const Ev& e, sdca_eval_record* r) {
  r->primal = static_cast<double>(e.primal);
  r->dual = static_cast<double>(e.dual);
  r->primal_loss = static_cast<double>(e.primal_loss);
  r->dual_loss = static_cast<double>(e.dual_loss);
  r->primal_regularizer = static_cast<double>(e.primal_regularizer);
  r->dual_regularizer = static_cast<double>(e.dual_regularizer);
}
template <class R>
double rank_of(const sdca::eval_train<R, sdca::multiclass_output>&) { return 0.0; }
template <class R>
double rank_of(const sdca::eval_train<R, sdca::multilabel_output>& e) {
  return static_cast<double>(e.rank_loss);
}
template <class R>
const std::vector<R>* accuracy_of(const sdca::eval_train<R, sdca::multiclass_output>& e) {
  return &e.accuracy;
}
template <class R>
const std::vector<R>* accuracy_of(const sdca::eval_train<R, sdca::multilabel_output>&) {
  return nullptr;
}

sdca::multiclass_output make_out(std::false_type, int64_t m, const int64_t* labels,
                                 const int64_t*, int64_t b, int64_t e) {
  std::vector<sdca::size_type> lab(labels + b, labels + e);
  return sdca::multiclass_output(static_cast<sdca::size_type>(m), lab);
}
sdca::multilabel_output make_out(std::true_type, int64_t m, const int64_t* labels,
                                 const int64_t* offsets, int64_t b, int64_t e) {
  std::vector<sdca::size_type> lab(labels + offsets[b], labels + offsets[e]);
  std::vector<sdca::size_type> off;
  for (int64_t i = b; i <= e; ++i)
    off.push_back(static_cast<sdca::size_type>(offsets[i] - offsets[b]));
  return sdca::multilabel_output(static_cast<sdca::size_type>(m), lab, off);
}

// The reference's whole evaluation pass, sdca::evaluate_dataset
// (solver/eval.h:15-51), over examples [b, e) of a feature input: a
// solver_context over that slice, with W as its primal variables (W0 as the
// initial ones, prox mode) and A as its dual variables.  The reference swaps
// entries of A and restores them (eval/dual.h:35-43): A is borrowed mutable.
template <class D, class R, class Out, template <class, class> class Obj>
void evaluate_slice(Obj<D, R> obj, int64_t d, int64_t m, int64_t b, int64_t e, const D* X,
                    D* W, const D* W0, D* A, const int64_t* labels, const int64_t* offsets,
                    sdca_eval_record* rec, std::vector<double>* acc) {
  typedef sdca::solver_context<D, R, sdca::feature_input, Out, Obj> Ctx;
  typename Ctx::train_set_type set(
      sdca::feature_input<D>(static_cast<sdca::size_type>(d),
                             static_cast<sdca::size_type>(e - b), X + d * b),
      make_out(std::integral_constant<bool, std::is_same<Out, sdca::multilabel_output>::value>(),
               m, labels, offsets, b, e));
  Ctx ctx(std::move(set), std::move(obj), A + m * b, W, W0);
  sdca::solver_scratch<D, sdca::feature_input> scratch;
  scratch.scores.resize(static_cast<size_t>(m));
  sdca::evaluate_dataset(ctx, ctx.train, scratch);
  const auto& ev = ctx.train.evals.back();
  record_out(ev, rec);
  rec->rank_loss = rank_of(ev);
  if (acc) {
    const auto* a = accuracy_of(ev);
    if (a) acc->assign(a->begin(), a->end());
  }
}

// evaluate_dataset on nthreads slices of the examples (harness-parallel:
// each thread runs the reference on its own slice; nthreads = 1 is the
// reference as shipped).  The slices' records are merged as one pass would
// have formed them: loss terms add, regularizers are those of the whole W,
// accuracies and rank losses are averaged with the slices' weights.
template <class D, class R, class Out, template <class, class> class Obj>
void evaluate_all(const Obj<D, R>& obj, int64_t d, int64_t m, int64_t n, const D* X, D* W,
                  const D* W0, D* A, const int64_t* labels, const int64_t* offsets,
                  sdca_eval_record* rec, double* accuracy, int nthreads) {
  if (nthreads < 1) nthreads = 1;
  if (n < 2 * nthreads) nthreads = 1;
  const int64_t chunk = (n + nthreads - 1) / nthreads;
  std::vector<sdca_eval_record> part(static_cast<size_t>(nthreads));
  std::vector<std::vector<double>> acc(static_cast<size_t>(nthreads));
  std::vector<int64_t> lo(static_cast<size_t>(nthreads)), hi(static_cast<size_t>(nthreads));
  std::vector<std::thread> pool;
  for (int w = 0; w < nthreads; ++w) {
    lo[w] = std::min(n, w * chunk);
    hi[w] = std::min(n, lo[w] + chunk);
    auto job = [&, w]() {
      if (lo[w] < hi[w])
        evaluate_slice<D, R, Out, Obj>(obj, d, m, lo[w], hi[w], X, W, W0, A, labels, offsets,
                                       &part[w], &acc[w]);
    };
    if (nthreads == 1) job();
    else pool.emplace_back(job);
  }
  for (auto& t : pool) t.join();
  if (nthreads == 1) {
    *rec = part[0];
    if (accuracy && !acc[0].empty())
      for (int64_t j = 0; j < m; ++j) accuracy[j] = acc[0][j];
    return;
  }
  sdca_eval_record r = part[0];
  r.primal_loss = r.dual_loss = r.rank_loss = 0;
  std::vector<double> a(static_cast<size_t>(m), 0.0);
  for (int w = 0; w < nthreads; ++w) {
    if (lo[w] >= hi[w]) continue;
    const double wt = static_cast<double>(hi[w] - lo[w]) / static_cast<double>(n);
    r.primal_loss += part[w].primal_loss;
    r.dual_loss += part[w].dual_loss;
    r.rank_loss += part[w].rank_loss * wt;
    for (size_t j = 0; j < acc[w].size(); ++j) a[j] += acc[w][j] * wt;
  }
  r.primal = r.primal_loss + r.primal_regularizer;
  r.dual = r.dual_loss - r.dual_regularizer;
  *rec = r;
  if (accuracy && !acc[0].empty())
    for (int64_t j = 0; j < m; ++j) accuracy[j] = a[j];
}

#define SDCA_REF_EVALUATE(OUT, OBJ)                                                         \
  evaluate_all<D, R, OUT>(OBJ, d, m, n, X, W, W0, A, labels, offsets, &rec[o],            \
                          o == 0 ? accuracy : nullptr, nthreads)

template <class D, class R>
int evaluate_impl(const sdca_objective* objs, int n_obj, int64_t d, int64_t m, int64_t n,
                  const D* X, D* W, const D* W0, D* A, const int64_t* labels,
                  const int64_t* offsets, sdca_eval_record* rec, double* accuracy,
                  int nthreads) {
  typedef sdca::multiclass_output MC;
  typedef sdca::multilabel_output ML;
  for (int o = 0; o < n_obj; ++o) {
    const sdca_objective& ob = objs[o];
    const R c = static_cast<R>(ob.c), g = static_cast<R>(ob.gamma);
    const sdca::size_type k = static_cast<sdca::size_type>(ob.k);
    switch (ob.kind) {
      case SDCA_OBJ_HINGE_TOPK: SDCA_REF_EVALUATE(MC, (sdca::l2_hinge_topk<D, R>(c, k))); break;
      case SDCA_OBJ_HINGE_TOPK_SMOOTH:
        SDCA_REF_EVALUATE(MC, (sdca::l2_hinge_topk_smooth<D, R>(c, g, k))); break;
      case SDCA_OBJ_TOPK_HINGE: SDCA_REF_EVALUATE(MC, (sdca::l2_topk_hinge<D, R>(c, k))); break;
      case SDCA_OBJ_TOPK_HINGE_SMOOTH:
        SDCA_REF_EVALUATE(MC, (sdca::l2_topk_hinge_smooth<D, R>(c, g, k))); break;
      case SDCA_OBJ_ENTROPY: SDCA_REF_EVALUATE(MC, (sdca::l2_entropy<D, R>(c))); break;
      case SDCA_OBJ_ENTROPY_TOPK: SDCA_REF_EVALUATE(MC, (sdca::l2_entropy_topk<D, R>(c, k))); break;
      case SDCA_OBJ_MULTILABEL_HINGE: SDCA_REF_EVALUATE(ML, (sdca::l2_multilabel_hinge<D, R>(c))); break;
      case SDCA_OBJ_MULTILABEL_HINGE_SMOOTH:
        SDCA_REF_EVALUATE(ML, (sdca::l2_multilabel_hinge_smooth<D, R>(c, g))); break;
      case SDCA_OBJ_MULTILABEL_ENTROPY:
        SDCA_REF_EVALUATE(ML, (sdca::l2_multilabel_entropy<D, R>(c))); break;
      default: return SDCA_ERR_ARG_RANGE;
    }
  }
  return 0;
}

// One epoch of the reference's example loop (solver.h:44-47) over `order`
// (NULL: 0..n-1): sdca::update_variables (update.h:52-85) on a
// solver_context over the whole training set, W and A updated in place.
// With epochs > 0 instead, the reference's own solve() runs that many epochs
// (its generator and std::shuffle give the order, solver.h:75-112) with no
// evaluation between epochs.
template <class Out, class D, class R, template <class, class> class Obj>
void epoch_run(Obj<D, R> obj, int64_t d, int64_t m, int64_t n, const D* X, D* W, D* A,
               const int64_t* labels, const int64_t* offsets, const int64_t* order,
               int64_t count, int64_t epochs) {
  typedef sdca::solver_context<D, R, sdca::feature_input, Out, Obj> Ctx;
  typename Ctx::train_set_type set(
      sdca::feature_input<D>(static_cast<sdca::size_type>(d), static_cast<sdca::size_type>(n), X),
      make_out(std::integral_constant<bool, std::is_same<Out, sdca::multilabel_output>::value>(),
               m, labels, offsets, 0, n));
  Ctx ctx(std::move(set), std::move(obj), A, W);
  if (epochs > 0) {
    sdca::logging::set_level(sdca::logging::level::none);
    ctx.criteria.max_epoch = static_cast<sdca::size_type>(epochs);
    ctx.criteria.eval_epoch = 0;
    ctx.criteria.eval_on_start = false;
    auto solver = sdca::make_solver(ctx);
    solver.solve();
    return;
  }
  sdca::solver_scratch<D, sdca::feature_input> scratch;
  scratch.init(ctx.train);
  for (int64_t q = 0; q < count; ++q)
    sdca::update_variables(static_cast<sdca::size_type>(order ? order[q] : q), ctx, scratch);
}

// The same on kernel input (update.h:88-107): K n x n column-major (column
// i = K_i), A m x n updated in place, no primal variables.
template <class Out, class D, class R, template <class, class> class Obj>
void epoch_kernel_run(Obj<D, R> obj, int64_t m, int64_t n, const D* K, D* A,
                      const int64_t* labels, const int64_t* offsets, const int64_t* order,
                      int64_t count, int64_t epochs) {
  typedef sdca::solver_context<D, R, sdca::kernel_input, Out, Obj> Ctx;
  typename Ctx::train_set_type set(
      sdca::kernel_input<D>(static_cast<sdca::size_type>(n), static_cast<sdca::size_type>(n), K),
      make_out(std::integral_constant<bool, std::is_same<Out, sdca::multilabel_output>::value>(),
               m, labels, offsets, 0, n));
  Ctx ctx(std::move(set), std::move(obj), A);
  if (epochs > 0) {
    sdca::logging::set_level(sdca::logging::level::none);
    ctx.criteria.max_epoch = static_cast<sdca::size_type>(epochs);
    ctx.criteria.eval_epoch = 0;
    ctx.criteria.eval_on_start = false;
    auto solver = sdca::make_solver(ctx);
    solver.solve();
    return;
  }
  sdca::solver_scratch<D, sdca::kernel_input> scratch;
  scratch.init(ctx.train);
  for (int64_t q = 0; q < count; ++q)
    sdca::update_variables(static_cast<sdca::size_type>(order ? order[q] : q), ctx, scratch);
}

#define SDCA_REF_EPOCH(OBJ)                                                               \
  epoch_run<sdca::multiclass_output, D, R>(OBJ, d, m, n, X, W, A, labels, nullptr, order,   \
                                           count, epochs)
#define SDCA_REF_EPOCH_ML(OBJ)                                                            \
  epoch_run<sdca::multilabel_output, D, R>(OBJ, d, m, n, X, W, A, labels, offsets, order,   \
                                           count, epochs)

#define SDCA_REF_EPOCH_K(OBJ)                                                             \
  epoch_kernel_run<sdca::multiclass_output, D, R>(OBJ, m, n, K, A, labels, nullptr, order, \
                                                  count, epochs)
#define SDCA_REF_EPOCH_K_ML(OBJ)                                                          \
  epoch_kernel_run<sdca::multilabel_output, D, R>(OBJ, m, n, K, A, labels, offsets, order, \
                                                  count, epochs)

template <class D, class R>
int epoch_kernel_impl(const sdca_objective& ob, int64_t m, int64_t n, const D* K, D* A,
                      const int64_t* labels, const int64_t* offsets, const int64_t* order,
                      int64_t count, int64_t epochs) {
  const R c = static_cast<R>(ob.c), g = static_cast<R>(ob.gamma);
  const sdca::size_type k = static_cast<sdca::size_type>(ob.k);
  switch (ob.kind) {
    case SDCA_OBJ_HINGE_TOPK: SDCA_REF_EPOCH_K((sdca::l2_hinge_topk<D, R>(c, k))); break;
    case SDCA_OBJ_HINGE_TOPK_SMOOTH: SDCA_REF_EPOCH_K((sdca::l2_hinge_topk_smooth<D, R>(c, g, k))); break;
    case SDCA_OBJ_TOPK_HINGE: SDCA_REF_EPOCH_K((sdca::l2_topk_hinge<D, R>(c, k))); break;
    case SDCA_OBJ_TOPK_HINGE_SMOOTH: SDCA_REF_EPOCH_K((sdca::l2_topk_hinge_smooth<D, R>(c, g, k))); break;
    case SDCA_OBJ_ENTROPY: SDCA_REF_EPOCH_K((sdca::l2_entropy<D, R>(c))); break;
    case SDCA_OBJ_ENTROPY_TOPK: SDCA_REF_EPOCH_K((sdca::l2_entropy_topk<D, R>(c, k))); break;
    case SDCA_OBJ_MULTILABEL_HINGE:
      SDCA_REF_EPOCH_K_ML((sdca::l2_multilabel_hinge<D, R>(c))); break;
    case SDCA_OBJ_MULTILABEL_HINGE_SMOOTH:
      SDCA_REF_EPOCH_K_ML((sdca::l2_multilabel_hinge_smooth<D, R>(c, g))); break;
    case SDCA_OBJ_MULTILABEL_ENTROPY:
      SDCA_REF_EPOCH_K_ML((sdca::l2_multilabel_entropy<D, R>(c))); break;
    default: return SDCA_ERR_ARG_RANGE;
  }
  return 0;
}

template <class D, class R>
int epoch_impl(const sdca_objective& ob, int64_t d, int64_t m, int64_t n, const D* X, D* W,
               D* A, const int64_t* labels, const int64_t* offsets, const int64_t* order,
               int64_t count, int64_t epochs) {
  const R c = static_cast<R>(ob.c), g = static_cast<R>(ob.gamma);
  const sdca::size_type k = static_cast<sdca::size_type>(ob.k);
  switch (ob.kind) {
    case SDCA_OBJ_HINGE_TOPK: SDCA_REF_EPOCH((sdca::l2_hinge_topk<D, R>(c, k))); break;
    case SDCA_OBJ_HINGE_TOPK_SMOOTH: SDCA_REF_EPOCH((sdca::l2_hinge_topk_smooth<D, R>(c, g, k))); break;
    case SDCA_OBJ_TOPK_HINGE: SDCA_REF_EPOCH((sdca::l2_topk_hinge<D, R>(c, k))); break;
    case SDCA_OBJ_TOPK_HINGE_SMOOTH: SDCA_REF_EPOCH((sdca::l2_topk_hinge_smooth<D, R>(c, g, k))); break;
    case SDCA_OBJ_ENTROPY: SDCA_REF_EPOCH((sdca::l2_entropy<D, R>(c))); break;
    case SDCA_OBJ_ENTROPY_TOPK: SDCA_REF_EPOCH((sdca::l2_entropy_topk<D, R>(c, k))); break;
    case SDCA_OBJ_MULTILABEL_HINGE:
      SDCA_REF_EPOCH_ML((sdca::l2_multilabel_hinge<D, R>(c))); break;
    case SDCA_OBJ_MULTILABEL_HINGE_SMOOTH:
      SDCA_REF_EPOCH_ML((sdca::l2_multilabel_hinge_smooth<D, R>(c, g))); break;
    case SDCA_OBJ_MULTILABEL_ENTROPY:
      SDCA_REF_EPOCH_ML((sdca::l2_multilabel_entropy<D, R>(c))); break;
    default: return SDCA_ERR_ARG_RANGE;
  }
  return 0;
}

}  // namespace

extern "C" {

// The reference's SDCA epoch on feature input (see epoch_run): X d x n,
// W d x m, A m x n, column-major (each example's / class's values
// contiguous), W and A updated in place; offsets (n + 1, CSR into labels)
// for the multilabel objectives, NULL for the multiclass ones.
int ref_epoch_features(const sdca_objective* obj, int data, int result, int64_t d, int64_t m,
                       int64_t n, const void* X, void* W, void* A, const int64_t* labels,
                       const int64_t* offsets, const int64_t* order, int64_t count,
                       int64_t epochs) {
  if (data == SDCA_F32 && result == SDCA_F32)
    return epoch_impl<float, float>(*obj, d, m, n, static_cast<const float*>(X),
        static_cast<float*>(W), static_cast<float*>(A), labels, offsets, order, count, epochs);
  if (data == SDCA_F32 && result == SDCA_F64)
    return epoch_impl<float, double>(*obj, d, m, n, static_cast<const float*>(X),
        static_cast<float*>(W), static_cast<float*>(A), labels, offsets, order, count, epochs);
  if (data == SDCA_F64 && result == SDCA_F64)
    return epoch_impl<double, double>(*obj, d, m, n, static_cast<const double*>(X),
        static_cast<double*>(W), static_cast<double*>(A), labels, offsets, order, count, epochs);
  return SDCA_ERR_PRECISION;
}

// The reference's SDCA epoch on kernel input (see epoch_kernel_run): K n x n
// (symmetric; column i = K_i), A m x n column-major, updated in place.
int ref_epoch_kernel(const sdca_objective* obj, int data, int result, int64_t m, int64_t n,
                     const void* K, void* A, const int64_t* labels, const int64_t* offsets,
                     const int64_t* order, int64_t count, int64_t epochs) {
  if (data == SDCA_F32 && result == SDCA_F32)
    return epoch_kernel_impl<float, float>(*obj, m, n, static_cast<const float*>(K),
        static_cast<float*>(A), labels, offsets, order, count, epochs);
  if (data == SDCA_F32 && result == SDCA_F64)
    return epoch_kernel_impl<float, double>(*obj, m, n, static_cast<const float*>(K),
        static_cast<float*>(A), labels, offsets, order, count, epochs);
  if (data == SDCA_F64 && result == SDCA_F64)
    return epoch_kernel_impl<double, double>(*obj, m, n, static_cast<const double*>(K),
        static_cast<double*>(A), labels, offsets, order, count, epochs);
  return SDCA_ERR_PRECISION;
}

int ref_prox(int op, int data, int result, int64_t m, int64_t n, void* x,
             const sdca_prox_params* p, const int64_t* col_p, sdca_thresholds* out,
             int nthreads) {
  if (data == SDCA_F32 && result == SDCA_F32)
    return prox_impl<float, float>(op, m, n, static_cast<float*>(x), p, col_p, out, nthreads);
  if (data == SDCA_F32 && result == SDCA_F64)
    return prox_impl<float, double>(op, m, n, static_cast<float*>(x), p, col_p, out, nthreads);
  if (data == SDCA_F64 && result == SDCA_F32)
    return prox_impl<double, float>(op, m, n, static_cast<double*>(x), p, col_p, out, nthreads);
  if (data == SDCA_F64 && result == SDCA_F64)
    return prox_impl<double, double>(op, m, n, static_cast<double*>(x), p, col_p, out, nthreads);
  return SDCA_ERR_PRECISION;
}

// ref_prox with the sets of each record (thresholds required).
int ref_prox_sets(int op, int data, int result, int64_t m, int64_t n, void* x,
                  const sdca_prox_params* p, const int64_t* col_p, sdca_thresholds* out,
                  sdca_prox_sets* sets, int nthreads) {
  if (!out) return SDCA_ERR_ARG_NULL;
  if (data == SDCA_F32 && result == SDCA_F32)
    return prox_impl<float, float>(op, m, n, static_cast<float*>(x), p, col_p, out, nthreads,
                                   sets);
  if (data == SDCA_F32 && result == SDCA_F64)
    return prox_impl<float, double>(op, m, n, static_cast<float*>(x), p, col_p, out, nthreads,
                                    sets);
  if (data == SDCA_F64 && result == SDCA_F32)
    return prox_impl<double, float>(op, m, n, static_cast<double*>(x), p, col_p, out, nthreads,
                                    sets);
  if (data == SDCA_F64 && result == SDCA_F64)
    return prox_impl<double, double>(op, m, n, static_cast<double*>(x), p, col_p, out,
                                     nthreads, sets);
  return SDCA_ERR_PRECISION;
}

int ref_eval_scores(const sdca_objective* objs, int n_obj, int data, int result,
                    int64_t m, int64_t n, const void* S, const void* A,
                    const int64_t* labels, const int64_t* offsets, double preg,
                    double dreg, sdca_eval_record* rec, double* accuracy,
                    double* per_example) {
  if (data == SDCA_F32 && result == SDCA_F32)
    return eval_impl<float, float>(objs, n_obj, m, n, static_cast<const float*>(S),
        static_cast<const float*>(A), labels, offsets, preg, dreg, rec, accuracy, per_example);
  if (data == SDCA_F32 && result == SDCA_F64)
    return eval_impl<float, double>(objs, n_obj, m, n, static_cast<const float*>(S),
        static_cast<const float*>(A), labels, offsets, preg, dreg, rec, accuracy, per_example);
  if (data == SDCA_F64 && result == SDCA_F64)
    return eval_impl<double, double>(objs, n_obj, m, n, static_cast<const double*>(S),
        static_cast<const double*>(A), labels, offsets, preg, dreg, rec, accuracy, per_example);
  return SDCA_ERR_PRECISION;
}

// The reference's evaluate_dataset over a feature input (see evaluate_all).
// X: d x n, W (and W0, NULL outside prox mode): d x m, A: m x n (borrowed
// mutable, restored), all column-major; offsets NULL for multiclass labels.
int ref_evaluate_dataset(const sdca_objective* objs, int n_obj, int data, int result,
                         int64_t d, int64_t m, int64_t n, const void* X, void* W,
                         const void* W0, void* A, const int64_t* labels,
                         const int64_t* offsets, sdca_eval_record* rec, double* accuracy,
                         int nthreads) {
  if (data == SDCA_F32 && result == SDCA_F32)
    return evaluate_impl<float, float>(objs, n_obj, d, m, n, static_cast<const float*>(X),
        static_cast<float*>(W), static_cast<const float*>(W0), static_cast<float*>(A), labels,
        offsets, rec, accuracy, nthreads);
  if (data == SDCA_F32 && result == SDCA_F64)
    return evaluate_impl<float, double>(objs, n_obj, d, m, n, static_cast<const float*>(X),
        static_cast<float*>(W), static_cast<const float*>(W0), static_cast<float*>(A), labels,
        offsets, rec, accuracy, nthreads);
  if (data == SDCA_F64 && result == SDCA_F64)
    return evaluate_impl<double, double>(objs, n_obj, d, m, n, static_cast<const double*>(X),
        static_cast<double*>(W), static_cast<const double*>(W0), static_cast<double*>(A), labels,
        offsets, rec, accuracy, nthreads);
  return SDCA_ERR_PRECISION;
}

// The reference's BLAS dot (math/blas.h:191-219) and the scores of one
// example (eval/scores.h:9-27), for the pins of the restatement's models.
float ref_blas_sdot(int n, const float* x, const float* y) { return sdca::sdca_blas_dot(n, x, y); }
double ref_blas_ddot(int n, const double* x, const double* y) { return sdca::sdca_blas_dot(n, x, y); }
void ref_blas_sgemv_t(int d, int m, const float* W, const float* x, float* s) {
  sdca::sdca_blas_gemv(d, m, W, x, s, CblasTrans);
}

double ref_lambert_w_exp_f64(double x) { return sdca::lambert_w_exp(x); }
float ref_lambert_w_exp_f32(float x) { return sdca::lambert_w_exp(x); }

}  // extern "C"
