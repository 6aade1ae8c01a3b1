// C entry points of the CPU oracle (TEST INFRASTRUCTURE ONLY: loaded by
// tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, never by
// the product library).
//
// oracle_prox          batch loop prox(dim, first, last, aux, ...) (proxdef.h:279-324)
// oracle_prox_sets     the same, also returning each record's sets (first / last
//                      over aux) and the branch that produced it
// oracle_eval_scores   per-example part of evaluate_dataset (eval.h:36-47) on given scores
// oracle_eval_features evaluate_dataset for feature input, with the scores
//                      gemv (eval/scores.h:21-26) as a plain loop
// oracle_epoch_features one SDCA epoch on feature input (solver.h:39-51,
//                      update.h:52-85) over a given example order
// oracle_epoch_kernel  the same on kernel input (update.h:88-107)
//
// Host pointers only.  `nthreads` > 1 splits columns / examples over
// std::threads, each with its own scratch (the reference is single-threaded;
// the split is a harness-level partition for the CPU baseline timing).
#include <type_traits>
#include <cstring>
#include <thread>

#include "oracle_epoch.hpp"
#include "oracle_eval.hpp"

namespace {

template <class F>
void parallel_for(int64_t n, int nthreads, F f) {
  if (nthreads <= 1 || n < 2 * nthreads) {
    f(static_cast<int64_t>(0), n, 0);
    return;
  }
  std::vector<std::thread> pool;
  int64_t chunk = (n + nthreads - 1) / nthreads;
  for (int w = 0; w < nthreads; ++w) {
    int64_t b = w * chunk, e = std::min(n, b + chunk);
    if (b >= e) break;
    pool.emplace_back(f, b, e, w);
  }
  for (auto& t : pool) t.join();
}

template <class D, class R>
void store_thr(sdca_thresholds* out, int64_t j, const orc::thr<R, D*>& t) {
  if (!out) return;
  out[j].t = static_cast<double>(t.t);
  out[j].lo = static_cast<double>(t.lo);
  out[j].hi = static_cast<double>(t.hi);
}

// n_hi = first - begin, n_mid = last - first over the block's scratch copy
// starting at `begin` (proxdef.h:29-67).
template <class D, class R>
void store_sets(sdca_prox_sets* out, int64_t j, const orc::thr<R, D*>& t, const D* begin) {
  if (!out) return;
  out[j].n_hi = static_cast<int64_t>(t.first - begin);
  out[j].n_mid = static_cast<int64_t>(t.last - t.first);
  out[j].branch = t.branch;
  out[j].reserved = 0;
}

template <class D, class R>
int prox_impl(int op, int64_t m, int64_t n, D* x, const sdca_prox_params* p,
              const int64_t* col_p, sdca_thresholds* thr_out, int nthreads,
              sdca_prox_sets* sets_out = nullptr) {
  const R lo = static_cast<R>(p->lo), hi = static_cast<R>(p->hi),
          rhs = static_cast<R>(p->rhs), rho = static_cast<R>(p->rho);
  const std::ptrdiff_t k = static_cast<std::ptrdiff_t>(p->k);
  if (op == SDCA_PROX_LAMBERT_W_EXP) {  // apply(dim, ..., lambert_w_exp_map<Data>)
    parallel_for(m * n, nthreads, [&](int64_t b, int64_t e, int) {
      for (int64_t i = b; i < e; ++i) x[i] = orc::lambert_w_exp(x[i]);
    });
    return 0;
  }
  parallel_for(n, nthreads, [&](int64_t b, int64_t e, int) {
    std::vector<D> aux(static_cast<size_t>(m));
    for (int64_t j = b; j < e; ++j) {
      D* col = x + j * m;
      std::copy(col, col + m, aux.begin());
      D* a = aux.data();
      D* a_end = a + m;
      if (op == SDCA_PROX_TWO_SIMPLEX || op == SDCA_PROX_TWO_SIMPLEX_SORT ||
          op == SDCA_PROX_TWO_ENTROPY) {
        std::ptrdiff_t pj = col_p ? static_cast<std::ptrdiff_t>(col_p[j])
                                  : static_cast<std::ptrdiff_t>(p->p);
        auto t = op == SDCA_PROX_TWO_SIMPLEX ? orc::two_simplex(a, a + pj, a + pj, a_end, rhs)
               : op == SDCA_PROX_TWO_SIMPLEX_SORT
                   ? orc::two_simplex_sort(a, a + pj, a + pj, a_end, rhs)
                   : orc::two_entropy(a, a + pj, a + pj, a_end, static_cast<R>(p->alpha));
        // The two-block batch loop (proxdef.h:301-324): the thresholds'
        // iterators point into aux, the clamp runs over the column.
        orc::thr<R, D*> t1 = t.first, t2 = t.second;
        orc::clamp(t1, col, col + pj);
        orc::clamp(t2, col + pj, col + m);
        if (thr_out) {
          store_thr<D, R>(thr_out, 2 * j, t1);
          store_thr<D, R>(thr_out, 2 * j + 1, t2);
        }
        store_sets<D, R>(sets_out, 2 * j, t1, a);
        store_sets<D, R>(sets_out, 2 * j + 1, t2, a + pj);
        continue;
      }
      orc::thr<R, D*> t;
      switch (op) {
        case SDCA_PROX_KNAPSACK_EQ: t = orc::knapsack_eq(a, a_end, lo, hi, rhs); break;
        case SDCA_PROX_KNAPSACK_LE: t = orc::knapsack_le(a, a_end, lo, hi, rhs); break;
        case SDCA_PROX_TOPK_SIMPLEX: t = orc::topk_simplex<R>(a, a_end, k, rhs); break;
        case SDCA_PROX_TOPK_CONE: t = orc::topk_cone<R>(a, a_end, k); break;
        case SDCA_PROX_ENTROPY: t = orc::entropy(a, a_end, hi, rhs); break;
        case SDCA_PROX_ENTROPY_NORM: t = orc::entropy_norm(a, a_end, hi, rhs); break;
        case SDCA_PROX_TOPK_ENTROPY: t = orc::topk_entropy<R>(a, a_end, k); break;
        case SDCA_PROX_KNAPSACK_LE_BIASED:
          t = orc::knapsack_le_biased(a, a_end, lo, hi, rhs, rho); break;
        case SDCA_PROX_TOPK_SIMPLEX_BIASED:
          t = orc::topk_simplex_biased<R>(a, a_end, k, rhs, rho); break;
        case SDCA_PROX_TOPK_CONE_BIASED: t = orc::topk_cone_biased<R>(a, a_end, k, rho); break;
        case SDCA_PROX_TOPK_ENTROPY_BIASED:
          t = orc::topk_entropy_biased<R>(a, a_end, k, static_cast<R>(p->alpha)); break;
        default: break;
      }
      orc::clamp(t, col, col + m);
      store_thr<D, R>(thr_out, j, t);
      store_sets<D, R>(sets_out, j, t, a);
    }
  });
  return 0;
}

struct eval_acc {
  std::vector<double> primal, dual, rank;
  std::vector<int64_t> hist;
};

// Per-example epilogue over examples [b, e) (eval.h:36-47).  Accumulates in
// the Result type in example order, as eval_train does.
template <class D, class R>
void eval_range(const std::vector<orc::objective<D, R>>& objs, int64_t m,
                int64_t b, int64_t e, const D* S, const D* A,
                const int64_t* labels, const int64_t* offsets,
                std::vector<R>& primal, std::vector<R>& dual,
                std::vector<R>& rank, std::vector<int64_t>& hist,
                double* per_example) {
  const size_t no = objs.size();
  std::vector<D> s(static_cast<size_t>(m)), work(static_cast<size_t>(m)),
      v(static_cast<size_t>(m));
  for (int64_t i = b; i < e; ++i) {
    std::copy(S + i * m, S + (i + 1) * m, s.begin());
    if (A) std::copy(A + i * m, A + (i + 1) * m, v.begin());
    else std::fill(v.begin(), v.end(), static_cast<D>(0));
    if (!offsets) {
      const int64_t y = labels[i];
      // eval_dual_loss: move_front, dual_loss, move_back (eval/dual.h:23-44)
      std::swap(v[0], v[y]);
      for (size_t o = 0; o < no; ++o) {
        R dl = objs[o].dual_loss(m, v.data());
        dual[o] += dl;
        if (per_example) per_example[(i * no + o) * 2 + 1] = static_cast<double>(dl);
      }
      // eval_primal_loss (eval/primal.h:27-53)
      std::swap(s[0], s[y]);
      D* it = std::partition(s.data() + 1, s.data() + m,
                             [&](const D& x) { return x >= s[0]; });
      hist[static_cast<size_t>(it - (s.data() + 1))] += 1;
      for (size_t o = 0; o < no; ++o) {
        // Each objective sees the scores as the partition left them.
        std::copy(s.begin(), s.end(), work.begin());
        R pl = objs[o].primal_loss(m, work.data());
        primal[o] += pl;
        if (per_example) per_example[(i * no + o) * 2] = static_cast<double>(pl);
      }
    } else {
      const int64_t* lab = labels + offsets[i];
      const std::ptrdiff_t p = static_cast<std::ptrdiff_t>(offsets[i + 1] - offsets[i]);
      orc::ml_move_front(lab, p, v.data());
      for (size_t o = 0; o < no; ++o) {
        R dl = objs[o].dual_loss_ml(m, p, v.data());
        dual[o] += dl;
        if (per_example) per_example[(i * no + o) * 2 + 1] = static_cast<double>(dl);
      }
      // eval_primal_loss multilabel (eval/primal.h:56-87)
      orc::ml_move_front(lab, p, s.data());
      D* neg_first = s.data() + p;
      D* neg_last = s.data() + m;
      R rl(0);
      for (std::ptrdiff_t g = 0; g < p; ++g) {
        const D gt = s[g];
        D* it = std::partition(neg_first, neg_last, [=](const D& x) { return x >= gt; });
        rl += static_cast<R>(std::distance(neg_first, it));
      }
      R rl_i = rl / static_cast<R>(p * (m - p));
      for (size_t o = 0; o < no; ++o) {
        rank[o] += rl_i;
        std::copy(s.begin(), s.end(), work.begin());
        R pl = objs[o].primal_loss_ml(m, p, work.data());
        primal[o] += pl;
        if (per_example) per_example[(i * no + o) * 2] = static_cast<double>(pl);
      }
    }
  }
}

template <class D, class R>
int eval_scores_impl(const sdca_objective* objs_in, int n_obj, int64_t m,
                     int64_t n, const D* S, const D* A, const int64_t* labels,
                     const int64_t* offsets, double preg, double dreg,
                     sdca_eval_record* rec, double* accuracy,
                     double* per_example, int nthreads) {
  std::vector<orc::objective<D, R>> objs;
  for (int o = 0; o < n_obj; ++o) objs.emplace_back(objs_in[o]);
  const size_t no = objs.size();
  int nt = std::max(1, nthreads);
  std::vector<std::vector<R>> P(nt, std::vector<R>(no, 0)), Q(nt, std::vector<R>(no, 0)),
      RK(nt, std::vector<R>(no, 0));
  std::vector<std::vector<int64_t>> H(nt, std::vector<int64_t>(static_cast<size_t>(m), 0));
  parallel_for(n, nt, [&](int64_t b, int64_t e, int w) {
    eval_range<D, R>(objs, m, b, e, S, A, labels, offsets, P[w], Q[w], RK[w], H[w],
                     per_example);
  });
  for (size_t o = 0; o < no; ++o) {
    R pl = 0, dl = 0, rk = 0;
    for (int w = 0; w < nt; ++w) { pl += P[w][o]; dl += Q[w][o]; rk += RK[w][o]; }
    // eval_end (eval/core.h:43-95) -> objective_base::update_all (objective_base.h:116-128)
    R pr = static_cast<R>(preg), dr = static_cast<R>(dreg);
    pl *= objs[o].coeff;
    rec[o].primal_loss = static_cast<double>(pl);
    rec[o].dual_loss = static_cast<double>(dl);
    rec[o].primal_regularizer = static_cast<double>(pr);
    rec[o].dual_regularizer = static_cast<double>(dr);
    rec[o].primal = static_cast<double>(pl + pr);
    rec[o].dual = static_cast<double>(dl - dr);
    rec[o].rank_loss = offsets ? static_cast<double>(rk / static_cast<R>(n)) : 0.0;
  }
  if (accuracy && !offsets) {
    std::vector<R> acc(static_cast<size_t>(m), 0);
    for (int w = 0; w < nt; ++w)
      for (int64_t j = 0; j < m; ++j) acc[j] += static_cast<R>(H[w][j]);
    std::partial_sum(acc.begin(), acc.end(), acc.begin());
    R coeff(1 / static_cast<R>(n));
    for (int64_t j = 0; j < m; ++j) accuracy[j] = static_cast<double>(acc[j] * coeff);
  }
  return 0;
}

// Regularizers for feature input (eval/regularizer.h:22-44,
// objective_base.h:59-89), with the dot in the Data type.
template <class D, class R>
void regularizers(int64_t dm, const D* W, const D* W0, double& preg, double& dreg) {
  R regul = static_cast<R>(orc::blas_dot<D>(dm, W, W)) / 2;
  R pr = 0, dr = 0;
  if (W0) {
    R prox = static_cast<R>(orc::blas_dot<D>(dm, W0, W));
    pr += regul - prox;
    dr += regul;
  } else {
    pr += regul;
    dr += regul;
  }
  preg = static_cast<double>(pr);
  dreg = static_cast<double>(dr);
}

// Dual regularizer of the kernel-input evaluation: the per-example
// regularizers_dual (objective_base.h:92-105, reached from the loop of
// eval.h:36-41 through eval/regularizer.h:81-98), 0.5 <a_i, s_i> added to
// both terms, summed over the examples in order.
template <class D, class R>
void dual_regularizer(int64_t m, int64_t n, const D* A, const D* S, double& preg, double& dreg) {
  R pr = 0, dr = 0;
  for (int64_t i = 0; i < n; ++i) {
    // The reference's dot in the data type (blas.h); for a long double
    // result the exact-arithmetic check: the dot accumulated in long double.
    R dot = 0;
    if (std::is_same<R, long double>::value) {
      for (int64_t j = 0; j < m; ++j)
        dot += static_cast<R>(A[i * m + j]) * static_cast<R>(S[i * m + j]);
    } else {
      dot = static_cast<R>(orc::blas_dot<D>(m, A + i * m, S + i * m));
    }
    R regul = dot / 2;
    pr += regul;
    dr += regul;
  }
  preg = static_cast<double>(pr);
  dreg = static_cast<double>(dr);
}

// scores = W' X as column dot products in the Data type.
template <class D>
void scores_impl(int64_t d, int64_t m, int64_t n, const D* X, const D* W, D* S,
                 int nthreads) {
  parallel_for(n, nthreads, [&](int64_t b, int64_t e, int) {
    for (int64_t i = b; i < e; ++i)
      for (int64_t j = 0; j < m; ++j)
        S[i * m + j] = orc::blas_dot<D>(d, W + j * d, X + i * d);
  });
}

}  // namespace

extern "C" {

int oracle_prox(int op, int data, int result, int64_t m, int64_t n, void* x,
                const sdca_prox_params* p, const int64_t* col_p,
                sdca_thresholds* thr_out, int nthreads) {
  if (data == SDCA_F32 && result == SDCA_F32)
    return prox_impl<float, float>(op, m, n, static_cast<float*>(x), p, col_p, thr_out, nthreads);
  if (data == SDCA_F32 && result == SDCA_F64)
    return prox_impl<float, double>(op, m, n, static_cast<float*>(x), p, col_p, thr_out, nthreads);
  if (data == SDCA_F64 && result == SDCA_F32)
    return prox_impl<double, float>(op, m, n, static_cast<double*>(x), p, col_p, thr_out, nthreads);
  if (data == SDCA_F64 && result == SDCA_F64)
    return prox_impl<double, double>(op, m, n, static_cast<double*>(x), p, col_p, thr_out, nthreads);
  // Long double arithmetic: the high-precision solution the parity tests use
  // to bound the rounding error of the float/double paths.
  if (data == SDCA_F32 && result == SDCA_LONG_DOUBLE)
    return prox_impl<float, long double>(op, m, n, static_cast<float*>(x), p, col_p, thr_out, nthreads);
  if (data == SDCA_F64 && result == SDCA_LONG_DOUBLE)
    return prox_impl<double, long double>(op, m, n, static_cast<double*>(x), p, col_p, thr_out, nthreads);
  return SDCA_ERR_PRECISION;
}

int oracle_prox_sets(int op, int data, int result, int64_t m, int64_t n, void* x,
                     const sdca_prox_params* p, const int64_t* col_p, sdca_thresholds* thr_out,
                     sdca_prox_sets* sets_out, int nthreads) {
  if (data == SDCA_F32 && result == SDCA_F32)
    return prox_impl<float, float>(op, m, n, static_cast<float*>(x), p, col_p, thr_out, nthreads,
                                   sets_out);
  if (data == SDCA_F32 && result == SDCA_F64)
    return prox_impl<float, double>(op, m, n, static_cast<float*>(x), p, col_p, thr_out,
                                    nthreads, sets_out);
  if (data == SDCA_F64 && result == SDCA_F32)
    return prox_impl<double, float>(op, m, n, static_cast<double*>(x), p, col_p, thr_out,
                                    nthreads, sets_out);
  if (data == SDCA_F64 && result == SDCA_F64)
    return prox_impl<double, double>(op, m, n, static_cast<double*>(x), p, col_p, thr_out,
                                     nthreads, sets_out);
  return SDCA_ERR_PRECISION;
}

int oracle_eval_scores(const sdca_objective* objs, int n_obj, int data, int result,
                       int64_t m, int64_t n, const void* S, const void* A,
                       const int64_t* labels, const int64_t* offsets, double preg,
                       double dreg, sdca_eval_record* rec, double* accuracy,
                       double* per_example, int nthreads) {
  if (data == SDCA_F32 && result == SDCA_F32)
    return eval_scores_impl<float, float>(objs, n_obj, m, n, static_cast<const float*>(S),
        static_cast<const float*>(A), labels, offsets, preg, dreg, rec, accuracy, per_example, nthreads);
  if (data == SDCA_F32 && result == SDCA_F64)
    return eval_scores_impl<float, double>(objs, n_obj, m, n, static_cast<const float*>(S),
        static_cast<const float*>(A), labels, offsets, preg, dreg, rec, accuracy, per_example, nthreads);
  if (data == SDCA_F64 && result == SDCA_F64)
    return eval_scores_impl<double, double>(objs, n_obj, m, n, static_cast<const double*>(S),
        static_cast<const double*>(A), labels, offsets, preg, dreg, rec, accuracy, per_example, nthreads);
  // Long double arithmetic: the high-precision losses the parity tests use to
  // bound the rounding error of the float/double paths.
  if (data == SDCA_F32 && result == SDCA_LONG_DOUBLE)
    return eval_scores_impl<float, long double>(objs, n_obj, m, n, static_cast<const float*>(S),
        static_cast<const float*>(A), labels, offsets, preg, dreg, rec, accuracy, per_example, nthreads);
  if (data == SDCA_F64 && result == SDCA_LONG_DOUBLE)
    return eval_scores_impl<double, long double>(objs, n_obj, m, n, static_cast<const double*>(S),
        static_cast<const double*>(A), labels, offsets, preg, dreg, rec, accuracy, per_example, nthreads);
  return SDCA_ERR_PRECISION;
}

int oracle_scores(int data, int64_t d, int64_t m, int64_t n, const void* X,
                  const void* W, void* S, int nthreads) {
  if (data == SDCA_F32)
    scores_impl<float>(d, m, n, static_cast<const float*>(X), static_cast<const float*>(W),
                       static_cast<float*>(S), nthreads);
  else if (data == SDCA_F64)
    scores_impl<double>(d, m, n, static_cast<const double*>(X), static_cast<const double*>(W),
                        static_cast<double*>(S), nthreads);
  else
    return SDCA_ERR_PRECISION;
  return 0;
}

int oracle_regularizers(int data, int result, int64_t dm, const void* W, const void* W0,
                        double* preg, double* dreg) {
  if (data == SDCA_F32 && result == SDCA_F32)
    regularizers<float, float>(dm, static_cast<const float*>(W), static_cast<const float*>(W0), *preg, *dreg);
  else if (data == SDCA_F32 && result == SDCA_F64)
    regularizers<float, double>(dm, static_cast<const float*>(W), static_cast<const float*>(W0), *preg, *dreg);
  else if (data == SDCA_F64 && result == SDCA_F64)
    regularizers<double, double>(dm, static_cast<const double*>(W), static_cast<const double*>(W0), *preg, *dreg);
  else
    return SDCA_ERR_PRECISION;
  return 0;
}

int oracle_dual_regularizer(int data, int result, int64_t m, int64_t n, const void* A,
                            const void* S, double* preg, double* dreg) {
  if (data == SDCA_F32 && result == SDCA_F32)
    dual_regularizer<float, float>(m, n, static_cast<const float*>(A), static_cast<const float*>(S), *preg, *dreg);
  else if (data == SDCA_F32 && result == SDCA_F64)
    dual_regularizer<float, double>(m, n, static_cast<const float*>(A), static_cast<const float*>(S), *preg, *dreg);
  else if (data == SDCA_F64 && result == SDCA_F64)
    dual_regularizer<double, double>(m, n, static_cast<const double*>(A), static_cast<const double*>(S), *preg, *dreg);
  else if (data == SDCA_F32 && result == SDCA_LONG_DOUBLE)
    dual_regularizer<float, long double>(m, n, static_cast<const float*>(A), static_cast<const float*>(S), *preg, *dreg);
  else
    return SDCA_ERR_PRECISION;
  return 0;
}

// X: n x d, W: m x d, A: n x m updated in place; order: count indices or
// NULL; reverse: the scores' dot products accumulated in Data, last term
// first.  Returns -1 for an objective without a multiclass update.
int oracle_epoch_features(const sdca_objective* obj, int data, int result, int64_t d, int64_t m,
                          int64_t n, const void* X, void* W, void* A, const int64_t* labels,
                          const int64_t* offsets, const int64_t* order, int64_t count,
                          int reverse) {
  if (data == SDCA_F32 && result == SDCA_F32)
    return orc::epoch<float, float>(*obj, d, m, n, static_cast<const float*>(X),
                                    static_cast<float*>(W), static_cast<float*>(A), labels, offsets,
                                    order, count, reverse != 0);
  if (data == SDCA_F32 && result == SDCA_F64)
    return orc::epoch<float, double>(*obj, d, m, n, static_cast<const float*>(X),
                                     static_cast<float*>(W), static_cast<float*>(A), labels,
                                     offsets, order, count, reverse != 0);
  if (data == SDCA_F64 && result == SDCA_F64)
    return orc::epoch<double, double>(*obj, d, m, n, static_cast<const double*>(X),
                                      static_cast<double*>(W), static_cast<double*>(A), labels,
                                      offsets, order, count, reverse != 0);
  if (data == SDCA_F32 && result == SDCA_LONG_DOUBLE)
    return orc::epoch<float, long double>(*obj, d, m, n, static_cast<const float*>(X),
                                          static_cast<float*>(W), static_cast<float*>(A), labels,
                                          offsets, order, count, reverse != 0);
  if (data == SDCA_F64 && result == SDCA_LONG_DOUBLE)
    return orc::epoch<double, long double>(*obj, d, m, n, static_cast<const double*>(X),
                                           static_cast<double*>(W), static_cast<double*>(A),
                                           labels, offsets, order, count, reverse != 0);
  return -2;
}

// One SDCA epoch on kernel input: K n x n (row i = K_i), A n x m updated in
// place; the rest as oracle_epoch_features.
int oracle_epoch_kernel(const sdca_objective* obj, int data, int result, int64_t m, int64_t n,
                        const void* K, void* A, const int64_t* labels, const int64_t* offsets,
                        const int64_t* order, int64_t count, int reverse) {
  if (data == SDCA_F32 && result == SDCA_F32)
    return orc::epoch_kernel<float, float>(*obj, m, n, static_cast<const float*>(K),
                                           static_cast<float*>(A), labels, offsets, order, count,
                                           reverse != 0);
  if (data == SDCA_F32 && result == SDCA_F64)
    return orc::epoch_kernel<float, double>(*obj, m, n, static_cast<const float*>(K),
                                            static_cast<float*>(A), labels, offsets, order, count,
                                            reverse != 0);
  if (data == SDCA_F64 && result == SDCA_F64)
    return orc::epoch_kernel<double, double>(*obj, m, n, static_cast<const double*>(K),
                                             static_cast<double*>(A), labels, offsets, order,
                                             count, reverse != 0);
  if (data == SDCA_F32 && result == SDCA_LONG_DOUBLE)
    return orc::epoch_kernel<float, long double>(*obj, m, n, static_cast<const float*>(K),
                                                 static_cast<float*>(A), labels, offsets, order,
                                                 count, reverse != 0);
  if (data == SDCA_F64 && result == SDCA_LONG_DOUBLE)
    return orc::epoch_kernel<double, long double>(*obj, m, n, static_cast<const double*>(K),
                                                  static_cast<double*>(A), labels, offsets, order,
                                                  count, reverse != 0);
  return -2;
}

double oracle_lambert_w_exp_f64(double x) { return orc::lambert_w_exp(x); }
float oracle_lambert_w_exp_f32(float x) { return orc::lambert_w_exp(x); }

}  // extern "C"
