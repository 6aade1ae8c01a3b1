// CPU restatement of one SDCA epoch on feature input (TEST INFRASTRUCTURE
// ONLY; see oracle.hpp for the rules on who may load it).
//
// The example loop of solver.h:39-51 over a given order, each step
// update_variables (update.h:52-85):
//   norm2 = <x_i, x_i> (scratch.h:27-41); nothing happens when norm2 <= 0;
//   scores = W' x_i (eval/scores.h:21-26);
//   a_old = a_i; the objective's update_dual_variables on the label-first
//   view (output.h:44-71 move_front / move_back);
//   diff = sum |a_old - a_new| (sdca_blas_asum); if diff > epsilon(Data):
//   W -= x_i (a_old - a_new)' (sdca_blas_ger with alpha -1).
// The objectives' updates (the six multiclass ones):
//   l2_hinge_topk          l2_hinge_topk.h:44-68    (prox_topk_simplex_biased, rho 1)
//   l2_hinge_topk_smooth   l2_hinge_topk.h:132-159  (rho = norm2 / (norm2 + gamma / c))
//   l2_topk_hinge          l2_topk_hinge.h:46-69    (prox_knapsack_le_biased, hi c / k)
//   l2_topk_hinge_smooth   l2_topk_hinge.h:137-163
//   l2_entropy             l2_entropy.h:48-74       (prox_two_entropy, alpha c norm2)
//   l2_entropy_topk        l2_entropy_topk.h:47-71  (prox_topk_entropy_biased)
// and the three multilabel ones, on the labels-first view
// (output.h:121-164, multilabel move_front / move_back):
//   l2_multilabel_hinge         l2_multilabel_hinge.h:40-66    (prox_two_simplex, rhs c)
//   l2_multilabel_hinge_smooth  l2_multilabel_hinge.h:137-166
//   l2_multilabel_entropy       l2_multilabel_entropy.h:43-69  (prox_two_entropy, alpha c norm2)
// BLAS calls are modelled as in oracle_eval.hpp: dot products exact and
// rounded once to Data (blas_dot), axpby and scal elementwise in Data, ger
// as w - x_l y_j per element.  `reverse` accumulates the score dot
// products in Data from the last feature down (a second, equally valid
// rounding: the spread between the two runs measures how the epoch carries
// the scores' rounding).
#ifndef SDCA_ORACLE_EPOCH_HPP
#define SDCA_ORACLE_EPOCH_HPP

#include <algorithm>
#include <cmath>
#include <limits>
#include <numeric>
#include <vector>

#include "oracle_eval.hpp"

namespace orc {

// reverse: the sum accumulated in Data from the last term down, rounding at
// every step (as a plain BLAS loop may), instead of the exact sum.
template <class D>
inline D dot_order(std::ptrdiff_t n, const D* x, const D* y, bool reverse) {
  if (!reverse) return blas_dot(n, x, y);
  D s = 0;
  for (std::ptrdiff_t i = n - 1; i >= 0; --i) s += x[i] * y[i];
  return s;
}

// The objective's update_dual_variables on v = a_i (label first, m entries)
// with scores s (label first).  Returns false for an objective without an
// update here.
template <class D, class R>
inline bool update_dual(const sdca_objective& ob, std::ptrdiff_t m, D norm2, D* v, D* s) {
  const R c = static_cast<R>(ob.c), gamma = static_cast<R>(ob.gamma);
  const std::ptrdiff_t k = static_cast<std::ptrdiff_t>(ob.k);
  D* first = v + 1;
  D* last = v + m;
  std::vector<D> aux(first, last);
  switch (ob.kind) {
    case SDCA_OBJ_HINGE_TOPK:
    case SDCA_OBJ_HINGE_TOPK_SMOOTH:
    case SDCA_OBJ_TOPK_HINGE:
    case SDCA_OBJ_TOPK_HINGE_SMOOTH: {
      const bool smooth = ob.kind == SDCA_OBJ_HINGE_TOPK_SMOOTH ||
                          ob.kind == SDCA_OBJ_TOPK_HINGE_SMOOTH;
      const R rhs = c, zero = 0;
      const R rho = smooth ? static_cast<R>(norm2) / (static_cast<R>(norm2) + gamma / c) : R(1);
      // 1. the vector to project: a s - b v (axpby), then + (a - v_0) off the label
      D a = smooth ? static_cast<D>(rho) / norm2 : D(1) / norm2;
      const D b = smooth ? -static_cast<D>(rho) : D(-1);
      for (std::ptrdiff_t j = 0; j < m; ++j) v[j] = a * s[j] + b * v[j];
      a -= v[0];
      for (D* x = first; x != last; ++x) *x += a;
      // 2. the proximal step (thresholds on a copy, clamp of the range)
      std::copy(first, last, aux.begin());
      thr<R, D*> t;
      if (ob.kind == SDCA_OBJ_HINGE_TOPK || ob.kind == SDCA_OBJ_HINGE_TOPK_SMOOTH)
        t = topk_simplex_biased<R>(aux.data(), aux.data() + (m - 1), k, rhs, rho);
      else
        t = knapsack_le_biased(aux.data(), aux.data() + (m - 1), zero,
                               c / static_cast<R>(k), rhs, rho);
      clamp(t, first, last);
      // 3. recover the variables
      v[0] = static_cast<D>(std::min(rhs, std::accumulate(first, last, zero)));
      for (D* x = first; x != last; ++x) *x *= D(-1);
      return true;
    }
    case SDCA_OBJ_ENTROPY: {
      for (std::ptrdiff_t j = 0; j < m; ++j) v[j] = D(1) * s[j] + (-norm2) * v[j];
      const R alpha = c * static_cast<R>(norm2);
      std::vector<D> all(v, v + m);
      auto tt = two_entropy(all.data(), all.data() + 1, all.data() + 1, all.data() + m, alpha);
      thr<R, D*> t1 = tt.first, t2 = tt.second;
      clamp(t1, v, v + 1);
      clamp(t2, v + 1, v + m);
      const D a = static_cast<D>(-c), b = static_cast<D>(c / R(1));
      v[0] = a * v[0] + b;
      for (D* x = first; x != last; ++x) *x *= a;
      return true;
    }
    case SDCA_OBJ_ENTROPY_TOPK: {
      const R alpha = c * static_cast<R>(norm2), zero = 0, one = 1;
      for (std::ptrdiff_t j = 0; j < m; ++j) v[j] = D(1) * s[j] + (-norm2) * v[j];
      const D a = -v[0];
      for (D* x = first; x != last; ++x) *x += a;
      std::copy(first, last, aux.begin());
      thr<R, D*> t = topk_entropy_biased<R>(aux.data(), aux.data() + (m - 1), k, alpha);
      clamp(t, first, last);
      v[0] = static_cast<D>(c * std::min(one, std::accumulate(first, last, zero)));
      for (D* x = first; x != last; ++x) *x *= static_cast<D>(-c);
      return true;
    }
    default:
      return false;
  }
}

// The multilabel objectives' update_dual_variables on v = a_i with its nl
// labels first (m entries) and scores s (same order).  The two-block prox
// runs on copies of the blocks (proxdef.h:259-276) and clamps v.
template <class D, class R>
inline bool update_dual_ml(const sdca_objective& ob, std::ptrdiff_t m, std::ptrdiff_t nl, D norm2,
                           D* v, D* s) {
  const R c = static_cast<R>(ob.c), gamma = static_cast<R>(ob.gamma);
  D* pos_first = v;
  D* pos_last = v + nl;
  D* neg_first = v + nl;
  D* neg_last = v + m;
  switch (ob.kind) {
    case SDCA_OBJ_MULTILABEL_HINGE:
    case SDCA_OBJ_MULTILABEL_HINGE_SMOOTH: {
      D a, b;
      if (ob.kind == SDCA_OBJ_MULTILABEL_HINGE) {
        a = D(1) / norm2;
        b = D(1);
      } else {
        const R gamma_div_c = gamma / c;
        a = static_cast<D>(R(1) / (static_cast<R>(norm2) + gamma_div_c));
        b = static_cast<D>(static_cast<R>(norm2) / (static_cast<R>(norm2) + gamma_div_c));
      }
      for (std::ptrdiff_t j = 0; j < m; ++j) v[j] = a * s[j] + (-b) * v[j];
      a /= 2;
      for (D* x = pos_first; x != pos_last; ++x) *x = a - *x;
      for (D* x = neg_first; x != neg_last; ++x) *x = a + *x;
      std::vector<D> pa(pos_first, pos_last), na(neg_first, neg_last);
      auto tt = two_simplex(pa.data(), pa.data() + nl, na.data(), na.data() + (m - nl), c);
      clamp(tt.first, pos_first, pos_last);
      clamp(tt.second, neg_first, neg_last);
      for (D* x = neg_first; x != neg_last; ++x) *x *= D(-1);
      return true;
    }
    case SDCA_OBJ_MULTILABEL_ENTROPY: {
      for (std::ptrdiff_t j = 0; j < m; ++j) v[j] = D(1) * s[j] + (-norm2) * v[j];
      const R alpha = c * static_cast<R>(norm2);
      std::vector<D> pa(pos_first, pos_last), na(neg_first, neg_last);
      auto tt = two_entropy(pa.data(), pa.data() + nl, na.data(), na.data() + (m - nl), alpha);
      clamp(tt.first, pos_first, pos_last);
      clamp(tt.second, neg_first, neg_last);
      const D a = static_cast<D>(-c), b = static_cast<D>(c / static_cast<R>(nl));
      for (D* x = pos_first; x != pos_last; ++x) *x = a * *x + b;
      for (D* x = neg_first; x != neg_last; ++x) *x *= a;
      return true;
    }
    default:
      return false;
  }
}

// The objective's update of example i (update_dual_variables,
// update.h:12-49): the label (multiclass) or the labels (multilabel, output.h:121-164)
// moved to the front of v = a_i and of the scores, the update, and v's
// entries moved back.  Returns false for an objective without an update.
template <class D, class R>
inline bool update_example(const sdca_objective& ob, std::ptrdiff_t m, const int64_t* labels,
                           const int64_t* offsets, std::ptrdiff_t i, D norm2, D* v, D* scores) {
  if (offsets) {
    const int64_t o0 = offsets[i], nl = offsets[i + 1] - offsets[i];
    for (int64_t q = 0; q < nl; ++q) {
      std::swap(v[q], v[labels[o0 + q]]);
      std::swap(scores[q], scores[labels[o0 + q]]);
    }
    if (!update_dual_ml<D, R>(ob, m, nl, norm2, v, scores)) return false;
    for (int64_t q = nl - 1; q >= 0; --q) std::swap(v[q], v[labels[o0 + q]]);
  } else {
    const std::ptrdiff_t y = static_cast<std::ptrdiff_t>(labels[i]);
    std::swap(v[0], v[y]);
    std::swap(scores[0], scores[y]);
    if (!update_dual<D, R>(ob, m, norm2, v, scores)) return false;
    std::swap(v[0], v[y]);
  }
  return true;
}

// One epoch over `order` (count entries; NULL: 0..n-1); offsets (n + 1,
// CSR into labels) for the multilabel objectives, NULL for the multiclass
// ones.  X: n x d, W: m x d,
// A: n x m (each example's / class's values contiguous, as the reference's
// column-major d x n, d x m and m x n matrices).
template <class D, class R>
inline int epoch(const sdca_objective& ob, std::ptrdiff_t d, std::ptrdiff_t m, std::ptrdiff_t n,
                 const D* X, D* W, D* A, const int64_t* labels, const int64_t* offsets,
                 const int64_t* order, std::ptrdiff_t count, bool reverse) {
  std::vector<D> norms(static_cast<size_t>(n)), scores(static_cast<size_t>(m)),
      copy(static_cast<size_t>(m));
  for (std::ptrdiff_t i = 0; i < n; ++i) norms[i] = blas_dot(d, X + d * i, X + d * i);
  for (std::ptrdiff_t q = 0; q < count; ++q) {
    const std::ptrdiff_t i = order ? static_cast<std::ptrdiff_t>(order[q]) : q;
    const D norm2 = norms[i];
    if (norm2 <= 0) continue;
    const D* x = X + d * i;
    for (std::ptrdiff_t j = 0; j < m; ++j) scores[j] = dot_order(d, W + d * j, x, reverse);
    D* v = A + m * i;
    std::copy(v, v + m, copy.begin());
    if (!update_example<D, R>(ob, m, labels, offsets, i, norm2, v, scores.data())) return -1;
    // var_copy = a_old - a_new; diff = asum
    long double asum = 0;
    for (std::ptrdiff_t j = 0; j < m; ++j) {
      copy[j] = copy[j] + D(-1) * v[j];
      asum += std::fabs(static_cast<long double>(copy[j]));
    }
    if (static_cast<D>(asum) > std::numeric_limits<D>::epsilon()) {
      for (std::ptrdiff_t j = 0; j < m; ++j) {
        D* w = W + d * j;
        const D yj = copy[j];
        for (std::ptrdiff_t l = 0; l < d; ++l) w[l] = w[l] - x[l] * yj;
      }
    }
  }
  return 0;
}

// One epoch on kernel input (update.h:88-107) over `order`: K is the
// training set's n x n kernel matrix (row i = K_i, the reference's column
// i), A: n x m updated in place.  norm2 = K_ii; scores = A' K_i, the gemv of
// eval/scores.h:30-47 over the n training examples (reverse: accumulated in
// Data from the last example, else exact); only the dual variables change.
template <class D, class R>
inline int epoch_kernel(const sdca_objective& ob, std::ptrdiff_t m, std::ptrdiff_t n, const D* K,
                        D* A, const int64_t* labels, const int64_t* offsets,
                        const int64_t* order, std::ptrdiff_t count, bool reverse) {
  std::vector<D> scores(static_cast<size_t>(m)), column(static_cast<size_t>(n));
  for (std::ptrdiff_t q = 0; q < count; ++q) {
    const std::ptrdiff_t i = order ? static_cast<std::ptrdiff_t>(order[q]) : q;
    const D* ki = K + n * i;
    const D norm2 = ki[i];
    if (norm2 <= 0) continue;
    for (std::ptrdiff_t j = 0; j < m; ++j) {
      for (std::ptrdiff_t l = 0; l < n; ++l) column[l] = A[m * l + j];
      scores[j] = dot_order(n, column.data(), ki, reverse);
    }
    if (!update_example<D, R>(ob, m, labels, offsets, i, norm2, A + m * i, scores.data()))
      return -1;
  }
  return 0;
}

}  // namespace orc

#endif
