// CPU restatement of libsdca's evaluation pass (TEST INFRASTRUCTURE ONLY; see
// oracle.hpp for the rules on who may load it).
//
// Objectives: primal_loss / dual_loss / loss coefficient of the eight
// feature-input objectives (objective/*.h), the per-example epilogue of
// evaluate_dataset (eval.h:36-47, eval/primal.h:27-87, eval/dual.h:23-63) and
// eval_end (eval/core.h:43-95).  The BLAS dot products of the reference
// (math/blas.h:191-219) are modelled as exact dot products rounded to the Data
// type (see blas_dot).
#ifndef SDCA_ORACLE_EVAL_HPP
#define SDCA_ORACLE_EVAL_HPP

#include "oracle.hpp"
#include "../include/sdca_hip.h"

namespace orc {

// cblas_?dot (math/blas.h:191-219).  The reference links whatever CBLAS the
// build selects (MKL, Accelerate, ...; cmake/SelectBLAS.cmake), so its
// accumulation order is unpinned; the oracle models it as the exact dot
// product rounded once to the Data type (accumulated in long double).
template <class D>
inline D blas_dot(std::ptrdiff_t n, const D* x, const D* y) {
  long double s = 0;
  for (std::ptrdiff_t i = 0; i < n; ++i) s += static_cast<long double>(x[i]) * y[i];
  return static_cast<D>(s);
}

template <class D, class R>
struct objective {
  int kind;
  R c, gamma;
  std::ptrdiff_t k;
  R coeff;     // objective_base::coeff_primal_loss
  R gdc, gd2c; // gamma / c, gamma / (2 c)
  R gdk;       // gamma / k
  R clogc;     // x_log_x(c)

  objective(const sdca_objective& o)
      : kind(o.kind), c(static_cast<R>(o.c)), gamma(static_cast<R>(o.gamma)),
        k(static_cast<std::ptrdiff_t>(o.k)) {
    gdc = gamma / c;
    gd2c = gamma / (2 * c);
    gdk = gamma / static_cast<R>(k);
    clogc = x_log_x(c);
    switch (kind) {
      case SDCA_OBJ_HINGE_TOPK:          // l2_hinge_topk.h:25-32
      case SDCA_OBJ_TOPK_HINGE:          // l2_topk_hinge.h:25-32
        coeff = c / static_cast<R>(k); break;
      case SDCA_OBJ_HINGE_TOPK_SMOOTH:   // l2_hinge_topk.h:109-120
      case SDCA_OBJ_TOPK_HINGE_SMOOTH:   // l2_topk_hinge.h:113-124
      case SDCA_OBJ_MULTILABEL_HINGE_SMOOTH:  // l2_multilabel_hinge.h:117-124
        coeff = c / gamma; break;
      default:
        coeff = c; break;
    }
  }

  bool multilabel() const { return kind >= SDCA_OBJ_MULTILABEL_HINGE; }

  // Multiclass primal loss with the ground truth at scores[0]; may reorder.
  R primal_loss(std::ptrdiff_t m, D* s) const {
    D* first = s + 1;
    D* last = s + m;
    switch (kind) {
      case SDCA_OBJ_HINGE_TOPK: {  // l2_hinge_topk.h:71-86
        const D a = 1 - s[0];
        for (D* x = first; x != last; ++x) *x += a;
        std::nth_element(first, first + k - 1, last, std::greater<D>());
        R zero(0);
        return std::max(zero, std::accumulate(first, first + k, zero));
      }
      case SDCA_OBJ_HINGE_TOPK_SMOOTH: {  // l2_hinge_topk.h:162-179
        const D a = 1 - s[0];
        for (D* x = first; x != last; ++x) *x += a;
        thr<R, D*> t = topk_simplex<R>(first, last, k, gamma);
        R hp = dot_x_prox(t, first, last);
        R pp = dot_prox_prox(t, first, last);
        return hp - static_cast<R>(0.5) * pp;
      }
      case SDCA_OBJ_TOPK_HINGE: {  // l2_topk_hinge.h:72-87
        const D a = 1 - s[0];
        for (D* x = first; x != last; ++x) *x += a;
        std::nth_element(first, first + k - 1, last, std::greater<D>());
        D* it = std::partition(first, first + k, [](D x) { return x > 0; });
        return std::accumulate(first, it, static_cast<R>(0));
      }
      case SDCA_OBJ_TOPK_HINGE_SMOOTH: {  // l2_topk_hinge.h:166-183
        const D a = 1 - s[0];
        for (D* x = first; x != last; ++x) *x += a;
        R lo(0), hi(gdk), rhs(gamma);
        thr<R, D*> t = knapsack_le(first, last, lo, hi, rhs);
        R hp = dot_x_prox(t, first, last);
        R pp = dot_prox_prox(t, first, last);
        return hp - static_cast<R>(0.5) * pp;
      }
      case SDCA_OBJ_ENTROPY: {  // l2_entropy.h:77-91
        R l = lse<R>(s, s + m);
        R avg = std::accumulate(s, s + 1, static_cast<R>(0)) / static_cast<R>(1);
        return l - avg;
      }
      case SDCA_OBJ_ENTROPY_TOPK: {  // l2_entropy_topk.h:74-94
        const D a = -s[0];
        for (D* x = first; x != last; ++x) *x += a;
        thr<R, D*> t = topk_entropy<R>(first, last, k);
        if (t.first == first) return t.t;
        R num_hi = static_cast<R>(std::distance(first, t.first));
        R sum_hi = std::accumulate(first, t.first, static_cast<R>(0));
        R sk = t.hi * static_cast<R>(k);
        return t.hi * (sum_hi + t.t * (static_cast<R>(k) - num_hi))
             - x_log_x(1 - sk) - num_hi * x_log_x(t.hi);
      }
      default:
        return 0;
    }
  }

  // Multilabel primal loss with the p positives at scores[0..p); may reorder.
  R primal_loss_ml(std::ptrdiff_t m, std::ptrdiff_t p, D* s) const {
    D *pos_first = s, *pos_last = s + p, *neg_first = s + p, *neg_last = s + m;
    switch (kind) {
      case SDCA_OBJ_MULTILABEL_HINGE: {  // l2_multilabel_hinge.h:69-84
        D min_pos = *std::min_element(pos_first, pos_last);
        D max_neg = *std::max_element(neg_first, neg_last);
        R zero(0), loss = static_cast<R>(max_neg - min_pos + 1);
        return std::max(zero, loss);
      }
      case SDCA_OBJ_MULTILABEL_HINGE_SMOOTH: {  // l2_multilabel_hinge.h:168-191
        const D a(0.5);
        for (D* x = pos_first; x != pos_last; ++x) *x = a - *x;
        for (D* x = neg_first; x != neg_last; ++x) *x += a;
        auto t = two_simplex(pos_first, pos_last, neg_first, neg_last, gamma);
        R pos_hp = dot_x_prox(t.first, pos_first, pos_last);
        R pos_pp = dot_prox_prox(t.first, pos_first, pos_last);
        R neg_hp = dot_x_prox(t.second, neg_first, neg_last);
        R neg_pp = dot_prox_prox(t.second, neg_first, neg_last);
        return (pos_hp + neg_hp) - static_cast<R>(0.5) * (pos_pp + neg_pp);
      }
      case SDCA_OBJ_MULTILABEL_ENTROPY: {  // l2_multilabel_entropy.h:72-86
        R l = lse<R>(pos_first, neg_last);
        R avg = std::accumulate(pos_first, pos_last, static_cast<R>(0))
              / static_cast<R>(p);
        return l - avg;
      }
      default:
        return 0;
    }
  }

  // Multiclass dual loss with the ground truth at A[0] (objective_base.h:49-56).
  R dual_loss(std::ptrdiff_t m, const D* A) const {
    switch (kind) {
      case SDCA_OBJ_HINGE_TOPK_SMOOTH:   // l2_hinge_topk.h:182-192
      case SDCA_OBJ_TOPK_HINGE_SMOOTH:   // l2_topk_hinge.h:186-196
        return static_cast<R>(A[0])
             - gd2c * static_cast<R>(blas_dot<D>(m - 1, A + 1, A + 1));
      case SDCA_OBJ_ENTROPY: {           // l2_entropy.h:94-114 (p = 1)
        R dl(0), p(1);
        { R a = A[0]; dl -= x_log_x(c - p * a); }
        dl /= p;
        for (std::ptrdiff_t j = 1; j < m; ++j) { R a = A[j]; dl -= x_log_x(-a); }
        R sum = static_cast<R>(0) + A[0];
        dl += clogc + std::log(p) * (c - sum);
        return dl;
      }
      case SDCA_OBJ_ENTROPY_TOPK: {      // l2_entropy_topk.h:97-107
        R dl = clogc - x_log_x(c - static_cast<R>(A[0]));
        for (std::ptrdiff_t j = 1; j < m; ++j) { R a = A[j]; dl -= x_log_x(-a); }
        return dl;
      }
      default:
        return static_cast<R>(A[0]);
    }
  }

  // Multilabel dual loss with the p positives at A[0..p).
  R dual_loss_ml(std::ptrdiff_t m, std::ptrdiff_t p, const D* A) const {
    switch (kind) {
      case SDCA_OBJ_MULTILABEL_HINGE:  // l2_multilabel_hinge.h:87-96
        return std::accumulate(A, A + p, static_cast<R>(0));
      case SDCA_OBJ_MULTILABEL_HINGE_SMOOTH: {  // l2_multilabel_hinge.h:194-208
        R l1 = std::accumulate(A, A + p, static_cast<R>(0));
        R l2 = std::accumulate(A + p, A + m, static_cast<R>(0));
        R sm = gdc * static_cast<R>(blas_dot<D>(m, A, A));
        return static_cast<R>(0.5) * (l1 - l2 - sm);
      }
      case SDCA_OBJ_MULTILABEL_ENTROPY: {  // l2_multilabel_entropy.h:89-109
        R dl(0), pp(static_cast<R>(p));
        for (std::ptrdiff_t j = 0; j < p; ++j) { R a = A[j]; dl -= x_log_x(c - pp * a); }
        dl /= pp;
        for (std::ptrdiff_t j = p; j < m; ++j) { R a = A[j]; dl -= x_log_x(-a); }
        R sum = std::accumulate(A, A + p, static_cast<R>(0));
        dl += clogc + std::log(pp) * (c - sum);
        return dl;
      }
      default:
        return 0;
    }
  }
};

// multilabel_output::move_front / move_back (data/output.h:120-165).
template <class D>
inline void ml_move_front(const int64_t* lab, std::ptrdiff_t p, D* x) {
  for (std::ptrdiff_t j = 0; j < p; ++j) std::swap(x[j], x[lab[j]]);
}
template <class D>
inline void ml_move_back(const int64_t* lab, std::ptrdiff_t p, D* x) {
  for (std::ptrdiff_t j = p - 1; j >= 0; --j) std::swap(x[j], x[lab[j]]);
}

}  // namespace orc

#endif
