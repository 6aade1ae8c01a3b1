// CPU restatement of libsdca's batched prox operators and evaluation pass.
//
// TEST INFRASTRUCTURE ONLY.  This header (and liboracle.so built from it) is
// the checker that the HIP path is compared against.  Only tests/,
// __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
// product library (libsdca_amd) never links or calls it.
//
// Every function restates one reference function step by step, with the same
// element types, comparison predicates and STL partition/selection calls, so
// that the results match the reference headers bit for bit when compiled with
// the same standard library.  Citations are relative to the reference tree
// (libsdca v0.3.1).  The build is -O3 without -ffast-math and without
// SDCA_ACCURATE_MATH, which is the reference's shipped macro set.
//
// Pins (tests/test_oracle_*.py):
//   * against the reference headers themselves (oracle/_ref, built from
//     /root/reference where that tree exists) on random and edge inputs;
//   * against committed golden vectors made from the same build
//     (tests/golden/);
//   * against closed forms and brute force: sort-based simplex projection,
//     KKT checks by enumeration of (|U|, |M|) for the top-k cone/simplex,
//     softmax for the entropic projection, mpmath Lambert W, the Omega known
//     answer and the two-simplex regression vector of the reference tests.
#ifndef SDCA_ORACLE_HPP
#define SDCA_ORACLE_HPP

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <functional>
#include <iterator>
#include <limits>
#include <numeric>
#include <utility>
#include <vector>

namespace orc {

// ---------------------------------------------------------------------------
// Threshold record (proxdef.h:29-67).  Over the permuted scratch copy,
// [begin, first) is fixed at hi, [first, last) is free and [last, end) is
// fixed at lo.  `kind` selects the elementwise map of the clamp pass
// (proxdef.h:164-196): 0 = identity, 1 = exp, 2 = lambert_w_exp.  `branch`
// names the return of the reference's threshold function that produced the
// record (an sdca_prox_branch value of the C ABI).
// ---------------------------------------------------------------------------
enum : int {
  B_SEARCH = 0, B_INACTIVE = 1, B_ZERO = 2, B_CONSTANT = 3, B_KNAPSACK = 4, B_SCAN = 5,
  B_DEFAULT = 6, B_U_EMPTY = 7, B_U_GROWN = 8, B_BELOW_RHS = 9
};

template <class R, class It>
struct thr {
  R t, lo, hi;
  It first, last;
  int kind;       // 3 = map_a * lambert_w_exp (a_lambert_w_exp_map, functor.h:30-38)
  double map_a;   // the map's constant, already rounded to Data
  int branch;
};

template <class T>
inline T tagged(T t, int branch) {
  t.branch = branch;
  return t;
}

template <class R, class It>
inline thr<R, It> make_thr(R t, R lo, R hi, It first, It last, int kind = 0,
                           double map_a = 1) {
  thr<R, It> r;
  r.t = t; r.lo = lo; r.hi = hi; r.first = first; r.last = last; r.kind = kind;
  r.map_a = map_a;
  r.branch = B_SEARCH;
  return r;
}

// exp_traits (log_exp.h:27-60): smallest argument with a normal exp().
template <class T> struct exp_min_arg;
template <> struct exp_min_arg<float> {
  static float get() { return -8.733654022216796875000000e+01f; }
};
template <> struct exp_min_arg<double> {
  static double get() { return std::log(std::numeric_limits<double>::min()); }
};
template <> struct exp_min_arg<long double> {
  static long double get() { return -1.135513711193302405799699e+04L; }
};

// x * log(x) with 0 log 0 = 0 (log_exp.h:76-80).
template <class T> inline T x_log_x(T x) { return (x > 0) ? x * std::log(x) : 0; }

// ---------------------------------------------------------------------------
// Lambert W of exp(x) (lambert.h:31-203).
// ---------------------------------------------------------------------------
template <class T>
inline T lw_step5(T w, T y) {  // order-5 Householder step, lambert.h:31-42
  T f0 = w - y, f1 = 1 + y;
  T f11 = f1 * f1, f0y = f0 * y;
  T f00y = f0 * f0y;
  return w - 4 * f0 * (6 * f1 * (f11 + f0y) + f00y)
    / (f11 * (24 * f11 + 36 * f0y) + f00y * (14 * y + f0 + 8));
}

template <class T>
inline T exp_approx(T x) {  // (1 + x/1024)^1024, lambert.h:53-62
  T y = 1 + x / static_cast<T>(1024);
  for (int i = 0; i < 10; ++i) y *= y;
  return y;
}

inline float lambert_w_exp(float x) {  // lambert.h:77-106
  float w;
  if (x > -1) {
    if (x <= 8) {
      w = lw_step5(x, 1.0f);
    } else {
      return (x <= 536870912) ? lw_step5(x - std::log(x), x) : x;
    }
  } else {
    if (x > -18) {
      w = exp_approx(x);
    } else {
      return (x > -104) ? std::exp(x) : 0.0f;
    }
  }
  return lw_step5(w, std::exp(x - w));
}

template <class T>
inline T lambert_w_exp_wide(T x) {  // double and long double, lambert.h:121-203
  T w;
  if (x > 0) {
    if (x <= 4) {
      w = lw_step5(x, static_cast<T>(1));
    } else if (x <= static_cast<T>(576460752303423488.0L)) {
      w = x - std::log(x);
      w = lw_step5(w, x);
    } else {
      return x;
    }
  } else {
    if (x > -36) {
      w = exp_approx(x);
      if (x > -20) w = lw_step5(w, exp_approx(x - w));
    } else {
      return (x > -746) ? std::exp(x) : static_cast<T>(0);
    }
  }
  return lw_step5(w, std::exp(x - w));
}
inline double lambert_w_exp(double x) { return lambert_w_exp_wide(x); }
inline long double lambert_w_exp(long double x) { return lambert_w_exp_wide(x); }

// ---------------------------------------------------------------------------
// log-sum-exp family (log_exp.h:88-338).
// ---------------------------------------------------------------------------
template <class R, class It>
inline R lse_at(It first, It last, It mx, R& s) {  // log_exp.h:134-152
  s = 0;
  R m = static_cast<R>(*mx);
  for (It a = first; a != mx; ++a) s += std::exp(static_cast<R>(*a) - m);
  for (It a = mx + 1; a != last; ++a) s += std::exp(static_cast<R>(*a) - m);
  return m + std::log1p(s);
}

template <class R, class It>
inline R lse(It first, It last) {  // log_exp.h:112-122
  if (first == last) return 0;
  R s;
  return lse_at<R>(first, last, std::max_element(first, last), s);
}

template <class R, class It>
inline R lse_both(It first, It last, It mx, R& l, R& l1) {  // log_exp.h:287-308
  R s;
  l = lse_at<R>(first, last, mx, s);
  R m = static_cast<R>(*mx);
  l1 = std::exp(-m);
  l1 = std::isfinite(l1) ? m + std::log1p(s + l1) : 0;
  return s;
}

// ---------------------------------------------------------------------------
// Continuous quadratic knapsack, Kiwiel variable fixing (knapsack_eq.h:25-109).
// ---------------------------------------------------------------------------
template <class R, class It>
inline thr<R, It> knapsack_eq(It first, It last, R lo, R hi, R rhs) {
  const R eps = std::numeric_limits<R>::epsilon()
              * std::max(static_cast<R>(1), std::abs(rhs));
  auto m = std::distance(first, last);
  R t = (std::accumulate(first, last, static_cast<R>(0)) - rhs)
        / static_cast<R>(m);
  It free_first(first), free_last(last);
  for (;;) {
    R cut = lo + t;
    It lo_begin = std::partition(free_first, free_last,
                                 [=](const R x) { return x > cut; });
    R sum_lo = std::accumulate(lo_begin, free_last, static_cast<R>(0));
    auto n_lo = std::distance(lo_begin, free_last);
    cut = hi + t;
    It hi_end = std::partition(free_first, lo_begin,
                               [=](const R x) { return x > cut; });
    R sum_hi = std::accumulate(free_first, hi_end, static_cast<R>(0));
    auto n_hi = std::distance(free_first, hi_end);

    R s_hi = static_cast<R>(n_hi) * hi;
    R s_lo = static_cast<R>(n_lo) * lo;
    R infeas = sum_hi + sum_lo - (s_hi + s_lo) - static_cast<R>(n_hi + n_lo) * t;
    R next;
    if (n_hi > 0 && infeas > eps) {
      free_first = hi_end;
      next = static_cast<R>(m) * t - sum_hi + s_hi;
      m -= n_hi;
    } else if (n_lo > 0 && infeas < -eps) {
      free_last = lo_begin;
      next = static_cast<R>(m) * t - sum_lo + s_lo;
      m -= n_lo;
    } else {
      free_first = hi_end;
      free_last = lo_begin;
      break;
    }
    if (m > 0) {
      t = next / static_cast<R>(m);
    } else {
      break;
    }
  }
  return make_thr(t, lo, hi, free_first, free_last);
}

// Inequality knapsack (knapsack_le.h:17-44).
template <class R, class It>
inline thr<R, It> knapsack_le(It first, It last, R lo, R hi, R rhs) {
  const R eps = std::numeric_limits<R>::epsilon()
              * std::max(static_cast<R>(1), std::abs(rhs));
  It mid_first = std::partition(first, last, [=](const R x) { return x >= hi; });
  It mid_last = std::partition(mid_first, last, [=](const R x) { return x > lo; });
  R s = std::accumulate(mid_first, mid_last, static_cast<R>(0))
      + hi * static_cast<R>(std::distance(first, mid_first))
      + lo * static_cast<R>(std::distance(mid_last, last));
  if (s > rhs + eps) return tagged(knapsack_eq(first, last, lo, hi, rhs), B_KNAPSACK);
  return tagged(make_thr(static_cast<R>(0), lo, hi, mid_first, mid_last), B_INACTIVE);
}

// ---------------------------------------------------------------------------
// Top-k cone (topk_cone.h:18-157).
// ---------------------------------------------------------------------------
enum class proj { zero, constant, general };

template <class R, class It>
inline proj cone_special_cases(It first, It last, std::ptrdiff_t k, R div,
                               thr<R, It>& out) {
  typedef typename std::iterator_traits<It>::value_type D;
  It k_last = first + k;
  std::nth_element(first, k_last - 1, last, std::greater<D>());
  const R eps = 16 * std::numeric_limits<R>::epsilon();
  R sum_k = std::accumulate(first, k_last, static_cast<R>(0));
  if (sum_k <= eps) {
    out = tagged(make_thr(static_cast<R>(0), static_cast<R>(0), static_cast<R>(0),
                          first, first), B_ZERO);
    return proj::zero;
  }
  R hi = sum_k / div;
  R t = static_cast<R>(*(k_last - 1)) - hi;
  if (k == std::distance(first, last) ||
      t >= static_cast<R>(*std::max_element(k_last, last)) - eps) {
    out = tagged(make_thr(t, static_cast<R>(0), hi, k_last, k_last), B_CONSTANT);
    return proj::constant;
  }
  return proj::general;
}

template <class R, class It>
inline thr<R, It> cone_search(It first, It last, std::ptrdiff_t k) {
  typedef typename std::iterator_traits<It>::value_type D;
  std::sort(first, last, std::greater<D>());
  It k_last = first + k;
  R k_u = static_cast<R>(k);
  R min_u = +std::numeric_limits<R>::infinity();
  R num_u = 0, sum_u = 0;
  const R eps = 16 * std::numeric_limits<R>::epsilon();
  for (It mf = first;;) {
    R min_m = +std::numeric_limits<R>::infinity();
    R max_m = -std::numeric_limits<R>::infinity();
    R sum_m = 0, num_m_sum_u = 0;
    R den = k_u * k_u;
    R k_u_sum_u = k_u * sum_u;
    for (It ml = mf;;) {
      R t = (num_u * sum_m - k_u_sum_u) / den;
      R hi = (num_m_sum_u + k_u * sum_m) / den;
      R tt = hi + t;
      if (max_m - eps <= tt && tt <= min_u + eps) {
        if (t <= min_m + eps &&
            ((ml == last) || static_cast<R>(*ml) - eps <= t)) {
          return tagged(make_thr(t, static_cast<R>(0), hi, mf, ml), B_SCAN);
        }
      }
      if (ml == last) break;
      min_m = static_cast<R>(*ml);
      max_m = static_cast<R>(*mf);
      sum_m += min_m;
      num_m_sum_u += sum_u;
      den += num_u;
      ++ml;
    }
    if (mf == k_last) break;
    min_u = static_cast<R>(*mf);
    sum_u += min_u;
    --k_u;
    ++num_u;
    ++mf;
  }
  return tagged(make_thr(static_cast<R>(0), static_cast<R>(0), static_cast<R>(0),
                         first, first), B_DEFAULT);
}

template <class R, class It>
inline thr<R, It> topk_cone(It first, It last, std::ptrdiff_t k) {
  thr<R, It> out;
  if (cone_special_cases(first, last, k, static_cast<R>(k), out) == proj::general)
    return cone_search<R>(first, last, k);
  return out;
}

// ---------------------------------------------------------------------------
// Top-k simplex (topk_simplex.h:9-68).
// ---------------------------------------------------------------------------
template <class R, class It>
inline bool topk_simplex_lt(It u_first, It u_last, R t, R k, R rhs, R eps) {
  if (u_first == u_last) return t < -eps;
  R num_u = static_cast<R>(std::distance(u_first, u_last));
  R sum_u = std::accumulate(u_first, u_last, static_cast<R>(0));
  return k * (sum_u + (k - num_u) * t) < rhs * num_u - eps;
}

template <class R, class It>
inline thr<R, It> topk_simplex(It first, It last, std::ptrdiff_t k, R rhs) {
  const R K = static_cast<R>(k), lo = 0;
  const R eps = std::numeric_limits<R>::epsilon()
              * std::max(static_cast<R>(1), std::abs(rhs));
  thr<R, It> out;
  switch (cone_special_cases(first, last, k, K, out)) {
    case proj::zero:
      break;
    case proj::constant:
      if (K * out.hi > rhs + eps)
        return tagged(knapsack_eq(first, last, lo, rhs / K, rhs), B_KNAPSACK);
      break;
    case proj::general: {
      thr<R, It> t = tagged(knapsack_eq(first, last, lo, rhs / K, rhs), B_KNAPSACK);
      if (topk_simplex_lt(first, t.first, t.t, K, rhs, eps))
        return cone_search<R>(first, last, k);
      return t;
    }
  }
  return out;
}

// ---------------------------------------------------------------------------
// Biased top-k cone and simplex, min 0.5 (<x,x> + rho <1,x>^2) - <a,x>
// (topk_cone_biased.h:9-137, topk_simplex_biased.h:9-71).
// ---------------------------------------------------------------------------
template <class R, class It>
inline thr<R, It> cone_biased_search(It first, It last, std::ptrdiff_t k, R rho) {
  typedef typename std::iterator_traits<It>::value_type D;
  std::sort(first, last, std::greater<D>());
  It k_last = first + k;
  R k_u = static_cast<R>(k);                                  // k - |U|
  R nu_rho = rho * static_cast<R>(k) * static_cast<R>(k);     // |U| + rho k^2
  R min_u = +std::numeric_limits<R>::infinity();
  R sum_u = 0;
  const R eps = 16 * std::numeric_limits<R>::epsilon();
  for (It mf = first;;) {
    R min_m = +std::numeric_limits<R>::infinity();
    R max_m = -std::numeric_limits<R>::infinity();
    R sum_m = 0, num_m_sum_u = 0;
    R den = k_u * k_u;
    R k_u_sum_u = k_u * sum_u;
    for (It ml = mf;;) {
      R t = (nu_rho * sum_m - k_u_sum_u) / den;
      R hi = (num_m_sum_u + k_u * sum_m) / den;
      R tt = hi + t;
      if (max_m - eps <= tt && tt <= min_u + eps) {
        if (t <= min_m + eps &&
            ((ml == last) || static_cast<R>(*ml) - eps <= t)) {
          return tagged(make_thr(t, static_cast<R>(0), hi, mf, ml), B_SCAN);
        }
      }
      if (ml == last) break;
      min_m = static_cast<R>(*ml);
      max_m = static_cast<R>(*mf);
      sum_m += min_m;
      num_m_sum_u += sum_u;
      den += nu_rho;
      ++ml;
    }
    if (mf == k_last) break;
    min_u = static_cast<R>(*mf);
    sum_u += min_u;
    --k_u;
    ++nu_rho;
    ++mf;
  }
  return tagged(make_thr(static_cast<R>(0), static_cast<R>(0), static_cast<R>(0),
                         first, first), B_DEFAULT);
}

template <class R, class It>
inline thr<R, It> topk_cone_biased(It first, It last, std::ptrdiff_t k, R rho) {
  const R K = static_cast<R>(k);
  thr<R, It> out;
  if (cone_special_cases(first, last, k, K + rho * K * K, out) == proj::general)
    return cone_biased_search<R>(first, last, k, rho);
  return out;
}

template <class R, class It>
inline bool topk_simplex_biased_lt(It u_first, It u_last, R t, R k, R rhs, R rho, R eps) {
  if (u_first == u_last) return t < rho * rhs - eps;
  R num_u = static_cast<R>(std::distance(u_first, u_last));
  R sum_u = std::accumulate(u_first, u_last, static_cast<R>(0));
  return k * (sum_u + (k - num_u) * t) < rhs * (num_u + rho * k * k) - eps;
}

template <class R, class It>
inline thr<R, It> topk_simplex_biased(It first, It last, std::ptrdiff_t k, R rhs, R rho) {
  const R K = static_cast<R>(k), lo = 0;
  const R eps = std::numeric_limits<R>::epsilon()
              * std::max(static_cast<R>(1), std::abs(rhs));
  thr<R, It> out;
  switch (cone_special_cases(first, last, k, K + rho * K * K, out)) {
    case proj::zero:
      break;
    case proj::constant:
      if (K * out.hi > rhs + eps)
        return tagged(knapsack_eq(first, last, lo, rhs / K, rhs), B_KNAPSACK);
      break;
    case proj::general: {
      thr<R, It> t = tagged(knapsack_eq(first, last, lo, rhs / K, rhs), B_KNAPSACK);
      if (topk_simplex_biased_lt(first, t.first, t.t, K, rhs, rho, eps))
        return cone_biased_search<R>(first, last, k, rho);
      return t;
    }
  }
  return out;
}

// ---------------------------------------------------------------------------
// Biased inequality knapsack, min 0.5 (<x,x> + rho <1,x>^2) - <a,x>,
// <1,x> <= rhs, lo <= x <= hi (knapsack_le_biased.h:10-130).
// ---------------------------------------------------------------------------
template <class R, class It>
inline thr<R, It> knapsack_le_biased_search(It first, It last, R lo, R hi, R rhs, R rho) {
  typedef typename std::iterator_traits<It>::value_type D;
  const R eps = std::numeric_limits<R>::epsilon()
              * std::max(static_cast<R>(1), std::abs(rhs));
  std::sort(first, last, std::greater<D>());
  const R rho_rhs = rho * rhs;
  const R rho_inv = static_cast<R>(1) / rho;
  const R num_x = static_cast<R>(std::distance(first, last));
  R num_u = 0, min_u = +std::numeric_limits<R>::infinity();
  for (It mf = first;;) {
    R min_m = +std::numeric_limits<R>::infinity();
    R max_m = -std::numeric_limits<R>::infinity();
    R num_m = 0, sum_m = 0;
    R num_l = num_x - num_u;
    for (It ml = mf;;) {
      R t = (lo * num_l + hi * num_u + sum_m) / (rho_inv + num_m);
      if (t <= rho_rhs + eps) {
        R tt = hi + t;
        if (max_m - eps <= tt && tt <= min_u + eps) {
          tt = lo + t;
          if (tt <= min_m + eps &&
              ((ml == last) || static_cast<R>(*ml) - eps <= tt)) {
            return tagged(make_thr(t, lo, hi, mf, ml), B_SCAN);
          }
        }
      }
      if (ml == last) break;
      min_m = static_cast<R>(*ml);
      max_m = static_cast<R>(*mf);
      sum_m += min_m;
      --num_l;
      ++num_m;
      ++ml;
    }
    if (mf == last) break;
    min_u = static_cast<R>(*mf);
    ++num_u;
    ++mf;
  }
  return tagged(make_thr(static_cast<R>(0), static_cast<R>(0), static_cast<R>(0),
                         first, first), B_DEFAULT);
}

template <class R, class It>
inline thr<R, It> knapsack_le_biased(It first, It last, R lo, R hi, R rhs, R rho) {
  if (rho == 0) return knapsack_le(first, last, lo, hi, rhs);
  const R eps = std::numeric_limits<R>::epsilon()
              * std::max(static_cast<R>(1), std::abs(rhs));
  thr<R, It> t = knapsack_eq(first, last, lo, hi, rhs);
  if (t.t >= rho * rhs - eps) return tagged(t, B_KNAPSACK);
  return knapsack_le_biased_search(first, last, lo, hi, rhs, rho);
}

// ---------------------------------------------------------------------------
// Entropic projections (entropy.h:19-53, entropy_norm.h:15-183).
// ---------------------------------------------------------------------------
template <class R, class It>
inline thr<R, It> entropy(It first, It last, R hi, R rhs) {
  const R eps = 16 * std::numeric_limits<R>::epsilon()
              * std::max(static_cast<R>(1), rhs);
  R lo(0), r(rhs), u = std::log(hi) + eps;
  R t = lse<R>(first, last) - std::log(rhs);
  It mf = first;
  for (;;) {
    R cut = t + u;
    It it = std::partition(mf, last, [=](R a) { return a > cut; });
    if (it == mf) break;
    r -= hi * static_cast<R>(std::distance(mf, it));
    mf = it;
    if (it == last) break;
    if (r <= eps) {
      t = static_cast<R>(*std::max_element(mf, last)) - exp_min_arg<R>::get() + 1;
      break;
    }
    t = lse<R>(mf, last) - std::log(r);
  }
  return make_thr(t, lo, hi, mf, last, 1);
}

template <class R, class It>
inline R sum_w_exp_step4(It first, It last, R rhs, R t) {  // entropy_norm.h:161-176
  R f0(0), f1(0), f2(0), f3(0);
  const R mt = -t;
  for (It a = first; a != last; ++a) {  // lambert.h:311-332
    R v = lambert_w_exp(static_cast<R>(*a) + mt);
    R d = 1 + v;
    R d3 = d * d * d;
    f0 += v;
    f1 += v / d;
    f2 += v / d3;
    f3 += v * (1 - 2 * v) / (d3 * d * d);
  }
  f0 -= rhs;
  R f02 = f0 * f2, f11 = f1 * f1;
  return t - 3 * f0 * (2 * f11 - f02) / (6 * f1 * (f02 - f11) - f0 * (f0 * f3));
}

template <class R, class It>
inline R solve_sum_w_exp(It first, It last, R rhs) {  // entropy_norm.h:110-134
  R t = (std::accumulate(first, last, static_cast<R>(0)) - rhs)
        / static_cast<R>(std::distance(first, last));
  It u_last = last;
  for (;;) {
    It it = std::partition(first, u_last, [=](R a) { return a > t; });
    if (it == u_last || it == first) break;
    u_last = it;
    t = (std::accumulate(first, u_last, static_cast<R>(0)) - rhs)
        / static_cast<R>(std::distance(first, u_last));
  }
  const R ub = static_cast<R>(*std::max_element(first, last)) - exp_min_arg<R>::get();
  const R eps = 16 * std::numeric_limits<R>::epsilon();
  for (std::size_t iter = 0; iter < 32; ++iter) {
    R prev(t);
    t = sum_w_exp_step4(first, last, rhs, std::min(t, ub));
    if (std::abs(prev - t) <= eps) break;
  }
  return t;
}

template <class R, class It>
inline thr<R, It> entropy_norm(It first, It last, R hi, R rhs) {
  const R eps = 16 * std::numeric_limits<R>::epsilon()
              * std::max(static_cast<R>(1), rhs);
  R lo(0), r(rhs), u = hi + std::log(hi) + eps;
  R t = solve_sum_w_exp(first, last, rhs);
  It mf = first;
  for (;;) {
    R cut = t + u;
    It it = std::partition(mf, last, [=](R a) { return a > cut; });
    if (it == mf) break;
    r -= hi * static_cast<R>(std::distance(mf, it));
    mf = it;
    if (it == last) break;
    if (r <= eps) {
      t = static_cast<R>(*std::max_element(mf, last)) - exp_min_arg<R>::get() + 1;
      break;
    }
    t = solve_sum_w_exp(mf, last, r);
  }
  return make_thr(t, lo, hi, mf, last, 2);
}

// Top-k entropy (topk_entropy.h:20-76).
template <class R, class It>
inline thr<R, It> topk_entropy(It first, It last, std::ptrdiff_t k) {
  const R eps = 16 * std::numeric_limits<R>::epsilon();
  const R K = static_cast<R>(k);
  It mx = std::max_element(first, last);
  R log_z, log_z_1;
  lse_both(first, last, mx, log_z, log_z_1);
  R t(log_z_1), lo(0), hi(1);
  if (k <= 1 || static_cast<R>(*mx) - eps <= log_z - std::log(K))
    return tagged(make_thr(t, lo, hi, first, last, 1), B_U_EMPTY);
  R min_u(0), sum_u(0), k_u(K), z(0);
  It mf = first;
  for (std::ptrdiff_t num_u = 1; num_u < k; ++num_u) {
    min_u = static_cast<R>(*mx);
    sum_u += min_u;
    std::swap(*mf, *mx);
    ++mf;
    --k_u;
    mx = std::max_element(mf, last);
    log_z = lse_at(mf, last, mx, z);
    R tt = log_z - std::log(k_u);
    if (static_cast<R>(*mx) - eps <= tt && tt <= min_u + eps) break;
  }
  R tmp = ((K - k_u) * log_z + k_u * std::log(k_u) - sum_u) / K;
  R mxv = static_cast<R>(*mx);
  if (tmp > mxv) {
    R a = (1 + z) * std::exp(mxv - tmp);
    t = tmp + std::log1p(a * K) - std::log(k_u);
    hi = a / (1 + a * K);
  } else {
    R a = std::exp(tmp - mxv) / K;
    t = mxv + std::log1p(z + a) - std::log(k_u / K);
    hi = (1 + z) / ((1 + z + a) * K);
  }
  return tagged(make_thr(t, lo, hi, mf, last, 1), B_U_GROWN);
}

// Biased top-k entropy (topk_entropy_biased.h:9-260):
//   min 0.5 alpha (<x,x> + s^2) + <x, log x> + (1 - s) log(1 - s) - <a, x>,
//   <1,x> = s <= 1, 0 <= x_i <= s / k;  x = clamp(W(exp(a - t)) / alpha).
// ---------------------------------------------------------------------------
// f0..f3 += sum over [first, last) of W(exp(a + t)) and its derivatives
// (lambert.h:253-332).
template <class R, class It>
inline void lw_sums(It first, It last, R t, R& f0, R& f1) {
  for (It a = first; a != last; ++a) {
    R v = lambert_w_exp(static_cast<R>(*a) + t);
    f0 += v;
    f1 += v / (1 + v);
  }
}
template <class R, class It>
inline void lw_sums(It first, It last, R t, R& f0, R& f1, R& f2, R& f3) {
  for (It a = first; a != last; ++a) {
    R v = lambert_w_exp(static_cast<R>(*a) + t);
    R d = 1 + v;
    R d3 = d * d * d;
    f0 += v;
    f1 += v / d;
    f2 += v / d3;
    f3 += v * (1 - 2 * v) / (d3 * d * d);
  }
}

// One Householder step for W(exp(alpha - t)) + sum_i W(exp(a_i - t)) = alpha
// (topk_entropy_biased.h:9-38); s = sum_i W(exp(a_i - t)) / alpha.
template <class R, class It>
inline void alpha_sum_w_exp_step4(It first, It last, R alpha, R& s, R& t) {
  R f0(0), f1(0), f2(0), f3(0);
  lw_sums(first, last, -t, f0, f1, f2, f3);
  s = f0 / alpha;
  lw_sums(&alpha, &alpha + 1, -t, f0, f1, f2, f3);
  f0 -= alpha;
  R f02 = f0 * f2, f11 = f1 * f1;
  R den = 6 * f1 * (f02 - f11) - f0 * (f0 * f3);
  if (std::abs(den) > 64 * std::numeric_limits<R>::min()) t -= 3 * f0 * (2 * f11 - f02) / den;
}

// Newton step on the KKT system in (s, t) for a given U
// (topk_entropy_biased.h:64-117).
template <class R, class It>
inline void topk_entropy_biased_newton(It first, It last, R K, R U, R C0, R C1, R C2, R C3,
                                       R C4, R C5, R& s, R& t) {
  R S0(0), S1(0);
  lw_sums(first, last, -t, S0, S1);
  R E = S0 + t * S1;
  R z, Az, Bz;
  if (s < static_cast<R>(0.5)) {
    z = s;
    Az = K * (z * (U + std::log1p(-z) + z / (1 - z)) - U * x_log_x(z)) - C0 * z;
    Bz = z * (C2 + K / (1 - z)) + C1;
  } else {
    z = 1 - s;
    Az = K * (z * (U - U * std::log1p(-z) - 1) + x_log_x(z) + 1) - C0 * z;
    Bz = z * (C2 + C1 / (1 - z)) + K;
  }
  R Dz = C3 * z - Bz * S1;
  if (std::abs(Dz) > 64 * std::numeric_limits<R>::min()) {
    s = (C4 * E * z - Az * S1) / Dz;
    t = (C5 * Az - E * Bz) / Dz;
  }
}

template <class R, class It>
inline thr<R, It> topk_entropy_biased(It first, It last, std::ptrdiff_t k, R alpha) {
  typedef typename std::iterator_traits<It>::value_type D;
  It max_el = std::max_element(first, last);
  R max = static_cast<R>(*max_el);
  const R eps = 16 * std::numeric_limits<R>::epsilon() * std::max(static_cast<R>(1), max);
  R s(0), t(max);
  // U empty (topk_entropy_biased.h:48-61, 211-215).
  for (std::size_t iter = 0; iter < 32; ++iter) {
    R t1(t);
    alpha_sum_w_exp_step4(first, last, alpha, s, t);
    if (std::abs(t1 - t) <= std::numeric_limits<R>::epsilon()) break;
  }
  const R lo(0), K(static_cast<R>(k));
  const double map_a = static_cast<double>(1 / static_cast<D>(alpha));
  if (k == 1) return tagged(make_thr(t, lo, s, first, last, 3, map_a), B_U_EMPTY);
  const R alpha_k(alpha / K);
  R tt = t + std::max(alpha_k * s + std::log(alpha_k * s), exp_min_arg<R>::get());
  if (max - eps <= tt) return tagged(make_thr(t, lo, s / K, first, last, 3, map_a), B_U_EMPTY);
  // U not empty: grow U by the largest remaining element (:235-259).
  std::swap(*first, *max_el);
  const R log_k = std::log(K), log_alpha = std::log(alpha);
  R min_u(max), sum_u(max);
  It mf = first + 1;
  for (std::ptrdiff_t num_u = 1; mf != last;) {
    max_el = std::max_element(mf, last);
    max = static_cast<R>(*max_el);
    s = static_cast<R>(0.999);
    t = max;
    {  // topk_entropy_biased_kkt_iterate (:144-176)
      const R U = static_cast<R>(num_u);
      const R lb(0), ub(1), eps16 = 16 * std::numeric_limits<R>::epsilon();
      const R C1 = U * K, C2 = (K + U) * alpha, C3 = (K - U) * (U - 1) * alpha;
      const R C4 = K * (U - 1), C5 = (1 - U / K) * alpha;
      const R C0 = C4 * log_alpha - C1 * log_k - sum_u;
      for (std::size_t iter = 0; iter < 32; ++iter) {
        R s1(s), t1(t);
        s = std::min(std::max(lb, s), ub);
        topk_entropy_biased_newton(mf, last, K, U, C0, C1, C2, C3, C4, C5, s, t);
        if (std::abs(s1 - s) + std::abs(t1 - t) <= eps16) break;
      }
      s = std::min(std::max(lb, s), ub);
    }
    tt = t + std::max(alpha_k * s + std::log(alpha_k * s), exp_min_arg<R>::get());
    if (max - eps <= tt && tt <= min_u + eps) break;
    if (++num_u > k) break;
    min_u = max;
    sum_u += max;
    std::swap(*mf, *max_el);
    ++mf;
  }
  return tagged(make_thr(t, lo, s / K, first, last, 3, map_a), B_U_GROWN);
}

// ---------------------------------------------------------------------------
// Two-block entropic projection (two_entropy.h:9-231):
//   x = W(exp(a - t)) / alpha,  y = W(exp(b - t - c)) / alpha,  c = alpha / |a|,
// with t the root of sum_i W(e^(a_i - t)) + sum_j W(e^(b_j - t - c)) = alpha.
// ---------------------------------------------------------------------------
template <class R, class It>
inline R two_w_step4(It af, It al, It bf, It bl, R alpha, R c, R& t) {  // :15-38
  R f0(0), f1(0), f2(0), f3(0);
  lw_sums(af, al, -t, f0, f1, f2, f3);
  lw_sums(bf, bl, -t - c, f0, f1, f2, f3);
  f0 -= alpha;
  R f02 = f0 * f2, f11 = f1 * f1;
  R den = 6 * f1 * (f02 - f11) - f0 * (f0 * f3);
  if (std::abs(den) > 64 * std::numeric_limits<R>::min()) t -= 3 * f0 * (2 * f11 - f02) / den;
  return f0;
}

template <class R, class It>
inline R two_w_value(It af, It al, It bf, It bl, R alpha, R c, R t) {  // :45-58
  R f0(0);
  for (It a = af; a != al; ++a) f0 += lambert_w_exp(static_cast<R>(*a) + (-t));
  for (It b = bf; b != bl; ++b) f0 += lambert_w_exp(static_cast<R>(*b) + (-t - c));
  return f0 - alpha;
}

template <class R, class It>
inline void two_w_bisection(It af, It al, It bf, It bl, R alpha, R c, R eps,
                            std::size_t max_num_iter, R& t, R& lb, R& ub, R& lf, R& uf) {  // :65-96
  for (std::size_t iter = 0; iter < max_num_iter; ++iter) {
    t = (lb + ub) / 2;
    R f1 = two_w_value(af, al, bf, bl, alpha, c, t);
    if (eps < f1 && f1 < lf) {
      lf = f1;
      lb = t;
    } else if (uf < f1 && f1 < -eps) {
      uf = f1;
      ub = t;
    } else {
      break;
    }
  }
  t = (lb + ub) / 2;
}

template <class R, class It>
inline std::pair<thr<R, It>, thr<R, It>> two_entropy(It af, It al, It bf, It bl, R alpha) {
  typedef typename std::iterator_traits<It>::value_type D;
  const std::size_t max_num_iter = 32;
  const R eps = std::numeric_limits<R>::epsilon();
  const R num_a = static_cast<R>(std::distance(af, al));
  const R num_b = static_cast<R>(std::distance(bf, bl));
  const R max_a = static_cast<R>(*std::max_element(af, al));
  const R max_b = static_cast<R>(*std::max_element(bf, bl));
  const R sum_a = std::accumulate(af, al, static_cast<R>(0));
  const R sum_b = std::accumulate(bf, bl, static_cast<R>(0));
  const R c = alpha / num_a;
  const R max = std::max(max_a, max_b - c);
  // Bracket guards (:159-163).
  R lb = std::numeric_limits<R>::lowest();
  R ub = max - 64 * exp_min_arg<R>::get();
  R lf = std::numeric_limits<R>::max();
  R uf = std::numeric_limits<R>::lowest();
  // Two guesses, each followed by one step (:165-175).
  R t01 = max - std::log(alpha);
  R t1(t01);
  R f1 = two_w_step4(af, al, bf, bl, alpha, c, t1);
  R t02 = (sum_a + sum_b - num_b * c - alpha) / (num_a + num_b);
  R t2(t02);
  R f2 = two_w_step4(af, al, bf, bl, alpha, c, t2);
  if (f1 > f2) {
    std::swap(t01, t02);
    std::swap(t1, t2);
    std::swap(f1, f2);
  }
  R t;
  if (f1 > 0) {
    lb = t01;
    lf = f1;
    t = t1;
  } else if (f2 < 0) {
    ub = t02;
    uf = f2;
    t = t2;
  } else {
    lb = t02;
    ub = t01;
    lf = f2;
    uf = f1;
    t = std::max(lb, std::min(std::abs(f1) < std::abs(f2) ? t1 : t2, ub));
    // The bisection count, converted to size_t as the reference converts it
    // (this file is compiled by the same compiler as the reference shim).
    const R log2_inv = static_cast<R>(1.4426950408889634);
    std::size_t num_iter = std::min(max_num_iter,
                                    static_cast<std::size_t>(std::log(ub - lb) * log2_inv));
    two_w_bisection(af, al, bf, bl, alpha, c, eps, num_iter, t, lb, ub, lf, uf);
  }
  // Householder steps kept inside the bracket (:207-220).
  for (std::size_t iter = 0; iter < max_num_iter; ++iter) {
    t1 = t;
    f1 = two_w_step4(af, al, bf, bl, alpha, c, t);
    if (0 <= f1 && f1 < lf) {
      lb = t1;
      lf = f1;
    } else if (uf < f1 && f1 <= 0) {
      ub = t1;
      uf = f1;
    }
    t = std::max(lb, std::min(t, ub));
    if (std::abs(t1 - t) <= eps) break;
  }
  const R lo(0), hi(1);
  const double map_a = static_cast<double>(1 / static_cast<D>(alpha));
  return std::make_pair(make_thr(t, lo, hi, af, al, 3, map_a),
                        make_thr(t + c, lo, hi, bf, bl, 3, map_a));
}

// ---------------------------------------------------------------------------
// Two-block simplex, <1,x> = <1,y> <= rhs (two_simplex.h:18-119).
template <class R, class It>
inline std::pair<thr<R, It>, thr<R, It>>
two_simplex(It a_first, It a_last, It b_first, It b_last, R rhs) {
  R t, s, lo(0), hi(rhs);
  const R eps = std::numeric_limits<R>::epsilon()
              * std::max(static_cast<R>(1), rhs);
  It x_last(a_last);
  for (;;) {
    t = (std::accumulate(a_first, x_last, static_cast<R>(0)) - rhs)
        / static_cast<R>(std::distance(a_first, x_last));
    It it = std::partition(a_first, x_last, [=](const R x) { return x > t; });
    if (it == x_last) break;
    x_last = it;
  }
  It y_last(b_last);
  for (;;) {
    s = (std::accumulate(b_first, y_last, static_cast<R>(0)) - rhs)
        / static_cast<R>(std::distance(b_first, y_last));
    It it = std::partition(b_first, y_last, [=](const R y) { return y > s; });
    if (it == y_last) break;
    y_last = it;
  }
  if (t + s >= -eps) {
    return std::make_pair(make_thr(t, lo, hi, a_first, x_last),
                          make_thr(s, lo, hi, b_first, y_last));
  }
  auto m = std::distance(a_first, x_last) + std::distance(b_first, y_last);
  t = (+std::accumulate(a_first, x_last, static_cast<R>(0))
       - std::accumulate(b_first, y_last, static_cast<R>(0))) / static_cast<R>(m);
  for (;;) {
    It x_it = std::partition(a_first, x_last, [=](const R x) { return x > t; });
    R sum_x = std::accumulate(x_it, x_last, static_cast<R>(0));
    auto n_x = std::distance(x_it, x_last);
    It y_it = std::partition(b_first, y_last, [=](const R y) { return y > -t; });
    R sum_y = std::accumulate(y_it, y_last, static_cast<R>(0));
    auto n_y = std::distance(y_it, y_last);
    R next, infeas = sum_x - sum_y - static_cast<R>(n_x + n_y) * t;
    if (n_y > 0 && infeas > eps) {
      y_last = y_it;
      next = static_cast<R>(m) * t + sum_y;
      m -= n_y;
    } else if (n_x > 0 && infeas < -eps) {
      x_last = x_it;
      next = static_cast<R>(m) * t - sum_x;
      m -= n_x;
    } else {
      x_last = x_it;
      y_last = y_it;
      break;
    }
    if (m > 0) {
      t = next / static_cast<R>(m);
    } else {
      break;
    }
  }
  return std::make_pair(tagged(make_thr(t, lo, hi, a_first, x_last), B_BELOW_RHS),
                        tagged(make_thr(-t, lo, hi, b_first, y_last), B_BELOW_RHS));
}

// The same problem by the sort-and-scan method (two_simplex_sort.h:15-111):
// both blocks sorted in descending order, then the common sum c is located
// on the grid of breakpoints where the number of active entries r, s grows.
template <class R, class It>
inline std::pair<thr<R, It>, thr<R, It>>
two_simplex_sort(It a_first, It a_last, It b_first, It b_last, R rhs) {
  const R lo(0), hi(rhs);
  const R eps = std::numeric_limits<R>::epsilon()
              * std::max(static_cast<R>(1), rhs);
  std::sort(a_first, a_last, std::greater<R>());
  std::sort(b_first, b_last, std::greater<R>());
  R c = 0, C = rhs, best_c = rhs, sum_mu = *a_first, sum_nu = *b_first;
  typename std::iterator_traits<It>::difference_type r = 1, s = 1;
  // Past the end, a pseudo point that ends the scan.
  auto a_at = [&](decltype(r) i) {
    return a_first + i != a_last ? static_cast<R>(a_first[i])
                                 : static_cast<R>(*std::prev(a_last)) - C;
  };
  auto b_at = [&](decltype(s) i) {
    return b_first + i != b_last ? static_cast<R>(b_first[i])
                                 : static_cast<R>(*std::prev(b_last)) - C;
  };
  R a_r = a_at(r), b_s = b_at(s);
  int branch = B_SEARCH;  // common sum rhs unless the scan stops inside
  while (c < C) {
    R copt = (s * sum_mu + r * sum_nu) / static_cast<R>(r + s);
    R next_cr = (sum_mu + a_r) - (r + 1) * a_r;
    R next_cs = (sum_nu + b_s) - (s + 1) * b_s;
    R next_c = std::min(std::min(next_cr, next_cs), C);
    if (c <= copt && copt < next_c) {
      best_c = copt;
      branch = B_BELOW_RHS;
      break;
    }
    if (next_c >= C - eps) {
      best_c = C;
      break;
    }
    if (next_cr < next_cs) {
      sum_mu += a_r;
      ++r;
      a_r = a_at(r);
    } else {
      sum_nu += b_s;
      ++s;
      b_s = b_at(s);
    }
    c = next_c;
  }
  R theta_a = (sum_mu - best_c) / static_cast<R>(r);
  R theta_b = (sum_nu - best_c) / static_cast<R>(s);
  return std::make_pair(tagged(make_thr(theta_a, lo, hi, a_first, a_first + r), branch),
                        tagged(make_thr(theta_b, lo, hi, b_first, b_first + s), branch));
}

// ---------------------------------------------------------------------------
// Clamp/map pass (proxdef.h:164-196): thresholds are cast to Data first.
// ---------------------------------------------------------------------------
template <class R, class It>
inline void clamp(const thr<R, It>& th, It first, It last) {
  typedef typename std::iterator_traits<It>::value_type D;
  const D t = static_cast<D>(th.t), lo = static_cast<D>(th.lo),
          hi = static_cast<D>(th.hi);
  for (It x = first; x != last; ++x) {
    D v = *x - t;
    if (th.kind == 1) v = std::exp(v);
    else if (th.kind == 2) v = lambert_w_exp(v);
    else if (th.kind == 3) v = static_cast<D>(th.map_a) * lambert_w_exp(v);
    *x = std::max(lo, std::min(v, hi));
  }
}

// <prox(x), prox(x)> and <x, prox(x)> from the threshold sets (proxdef.h:332-370).
template <class R, class It>
inline R dot_prox_prox(const thr<R, It>& t, It first, It last) {
  R num_hi = static_cast<R>(std::distance(first, t.first));
  R num_mi = static_cast<R>(std::distance(t.first, t.last));
  R num_lo = static_cast<R>(std::distance(t.last, last));
  R sum_mi = std::accumulate(t.first, t.last, static_cast<R>(0));
  R dot_mi(0);
  for (It a = t.first; a != t.last; ++a) { R x = *a; dot_mi += x * x; }
  return t.hi * t.hi * num_hi + t.t * t.t * num_mi + t.lo * t.lo * num_lo
       + dot_mi - static_cast<R>(2) * t.t * sum_mi;
}

template <class R, class It>
inline R dot_x_prox(const thr<R, It>& t, It first, It last) {
  R sum_hi = std::accumulate(first, t.first, static_cast<R>(0));
  R sum_mi = std::accumulate(t.first, t.last, static_cast<R>(0));
  R sum_lo = std::accumulate(t.last, last, static_cast<R>(0));
  R dot_mi(0);
  for (It a = t.first; a != t.last; ++a) { R x = *a; dot_mi += x * x; }
  return t.hi * sum_hi - t.t * sum_mi + t.lo * sum_lo + dot_mi;
}

}  // namespace orc

#endif
