// Lambert-map thresholds of one column held in LDS, solved by one wave:
//
// * biased top-k entropy (topk_entropy_biased.h:179-268): (t, hi) from the
//   order-4 Householder iteration on W(e^(alpha - t)) + sum_i W(e^(a_i - t))
//   = alpha while no entry is capped (:9-61), then, while the feasibility
//   test fails, the set U of capped entries grows by the largest remaining
//   entry and (s, t) come from the Newton iteration on the two-equation
//   system of :120-176;
// * two-block entropy (two_entropy.h:109-231): t from the reference's two
//   guesses, bisection and bracketed Householder steps on
//   sum W(e^(a - t)) + sum W(e^(b - t - c)) = alpha.
//
// Each pass is a sum of W(e^(x_i + shift)) and its derivatives over the
// column: each of the NT threads (one wave, or a whole workgroup of NT)
// sums a stride-NT share, and the group reduction gives every thread the
// totals, so the scalar updates run uniformly on all of them.  `lane` is the
// thread's index in the group.
// Used by the wave-per-column prox kernels and the SDCA epoch.
#ifndef SDCA_HIP_PROX_LAMBERT_WAVE_HPP
#define SDCA_HIP_PROX_LAMBERT_WAVE_HPP

#include "common.hpp"
#include "prox_impl.hpp"

namespace sdca_gpu {

// f0 = sum_i W(e^(s_i + t_i)) with t_i = ta for i < p and tb beyond
// (sum_lambert_w_exp, lambert.h:220-237).
// wout (optional, the wave's LDS array of R): each pass leaves its W values
// there, for the output map.
// NT > 64 (a whole workgroup on one column: a few entries per thread, one
// wave per SIMD, the passes latency-bound) takes the thread's entries four at
// a time with the branch-free W so that their chains overlap: loads read a
// clamped index, entries past m add zero, and the sums keep their order.
constexpr int kLwBlock = 4;

template <class D, class R, int NT = 64>
__device__ inline R lw_sum0(const D* s, int m, int p, int lane, R ta, R tb) {
  R a0(0);
  if constexpr (NT > 64) {
    for (int i0 = lane; i0 < m; i0 += kLwBlock * NT) {
      R v[kLwBlock];
#pragma unroll
      for (int u = 0; u < kLwBlock; ++u) {
        const int i = i0 + u * NT;
        const int ic = i < m ? i : m - 1;
        v[u] = lambert_w_exp_nb(static_cast<R>(s[ic]) + (ic < p ? ta : tb));
      }
#pragma unroll
      for (int u = 0; u < kLwBlock; ++u) a0 += (i0 + u * NT < m) ? v[u] : R(0);
    }
  } else {
    for (int i = lane; i < m; i += NT) a0 += lambert_w_exp(static_cast<R>(s[i]) + (i < p ? ta : tb));
  }
  return group_sum<NT>(a0);
}

// f0 = sum_i W(e^(s_i + t)), f1 = sum_i W / (1 + W) (lambert.h:253-271).
template <class D, class R, int NT = 64>
__device__ inline void lw_sums2(const D* s, int m, int lane, R t, R& f0, R& f1,
                                R* wout = nullptr) {
  R a0(0), a1(0);
  if constexpr (NT > 64) {
    for (int i0 = lane; i0 < m; i0 += kLwBlock * NT) {
      R v[kLwBlock];
#pragma unroll
      for (int u = 0; u < kLwBlock; ++u) {
        const int i = i0 + u * NT;
        v[u] = lambert_w_exp_nb(static_cast<R>(s[i < m ? i : m - 1]) + t);
      }
#pragma unroll
      for (int u = 0; u < kLwBlock; ++u) {
        const int i = i0 + u * NT;
        const bool ok = i < m;
        if (wout && ok) wout[i] = v[u];
        a0 += ok ? v[u] : R(0);
        a1 += ok ? div_near(v[u], R(1) + v[u]) : R(0);
      }
    }
  } else {
    for (int i = lane; i < m; i += NT) {
      const R v = lambert_w_exp(static_cast<R>(s[i]) + t);
      if (wout) wout[i] = v;
      a0 += v;
      a1 += div_near(v, R(1) + v);
    }
  }
  group_sums<NT>(a0, a1);
  f0 = a0;
  f1 = a1;
}

// Largest move dt of the shift for which a pass takes W(e^(y - dt)) from
// the previous pass's W(e^y) by the Taylor step lambert_w_exp_shift instead
// of a new evaluation: the omitted fourth-order term is below dt^4 w / 24,
// 4e-10 w for float at 1e-2 and 4e-18 w for double at 1e-4, under the
// rounding of the sums either way.
template <class R>
__device__ constexpr R lw_shift_max() {
  return sizeof(R) == 4 ? R(1e-2) : R(kLambertShiftMax);
}

// The terms of the derivative sums of one W value: W / (1 + W),
// W / (1 + W)^3 and W (1 - 2W) / (1 + W)^5 from one reciprocal of 1 + W
// (they steer the steps; the root is where the sum of W equals its target).
template <class R>
__device__ inline void lw_terms(R v, R& a1, R& a2, R& a3) {
  const R rd = div_near(R(1), R(1) + v);
  const R rd2 = rd * rd;
  const R rd3 = rd2 * rd;
  a1 = v * rd;
  a2 = v * rd3;
  a3 = v * (R(1) - R(2) * v) * (rd3 * rd2);
}

// f0..f3: W and its first three derivatives in t (lambert.h:308-332), with
// the shift ta for entries below p and tb beyond.
// win (optional, with wout the same LDS array): W of every entry at shifts
// larger by wdt (|wdt| <= lw_shift_max), from the previous pass; this pass
// then takes each W by the Taylor step from it instead of a new evaluation.
template <class D, class R, int NT = 64>
__device__ inline void lw_sums4(const D* s, int m, int lane, R t, R& f0, R& f1, R& f2, R& f3,
                                int p = -1, R tb = R(0), R* wout = nullptr,
                                const R* win = nullptr, R wdt = R(0)) {
  if (p < 0) {
    p = m;
    tb = t;
  }
  R a0(0), a1(0), a2(0), a3(0);
  if constexpr (NT > 64) {
    for (int i0 = lane; i0 < m; i0 += kLwBlock * NT) {
      R v[kLwBlock];
#pragma unroll
      for (int u = 0; u < kLwBlock; ++u) {
        const int i = i0 + u * NT;
        const int ic = i < m ? i : m - 1;
        v[u] = win ? lambert_w_exp_shift(win[ic], wdt)
                   : lambert_w_exp_nb(static_cast<R>(s[ic]) + (ic < p ? t : tb));
      }
#pragma unroll
      for (int u = 0; u < kLwBlock; ++u) {
        const int i = i0 + u * NT;
        const bool ok = i < m;
        if (wout && ok) wout[i] = v[u];
        R b1, b2, b3;
        lw_terms(v[u], b1, b2, b3);
        a0 += ok ? v[u] : R(0);
        a1 += ok ? b1 : R(0);
        a2 += ok ? b2 : R(0);
        a3 += ok ? b3 : R(0);
      }
    }
  } else {
    for (int i = lane; i < m; i += NT) {
      const R v = win ? lambert_w_exp_shift(win[i], wdt)
                      : lambert_w_exp(static_cast<R>(s[i]) + (i < p ? t : tb));
      if (wout) wout[i] = v;
      R b1, b2, b3;
      lw_terms(v, b1, b2, b3);
      a0 += v;
      a1 += b1;
      a2 += b2;
      a3 += b3;
    }
  }
  group_sums<NT>(a0, a1, a2, a3);
  f0 = a0;
  f1 = a1;
  f2 = a2;
  f3 = a3;
}

// Largest entry of the LDS column and the lowest index holding it (an index
// below m for m >= 1, also when every entry is -inf).
template <class D, int NT = 64>
__device__ inline void wave_argmax(const D* s, int m, int lane, D& mx, int& idx) {
  D best = -num<D>::inf();
  int at = m;
  for (int i = lane; i < m; i += NT) {
    const D v = s[i];
    if (v > best || at == m) {
      best = v;
      at = i;
    }
  }
  mx = group_max<NT>(best);
  idx = group_min<NT>(best == mx ? at : m);
}

template <class R>
__device__ inline R log_w_inverse_or_min(R w) {
  // max(lambert_w_exp_inverse(w), exp_min_arg) (lambert.h:210-214, log_exp.h:27-52)
  const R v = w + dlog(w);
  return (v < num<R>::exp_min_arg()) ? num<R>::exp_min_arg() : v;
}

// One pass of the uncapped solve: the order-4 Householder step on
// g(t) = W(e^(alpha - t)) + sum_i W(e^(a_i - t)) - alpha
// (topk_entropy_biased.h:9-38), with [lo, hi] the root bracket narrowed by
// the sign of g(t); a step that leaves it becomes the Newton step, or the
// bisection when that leaves it too.  *s_out (if given) receives
// sum_i W(e^(a_i - t)) / alpha at the pass's t, as the reference's s.
// Returns false if g(t) or the step is not finite.
// ds_out (if given) receives the first two t-derivatives of that s with
// the sign of a step down in t: sum_i W / (1 + W) / alpha and
// sum_i W / (1 + W)^3 / alpha.
// noise_out (if given) is set when |g(t)| is within 16 ulps of the sum it
// is formed from: the step is then below what the sums' rounding resolves.
template <class D, class R, int NT = 64>
__device__ inline bool guarded_step(const D* s, int m, int lane, R alpha, R& t, R& lo, R& hi,
                                    R* s_out, R* wout = nullptr, R* ds_out = nullptr,
                                    bool* noise_out = nullptr) {
  R f0, f1, f2, f3;
  lw_sums4<D, R, NT>(s, m, lane, -t, f0, f1, f2, f3, -1, R(0), wout);
  if (s_out) *s_out = f0 / alpha;
  if (ds_out) {
    ds_out[0] = f1 / alpha;
    ds_out[1] = f2 / alpha;
  }
  {
    const R v = lambert_w_exp(alpha - t);
    const R d = R(1) + v;
    const R d3 = d * d * d;
    f0 += v;
    f1 += v / d;
    f2 += v / d3;
    f3 += v * (R(1) - R(2) * v) / (d3 * d * d);
  }
  if (noise_out) *noise_out = fabs(f0 - alpha) <= R(16) * num<R>::eps() * (fabs(f0) + alpha);
  f0 -= alpha;
  if (f0 > R(0)) lo = (t > lo) ? t : lo;
  else if (f0 < R(0)) hi = (t < hi) ? t : hi;
  const R f02 = f0 * f2, f11 = f1 * f1;
  const R den = R(6) * f1 * (f02 - f11) - f0 * (f0 * f3);
  R step = (fabs(den) > R(64) * num<R>::min_normal()) ? R(3) * f0 * (R(2) * f11 - f02) / den : R(0);
  R tn = t - step;
  // Inside the bracket, or a correction below the resolution of t.
  bool ok = isfinite(tn) && ((tn > lo && tn < hi) || (step != R(0) && tn == t));
  if (!ok) {
    step = (f1 > R(0)) ? -f0 / f1 : R(0);  // Newton: f1 = -g'(t)
    tn = t - step;
    ok = isfinite(tn) && ((tn > lo && tn < hi) || (step != R(0) && tn == t));
    if (!ok) tn = lo + (hi - lo) * R(0.5);
  }
  t = tn;
  return isfinite(f0) && isfinite(tn);
}

// Upper bound of the root of sum_i W(e^(x_i - t)) = rhs over the values
// x_i = s[i] + (i < p ? 0 : -c) (and the extra value e, if finite), and
// whether it is close: W(e^y) <= e^y, so the root lies at or below
// t_lse = log sum exp(x) - log(rhs), within about e^(max - t_lse) of it when
// every value sits below t_lse (small W, W(e^y) ~ e^y).  Single precision:
// a start for the iterations, which end on the root whatever their start.
template <class D, class R, int NT = 64>
__device__ inline bool lse_start(const D* s, int m, int p, R c, R e, R mx, R rhs, int lane,
                                 R& t_lse) {
  // the extra value once (by the group's first thread), the column's values
  // by their threads
  float se = (lane == 0 && e > -num<R>::inf()) ? expf(static_cast<float>(e - mx)) : 0.0f;
  for (int i = lane; i < m; i += NT)
    se += expf(static_cast<float>(static_cast<R>(s[i]) - (i < p ? R(0) : c) - mx));
  se = group_sum<NT>(se);
  t_lse = mx + static_cast<R>(logf(se)) - dlog(rhs);
  return mx - t_lse <= R(-1);
}

// The series start of a Lambert-map solve over the column s[0, m) and the
// extra value e (if finite), with mx the largest of them: where every value
// sits at least 3 below the log-sum-exp bound t_lse of sum W(e^(x - t)) =
// rhs, every argument at the root is at most ~0.05 and
// sum W(e^(x - t)) = sum_k c_k S_k u^k (u = e^(mx - t), S_k the power sums
// of e^(x - mx), W's series c = 1, -1, 3/2, -8/3, 125/24); t0 is the root
// of that five-term model by Newton in u from rhs / S_1, within ~11 u^5
// (relative) of the true one (as lds_solve_sum_w_exp in prox_impl.hpp).
// Returns whether the start applies.
template <class D, class R, int NT = 64>
__device__ inline bool series_start(const D* s, int m, R e, R mx, R rhs, int lane, R& t0) {
  float s1 = 0.0f, s2 = 0.0f, s3 = 0.0f, s4 = 0.0f, s5 = 0.0f;
  auto add = [&](float v) {
    const float v2 = v * v;
    s1 += v;
    s2 += v2;
    s3 += v2 * v;
    s4 += v2 * v2;
    s5 += v2 * (v2 * v);
  };
  if (lane == 0 && e > -num<R>::inf()) add(expf(static_cast<float>(e - mx)));
  for (int i = lane; i < m; i += NT) add(expf(static_cast<float>(static_cast<R>(s[i]) - mx)));
  group_sums<NT>(s1, s2, s3, s4, s5);
  const R t_lse = mx + static_cast<R>(logf(s1)) - dlog(rhs);
  if (!(mx - t_lse <= R(-3))) return false;
  const R S1 = s1, S2 = s2, S3 = s3, S4 = s4, S5 = s5;
  R u = rhs / S1;
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const R g = u * (S1 + u * (-S2 + u * (R(1.5) * S3 + u * (R(-8.0 / 3.0) * S4 +
                                                             u * (R(125.0 / 24.0) * S5))))) - rhs;
    const R gp = S1 + u * (R(-2) * S2 + u * (R(4.5) * S3 + u * (R(-32.0 / 3.0) * S4 +
                                                                  u * (R(625.0 / 24.0) * S5))));
    u -= g / gp;
  }
  t0 = mx - dlog(u);
  return isfinite(t0);
}

// W(e^x) for x whose e^x is at most ~0.06: the series value corrected by
// the reference's order-5 step (lambert.h:31-42), exact to double rounding.
__device__ inline double lambert_w_exp_small(double x) {
  const double z = exp_fast(x);
  const double w0 = lambert_w_series5(z);
  return lw_step5(w0, z * exp_neg_small(w0));
}

// Thresholds (t, 0, hi) of one column whose copy is in s[0, m); entries of U
// are overwritten with -inf.  With wl (the wave's LDS array of R), the last
// pass's W values are left there and *tw receives the t they were taken at.
// NOISE_STOP (the epoch's solves): the uncapped iteration also ends once
// g(t) is at the rounding level of its sums (the reference's test, a step
// of at most epsilon, then waits for t to stop moving between neighbouring
// floats, which takes several more passes and lands within that level too).
template <class D, class R, int NT = 64, bool NOISE_STOP = false>
__device__ void entbias_thresholds(D* s, int m, int lane, int k, R alpha, R& t_out,
                                   R& hi_out, R* wl = nullptr, R* tw = nullptr,
                                   int* branch = nullptr) {
  const R eps_r = num<R>::eps();
  const R tiny = R(64) * num<R>::min_normal();
  D mx_d;
  int mx_i;
  wave_argmax<D, NT>(s, m, lane, mx_d, mx_i);
  R max = static_cast<R>(mx_d);
  const R eps = R(16) * eps_r * (max > R(1) ? max : R(1));

  // U empty: Householder on alpha_sum_w_exp (topk_entropy_biased.h:9-61),
  // from the reference's start t = max with its steps and stopping test.
  // g(t) = W(e^(alpha - t)) + sum_i W(e^(a_i - t)) - alpha is convex and
  // decreasing with its root in [-log alpha, log((e^alpha + m e^max) / alpha)]
  // (W(e^x) <= e^x), and every pass narrows that bracket by the sign of g.
  // A step that leaves the bracket is replaced by the Newton step, or by
  // bisection when that leaves it too.  Far below the root the order-4
  // correction can point the wrong way; the reference then wanders and, if it
  // has not come back within its 32 steps, returns an iterate that is not a
  // root (and that depends on the rounding of its sums).  Steps inside the
  // bracket are the reference's own, so wherever the reference settles both
  // reach the same root; elsewhere this solve still reaches it, within 64
  // passes.
  R sv(0), t(max);
  R br_lo = -dlog(alpha), br_hi;
  {
    const R top = (alpha > max) ? alpha : max;
    br_hi = top + dlog(dexp(alpha - top) + static_cast<R>(m) * dexp(max - top)) - dlog(alpha);
  }
  // Where every value lies well below the log-sum-exp bound, the iteration
  // starts there (one single-precision pass instead of about three from
  // t = max on U(-10, 10) columns); the bracket is kept as it is.
  // The epoch's solves (NOISE_STOP) start there whenever it lies inside the
  // bracket: an upper bound of the root, nearer to it than t = max on their
  // columns (about three passes instead of five).
  {
    R t_lse;
    const R top = (alpha > max) ? alpha : max;
    const bool close = lse_start<D, R, NT>(s, m, m, R(0), alpha, top, alpha, lane, t_lse);
    if (close && t_lse > br_lo && t_lse < br_hi) {
      t = t_lse;
    } else if (NOISE_STOP && t_lse > br_lo) {
      t = (t_lse < br_hi) ? t_lse : br_hi;  // equal values put t_lse on br_hi
    }
  }
  bool warm = false;
  bool solved = false;
  if constexpr (sizeof(R) == 8 && NT == 64) {
    // Series start (every value, alpha included, at least 3 below the
    // log-sum-exp bound, as on U(-10, 10) columns): one double pass at the
    // series root t0 with every W from the series and the order-5 step,
    // then the order-4 Householder step; accepted when it stays inside the
    // bracket and moves t by at most 3e-5 (the next correction is then below
    // 1e-18).  s at t0 is carried to the final t by its Taylor series, as
    // after the warm start below.
    const R top = (alpha > max) ? alpha : max;
    R t0;
    if (wl && series_start<D, R, NT>(s, m, alpha, top, alpha, lane, t0) && t0 > br_lo &&
        t0 < br_hi) {
      R f0 = 0, f1 = 0, f2 = 0, f3 = 0;
      for (int i = lane; i < m; i += NT) {
        const R w = lambert_w_exp_small(static_cast<R>(s[i]) - t0);
        wl[i] = w;
        R b1, b2, b3;
        lw_terms(w, b1, b2, b3);
        f0 += w;
        f1 += b1;
        f2 += b2;
        f3 += b3;
      }
      group_sums<NT>(f0, f1, f2, f3);
      const R s0 = f0 / alpha, d0 = f1 / alpha, d1 = f2 / alpha;
      const R v = lambert_w_exp_small(alpha - t0);
      R b1, b2, b3;
      lw_terms(v, b1, b2, b3);
      const R g = f0 + v - alpha;
      const R g1 = f1 + b1, g2 = f2 + b2, g3 = f3 + b3;
      const R g02 = g * g2, g11 = g1 * g1;
      const R t1 = t0 - R(3) * g * (R(2) * g11 - g02) / (R(6) * g1 * (g02 - g11) - g * (g * g3));
      if (isfinite(t1) && t1 > br_lo && t1 < br_hi &&
          fabs(t1 - t0) <= R(3e-5) * dmax(R(1), fabs(t1))) {
        const R dt = t1 - t0;
        sv = s0 - dt * d0 + R(0.5) * dt * dt * d1;
        if (tw) *tw = t0;
        t = t1;
        solved = true;
      }
    }
  }
  if constexpr (sizeof(R) == 8) {
    // The same guarded iteration in single precision first (a Lambert pass
    // costs about a third): it ends once a step moves t by at most 3e-3
    // (relative), where the next order-4 correction is below single
    // precision, and the double loop then starts within ~1e-7 of the root
    // and needs one or two passes instead of about five.  Its estimate is
    // used only if it ended so.
    float tf = static_cast<float>(t);
    float lo_f = static_cast<float>(br_lo), hi_f = static_cast<float>(br_hi);
    const float alpha_f = static_cast<float>(alpha);
    bool settled = false;
    for (int iter = 0; iter < 16 && !settled && !solved; ++iter) {
      const float t1 = tf;
      bool ok = guarded_step<D, float, NT>(s, m, lane, alpha_f, tf, lo_f, hi_f, nullptr);
      settled = ok && fabsf(t1 - tf) <= 3.0e-3f * fmaxf(1.0f, fabsf(tf));
    }
    if (settled) t = static_cast<R>(tf);
    warm = settled;
  }
  for (int iter = 0; iter < 64 && !solved; ++iter) {
    const R t1 = t;
    if (tw) *tw = t;
    R ds[2];
    bool noise = false;
    const bool ok = guarded_step<D, R, NT>(s, m, lane, alpha, t, br_lo, br_hi, &sv, wl, ds,
                                           NOISE_STOP ? &noise : nullptr);
    if (fabs(t1 - t) <= eps_r) break;
    if (NOISE_STOP && ok && noise) break;
    // From a settled single-precision start a first step of at most 1e-6
    // leaves an order-4 correction of ~1e-24: the confirming pass is
    // skipped, and s (the pass's sum at t1) is carried to the final t by its
    // Taylor series (third-order term ~1e-18 s).
    if (warm && ok && iter == 0 && fabs(t1 - t) <= R(1e-6) * dmax(R(1), fabs(t))) {
      const R dt = t - t1;
      sv += -dt * ds[0] + R(0.5) * dt * dt * ds[1];
      break;
    }
  }
  const R K = static_cast<R>(k);
  t_out = t;
  if (branch) *branch = SDCA_BRANCH_U_EMPTY;
  if (k == 1) {
    hi_out = sv;
    return;
  }
  const R alpha_k = alpha / K;
  R tt = t + log_w_inverse_or_min(alpha_k * sv);
  if (max - eps <= tt) {
    hi_out = sv / K;
    return;
  }
  if (branch) *branch = SDCA_BRANCH_U_GROWN;

  // U not empty (topk_entropy_biased.h:224-266).
  if (lane == 0) s[mx_i] = -num<D>::inf();
  group_lds_sync<NT>();
  const R log_k = dlog(K), log_alpha = dlog(alpha);
  R min_u(max), sum_u(max);
  int num_u = 1;
  for (int remaining = m - 1; remaining > 0;) {
    wave_argmax<D, NT>(s, m, lane, mx_d, mx_i);
    max = static_cast<R>(mx_d);
    sv = R(0.999);
    t = max;
    {  // Newton on the KKT system (topk_entropy_biased.h:64-176)
      const R U = static_cast<R>(num_u);
      const R C1 = U * K, C2 = (K + U) * alpha, C3 = (K - U) * (U - R(1)) * alpha;
      const R C4 = K * (U - R(1)), C5 = (R(1) - U / K) * alpha;
      const R C0 = C4 * log_alpha - C1 * log_k - sum_u;
      const R tol = R(16) * eps_r;
      for (int iter = 0; iter < 32; ++iter) {
        const R s1 = sv, t1 = t;
        sv = (sv < R(0)) ? R(0) : ((sv > R(1)) ? R(1) : sv);
        R S0, S1;
        if (tw) *tw = t;
        lw_sums2<D, R, NT>(s, m, lane, -t, S0, S1, wl);
        const R E = S0 + t * S1;
        R z, Az, Bz;
        if (sv < R(0.5)) {
          z = sv;
          Az = K * (z * (U + dlog1p(-z) + z / (R(1) - z)) - U * x_log_x(z)) - C0 * z;
          Bz = z * (C2 + K / (R(1) - z)) + C1;
        } else {
          z = R(1) - sv;
          Az = K * (z * (U - U * dlog1p(-z) - R(1)) + x_log_x(z) + R(1)) - C0 * z;
          Bz = z * (C2 + C1 / (R(1) - z)) + K;
        }
        const R Dz = C3 * z - Bz * S1;
        if (fabs(Dz) > tiny) {
          sv = (C4 * E * z - Az * S1) / Dz;
          t = (C5 * Az - E * Bz) / Dz;
        }
        if (fabs(s1 - sv) + fabs(t1 - t) <= tol) break;
      }
      sv = (sv < R(0)) ? R(0) : ((sv > R(1)) ? R(1) : sv);
    }
    tt = t + log_w_inverse_or_min(alpha_k * sv);
    if (max - eps <= tt && tt <= min_u + eps) break;
    if (++num_u > k) break;
    min_u = max;
    sum_u += max;
    if (lane == 0) s[mx_i] = -num<D>::inf();
    group_lds_sync<NT>();
    --remaining;
  }
  t_out = t;
  hi_out = sv / K;
}

// One order-4 Householder step on the two-block sum (two_entropy.h:15-38);
// returns f(t) at the old t.
// win / wdt: as for lw_sums4 (the previous pass's W, taken at t - wdt).
template <class D, class R, int NT = 64>
__device__ inline R two_w_step4(const D* s, int m, int p, int lane, R alpha, R c, R& t,
                                R* wout = nullptr, const R* win = nullptr, R wdt = R(0)) {
  R f0, f1, f2, f3;
  lw_sums4<D, R, NT>(s, m, lane, -t, f0, f1, f2, f3, p, -t - c, wout, win, wdt);
  f0 -= alpha;
  const R f02 = f0 * f2, f11 = f1 * f1;
  const R den = R(6) * f1 * (f02 - f11) - f0 * (f0 * f3);
  if (fabs(den) > R(64) * num<R>::min_normal()) t -= R(3) * f0 * (R(2) * f11 - f02) / den;
  return f0;
}

// The reference's bisection count, static_cast<std::size_t>(log(ub - lb) /
// log 2) capped at 32, with the conversion as the reference's x86-64 build
// performs it: truncation toward zero, and a value at or below -1 (or NaN)
// wrapping to a huge count, hence 32.
template <class R>
__device__ inline int bisection_count(R v) {
  if (!(v > R(-1))) return 32;
  if (v >= R(32)) return 32;
  return (v > R(0)) ? static_cast<int>(v) : 0;
}

// Thresholds t (block a) and t + c (block b) of one column in s[0, m), split p.
// With wl, the last pass's W values are left there and *tw receives its t.
// NOISE_STOP: as for entbias_thresholds, the Householder steps also end
// once f(t) is at the rounding level of its sums.
template <class D, class R, int NT = 64, bool NOISE_STOP = false>
__device__ void twoent_thresholds(const D* s, int m, int p, int lane, R alpha, R& t_out,
                                  R& c_out, R* wl = nullptr, R* tw = nullptr) {
  const R eps = num<R>::eps();
  const R num_a = static_cast<R>(p), num_b = static_cast<R>(m - p);
  R max_a = -num<R>::inf(), max_b = -num<R>::inf(), sum_a = 0, sum_b = 0;
  for (int i = lane; i < m; i += NT) {
    const R x = static_cast<R>(s[i]);
    if (i < p) {
      max_a = (x > max_a) ? x : max_a;
      sum_a += x;
    } else {
      max_b = (x > max_b) ? x : max_b;
      sum_b += x;
    }
  }
  max_a = group_max<NT>(max_a);
  max_b = group_max<NT>(max_b);
  group_sums<NT>(sum_a, sum_b);
  const R c = alpha / num_a;
  const R max = (max_a > max_b - c) ? max_a : max_b - c;
  // Bracket guards (two_entropy.h:159-163).
  R lb = -num<R>::max_finite();
  R ub = max - R(64) * num<R>::exp_min_arg();
  R lf = num<R>::max_finite();
  R uf = -num<R>::max_finite();
  R t, t1, f1;
  // Where every value lies well below the log-sum-exp bound, the steps below
  // start there (two or three passes on U(-10, 10) columns instead of the
  // reference's two guesses and its bisection); they end on the same root.
  R t_lse;
  if (lse_start<D, R, NT>(s, m, p, c, -num<R>::inf(), max, alpha, lane, t_lse)) {
    t = t_lse;
  } else {
    // Two guesses, each followed by one step (:165-175).
    R t01 = max - dlog(alpha);
    t1 = t01;
    f1 = two_w_step4<D, R, NT>(s, m, p, lane, alpha, c, t1);
    R t02 = (sum_a + sum_b - num_b * c - alpha) / (num_a + num_b);
    R t2 = t02;
    R f2 = two_w_step4<D, R, NT>(s, m, p, lane, alpha, c, t2);
    if (f1 > f2) {
      R x = t01; t01 = t02; t02 = x;
      x = t1; t1 = t2; t2 = x;
      x = f1; f1 = f2; f2 = x;
    }
    if (f1 > R(0)) {
      lb = t01;
      lf = f1;
      t = t1;
    } else if (f2 < R(0)) {
      ub = t02;
      uf = f2;
      t = t2;
    } else {
      lb = t02;
      ub = t01;
      lf = f2;
      uf = f1;
      const R g = (fabs(f1) < fabs(f2)) ? t1 : t2;
      t = (lb > ((g < ub) ? g : ub)) ? lb : ((g < ub) ? g : ub);
      // Bisection (:75-96, 193-203).
      const int num_iter = bisection_count(dlog(ub - lb) * static_cast<R>(1.4426950408889634));
      for (int iter = 0; iter < num_iter; ++iter) {
        t = (lb + ub) / R(2);
        const R fv = lw_sum0<D, R, NT>(s, m, p, lane, -t, -t - c) - alpha;
        if (eps < fv && fv < lf) {
          lf = fv;
          lb = t;
        } else if (uf < fv && fv < -eps) {
          uf = fv;
          ub = t;
        } else {
          break;
        }
      }
      t = (lb + ub) / R(2);
    }
  }
  // Householder steps kept inside the bracket (:207-220).  With wl, a pass
  // whose t moved by at most lw_shift_max from the previous pass's takes its
  // W values by the Taylor step from that pass's (left in wl).
  bool have_w = false;
  R t_w = 0;
  for (int iter = 0; iter < 32; ++iter) {
    t1 = t;
    if (tw) *tw = t;
    const bool shift = have_w && fabs(t1 - t_w) <= lw_shift_max<R>();
    f1 = two_w_step4<D, R, NT>(s, m, p, lane, alpha, c, t, wl, shift ? wl : nullptr, t1 - t_w);
    have_w = wl != nullptr;
    t_w = t1;
    if (R(0) <= f1 && f1 < lf) {
      lb = t1;
      lf = f1;
    } else if (uf < f1 && f1 <= R(0)) {
      ub = t1;
      uf = f1;
    }
    t = (lb > ((t < ub) ? t : ub)) ? lb : ((t < ub) ? t : ub);
    if (fabs(t1 - t) <= eps) break;
    if (NOISE_STOP && fabs(f1) <= R(16) * eps * (fabs(f1 + alpha) + alpha)) break;
  }
  t_out = t;
  c_out = c;
}

}  // namespace sdca_gpu

#endif
