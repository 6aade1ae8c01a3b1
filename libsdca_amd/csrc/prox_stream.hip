// Columns above the 128 KiB that any kernel stages in LDS: one workgroup of
// kStreamThreads per column, the column read from global memory on every
// pass (it stays in the L2 / MALL between passes), thread i taking the
// entries i, i + kStreamThreads, ... so each pass is a coalesced sweep.
//
// The operators whose thresholds come from sweeps alone: the knapsack
// (knapsack_eq.h:25-109, knapsack_le.h:17-44: Kiwiel's variable fixing)
// and the entropic projections (entropy.h:19-53, entropy_norm.h:84-181).
// Their fixed sets are value cuts, as in the reference's partitions: the
// knapsack's working set is the interval (w_lo, w_hi] of values (a fixing
// step fixes every value beyond the step's cut), and the entropic fixed set
// is every value above the smallest cut so far.  The predicates, epsilons,
// starting points and stopping rules are those of the register kernels
// (knapsack_eq_regs, ent_family and lds_solve_sum_w_exp in prox_impl.hpp),
// with the sums taken in the sweep's order.
#include "common.hpp"
#include "prox_impl.hpp"
#include "prox_launch.hpp"

namespace sdca_gpu {

namespace {

constexpr int kStreamThreads = 1024;
enum StreamOp { SK_KNAP_EQ = 0, SK_KNAP_LE = 1, SK_ENT = 2, SK_ENT_NORM = 3 };

template <class D, class R>
struct Column {
  const D* x;
  int64_t m;
  __device__ R at(int64_t i) const { return static_cast<R>(x[i]); }
};

// Kiwiel's variable fixing (knapsack_eq.h:25-109) over the column's values
// in (w_lo, w_hi]; returns the threshold applied, recomputed from the final
// free set (the register kernels' t_acc), and the final counts at hi and
// free in n_u_out, n_f_out.
template <class D, class R>
__device__ R stream_knapsack_eq(const Column<D, R>& col, R lo, R hi, R rhs, int64_t& n_u_out,
                                int64_t& n_f_out) {
  constexpr int G = kStreamThreads;
  const int tid = static_cast<int>(threadIdx.x);
  const int64_t m = col.m;
  const R eps = num<R>::eps() * dmax(R(1), fabs(rhs));
  R total = 0;
  for (int64_t i = tid; i < m; i += G) total += col.at(i);
  total = group_sum<G>(total);
  R w_lo = -num<R>::inf(), w_hi = num<R>::inf();
  int64_t mc = m, n_u = 0;
  R t = div_near(total - rhs, static_cast<R>(mc));
  for (int64_t iter = 0; iter <= m; ++iter) {
    const R c_lo = lo + t, c_hi = hi + t;
    R s_lo = 0, s_hi = 0;
    int n_lo = 0, n_hi = 0;
    for (int64_t i = tid; i < m; i += G) {
      const R x = col.at(i);
      const bool in = x > w_lo && !(x > w_hi);
      const bool l = in && x <= c_lo, h = in && x > c_hi;
      s_lo += l ? x : R(0);
      s_hi += h ? x : R(0);
      n_lo += l ? 1 : 0;
      n_hi += h ? 1 : 0;
    }
    group_sums<G>(s_lo, s_hi, n_lo, n_hi);
    const R sh = static_cast<R>(n_hi) * hi, sl = static_cast<R>(n_lo) * lo;
    const R infeas = s_hi + s_lo - (sh + sl) - static_cast<R>(n_hi + n_lo) * t;
    const bool fix_hi = n_hi > 0 && infeas > eps;
    const bool fix_lo = !fix_hi && n_lo > 0 && infeas < -eps;
    if (!fix_hi && !fix_lo) {
      n_u += n_hi;
      const int64_t n_f = mc - n_lo - n_hi;
      n_u_out = n_u;
      n_f_out = n_f;
      if (n_f <= 0) return t;
      R s_f = 0;
      for (int64_t i = tid; i < m; i += G) {
        const R x = col.at(i);
        s_f += (x > w_lo && !(x > w_hi) && x > c_lo && !(x > c_hi)) ? x : R(0);
      }
      s_f = group_sum<G>(s_f);
      const int64_t n_l = m - n_u - n_f;
      return div_near(s_f + static_cast<R>(n_u) * hi + static_cast<R>(n_l) * lo - rhs,
                      static_cast<R>(n_f));
    }
    R next;
    if (fix_hi) {
      w_hi = dmin(w_hi, c_hi);
      next = static_cast<R>(mc) * t - s_hi + sh;
      mc -= n_hi;
      n_u += n_hi;
    } else {
      w_lo = dmax(w_lo, c_lo);
      next = static_cast<R>(mc) * t - s_lo + sl;
      mc -= n_lo;
    }
    if (mc <= 0) break;
    t = div_near(next, static_cast<R>(mc));
  }
  n_u_out = n_u;
  n_f_out = 0;
  return t;
}

// Largest value not above w_hi, the count of entries equal to it, and
// sum exp(x - max) over the other entries not above w_hi: log_sum_exp with
// one maximum excluded (math/log_exp.h:134-152).
template <class D, class R>
__device__ void stream_lse_excl(const Column<D, R>& col, R w_hi, R& mx, R& s) {
  constexpr int G = kStreamThreads;
  const int tid = static_cast<int>(threadIdx.x);
  R lm = -num<R>::inf();
  for (int64_t i = tid; i < col.m; i += G) {
    const R x = col.at(i);
    lm = (!(x > w_hi) && x > lm) ? x : lm;
  }
  mx = group_max<G>(lm);
  R ls = 0;
  int nmax = 0;
  for (int64_t i = tid; i < col.m; i += G) {
    const R x = col.at(i);
    if (!(x > w_hi)) {
      if (x == mx) ++nmax;
      else ls += dexp(x - mx);
    }
  }
  group_sums<G>(ls, nmax);
  s = ls + static_cast<R>(nmax - 1);
}

template <class D, class R>
__device__ R stream_max(const Column<D, R>& col, R w_hi) {
  R lm = -num<R>::inf();
  for (int64_t i = threadIdx.x; i < col.m; i += kStreamThreads) {
    const R x = col.at(i);
    lm = (!(x > w_hi) && x > lm) ? x : lm;
  }
  return group_max<kStreamThreads>(lm);
}

// One sweep of W(exp(x - tc)) and its first three derivatives over the
// entries not above w_hi (entropy_norm.h:84-102); SERIES: each W from the
// series start and one order-5 step (every argument at most ~0.05).
template <class D, class R, class T, bool SERIES>
__device__ void stream_w_sums(const Column<D, R>& col, R w_hi, T tc, T& f0, T& f1, T& f2,
                              T& f3) {
  f0 = f1 = f2 = f3 = T(0);
  for (int64_t i = threadIdx.x; i < col.m; i += kStreamThreads) {
    const R xr = col.at(i);
    if (!(xr > w_hi)) {
      T w;
      if constexpr (SERIES) {
        const T z = exp_fast(static_cast<T>(xr) - tc);
        const T w0 = lambert_w_series5(z);
        w = lw_step5(w0, z * exp_neg_small(w0));
      } else {
        w = lambert_w_exp(static_cast<T>(xr) - tc);
      }
      const T rd = div_near(T(1), T(1) + w);
      const T rd2 = rd * rd;
      const T rd3 = rd2 * rd;
      f0 += w;
      f1 += w * rd;
      f2 += w * rd3;
      f3 += w * (T(1) - T(2) * w) * (rd3 * rd2);
    }
  }
  group_sums<kStreamThreads>(f0, f1, f2, f3);
}

template <class T>
__device__ inline T householder4(T tc, T f0, T f1, T f2, T f3) {
  const T f02 = f0 * f2, f11 = f1 * f1;
  return tc - T(3) * f0 * (T(2) * f11 - f02) / (T(6) * f1 * (f02 - f11) - f0 * (f0 * f3));
}

// solve_sum_w_exp (entropy_norm.h:110-134) over the entries not above w_hi
// (count of them): the root t of sum W(exp(x - t)) = rhs, with the
// register kernel's starts (lds_solve_sum_w_exp).  *series is set when the
// root came from the series start (every W at the root then follows from
// the series and one step).
template <class D, class R>
__device__ R stream_solve_sum_w_exp(const Column<D, R>& col, R w_hi, int64_t count, R rhs,
                                    bool* series) {
  constexpr int G = kStreamThreads;
  const int tid = static_cast<int>(threadIdx.x);
  *series = false;
  const R mx = stream_max(col, w_hi);
  float se = 0.0f, s2 = 0.0f, s3 = 0.0f, s4 = 0.0f, s5 = 0.0f;
  for (int64_t i = tid; i < col.m; i += G) {
    const R x = col.at(i);
    const float e = !(x > w_hi) ? expf(static_cast<float>(x - mx)) : 0.0f;
    se += e;
    const float e2 = e * e;
    s2 += e2;
    s3 += e2 * e;
    s4 += e2 * e2;
    s5 += e2 * (e2 * e);
  }
  group_sums<G>(se, s2, s3, s4, s5);
  const R t_lse = mx + static_cast<R>(logf(se)) - dlog(rhs);
  R t = t_lse;
  bool started = false;
  if constexpr (sizeof(R) == 8) {
    if (mx - t_lse <= R(-3)) {  // the series start of lds_solve_sum_w_exp
      const R S1 = se, S2 = s2, S3 = s3, S4 = s4, S5 = s5;
      R u = rhs / S1;
      for (int it = 0; it < 4; ++it) {
        const R g =
            u * (S1 + u * (-S2 + u * (R(1.5) * S3 + u * (R(-8.0 / 3.0) * S4 +
                                                         u * (R(125.0 / 24.0) * S5))))) - rhs;
        const R gp = S1 + u * (R(-2) * S2 + u * (R(4.5) * S3 + u * (R(-32.0 / 3.0) * S4 +
                                                                      u * (R(625.0 / 24.0) * S5))));
        u -= g / gp;
      }
      const R t0 = mx - dlog(u);
      R f0, f1, f2, f3;
      stream_w_sums<D, R, R, true>(col, w_hi, t0, f0, f1, f2, f3);
      const R t1 = householder4(t0, f0 - rhs, f1, f2, f3);
      if (isfinite(t1) && fabs(t1 - t0) <= R(3e-5) * dmax(R(1), fabs(t1))) {
        *series = true;
        return t1;
      }
      if (isfinite(t1)) {
        t = t1;
        started = true;
      }
    }
  }
  if (!started && !(mx - t_lse <= R(-1))) {
    // The reference's start (entropy_norm.h:119-131): the mean, then the
    // mean over U = {x > t} while U shrinks and stays non-empty.
    R s = 0;
    for (int64_t i = tid; i < col.m; i += G) {
      const R x = col.at(i);
      s += !(x > w_hi) ? x : R(0);
    }
    s = group_sum<G>(s);
    t = (s - rhs) / static_cast<R>(count);
    R u_cut = -num<R>::inf();
    int64_t u_count = count;
    for (int64_t it = 0; it < count + 1; ++it) {
      R su = 0;
      int cu = 0;
      for (int64_t i = tid; i < col.m; i += G) {
        const R x = col.at(i);
        const bool in = !(x > w_hi) && x > u_cut && x > t;
        su += in ? x : R(0);
        cu += in ? 1 : 0;
      }
      group_sums<G>(su, cu);
      if (cu == u_count || cu == 0) break;
      u_cut = dmax(u_cut, t);
      u_count = cu;
      t = (su - rhs) / static_cast<R>(cu);
    }
  }
  const R ub = mx - num<R>::exp_min_arg();
  const R eps16 = R(16) * num<R>::eps();
  bool warm = false;
  if constexpr (sizeof(R) == 8) {
    // Single-precision steps first, used only if they settle.
    float tf = static_cast<float>(t);
    const float ubf = static_cast<float>(ub);
    bool settled = false;
    for (int iter = 0; iter < 4; ++iter) {
      const float prev = tf;
      const float tc = fminf(tf, ubf);
      float f0 = 0, f1 = 0, f2 = 0, f3 = 0;
      for (int64_t i = tid; i < col.m; i += G) {
        const R x = col.at(i);
        if (!(x > w_hi)) {
          const float w = lambert_w_exp(static_cast<float>(x) - tc);
          const float rd = div_near(1.0f, 1.0f + w);
          const float rd2 = rd * rd;
          const float rd3 = rd2 * rd;
          f0 += w;
          f1 += w * rd;
          f2 += w * rd3;
          f3 += w * (1.0f - 2.0f * w) * (rd3 * rd2);
        }
      }
      group_sums<G>(f0, f1, f2, f3);
      tf = householder4(tc, f0 - static_cast<float>(rhs), f1, f2, f3);
      if (!(fabsf(tf) <= 3.0e38f)) break;
      if (fabsf(prev - tf) <= 3.0e-3f * fmaxf(1.0f, fabsf(tf))) {
        settled = true;
        break;
      }
    }
    if (settled) t = static_cast<R>(tf);
    warm = settled;
  }
  for (int iter = 0; iter < 32; ++iter) {
    const R prev = t;
    const R tc = dmin(t, ub);
    R f0, f1, f2, f3;
    stream_w_sums<D, R, R, false>(col, w_hi, tc, f0, f1, f2, f3);
    t = householder4(tc, f0 - rhs, f1, f2, f3);
    if (fabs(prev - t) <= eps16) break;
    if (warm && iter == 0 && fabs(prev - t) <= R(1e-6) * dmax(R(1), fabs(t))) break;
  }
  return t;
}

template <int OPK, class D, class R>
__global__ void __launch_bounds__(kStreamThreads)
stream_kernel(const D* __restrict__ in, D* __restrict__ out, int64_t m, int64_t n,
              ProxParamsT<R> pp, sdca_thresholds* __restrict__ thr,
              sdca_prox_sets* __restrict__ sets) {
  constexpr int G = kStreamThreads;
  const int tid = static_cast<int>(threadIdx.x);
  for (int64_t j = blockIdx.x; j < n; j += gridDim.x) {
    const Column<D, R> col{in + j * m, m};
    D* const y = out + j * m;
    R t = 0, lo = pp.lo, hi = pp.hi;
    bool series = false;
    int64_t set_hi = 0, set_mid = 0;
    int branch = SDCA_BRANCH_SEARCH;
    if constexpr (OPK == SK_KNAP_EQ || OPK == SK_KNAP_LE) {
      bool active = true;
      if constexpr (OPK == SK_KNAP_LE) {
        // knapsack_le.h:17-44: the sum constraint is inactive unless the
        // clamped values exceed rhs.
        const R eps = num<R>::eps() * dmax(R(1), fabs(pp.rhs));
        R s_mid = 0;
        int n_hi = 0, n_mid = 0;
        for (int64_t i = tid; i < m; i += G) {
          const R x = col.at(i);
          if (x >= hi) ++n_hi;
          else if (x > lo) { s_mid += x; ++n_mid; }
        }
        group_sums<G>(s_mid, n_hi, n_mid);
        const int64_t n_lo = m - n_hi - n_mid;
        const R s = s_mid + hi * static_cast<R>(n_hi) + lo * static_cast<R>(n_lo);
        active = s > pp.rhs + eps;
        branch = active ? SDCA_BRANCH_KNAPSACK : SDCA_BRANCH_INACTIVE;
        set_hi = n_hi;
        set_mid = n_mid;
      }
      if (active) t = stream_knapsack_eq(col, lo, hi, pp.rhs, set_hi, set_mid);
    } else {
      // entropy.h:30-49, entropy_norm.h:157-178
      constexpr bool NORM = OPK == SK_ENT_NORM;
      lo = R(0);
      const R rhs = pp.rhs;
      const R eps = R(16) * num<R>::eps() * dmax(R(1), rhs);
      const R u = NORM ? hi + dlog(hi) + eps : dlog(hi) + eps;
      R r = rhs;
      R w_hi = num<R>::inf();  // entries above it are fixed at hi
      int64_t nfixed = 0;
      if constexpr (!NORM) {
        R mx, s;
        stream_lse_excl(col, w_hi, mx, s);
        t = mx + dlog1p(s) - dlog(r);
      }
      for (int64_t iter = 0; iter <= m; ++iter) {
        if constexpr (NORM) {
          t = stream_solve_sum_w_exp(col, w_hi, m - nfixed, r, &series);
        } else if (iter > 0) {
          R mx, s;
          stream_lse_excl(col, w_hi, mx, s);
          t = mx + dlog1p(s) - dlog(r);
        }
        const R cut = t + u;
        int cnt = 0;
        for (int64_t i = tid; i < m; i += G) {
          const R x = col.at(i);
          cnt += (!(x > w_hi) && x > cut) ? 1 : 0;
        }
        cnt = group_sum<G>(cnt);
        if (cnt == 0) break;
        series = false;
        w_hi = dmin(w_hi, cut);
        r -= hi * static_cast<R>(cnt);
        nfixed += cnt;
        if (nfixed == m) break;
        if (r <= eps) {
          t = stream_max(col, w_hi) - num<R>::exp_min_arg() + R(1);
          break;
        }
      }
      set_hi = nfixed;
      set_mid = m - nfixed;
    }
    // The clamp / map pass (proxdef.h:164-196), t, lo, hi cast to Data.
    const D td = static_cast<D>(t), lod = static_cast<D>(lo), hid = static_cast<D>(hi);
    for (int64_t i = tid; i < m; i += G) {
      const D x = col.x[i];
      D v;
      if constexpr (OPK == SK_ENT) {
        v = dexp(x - td);
      } else if constexpr (OPK == SK_ENT_NORM) {
        if constexpr (sizeof(R) == 8 && sizeof(D) == 8) {
          if (series) {
            // every argument is in the series' range at this root
            const double z = exp_fast(static_cast<double>(x) - static_cast<double>(t));
            const double w0 = lambert_w_series5(z);
            v = lw_step5(w0, z * exp_neg_small(w0));
          } else {
            v = lambert_w_exp(x - td);
          }
        } else {
          v = lambert_w_exp(x - td);
        }
      } else {
        v = x - td;
      }
      y[i] = clamp_ref(v, lod, hid);
    }
    if (thr && tid == 0) {
      thr[j].t = static_cast<double>(t);
      thr[j].lo = static_cast<double>(lo);
      thr[j].hi = static_cast<double>(hi);
    }
    if (sets && tid == 0) sets[j] = sdca_prox_sets{set_hi, set_mid, branch, 0};
    __syncthreads();  // the next column's sweeps reuse the reduction scratch
  }
}

template <int OPK, class D, class R>
hipError_t launch_t(const ProxLaunch& a) {
  ProxParamsT<R> pp;
  pp.lo = static_cast<R>(a.lo);
  pp.hi = static_cast<R>(a.hi);
  pp.rhs = static_cast<R>(a.rhs);
  pp.rho = R(0);
  pp.k = 1;
  pp.op = a.op;
  pp.p = 0;
  const int64_t grid = a.n < 8192 ? a.n : 8192;
  hipLaunchKernelGGL((stream_kernel<OPK, D, R>), dim3(static_cast<unsigned>(grid)),
                     dim3(kStreamThreads), 0, a.stream, static_cast<const D*>(a.in),
                     static_cast<D*>(a.out), a.m, a.n, pp, a.thr, a.sets);
  return hipGetLastError();
}

template <int OPK>
hipError_t launch_types(const ProxLaunch& a) {
  if (a.data == SDCA_F32 && a.result == SDCA_F32) return launch_t<OPK, float, float>(a);
  if (a.data == SDCA_F32 && a.result == SDCA_F64) return launch_t<OPK, float, double>(a);
  if (a.data == SDCA_F64 && a.result == SDCA_F64) return launch_t<OPK, double, double>(a);
  if (a.data == SDCA_F64 && a.result == SDCA_F32) return launch_t<OPK, double, float>(a);
  return hipErrorInvalidValue;
}

}  // namespace

bool stream_supported(int op) {
  return op == OP_KNAPSACK_EQ || op == OP_KNAPSACK_LE || op == OP_ENTROPY ||
         op == OP_ENTROPY_NORM;
}

hipError_t launch_stream(const ProxLaunch& a) {
  if (a.n == 0) return hipSuccess;
  switch (a.op) {
    case OP_KNAPSACK_EQ: return launch_types<SK_KNAP_EQ>(a);
    case OP_KNAPSACK_LE: return launch_types<SK_KNAP_LE>(a);
    case OP_ENTROPY: return launch_types<SK_ENT>(a);
    case OP_ENTROPY_NORM: return launch_types<SK_ENT_NORM>(a);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace sdca_gpu
