// Batched column prox kernels for gfx950 (one template, five operator
// families).  Replaces the batch loop prox(dim, first, last, aux, ...)
// (proxdef.h:279-324) of libsdca v0.3.1.
//
// Layout.  The input is an m x n column-major matrix; columns are contiguous.
// A one-wave workgroup owns B = 64 / G consecutive columns: it copies their
// B*m contiguous elements into LDS with 16-byte loads (fully coalesced), then
// each group of G adjacent lanes takes one column, lane g holding elements
// g, g+G, g+2G, ... in C registers (slots past m hold -inf, which every pass
// below ignores by construction).  Thresholds are found in registers with
// group reductions over the G lanes; the clamp/map result goes back through
// LDS and out with 16-byte stores.  HBM traffic is one read and one write of
// the matrix.
//
// Semantics.  Each family restates the reference algorithm on register
// values: the same threshold formulas, the same case tests and epsilons and
// the same arithmetic type (Result R) for every quantity, with the partitions
// of the reference expressed as value cuts (a partition by `x > c` keeps a
// set {x > cut}).  Sums run in a different order than the reference's
// std::accumulate, so thresholds agree to rounding.  Columns whose case needs
// the reference's full sort (topk_cone_search with |U| > 0, ties at zero,
// k beyond the register list) are flagged into a list that the
// workgroup-per-column kernel in prox_slow.hip finishes.
#ifndef SDCA_HIP_PROX_IMPL_HPP
#define SDCA_HIP_PROX_IMPL_HPP

#include "common.hpp"
#include "prox_launch.hpp"

namespace sdca_gpu {

enum Family { FAM_KNAP = 0, FAM_TOPK = 1, FAM_ENT = 2, FAM_TOPKENT = 3, FAM_TWO = 4 };

template <class R>
struct ProxParamsT {
  R lo, hi, rhs;
  R rhs_k;  // rhs / k in R, formed once on the host (the top-k simplex's upper bound)
  R rho;  // biased operators only (0 for the others)
  int k;
  int op;
  int p;
};

// Result of the threshold search for one column.
template <class R>
struct ColThr {
  R t, lo, hi;     // first (or only) block
  R t2, lo2, hi2;  // second block (two-block operator)
  int kind;        // elementwise map of the clamp: 0 identity, 1 exp, 2 W(exp)
  bool slow;       // column deferred to the workgroup-per-column kernel
  // The record's sets (sdca_prox_sets) and the branch that produced it:
  // n_hi < 0 leaves them to be counted from the column by the record's cuts
  // (x > t + hi at hi, x > t + lo free); n_mid2 is block b's free count (its
  // n_hi is 0).
  int branch;
  int n_hi, n_mid, n_mid2;
};

template <class R>
__device__ inline ColThr<R> make_thr(R t, R lo, R hi, int kind = 0) {
  ColThr<R> r;
  r.t = t; r.lo = lo; r.hi = hi;
  r.t2 = t; r.lo2 = lo; r.hi2 = hi;
  r.kind = kind;
  r.slow = false;
  r.branch = SDCA_BRANCH_SEARCH;
  r.n_hi = -1;
  r.n_mid = 0;
  r.n_mid2 = 0;
  return r;
}

// r with its branch and, when n_hi >= 0, its sets.
template <class R>
__device__ inline ColThr<R> tag_thr(ColThr<R> r, int branch, int n_hi = -1, int n_mid = 0) {
  r.branch = branch;
  r.n_hi = n_hi;
  r.n_mid = n_mid;
  return r;
}

template <class R>
__device__ inline ColThr<R> slow_thr() {
  ColThr<R> r = make_thr<R>(R(0), R(0), R(0));
  r.slow = true;
  return r;
}

// Sum of the valid slots (padding, and excluded slots, hold -inf).
template <int G, int C, class D, class R>
__device__ inline R total_sum(const D (&v)[C], int nvalid) {
  R s = 0;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const R x = static_cast<R>(v[c]);
    s += (c < nvalid && x > -num<R>::inf()) ? x : R(0);
  }
  return group_sum<G>(s);
}

// ---------------------------------------------------------------------------
// Kiwiel variable fixing (knapsack_eq.h:25-109).  The free set of the
// reference is the value interval (lo_cut, hi_cut]: fixing the upper
// candidates {x > hi + t} lowers hi_cut, fixing the lower candidates
// {x <= lo + t} raises lo_cut.  On exit the final candidates are folded into
// the fixed sets exactly as the reference's last partition does.
// ---------------------------------------------------------------------------
template <class R>
struct KnapState {
  R t;               // the iteration's last t (knapsack_eq.h:79-84): branch tests use it
  R t_acc;           // t recomputed from the final free set (the threshold applied)
  R lo_cut, hi_cut;  // fixed sets: x <= lo_cut at lo, x > hi_cut at hi
  R c_lo, c_hi;      // final candidate cuts inside the free interval
  int n_u;           // |U| = number at hi (fixed + final candidates)
  R sum_u;           // sum over U
  int n_f;           // |F| = number free at the end
};

// The fixing may start with the n_u0 values above hi_cut0 (sum sum_u0)
// already at the upper bound, when those are known to end there; the
// iteration is then Kiwiel's on the remaining problem.
//
// Each lane keeps a working copy w of its slots in which every fixed value
// (and padding) is NaN: both candidate tests (w <= lo + t, w > hi + t) are
// false for NaN, so a slot costs two compares and the fixing of a set is one
// select.  The low and high counts travel in one integer (n_lo + 2^16 n_hi;
// at most m <= 2048 each) through the group sum.
//
// WL: the working copy lives in the column's own LDS slots (wl = the lane's
// first slot, slot c at wl[G c]; padding slots are neither read nor written,
// their stores go to the lane's dummy word) instead of C more registers.
// The caller must not need the LDS copy of the column afterwards.
template <int G, int C, class D, class R, bool WL = false>
__device__ inline KnapState<R> knapsack_eq_regs(const D (&v)[C], int m, int nvalid, R total,
                                                R lo, R hi, R rhs, R hi_cut0 = num<R>::inf(),
                                                int n_u0 = 0, R sum_u0 = 0, D* wl = nullptr,
                                                D* wl_dummy = nullptr) {
  const R eps = num<R>::eps() * dmax(R(1), fabs(rhs));
  const R qnan = num<R>::quiet_nan();
  R w[WL ? 1 : C];
  constexpr int UW = WL ? 1 : C;  // the LDS loops stay rolled (their registers are the point)
  auto get = [&](int c) -> R {
    if constexpr (WL) {
      const R x = static_cast<R>(wl[G * c]);
      return c < nvalid ? x : qnan;
    } else {
      return w[c];
    }
  };
  auto put = [&](int c, R x) {
    if constexpr (WL) {
      D* dst = c < nvalid ? wl + G * c : wl_dummy;
      *dst = static_cast<D>(x);
    } else {
      w[c] = x;
    }
  };
  int mc = m - n_u0;
  R t = div_near(total - sum_u0 - rhs + static_cast<R>(n_u0) * hi, static_cast<R>(mc));
  R t_acc = t;
  bool have_acc = false;
  int n_f = 0;
  KnapState<R> st;
  st.lo_cut = -num<R>::inf();
  st.hi_cut = hi_cut0;
  st.c_lo = -num<R>::inf();
  st.c_hi = num<R>::inf();
  st.n_u = n_u0;
  st.sum_u = sum_u0;
#pragma unroll UW
  for (int c = 0; c < C; ++c) {
    const R x = static_cast<R>(v[c]);
    put(c, (x > -num<R>::inf() && !(x > hi_cut0)) ? x : qnan);
  }
  for (int iter = 0; iter <= m; ++iter) {
    const R c_lo = lo + t, c_hi = hi + t;
    R s_lo = 0, s_hi = 0;
    int n_lh = 0;
#pragma unroll UW
    for (int c = 0; c < C; ++c) {
      const R wc = get(c);
      const bool lo_c = wc <= c_lo;
      const bool hi_c = wc > c_hi;
      s_lo += lo_c ? wc : R(0);
      s_hi += hi_c ? wc : R(0);
      n_lh += (lo_c ? 1 : 0) + (hi_c ? 0x10000 : 0);
    }
    group_sums<G>(s_lo, s_hi, n_lh);
    const int n_lo = n_lh & 0xffff, n_hi = n_lh >> 16;
    const R sh = static_cast<R>(n_hi) * hi;
    const R sl = static_cast<R>(n_lo) * lo;
    const R infeas = s_hi + s_lo - (sh + sl) - static_cast<R>(n_hi + n_lo) * t;
    const bool fix_hi = n_hi > 0 && infeas > eps;
    const bool fix_lo = !fix_hi && n_lo > 0 && infeas < -eps;
    if (!fix_hi && !fix_lo) {
      st.c_lo = c_lo;
      st.c_hi = c_hi;
      st.n_u += n_hi;
      st.sum_u += s_hi;
      n_f = mc - n_lo - n_hi;
      break;
    }
    R next;
    if (fix_hi) {
      st.hi_cut = dmin(st.hi_cut, dmax(c_lo, c_hi));
      next = static_cast<R>(mc) * t - s_hi + sh;
      mc -= n_hi;
      st.n_u += n_hi;
      st.sum_u += s_hi;
    } else {
      st.lo_cut = dmax(st.lo_cut, c_lo);
      next = static_cast<R>(mc) * t - s_lo + sl;
      mc -= n_lo;
    }
#pragma unroll UW
    for (int c = 0; c < C; ++c) {
      const R wc = get(c);
      const bool fixed = fix_hi ? (wc > c_hi) : (wc <= c_lo);
      put(c, fixed ? qnan : wc);
    }
    if (mc > 0) {
      t = div_near(next, static_cast<R>(mc));
    } else {
      break;
    }
  }
  // The iteration's t carries the rounding of its incremental updates
  // (m t - sum + n hi is a difference of large sums, then divided by the
  // shrinking free count: in float at m = 100 that is ~1e-5 of t).  The
  // threshold applied is formed once more from the final free set F (the
  // free values between the last pass's candidate cuts),
  // t = (sum_F a + |U| hi + |L| lo - rhs) / |F|, as the reference's
  // SDCA_ACCURATE_MATH build does (knapsack_eq.h:87-106, Lemma 5.3 of
  // Kiwiel's paper); the branch tests keep the iteration's t.  It runs once
  // after the loop, for every column of the wave together, rather than in
  // the pass where each column ends.  n_f is the same on every lane of a
  // group (it comes from group sums), so the group sum below sees its
  // whole group.
  if (n_f > 0) {
    R s_f = 0;
#pragma unroll UW
    for (int c = 0; c < C; ++c) {
      const R wc = get(c);
      s_f += (wc > st.c_lo && !(wc > st.c_hi)) ? wc : R(0);
    }
    s_f = group_sum<G>(s_f);
    const int n_l = m - st.n_u - n_f;
    t_acc = div_near(s_f + static_cast<R>(st.n_u) * hi + static_cast<R>(n_l) * lo - rhs,
                     static_cast<R>(n_f));
    have_acc = true;
  }
  st.t = t;
  st.t_acc = have_acc ? t_acc : t;
  st.n_f = n_f;
  return st;
}

// The root of t / rho = sum_i clamp(a_i - t, lo, hi): the solution of
// knapsack_le_biased_search (knapsack_le_biased.h:10-92) when the sum
// constraint is inactive.  That search walks the sorted column for the
// partition (U at hi, M inside, L at lo) with
//   t = (lo |L| + hi |U| + sum_M a) / (1 / rho + |M|);
// here the partition comes from variable fixing as in knapsack_eq_regs (the
// left side is increasing in t, so a positive clamp excess at the trial t
// means the root is below it and the values above hi + t end at hi; a
// negative one fixes those at lo).  Each trial t is formed as above from the
// sum over the values still free, not updated from the previous one: that
// keeps the large fixed values out of the final sum, as the reference's
// sum over M does.
template <int G, int C, class D, class R>
__device__ inline R knapsack_biased_regs(const D (&v)[C], int m, R total, R lo, R hi, R rhs,
                                         R rho_inv) {
  const R eps = num<R>::eps() * dmax(R(1), fabs(rhs));
  const R qnan = num<R>::quiet_nan();
  int n_l = 0, n_u = 0;
  R s_free = total;
  R w[C];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const R x = static_cast<R>(v[c]);
    w[c] = (x > -num<R>::inf()) ? x : qnan;
  }
  R t = 0;
  for (int iter = 0; iter <= m; ++iter) {
    const int n_m = m - n_l - n_u;
    t = (lo * static_cast<R>(n_l) + hi * static_cast<R>(n_u) + s_free) /
        (rho_inv + static_cast<R>(n_m));
    if (n_m == 0) break;
    const R c_lo = lo + t, c_hi = hi + t;
    R s_lo = 0, s_hi = 0;
    int n_lh = 0;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const bool lo_c = w[c] <= c_lo;
      const bool hi_c = w[c] > c_hi;
      s_lo += lo_c ? w[c] : R(0);
      s_hi += hi_c ? w[c] : R(0);
      n_lh += (lo_c ? 1 : 0) + (hi_c ? 0x10000 : 0);
    }
    group_sums<G>(s_lo, s_hi, n_lh);
    const int n_lo = n_lh & 0xffff, n_hi = n_lh >> 16;
    const R infeas = s_hi + s_lo - (static_cast<R>(n_hi) * hi + static_cast<R>(n_lo) * lo) -
                     static_cast<R>(n_hi + n_lo) * t;
    const bool fix_hi = n_hi > 0 && infeas > eps;
    const bool fix_lo = !fix_hi && n_lo > 0 && infeas < -eps;
    if (!fix_hi && !fix_lo) break;
    R sf = 0;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const bool fixed = fix_hi ? (w[c] > c_hi) : (w[c] <= c_lo);
      w[c] = fixed ? qnan : w[c];
      sf += (w[c] == w[c]) ? w[c] : R(0);
    }
    s_free = group_sum<G>(sf);
    if (fix_hi) n_u += n_hi;
    else n_l += n_lo;
  }
  return t;
}

// ---------------------------------------------------------------------------
// Knapsack family: knapsack_eq (knapsack_eq.h:25-109) and knapsack_le
// (knapsack_le.h:17-44).
// ---------------------------------------------------------------------------
template <int G, int C, class D, class R>
__device__ inline ColThr<R> knap_family(const D (&v)[C], int m, int nvalid,
                                        const ProxParamsT<R>& pp) {
  const R lo = pp.lo, hi = pp.hi, rhs = pp.rhs;
  // knapsack_le_biased with rho = 0 is knapsack_le (knapsack_le_biased.h:113-115).
  const bool biased = pp.op == OP_KNAPSACK_LE_BIASED && pp.rho != R(0);
  if (pp.op == OP_KNAPSACK_LE || (pp.op == OP_KNAPSACK_LE_BIASED && !biased)) {
    const R eps = num<R>::eps() * dmax(R(1), fabs(rhs));
    R s_mid = 0;
    int n_hi = 0, n_mid = 0;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const R x = static_cast<R>(v[c]);
      if (x >= hi) ++n_hi;
      else if (x > lo) { s_mid += x; ++n_mid; }
    }
    group_sums<G>(s_mid, n_hi, n_mid);
    const int n_lo = m - n_hi - n_mid;
    const R s = s_mid + hi * static_cast<R>(n_hi) + lo * static_cast<R>(n_lo);
    if (!(s > rhs + eps)) return tag_thr(make_thr<R>(R(0), lo, hi), SDCA_BRANCH_INACTIVE, n_hi, n_mid);
  }
  const R total = total_sum<G, C, D, R>(v, nvalid);
  KnapState<R> st = knapsack_eq_regs<G, C, D, R>(v, m, nvalid, total, lo, hi, rhs);
  if (biased) {
    // knapsack_le_biased.h:117-128: the equality solution stands if
    // t >= rho rhs - eps; otherwise the sum constraint is inactive.
    const R eps = num<R>::eps() * dmax(R(1), fabs(rhs));
    if (!(st.t >= pp.rho * rhs - eps))
      return tag_thr(make_thr<R>(knapsack_biased_regs<G, C, D, R>(v, m, total, lo, hi, rhs,
                                                                  R(1) / pp.rho),
                                 lo, hi),
                     SDCA_BRANCH_SCAN);
  }
  return tag_thr(make_thr<R>(st.t_acc, lo, hi),
                 pp.op == OP_KNAPSACK_EQ ? SDCA_BRANCH_SEARCH : SDCA_BRANCH_KNAPSACK, st.n_u,
                 st.n_f);
}

// ---------------------------------------------------------------------------
// Top-k family: topk_cone (topk_cone.h:18-157) and topk_simplex
// (topk_simplex.h:9-68).  The k largest values come from a sorted register
// list of KM + 1 entries per lane (median-of-three insertion), merged across
// the group; k <= KM.
// ---------------------------------------------------------------------------
// topk_cone_search (topk_cone.h:58-133) when the answer has U empty: then
// t = 0 exactly, M = {x > 16 eps} and hi = k sum(M) / k^2; valid if
// hi >= max(M) - 16 eps.  Any other outcome (U non-empty, or values within
// 16 eps of zero that the reference may place in M) goes to the slow path.
template <int G, int C, class D, class R>
__device__ inline ColThr<R> cone_search_u0(const D (&v)[C], R K, R largest) {
  const R eps16 = R(16) * num<R>::eps();
  R s_p = 0;
  int n_p = 0, n_z = 0;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const R x = static_cast<R>(v[c]);
    const bool pos = x > eps16;
    s_p += pos ? x : R(0);
    n_p += pos ? 1 : 0;
    n_z += (!pos && x >= -eps16) ? 1 : 0;
  }
  group_sums<G>(s_p, n_p, n_z);
  if (n_z > 0) return slow_thr<R>();
  const R den = K * K;
  const R t = (R(0) * s_p - K * R(0)) / den;
  const R hi = (R(0) + K * s_p) / den;
  const R max_m = (n_p > 0) ? largest : -num<R>::inf();
  const R tt = hi + t;
  if (max_m - eps16 <= tt) return tag_thr(make_thr<R>(t, R(0), hi), SDCA_BRANCH_SCAN, 0, n_p);
  return slow_thr<R>();
}

// thresholds_topk_cone_biased_search (topk_cone_biased.h:9-80) on the sorted
// top list: the reference's scan over U = the u largest and M = the next
// ones, with its incremental sums in its order, so each trial t and hi are
// the reference's values.
//
// For a given U the scan takes M = top[u, e) for growing e and accepts the
// first e whose t satisfies the four conditions, among them t <= min(M) + eps.
// Each step moves t to a weighted mean of t and the entry added,
//   t' = (D t + nu a_e) / (D + nu),
// so once t >= min(M) it stays there, and for any M reaching past the list,
//   t' - min(M) >= D (t - top[L-1]) / (D + (m - L) nu)
// with t and D taken at the end of the list.  When that bound clears eps
// (plus rounding) no M beyond the list can be accepted, and the scan goes on
// to the next U as the reference's would; otherwise the column is deferred.
//
// The scans for different U are independent: lane g of the group runs
// u = g, g + G, ... (setting up sum_U, k - |U| and |U| + rho k^2 by the
// reference's own sequence of updates), and the outcome is that of the
// smallest u whose scan accepts or cannot be certified.
template <int G, int L, class D, class R>
__device__ inline ColThr<R> cone_biased_regs(const D (&top)[L], int m, int k, R rho) {
  const R eps = R(16) * num<R>::eps();
  const int g = static_cast<int>(threadIdx.x) % G;
  int found_u = k + 1;
  int found_kind = 0;  // 1: accepted, 2: deferred
  int found_e = 0;     // M = top[u, e)
  R found_t = 0, found_hi = 0;
#pragma unroll 1
  for (int u = g; u <= k; u += G) {
    R k_u = static_cast<R>(k);
    R nu_rho = rho * static_cast<R>(k) * static_cast<R>(k);
    R min_u = num<R>::inf();
    R sum_u = 0;
#pragma unroll
    for (int i = 0; i < L; ++i) {
      if (i < u) {
        min_u = static_cast<R>(top[i]);
        sum_u += min_u;
        k_u -= R(1);
        nu_rho += R(1);
      }
    }
    R min_m = num<R>::inf(), max_m = -num<R>::inf();
    R sum_m = 0, num_m_sum_u = 0;
    R den = k_u * k_u;
    const R k_u_sum_u = k_u * sum_u;
    int kind = 0, re = u;
    R rt = 0, rhi = 0;
#pragma unroll 1
    for (int e = u;; ++e) {  // M = top[u, e)
      const R t = (nu_rho * sum_m - k_u_sum_u) / den;
      const R hi = (num_m_sum_u + k_u * sum_m) / den;
      const R tt = hi + t;
      const bool pass = max_m - eps <= tt && tt <= min_u + eps && t <= min_m + eps;
      if (e == m) {
        if (pass) { kind = 1; rt = t; rhi = hi; re = e; }
        break;
      }
      if (e >= L) {
        if (pass) { kind = 2; break; }  // the last test needs top[e]
        const R last = static_cast<R>(top[L - 1]);
        const R tol = R(2) * eps + R(8) * num<R>::eps() * dmax(fabs(t), fabs(last));
        if (!(den * (t - last) > tol * (den + static_cast<R>(m - L) * nu_rho))) kind = 2;
        break;
      }
      if (pass && static_cast<R>(top[e]) - eps <= t) { kind = 1; rt = t; rhi = hi; re = e; break; }
      min_m = static_cast<R>(top[e]);
      max_m = static_cast<R>(top[u]);
      sum_m += min_m;
      num_m_sum_u += sum_u;
      den += nu_rho;
    }
    if (kind != 0) {
      found_u = u;
      found_kind = kind;
      found_t = rt;
      found_hi = rhi;
      found_e = re;
      break;
    }
  }
  const int u_min = group_min<G>(found_u);
  if (u_min > k)  // the reference's default
    return tag_thr(make_thr<R>(R(0), R(0), R(0)), SDCA_BRANCH_DEFAULT, 0, 0);
  const int src = (static_cast<int>(threadIdx.x) & 63) - g + u_min % G;
  const int kind = __shfl(found_kind, src, 64);
  if (kind == 2) return slow_thr<R>();
  return tag_thr(make_thr<R>(__shfl(found_t, src, 64), R(0), __shfl(found_hi, src, 64)),
                 SDCA_BRANCH_SCAN, u_min, __shfl(found_e, src, 64) - u_min);
}

// Candidate slots per lane for the top-k simplex's knapsack: the group holds
// up to G * kCandSlots<G> candidates in registers; columns with more run the
// variable fixing over all register slots instead.
template <int G>
constexpr int kCandSlots = (G <= 2) ? 8 : (G <= 4) ? 4 : (G <= 16) ? 2 : 1;

// Lane J's value of a quad (the group of four lanes a lane belongs to).
template <int J, class T>
__device__ inline T quad_lane(T v) {
  if constexpr (sizeof(T) == 8) {
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(b & 0xffffffffll), J * 0x55,
                                               0xF, 0xF, true);
    const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(b >> 32), J * 0x55, 0xF, 0xF,
                                               true);
    return __longlong_as_double((static_cast<long long>(hi) << 32) |
                                static_cast<long long>(static_cast<unsigned>(lo)));
  } else {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(0, __float_as_int(v), J * 0x55, 0xF, 0xF, true));
  }
}

// max(a, b) where bound is +inf, min(a, b) where it is -inf.
__device__ inline float max_or_min(float a, float b, float bound) {
  return __builtin_amdgcn_fmed3f(a, b, bound);
}
__device__ inline double max_or_min(double a, double b, double bound) {
  return (bound > 0) ? ((a < b) ? b : a) : ((b < a) ? b : a);
}

// Descending bitonic sort of the N = G * CC values of a group of G = 4
// lanes (a quad), element i = g CC + c in slot c of lane g: strides
// below CC exchange slots of a lane, strides CC and 2 CC exchange lanes by
// quad permutations.  Every compare-exchange keeps the larger value at the
// lower index where its block sorts descending, the smaller where it sorts
// ascending (Batcher's network); a lane's direction is the same for all its
// slots in each pass, so each exchange is one median with a bound of +inf
// (keep the larger) or -inf (keep the smaller).
template <int G, int CC, class D>
__device__ inline void group_sort_desc(D (&x)[CC], int g) {
  constexpr int N = G * CC;
  static_assert(G == 4, "quads");
  static_assert((CC & (CC - 1)) == 0, "slots a power of two");
  const D pinf = net_inf(D(0));
#pragma unroll
  for (int size = 2; size <= N; size <<= 1) {
#pragma unroll
    for (int stride = size / 2; stride > 0; stride >>= 1) {
      if (stride < CC) {
#pragma unroll
        for (int c = 0; c < CC; ++c) {
          if ((c & stride) == 0) {
            const bool desc = size == N || ((g * CC + c) & size) == 0;
            const D b = desc ? pinf : -pinf;
            const D lo = x[c], hi = x[c + stride];
            x[c] = max_or_min(lo, hi, b);
            x[c + stride] = max_or_min(lo, hi, -b);
          }
        }
      } else {
        const int lanes = stride / CC;  // 1 or 2: the partner is lane g ^ lanes
        const bool desc = size == N || ((g * CC) & size) == 0;
        const bool lower = (g & lanes) == 0;
        const D b = (lower == desc) ? pinf : -pinf;
#pragma unroll
        for (int c = 0; c < CC; ++c) {
          const D y = (lanes == 1) ? xor_lane<1>(x[c]) : xor_lane<2>(x[c]);
          x[c] = max_or_min(x[c], y, b);
        }
      }
    }
  }
}

// The exact root of the top-k simplex's knapsack from its sorted
// candidates, for groups of 4 lanes: the <= N = G * CC candidates (every
// value above a_(k) - hi - slack; the rest end at 0) at lds_col[0, total)
// are sorted descending across the group, a_0 >= a_1 >= ...  With
// f(t) = sum_i clamp(a_i - t, 0, hi), the root t* of f(t) = rhs has
// U = ranks [0, u) at hi, M = ranks [u, e) free and the rest at 0, where
//   * e is the first rank with f(a_e) >= rhs (a_e <= t*, f decreasing),
//     from prefix sums and the sorted top list every lane holds, each lane
//     testing its own ranks at once;
//   * u is the U count for which t_u = (sum_M a + u hi - rhs) / (e - u)
//     (t = (sum_F a + |U| hi + |L| lo - rhs) / |F|, knapsack_eq.h:87-106)
//     puts a_(u-1) at or above t_u + hi and a_u below it; u < k.
// That is the partition Kiwiel's variable fixing ends with
// (knapsack_eq.h:25-109), found with a fixed instruction count instead of a
// data-dependent number of passes (a wave pays for the slowest of its
// columns).  The sum over M is taken once more directly for the threshold
// applied.  Where M is empty (every one of the k largest at hi: f is flat
// at k hi over [a_k, a_(k-1) - hi]), any t of that interval gives the same
// projection; the record takes its midpoint.  The f tests allow eps
// (= eps max(1, |rhs|), the fixing's own tolerance) for the rounding of
// k hi against rhs.  Returns false, for the variable fixing to decide, when
// no u fits (ties with a threshold at rounding level), hi <= 0 or a value
// is not finite.
template <int G, int CC, int L, class D, class R>
__device__ inline bool topk_sorted_root(const D* lds_col, int total, const D (&top)[L], int k,
                                        R hi, R rhs, KnapState<R>& st) {
  constexpr int N = G * CC;
  const int g = static_cast<int>(threadIdx.x) % G;
  const R eps = num<R>::eps() * dmax(R(1), fabs(rhs));
  D x[CC];
#pragma unroll
  for (int c = 0; c < CC; ++c) {
    const int i = g * CC + c;
    const D v = lds_col[i];
    x[c] = (i < total) ? v : -num<D>::inf();
  }
  group_sort_desc<G, CC>(x, g);
  // Exclusive prefix sums: within the lane (ex), then the lanes before it
  // (base), every lane adding the lane totals in the same order.
  R ex[CC];
  R tot = 0;
#pragma unroll
  for (int c = 0; c < CC; ++c) {
    ex[c] = tot;
    tot += (g * CC + c < total) ? static_cast<R>(x[c]) : R(0);
  }
  const R t0 = quad_lane<0>(tot), t1 = quad_lane<1>(tot), t2 = quad_lane<2>(tot),
          t3 = quad_lane<3>(tot);
  const R base = (g >= 1 ? t0 : R(0)) + (g >= 2 ? t1 : R(0)) + (g >= 3 ? t2 : R(0));
  const R all = ((t0 + t1) + t2) + t3;
  // The f test on the lane's ranks; e = the first passing rank (ranks at or
  // past total hold the values below the cut, which pass).  With
  // f(a_r) = sum_{i<r} (a_i - a_r) - sum_{i<r} max(a_i - hi - a_r, 0), the
  // second sum runs over the values above a_r + hi: the k largest cover it
  // unless more than k values lie there, and then f(a_r) >= k hi passes
  // either way.
  R thj[L - 1];
#pragma unroll
  for (int j = 0; j < L - 1; ++j)
    thj[j] = (j < k) ? static_cast<R>(top[j]) - hi : -num<R>::inf();
  const R target = rhs - eps;
  int e = N;
#pragma unroll
  for (int c = CC - 1; c >= 0; --c) {
    const int r = g * CC + c;
    const R a = static_cast<R>(x[c]);
    R over = 0;
#pragma unroll
    for (int j = 0; j < L - 1; ++j) over += dmax(thj[j] - a, R(0));
    const R f = ((base + ex[c]) - static_cast<R>(r) * a) - over;
    const bool pass = r >= total || f >= target;
    e = pass ? r : e;
  }
  e = group_min<G>(e);
  if (e > total) e = total;
  // Prefix sums of the k largest from the top list: pk[j] = sum of top[0, j).
  R pk[L];
  pk[0] = 0;
#pragma unroll
  for (int j = 1; j < L; ++j) pk[j] = pk[j - 1] + static_cast<R>(top[j - 1]);
  // sum of ranks [0, e) and a_e: the owner lane's, summed over the group
  // (the other lanes give 0; a_e = -inf past the candidates).
  R pe = 0, ae = 0;
#pragma unroll
  for (int c = 0; c < CC; ++c) {
    const bool own = g * CC + c == e;
    pe = own ? base + ex[c] : pe;
    ae = own ? static_cast<R>(x[c]) : ae;
  }
  group_sums<G>(pe, ae);
  if (e >= N) {
    pe = all;
    ae = -num<R>::inf();
  }
  // u: the smallest U count whose t_u = num / (e - u) puts a_(u-1) at or
  // above t_u + hi and a_u below it (compared without the division).
  int u = -1;
#pragma unroll
  for (int j = L - 2; j >= 0; --j) {
    if (j < k && j < e) {
      const R den = static_cast<R>(e - j);
      const R num_j = (pe - pk[j]) + static_cast<R>(j) * hi - rhs;
      const bool above = j == 0 || (static_cast<R>(top[j > 0 ? j - 1 : 0]) - hi) * den >= num_j;
      const bool below = (static_cast<R>(top[j]) - hi) * den < num_j;
      u = (above && below) ? j : u;
    }
  }
  const bool usable = hi > 0 && static_cast<R>(top[0]) < num<R>::inf();
  st.lo_cut = -num<R>::inf();
  st.hi_cut = num<R>::inf();
  if (u >= 0) {
    // The threshold applied, from the sum over M taken directly; the sets
    // as value cuts (U = values above a_u, M = the rest above a_e).
    R sm = 0;
#pragma unroll
    for (int c = 0; c < CC; ++c) {
      const int r = g * CC + c;
      sm += (r >= u && r < e) ? static_cast<R>(x[c]) : R(0);
    }
    sm = group_sum<G>(sm);
    const R t = div_near(sm + static_cast<R>(u) * hi - rhs, static_cast<R>(e - u));
    R su = 0, au = 0;
#pragma unroll
    for (int j = 0; j < L - 1; ++j) {
      su = (j == u) ? pk[j] : su;
      au = (j == u) ? static_cast<R>(top[j]) : au;
    }
    st.t = t;
    st.t_acc = t;
    st.n_u = u;
    st.sum_u = su;
    st.c_hi = au;
    st.c_lo = ae;
    st.n_f = e - u;
    return usable;
  }
  // M empty: the k largest at hi, the rest (a_k = the largest of them) at 0.
  R kth = 0, ak = -num<R>::inf(), sk = 0;
#pragma unroll
  for (int j = 0; j < L; ++j) {
    kth = (j == k - 1) ? static_cast<R>(top[j]) : kth;
    ak = (j == k) ? static_cast<R>(top[j]) : ak;
    sk = (j == k) ? pk[j] : sk;
  }
  if (e == k && ak <= kth - hi) {
    const R t = (ak > -num<R>::inf()) ? R(0.5) * ak + R(0.5) * (kth - hi) : kth - hi;
    st.t = t;
    st.t_acc = t;
    st.n_u = k;
    st.sum_u = sk;
    st.c_hi = ak;
    st.c_lo = ak;
    st.n_f = 0;
    return usable;
  }
  return false;
}

// Variable fixing for the top-k simplex's knapsack (lo = 0, hi = rhs / k):
// its root t* satisfies sum_i clamp(a_i - t*, 0, hi) = k hi, hence
// a_(k) - hi <= t* < a_(k) (the k largest each give hi at t = a_(k) - hi;
// fewer than k can be positive at t = a_(k)).  Elements at or below a_(k) - hi
// end at the lower bound whatever the iteration does, so the fixing runs over
// the few values above that cut only.  The candidates are compacted through
// the column's LDS slots into kCandSlots registers per lane (candidate i to
// lane i % G), and the register variable fixing runs on them with group sums.
// The cut is widened by a few ulps so that rounding of hi = rhs / k cannot
// drop a contributor.  lds_col is scratch: the column's LDS words, slot c of
// lane g at lds_col[g + G c] for c < nvalid (nothing outside them is touched
// but the lane's own dummy word).  LDS_FALLBACK: when there are too many
// candidates for the registers, the fixing over every slot keeps its working
// copy in those LDS words (for callers where that case is rare and the
// registers set the occupancy) rather than in C more registers.
template <int G, int C, int L, class D, class R, bool LDS_FALLBACK>
__device__ inline KnapState<R> topk_knapsack(const D (&v)[C], const D (&top)[L], int m,
                                             int nvalid, int k, R kth, R hi, R rhs, D* lds_col,
                                             D* lds_dummy, bool lane_lists = false) {
  const R slack = (fabs(kth) + hi) * (R(16) * num<R>::eps());
  const R cut = kth - hi - slack;
  if constexpr (G > 1) {
    constexpr int CC = kCandSlots<G>;
    const int g = static_cast<int>(threadIdx.x) % G;
    // lane_lists: each lane's own top-L list (sorted, before the group
    // merge) sits at lds_col[g L, g L + L).  A lane whose L-th largest is at
    // or below the cut holds all its candidates there, as a prefix of the
    // list: they are counted and compacted from L words instead of C slots.
    D own[L];
    int cn = 0;
    bool from_lists = false;
    if (lane_lists) {
#pragma unroll
      for (int i = 0; i < L; ++i) {
        own[i] = lds_col[g * L + i];
        cn += (static_cast<R>(own[i]) > cut) ? 1 : 0;
      }
      from_lists = group_min<G>(static_cast<R>(own[L - 1]) > cut ? 0 : 1) == 1;
    }
    if (!from_lists) {
      cn = 0;
#pragma unroll
      for (int c = 0; c < C; ++c) cn += (static_cast<R>(v[c]) > cut) ? 1 : 0;
    }
    // A workgroup-wide group forms the candidates' sum in the same exchange
    // as their count (for the fixing over more candidates than registers,
    // below).
    R cand_wg = 0;
    int total;
    if constexpr (G > 64) {
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const R x = static_cast<R>(v[c]);
        cand_wg += (c < nvalid && x > cut) ? x : R(0);
      }
      total = cn;
      group_sums<G>(total, cand_wg);
    } else {
      total = group_sum<G>(cn);
    }
    if (total <= G * CC) {
      // Branch-free compaction: every slot is stored, non-candidates to the
      // lane's own dummy word (distinct per lane, so no bank serialisation).
      // (For a workgroup-wide group the scan's barriers also order these
      // stores after the other waves' reads of an earlier compaction.)  The
      // lists were read above, before these stores overwrite them.
      int pos = group_exclusive_scan<G>(cn, g);
      if (from_lists) {
#pragma unroll
        for (int i = 0; i < L; ++i) {
          D* dst = (i < cn) ? lds_col + pos + i : lds_dummy;
          *dst = own[i];
        }
      } else {
#pragma unroll
        for (int c = 0; c < C; ++c) {
          const bool pr = static_cast<R>(v[c]) > cut;
          D* dst = pr ? lds_col + pos : lds_dummy;
          *dst = v[c];
          pos += pr ? 1 : 0;
        }
      }
      group_lds_sync<G>();
      if constexpr (G == 4) {
        KnapState<R> st;
        if (topk_sorted_root<G, CC, L, D, R>(lds_col, total, top, k, hi, rhs, st)) return st;
      }
      // Candidate i sits at lds_col[i]; lane g takes i = g, g + G, ...  The
      // reads stay inside the tile: G * CC <= 16 <= m for G = 4 and 2, and
      // G * CC <= G <= m for larger G.
      D cand[CC];
      R csum = 0;
#pragma unroll
      for (int c = 0; c < CC; ++c) {
        const D x = lds_col[g + G * c];
        const bool ok = g + G * c < total;
        cand[c] = ok ? x : -num<D>::inf();
        csum += ok ? static_cast<R>(x) : R(0);
      }
      csum = group_sum<G>(csum);
      // Values at or above a_(k) + hi end at the upper bound (t* < a_(k)), so
      // the fixing starts with them fixed; they are among the k - 1 largest,
      // i.e. in the sorted top list every lane of the group holds.
      const R ucut = kth + hi + slack;
      int n_u0 = 0;
      R sum_u0 = 0;
#pragma unroll
      for (int i = 0; i < L; ++i) {
        const bool u = static_cast<R>(top[i]) > ucut;
        n_u0 += u ? 1 : 0;
        sum_u0 += u ? static_cast<R>(top[i]) : R(0);
      }
      return knapsack_eq_regs<G, CC, D, R>(cand, total, total, csum, R(0), hi, rhs, ucut, n_u0,
                                           sum_u0);
    }
    if constexpr (G > 64) {
      // More candidates than registers on a workgroup-wide group (the
      // epoch's columns): the same fixing over the candidates in their
      // slots, the others left out as padding (they end at the lower bound,
      // 0), and the upper values of the top list fixed at the start, as the
      // register path does; fewer passes than the fixing over every value.
      D w[C];
#pragma unroll
      for (int c = 0; c < C; ++c) w[c] = (static_cast<R>(v[c]) > cut) ? v[c] : -num<D>::inf();
      const R ucut = kth + hi + slack;
      int n_u0 = 0;
      R sum_u0 = 0;
#pragma unroll
      for (int i = 0; i < L; ++i) {
        const bool u = static_cast<R>(top[i]) > ucut;
        n_u0 += u ? 1 : 0;
        sum_u0 += u ? static_cast<R>(top[i]) : R(0);
      }
      return knapsack_eq_regs<G, C, D, R, LDS_FALLBACK>(
          w, total, nvalid, cand_wg, R(0), hi, rhs, ucut, n_u0, sum_u0,
          lds_col + static_cast<int>(threadIdx.x) % G, lds_dummy);
    }
  }
  const R all = total_sum<G, C, D, R>(v, nvalid);
  return knapsack_eq_regs<G, C, D, R, (LDS_FALLBACK && G > 1)>(
      v, m, nvalid, all, R(0), hi, rhs, num<R>::inf(), 0, R(0),
      lds_col + static_cast<int>(threadIdx.x) % G, lds_dummy);
}

// LDS_FALLBACK: the variable fixing over every slot (more candidates than
// the candidate registers hold) keeps its working copy in the column's LDS
// slots (the column kernels, whose registers set the occupancy) or in C
// registers (false: the epoch's single workgroup, where that case is common
// in the first epoch and registers are plentiful).
template <int G, int C, int KM, class D, class R, bool LDS_FALLBACK = true>
__device__ inline ColThr<R> topk_family(const D (&v)[C], int m, int nvalid,
                                        const ProxParamsT<R>& pp, D* lds_col, D* lds_dummy) {
  const int k = pp.k;
  const R K = static_cast<R>(k);
  const R eps16 = R(16) * num<R>::eps();
  constexpr int L = KM + 1;
  D top[L];
#pragma unroll
  for (int i = 0; i < L; ++i) top[i] = -num<D>::inf();
  if constexpr (L == 16 && C >= 16) {
    // The first 16 slots by a sorting network (80 max/min pairs), the rest
    // by insertion: 304 operations instead of 16 med3 for every slot.
#pragma unroll
    for (int i = 0; i < L; ++i) top[i] = v[i];
    bitonic_sort_desc<L>(top);
#pragma unroll
    for (int c = L; c < C; ++c) top_insert(top, v[c]);
  } else {
    top_fill<0>(top, v, net_inf(D(0)));  // -inf padding leaves it unchanged
  }
  // Groups of four lanes keep each lane's own list in the column's LDS words
  // (free once the slots are in registers) for the candidate compaction of
  // the knapsack below.
  const bool lane_lists = G == 4 && m >= G * L;
  if (lane_lists) {
    const int g = static_cast<int>(threadIdx.x) % G;
#pragma unroll
    for (int i = 0; i < L; ++i) lds_col[g * L + i] = top[i];
  }
  top_merge<G>(top);
  R sum_k = 0, kth = static_cast<R>(top[0]), next = -num<R>::inf();
#pragma unroll
  for (int i = 0; i < L; ++i) {
    if (i < k) sum_k += static_cast<R>(top[i]);
    if (i == k - 1) kth = static_cast<R>(top[i]);
    if (i == k) next = static_cast<R>(top[i]);
  }
  const R largest = static_cast<R>(top[0]);
  // topk_cone_special_cases (topk_cone.h:18-55), whose divisor is k, or
  // k + rho k^2 for the biased simplex (topk_simplex_biased.h:50-51).
  const bool biased = pp.op == OP_TOPK_SIMPLEX_BIASED || pp.op == OP_TOPK_CONE_BIASED;
  if (sum_k <= eps16) return tag_thr(make_thr<R>(R(0), R(0), R(0)), SDCA_BRANCH_ZERO, 0, 0);
  const R hi_c = sum_k / (biased ? K + pp.rho * K * K : K);
  const R t_c = kth - hi_c;
  const bool constant = (k == m) || (t_c >= next - eps16);
  if (pp.op == OP_TOPK_CONE) {
    if (constant) return tag_thr(make_thr<R>(t_c, R(0), hi_c), SDCA_BRANCH_CONSTANT, k, 0);
    return cone_search_u0<G, C, D, R>(v, K, largest);
  }
  if (pp.op == OP_TOPK_CONE_BIASED) {  // thresholds_topk_cone_biased (topk_cone_biased.h:98-113)
    if (constant) return tag_thr(make_thr<R>(t_c, R(0), hi_c), SDCA_BRANCH_CONSTANT, k, 0);
    return cone_biased_regs<G, L, D, R>(top, m, k, pp.rho);
  }
  // thresholds_topk_simplex (topk_simplex.h:39-68) and
  // thresholds_topk_simplex_biased (topk_simplex_biased.h:40-71)
  const R rhs = pp.rhs;
  const R eps = num<R>::eps() * dmax(R(1), fabs(rhs));
  if (constant && !(K * hi_c > rhs + eps))
    return tag_thr(make_thr<R>(t_c, R(0), hi_c), SDCA_BRANCH_CONSTANT, k, 0);
  const R hi = pp.rhs_k;  // rhs / K (topk_simplex.h:56)
  // More than G * kCandSlots candidates is rare for the prox inputs: the LDS
  // working copy keeps the kernel's register peak at the candidate path's.
  KnapState<R> st = topk_knapsack<G, C, L, D, R, LDS_FALLBACK>(v, top, m, nvalid, k, kth, hi,
                                                                rhs, lds_col, lds_dummy,
                                                                lane_lists);
  if (!constant) {
    // is_topk_simplex_lt (topk_simplex.h:9-27), is_topk_simplex_biased_lt
    // (topk_simplex_biased.h:9-28), over U = [first, t.first)
    bool lt;
    if (biased) {
      if (st.n_u == 0) {
        lt = st.t < pp.rho * rhs - eps;
      } else {
        const R num_u = static_cast<R>(st.n_u);
        lt = K * (st.sum_u + (K - num_u) * st.t) < rhs * (num_u + pp.rho * K * K) - eps;
      }
      // The biased cone search (topk_cone_biased.h:58-137) runs on the
      // sorted column in the workgroup-per-column kernel.
      if (lt) return slow_thr<R>();
    } else {
      if (st.n_u == 0) {
        lt = st.t < -eps;
      } else {
        const R num_u = static_cast<R>(st.n_u);
        lt = K * (st.sum_u + (K - num_u) * st.t) < rhs * num_u - eps;
      }
      if (lt) return cone_search_u0<G, C, D, R>(v, K, largest);
    }
  }
  return tag_thr(make_thr<R>(st.t_acc, R(0), hi), SDCA_BRANCH_KNAPSACK, st.n_u, st.n_f);
}

// ---------------------------------------------------------------------------
// log-sum-exp over the slots in `mask`, excluding exactly one maximum element
// (the first in lane/slot order), as log_sum_exp(first, last, max, s)
// (math/log_exp.h:134-152) excludes its `max` iterator.  Returns s.
// ---------------------------------------------------------------------------
template <int G, int C, class D, class R>
__device__ inline R lse_sum_excl(const D (&v)[C], const bool (&mask)[C], R mx) {
  int first_c = C;
#pragma unroll
  for (int c = C - 1; c >= 0; --c)
    if (mask[c] && static_cast<R>(v[c]) == mx) first_c = c;
  const int g = static_cast<int>(threadIdx.x) % G;
  const int owner = group_min<G>(first_c < C ? g : G);
  R s = 0;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const bool skip = (g == owner) && (c == first_c);
    if (mask[c] && !skip) s += dexp(static_cast<R>(v[c]) - mx);
  }
  return group_sum<G>(s);
}

template <int G, int C, class D, class R>
__device__ inline R masked_max(const D (&v)[C], const bool (&mask)[C]) {
  R mx = -num<R>::inf();
#pragma unroll
  for (int c = 0; c < C; ++c)
    if (mask[c]) mx = dmax(mx, static_cast<R>(v[c]));
  return group_max<G>(mx);
}

// ---------------------------------------------------------------------------
// Entropic family: entropy (entropy.h:19-53) and entropy_norm
// (entropy_norm.h:146-181), on the column's LDS copy.  Slot c of the lane is
// x[G c]; the free set is a bit mask over the lane's slots.  Every pass is a
// rolled loop that reads its slot from LDS: with C slots unrolled and held in
// registers, C exp / Lambert evaluations would be live at once (in double,
// more than 150 VGPRs and two waves per SIMD).
// ---------------------------------------------------------------------------
template <int C>
__device__ inline unsigned slot_bits(int nvalid) {
  return nvalid >= 32 ? 0xffffffffu : ((1u << nvalid) - 1u);
}

template <int G, int C, class D, class R>
__device__ inline R lds_masked_max(const D* x, unsigned bits) {
  R mx = -num<R>::inf();
#pragma unroll 4
  for (int c = 0; c < C; ++c) {
    const R y = static_cast<R>(x[G * c]);
    mx = (((bits >> c) & 1u) && y > mx) ? y : mx;
  }
  return group_max<G>(mx);
}

// sum of exp(x - mx) over the free slots except exactly one maximum element
// (the first in lane/slot order), as log_sum_exp(first, last, max, s)
// (math/log_exp.h:134-152) excludes its `max` iterator.
template <int G, int C, class D, class R>
__device__ inline R lds_lse_sum_excl(const D* x, unsigned bits, R mx) {
  int first_c = C;
#pragma unroll 4
  for (int c = C - 1; c >= 0; --c)
    first_c = (((bits >> c) & 1u) && static_cast<R>(x[G * c]) == mx) ? c : first_c;
  const int g = static_cast<int>(threadIdx.x) % G;
  const int owner = group_min<G>(first_c < C ? g : G);
  if (g == owner) bits &= ~(1u << first_c);
  R s = 0;
#pragma unroll 4
  for (int c = 0; c < C; ++c)
    if ((bits >> c) & 1u) s += dexp(static_cast<R>(x[G * c]) - mx);
  return group_sum<G>(s);
}

// solve_sum_w_exp (entropy_norm.h:110-134) over the free slots (count of
// them in the column).  With wl (the lane's slots of an LDS array of R), the
// last Householder pass leaves W(exp(x - tc)) of every free slot there and
// tc in *tw: the output map is then a short Taylor step from them.
template <int G, int C, class D, class R>
__device__ __forceinline__ R lds_solve_sum_w_exp(const D* x, unsigned bits, int count, R rhs,
                                                 R* wl = nullptr, R* tw = nullptr) {
  // Start.  W(e^y) <= e^y, so the root lies at or below
  // t_lse = log sum exp(x) - log(rhs), and within about e^(max - t_lse) of it
  // when every free value sits well below t_lse (small W, W(e^y) ~ e^y).
  // There the iteration starts from t_lse: one single-precision step settles
  // it on U(-10, 10) columns, against three from the reference's heuristic
  // start (below), which the other columns keep.  The root, and the
  // stopping rule that ends on it, are the same.
  const R mx = lds_masked_max<G, C, D, R>(x, bits);
  // sum_i e_i with e_i = exp(x_i - mx), and for a double Result the power
  // sums S_k = sum_i e_i^k, k = 2..5, of the series start below.
  float se = 0.0f, s2 = 0.0f, s3 = 0.0f, s4 = 0.0f, s5 = 0.0f;
#pragma unroll 4
  for (int c = 0; c < C; ++c) {
    const float e =
        ((bits >> c) & 1u) ? expf(static_cast<float>(static_cast<R>(x[G * c]) - mx)) : 0.0f;
    se += e;
    if constexpr (sizeof(R) == 8) {
      const float e2 = e * e;
      s2 += e2;
      s3 += e2 * e;
      s4 += e2 * e2;
      s5 += e2 * (e2 * e);
    }
  }
  if constexpr (sizeof(R) == 8) group_sums<G>(se, s2, s3, s4, s5);
  else se = group_sum<G>(se);
  const R t_lse = mx + static_cast<R>(logf(se)) - dlog(rhs);
  R t = t_lse;
  bool started = false;
  if constexpr (sizeof(R) == 8) {
    // Series start.  Where every value sits at least 3 below t_lse, every
    // argument z_i = exp(x_i - t) at the root is at most ~0.05, inside the
    // radius 1/e of W(z) = z - z^2 + 3/2 z^3 - 8/3 z^4 + 125/24 z^5 - ...
    // With u = exp(mx - t), sum_i W(z_i) = sum_k c_k S_k u^k: the root of
    // the five-term model (Newton in u from rhs / S_1, the log-sum-exp bound)
    // is within ~11 u^5 (relative) of the true one.  One double pass at that
    // t0 then evaluates every W(z_i) exactly (the series value corrected by
    // the reference's order-5 step, lambert.h:31-42, whose error after one
    // step is the fifth power of the series' ~1e-5) and the order-4
    // Householder step of entropy_norm.h:84-102 lands on the root to double
    // precision: one pass at ~80 instructions per element instead of a
    // single- and a double-precision Lambert pass (~190).  Other columns,
    // and a step larger than the start's error allows, take the general
    // path below; the root is the same.
    if (wl != nullptr && mx - t_lse <= R(-3)) {
      const R S1 = se, S2 = s2, S3 = s3, S4 = s4, S5 = s5;
      R u = rhs / S1;
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const R g =
            u * (S1 + u * (-S2 + u * (R(1.5) * S3 + u * (R(-8.0 / 3.0) * S4 +
                                                         u * (R(125.0 / 24.0) * S5))))) - rhs;
        const R gp = S1 + u * (R(-2) * S2 + u * (R(4.5) * S3 + u * (R(-32.0 / 3.0) * S4 +
                                                                      u * (R(625.0 / 24.0) * S5))));
        u -= g / gp;
      }
      const R t0 = mx - dlog(u);
      R f0 = 0, f1 = 0, f2 = 0, f3 = 0;
#pragma unroll 1
      for (int c = 0; c < C; ++c) {
        if ((bits >> c) & 1u) {
          const R z = exp_fast(static_cast<R>(x[G * c]) - t0);
          const R w0 = lambert_w_series5(z);
          const R w = lw_step5(w0, z * exp_neg_small(w0));
          wl[G * c] = w;
          const R rd = div_near(R(1), R(1) + w);
          const R rd2 = rd * rd;
          const R rd3 = rd2 * rd;
          f0 += w;
          f1 += w * rd;
          f2 += w * rd3;
          f3 += w * (R(1) - R(2) * w) * (rd3 * rd2);
        }
      }
      group_sums<G>(f0, f1, f2, f3);
      f0 -= rhs;
      const R f02 = f0 * f2, f11 = f1 * f1;
      const R t1 =
          t0 - R(3) * f0 * (R(2) * f11 - f02) / (R(6) * f1 * (f02 - f11) - f0 * (f0 * f3));
      // The start's error (~1e-6 here) bounds the step; a step of at most
      // 3e-5 leaves an order-4 correction below 1e-18.
      if (isfinite(t1) && fabs(t1 - t0) <= R(3e-5) * dmax(R(1), fabs(t1))) {
        if (tw) *tw = t0;
        return t1;
      }
      if (isfinite(t1)) {
        t = t1;
        started = true;
      }
    }
  }
  if (!started && !(mx - t_lse <= R(-1))) {
    R s = 0;
#pragma unroll 4
    for (int c = 0; c < C; ++c) s += ((bits >> c) & 1u) ? static_cast<R>(x[G * c]) : R(0);
    s = group_sum<G>(s);
    t = (s - rhs) / static_cast<R>(count);
    // Heuristic refinement: U = {a > t} shrinks while it stays non-trivial.
    R u_cut = -num<R>::inf();
    int u_count = count;
    for (int it = 0; it < count + 1; ++it) {
      R su = 0;
      int cu = 0;
#pragma unroll 4
      for (int c = 0; c < C; ++c) {
        const R y = static_cast<R>(x[G * c]);
        const bool in = ((bits >> c) & 1u) && y > u_cut && y > t;
        su += in ? y : R(0);
        cu += in ? 1 : 0;
      }
      group_sums<G>(su, cu);
      if (cu == u_count || cu == 0) break;
      u_cut = dmax(u_cut, t);
      u_count = cu;
      t = (su - rhs) / static_cast<R>(cu);
    }
  }
  // Householder iterations of order 4 (entropy_norm.h:84-102).
  const R ub = mx - num<R>::exp_min_arg();
  const R eps16 = R(16) * num<R>::eps();
  bool warm = false;
  if constexpr (sizeof(R) == 8) {
    // The iteration converges to the root of sum W(exp(x - t)) = rhs from
    // any start near it, and its stopping rule |dt| <= 16 eps is checked in
    // double below; single-precision steps (about a third of the cost) bring
    // t to single precision first (three passes on U(-10, 10) columns), so
    // the double loop needs one Lambert pass instead of about five.  The
    // single-precision estimate is used only if its own steps settled.
    float tf = static_cast<float>(t);
    const float ubf = static_cast<float>(ub);
    bool settled = false;
    for (int iter = 0; iter < 4; ++iter) {
      const float prev = tf;
      const float tc = fminf(tf, ubf);
      float f0 = 0, f1 = 0, f2 = 0, f3 = 0;
#pragma unroll 1
      for (int c = 0; c < C; ++c) {
        if ((bits >> c) & 1u) {
          const float w = lambert_w_exp(static_cast<float>(x[G * c]) - tc);
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
      f0 -= static_cast<float>(rhs);
      const float f02 = f0 * f2, f11 = f1 * f1;
      tf = tc - 3.0f * f0 * (2.0f * f11 - f02) / (6.0f * f1 * (f02 - f11) - f0 * (f0 * f3));
      if (!(fabsf(tf) <= 3.0e38f)) break;
      // A step of at most 3e-3 (relative) leaves an order-4 correction of
      // ~1e-9 for the next one: below single precision, so the pass that
      // would confirm it is skipped.
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
    const R mt = -tc;
    if (tw) *tw = tc;
    R f0 = 0, f1 = 0, f2 = 0, f3 = 0;
#pragma unroll 1
    for (int c = 0; c < C; ++c) {
      if ((bits >> c) & 1u) {
        const R w = lambert_w_exp(static_cast<R>(x[G * c]) + mt);
        if (wl) wl[G * c] = w;
        // The derivative sums steer the step only (the root is f0 = rhs),
        // so they share one reciprocal of 1 + w.
        const R rd = div_near(R(1), R(1) + w);
        const R rd2 = rd * rd;
        const R rd3 = rd2 * rd;
        f0 += w;
        f1 += w * rd;
        f2 += w * rd3;
        f3 += w * (R(1) - R(2) * w) * (rd3 * rd2);
      }
    }
    group_sums<G>(f0, f1, f2, f3);
    f0 -= rhs;
    const R f02 = f0 * f2, f11 = f1 * f1;
    t = tc - R(3) * f0 * (R(2) * f11 - f02) / (R(6) * f1 * (f02 - f11) - f0 * (f0 * f3));
    if (fabs(prev - t) <= eps16) break;
    // From a settled single-precision start the first double step moves t by
    // about the single-precision rounding (~1e-8); when it moves by at most
    // 1e-6 the order-4 step's next correction is ~1e-24, far below the 1e-12
    // the results are held to, so the pass that would only confirm it is
    // skipped.
    if (warm && iter == 0 && fabs(prev - t) <= R(1e-6) * dmax(R(1), fabs(t))) break;
  }
  return t;
}

// Forced inline: outlined, the call convention alone costs the kernel ~80
// VGPRs (three waves per SIMD instead of eight).
// For the exp map the first threshold pass also keeps e_c = exp(x_c - mx0)
// (mx0 the column maximum) in registers, and when t >= mx0 the clamp pass
// writes e_c * exp(mx0 - t) instead of evaluating exp(x_c - t) again (the
// same value to a few ulps; with t >= mx0 an underflowed e_c means an
// underflowed result).
// NORM with wl: the last solve's W values stay in wl (see
// lds_solve_sum_w_exp); *wbits receives the slots whose value belongs to
// the returned threshold (the free slots, 0 if the threshold came otherwise)
// and *tw the point tc they were evaluated at.
template <bool NORM, int G, int C, class D, class R>
__device__ __forceinline__ ColThr<R> ent_family(const D* x, int m, int nvalid,
                                                const ProxParamsT<R>& pp, R (&e)[C],
                                                R& scale, R* wl = nullptr, R* tw = nullptr,
                                                unsigned* wbits = nullptr) {
  const R hi = pp.hi, rhs = pp.rhs;
  const R eps = R(16) * num<R>::eps() * dmax(R(1), rhs);
  const R u = NORM ? hi + dlog(hi) + eps : dlog(hi) + eps;
  R r = rhs;
  unsigned freeb = slot_bits<C>(nvalid);
  R t = 0;
  R mx0 = 0;
  int nfixed = 0;
  if constexpr (!NORM) {
    // log_sum_exp with the first maximum excluded (math/log_exp.h:134-152).
    mx0 = lds_masked_max<G, C, D, R>(x, freeb);
    int first_c = C;
#pragma unroll
    for (int c = C - 1; c >= 0; --c)
      first_c = (((freeb >> c) & 1u) && static_cast<R>(x[G * c]) == mx0) ? c : first_c;
    const int g = static_cast<int>(threadIdx.x) % G;
    const int owner = group_min<G>(first_c < C ? g : G);
    R sum = 0;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const bool ok = (freeb >> c) & 1u;
      e[c] = ok ? dexp(static_cast<R>(x[G * c]) - mx0) : R(0);
      sum += (ok && !(g == owner && c == first_c)) ? e[c] : R(0);
    }
    t = mx0 + dlog1p(group_sum<G>(sum)) - dlog(r);
  }
  // Threshold over the free set, then fix {x > t + u} at hi and repeat
  // (entropy.h:30-49, entropy_norm.h:157-178).
  for (int iter = 0; iter <= m; ++iter) {
    if constexpr (NORM) {
      t = lds_solve_sum_w_exp<G, C, D, R>(x, freeb, m - nfixed, r, wl, tw);
      if (wbits) *wbits = freeb;
    } else if (iter > 0) {
      const R mx = lds_masked_max<G, C, D, R>(x, freeb);
      t = mx + dlog1p(lds_lse_sum_excl<G, C, D, R>(x, freeb, mx)) - dlog(r);
    }
    const R cut = t + u;
    int cnt = 0;
#pragma unroll 4
    for (int c = 0; c < C; ++c) {
      const bool fix = ((freeb >> c) & 1u) && static_cast<R>(x[G * c]) > cut;
      cnt += fix ? 1 : 0;
      freeb &= fix ? ~(1u << c) : ~0u;
    }
    cnt = group_sum<G>(cnt);
    if (cnt == 0) break;
    // The solve's W values no longer belong to the final threshold.
    if (wbits) *wbits = 0u;
    r -= hi * static_cast<R>(cnt);
    nfixed += cnt;
    if (nfixed == m) break;
    if (r <= eps) {
      t = lds_masked_max<G, C, D, R>(x, freeb) - num<R>::exp_min_arg() + R(1);
      break;
    }
  }
  if constexpr (!NORM) scale = dexp(mx0 - t);
  return tag_thr(make_thr<R>(t, R(0), hi, NORM ? 2 : 1), SDCA_BRANCH_SEARCH, nfixed, m - nfixed);
}

// ---------------------------------------------------------------------------
// Top-k entropy (topk_entropy.h:20-76).  U grows by removing the current
// maximum; membership is a per-lane slot mask.
// ---------------------------------------------------------------------------
template <int G, int C, class D, class R>
__device__ inline void masked_argmax(const D (&v)[C], const bool (&mask)[C], R& mx,
                                     int& owner, int& slot) {
  R lm = -num<R>::inf();
  int lc = C;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const R x = static_cast<R>(v[c]);
    if (mask[c] && (lc == C || x > lm)) { lm = x; lc = c; }
  }
  mx = group_max<G>(lm);
  const int g = static_cast<int>(threadIdx.x) % G;
  owner = group_min<G>((lc < C && lm == mx) ? g : G);
  slot = lc;
}

template <int G, int C, class D, class R>
__device__ inline ColThr<R> topkent_family(const D (&v)[C], int m, int nvalid,
                                           const ProxParamsT<R>& pp, int* n_u_out = nullptr,
                                           R* sum_u_out = nullptr) {
  const int k = pp.k;
  const R eps = R(16) * num<R>::eps();
  const R K = static_cast<R>(k);
  const int g = static_cast<int>(threadIdx.x) % G;
  bool rest[C];
#pragma unroll
  for (int c = 0; c < C; ++c) rest[c] = c < nvalid;
  R mx;
  int owner, slot;
  masked_argmax<G, C, D, R>(v, rest, mx, owner, slot);
  R z = lse_sum_excl<G, C, D, R>(v, rest, mx);
  R log_z = mx + dlog1p(z);
  R l1 = dexp(-mx);
  R log_z_1 = isfinite(l1) ? mx + dlog1p(z + l1) : R(0);
  if (n_u_out) *n_u_out = 0;
  if (sum_u_out) *sum_u_out = R(0);
  if (k <= 1 || mx - eps <= log_z - dlog(K))
    return tag_thr(make_thr<R>(log_z_1, R(0), R(1), 1), SDCA_BRANCH_U_EMPTY, 0, m);
  R sum_u = 0, k_u = K;
  int n_u = 0;
  for (int num_u = 1; num_u < k; ++num_u) {
    const R min_u = mx;
    sum_u += min_u;
    ++n_u;
    if (g == owner) {
#pragma unroll
      for (int c = 0; c < C; ++c)
        if (c == slot) rest[c] = false;
    }
    k_u -= R(1);
    masked_argmax<G, C, D, R>(v, rest, mx, owner, slot);
    z = lse_sum_excl<G, C, D, R>(v, rest, mx);
    log_z = mx + dlog1p(z);
    const R tt = log_z - dlog(k_u);
    if (mx - eps <= tt && tt <= min_u + eps) break;
  }
  if (n_u_out) *n_u_out = n_u;
  if (sum_u_out) *sum_u_out = sum_u;
  const R tmp = ((K - k_u) * log_z + k_u * dlog(k_u) - sum_u) / K;
  R t, hi;
  if (tmp > mx) {
    const R a = (R(1) + z) * dexp(mx - tmp);
    t = tmp + dlog1p(a * K) - dlog(k_u);
    hi = a / (R(1) + a * K);
  } else {
    const R a = dexp(tmp - mx) / K;
    t = mx + dlog1p(z + a) - dlog(k_u / K);
    hi = (R(1) + z) / ((R(1) + z + a) * K);
  }
  return tag_thr(make_thr<R>(t, R(0), hi, 1), SDCA_BRANCH_U_GROWN, n_u, m - n_u);
}

// ---------------------------------------------------------------------------
// Two-block simplex (two_simplex.h:18-119).  Block a = rows [0, p), block
// b = rows [p, m); the sets kept by the reference's partitions are
// {x > x_cut} and {y > y_cut}.
// ---------------------------------------------------------------------------
// CA: the slots that may hold rows of block a (slot c holds row g + G c, so
// c < ceil(p / G)); the passes over block a visit only those, and the joint
// passes treat the others as block b alone.
// Candidate slots per lane for block b's phase 1 (see two_family_slots).
constexpr int kTwoCand = 4;

template <int G, int C, int CA, class D, class R>
__device__ inline ColThr<R> two_family_slots(const D (&v)[C], int m, int p,
                                             const ProxParamsT<R>& pp, D* lds_col = nullptr,
                                             D* lds_dummy = nullptr) {
  const R rhs = pp.rhs;
  const R eps = num<R>::eps() * dmax(R(1), rhs);
  const int g = static_cast<int>(threadIdx.x) % G;
  // Recomputed where used (one compare) rather than held as C lane masks.
  auto in_a = [&](int c) -> bool { return c < CA && (g + G * c) < p; };
  R cuts[2];
  R res[2];
  R maxs[2];
  int cnt[2];
  // Phase 1: each block on its own simplex <1, x> = rhs, by the reference's
  // iteration t = (sum(S) - rhs) / |S|, S <- {x in S : x > t} until S stays.
  // Its fixed point depends only on starting from a superset of the final
  // S, so S starts at {x > max - rhs} (a final member x has x > t and the
  // block maximum satisfies max - t <= rhs) instead of the whole block; each
  // pass gives the sum and count for the next threshold and the test.
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    R mx = -num<R>::inf();
#pragma unroll
    for (int c = 0; c < C; ++c) {
      if (b == 0 && c >= CA) continue;
      const R x = static_cast<R>(v[c]);
      mx = (in_a(c) == (b == 0) && x > mx) ? x : mx;
    }
    mx = group_max<G>(mx);
    maxs[b] = mx;
    R cut = mx - rhs;
    if constexpr (CA == 1 && G <= 64 && C >= 8) {
      // Block b of a column whose block a sits in slot 0 (the multilabel
      // duals): every value the iteration can keep is above max - rhs, a
      // few of the C slots on N(0,1) columns.  They are compacted through
      // the column's LDS words (free: the slots are in registers, and the
      // output is written from them) into kTwoCand slots per lane, and the
      // iteration runs on those; more candidates than that take the passes
      // over every slot below.  The sums are the same set's, in another
      // order.
      if (b == 1 && lds_col != nullptr) {
        int cn = 0;
#pragma unroll
        for (int c = 0; c < C; ++c)
          cn += (!in_a(c) && static_cast<R>(v[c]) > cut) ? 1 : 0;
        const int total = group_sum<G>(cn);
        if (total <= G * kTwoCand) {
          int pos = group_exclusive_scan<G>(cn, g);
#pragma unroll
          for (int c = 0; c < C; ++c) {
            const bool pr = !in_a(c) && static_cast<R>(v[c]) > cut;
            D* dst = pr ? lds_col + pos : lds_dummy;
            *dst = v[c];
            pos += pr ? 1 : 0;
          }
          group_lds_sync<G>();
          R cand[kTwoCand];
          R sb = 0;
          int nb = 0;
#pragma unroll
          for (int q = 0; q < kTwoCand; ++q) {
            const int i = g + G * q;
            const D x = lds_col[i < total ? i : 0];
            cand[q] = i < total ? static_cast<R>(x) : -num<R>::inf();
            sb += i < total ? cand[q] : R(0);
            nb += i < total ? 1 : 0;
          }
          group_sums<G>(sb, nb);
          R tb = 0;
          for (int it = 0; it <= m; ++it) {
            tb = div_near(sb - rhs, static_cast<R>(nb));
            R s2 = 0;
            int n2 = 0;
#pragma unroll
            for (int q = 0; q < kTwoCand; ++q) {
              const bool in = cand[q] > cut && cand[q] > tb;
              s2 += in ? cand[q] : R(0);
              n2 += in ? 1 : 0;
            }
            group_sums<G>(s2, n2);
            if (n2 == nb) break;
            cut = dmax(cut, tb);
            sb = s2;
            nb = n2;
          }
          cuts[b] = cut;
          cnt[b] = nb;
          res[b] = tb;
          continue;
        }
      }
    }
    R sb = 0;
    int nb = 0;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      if (b == 0 && c >= CA) continue;
      const R x = static_cast<R>(v[c]);
      const bool in = in_a(c) == (b == 0) && x > cut;
      sb += in ? x : R(0);
      nb += in ? 1 : 0;
    }
    group_sums<G>(sb, nb);
    R tb = 0;
    for (int it = 0; it <= m; ++it) {
      tb = div_near(sb - rhs, static_cast<R>(nb));
      R s2 = 0;
      int n2 = 0;
#pragma unroll
      for (int c = 0; c < C; ++c) {
        if (b == 0 && c >= CA) continue;
        const R x = static_cast<R>(v[c]);
        const bool in = in_a(c) == (b == 0) && x > cut && x > tb;
        s2 += in ? x : R(0);
        n2 += in ? 1 : 0;
      }
      group_sums<G>(s2, n2);
      if (n2 == nb) break;
      cut = dmax(cut, tb);
      sb = s2;
      nb = n2;
    }
    cuts[b] = cut;
    cnt[b] = nb;
    res[b] = tb;
  }
  R t = res[0];
  const R s = res[1];
  if (t + s >= -eps) {
    ColThr<R> r = tag_thr(make_thr<R>(t, R(0), rhs), SDCA_BRANCH_SEARCH, 0, cnt[0]);
    r.t2 = s;
    r.n_mid2 = cnt[1];
    return r;
  }
  // two_simplex_sort (two_simplex_sort.h:15-111) solves the same problem by a
  // scan over both sorted blocks and agrees with the above wherever the
  // common sum is positive; where the optimum is x = y = 0 its scan ends at
  // the sum rhs instead.  Such columns (and those within a margin of it)
  // are deferred to the sort-and-scan kernel.
  const bool sort_op = pp.op == OP_TWO_SIMPLEX_SORT;
  // Phase 2: joint variable fixing with s = -t; ca, cb: the blocks' kept
  // counts.
  int mc = cnt[0] + cnt[1];
  int ca = cnt[0], cb = cnt[1];
  {
    R sa = 0, sb = 0;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const R x = static_cast<R>(v[c]);
      if (in_a(c) && x > cuts[0]) sa += x;
      if (!in_a(c) && x > cuts[1]) sb += x;
    }
    group_sums<G>(sa, sb);
    t = (+sa - sb) / static_cast<R>(mc);
  }
  for (int it = 0; it <= m; ++it) {
    R sum_x = 0, sum_y = 0;
    int n_x = 0, n_y = 0;
    const R mt = -t;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const R x = static_cast<R>(v[c]);
      if (in_a(c)) {
        if (x > cuts[0] && !(x > t)) { sum_x += x; ++n_x; }
      } else {
        if (x > cuts[1] && !(x > mt)) { sum_y += x; ++n_y; }
      }
    }
    group_sums<G>(sum_x, sum_y, n_x, n_y);
    const R infeas = sum_x - sum_y - static_cast<R>(n_x + n_y) * t;
    R next;
    if (n_y > 0 && infeas > eps) {
      cuts[1] = dmax(cuts[1], mt);
      next = static_cast<R>(mc) * t + sum_y;
      mc -= n_y;
      cb -= n_y;
    } else if (n_x > 0 && infeas < -eps) {
      cuts[0] = dmax(cuts[0], t);
      next = static_cast<R>(mc) * t - sum_x;
      mc -= n_x;
      ca -= n_x;
    } else {
      ca -= n_x;  // two_simplex.h:100-103: both blocks keep {x > t}, {y > -t}
      cb -= n_y;
      break;
    }
    if (mc > 0) {
      t = next / static_cast<R>(mc);
    } else {
      break;
    }
  }
  if (sort_op) {
    const R margin = R(1e-3) * dmax(R(1), fabs(t));
    if (maxs[0] - t <= margin || maxs[1] + t <= margin) return slow_thr<R>();
  }
  ColThr<R> r = tag_thr(make_thr<R>(t, R(0), rhs), SDCA_BRANCH_BELOW_RHS, 0, ca);
  r.t2 = -t;
  r.n_mid2 = cb;
  return r;
}

// two_family_slots over a column held in memory (LDS or global) instead of
// register slots, thread g of the group taking entries g, g + G, ... (the
// slot layout's order, so the sums are the same): the same passes, for
// columns beyond the register slots.  Block a = entries [0, p).
template <int G, class D, class R>
__device__ inline ColThr<R> two_family_array(const D* x, int m, int p, const ProxParamsT<R>& pp) {
  const R rhs = pp.rhs;
  const R eps = num<R>::eps() * dmax(R(1), rhs);
  const int g = static_cast<int>(threadIdx.x) % G;
  R cuts[2];
  R res[2];
  int cnt[2];
  // Phase 1 per block: S starts at {x > max - rhs} and shrinks to
  // {x in S : x > t} until it stays (two_simplex.h:44-67).
  for (int b = 0; b < 2; ++b) {
    const int j0 = b == 0 ? 0 : p, j1 = b == 0 ? p : m;
    R mx = -num<R>::inf();
    for (int j = j0 + g; j < j1; j += G) {
      const R v = static_cast<R>(x[j]);
      mx = v > mx ? v : mx;
    }
    mx = group_max<G>(mx);
    R cut = mx - rhs;
    R sb = 0;
    int nb = 0;
    for (int j = j0 + g; j < j1; j += G) {
      const R v = static_cast<R>(x[j]);
      const bool in = v > cut;
      sb += in ? v : R(0);
      nb += in ? 1 : 0;
    }
    group_sums<G>(sb, nb);
    R tb = 0;
    for (int it = 0; it <= m; ++it) {
      tb = div_near(sb - rhs, static_cast<R>(nb));
      R s2 = 0;
      int n2 = 0;
      for (int j = j0 + g; j < j1; j += G) {
        const R v = static_cast<R>(x[j]);
        const bool in = v > cut && v > tb;
        s2 += in ? v : R(0);
        n2 += in ? 1 : 0;
      }
      group_sums<G>(s2, n2);
      if (n2 == nb) break;
      cut = dmax(cut, tb);
      sb = s2;
      nb = n2;
    }
    cuts[b] = cut;
    cnt[b] = nb;
    res[b] = tb;
  }
  R t = res[0];
  const R s = res[1];
  if (t + s >= -eps) {
    ColThr<R> r = tag_thr(make_thr<R>(t, R(0), rhs), SDCA_BRANCH_SEARCH, 0, cnt[0]);
    r.t2 = s;
    r.n_mid2 = cnt[1];
    return r;
  }
  // Phase 2: joint variable fixing with s = -t (two_simplex.h:69-117).
  int mc = cnt[0] + cnt[1];
  int ca = cnt[0], cb = cnt[1];
  {
    R sa = 0, sbb = 0;
    for (int j = g; j < m; j += G) {
      const R v = static_cast<R>(x[j]);
      if (j < p && v > cuts[0]) sa += v;
      if (j >= p && v > cuts[1]) sbb += v;
    }
    group_sums<G>(sa, sbb);
    t = (+sa - sbb) / static_cast<R>(mc);
  }
  for (int it = 0; it <= m; ++it) {
    R sum_x = 0, sum_y = 0;
    int n_x = 0, n_y = 0;
    const R mt = -t;
    for (int j = g; j < m; j += G) {
      const R v = static_cast<R>(x[j]);
      if (j < p) {
        if (v > cuts[0] && !(v > t)) { sum_x += v; ++n_x; }
      } else {
        if (v > cuts[1] && !(v > mt)) { sum_y += v; ++n_y; }
      }
    }
    group_sums<G>(sum_x, sum_y, n_x, n_y);
    const R infeas = sum_x - sum_y - static_cast<R>(n_x + n_y) * t;
    R next;
    if (n_y > 0 && infeas > eps) {
      cuts[1] = dmax(cuts[1], mt);
      next = static_cast<R>(mc) * t + sum_y;
      mc -= n_y;
      cb -= n_y;
    } else if (n_x > 0 && infeas < -eps) {
      cuts[0] = dmax(cuts[0], t);
      next = static_cast<R>(mc) * t - sum_x;
      mc -= n_x;
      ca -= n_x;
    } else {
      ca -= n_x;
      cb -= n_y;
      break;
    }
    if (mc > 0) {
      t = next / static_cast<R>(mc);
    } else {
      break;
    }
  }
  ColThr<R> r = tag_thr(make_thr<R>(t, R(0), rhs), SDCA_BRANCH_BELOW_RHS, 0, ca);
  r.t2 = -t;
  r.n_mid2 = cb;
  return r;
}

// Two-block simplex of one column per lane group.  When no column of the
// wave has more than G rows in block a (the multilabel duals: p <= 5 of
// m = 200 rows), block a lies in slot 0 of every lane and the passes over it
// are one slot long; the results are the same as the general form's.
template <int G, int C, class D, class R>
__device__ inline ColThr<R> two_family(const D (&v)[C], int m, int p, const ProxParamsT<R>& pp,
                                       D* lds_col = nullptr, D* lds_dummy = nullptr) {
  if constexpr (C > 1) {
    const int a_slots = __builtin_amdgcn_readfirstlane(group_max<64>((p + G - 1) / G));
    if (a_slots <= 1) return two_family_slots<G, C, 1, D, R>(v, m, p, pp, lds_col, lds_dummy);
  }
  return two_family_slots<G, C, C, D, R>(v, m, p, pp);
}

// ---------------------------------------------------------------------------
// Tile copies between global memory and LDS, 16 bytes per lane when both
// sides are 16-byte aligned.
// ---------------------------------------------------------------------------
template <int BT, class D>
__device__ inline void tile_copy(D* __restrict__ dst, const D* __restrict__ src,
                                 int64_t count) {
  const int64_t bytes = count * static_cast<int64_t>(sizeof(D));
  const bool vec = ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0;
  if (vec) {
    const int64_t nv = bytes / 16;
    const uint4* s4 = reinterpret_cast<const uint4*>(src);
    uint4* d4 = reinterpret_cast<uint4*>(dst);
    for (int64_t i = threadIdx.x; i < nv; i += BT) d4[i] = s4[i];
    const int64_t done = nv * 16 / static_cast<int64_t>(sizeof(D));
    for (int64_t i = done + threadIdx.x; i < count; i += BT) dst[i] = src[i];
  } else {
    for (int64_t i = threadIdx.x; i < count; i += BT) dst[i] = src[i];
  }
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Global -> LDS copy of a column tile with every 16-byte load of the thread
// issued before the first LDS store (NV = the most loads a thread can have
// for this configuration), so the whole tile is in flight at once.  Blocks
// are one wave, so a tile is a few KiB: HBM streams best when many small
// blocks each touch a short contiguous range (a 32 KiB-per-block copy runs
// ~30% slower than a 4 KiB one on MI355X).  Lanes past the tile's last
// 16-byte word repeat that word (same address, same value), so the copy has
// no per-load branch.
template <int NV, int BT, class D>
__device__ inline void tile_load(D* __restrict__ dst, const D* __restrict__ src, int64_t count) {
  const int64_t bytes = count * static_cast<int64_t>(sizeof(D));
  const bool vec = ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0;
  if (!vec || bytes % 16 != 0) {
    tile_copy<BT>(dst, src, count);
    return;
  }
  const int last = static_cast<int>(bytes / 16) - 1;
  const u32x4* s4 = reinterpret_cast<const u32x4*>(src);
  u32x4* d4 = reinterpret_cast<u32x4*>(dst);
  const int tid = static_cast<int>(threadIdx.x);
  u32x4 r[NV];
  if (last >= (NV - 1) * BT - 1) {
    // Every load but the last in range for every lane (whole tiles): one
    // base address with constant offsets, the clamp on the last load only.
#pragma unroll
    for (int i = 0; i < NV - 1; ++i) r[i] = __builtin_nontemporal_load(s4 + i * BT + tid);
    const int idx = min((NV - 1) * BT + tid, last);
    r[NV - 1] = __builtin_nontemporal_load(s4 + idx);
#pragma unroll
    for (int i = 0; i < NV - 1; ++i) d4[i * BT + tid] = r[i];
    d4[idx] = r[NV - 1];
    return;
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = min(i * BT + tid, last);
    r[i] = __builtin_nontemporal_load(s4 + idx);
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = min(i * BT + tid, last);
    d4[idx] = r[i];
  }
}

// LDS -> global copy; stores are fire-and-forget, streamed past the caches.
template <int NV, int BT, class D>
__device__ inline void tile_store(D* __restrict__ dst, const D* __restrict__ src, int64_t count) {
  const int64_t bytes = count * static_cast<int64_t>(sizeof(D));
  const bool vec = ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0;
  if (!vec || bytes % 16 != 0) {
    tile_copy<BT>(dst, src, count);
    return;
  }
  const int last = static_cast<int>(bytes / 16) - 1;
  const u32x4* s4 = reinterpret_cast<const u32x4*>(src);
  u32x4* d4 = reinterpret_cast<u32x4*>(dst);
  const int tid = static_cast<int>(threadIdx.x);
  if (last >= (NV - 1) * BT - 1) {
#pragma unroll
    for (int i = 0; i < NV - 1; ++i)
      __builtin_nontemporal_store(s4[i * BT + tid], d4 + i * BT + tid);
    const int idx = min((NV - 1) * BT + tid, last);
    __builtin_nontemporal_store(s4[idx], d4 + idx);
    return;
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int idx = min(i * BT + tid, last);
    __builtin_nontemporal_store(s4[idx], d4 + idx);
  }
}

// The Lambert map's LDS array of W values: after the tile of B m + slack
// words of D (8-byte aligned), the same shape in R.
template <class D, class R>
__device__ __host__ inline size_t w_lds_offset(int B, int64_t m, int64_t slack) {
  return ((static_cast<size_t>(B) * static_cast<size_t>(m) + static_cast<size_t>(slack)) *
              sizeof(D) + 7) & ~static_cast<size_t>(7);
}
template <class D, class R>
__device__ inline R* w_lds(unsigned char* smem, int B, int m, int slack) {
  return reinterpret_cast<R*>(smem + w_lds_offset<D, R>(B, m, slack));
}

// ---------------------------------------------------------------------------
// One tile of the batched kernel, once its B*m words are in LDS: the
// threshold search per column and the map, written back to the tile in
// place.  Block = BT threads (one wave) = BT / G columns of G lanes each.
// FULL: m == G * C, so every slot of an active lane is valid.
// ---------------------------------------------------------------------------
template <int FAM, int KM, class D, class R, int G, int C, int BT, bool FULL>
__device__ __forceinline__ void columns_tile(unsigned char* smem_raw, int m, int64_t col0,
                                             int ncols, const ProxParamsT<R>& pp,
                                             const int64_t* __restrict__ col_p,
                                             sdca_thresholds* __restrict__ thr,
                                             int* __restrict__ slow,
                                             sdca_prox_sets* __restrict__ sets) {
  D* tile = reinterpret_cast<D*>(smem_raw);
  constexpr int B = BT / G;
  const int lc = static_cast<int>(threadIdx.x) / G;
  const int g = static_cast<int>(threadIdx.x) % G;
  const bool active = lc < ncols;
  const int64_t j = col0 + lc;
  const int nvalid = active ? (FULL ? C : (m - g + G - 1) / G) : 0;
  // Slot c of this lane is tile word lc * m + g + G c: a per-lane base and a
  // compile-time offset, so every slot access is one LDS instruction.
  D* const col = tile + lc * m;
  D* const mine = col + g;
  // Unless FULL, the tile has G*C - m words of slack after the B*m elements
  // (the last column's slot reads end there), so every slot read stays
  // inside the allocation and the loop needs no branch; past that sit BT
  // per-lane dummy words for predicated stores (not allocated for the
  // entropic families, which never store through them).
  D* const lds_dummy = tile + B * m + (FULL ? 0 : G * C - m) + threadIdx.x;
  D v[C];
  if (FULL && ncols == B) {
#pragma unroll
    for (int c = 0; c < C; ++c) v[c] = mine[G * c];
  } else {
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const D x = mine[G * c];
      v[c] = (c < nvalid) ? x : -num<D>::inf();
    }
  }

  ColThr<R> th;
  int p = pp.p;
  // exp(x - mx0) per slot and exp(mx0 - t) from the exp-map family.
  R ecache[C];
  R escale = 0;
  // The Lambert map's last W values (an LDS array of R after the tile, for
  // Result types at least as wide as the data: otherwise the map is
  // evaluated in the data type) and the point they were taken at.  One-wave
  // workgroups only: a workgroup-wide column has no LDS to spare.
  constexpr bool kWReuse = FAM == FAM_ENT && KM == 1 && sizeof(R) >= sizeof(D) && BT == 64;
  R* const wl = kWReuse ? w_lds<D, R>(smem_raw, B, m, FULL ? 0 : G * C - m) + lc * m + g : nullptr;
  R tw = 0;
  unsigned wbits = 0;
  if constexpr (FAM == FAM_KNAP) {
    th = knap_family<G, C, D, R>(v, m, nvalid, pp);
  } else if constexpr (FAM == FAM_TOPK) {
    th = topk_family<G, C, KM, D, R>(v, m, nvalid, pp, col, lds_dummy);
  } else if constexpr (FAM == FAM_ENT) {
    th = ent_family<KM == 1, G, C, D, R>(mine, m, nvalid, pp, ecache, escale, wl, &tw, &wbits);
  } else if constexpr (FAM == FAM_TOPKENT) {
    th = topkent_family<G, C, D, R>(v, m, nvalid, pp);
  } else {
    if (col_p && active) p = clamp_split(col_p[j], m);
    th = two_family<G, C, D, R>(v, m, p, pp, col, lds_dummy);
  }

  // The threshold search may have used the column's LDS slots as scratch.
  __syncthreads();
  if (active) {
    // Deferred columns keep their input: the workgroup-per-column kernel
    // reads it again (in place when in == out).  For the clamp-only families
    // that is the clamp with t = 0, lo = -inf, hi = +inf; the entropic maps
    // select the input instead.
    constexpr bool kClampOnly = FAM == FAM_KNAP || FAM == FAM_TOPK || FAM == FAM_TWO;
    if (kClampOnly && th.slow) {
      th.t = th.t2 = R(0);
      th.lo = th.lo2 = -num<R>::inf();
      th.hi = th.hi2 = num<R>::inf();
    }
    const D t1 = static_cast<D>(th.t), lo1 = static_cast<D>(th.lo), hi1 = static_cast<D>(th.hi);
    const D t2 = static_cast<D>(th.t2), lo2 = static_cast<D>(th.lo2), hi2 = static_cast<D>(th.hi2);
    const D he1 = lo1 < hi1 ? hi1 : lo1, he2 = lo2 < hi2 ? hi2 : lo2;
    // The elementwise map is fixed per family (and per launch for the
    // entropic family, from the uniform op argument), so the slot loop has no
    // per-lane branch.
    auto write_slots = [&](auto map) {
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const D y = map(c);
        if (FULL) {
          mine[G * c] = y;
        } else {
          D* dst = (c < nvalid) ? mine + G * c : lds_dummy;
          *dst = y;
        }
      }
    };
    // The exp / Lambert maps run in a rolled loop over the LDS copy of the
    // slots (in place), for the same register reason as above.
    auto write_rolled = [&](auto map) {
      if (th.slow) return;
#pragma unroll 2
      for (int c = 0; c < C; ++c) {
        if (c < nvalid) mine[G * c] = map(mine[G * c]);
      }
    };
    if constexpr (FAM == FAM_ENT) {
      if constexpr (KM == 0) {
        // The cached exp(x - mx0) may have underflowed where exp(x - t) does
        // not when t < mx0 (after fixing, or for a large rhs); then the map
        // is evaluated directly.
        // Double data with a float Result: the map is evaluated in the data
        // type, as the reference's prox does (proxdef.h:181-196), not from
        // the float cache.
        if (!th.slow && escale <= R(1) && sizeof(R) >= sizeof(D)) {
#pragma unroll
          for (int c = 0; c < C; ++c) {
            if (c < nvalid)
              mine[G * c] = clamp_ref(static_cast<D>(ecache[c] * escale), lo1, hi1);
          }
        } else {
          write_rolled([&](D x) { return clamp_ref(dexp(x - t1), lo1, hi1); });
        }
      } else if constexpr (kWReuse) {
        // W(exp(x - t)) = W(exp((x - tc) - dt)) from w = W(exp(x - tc)),
        // dt = t - tc (a settled iteration's last step, ~1e-6).  Slots
        // outside the last solve's free set (fixed at hi by an earlier pass),
        // and columns whose last step was larger, evaluate the map.
        if (!th.slow) {
          const R dt = th.t - tw;
          const unsigned tay = fabs(dt) <= R(kLambertShiftMax) ? wbits : 0u;
#pragma unroll 2
          for (int c = 0; c < C; ++c) {
            if (c < nvalid) {
              D y;
              if ((tay >> c) & 1u) {
                y = static_cast<D>(lambert_w_exp_shift(wl[G * c], dt));
              } else {
                y = lambert_w_exp(mine[G * c] - t1);
              }
              mine[G * c] = clamp_ref(y, lo1, hi1);
            }
          }
        }
      } else {
        write_rolled([&](D x) { return clamp_ref(lambert_w_exp(x - t1), lo1, hi1); });
      }
    } else if constexpr (FAM == FAM_TOPKENT) {
      write_rolled([&](D x) { return clamp_ref(dexp(x - t1), lo1, hi1); });
    } else if constexpr (FAM == FAM_TWO) {
      write_slots([&](int c) {
        return (g + G * c >= p) ? clamp_med3(v[c] - t2, lo2, he2) : clamp_med3(v[c] - t1, lo1, he1);
      });
    } else {
      write_slots([&](int c) { return clamp_med3(v[c] - t1, lo1, he1); });
    }
    // The record's sets: from the search where it knows them, else counted
    // by the record's cuts over the slots (the input values).
    int set_hi = th.n_hi, set_mid = th.n_mid;
    if constexpr (FAM == FAM_KNAP || FAM == FAM_TOPK) {
      if (sets && !th.slow && set_hi < 0) {
        const R chi = th.t + th.hi, clo = th.t + th.lo;
        int nh = 0, nm = 0;
#pragma unroll
        for (int c = 0; c < C; ++c) {
          const R x = static_cast<R>(v[c]);
          const bool ok = FULL || c < nvalid;
          const bool h = ok && x > chi;
          nh += h ? 1 : 0;
          nm += (ok && !h && x > clo) ? 1 : 0;
        }
        group_sums<G>(nh, nm);
        set_hi = nh;
        set_mid = nm;
      }
    }
    if (g == 0) {
      if (sets && !th.slow) {
        if (FAM == FAM_TWO) {
          sets[2 * j] = sdca_prox_sets{0, th.n_mid, th.branch, 0};
          sets[2 * j + 1] = sdca_prox_sets{0, th.n_mid2, th.branch, 0};
        } else {
          sets[j] = sdca_prox_sets{set_hi, set_mid, th.branch, 0};
        }
      }
      if (th.slow) {
        const int pos = atomicAdd(slow, 1);
        slow[2 + pos] = static_cast<int>(j);
      } else if (thr) {
        if (FAM == FAM_TWO) {
          thr[2 * j].t = static_cast<double>(th.t);
          thr[2 * j].lo = static_cast<double>(th.lo);
          thr[2 * j].hi = static_cast<double>(th.hi);
          thr[2 * j + 1].t = static_cast<double>(th.t2);
          thr[2 * j + 1].lo = static_cast<double>(th.lo2);
          thr[2 * j + 1].hi = static_cast<double>(th.hi2);
        } else {
          thr[j].t = static_cast<double>(th.t);
          thr[j].lo = static_cast<double>(th.lo);
          thr[j].hi = static_cast<double>(th.hi);
        }
      }
    }
  }
}

// The batched kernel: a workgroup takes one tile (B columns): load, search,
// map, store.  The two-block simplex of 200-row fp32 columns (the
// multilabel duals' shape, eight lanes of 25 slots) asks for five waves per
// SIMD: left alone the compiler takes 98 VGPRs (four waves), with the hint
// 71, no spills, and the column kernel runs 3-7 % faster (0.1455 -> 0.141 ms
// per 500,000 columns, 0.154 -> 0.143 ms over the first steps).
template <int FAM, int KM, class D, class R, int G, int C, int BT, bool FULL>
__global__ void __launch_bounds__(BT) __attribute__((amdgpu_waves_per_eu(
    (FAM == FAM_TWO && BT == 64 && G == 8 && C == 25 && sizeof(D) == 4 && sizeof(R) == 4)
        ? 5 : 1)))
prox_columns_kernel(const D* __restrict__ in, D* __restrict__ out, int64_t m64,
                    int64_t n, ProxParamsT<R> pp, const int64_t* __restrict__ col_p,
                    sdca_thresholds* __restrict__ thr, int* __restrict__ slow,
                    sdca_prox_sets* __restrict__ sets) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  D* tile = reinterpret_cast<D*>(smem_raw);
  constexpr int B = BT / G;
  // Most 16-byte transfers per thread: B m sizeof(D) / (16 BT) <= C sizeof(D) / 16.
  constexpr int NV = (C * static_cast<int>(sizeof(D)) + 15) / 16;
  const int m = FULL ? G * C : static_cast<int>(m64);
  const int64_t col0 = static_cast<int64_t>(blockIdx.x) * B;
  const int ncols = static_cast<int>(min(static_cast<int64_t>(B), n - col0));
  const int64_t count = static_cast<int64_t>(ncols) * m;
  tile_load<NV, BT>(tile, in + col0 * m, count);
  __syncthreads();
  columns_tile<FAM, KM, D, R, G, C, BT, FULL>(smem_raw, m, col0, ncols, pp, col_p, thr, slow,
                                              sets);
  __syncthreads();
  tile_store<NV, BT>(out + col0 * m, tile, count);
}

}  // namespace sdca_gpu

#endif
