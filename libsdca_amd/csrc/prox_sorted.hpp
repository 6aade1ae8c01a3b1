// Per-column threshold routines on a column sorted in LDS (descending, the
// order the reference's std::sort(greater) produces): the reference's
// sequential steps - the special cases (topk_cone.h:18-55), the Kiwiel loop
// (knapsack_eq.h:25-109) whose partitions are contiguous ranges of the sorted
// column, the top-k simplex test (topk_simplex.h:9-68), the O(k m) searches
// topk_cone_search (topk_cone.h:58-133) and knapsack_le_biased_search - run
// by one wave, with the reference's tests in its order; the partitions are
// found by binary search and the range sums by the wave's 64 lanes
// (compensated), the scans' incremental sums in the reference's order.  Used
// by the workgroup-per-column prox kernel and the SDCA epoch.
#ifndef SDCA_HIP_PROX_SORTED_HPP
#define SDCA_HIP_PROX_SORTED_HPP

#include "common.hpp"
#include "prox_impl.hpp"
#include "prox_launch.hpp"

namespace sdca_gpu {

// Sums over ranges of the sorted column, by the 64 lanes of a wave (every
// lane calls it and receives the sum).  Summing a sorted sequence is the
// worst case for rounding (all positives, then the cancelling negatives), so
// each lane's strided part is compensated (Neumaier) in double and the
// lanes' (sum, compensation) pairs are combined the same way, lane ^ 32,
// ^ 16, ... (every lane ends with the same bits).
template <int OFF>
__device__ inline void neumaier_xor(double& acc, double& comp) {
  const double a2 = xor_lane<OFF, true>(acc), c2 = xor_lane<OFF, true>(comp);
  const double t = acc + a2;
  comp += c2 + ((fabs(acc) >= fabs(a2)) ? (acc - t) + a2 : (a2 - t) + acc);
  acc = t;
}
template <class R, class D>
__device__ R sum_range(const D* s, int b, int e) {
  double acc = 0, comp = 0;
  for (int i = b + (static_cast<int>(threadIdx.x) & 63); i < e; i += 64) {
    const double x = static_cast<double>(static_cast<R>(s[i]));
    const double t = acc + x;
    comp += (fabs(acc) >= fabs(x)) ? (acc - t) + x : (x - t) + acc;
    acc = t;
  }
  neumaier_xor<32>(acc, comp);
  neumaier_xor<16>(acc, comp);
  neumaier_xor<8>(acc, comp);
  neumaier_xor<4>(acc, comp);
  neumaier_xor<2>(acc, comp);
  neumaier_xor<1>(acc, comp);
  return static_cast<R>(acc + comp);
}

// The first index of [b, e) whose value fails x > c (x >= c with GE) in a
// column sorted in descending order, e if none: the end of the prefix the
// reference's partitions put first (binary search; the same in every lane).
template <class R, class D, bool GE = false>
__device__ inline int prefix_end(const D* s, int b, int e, R c) {
  while (b < e) {
    const int mid = b + ((e - b) >> 1);
    const R x = static_cast<R>(s[mid]);
    if (GE ? x >= c : x > c) b = mid + 1;
    else e = mid;
  }
  return b;
}

// Kiwiel variable fixing on a column sorted in descending order, by the 64
// lanes of a wave: its partitions are the sorted column's prefixes (found by
// binary search), its sums range sums.
template <class D, class R>
__device__ KnapState<R> knapsack_sorted(const D* s, int m, R lo, R hi, R rhs) {
  const R eps = num<R>::eps() * dmax(R(1), fabs(rhs));
  int mc = m;
  R t = (sum_range<R>(s, 0, m) - rhs) / static_cast<R>(m);
  int f = 0, l = m;  // free range [f, l)
  KnapState<R> st;
  st.n_u = 0;
  st.sum_u = 0;
  for (int iter = 0; iter <= m; ++iter) {
    const R c_lo = lo + t, c_hi = hi + t;
    const int p_lo = prefix_end<R>(s, f, l, c_lo);     // first free index with !(x > c_lo)
    const int p_hi = prefix_end<R>(s, f, p_lo, c_hi);  // end of the prefix with x > c_hi
    const R s_lo = sum_range<R>(s, p_lo, l);
    const int n_lo = l - p_lo;
    const R s_hi = sum_range<R>(s, f, p_hi);
    const int n_hi = p_hi - f;
    const R sh = static_cast<R>(n_hi) * hi;
    const R sl = static_cast<R>(n_lo) * lo;
    const R infeas = s_hi + s_lo - (sh + sl) - static_cast<R>(n_hi + n_lo) * t;
    R next;
    if (n_hi > 0 && infeas > eps) {
      f = p_hi;
      next = static_cast<R>(mc) * t - s_hi + sh;
      mc -= n_hi;
    } else if (n_lo > 0 && infeas < -eps) {
      l = p_lo;
      next = static_cast<R>(mc) * t - s_lo + sl;
      mc -= n_lo;
    } else {
      f = p_hi;
      l = p_lo;
      break;
    }
    if (mc > 0) {
      t = next / static_cast<R>(mc);
    } else {
      break;
    }
  }
  st.t = t;
  // The threshold applied is formed once more from the final free range
  // (knapsack_eq.h:87-106, SDCA_ACCURATE_MATH), as in the register kernel.
  st.t_acc = (l > f) ? (sum_range<R>(s, f, l) + static_cast<R>(f) * hi +
                        static_cast<R>(m - l) * lo - rhs) / static_cast<R>(l - f)
                     : t;
  st.n_u = f;
  st.n_f = l - f;
  st.sum_u = sum_range<R>(s, 0, f);
  return st;
}

// The U/M searches below try |U| = 0, 1, 2, ... in turn and return the
// first |U| whose scan over M accepts.  Called by all 64 lanes of a wave:
// lane l scans |U| = l, l + 64, ... (each setting up its U by the
// reference's own sequence of updates, so every trial value is the
// reference's), and the smallest accepting |U| of the wave is the answer.
// Returns its (t, hi) and the end e of its M = [u, e) in every lane, u in
// u_found; found = false gives the default.
template <class R>
__device__ inline bool wave_first_accept(int& u_found, R& t, R& hi, int& e) {
  const int best = group_min<64>(u_found);
  if (best == INT_MAX) return false;
  t = __shfl(t, best & 63, 64);
  hi = __shfl(hi, best & 63, 64);
  e = __shfl(e, best & 63, 64);
  u_found = best;
  return true;
}

// topk_cone_search (topk_cone.h:58-133) and its biased form
// thresholds_topk_cone_biased_search (topk_cone_biased.h:9-106) on the sorted
// column: the latter starts the |U| + rho k^2 term at rho k^2 (rho = 0 gives
// the former's steps exactly).
template <class D, class R>
__device__ void cone_search_sorted(const D* s, int m, int k, R rho, R& t_out, R& hi_out,
                                   int& branch, int& n_hi, int& n_mid) {
  const R eps = R(16) * num<R>::eps();
  int found = INT_MAX, fe = 0;
  R ft = 0, fh = 0;
  for (int mf = static_cast<int>(threadIdx.x) & 63; mf <= k && found == INT_MAX; mf += 64) {
    R k_u = static_cast<R>(k);
    R min_u = num<R>::inf();
    R num_u = rho * static_cast<R>(k) * static_cast<R>(k), sum_u = 0;
    for (int i = 0; i < mf; ++i) {
      min_u = static_cast<R>(s[i]);
      sum_u += min_u;
      k_u -= R(1);
      num_u += R(1);
    }
    R min_m = num<R>::inf();
    R max_m = -num<R>::inf();
    R sum_m = 0, num_m_sum_u = 0;
    R den = k_u * k_u;
    const R k_u_sum_u = k_u * sum_u;
    for (int ml = mf;;) {
      const R t = (num_u * sum_m - k_u_sum_u) / den;
      const R hi = (num_m_sum_u + k_u * sum_m) / den;
      const R tt = hi + t;
      if (max_m - eps <= tt && tt <= min_u + eps) {
        if (t <= min_m + eps && (ml == m || static_cast<R>(s[ml]) - eps <= t)) {
          found = mf;
          fe = ml;
          ft = t;
          fh = hi;
          break;
        }
      }
      if (ml == m) break;
      min_m = static_cast<R>(s[ml]);
      max_m = static_cast<R>(s[mf]);
      sum_m += min_m;
      num_m_sum_u += sum_u;
      den += num_u;
      ++ml;
    }
  }
  if (wave_first_accept(found, ft, fh, fe)) {
    branch = SDCA_BRANCH_SCAN;
    n_hi = found;
    n_mid = fe - found;
  } else {
    ft = fh = 0;
    branch = SDCA_BRANCH_DEFAULT;
    n_hi = n_mid = 0;
  }
  t_out = ft;
  hi_out = fh;
}

// thresholds_knapsack_le_biased_search (knapsack_le_biased.h:10-92) on the
// sorted column: grow U, and for each U grow M, until the candidate t
// satisfies the reference's interval tests; default 0.
template <class D, class R>
__device__ void knapsack_le_biased_sorted(const D* s, int m, R lo, R hi, R rhs, R rho,
                                          R& t_out, R& lo_out, R& hi_out, int& branch,
                                          int& n_hi, int& n_mid) {
  const R eps = num<R>::eps() * dmax(R(1), fabs(rhs));
  const R rho_rhs = rho * rhs;
  const R rho_inv = R(1) / rho;
  const R num_x = static_cast<R>(m);
  int found = INT_MAX, fe = 0;
  R ft = 0, unused = 0;
  for (int mf = static_cast<int>(threadIdx.x) & 63; mf <= m && found == INT_MAX; mf += 64) {
    // |U| = mf: the reference reaches it with num_u counted up by ones and
    // min_u = s[mf - 1].
    const R num_u = static_cast<R>(mf);
    const R min_u = mf > 0 ? static_cast<R>(s[mf - 1]) : num<R>::inf();
    R min_m = num<R>::inf();
    R max_m = -num<R>::inf();
    R num_m = 0, sum_m = 0;
    R num_l = num_x - num_u;
    for (int ml = mf;;) {
      const R t = (lo * num_l + hi * num_u + sum_m) / (rho_inv + num_m);
      if (t <= rho_rhs + eps) {
        R tt = hi + t;
        if (max_m - eps <= tt && tt <= min_u + eps) {
          tt = lo + t;
          if (tt <= min_m + eps && (ml == m || static_cast<R>(s[ml]) - eps <= tt)) {
            found = mf;
            fe = ml;
            ft = t;
            break;
          }
        }
      }
      if (ml == m) break;
      min_m = static_cast<R>(s[ml]);
      max_m = static_cast<R>(s[mf]);
      sum_m += min_m;
      num_l -= R(1);
      num_m += R(1);
      ++ml;
    }
  }
  if (wave_first_accept(found, ft, unused, fe)) {
    t_out = ft;
    lo_out = lo;
    hi_out = hi;
    branch = SDCA_BRANCH_SCAN;
    n_hi = found;
    n_mid = fe - found;
  } else {
    t_out = 0;
    lo_out = 0;
    hi_out = 0;
    branch = SDCA_BRANCH_DEFAULT;
    n_hi = n_mid = 0;
  }
}

// The record of the column's threshold function, with its branch
// (sdca_prox_branch) and sets: n_hi, n_mid are positions in the sorted
// column.
template <class D, class R>
__device__ void thresholds_sorted(const D* s, int m, int op, R lo, R hi, R rhs, R rho, int k,
                                  R& t_out, R& lo_out, R& hi_out, int& branch, int& n_hi,
                                  int& n_mid) {
  if (op == OP_KNAPSACK_LE_BIASED && rho != R(0)) {
    // knapsack_le_biased.h:102-130: the equality solution if its t is at
    // least rho rhs, else the search.
    lo_out = lo;
    hi_out = hi;
    const R eps = num<R>::eps() * dmax(R(1), fabs(rhs));
    const KnapState<R> st = knapsack_sorted<D, R>(s, m, lo, hi, rhs);
    if (st.t >= rho * rhs - eps) {
      t_out = st.t_acc;
      branch = SDCA_BRANCH_KNAPSACK;
      n_hi = st.n_u;
      n_mid = st.n_f;
      return;
    }
    knapsack_le_biased_sorted<D, R>(s, m, lo, hi, rhs, rho, t_out, lo_out, hi_out, branch, n_hi,
                                    n_mid);
    return;
  }
  if (op == OP_KNAPSACK_EQ || op == OP_KNAPSACK_LE || op == OP_KNAPSACK_LE_BIASED) {
    lo_out = lo;
    hi_out = hi;
    if (op != OP_KNAPSACK_EQ) {  // knapsack_le, and knapsack_le_biased with rho = 0
      // knapsack_le.h:30-46 on the sorted column
      const R eps = num<R>::eps() * dmax(R(1), fabs(rhs));
      const int e_hi = prefix_end<R, D, true>(s, 0, m, hi);
      const int e_mid = prefix_end<R>(s, e_hi, m, lo);
      const R sum = sum_range<R>(s, e_hi, e_mid) + hi * static_cast<R>(e_hi)
                  + lo * static_cast<R>(m - e_mid);
      if (!(sum > rhs + eps)) {
        t_out = 0;
        branch = SDCA_BRANCH_INACTIVE;
        n_hi = e_hi;
        n_mid = e_mid - e_hi;
        return;
      }
    }
    const KnapState<R> st = knapsack_sorted<D, R>(s, m, lo, hi, rhs);
    t_out = st.t_acc;
    branch = op == OP_KNAPSACK_EQ ? SDCA_BRANCH_SEARCH : SDCA_BRANCH_KNAPSACK;
    n_hi = st.n_u;
    n_mid = st.n_f;
    return;
  }
  const R K = static_cast<R>(k);
  const R eps16 = R(16) * num<R>::eps();
  const R sum_k = sum_range<R>(s, 0, k);
  if (sum_k <= eps16) {
    t_out = 0; lo_out = 0; hi_out = 0;
    branch = SDCA_BRANCH_ZERO;
    n_hi = n_mid = 0;
    return;
  }
  // topk_cone_special_cases with divisor K (+ rho K^2 for the biased forms,
  // topk_cone_biased.h:117, topk_simplex_biased.h:53).
  const R hi_c = sum_k / (K + rho * K * K);
  const R t_c = static_cast<R>(s[k - 1]) - hi_c;
  const bool constant = (k == m) || (t_c >= static_cast<R>(s[k]) - eps16);
  lo_out = 0;
  if (op == OP_TOPK_CONE || op == OP_TOPK_CONE_BIASED) {
    if (constant) {
      t_out = t_c;
      hi_out = hi_c;
      branch = SDCA_BRANCH_CONSTANT;
      n_hi = k;
      n_mid = 0;
    } else {
      cone_search_sorted<D, R>(s, m, k, rho, t_out, hi_out, branch, n_hi, n_mid);
    }
    return;
  }
  const R eps = num<R>::eps() * dmax(R(1), fabs(rhs));
  if (constant && !(K * hi_c > rhs + eps)) {
    t_out = t_c;
    hi_out = hi_c;
    branch = SDCA_BRANCH_CONSTANT;
    n_hi = k;
    n_mid = 0;
    return;
  }
  KnapState<R> st = knapsack_sorted<D, R>(s, m, R(0), rhs / K, rhs);
  if (!constant) {
    // is_topk_simplex_lt (topk_simplex.h:9-27) / is_topk_simplex_biased_lt
    // (topk_simplex_biased.h:9-28); rho = 0 gives the former exactly.
    bool lt;
    if (st.n_u == 0) {
      lt = st.t < rho * rhs - eps;
    } else {
      const R num_u = static_cast<R>(st.n_u);
      lt = K * (st.sum_u + (K - num_u) * st.t) < rhs * (num_u + rho * K * K) - eps;
    }
    if (lt) {
      cone_search_sorted<D, R>(s, m, k, rho, t_out, hi_out, branch, n_hi, n_mid);
      return;
    }
  }
  t_out = st.t_acc;
  hi_out = rhs / K;
  branch = SDCA_BRANCH_KNAPSACK;
  n_hi = st.n_u;
  n_mid = st.n_f;
}

// Descending sort of s[0, len) by the whole workgroup, without padding:
// Batcher's bitonic network in the form whose merges all run one way (the
// first stage of a merge of size `size` compares i with its mirror
// i ^ (size - 1), the later stages i with i ^ stride), over the next power
// of two.  Positions at or beyond len stand for -inf: such a position is
// always the larger index of its comparators, where a descending comparator
// leaves -inf in place, so those comparators are skipped and the array
// holds only the len values.
template <class D>
__device__ void sort_desc_unpadded(D* s, int len) {
  int pow2 = 1;
  while (pow2 < len) pow2 <<= 1;
  for (int size = 2; size <= pow2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const int mask = (stride == (size >> 1)) ? size - 1 : stride;
      for (int i = threadIdx.x; i < len; i += blockDim.x) {
        const int partner = i ^ mask;
        if (partner > i && partner < len) {
          const D a = s[i], b = s[partner];
          if (a < b) {
            s[i] = b;
            s[partner] = a;
          }
        }
      }
      __syncthreads();
    }
  }
}

}  // namespace sdca_gpu

#endif
