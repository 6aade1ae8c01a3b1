// Per-example epilogue of the evaluation pass (eval.h:36-47) on the score
// matrix: dual loss, top-k count / rank loss and the primal loss of every
// requested objective, one group of G lanes per example.
//
// Per example the scores row (m contiguous floats) is read straight into C
// register slots per lane (lane g holds classes g, g+G, ...; coalesced), and
// each objective restates its reference primal_loss / dual_loss:
//   multiclass (label y; the reference swaps s_y to the front, eval/primal.h:27-53)
//     count      #{j != y : s_j >= s_y}                          (ties count against)
//     hinge_topk max(0, sum of the k largest h_j), h_j = s_j + (1 - s_y)  (l2_hinge_topk.h:71-86)
//     topk_hinge sum of the positive h_j among the k largest              (l2_topk_hinge.h:72-87)
//     *_smooth   <h, p> - <p, p> / 2 with p the top-k simplex / knapsack_le projection of h
//                (l2_hinge_topk.h:162-179, l2_topk_hinge.h:166-183), from the threshold sets
//                as dot_x_prox / dot_prox_prox do (proxdef.h:332-370)
//     entropy    lse(s) - s_y                                              (l2_entropy.h:77-91)
//     entropy_topk  via the top-k entropy thresholds of s_j - s_y          (l2_entropy_topk.h:74-94)
//   multilabel (positives P, eval/primal.h:56-87)
//     rank loss  #{(p, n): s_n >= s_p} / (|P| |N|)
//     hinge      max(0, max_N s - min_P s + 1)                             (l2_multilabel_hinge.h:69-84)
//     smooth     two-simplex projection of (1/2 - s_P, 1/2 + s_N)          (l2_multilabel_hinge.h:168-191)
//     entropy    lse(s) - mean_P s                                         (l2_multilabel_entropy.h:72-86)
// Losses are written per example (in double) and reduced afterwards in a
// fixed order, so the totals are deterministic.  Examples whose top-k
// simplex needs the reference's full topk_cone_search are listed and
// finished by the workgroup-per-example kernel at the end of this file.
#include "eval_launch.hpp"
#include "prox_impl.hpp"

namespace sdca_gpu {

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <class R>
struct SetStats {
  R sum_u, sum_m, dot_m;
  int n_u, n_m;
};

// The threshold of a knapsack with lo = 0 formed from its final sets,
// t = (sum_M h + |U| hi - rhs) / |M| (knapsack_eq.h:87-106 with
// SDCA_ACCURATE_MATH): the iteration's own t carries the rounding of its
// incremental updates, which the loss would inherit.  Without free values t
// is any point between the sets and the loss does not depend on it.
template <class R>
__device__ inline R set_threshold(R t_iter, R hi, R rhs, const SetStats<R>& st) {
  if (st.n_m == 0) return t_iter;
  return (st.sum_m + hi * static_cast<R>(st.n_u) - rhs) / static_cast<R>(st.n_m);
}

// <h, p> - <p, p> / 2 at p = clamp(h - t, 0, hi), the projection of a knapsack
// whose sum constraint sum(p) = rhs is active, formed entry by entry and
// minus t (sum(p) - rhs).  The loss as a function of t has slope -|M| t at
// the root (|M| the free count), so the rounding of t alone (half an ulp of
// t ~ 1 in float, times |M| ~ 200 at m = 1000) would move it by 1e-5; the
// added term is zero at the exact root and cancels that slope, leaving an
// error of order |M| dt^2.  The sums over (h, p), each term at most hi in
// size, avoid the cancellation of the set-sum form below (t sum_M h against
// sum_M h^2, both ~|M|).
template <int G, int C, class D, class R>
__device__ inline R clamp_loss(const D (&h)[C], R t, R hi, R rhs) {
  R hp = 0, pp = 0, sp = 0;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const R x = static_cast<R>(h[c]);
    const bool ok = x > -num<R>::inf();
    const R p = ok ? clamp_ref(x - t, R(0), hi) : R(0);
    hp += ok ? x * p : R(0);
    pp += p * p;
    sp += p;
  }
  hp = group_sum<G>(hp);
  pp = group_sum<G>(pp);
  sp = group_sum<G>(sp);
  return hp - R(0.5) * pp - t * (sp - rhs);
}

// <h, p> - <p, p> / 2 from the threshold sets with lo = 0
// (dot_x_prox - dot_prox_prox / 2, proxdef.h:332-370).
template <class R>
__device__ inline R smooth_loss(R t, R hi, const SetStats<R>& st) {
  const R hp = hi * st.sum_u - t * st.sum_m + st.dot_m;
  const R pp = hi * hi * static_cast<R>(st.n_u) + t * t * static_cast<R>(st.n_m) + st.dot_m
             - R(2) * t * st.sum_m;
  return hp - R(0.5) * pp;
}

// Set statistics of a Kiwiel result (knapsack_eq.h:46-85): U = fixed at hi
// plus the final upper candidates, M = the remaining free elements, L = the
// rest; `cand` restricts the sets to values above the candidate cut.
template <int G, int C, class D, class R>
__device__ inline SetStats<R> knap_sets(const D (&h)[C], const KnapState<R>& st, R cand_cut) {
  SetStats<R> r;
  r.sum_u = r.sum_m = r.dot_m = 0;
  r.n_u = r.n_m = 0;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const R x = static_cast<R>(h[c]);
    const bool cand = x > cand_cut;
    const bool fixed_hi = x > st.hi_cut;
    const bool fr = (x > st.lo_cut) && !fixed_hi;
    const bool gl = x > st.c_lo;
    const bool in_u = cand && (fixed_hi || (fr && gl && x > st.c_hi));
    const bool in_m = cand && fr && gl && !(x > st.c_hi);
    r.sum_u += in_u ? x : R(0);
    r.n_u += in_u ? 1 : 0;
    r.sum_m += in_m ? x : R(0);
    r.dot_m += in_m ? x * x : R(0);
    r.n_m += in_m ? 1 : 0;
  }
  r.sum_u = group_sum<G>(r.sum_u);
  r.sum_m = group_sum<G>(r.sum_m);
  r.dot_m = group_sum<G>(r.dot_m);
  r.n_u = group_sum<G>(r.n_u);
  r.n_m = group_sum<G>(r.n_m);
  return r;
}

// Smooth top-k hinge loss (l2_hinge_topk.h:162-179) of the m' = m - 1 values
// h (padding and the label's slot hold -inf).  Returns false when the
// example needs the full topk_cone_search.  lds_col is the example's row of
// m words in LDS, used as scratch; nvalid counts the lane's slots inside it.
template <int G, int C, int KM, class D, class R>
__device__ inline bool smooth_topk_hinge(const D (&h)[C], int mp, int nvalid, int k, R gamma,
                                         D* lds_col, D* lds_dummy, R& loss) {
  constexpr int L = KM + 1;
  const R K = static_cast<R>(k);
  const R eps16 = R(16) * num<R>::eps();
  D top[L];
#pragma unroll
  for (int i = 0; i < L; ++i) top[i] = -num<D>::inf();
#pragma unroll
  for (int c = 0; c < C; ++c) top_insert(top, h[c]);
  top_merge<G>(top);
  R sum_k = 0, kth = static_cast<R>(top[0]), next = -num<R>::inf();
#pragma unroll
  for (int i = 0; i < L; ++i) {
    if (i < k) sum_k += static_cast<R>(top[i]);
    if (i == k - 1) kth = static_cast<R>(top[i]);
    if (i == k) next = static_cast<R>(top[i]);
  }
  const R largest = static_cast<R>(top[0]);
  // thresholds_topk_simplex(h, k, gamma) (topk_simplex.h:39-68)
  if (sum_k <= eps16) {  // zero projection
    loss = 0;
    return true;
  }
  const R hi_c = sum_k / K;
  const R t_c = kth - hi_c;
  const bool constant = (k == mp) || (t_c >= next - eps16);
  const R eps = num<R>::eps() * dmax(R(1), fabs(gamma));
  if (constant && !(K * hi_c > gamma + eps)) {
    // U = the k largest, M empty (topk_cone.h:43-51)
    const R hp = hi_c * sum_k;
    const R pp = hi_c * hi_c * K;
    loss = hp - R(0.5) * pp;
    return true;
  }
  const R hi = gamma / K;
  // Scores of an untrained model put every h within hi of the k-th largest:
  // the fixing over all slots is common here and stays in registers.
  KnapState<R> st = topk_knapsack<G, C, L, D, R, false>(h, top, mp, nvalid, k, kth, hi, gamma,
                                                         lds_col, lds_dummy);
  if (!constant) {
    bool lt;
    if (st.n_u == 0) {
      lt = st.t < -eps;
    } else {
      const R num_u = static_cast<R>(st.n_u);
      lt = K * (st.sum_u + (K - num_u) * st.t) < gamma * num_u - eps;
    }
    if (lt) {
      // topk_cone_search with U empty: t = 0, M = {h > 16 eps}; else defer.
      ColThr<R> cs = cone_search_u0<G, C, D, R>(h, K, largest);
      if (cs.slow) return false;
      R dot = 0;
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const R x = static_cast<R>(h[c]);
        dot += (x > eps16) ? x * x : R(0);
      }
      dot = group_sum<G>(dot);
      loss = R(0.5) * dot;
      return true;
    }
  }
  // The candidate cut used by topk_knapsack: values at or below it are in L.
  const R cut = kth - hi - (fabs(kth) + hi) * (R(16) * num<R>::eps());
  const SetStats<R> ss = knap_sets<G, C, D, R>(h, st, cut);
  loss = clamp_loss<G, C, D, R>(h, set_threshold(st.t, hi, gamma, ss), hi, gamma);
  return true;
}

// The k + 1 largest of h for k above the register list (KM): k + 1 passes of
// a group argmax, each removing one element (ties are taken one at a time,
// as nth_element's order does).  sum_k: the k largest; sum_pos: the positive
// ones among them; kth, next: the k-th and (k+1)-th; largest: the first.
template <int G, int C, class D, class R>
__device__ inline void topk_scan(const D (&h)[C], int k, R& sum_k, R& sum_pos, R& kth, R& next,
                                 R& largest) {
  bool rest[C];
#pragma unroll
  for (int c = 0; c < C; ++c) rest[c] = static_cast<R>(h[c]) > -num<R>::inf();
  const int g = static_cast<int>(threadIdx.x) % G;
  sum_k = sum_pos = 0;
  kth = next = largest = -num<R>::inf();
  for (int q = 0; q <= k; ++q) {
    R mx;
    int owner, slot;
    masked_argmax<G, C, D, R>(h, rest, mx, owner, slot);
    if (q == 0) largest = mx;
    if (q < k) {
      sum_k += mx;
      sum_pos += mx > R(0) ? mx : R(0);
      if (q == k - 1) kth = mx;
    } else {
      next = mx;
    }
    if (g == owner) {
#pragma unroll
      for (int c = 0; c < C; ++c)
        if (c == slot) rest[c] = false;
    }
  }
}

// smooth_topk_hinge for k above the register list: the same special cases
// (topk_cone.h:18-55) from topk_scan, the knapsack over every slot, the same
// cone-search test and deferral.
template <int G, int C, class D, class R>
__device__ inline bool smooth_topk_hinge_bigk(const D (&h)[C], int mp, int nvalid, int k, R gamma,
                                              R& loss) {
  const R K = static_cast<R>(k);
  const R eps16 = R(16) * num<R>::eps();
  R sum_k, sum_pos, kth, next, largest;
  topk_scan<G, C, D, R>(h, k, sum_k, sum_pos, kth, next, largest);
  if (sum_k <= eps16) {
    loss = 0;
    return true;
  }
  const R hi_c = sum_k / K;
  const R t_c = kth - hi_c;
  const bool constant = (k == mp) || (t_c >= next - eps16);
  const R eps = num<R>::eps() * dmax(R(1), fabs(gamma));
  if (constant && !(K * hi_c > gamma + eps)) {
    loss = hi_c * sum_k - R(0.5) * (hi_c * hi_c * K);
    return true;
  }
  const R hi = gamma / K;
  const R total = total_sum<G, C, D, R>(h, nvalid);
  KnapState<R> st = knapsack_eq_regs<G, C, D, R>(h, mp, nvalid, total, R(0), hi, gamma);
  if (!constant) {
    bool lt;
    if (st.n_u == 0) {
      lt = st.t < -eps;
    } else {
      const R num_u = static_cast<R>(st.n_u);
      lt = K * (st.sum_u + (K - num_u) * st.t) < gamma * num_u - eps;
    }
    if (lt) {
      ColThr<R> cs = cone_search_u0<G, C, D, R>(h, K, largest);
      if (cs.slow) return false;
      R dot = 0;
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const R x = static_cast<R>(h[c]);
        dot += (x > eps16) ? x * x : R(0);
      }
      dot = group_sum<G>(dot);
      loss = R(0.5) * dot;
      return true;
    }
  }
  const SetStats<R> ss = knap_sets<G, C, D, R>(h, st, -num<R>::inf());
  loss = clamp_loss<G, C, D, R>(h, set_threshold(st.t, hi, gamma, ss), hi, gamma);
  return true;
}

// Smooth top-k hinge beta (l2_topk_hinge.h:166-183): knapsack_le(h, 0, gamma/k, gamma).
template <int G, int C, class D, class R>
__device__ inline R smooth_topk_hinge_beta(const D (&h)[C], int mp, int k, R gamma) {
  const R lo = 0, hi = gamma / static_cast<R>(k), rhs = gamma;
  const R eps = num<R>::eps() * dmax(R(1), fabs(rhs));
  // knapsack_le.h:30-46: U = {x >= hi}, M = {lo < x < hi}, L = the rest
  SetStats<R> s;
  s.sum_u = s.sum_m = s.dot_m = 0;
  s.n_u = s.n_m = 0;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const R x = static_cast<R>(h[c]);
    const bool u = x >= hi;
    const bool mm = !u && x > lo;
    s.sum_u += u ? x : R(0);
    s.n_u += u ? 1 : 0;
    s.sum_m += mm ? x : R(0);
    s.dot_m += mm ? x * x : R(0);
    s.n_m += mm ? 1 : 0;
  }
  s.sum_u = group_sum<G>(s.sum_u);
  s.sum_m = group_sum<G>(s.sum_m);
  s.dot_m = group_sum<G>(s.dot_m);
  s.n_u = group_sum<G>(s.n_u);
  s.n_m = group_sum<G>(s.n_m);
  const int n_l = mp - s.n_u - s.n_m;
  const R sum = s.sum_m + hi * static_cast<R>(s.n_u) + lo * static_cast<R>(n_l);
  if (!(sum > rhs + eps)) {
    // thresholds (0, lo, hi): <h,p> = hi sum_U + dot_M, <p,p> = hi^2 |U| + dot_M
    return smooth_loss(R(0), hi, s);
  }
  R total = 0;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const R x = static_cast<R>(h[c]);
    total += (x > -num<R>::inf()) ? x : R(0);
  }
  total = group_sum<G>(total);
  KnapState<R> st = knapsack_eq_regs<G, C, D, R>(h, mp, C, total, lo, hi, rhs);
  const SetStats<R> ss = knap_sets<G, C, D, R>(h, st, -num<R>::inf());
  return clamp_loss<G, C, D, R>(h, set_threshold(st.t, hi, rhs, ss), hi, rhs);
}

template <int G, int C, class D, class R>
__device__ inline R lse_all(const D (&v)[C], int nvalid) {
  bool mask[C];
#pragma unroll
  for (int c = 0; c < C; ++c) mask[c] = c < nvalid;
  const R mx = masked_max<G, C, D, R>(v, mask);
  return mx + dlog1p(lse_sum_excl<G, C, D, R>(v, mask, mx));
}

// The per-example part of the multiclass evaluation (eval.h:36-47) for
// example i (active: a real example; inactive groups compute on example 0
// and store nothing), its m scores at srow (global memory, or the LDS tile
// of the fused kernel), g the lane's index in its group of G.  lds_col is
// the example's row of m words of LDS scratch (it may be the scores' own
// row: they are read into registers first), lds_dummy the lane's dummy word.
// save_row (or NULL): where the example's scores are written when one of its
// objectives is deferred to eval_slow_kernel, which reads them from global
// memory (the fused kernel keeps scores out of it otherwise).  Returns true
// when some objective of the example was deferred.
// MASK: the objective kinds compiled in (bit sdca_objective_kind; the
// others are skipped), HAS_A: whether dual variables may be given.  The fused
// kernel instantiates the set it runs to keep its registers down.  BIGK:
// top-k objectives with k above the register list (KM) are compiled in (the
// launch picks this variant only for them: the passes cost registers).
constexpr unsigned kAllMulticlass = 0x3fu;
template <int G, int C, int KM, class D, class R, unsigned MASK = kAllMulticlass,
          bool HAS_A = true, bool BIGK = false>
__device__ __forceinline__ bool eval_example_mc(const D* srow, const D* __restrict__ A,
                                                const int64_t* __restrict__ labels, int m,
                                                int64_t i, int64_t ii, bool active, int g,
                                                const EvalObjs& objs,
                                                double* __restrict__ per_example,
                                                int* __restrict__ counts, int* __restrict__ slow,
                                                int* __restrict__ bad, D* lds_col, D* lds_dummy,
                                                D* save_row = nullptr) {
  const int64_t m64 = m;
  // Device-resident labels reach the kernel unchecked: a label outside
  // [0, m) raises *bad (the call then fails with the reference's label
  // error, data/output.h:169-182) and is read as 0, so no load leaves the row.
  const int64_t yl = labels[ii];
  const bool bad_y = yl < 0 || yl >= m64;
  if (active && bad_y && g == 0) bad[0] = 1;
  const int y = bad_y ? 0 : static_cast<int>(yl);
  const D sy = srow[y];
  const int nvalid = (m - g + G - 1) / G;
  D s[C];
#pragma unroll
  for (int c = 0; c < C; ++c) s[c] = (c < nvalid) ? srow[g + G * c] : -num<D>::inf();

  // eval_primal_loss: count of j != y with s_j >= s_y (eval/primal.h:44-49)
  int cnt = 0;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int idx = g + G * c;
    cnt += (c < nvalid && idx != y && s[c] >= sy) ? 1 : 0;
  }
  cnt = group_sum<G>(cnt);
  if (active && g == 0) counts[i] = cnt;

  // Dual variables of the example.
  D a[C];
  D ay = 0;
  if (HAS_A && A) {
    const D* arow = A + ii * m64;
    ay = arow[y];
#pragma unroll
    for (int c = 0; c < C; ++c) a[c] = (c < nvalid) ? arow[g + G * c] : D(0);
  } else {
#pragma unroll
    for (int c = 0; c < C; ++c) a[c] = 0;
  }

  bool any_deferred = false;
  for (int o = 0; o < objs.n; ++o) {
    const EvalObj ob = objs.o[o];
    const R c_ = static_cast<R>(ob.c), gamma = static_cast<R>(ob.gamma);
    const int k = ob.k;
    R primal = 0, dual = 0;
    bool deferred = false;
    // h_j = s_j + (1 - s_y) for j != y, in the Data type (l2_hinge_topk.h:73-74)
    const D shift1 = D(1) - sy;
    D h[C];
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int idx = g + G * c;
      h[c] = (c < nvalid && idx != y) ? s[c] + shift1 : -num<D>::inf();
    }
    switch (ob.kind) {
      case SDCA_OBJ_HINGE_TOPK:
      case SDCA_OBJ_TOPK_HINGE: {
        if constexpr ((MASK & ((1u << SDCA_OBJ_HINGE_TOPK) | (1u << SDCA_OBJ_TOPK_HINGE))) == 0) break;
        dual = static_cast<R>(ay);
        if constexpr (BIGK) {
          if (k > KM) {  // l2_hinge_topk.h:71-86, l2_topk_hinge.h:72-87 by passes
            R sum_k, sum_pos, kth, next, largest;
            topk_scan<G, C, D, R>(h, k, sum_k, sum_pos, kth, next, largest);
            primal = (ob.kind == SDCA_OBJ_HINGE_TOPK) ? dmax(R(0), sum_k) : sum_pos;
            break;
          }
        }
        constexpr int L = KM + 1;
        D top[L];
#pragma unroll
        for (int q = 0; q < L; ++q) top[q] = -num<D>::inf();
#pragma unroll
        for (int c = 0; c < C; ++c) top_insert(top, h[c]);
        top_merge<G>(top);
        R sum = 0;
#pragma unroll
        for (int q = 0; q < L; ++q) {
          const R x = static_cast<R>(top[q]);
          if (q < k) sum += (ob.kind == SDCA_OBJ_HINGE_TOPK || top[q] > D(0)) ? x : R(0);
        }
        primal = (ob.kind == SDCA_OBJ_HINGE_TOPK) ? dmax(R(0), sum) : sum;
        dual = static_cast<R>(ay);
        break;
      }
      case SDCA_OBJ_HINGE_TOPK_SMOOTH: {
        if constexpr ((MASK & (1u << SDCA_OBJ_HINGE_TOPK_SMOOTH)) == 0) break;
        if constexpr (BIGK) {
          if (k > KM) {
            deferred = !smooth_topk_hinge_bigk<G, C, D, R>(h, m - 1, nvalid, k, gamma, primal);
            break;
          }
        }
        deferred = !smooth_topk_hinge<G, C, KM, D, R>(h, m - 1, nvalid, k, gamma, lds_col,
                                                      lds_dummy, primal);
        break;
      }
      case SDCA_OBJ_TOPK_HINGE_SMOOTH: {
        if constexpr ((MASK & (1u << SDCA_OBJ_TOPK_HINGE_SMOOTH)) == 0) break;
        primal = smooth_topk_hinge_beta<G, C, D, R>(h, m - 1, k, gamma);
        break;
      }
      case SDCA_OBJ_ENTROPY: {
        if constexpr ((MASK & (1u << SDCA_OBJ_ENTROPY)) == 0) break;
        primal = lse_all<G, C, D, R>(s, nvalid) - static_cast<R>(sy);
        break;
      }
      case SDCA_OBJ_ENTROPY_TOPK: {
        if constexpr ((MASK & (1u << SDCA_OBJ_ENTROPY_TOPK)) == 0) break;
        // a_j = s_j - s_y (l2_entropy_topk.h:78-80), then the top-k entropy thresholds
        const D shift0 = -sy;
        D v[C];
#pragma unroll
        for (int c = 0; c < C; ++c) {
          const int idx = g + G * c;
          v[c] = (c < nvalid && idx != y) ? s[c] + shift0 : -num<D>::inf();
        }
        ProxParamsT<R> pp;
        pp.lo = 0; pp.hi = 1; pp.rhs = 1; pp.k = k; pp.op = OP_TOPK_ENTROPY; pp.p = 0;
        int n_u = 0;
        R sum_u = 0;
        ColThr<R> th = topkent_family<G, C, D, R>(v, m - 1, C, pp, &n_u, &sum_u);
        if (n_u == 0) {
          primal = th.t;  // t = log(1 + sum exp) when U stays empty
        } else {
          const R num_hi = static_cast<R>(n_u);
          const R sk = th.hi * static_cast<R>(k);
          primal = th.hi * (sum_u + th.t * (static_cast<R>(k) - num_hi)) - x_log_x(R(1) - sk)
                 - num_hi * x_log_x(th.hi);
        }
        break;
      }
      default:
        break;
    }
    // Dual losses with the ground truth at position 0 (eval/dual.h:23-44).
    switch (ob.kind) {
      case SDCA_OBJ_HINGE_TOPK_SMOOTH:
      case SDCA_OBJ_TOPK_HINGE_SMOOTH: {  // l2_hinge_topk.h:182-192
        if constexpr (!HAS_A) {
          dual = 0;
          break;
        }
        R sq = 0;
#pragma unroll
        for (int c = 0; c < C; ++c) {
          const int idx = g + G * c;
          const R x = static_cast<R>(a[c]);
          sq += (c < nvalid && idx != y) ? x * x : R(0);
        }
        sq = group_sum<G>(sq);
        dual = static_cast<R>(ay) - (gamma / (R(2) * c_)) * sq;
        break;
      }
      case SDCA_OBJ_ENTROPY:
      case SDCA_OBJ_ENTROPY_TOPK: {  // l2_entropy.h:94-114, l2_entropy_topk.h:97-107
        if constexpr (!HAS_A) {
          // A = 0: c log c - x log x(c) - sum x log x(0) = 0
          dual = x_log_x(c_) - x_log_x(c_);
          break;
        }
        R acc = 0;
#pragma unroll
        for (int c = 0; c < C; ++c) {
          const int idx = g + G * c;
          acc += (c < nvalid && idx != y) ? x_log_x(-static_cast<R>(a[c])) : R(0);
        }
        acc = group_sum<G>(acc);
        dual = x_log_x(c_) - x_log_x(c_ - static_cast<R>(ay)) - acc;
        break;
      }
      default:
        dual = static_cast<R>(ay);
        break;
    }
    if (active && g == 0) {
      per_example[(i * objs.n + o) * 2] = static_cast<double>(primal);
      per_example[(i * objs.n + o) * 2 + 1] = static_cast<double>(dual);
      if (deferred) {
        const int pos = atomicAdd(slow, 1);
        slow[1 + 2 * pos] = static_cast<int>(i);
        slow[2 + 2 * pos] = o;
      }
    }
    any_deferred = any_deferred || deferred;
  }
  if (save_row && active && any_deferred) {
#pragma unroll
    for (int c = 0; c < C; ++c)
      if (c < nvalid) save_row[g + G * c] = s[c];
  }
  return any_deferred;
}

// BT threads per workgroup: one wave of 64 / G examples, or (G = BT) one
// example per workgroup for m above one wave's registers.
// WPE: the fewest waves per SIMD the register allocation must allow (1: no
// constraint).  The float kernels on one-wave workgroups with up to 16
// slots per lane ask for 3 (32 slots would spill 145 registers): at C4
// (64 lanes x 16 slots) that takes 168 registers instead of 189, with a few
// spilled to scratch, and the epilogue 0.67 ms instead of 0.81 ms.
template <int G, int C, int KM, class D, class R, int BT = 64, bool BIGK = false, int WPE = 1>
__global__ void __launch_bounds__(BT) __attribute__((amdgpu_waves_per_eu(WPE)))
eval_multiclass_kernel(const D* __restrict__ S, const D* __restrict__ A,
                       const int64_t* __restrict__ labels, int64_t m64, int64_t n, EvalObjs objs,
                       double* __restrict__ per_example, int* __restrict__ counts,
                       int* __restrict__ slow, int* __restrict__ bad) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  D* lds = reinterpret_cast<D*>(smem_raw);
  constexpr int B = BT / G;
  const int m = static_cast<int>(m64);
  const int lc = static_cast<int>(threadIdx.x) / G;
  const int g = static_cast<int>(threadIdx.x) % G;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * B + lc;
  const bool active = i < n;
  const int64_t ii = active ? i : 0;  // inactive groups compute on example 0, store nothing
  eval_example_mc<G, C, KM, D, R, kAllMulticlass, true, BIGK>(S + ii * m64, A, labels, m, i, ii,
                                                              active, g, objs,
                                  per_example, counts, slow, bad, lds + lc * m,
                                  lds + B * m + threadIdx.x);
}

// Two-block simplex sets (two_simplex.h:18-119) with block a = the slots in
// `in_a_bits`: the projection of (a, b) onto {x, y >= 0, <1,x> = <1,y> <= rhs}.
// Returns the smooth multilabel loss <h, p> - <p, p> / 2 summed over both
// blocks (lo = 0 and U is empty in both, so only the free sets count).
template <int G, int C, class D, class R>
__device__ inline R smooth_two_simplex_loss(const D (&v)[C], unsigned in_a_bits, int p, int mn,
                                            R rhs) {
  auto in_a = [&](int c) -> bool { return (in_a_bits >> c) & 1u; };
  const R eps = num<R>::eps() * dmax(R(1), rhs);
  R cuts[2];
  R res[2];
  int cnt[2] = {p, mn};
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    R cut = -num<R>::inf();
    R tb = 0;
    for (int it = 0; it <= p + mn; ++it) {
      R s = 0;
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const R x = static_cast<R>(v[c]);
        s += (in_a(c) == (b == 0) && x > cut) ? x : R(0);
      }
      s = group_sum<G>(s);
      tb = (s - rhs) / static_cast<R>(cnt[b]);
      int above = 0;
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const R x = static_cast<R>(v[c]);
        above += (in_a(c) == (b == 0) && x > cut && x > tb) ? 1 : 0;
      }
      above = group_sum<G>(above);
      if (above == cnt[b]) break;
      cut = dmax(cut, tb);
      cnt[b] = above;
    }
    cuts[b] = cut;
    res[b] = tb;
  }
  R t = res[0], s2 = res[1];
  if (!(t + s2 >= -eps)) {
    int mc = cnt[0] + cnt[1];
    R sa = 0, sb = 0;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const R x = static_cast<R>(v[c]);
      sa += (in_a(c) && x > cuts[0]) ? x : R(0);
      sb += (!in_a(c) && x > cuts[1]) ? x : R(0);
    }
    sa = group_sum<G>(sa);
    sb = group_sum<G>(sb);
    t = (+sa - sb) / static_cast<R>(mc);
    for (int it = 0; it <= p + mn; ++it) {
      R sum_x = 0, sum_y = 0;
      int n_x = 0, n_y = 0;
      const R mt = -t;
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const R x = static_cast<R>(v[c]);
        const bool lx = in_a(c) && x > cuts[0] && !(x > t);
        const bool ly = !in_a(c) && x > cuts[1] && !(x > mt);
        sum_x += lx ? x : R(0);
        n_x += lx ? 1 : 0;
        sum_y += ly ? x : R(0);
        n_y += ly ? 1 : 0;
      }
      sum_x = group_sum<G>(sum_x);
      sum_y = group_sum<G>(sum_y);
      n_x = group_sum<G>(n_x);
      n_y = group_sum<G>(n_y);
      const R infeas = sum_x - sum_y - static_cast<R>(n_x + n_y) * t;
      R next;
      if (n_y > 0 && infeas > eps) {
        cuts[1] = dmax(cuts[1], mt);
        next = static_cast<R>(mc) * t + sum_y;
        mc -= n_y;
      } else if (n_x > 0 && infeas < -eps) {
        cuts[0] = dmax(cuts[0], t);
        next = static_cast<R>(mc) * t - sum_x;
        mc -= n_x;
      } else {
        cuts[0] = dmax(cuts[0], t);
        cuts[1] = dmax(cuts[1], mt);
        break;
      }
      if (mc > 0) {
        t = next / static_cast<R>(mc);
      } else {
        break;
      }
    }
    s2 = -t;
  }
  // Free sets: {x in a: x > cuts[0]} with threshold t, {y in b: y > cuts[1]} with s2.
  R sm[2] = {0, 0}, dm[2] = {0, 0};
  int nm[2] = {0, 0};
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const R x = static_cast<R>(v[c]);
    const bool fa = in_a(c) && x > cuts[0];
    const bool fb = !in_a(c) && x > cuts[1];
    sm[0] += fa ? x : R(0);
    dm[0] += fa ? x * x : R(0);
    nm[0] += fa ? 1 : 0;
    sm[1] += fb ? x : R(0);
    dm[1] += fb ? x * x : R(0);
    nm[1] += fb ? 1 : 0;
  }
  R loss = 0;
  const R th[2] = {t, s2};
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    SetStats<R> st;
    st.sum_u = 0;
    st.n_u = 0;
    st.sum_m = group_sum<G>(sm[b]);
    st.dot_m = group_sum<G>(dm[b]);
    st.n_m = group_sum<G>(nm[b]);
    loss += smooth_loss(th[b], rhs, st);
  }
  return loss;
}

// WPE: as eval_multiclass_kernel's.  The float kernel on 8 lanes x 25 slots
// (C5) asks for 4 waves per SIMD: 127 registers instead of 134, no spills,
// its epilogue 0.51 ms instead of 0.58 ms.
template <int G, int C, class D, class R, int BT = 64, int WPE = 1>
__global__ void __launch_bounds__(BT) __attribute__((amdgpu_waves_per_eu(WPE)))
eval_multilabel_kernel(const D* __restrict__ S, const D* __restrict__ A,
                       const int64_t* __restrict__ labels, const int64_t* __restrict__ offsets,
                       int64_t m64, int64_t n, EvalObjs objs, double* __restrict__ per_example,
                       double* __restrict__ rank, int* __restrict__ bad) {
  constexpr int B = BT / G;
  const int m = static_cast<int>(m64);
  const int lc = static_cast<int>(threadIdx.x) / G;
  const int g = static_cast<int>(threadIdx.x) % G;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * B + lc;
  const bool active = i < n;
  const int64_t ii = active ? i : 0;
  // The CSR rules of data/output.h:185-208, checked here for device-resident
  // labels: the first offset is 0, the labels of an example lie inside
  // [0, offsets[n]) with 1..m-1 of them, sorted, distinct and in [0, m).  An
  // example that breaks them raises *bad and is evaluated as the valid
  // example {label 0}, so that no load leaves the label array.
  const int64_t off0 = offsets[ii];
  const int64_t off1 = offsets[ii + 1];
  bool ok = off0 >= 0 && (ii > 0 || off0 == 0) && off1 <= offsets[n] && off1 - off0 >= 1 &&
            off1 - off0 <= m64 - 1;
  if (ok) {
    int64_t prev = -1;
    for (int64_t q = off0; q < off1; ++q) {
      const int64_t lab = labels[q];
      ok = ok && lab > prev && lab < m64;
      prev = lab;
    }
  }
  if (active && !ok && g == 0) bad[0] = 1;
  const int p = ok ? static_cast<int>(off1 - off0) : 1;
  auto label_at = [&](int q) -> int { return ok ? static_cast<int>(labels[off0 + q]) : 0; };
  const int nvalid = (m - g + G - 1) / G;
  const D* srow = S + ii * m64;
  D s[C];
#pragma unroll
  for (int c = 0; c < C; ++c) s[c] = (c < nvalid) ? srow[g + G * c] : -num<D>::inf();
  // Positives of this lane as a slot mask: label j sits in slot (j - g) / G
  // of lane g when j - g is a multiple of G.
  unsigned posb = 0;
  for (int q = 0; q < p; ++q) {
    const int rel = label_at(q) - g;
    if (rel >= 0 && rel % G == 0) posb |= 1u << (rel / G);
  }
  auto pos = [&](int c) -> bool { return (posb >> c) & 1u; };
  // Rank loss (eval/primal.h:70-79): for each positive, the negatives >= it.
  R rl = 0;
  for (int q = 0; q < p; ++q) {
    const int lab = label_at(q);
    const D sp = srow[lab];
    int cn = 0;
#pragma unroll
    for (int c = 0; c < C; ++c) cn += (c < nvalid && !pos(c) && s[c] >= sp) ? 1 : 0;
    rl += static_cast<R>(group_sum<G>(cn));
  }
  const R rank_i = rl / static_cast<R>(p * (m - p));
  if (active && g == 0) rank[i] = static_cast<double>(rank_i);

  // The dual terms that do not depend on the objective, from one pass over
  // the example's row of A (l2_multilabel_hinge.h:87-96, :194-208,
  // l2_multilabel_entropy.h:89-109): sum over positives and negatives, the
  // squared norm and the negatives' sum of x log x at -a.  A is NULL for a
  // test set, whose records hold no dual terms.
  const D* arow = A ? A + ii * m64 : nullptr;
  R s_pos = 0, s_neg = 0, sq = 0, xl_neg = 0;
  if (A) {
#pragma unroll
    for (int c = 0; c < C; ++c) {
      if (c < nvalid) {
        const R x = static_cast<R>(arow[g + G * c]);
        s_pos += pos(c) ? x : R(0);
        s_neg += pos(c) ? R(0) : x;
        sq += x * x;
        xl_neg += pos(c) ? R(0) : x_log_x(-x);
      }
    }
    s_pos = group_sum<G>(s_pos);
    s_neg = group_sum<G>(s_neg);
    sq = group_sum<G>(sq);
    xl_neg = group_sum<G>(xl_neg);
  }
  const R pr = static_cast<R>(p);

  for (int o = 0; o < objs.n; ++o) {
    const EvalObj ob = objs.o[o];
    const R c_ = static_cast<R>(ob.c), gamma = static_cast<R>(ob.gamma);
    R primal = 0, dual = 0;
    switch (ob.kind) {
      case SDCA_OBJ_MULTILABEL_HINGE: {  // l2_multilabel_hinge.h:69-84
        D mn = num<D>::inf(), mx = -num<D>::inf();
#pragma unroll
        for (int c = 0; c < C; ++c) {
          if (c < nvalid) {
            mn = pos(c) ? ((s[c] < mn) ? s[c] : mn) : mn;
            mx = !pos(c) ? ((mx < s[c]) ? s[c] : mx) : mx;
          }
        }
        mn = group_min<G>(mn);
        mx = group_max<G>(mx);
        primal = dmax(R(0), static_cast<R>(mx - mn + D(1)));
        break;
      }
      case SDCA_OBJ_MULTILABEL_HINGE_SMOOTH: {  // l2_multilabel_hinge.h:168-191
        const D half(0.5);
        D v[C];
#pragma unroll
        for (int c = 0; c < C; ++c)
          v[c] = (c < nvalid) ? (pos(c) ? half - s[c] : s[c] + half) : -num<D>::inf();
        primal = smooth_two_simplex_loss<G, C, D, R>(v, posb, p, m - p, gamma);
        break;
      }
      case SDCA_OBJ_MULTILABEL_ENTROPY: {  // l2_multilabel_entropy.h:72-86
        R sp = 0;
#pragma unroll
        for (int c = 0; c < C; ++c) sp += (c < nvalid && pos(c)) ? static_cast<R>(s[c]) : R(0);
        sp = group_sum<G>(sp);
        primal = lse_all<G, C, D, R>(s, nvalid) - sp / static_cast<R>(p);
        break;
      }
      default:
        break;
    }
    switch (ob.kind) {
      case SDCA_OBJ_MULTILABEL_HINGE: dual = s_pos; break;  // l2_multilabel_hinge.h:87-96
      case SDCA_OBJ_MULTILABEL_HINGE_SMOOTH:                 // l2_multilabel_hinge.h:194-208
        dual = R(0.5) * (s_pos - s_neg - (gamma / c_) * sq);
        break;
      case SDCA_OBJ_MULTILABEL_ENTROPY: {                    // l2_multilabel_entropy.h:89-109
        // x log x at c - p a_j over the positives, from their labels (every
        // lane of the group the same, in label order).
        R xl_pos = 0;
        for (int q = 0; q < p; ++q) {
          const R x = arow ? static_cast<R>(arow[label_at(q)]) : R(0);
          xl_pos += x_log_x(c_ - pr * x);
        }
        dual = -xl_pos / pr - xl_neg + x_log_x(c_) + dlog(pr) * (c_ - s_pos);
        break;
      }
      default: break;
    }
    if (active && g == 0) {
      per_example[(i * objs.n + o) * 2] = static_cast<double>(primal);
      per_example[(i * objs.n + o) * 2 + 1] = static_cast<double>(dual);
    }
  }
}

// ---------------------------------------------------------------------------
// Deferred smooth top-k hinge examples: the h values of the example are
// sorted in LDS and one lane runs the reference's thresholds_topk_simplex on
// them (special cases, Kiwiel on contiguous ranges, topk_cone_search), then
// the loss from the sorted threshold sets.
// ---------------------------------------------------------------------------
template <class D, class R>
__device__ R sorted_sum(const D* s, int b, int e) {
  double acc = 0, comp = 0;
  for (int q = b; q < e; ++q) {
    const double x = static_cast<double>(static_cast<R>(s[q]));
    const double t = acc + x;
    comp += (fabs(acc) >= fabs(x)) ? (acc - t) + x : (x - t) + acc;
    acc = t;
  }
  return static_cast<R>(acc + comp);
}

template <class D, class R>
__device__ R sorted_dot(const D* s, int b, int e) {
  double acc = 0;
  for (int q = b; q < e; ++q) {
    const double x = static_cast<double>(static_cast<R>(s[q]));
    acc += x * x;
  }
  return static_cast<R>(acc);
}

template <class D, class R>
__device__ R smooth_topk_sorted(const D* s, int mp, int k, R gamma) {
  const R K = static_cast<R>(k);
  const R eps16 = R(16) * num<R>::eps();
  const R sum_k = sorted_sum<D, R>(s, 0, k);
  if (sum_k <= eps16) return R(0);
  const R hi_c = sum_k / K;
  const R t_c = static_cast<R>(s[k - 1]) - hi_c;
  const bool constant = (k == mp) || (t_c >= static_cast<R>(s[k]) - eps16);
  const R eps = num<R>::eps() * dmax(R(1), fabs(gamma));
  if (constant && !(K * hi_c > gamma + eps)) return hi_c * sum_k - R(0.5) * hi_c * hi_c * K;
  // Kiwiel on the sorted values: U = [0, f), M = [f, l), L = [l, mp)
  const R hi = gamma / K;
  int mc = mp, f = 0, l = mp;
  R t = (sorted_sum<D, R>(s, 0, mp) - gamma) / static_cast<R>(mp);
  for (int iter = 0; iter <= mp; ++iter) {
    const R c_lo = t, c_hi = hi + t;
    int p_lo = f;
    while (p_lo < l && static_cast<R>(s[p_lo]) > c_lo) ++p_lo;
    int p_hi = f;
    while (p_hi < p_lo && static_cast<R>(s[p_hi]) > c_hi) ++p_hi;
    const R s_lo = sorted_sum<D, R>(s, p_lo, l);
    const int n_lo = l - p_lo;
    const R s_hi = sorted_sum<D, R>(s, f, p_hi);
    const int n_hi = p_hi - f;
    const R sh = static_cast<R>(n_hi) * hi;
    const R infeas = s_hi + s_lo - sh - static_cast<R>(n_hi + n_lo) * t;
    R next;
    if (n_hi > 0 && infeas > eps) {
      f = p_hi;
      next = static_cast<R>(mc) * t - s_hi + sh;
      mc -= n_hi;
    } else if (n_lo > 0 && infeas < -eps) {
      l = p_lo;
      next = static_cast<R>(mc) * t - s_lo;
      mc -= n_lo;
    } else {
      f = p_hi;
      l = p_lo;
      break;
    }
    if (mc > 0) t = next / static_cast<R>(mc);
    else break;
  }
  bool lt = false;
  if (!constant) {
    if (f == 0) {
      lt = t < -eps;
    } else {
      const R num_u = static_cast<R>(f);
      lt = K * (sorted_sum<D, R>(s, 0, f) + (K - num_u) * t) < gamma * num_u - eps;
    }
  }
  R th = hi;
  if (lt) {
    // topk_cone_search (topk_cone.h:58-133) on the sorted values
    R k_u = K, min_u = num<R>::inf(), num_u = 0, sum_u = 0;
    bool found = false;
    for (int mf = 0; !found;) {
      R min_m = num<R>::inf(), max_m = -num<R>::inf(), sum_m = 0, num_m_sum_u = 0;
      R den = k_u * k_u;
      const R k_u_sum_u = k_u * sum_u;
      for (int ml = mf;;) {
        const R tt_ = (num_u * sum_m - k_u_sum_u) / den;
        const R hh = (num_m_sum_u + k_u * sum_m) / den;
        const R tt = hh + tt_;
        if (max_m - eps16 <= tt && tt <= min_u + eps16 && tt_ <= min_m + eps16 &&
            (ml == mp || static_cast<R>(s[ml]) - eps16 <= tt_)) {
          t = tt_;
          th = hh;
          f = mf;
          l = ml;
          found = true;
          break;
        }
        if (ml == mp) break;
        min_m = static_cast<R>(s[ml]);
        max_m = static_cast<R>(s[mf]);
        sum_m += min_m;
        num_m_sum_u += sum_u;
        den += num_u;
        ++ml;
      }
      if (found || mf == k) break;
      min_u = static_cast<R>(s[mf]);
      sum_u += min_u;
      k_u -= R(1);
      num_u += R(1);
      ++mf;
    }
    if (!found) return R(0);  // default zero thresholds
  }
  if (!lt) {
    // The knapsack's root: the threshold formed from the final free range
    // and the loss summed entry by entry minus t (sum p - gamma), as the
    // register epilogue does (set_threshold, clamp_loss).
    if (l > f)
      t = (sorted_sum<D, R>(s, f, l) + static_cast<R>(f) * hi - gamma) / static_cast<R>(l - f);
    double hp = 0, pp = 0, sp = 0;
    for (int q = 0; q < mp; ++q) {
      const R x = static_cast<R>(s[q]);
      const R p = clamp_ref(x - t, R(0), hi);
      hp += static_cast<double>(x * p);
      pp += static_cast<double>(p * p);
      sp += static_cast<double>(p);
    }
    return static_cast<R>(hp) - R(0.5) * static_cast<R>(pp) - t * (static_cast<R>(sp) - gamma);
  }
  SetStats<R> st;
  st.sum_u = sorted_sum<D, R>(s, 0, f);
  st.n_u = f;
  st.sum_m = sorted_sum<D, R>(s, f, l);
  st.dot_m = sorted_dot<D, R>(s, f, l);
  st.n_m = l - f;
  return smooth_loss(t, th, st);
}

template <class D, class R>
__global__ void __launch_bounds__(256)
eval_slow_kernel(const D* __restrict__ S, const int64_t* __restrict__ labels, int64_t m64,
                 EvalObjs objs, double* __restrict__ per_example, const int* __restrict__ slow,
                 int pow2) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  D* s = reinterpret_cast<D*>(smem_raw);
  const int m = static_cast<int>(m64);
  const int count = slow[0];
  for (int w = blockIdx.x; w < count; w += gridDim.x) {
    const int64_t i = slow[1 + 2 * w];
    const int o = slow[2 + 2 * w];
    const D* srow = S + i * m64;
    const int64_t yl = labels[i];
    const int y = (yl < 0 || yl >= m64) ? 0 : static_cast<int>(yl);  // flagged by the epilogue
    const D shift1 = D(1) - srow[y];
    // h over j != y, compacted: positions after y move down by one.
    for (int q = threadIdx.x; q < pow2; q += blockDim.x) {
      D v = -num<D>::inf();
      if (q < m - 1) v = srow[q < y ? q : q + 1] + shift1;
      s[q] = v;
    }
    __syncthreads();
    for (int size = 2; size <= pow2; size <<= 1) {
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        for (int q = threadIdx.x; q < pow2; q += blockDim.x) {
          const int partner = q ^ stride;
          if (partner > q) {
            const bool desc = (q & size) == 0;
            const D a = s[q], b = s[partner];
            if (desc ? (a < b) : (b < a)) {
              s[q] = b;
              s[partner] = a;
            }
          }
        }
        __syncthreads();
      }
    }
    if (threadIdx.x == 0) {
      const EvalObj ob = objs.o[o];
      per_example[(i * objs.n + o) * 2] = static_cast<double>(
          smooth_topk_sorted<D, R>(s, m - 1, ob.k, static_cast<R>(ob.gamma)));
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Fused evaluation pass (feature input, fp32 data, multiclass): scores
// W' x_i on the matrix cores and the per-example epilogue in one kernel, the
// scores never stored.  A workgroup of four waves owns E = 32 examples and
// every class (m <= 1024, padded to 4 NBW 32): wave w accumulates the
// 32 x (32 NBW) block of classes [32 NBW w, 32 NBW (w + 1)) in NBW
// v_mfma_f32_32x32x2f32 accumulators (16 NBW fp32 per lane).  The reduction
// runs in slabs of 8 with the next slab prefetched into registers while the
// current one is multiplied out of LDS ([k][row], padded rows), and visits k
// in the same pairs and operand lanes as the unfused score GEMMs (step t of
// each group of 8 sums k = 8g + t and 8g + 4 + t), so every score is
// bit-identical to the unfused path's wherever that path uses the MFMA
// score kernel (below 2^32 multiply-adds or 512 classes).  Then, for each half
// of the 32 examples, the accumulators are written to the LDS the slabs used
// (16 x m scores) and each wave runs the per-example epilogue
// (eval_example_mc) on four of them with one example per wave (G = 64),
// while the other workgroup of its CU (two fit: 68 KB of LDS each) keeps the
// matrix cores busy.  W (16 MB at C4) is re-read by every workgroup from the
// L2 / Infinity Cache: 32 examples per read give 16 flop per byte.
// ---------------------------------------------------------------------------
constexpr int kFusedE = 32;   // examples per workgroup
constexpr int kFusedBK = 8;   // reduction slab

template <int NBW>
struct FusedShape {
  static constexpr int BN = 4 * NBW * 32;         // padded classes
  static constexpr int LDA = kFusedE + 4, LDB = BN + 4;
  static constexpr int FLOATS = 2 * kFusedBK * LDA + 2 * kFusedBK * LDB;
  static constexpr int NVA = (kFusedE * kFusedBK / 4 + 255) / 256;
  static constexpr int NVB = (BN * kFusedBK / 4 + 255) / 256;
};

// The slab [k0, k0 + 8) of rows [r0, r0 + ROWS) of a (rows x d) matrix into
// float4 registers (two per row); rows past `rows` and columns past d read 0.
template <int ROWS, int NV>
__device__ inline void fused_load(const float* __restrict__ src, int64_t rows, int64_t d,
                                  int64_t r0, int64_t k0, bool vec, f32x4 (&r)[NV]) {
#pragma unroll
  for (int h = 0; h < NV; ++h) {
    const int f = static_cast<int>(threadIdx.x) + 256 * h;
    const int row = f >> 1, q = f & 1;
    const int64_t gr = r0 + row;
    const int64_t gk = k0 + 4 * q;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (f < ROWS * 2 && gr < rows) {
      const float* p = src + gr * d + gk;
      if (vec && gk + 4 <= d) {
        v = *reinterpret_cast<const f32x4*>(p);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (gk + e < d) v[e] = p[e];
      }
    }
    r[h] = v;
  }
}

// The float4 of a slab into LDS transposed to [k][row].
template <int ROWS, int NV>
__device__ inline void fused_store(float* __restrict__ lds, int ld, const f32x4 (&r)[NV]) {
#pragma unroll
  for (int h = 0; h < NV; ++h) {
    const int f = static_cast<int>(threadIdx.x) + 256 * h;
    const int row = f >> 1, q = f & 1;
    if (f < ROWS * 2) {
#pragma unroll
      for (int e = 0; e < 4; ++e) lds[(4 * q + e) * ld + row] = r[h][e];
    }
  }
}

template <int NBW, int G, int C, int KM, class R, unsigned MASK, bool HAS_A>
__global__ void __launch_bounds__(256, 2)
eval_fused_mc_kernel(const float* __restrict__ X, const float* __restrict__ W,
                     const float* __restrict__ A, const int64_t* __restrict__ labels, int64_t n,
                     int64_t m64, int64_t d, EvalObjs objs, double* __restrict__ per_example,
                     int* __restrict__ counts, int* __restrict__ slow, int* __restrict__ bad,
                     float* __restrict__ s_deferred, int vec) {
  typedef FusedShape<NBW> Sh;
  __shared__ __align__(16) float smem[Sh::FLOATS];
  float* const As0 = smem;
  float* const Bs0 = smem + 2 * kFusedBK * Sh::LDA;
  const int m = static_cast<int>(m64);
  const int64_t i0 = static_cast<int64_t>(blockIdx.x) * kFusedE;
  const int lane = static_cast<int>(threadIdx.x) & 63;
  const int wave = static_cast<int>(threadIdx.x) >> 6;
  const int lr = lane & 31, lk = lane >> 5;
  const int c0 = wave * NBW * 32;  // first class of this wave's block

  f32x16 acc[NBW];
#pragma unroll
  for (int b = 0; b < NBW; ++b)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[b][e] = 0.f;

  const bool vv = vec != 0;
  f32x4 ra[Sh::NVA], rb[Sh::NVB];
  fused_load<kFusedE, Sh::NVA>(X, n, d, i0, 0, vv, ra);
  fused_load<Sh::BN, Sh::NVB>(W, m64, d, 0, 0, vv, rb);
  fused_store<kFusedE, Sh::NVA>(As0, Sh::LDA, ra);
  fused_store<Sh::BN, Sh::NVB>(Bs0, Sh::LDB, rb);
  __syncthreads();
  const int64_t nslabs = (d + kFusedBK - 1) / kFusedBK;
  for (int64_t sl = 0; sl < nslabs; ++sl) {
    const int cur = static_cast<int>(sl & 1);
    const bool more = sl + 1 < nslabs;
    if (more) {
      fused_load<kFusedE, Sh::NVA>(X, n, d, i0, (sl + 1) * kFusedBK, vv, ra);
      fused_load<Sh::BN, Sh::NVB>(W, m64, d, 0, (sl + 1) * kFusedBK, vv, rb);
    }
    const float* as = As0 + cur * kFusedBK * Sh::LDA;
    const float* bs = Bs0 + cur * kFusedBK * Sh::LDB;
#pragma unroll
    for (int kk = 0; kk < kFusedBK; kk += 2) {
      // MFMA step kk / 2 of the slab's group of 8 sums k = kk / 2 (lanes
      // 0-31) and k = 4 + kk / 2 (lanes 32-63): the k order of every score
      // GEMM here.
      const int kr = 4 * lk + (kk >> 1);
      const float av = as[kr * Sh::LDA + lr];
      float bv[NBW];
#pragma unroll
      for (int b = 0; b < NBW; ++b) bv[b] = bs[kr * Sh::LDB + c0 + 32 * b + lr];
#pragma unroll
      for (int b = 0; b < NBW; ++b)
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv[b], acc[b], 0, 0, 0);
    }
    if (more) {
      fused_store<kFusedE, Sh::NVA>(As0 + (cur ^ 1) * kFusedBK * Sh::LDA, Sh::LDA, ra);
      fused_store<Sh::BN, Sh::NVB>(Bs0 + (cur ^ 1) * kFusedBK * Sh::LDB, Sh::LDB, rb);
    }
    __syncthreads();
  }

  // Accumulator r of lane l holds example 8 (r / 4) + 4 (l / 32) + r % 4 and
  // class l % 32 of its block: r < 8 are examples 0-15, r >= 8 are 16-31.
  float* const ss = smem;                           // 16 x m scores
  float* const dummies = smem + kFusedE / 2 * m;    // one word per thread
#pragma unroll
  for (int half = 0; half < 2; ++half) {
#pragma unroll
    for (int b = 0; b < NBW; ++b) {
      const int col = c0 + 32 * b + lr;
      if (col < m) {
#pragma unroll
        for (int r = 8 * half; r < 8 * half + 8; ++r) {
          const int row = 8 * (r / 4) + 4 * lk + (r % 4) - 16 * half;
          ss[row * m + col] = acc[b][r];
        }
      }
    }
    __syncthreads();
    // Groups of G lanes per example, as the two-kernel epilogue uses for
    // this m (so the per-example sums run in the same order): a wave pass
    // covers 64 / G examples, the four waves 256 / G.
    constexpr int B = 64 / G;
    constexpr int PASSES = (kFusedE / 2 + 4 * B - 1) / (4 * B);
#pragma unroll 1
    for (int q = 0; q < PASSES; ++q) {
      const int row0 = (q * 4 + wave) * B;  // first example of this wave pass
      if (row0 >= kFusedE / 2) break;       // wave-uniform
      // B divides 16, so every group of the pass has its own row of the
      // half; past n a group computes on its (zero) row and stores nothing.
      const int row = row0 + lane / G;
      const int64_t i = i0 + 16 * half + row;
      const bool active = i < n;
      const int64_t ii = active ? i : 0;
      float* const srow = ss + row * m;
      eval_example_mc<G, C, KM, float, R, MASK, HAS_A>(
          srow, A, labels, m, i, ii, active, lane % G, objs, per_example, counts, slow, bad,
          srow, dummies + threadIdx.x, s_deferred + ii * m64);
    }
    __syncthreads();
  }
}

template <int NBW, class R, unsigned MASK, bool HAS_A>
hipError_t launch_fused_set(const float* X, const float* W, const EvalLaunch& a, int64_t d,
                            float* s_deferred, bool km8) {
  const int64_t grid = (a.n + kFusedE - 1) / kFusedE;
  const int vec = (d % 4 == 0 && (reinterpret_cast<uintptr_t>(X) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(W) & 15) == 0) ? 1 : 0;
  // (G, C) as launch_typed picks for the two-kernel epilogue.
#define SDCA_FUSED_LAUNCH(G_, KM_)                                                          \
  hipLaunchKernelGGL((eval_fused_mc_kernel<NBW, G_, 16, KM_, R, MASK, HAS_A>),             \
                     dim3(static_cast<unsigned>(grid)), dim3(256), 0, a.stream, X, W,       \
                     static_cast<const float*>(a.A), a.labels, a.n, a.m, d, a.objs,         \
                     a.per_example, a.counts, a.slow, a.bad, s_deferred, vec)
  if (a.m <= 64) {
    if (!km8) SDCA_FUSED_LAUNCH(4, 5); else SDCA_FUSED_LAUNCH(4, 8);
  } else if (a.m <= 256) {
    if (!km8) SDCA_FUSED_LAUNCH(16, 5); else SDCA_FUSED_LAUNCH(16, 8);
  } else {
    if (!km8) SDCA_FUSED_LAUNCH(64, 5); else SDCA_FUSED_LAUNCH(64, 8);
  }
#undef SDCA_FUSED_LAUNCH
  return hipGetLastError();
}

// The objective sets with their own instantiation: the smooth top-k hinge
// with the softmax cross-entropy (the C4 pair), either alone, without
// dual variables (a cold start); anything else takes the general form.
constexpr unsigned kSmoothEntropy =
    (1u << SDCA_OBJ_HINGE_TOPK_SMOOTH) | (1u << SDCA_OBJ_ENTROPY);

template <int NBW, class R>
hipError_t launch_fused_nbw(const float* X, const float* W, const EvalLaunch& a, int64_t d,
                            float* s_deferred) {
  int kmax = 1;
  unsigned kinds = 0;
  for (int o = 0; o < a.objs.n; ++o) {
    kmax = a.objs.o[o].k > kmax ? a.objs.o[o].k : kmax;
    kinds |= 1u << a.objs.o[o].kind;
  }
  const bool km8 = kmax > 5;
  if (a.A || (kinds & ~kSmoothEntropy) != 0) return hipErrorInvalidValue;
  return launch_fused_set<NBW, R, kSmoothEntropy, false>(X, W, a, d, s_deferred, km8);
}

template <class R>
hipError_t launch_fused_typed(const float* X, const float* W, const EvalLaunch& a, int64_t d,
                              float* s_deferred) {
  // Classes per wave in blocks of 32: the fewest that cover m (m <= 1024).
  if (a.m <= 128) return launch_fused_nbw<1, R>(X, W, a, d, s_deferred);
  if (a.m <= 256) return launch_fused_nbw<2, R>(X, W, a, d, s_deferred);
  if (a.m <= 512) return launch_fused_nbw<4, R>(X, W, a, d, s_deferred);
  return launch_fused_nbw<8, R>(X, W, a, d, s_deferred);
}

template <class D, class R, int G, int C, int KM, int BT = 64, bool BIGK = false>
hipError_t launch_mc(const EvalLaunch& a) {
  constexpr int B = BT / G;
  if (a.m > static_cast<int64_t>(G) * C) return hipErrorInvalidValue;
  const int64_t blocks = (a.n + B - 1) / B;
  // B rows of scratch and BT dummy words.
  const size_t shmem = (static_cast<size_t>(B) * a.m + BT) * sizeof(D);
  constexpr int WPE = (sizeof(D) == 4 && sizeof(R) == 4 && BT == 64 && !BIGK && C <= 16) ? 3 : 1;
  hipLaunchKernelGGL((eval_multiclass_kernel<G, C, KM, D, R, BT, BIGK, WPE>),
                     dim3(static_cast<unsigned>(blocks)), dim3(BT), shmem, a.stream,
                     static_cast<const D*>(a.S), static_cast<const D*>(a.A), a.labels, a.m, a.n,
                     a.objs, a.per_example, a.counts, a.slow, a.bad);
  return hipGetLastError();
}

template <class D, class R, int G, int C, int BT = 64>
hipError_t launch_ml(const EvalLaunch& a) {
  constexpr int B = BT / G;
  if (a.m > static_cast<int64_t>(G) * C) return hipErrorInvalidValue;
  const int64_t blocks = (a.n + B - 1) / B;
  constexpr int WPE = (sizeof(D) == 4 && sizeof(R) == 4 && BT == 64 && G == 8 && C == 25) ? 4 : 1;
  hipLaunchKernelGGL((eval_multilabel_kernel<G, C, D, R, BT, WPE>), dim3(static_cast<unsigned>(blocks)),
                     dim3(BT), 0, a.stream, static_cast<const D*>(a.S), static_cast<const D*>(a.A),
                     a.labels, a.offsets, a.m, a.n, a.objs, a.per_example, a.rank, a.bad);
  return hipGetLastError();
}

// Rows above kRegMaxM: one example per workgroup (kWideThreads threads, the
// largest fp32 rows kMaxWideThreads), C slots per thread; every top-k
// variant compiled in.
template <class D, class R>
hipError_t launch_wide(const EvalLaunch& a) {
  constexpr int G = kWideThreads, G2 = kMaxWideThreads;
  if (a.offsets) {
    if (a.m <= 8 * G) return launch_ml<D, R, G, 8, G>(a);
    if (a.m <= 16 * G) return launch_ml<D, R, G, 16, G>(a);
    if (a.m <= 32 * G) return launch_ml<D, R, G, 32, G>(a);
    if constexpr (sizeof(D) == 4) return launch_ml<D, R, G2, 32, G2>(a);
    return hipErrorInvalidValue;
  }
  if (a.m <= 8 * G) return launch_mc<D, R, G, 8, 8, G, true>(a);
  if (a.m <= 16 * G) return launch_mc<D, R, G, 16, 8, G, true>(a);
  if (a.m <= 32 * G) return launch_mc<D, R, G, 32, 8, G, true>(a);
  if constexpr (sizeof(D) == 4) return launch_mc<D, R, G2, 32, 8, G2, true>(a);
  return hipErrorInvalidValue;
}

template <class D, class R>
hipError_t launch_typed(const EvalLaunch& a) {
  if (a.m > kRegMaxM) return launch_wide<D, R>(a);
  if (a.offsets) {
    if (a.m <= 64) return launch_ml<D, R, 4, 16>(a);
    // Eight lanes of 25 slots hold m = 200 exactly (four examples per wave
    // would leave 56 of 256 slots empty): the C5 multilabel epilogue takes
    // 0.56 ms against 0.66 ms on sixteen lanes of 16.
    if (a.m > 128 && a.m <= 200) return launch_ml<D, R, 8, 25>(a);
    if (a.m <= 256) return launch_ml<D, R, 16, 16>(a);
    if (a.m <= 1024) return launch_ml<D, R, 64, 16>(a);
    return launch_ml<D, R, 64, 32>(a);
  }
  int kmax = 1;
  for (int o = 0; o < a.objs.n; ++o) kmax = a.objs.o[o].k > kmax ? a.objs.o[o].k : kmax;
  if (kmax > kEvalMaxK) {
    if (a.m <= 64) return launch_mc<D, R, 4, 16, 8, 64, true>(a);
    if (a.m <= 256) return launch_mc<D, R, 16, 16, 8, 64, true>(a);
    if (a.m <= 1024) return launch_mc<D, R, 64, 16, 8, 64, true>(a);
    return launch_mc<D, R, 64, 32, 8, 64, true>(a);
  }
  // Double data: twice the lanes of the float mapping at half the slots
  // (rows of 513-1024 classes: one example per two-wave workgroup).  Sixteen
  // double slots per lane need 350 registers (one wave per SIMD, with
  // spills); eight need 180-230 (two waves).  The epilogue in double takes
  // 2.18 / 1.90 / 0.93 / 0.90 / 2.38 ms against 2.57 / 2.35 / 1.31 / 2.25 /
  // 2.85 ms at m = 50 / 100 / 200 / 400 / 1000 (the last at the C4 shape).
  // (fp32 data keeps its mapping: its fused pass forms the same sums.)
  if constexpr (sizeof(D) == 8) {
    if (a.m <= 1024) {
      if (kmax <= 5) {
        if (a.m <= 64) return launch_mc<D, R, 8, 8, 5>(a);
        if (a.m <= 256) return launch_mc<D, R, 32, 8, 5>(a);
        if (a.m <= 512) return launch_mc<D, R, 64, 8, 5>(a);
        return launch_mc<D, R, 128, 8, 5, 128>(a);
      }
      if (a.m <= 64) return launch_mc<D, R, 8, 8, 8>(a);
      if (a.m <= 256) return launch_mc<D, R, 32, 8, 8>(a);
      if (a.m <= 512) return launch_mc<D, R, 64, 8, 8>(a);
      return launch_mc<D, R, 128, 8, 8, 128>(a);
    }
  }
  if (kmax <= 5) {
    if (a.m <= 64) return launch_mc<D, R, 4, 16, 5>(a);
    if (a.m <= 256) return launch_mc<D, R, 16, 16, 5>(a);
    if (a.m <= 1024) return launch_mc<D, R, 64, 16, 5>(a);
    return launch_mc<D, R, 64, 32, 5>(a);
  }
  if (a.m <= 64) return launch_mc<D, R, 4, 16, 8>(a);
  if (a.m <= 256) return launch_mc<D, R, 16, 16, 8>(a);
  if (a.m <= 1024) return launch_mc<D, R, 64, 16, 8>(a);
  return launch_mc<D, R, 64, 32, 8>(a);
}

template <class D, class R>
hipError_t launch_slow_typed(const EvalLaunch& a) {
  int pow2 = 1;
  while (pow2 < a.m) pow2 <<= 1;
  hipLaunchKernelGGL((eval_slow_kernel<D, R>), dim3(256), dim3(256),
                     static_cast<size_t>(pow2) * sizeof(D), a.stream, static_cast<const D*>(a.S),
                     a.labels, a.m, a.objs, a.per_example, a.slow, pow2);
  return hipGetLastError();
}

// Deterministic sums in two levels: workgroup b sums examples
// [b chunk, (b + 1) chunk) of every output (2 n_obj loss sums, then the rank
// loss) in a fixed strided order and LDS tree, and one workgroup sums the
// partials in a fixed tree.  The chunking depends on n only, so the totals do
// not depend on scheduling.
constexpr int kReduceBlocks = 1024;

__global__ void __launch_bounds__(256)
reduce_partial_kernel(const double* __restrict__ per_example, int64_t n, int n_obj,
                      const double* __restrict__ rank, int64_t chunk,
                      double* __restrict__ partials) {
  __shared__ double part[256];
  const int outs = 2 * n_obj + 1;
  const int64_t b0 = static_cast<int64_t>(blockIdx.x) * chunk;
  const int64_t b1 = (b0 + chunk < n) ? b0 + chunk : n;
  for (int out = 0; out < outs; ++out) {
    double acc = 0;
    if (out < 2 * n_obj) {
      for (int64_t i = b0 + threadIdx.x; i < b1; i += 256) acc += per_example[i * 2 * n_obj + out];
    } else if (rank) {
      for (int64_t i = b0 + threadIdx.x; i < b1; i += 256) acc += rank[i];
    }
    part[threadIdx.x] = acc;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
      if (static_cast<int>(threadIdx.x) < w) part[threadIdx.x] += part[threadIdx.x + w];
      __syncthreads();
    }
    if (threadIdx.x == 0) partials[static_cast<int64_t>(blockIdx.x) * outs + out] = part[0];
    __syncthreads();
  }
}

__global__ void __launch_bounds__(256)
reduce_final_kernel(const double* __restrict__ partials, int nb, int n_obj,
                    double* __restrict__ sums, double* __restrict__ rank_sum) {
  __shared__ double part[256];
  const int outs = 2 * n_obj + 1;
  for (int out = 0; out < outs; ++out) {
    double acc = 0;
    for (int b = threadIdx.x; b < nb; b += 256) acc += partials[static_cast<int64_t>(b) * outs + out];
    part[threadIdx.x] = acc;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
      if (static_cast<int>(threadIdx.x) < w) part[threadIdx.x] += part[threadIdx.x + w];
      __syncthreads();
    }
    if (threadIdx.x == 0) {
      if (out < 2 * n_obj) sums[out] = part[0];
      else if (rank_sum) *rank_sum = part[0];
    }
    __syncthreads();
  }
}

__global__ void __launch_bounds__(256)
hist_kernel(const int* __restrict__ counts, int64_t n, unsigned long long* __restrict__ hist) {
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256)
    atomicAdd(hist + counts[i], 1ull);
}

__global__ void zero_u64_kernel(unsigned long long* p, int64_t count) {
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < count; i += static_cast<int64_t>(gridDim.x) * 256)
    p[i] = 0;
}

template <class D>
__global__ void __launch_bounds__(256)
regularizer_kernel(const D* __restrict__ W, const D* __restrict__ W0, int64_t count,
                   double* __restrict__ partials) {
  __shared__ double p0[256], p1[256];
  double a0 = 0, a1 = 0;
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < count; i += static_cast<int64_t>(gridDim.x) * 256) {
    const double w = static_cast<double>(W[i]);
    a0 += w * w;
    if (W0) a1 += static_cast<double>(W0[i]) * w;
  }
  p0[threadIdx.x] = a0;
  p1[threadIdx.x] = a1;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (static_cast<int>(threadIdx.x) < w) {
      p0[threadIdx.x] += p0[threadIdx.x + w];
      p1[threadIdx.x] += p1[threadIdx.x + w];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    partials[2 * blockIdx.x] = p0[0];
    partials[2 * blockIdx.x + 1] = p1[0];
  }
}

// Sums the per-workgroup partials in a fixed strided order and LDS tree.
__global__ void __launch_bounds__(256)
regularizer_final(const double* __restrict__ partials, int nb, double* out) {
  __shared__ double p0[256], p1[256];
  double a0 = 0, a1 = 0;
  for (int b = threadIdx.x; b < nb; b += 256) {
    a0 += partials[2 * b];
    a1 += partials[2 * b + 1];
  }
  p0[threadIdx.x] = a0;
  p1[threadIdx.x] = a1;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (static_cast<int>(threadIdx.x) < w) {
      p0[threadIdx.x] += p0[threadIdx.x + w];
      p1[threadIdx.x] += p1[threadIdx.x + w];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    out[0] = 0.5 * p0[0];
    out[1] = p1[0];
  }
}

// out (cols x rows, row-major) = in (rows x cols, row-major)^T through a
// padded 32 x 32 LDS tile: both the reads and the writes are coalesced.
template <class D>
__global__ void __launch_bounds__(256)
transpose_kernel(const D* __restrict__ in, D* __restrict__ out, int64_t rows, int64_t cols) {
  __shared__ D tile[32][33];
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 32, c0 = static_cast<int64_t>(blockIdx.x) * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8 threads
  for (int k = ty; k < 32; k += 8) {
    const int64_t r = r0 + k, c = c0 + tx;
    if (r < rows && c < cols) tile[k][tx] = in[r * cols + c];
  }
  __syncthreads();
  for (int k = ty; k < 32; k += 8) {
    const int64_t c = c0 + k, r = r0 + tx;
    if (r < rows && c < cols) out[c * rows + r] = tile[tx][k];
  }
}

// Per-example dual regularizer of the kernel-input evaluation,
// static_cast<Result>(dot(a_i, s_i)) / 2 (objective_base.h:92-105), one wave
// per example; the dot is accumulated in double and rounded to Data as the
// Data-typed BLAS dot returns it.
template <class D, class R>
__global__ void __launch_bounds__(256)
dualreg_kernel(const D* __restrict__ A, const D* __restrict__ S, int64_t m, int64_t n,
               double* __restrict__ per_example) {
  const int lane = threadIdx.x & 63;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (i >= n) return;
  const D* a = A + i * m;
  const D* sc = S + i * m;
  double acc = 0;
  for (int64_t c = lane; c < m; c += 64) acc += static_cast<double>(a[c]) * static_cast<double>(sc[c]);
  acc = group_sum<64>(acc);
  if (lane == 0)
    per_example[i] = static_cast<double>(static_cast<R>(static_cast<D>(acc)) / R(2));
}

// Deterministic sum of x[0, n) into *out: one workgroup, fixed strided order
// and a fixed LDS tree.
__global__ void __launch_bounds__(256)
sum_kernel(const double* __restrict__ x, int64_t n, double* __restrict__ out) {
  __shared__ double part[256];
  double acc = 0;
  for (int64_t i = threadIdx.x; i < n; i += 256) acc += x[i];
  part[threadIdx.x] = acc;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (static_cast<int>(threadIdx.x) < w) part[threadIdx.x] += part[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) *out = part[0];
}

template <class D>
__global__ void __launch_bounds__(256)
add_kernel(D* __restrict__ y, const D* __restrict__ x, int64_t count) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < count;
       i += static_cast<int64_t>(gridDim.x) * 256)
    y[i] = x[i] + y[i];
}



}  // namespace

hipError_t launch_eval_epilogue(const EvalLaunch& a) {
  if (a.data == SDCA_F32 && a.result == SDCA_F32) return launch_typed<float, float>(a);
  if (a.data == SDCA_F32 && a.result == SDCA_F64) return launch_typed<float, double>(a);
  if (a.data == SDCA_F64 && a.result == SDCA_F64) return launch_typed<double, double>(a);
  return hipErrorInvalidValue;
}

hipError_t launch_eval_slow(const EvalLaunch& a) {
  if (a.data == SDCA_F32 && a.result == SDCA_F32) return launch_slow_typed<float, float>(a);
  if (a.data == SDCA_F32 && a.result == SDCA_F64) return launch_slow_typed<float, double>(a);
  if (a.data == SDCA_F64 && a.result == SDCA_F64) return launch_slow_typed<double, double>(a);
  return hipErrorInvalidValue;
}

bool eval_fused_supported(const EvalLaunch& a, int64_t d) {
  (void)d;
  if (!(a.data == SDCA_F32 && (a.result == SDCA_F32 || a.result == SDCA_F64) && !a.offsets &&
        a.m >= 2 && a.m <= 1024))
    return false;
  // The general objective set needs more registers than two workgroups per
  // CU allow (it spills); it keeps the two-kernel form.
  unsigned kinds = 0;
  for (int o = 0; o < a.objs.n; ++o) {
    kinds |= 1u << a.objs.o[o].kind;
    if (a.objs.o[o].k > kEvalMaxK) return false;  // the register top list only
  }
  return !a.A && (kinds & ~kSmoothEntropy) == 0;
}

hipError_t launch_eval_fused(const float* X, const float* W, const EvalLaunch& a, int64_t d,
                             float* s_deferred) {
  if (!eval_fused_supported(a, d)) return hipErrorInvalidValue;
  if (a.result == SDCA_F32) return launch_fused_typed<float>(X, W, a, d, s_deferred);
  return launch_fused_typed<double>(X, W, a, d, s_deferred);
}

int64_t eval_reduce_scratch(int n_obj) {
  return static_cast<int64_t>(kReduceBlocks) * (2 * n_obj + 1);
}

hipError_t launch_eval_reduce(const EvalLaunch& a, double* sums, double* rank_sum,
                              unsigned long long* hist, double* partials) {
  const int64_t chunk_min = 2048;
  int64_t nb = (a.n + chunk_min - 1) / chunk_min;
  if (nb > kReduceBlocks) nb = kReduceBlocks;
  if (nb < 1) nb = 1;
  const int64_t chunk = (a.n + nb - 1) / nb;
  hipLaunchKernelGGL(reduce_partial_kernel, dim3(static_cast<unsigned>(nb)), dim3(256), 0, a.stream,
                     a.per_example, a.n, a.objs.n, a.rank, chunk, partials);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(reduce_final_kernel, dim3(1), dim3(256), 0, a.stream, partials,
                     static_cast<int>(nb), a.objs.n, sums, rank_sum);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (hist && a.counts) {
    hipLaunchKernelGGL(zero_u64_kernel, dim3(static_cast<unsigned>((a.m + 255) / 256)), dim3(256), 0,
                       a.stream, hist, a.m);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    int64_t blocks = (a.n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(hist_kernel, dim3(static_cast<unsigned>(blocks > 0 ? blocks : 1)), dim3(256),
                       0, a.stream, a.counts, a.n, hist);
    e = hipGetLastError();
  }
  return e;
}

hipError_t launch_regularizer(int data, const void* W, const void* W0, int64_t count,
                              double* partials, double* out, hipStream_t stream) {
  int64_t blocks = (count + 255) / 256;
  if (blocks > 512) blocks = 512;
  if (blocks < 1) blocks = 1;
  if (data == SDCA_F32) {
    hipLaunchKernelGGL(regularizer_kernel<float>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       stream, static_cast<const float*>(W), static_cast<const float*>(W0), count,
                       partials);
  } else {
    hipLaunchKernelGGL(regularizer_kernel<double>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       stream, static_cast<const double*>(W), static_cast<const double*>(W0), count,
                       partials);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(regularizer_final, dim3(1), dim3(256), 0, stream, partials,
                     static_cast<int>(blocks), out);
  return hipGetLastError();
}

hipError_t launch_transpose(int data, const void* in, void* out, int64_t rows, int64_t cols,
                            hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((cols + 31) / 32), static_cast<unsigned>((rows + 31) / 32));
  if (data == SDCA_F32)
    hipLaunchKernelGGL(transpose_kernel<float>, grid, dim3(256), 0, stream,
                       static_cast<const float*>(in), static_cast<float*>(out), rows, cols);
  else
    hipLaunchKernelGGL(transpose_kernel<double>, grid, dim3(256), 0, stream,
                       static_cast<const double*>(in), static_cast<double*>(out), rows, cols);
  return hipGetLastError();
}

hipError_t launch_add(int data, void* y, const void* x, int64_t count, hipStream_t stream) {
  int64_t blocks = (count + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  if (data == SDCA_F32)
    hipLaunchKernelGGL(add_kernel<float>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                       static_cast<float*>(y), static_cast<const float*>(x), count);
  else
    hipLaunchKernelGGL(add_kernel<double>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                       static_cast<double*>(y), static_cast<const double*>(x), count);
  return hipGetLastError();
}

hipError_t launch_dual_regularizer(int data, int result, const void* A, const void* S, int64_t m,
                                   int64_t n, double* per_example, double* out,
                                   hipStream_t stream) {
  const unsigned blocks = static_cast<unsigned>((n + 3) / 4);
  if (data == SDCA_F32 && result == SDCA_F32)
    hipLaunchKernelGGL((dualreg_kernel<float, float>), dim3(blocks), dim3(256), 0, stream,
                       static_cast<const float*>(A), static_cast<const float*>(S), m, n, per_example);
  else if (data == SDCA_F32)
    hipLaunchKernelGGL((dualreg_kernel<float, double>), dim3(blocks), dim3(256), 0, stream,
                       static_cast<const float*>(A), static_cast<const float*>(S), m, n, per_example);
  else
    hipLaunchKernelGGL((dualreg_kernel<double, double>), dim3(blocks), dim3(256), 0, stream,
                       static_cast<const double*>(A), static_cast<const double*>(S), m, n,
                       per_example);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(sum_kernel, dim3(1), dim3(256), 0, stream, per_example, n, out);
  return hipGetLastError();
}



}  // namespace sdca_gpu
