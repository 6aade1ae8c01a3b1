// Workgroup-per-column prox kernel: the columns the register kernel defers
// (topk_cone_search with U non-empty, zero-band ties, k > kTopkMaxK) and the
// knapsack operators for m beyond the register kernel.
//
// The column is sorted in LDS (bitonic, descending, the order the reference's
// std::sort(greater) produces), then the first wave runs the reference's
// steps on the sorted values - the special cases (topk_cone.h:18-55), the
// Kiwiel loop (knapsack_eq.h:25-109) whose partitions are contiguous ranges
// of the sorted column (binary searches, range sums over the wave), the
// top-k simplex test (topk_simplex.h:9-68) and the O(k m) search
// topk_cone_search (topk_cone.h:58-133) in the same order - and the
// workgroup clamps the column from global memory.
// Columns come from a device list written by the register kernel, so no host
// round trip is needed; every workgroup exits after the list is drained.
#include <algorithm>
#include <climits>

#include "common.hpp"
#include "prox_impl.hpp"
#include "prox_launch.hpp"
#include "prox_sorted.hpp"

namespace sdca_gpu {

namespace {

// GV: columns beyond the LDS; each workgroup sorts its column in its own
// pow2-word slice of gscratch (device memory) instead.
template <class D, class R, bool GV = false>
__global__ void __launch_bounds__(256)
prox_slow_kernel(const D* __restrict__ in, D* __restrict__ out, int64_t m64, int64_t n,
                 ProxParamsT<R> pp, sdca_thresholds* __restrict__ thr,
                 int* __restrict__ slow, int all_columns, int pow2,
                 sdca_prox_sets* __restrict__ sets, D* __restrict__ gscratch) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  D* s = GV ? gscratch + static_cast<int64_t>(blockIdx.x) * pow2 : reinterpret_cast<D*>(smem_raw);
  __shared__ R sh_t, sh_lo, sh_hi;
  const int m = static_cast<int>(m64);
  const int64_t count = all_columns ? n : static_cast<int64_t>(slow[0]);
  for (int64_t w = blockIdx.x; w < count; w += gridDim.x) {
    const int64_t j = all_columns ? w : static_cast<int64_t>(slow[2 + w]);
    const D* col = in + j * m64;
    for (int i = threadIdx.x; i < pow2; i += blockDim.x)
      s[i] = (i < m) ? col[i] : -num<D>::inf();
    __syncthreads();
    // Bitonic sort, descending.
    for (int size = 2; size <= pow2; size <<= 1) {
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        for (int i = threadIdx.x; i < pow2; i += blockDim.x) {
          const int partner = i ^ stride;
          if (partner > i) {
            const bool desc = (i & size) == 0;
            const D a = s[i], b = s[partner];
            if (desc ? (a < b) : (b < a)) {
              s[i] = b;
              s[partner] = a;
            }
          }
        }
        __syncthreads();
      }
    }
    // The first wave computes the thresholds: the scalar parts in every lane
    // alike, the U/M searches split over its lanes.
    if (threadIdx.x < 64) {
      R t, lo, hi;
      int branch, n_hi, n_mid;
      thresholds_sorted<D, R>(s, m, pp.op, pp.lo, pp.hi, pp.rhs, pp.rho, pp.k, t, lo, hi,
                              branch, n_hi, n_mid);
      if (threadIdx.x == 0) {
        sh_t = t;
        sh_lo = lo;
        sh_hi = hi;
        if (thr) {
          thr[j].t = static_cast<double>(t);
          thr[j].lo = static_cast<double>(lo);
          thr[j].hi = static_cast<double>(hi);
        }
        if (sets) sets[j] = sdca_prox_sets{n_hi, n_mid, branch, 0};
      }
    }
    __syncthreads();
    const D t = static_cast<D>(sh_t), lo = static_cast<D>(sh_lo), hi = static_cast<D>(sh_hi);
    D* dst = out + j * m64;
    for (int i = threadIdx.x; i < m; i += blockDim.x) dst[i] = clamp_ref(col[i] - t, lo, hi);
    __syncthreads();
  }
  // List mode: the list's counters [count, done] must be zero for the next
  // call on the stream.  With an empty list they already are; otherwise the
  // min(grid, count) workgroups that took columns count themselves out and
  // the last of them zeroes both (each has read the count before it
  // increments done).
  const int64_t workers = count < static_cast<int64_t>(gridDim.x) ? count : gridDim.x;
  if (!all_columns && static_cast<int64_t>(blockIdx.x) < workers && threadIdx.x == 0) {
    __threadfence();
    if (atomicAdd(slow + 1, 1) == static_cast<int>(workers) - 1) {
      atomicExch(slow, 0);
      atomicExch(slow + 1, 0);
    }
  }
}

template <class D, class R>
hipError_t launch_slow_t(const ProxLaunch& a, bool all_columns) {
  ProxParamsT<R> pp;
  pp.lo = static_cast<R>(a.lo);
  pp.hi = static_cast<R>(a.hi);
  pp.rhs = static_cast<R>(a.rhs);
  const bool biased = a.op == OP_KNAPSACK_LE_BIASED || a.op == OP_TOPK_SIMPLEX_BIASED ||
                      a.op == OP_TOPK_CONE_BIASED;
  pp.rho = biased ? static_cast<R>(a.rho) : R(0);
  pp.k = static_cast<int>(a.k);
  pp.op = a.op;
  pp.p = static_cast<int>(a.p);
  int pow2 = 1;
  while (pow2 < a.m) pow2 <<= 1;
  // List mode: the list is a small fraction of the n columns and usually
  // empty; the grid grows with n (about one workgroup per 1024 columns,
  // 512 to 1024: four per CU), so that a long list finds workgroups on
  // every CU while an empty one costs little to launch (the launch of 3906
  // workgroups for an empty C2 list took 0.5 % of the step; 1024 runs the
  // biased cone's deferred columns as fast).
  const int64_t cap = all_columns ? 4096 : std::min<int64_t>(1024, std::max<int64_t>(512, a.n / 1024));
  const int64_t grid = a.n < cap ? a.n : cap;
  // One wave per workgroup for short columns (the sort's stages then need
  // no cross-wave barrier and four times as many columns are in flight),
  // four waves beyond 256 rows.
  const int threads = pow2 <= 256 ? 64 : 256;
  hipLaunchKernelGGL((prox_slow_kernel<D, R>), dim3(static_cast<unsigned>(grid > 0 ? grid : 1)),
                     dim3(threads), static_cast<size_t>(pow2) * sizeof(D), a.stream,
                     static_cast<const D*>(a.in), static_cast<D*>(a.out), a.m, a.n, pp,
                     a.thr, a.slow, all_columns ? 1 : 0, pow2, a.sets, static_cast<D*>(nullptr));
  return hipGetLastError();
}

// Every column, each sorted in a pow2-word slice of scratch (device memory;
// scratch_bytes of it): one workgroup per slice.
template <class D, class R>
hipError_t launch_slow_global_t(const ProxLaunch& a, void* scratch, size_t scratch_bytes) {
  ProxParamsT<R> pp;
  pp.lo = static_cast<R>(a.lo);
  pp.hi = static_cast<R>(a.hi);
  pp.rhs = static_cast<R>(a.rhs);
  const bool biased = a.op == OP_KNAPSACK_LE_BIASED || a.op == OP_TOPK_SIMPLEX_BIASED ||
                      a.op == OP_TOPK_CONE_BIASED;
  pp.rho = biased ? static_cast<R>(a.rho) : R(0);
  pp.k = static_cast<int>(a.k);
  pp.op = a.op;
  pp.p = static_cast<int>(a.p);
  int64_t pow2 = 1;
  while (pow2 < a.m) pow2 <<= 1;
  int64_t grid = static_cast<int64_t>(scratch_bytes / (static_cast<size_t>(pow2) * sizeof(D)));
  if (grid > a.n) grid = a.n;
  if (grid > 4096) grid = 4096;
  if (grid < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL((prox_slow_kernel<D, R, true>), dim3(static_cast<unsigned>(grid)),
                     dim3(256), 0, a.stream, static_cast<const D*>(a.in), static_cast<D*>(a.out),
                     a.m, a.n, pp, a.thr, a.slow, 1, static_cast<int>(pow2), a.sets,
                     static_cast<D*>(scratch));
  return hipGetLastError();
}

// thresholds_two_simplex_sort (two_simplex_sort.h:15-111) on the two sorted
// blocks a[0, p), b[0, q): the common sum c is scanned over the breakpoints
// where the active counts r, s grow; past the end of a block the reference
// uses the pseudo point last - rhs.
// Also returns the active counts r, s (the records' free sets) and the
// branch: SDCA_BRANCH_BELOW_RHS when the optimum falls inside the scan.
template <class D, class R>
__device__ void two_sort_thresholds(const D* a, int p, const D* b, int q, R rhs, R& theta_a,
                                    R& theta_b, int& r_out, int& s_out, int& branch) {
  const R eps = num<R>::eps() * dmax(R(1), rhs);
  const R C = rhs;
  R c = 0, best_c = rhs;
  R sum_mu = static_cast<R>(a[0]), sum_nu = static_cast<R>(b[0]);
  int r = 1, s = 1;
  auto a_at = [&](int i) { return i < p ? static_cast<R>(a[i]) : static_cast<R>(a[p - 1]) - C; };
  auto b_at = [&](int i) { return i < q ? static_cast<R>(b[i]) : static_cast<R>(b[q - 1]) - C; };
  R a_r = a_at(r), b_s = b_at(s);
  branch = SDCA_BRANCH_SEARCH;
  while (c < C) {
    const R copt = (static_cast<R>(s) * sum_mu + static_cast<R>(r) * sum_nu) / static_cast<R>(r + s);
    const R next_cr = (sum_mu + a_r) - static_cast<R>(r + 1) * a_r;
    const R next_cs = (sum_nu + b_s) - static_cast<R>(s + 1) * b_s;
    const R next_c = dmin(dmin(next_cr, next_cs), C);
    if (c <= copt && copt < next_c) {
      best_c = copt;
      branch = SDCA_BRANCH_BELOW_RHS;
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
  theta_a = (sum_mu - best_c) / static_cast<R>(r);
  theta_b = (sum_nu - best_c) / static_cast<R>(s);
  r_out = r;
  s_out = s;
}

// Two-block simplex by sort and scan: one workgroup per column, the column
// in LDS (m words) with each block sorted in place, one lane scans, the
// workgroup clamps the column.
template <class D, class R, bool GV = false>
__global__ void __launch_bounds__(256)
two_sort_kernel(const D* __restrict__ in, D* __restrict__ out, int64_t m64, int64_t n, R rhs,
                int64_t p_all, const int64_t* __restrict__ col_p,
                sdca_thresholds* __restrict__ thr, int* __restrict__ slow, int all_columns,
                sdca_prox_sets* __restrict__ sets, D* __restrict__ gscratch) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  // GV: beyond the LDS, each workgroup's column in its m-word slice of
  // gscratch (device memory).
  D* sa = GV ? gscratch + static_cast<int64_t>(blockIdx.x) * m64 : reinterpret_cast<D*>(smem_raw);
  __shared__ R sh_ta, sh_tb;
  const int m = static_cast<int>(m64);
  const int64_t count = all_columns ? n : static_cast<int64_t>(slow[0]);
  for (int64_t w = blockIdx.x; w < count; w += gridDim.x) {
    const int64_t j = all_columns ? w : static_cast<int64_t>(slow[2 + w]);
    const int p = clamp_split(col_p ? col_p[j] : p_all, m);
    const int q = m - p;
    const D* col = in + j * m64;
    D* sb = sa + p;
    for (int i = threadIdx.x; i < m; i += blockDim.x) sa[i] = col[i];
    __syncthreads();
    sort_desc_unpadded(sa, p);
    sort_desc_unpadded(sb, q);
    if (threadIdx.x == 0) {
      R ta, tb;
      int ra, rb, branch;
      two_sort_thresholds<D, R>(sa, p, sb, q, rhs, ta, tb, ra, rb, branch);
      if (sets) {
        sets[2 * j] = sdca_prox_sets{0, ra, branch, 0};
        sets[2 * j + 1] = sdca_prox_sets{0, rb, branch, 0};
      }
      sh_ta = ta;
      sh_tb = tb;
      if (thr) {
        thr[2 * j].t = static_cast<double>(ta);
        thr[2 * j].lo = 0;
        thr[2 * j].hi = static_cast<double>(rhs);
        thr[2 * j + 1].t = static_cast<double>(tb);
        thr[2 * j + 1].lo = 0;
        thr[2 * j + 1].hi = static_cast<double>(rhs);
      }
    }
    __syncthreads();
    const D ta = static_cast<D>(sh_ta), tb = static_cast<D>(sh_tb), hi = static_cast<D>(rhs);
    D* dst = out + j * m64;
    for (int i = threadIdx.x; i < m; i += blockDim.x)
      dst[i] = clamp_ref(col[i] - (i < p ? ta : tb), D(0), hi);
    __syncthreads();
  }
  // List mode: the last of the workgroups that took a column zeroes the
  // list's counters for the next call (as in prox_slow_kernel).
  const int64_t workers = count < static_cast<int64_t>(gridDim.x) ? count : gridDim.x;
  if (!all_columns && static_cast<int64_t>(blockIdx.x) < workers && threadIdx.x == 0) {
    __threadfence();
    if (atomicAdd(slow + 1, 1) == static_cast<int>(workers) - 1) {
      atomicExch(slow, 0);
      atomicExch(slow + 1, 0);
    }
  }
}

template <class D, class R>
hipError_t launch_two_sort_t(const ProxLaunch& a, bool all_columns) {
  // List mode: the list is a small fraction of the n columns and usually
  // empty; the grid grows with n (about one workgroup per 1024 columns,
  // 512 to 4096), so that a long list finds workgroups on every CU while
  // an empty one on a small batch costs little to launch.
  const int64_t cap = all_columns ? 4096 : std::min<int64_t>(4096, std::max<int64_t>(512, a.n / 1024));
  const int64_t grid = a.n < cap ? a.n : cap;
  hipLaunchKernelGGL((two_sort_kernel<D, R>), dim3(static_cast<unsigned>(grid > 0 ? grid : 1)),
                     dim3(256), static_cast<size_t>(a.m) * sizeof(D), a.stream,
                     static_cast<const D*>(a.in), static_cast<D*>(a.out), a.m, a.n,
                     static_cast<R>(a.rhs), a.p, a.col_p, a.thr, a.slow, all_columns ? 1 : 0,
                     a.sets, static_cast<D*>(nullptr));
  return hipGetLastError();
}

template <class D, class R>
hipError_t launch_two_sort_global_t(const ProxLaunch& a, void* scratch, size_t scratch_bytes) {
  int64_t grid = static_cast<int64_t>(scratch_bytes / (static_cast<size_t>(a.m) * sizeof(D)));
  if (grid > a.n) grid = a.n;
  if (grid > 4096) grid = 4096;
  if (grid < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL((two_sort_kernel<D, R, true>), dim3(static_cast<unsigned>(grid)), dim3(256),
                     0, a.stream, static_cast<const D*>(a.in), static_cast<D*>(a.out), a.m, a.n,
                     static_cast<R>(a.rhs), a.p, a.col_p, a.thr, a.slow, 1, a.sets,
                     static_cast<D*>(scratch));
  return hipGetLastError();
}

// The two-block simplex (two_simplex.h:18-119) of one column per 256-thread
// workgroup, its passes reading the column from device memory
// (two_family_array): columns beyond the LDS.
template <class D, class R>
__global__ void __launch_bounds__(256)
two_global_kernel(const D* __restrict__ in, D* __restrict__ out, int64_t m64, int64_t n,
                  ProxParamsT<R> pp, const int64_t* __restrict__ col_p,
                  sdca_thresholds* __restrict__ thr, sdca_prox_sets* __restrict__ sets) {
  const int m = static_cast<int>(m64);
  for (int64_t j = blockIdx.x; j < n; j += gridDim.x) {
    const int p = clamp_split(col_p ? col_p[j] : static_cast<int64_t>(pp.p), m);
    const D* col = in + j * m64;
    const ColThr<R> th = two_family_array<256, D, R>(col, m, p, pp);
    if (threadIdx.x == 0) {
      if (thr) {
        thr[2 * j] = sdca_thresholds{static_cast<double>(th.t), static_cast<double>(th.lo),
                                     static_cast<double>(th.hi)};
        thr[2 * j + 1] = sdca_thresholds{static_cast<double>(th.t2), static_cast<double>(th.lo2),
                                         static_cast<double>(th.hi2)};
      }
      if (sets) {
        sets[2 * j] = sdca_prox_sets{0, th.n_mid, th.branch, 0};
        sets[2 * j + 1] = sdca_prox_sets{0, th.n_mid2, th.branch, 0};
      }
    }
    // Every read of the column is behind the solve's last group sum; the
    // clamp may then overwrite it (in == out).
    __syncthreads();
    const D ta = static_cast<D>(th.t), tb = static_cast<D>(th.t2), hi = static_cast<D>(th.hi);
    const D he = D(0) < hi ? hi : D(0);
    D* dst = out + j * m64;
    for (int i = threadIdx.x; i < m; i += 256)
      dst[i] = clamp_med3(col[i] - (i < p ? ta : tb), D(0), he);
    __syncthreads();
  }
}

// thresholds_topk_entropy (topk_entropy.h:20-76) of one column per
// 256-thread workgroup, the column copied into its m-word slice of
// gscratch (device memory), where the entries moved into U are set to -inf:
// the steps of topkent_family (the register kernel's form) over the slice,
// each maximum the first in index order, each log-sum-exp over the rest
// with that maximum excluded.  Columns beyond the LDS.
template <class D, class R>
__device__ inline void slice_argmax(const D* s, int m, R& mx, int& at) {
  R lm = -num<R>::inf();
  int li = INT_MAX;
  for (int i = threadIdx.x; i < m; i += 256) {
    const R x = static_cast<R>(s[i]);
    if (li == INT_MAX || x > lm) {
      lm = x;
      li = i;
    }
  }
  mx = group_max<256>(lm);
  at = group_min<256>((li != INT_MAX && lm == mx) ? li : INT_MAX);
}

template <class D, class R>
__device__ inline R slice_lse_excl(const D* s, int m, R mx, int at) {
  R z = 0;
  for (int i = threadIdx.x; i < m; i += 256) {
    const R x = static_cast<R>(s[i]);
    if (i != at && x > -num<R>::inf()) z += dexp(x - mx);
  }
  return group_sum<256>(z);
}

template <class D, class R>
__global__ void __launch_bounds__(256)
topkent_global_kernel(const D* __restrict__ in, D* __restrict__ out, int64_t m64, int64_t n,
                      int k, sdca_thresholds* __restrict__ thr,
                      sdca_prox_sets* __restrict__ sets, D* __restrict__ gscratch) {
  const int m = static_cast<int>(m64);
  D* const s = gscratch + static_cast<int64_t>(blockIdx.x) * m64;
  const R eps = R(16) * num<R>::eps();
  const R K = static_cast<R>(k);
  for (int64_t j = blockIdx.x; j < n; j += gridDim.x) {
    const D* col = in + j * m64;
    for (int i = threadIdx.x; i < m; i += 256) s[i] = col[i];
    __syncthreads();
    R mx;
    int at;
    slice_argmax<D, R>(s, m, mx, at);
    R z = slice_lse_excl<D, R>(s, m, mx, at);
    R log_z = mx + dlog1p(z);
    const R l1 = dexp(-mx);
    R t, hi;
    int branch, n_u = 0;
    if (k <= 1 || mx - eps <= log_z - dlog(K)) {
      t = isfinite(l1) ? mx + dlog1p(z + l1) : R(0);
      hi = R(1);
      branch = SDCA_BRANCH_U_EMPTY;
    } else {
      R sum_u = 0, k_u = K;
      for (int num_u = 1; num_u < k; ++num_u) {
        const R min_u = mx;
        sum_u += min_u;
        ++n_u;
        // every thread has read the slice (the last group sum) before the
        // owner of the maximum removes it
        if (static_cast<int>(threadIdx.x) == at % 256) s[at] = -num<D>::inf();
        __syncthreads();
        k_u -= R(1);
        slice_argmax<D, R>(s, m, mx, at);
        z = slice_lse_excl<D, R>(s, m, mx, at);
        log_z = mx + dlog1p(z);
        const R tt = log_z - dlog(k_u);
        if (mx - eps <= tt && tt <= min_u + eps) break;
      }
      const R tmp = ((K - k_u) * log_z + k_u * dlog(k_u) - sum_u) / K;
      if (tmp > mx) {
        const R a = (R(1) + z) * dexp(mx - tmp);
        t = tmp + dlog1p(a * K) - dlog(k_u);
        hi = a / (R(1) + a * K);
      } else {
        const R a = dexp(tmp - mx) / K;
        t = mx + dlog1p(z + a) - dlog(k_u / K);
        hi = (R(1) + z) / ((R(1) + z + a) * K);
      }
      branch = SDCA_BRANCH_U_GROWN;
    }
    if (threadIdx.x == 0) {
      if (thr) thr[j] = sdca_thresholds{static_cast<double>(t), 0.0, static_cast<double>(hi)};
      if (sets) sets[j] = sdca_prox_sets{n_u, m - n_u, branch, 0};
    }
    const D td = static_cast<D>(t), hd = static_cast<D>(hi);
    D* dst = out + j * m64;
    for (int i = threadIdx.x; i < m; i += 256) dst[i] = clamp_ref(dexp(col[i] - td), D(0), hd);
    __syncthreads();  // the slice's last reads before the next column's copy
  }
}

template <class D, class R>
hipError_t launch_topkent_global_t(const ProxLaunch& a, void* scratch, size_t scratch_bytes) {
  int64_t grid = static_cast<int64_t>(scratch_bytes / (static_cast<size_t>(a.m) * sizeof(D)));
  if (grid > a.n) grid = a.n;
  if (grid > 4096) grid = 4096;
  if (grid < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL((topkent_global_kernel<D, R>), dim3(static_cast<unsigned>(grid)), dim3(256),
                     0, a.stream, static_cast<const D*>(a.in), static_cast<D*>(a.out), a.m, a.n,
                     static_cast<int>(a.k), a.thr, a.sets, static_cast<D*>(scratch));
  return hipGetLastError();
}

template <class D, class R>
hipError_t launch_two_global_t(const ProxLaunch& a) {
  ProxParamsT<R> pp;
  pp.lo = R(0);
  pp.hi = static_cast<R>(a.rhs);
  pp.rhs = static_cast<R>(a.rhs);
  pp.rho = R(0);
  pp.k = 1;
  pp.rhs_k = R(0);
  pp.op = a.op;
  pp.p = static_cast<int>(a.p);
  const int64_t grid = a.n < 4096 ? a.n : 4096;
  hipLaunchKernelGGL((two_global_kernel<D, R>), dim3(static_cast<unsigned>(grid > 0 ? grid : 1)),
                     dim3(256), 0, a.stream, static_cast<const D*>(a.in), static_cast<D*>(a.out),
                     a.m, a.n, pp, a.col_p, a.thr, a.sets);
  return hipGetLastError();
}

__global__ void clear_kernel(int* p, int count) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < count) p[i] = 0;
}

template <class D>
__global__ void __launch_bounds__(256) lambert_kernel(const D* __restrict__ in, D* __restrict__ out,
                                                      int64_t count) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride)
    out[i] = lambert_w_exp_mixed(in[i]);
}

}  // namespace

hipError_t launch_slow(const ProxLaunch& a, bool all_columns) {
  if (a.data == SDCA_F32 && a.result == SDCA_F32) return launch_slow_t<float, float>(a, all_columns);
  if (a.data == SDCA_F32 && a.result == SDCA_F64) return launch_slow_t<float, double>(a, all_columns);
  if (a.data == SDCA_F64 && a.result == SDCA_F64) return launch_slow_t<double, double>(a, all_columns);
  if (a.data == SDCA_F64 && a.result == SDCA_F32) return launch_slow_t<double, float>(a, all_columns);
  return hipErrorInvalidValue;
}

hipError_t launch_two_sort(const ProxLaunch& a, bool all_columns) {
  if (a.data == SDCA_F32 && a.result == SDCA_F32) return launch_two_sort_t<float, float>(a, all_columns);
  if (a.data == SDCA_F32 && a.result == SDCA_F64) return launch_two_sort_t<float, double>(a, all_columns);
  if (a.data == SDCA_F64 && a.result == SDCA_F64) return launch_two_sort_t<double, double>(a, all_columns);
  if (a.data == SDCA_F64 && a.result == SDCA_F32) return launch_two_sort_t<double, float>(a, all_columns);
  return hipErrorInvalidValue;
}

hipError_t launch_slow_global(const ProxLaunch& a, void* scratch, size_t scratch_bytes) {
  if (a.data == SDCA_F32 && a.result == SDCA_F32)
    return launch_slow_global_t<float, float>(a, scratch, scratch_bytes);
  if (a.data == SDCA_F32 && a.result == SDCA_F64)
    return launch_slow_global_t<float, double>(a, scratch, scratch_bytes);
  if (a.data == SDCA_F64 && a.result == SDCA_F64)
    return launch_slow_global_t<double, double>(a, scratch, scratch_bytes);
  if (a.data == SDCA_F64 && a.result == SDCA_F32)
    return launch_slow_global_t<double, float>(a, scratch, scratch_bytes);
  return hipErrorInvalidValue;
}

hipError_t launch_two_sort_global(const ProxLaunch& a, void* scratch, size_t scratch_bytes) {
  if (a.data == SDCA_F32 && a.result == SDCA_F32)
    return launch_two_sort_global_t<float, float>(a, scratch, scratch_bytes);
  if (a.data == SDCA_F32 && a.result == SDCA_F64)
    return launch_two_sort_global_t<float, double>(a, scratch, scratch_bytes);
  if (a.data == SDCA_F64 && a.result == SDCA_F64)
    return launch_two_sort_global_t<double, double>(a, scratch, scratch_bytes);
  if (a.data == SDCA_F64 && a.result == SDCA_F32)
    return launch_two_sort_global_t<double, float>(a, scratch, scratch_bytes);
  return hipErrorInvalidValue;
}

hipError_t launch_topkent_global(const ProxLaunch& a, void* scratch, size_t scratch_bytes) {
  if (a.data == SDCA_F32 && a.result == SDCA_F32)
    return launch_topkent_global_t<float, float>(a, scratch, scratch_bytes);
  if (a.data == SDCA_F32 && a.result == SDCA_F64)
    return launch_topkent_global_t<float, double>(a, scratch, scratch_bytes);
  if (a.data == SDCA_F64 && a.result == SDCA_F64)
    return launch_topkent_global_t<double, double>(a, scratch, scratch_bytes);
  if (a.data == SDCA_F64 && a.result == SDCA_F32)
    return launch_topkent_global_t<double, float>(a, scratch, scratch_bytes);
  return hipErrorInvalidValue;
}

hipError_t launch_two_global(const ProxLaunch& a) {
  if (a.data == SDCA_F32 && a.result == SDCA_F32) return launch_two_global_t<float, float>(a);
  if (a.data == SDCA_F32 && a.result == SDCA_F64) return launch_two_global_t<float, double>(a);
  if (a.data == SDCA_F64 && a.result == SDCA_F64) return launch_two_global_t<double, double>(a);
  if (a.data == SDCA_F64 && a.result == SDCA_F32) return launch_two_global_t<double, float>(a);
  return hipErrorInvalidValue;
}

hipError_t launch_clear(int* p, int count, hipStream_t stream) {
  hipLaunchKernelGGL(clear_kernel, dim3((count + 255) / 256), dim3(256), 0, stream, p, count);
  return hipGetLastError();
}

hipError_t launch_lambert(const ProxLaunch& a) {
  const int64_t count = a.m * a.n;
  int64_t blocks = (count + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  if (a.data == SDCA_F32) {
    hipLaunchKernelGGL(lambert_kernel<float>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       a.stream, static_cast<const float*>(a.in), static_cast<float*>(a.out), count);
  } else {
    hipLaunchKernelGGL(lambert_kernel<double>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       a.stream, static_cast<const double*>(a.in), static_cast<double*>(a.out), count);
  }
  return hipGetLastError();
}

}  // namespace sdca_gpu
