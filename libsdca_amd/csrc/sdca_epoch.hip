// One SDCA epoch on feature input: the example loop of solver.h:39-51 over a
// given order, each step update_variables (update.h:52-85) with the
// objective's update_dual_variables, for the six multiclass objectives:
//   l2_hinge_topk(_smooth)   prox_topk_simplex_biased  (l2_hinge_topk.h:44-68, 132-159)
//   l2_topk_hinge(_smooth)   prox_knapsack_le_biased   (l2_topk_hinge.h:46-69, 137-163)
//   l2_entropy               prox_two_entropy          (l2_entropy.h:48-74)
//   l2_entropy_topk          prox_topk_entropy_biased  (l2_entropy_topk.h:47-71)
//
// The loop is sequential through W (each example's scores depend on every
// earlier update), so it runs blocked, with the same arithmetic as the
// sequential loop up to the order of the sums in the scores.  For a block
// of B examples in the given order, with rows X_B and W_B = W at its start:
//   S = X_B W_B' and G = X_B X_B' on the matrix cores (the score GEMM);
//   one workgroup takes the block's examples in order: the scores of
//   example k are S_k - sum_{k' < k} G_{k'k} delta_{k'} (W_B with the
//   block's earlier rank-1 updates, applied to x_k), then the dual update
//   of a_i, delta_k = a_old - a_new (zero when sum |delta_k| <= epsilon,
//   where the reference skips the W update), a_i <- a_new;
//   W -= delta_B' X_B: the block's rank-1 updates, applied in order per
//   element.
// Only the last two steps are sequential; the block kernel's dual update is
// the per-column routine of the prox kernels for the same operator (the
// sorted-column thresholds for the simplex and knapsack forms, the one-wave
// Lambert solves for the entropic ones).
#include "common.hpp"
#include "epoch_launch.hpp"
#include "eval_launch.hpp"
#include "prox_impl.hpp"
#include "prox_lambert_wave.hpp"
#include "prox_launch.hpp"
#include "prox_sorted.hpp"

namespace sdca_gpu {

namespace {

constexpr int kEpochThreads = 256;
// LDS of the block kernel (gfx950: 160 KiB per workgroup), less the static
// arrays.
constexpr size_t kEpochLdsBytes = 150 * 1024;
constexpr int kRankJ = 8;  // classes per workgroup of the rank-B update

struct EpochObj {
  int kind;
  int k;
  double c, gamma;
};

// Words of the thresholds' column in LDS: m values, or G C for the register
// form, whose LDS scratch is the slot layout of the whole workgroup.
__host__ __device__ inline int epoch_column_words(int m, int C) {
  const int w = kEpochThreads * C > m ? kEpochThreads * C : m;
  return (w + 3) & ~3;
}

// ||x_i||^2 in the data type (scratch.h:37-40), one wave per example.
template <class D>
__global__ void __launch_bounds__(256)
norms_kernel(const D* __restrict__ X, int64_t n, int64_t d, D* __restrict__ norms) {
  const int lane = static_cast<int>(threadIdx.x) & 63;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (i >= n) return;  // whole waves
  const D* x = X + i * d;
  D s = 0;
  for (int64_t l = lane; l < d; l += 64) s += x[l] * x[l];
  s = group_sum<64>(s);
  if (lane == 0) norms[i] = s;
}

// Rows of the block (one workgroup per row) and their example indices.  An
// index outside [0, n) raises *bad and is read as 0.
template <class D>
__global__ void __launch_bounds__(256)
gather_kernel(const D* __restrict__ X, const int64_t* __restrict__ order, int64_t q0, int64_t n,
              int64_t d, D* __restrict__ XB, int64_t* __restrict__ idx, int* __restrict__ bad) {
  const int k = blockIdx.x;
  int64_t i = order ? order[q0 + k] : q0 + k;
  if (i < 0 || i >= n) {
    if (threadIdx.x == 0) bad[0] = 1;
    i = 0;
  }
  if (threadIdx.x == 0) idx[k] = i;
  const D* src = X + i * d;
  D* dst = XB + static_cast<int64_t>(k) * d;
  for (int64_t l = threadIdx.x; l < d; l += 256) dst[l] = src[l];
}

// The block's examples in order (one workgroup of G threads, all of which
// run every step, including the thresholds).  S: nb x m scores at W_B: after
// example k, row k' > k loses G_{kk'} delta_k (each thread owns the same
// classes j in every row, so the rows it reads are the ones it wrote); the
// rows live in LDS when s_lds (copied in first), else in S itself.
// Gm: nb x nb Gram matrix, Delta: nb x m.  C, KM: the register form of the
// simplex / knapsack thresholds for m - 1 <= G C values (C = 0: the
// sorted-column form only) and k <= KM.
template <class D, class R, int C, int KM>
__global__ void __launch_bounds__(kEpochThreads)
epoch_block_kernel(D* __restrict__ S, const D* __restrict__ Gm, const int64_t* __restrict__ idx,
                   int nb, const D* __restrict__ norms, const int64_t* __restrict__ labels,
                   D* __restrict__ A, D* __restrict__ Delta, EpochObj ob, int m, int s_lds,
                   int* __restrict__ bad) {
  constexpr int G = kEpochThreads;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int cw = epoch_column_words(m, C);
  D* const v = reinterpret_cast<D*>(smem_raw);  // the example's vector, m values
  D* const cb = v + ((m + 3) & ~3);             // the column the thresholds read (cw words)
  D* const dummy = cb + cw;                     // G per-thread dummy words
  D* const Sx = s_lds ? dummy + G : S;          // the block's running scores
  __shared__ R sh_t, sh_lo, sh_hi;
  __shared__ int sh_slow;
  __shared__ D g_row[kEpochBlock];
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  const int kind = ob.kind;
  const R c = static_cast<R>(ob.c), gamma = static_cast<R>(ob.gamma);
  const bool hinge = kind <= SDCA_OBJ_TOPK_HINGE_SMOOTH;
  const bool smooth = kind == SDCA_OBJ_HINGE_TOPK_SMOOTH || kind == SDCA_OBJ_TOPK_HINGE_SMOOTH;
  const bool simplex = kind == SDCA_OBJ_HINGE_TOPK || kind == SDCA_OBJ_HINGE_TOPK_SMOOTH;
  const int op = simplex ? OP_TOPK_SIMPLEX_BIASED : OP_KNAPSACK_LE_BIASED;
  const R knap_hi = simplex ? R(0) : c / static_cast<R>(ob.k);
  if (s_lds) {
    for (int64_t e = tid; e < static_cast<int64_t>(nb) * m; e += G) Sx[e] = S[e];
    __syncthreads();
  }
  for (int k = 0; k < nb; ++k) {
    const int64_t i = idx[k];
    const D norm2 = norms[i];
    D* const arow = A + i * m;
    D* const drow = Delta + static_cast<int64_t>(k) * m;
    const D* const srow = Sx + static_cast<int64_t>(k) * m;
    if (!(norm2 > D(0))) {  // update.h:62: the example changes nothing
      for (int j = tid; j < m; j += G) drow[j] = D(0);
      continue;
    }
    int64_t yl = labels[i];
    if (yl < 0 || yl >= m) {
      if (tid == 0) bad[0] = 1;
      yl = 0;
    }
    const int y = static_cast<int>(yl);
    // 1. The vector to project: axpby(pa, scores, pb, a_old).
    R rho = R(1);
    D pa = D(1), pb = -norm2;  // the entropic objectives
    if (hinge) {
      rho = smooth ? static_cast<R>(norm2) / (static_cast<R>(norm2) + gamma / c) : R(1);
      pa = smooth ? static_cast<D>(rho) / norm2 : D(1) / norm2;
      pb = smooth ? -static_cast<D>(rho) : D(-1);
    }
    for (int j = tid; j < m; j += G) v[j] = pa * srow[j] + pb * arow[j];
    __syncthreads();
    const D vy = v[y];
    if (kind == SDCA_OBJ_ENTROPY) {
      // prox_two_entropy over (label | the rest), alpha = c norm2
      for (int j = tid; j < m; j += G) cb[j == y ? 0 : (j < y ? j + 1 : j)] = v[j];
      __syncthreads();
      const R alpha = c * static_cast<R>(norm2);
      R t, c2;
      twoent_thresholds<D, R, G>(cb, m, 1, tid, alpha, t, c2);
      const D map_a = D(1) / static_cast<D>(alpha);
      const D ta = static_cast<D>(t), tb = static_cast<D>(t + c2);
      const D na = static_cast<D>(-c), nbias = static_cast<D>(c / R(1));
      for (int j = tid; j < m; j += G) {
        const D x = clamp_ref(map_a * lambert_w_exp(v[j] - (j == y ? ta : tb)), D(0), D(1));
        v[j] = (j == y) ? na * x + nbias : na * x;
      }
    } else {
      // The off-label entries shifted by (pa - v_y) (hinge) or -v_y (top-k
      // entropy), compacted into cb.
      const D shift = hinge ? pa - vy : -vy;
      for (int j = tid; j < m; j += G) {
        if (j != y) {
          const D x = v[j] + shift;
          v[j] = x;
          cb[j < y ? j : j - 1] = x;
        }
      }
      __syncthreads();
      const int mp = m - 1;
      if (hinge) {
        bool sorted_form = true;
        if constexpr (C > 0) {
          // The register form over the whole workgroup (slot c of thread g
          // = entry g + G c), which defers to the sorted form only where the
          // reference's biased cone search is needed
          // (topk_simplex_biased.h:57-66).
          D vr[C];
          const int nvalid = (mp - tid + G - 1) / G;
#pragma unroll
          for (int q = 0; q < C; ++q) vr[q] = (q < nvalid) ? cb[tid + G * q] : -num<D>::inf();
          ProxParamsT<R> pp;
          pp.lo = R(0);
          pp.hi = knap_hi;
          pp.rhs = c;
          pp.rho = rho;
          pp.k = ob.k;
          pp.op = op;
          pp.p = 0;
          const ColThr<R> th = simplex
              ? topk_family<G, C, KM, D, R>(vr, mp, nvalid, pp, cb, dummy + tid)
              : knap_family<G, C, D, R>(vr, mp, nvalid, pp);
          if (tid == 0) {
            sh_slow = th.slow ? 1 : 0;
            sh_t = th.t;
            sh_lo = th.lo;
            sh_hi = th.hi;
          }
          __syncthreads();
          sorted_form = sh_slow != 0;
          if (sorted_form) {  // cb served as scratch: compact it again
            for (int j = tid; j < m; j += G)
              if (j != y) cb[j < y ? j : j - 1] = v[j];
            __syncthreads();
          }
        }
        if (sorted_form) {
          sort_desc_unpadded(cb, mp);
          if (tid < 64) {
            R t, lo, hi;
            thresholds_sorted<D, R>(cb, mp, op, R(0), knap_hi, c, rho, ob.k, t, lo, hi);
            if (lane == 0) {
              sh_t = t;
              sh_lo = lo;
              sh_hi = hi;
            }
          }
        }
      } else {  // prox_topk_entropy_biased, alpha = c norm2
        R t, hi;
        entbias_thresholds<D, R, G>(cb, mp, tid, ob.k, c * static_cast<R>(norm2), t, hi);
        if (tid == 0) {
          sh_t = t;
          sh_lo = R(0);
          sh_hi = hi;
        }
      }
      __syncthreads();
      const D t = static_cast<D>(sh_t), lo = static_cast<D>(sh_lo), hi = static_cast<D>(sh_hi);
      const D map_a = hinge ? D(1) : D(1) / static_cast<D>(c * static_cast<R>(norm2));
      R part = 0;
      for (int j = tid; j < m; j += G) {
        if (j != y) {
          const D x = hinge ? clamp_ref(v[j] - t, lo, hi)
                            : clamp_ref(map_a * lambert_w_exp(v[j] - t), D(0), hi);
          v[j] = x;
          part += static_cast<R>(x);
        }
      }
      const R sum = group_sum<G>(part);
      // 3. Recover the variables: the label's entry from the sum, the others
      // negated (and scaled by c for the top-k entropy).
      const D scale = hinge ? D(-1) : static_cast<D>(-c);
      for (int j = tid; j < m; j += G) {
        if (j == y) {
          v[j] = hinge ? static_cast<D>(dmin(c, sum)) : static_cast<D>(c * dmin(R(1), sum));
        } else {
          v[j] = v[j] * scale;
        }
      }
    }
    // a_old - a_new (sdca_blas_axpy with -1), its 1-norm, a_i <- a_new.
    D part = 0;
    for (int j = tid; j < m; j += G) {
      const D an = v[j];
      const D dl = arow[j] + D(-1) * an;
      drow[j] = dl;
      arow[j] = an;
      part += fabs(dl);
    }
    const D asum = group_sum<G>(part);  // also orders v's last reads before the next writes
    if (asum > num<D>::eps() && k + 1 < nb) {
      // The later rows of the block see this update: S_k' -= G_kk' delta_k.
      if (tid < nb) g_row[tid] = Gm[k * nb + tid];
      __syncthreads();
      for (int j = tid; j < m; j += G) {
        const D dl = drow[j];
        for (int q = k + 1; q < nb; ++q) Sx[static_cast<int64_t>(q) * m + j] -= g_row[q] * dl;
      }
    } else if (!(asum > num<D>::eps())) {
      for (int j = tid; j < m; j += G) drow[j] = D(0);
    }
    __syncthreads();
  }
}

// The block's skinny products P = X_B Y' (nb <= kEpochBlock rows; Y: M x d,
// the primal variables or X_B itself), split over the features: workgroup
// (bx, ks) has four waves of JW classes each over features
// [ks kc, (ks + 1) kc), lane l taking features l, l + 64, ...; the partial
// sums of the splits are added in split order by skinny_sum_kernel.
template <class D, int JW>
__global__ void __launch_bounds__(256)
skinny_partial_kernel(const D* __restrict__ XB, const D* __restrict__ Y, D* __restrict__ P,
                      int nb, int64_t M, int64_t d, int64_t kc) {
  const int wave = static_cast<int>(threadIdx.x) >> 6, lane = static_cast<int>(threadIdx.x) & 63;
  const int64_t j0 = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * JW;
  const int64_t l0 = static_cast<int64_t>(blockIdx.y) * kc;
  const int64_t l1 = (l0 + kc < d) ? l0 + kc : d;
  D acc[JW][kEpochBlock];
#pragma unroll
  for (int jw = 0; jw < JW; ++jw)
#pragma unroll
    for (int e = 0; e < kEpochBlock; ++e) acc[jw][e] = D(0);
  for (int64_t l = l0 + lane; l < l1; l += 64) {
    D y[JW];
#pragma unroll
    for (int jw = 0; jw < JW; ++jw) y[jw] = (j0 + jw < M) ? Y[(j0 + jw) * d + l] : D(0);
#pragma unroll
    for (int e = 0; e < kEpochBlock; ++e) {
      if (e < nb) {
        const D x = XB[static_cast<int64_t>(e) * d + l];
#pragma unroll
        for (int jw = 0; jw < JW; ++jw) acc[jw][e] += x * y[jw];
      }
    }
  }
  D* const out = P + static_cast<int64_t>(blockIdx.y) * kEpochBlock * M;
#pragma unroll
  for (int jw = 0; jw < JW; ++jw) {
#pragma unroll
    for (int e = 0; e < kEpochBlock; ++e) {
      const D s = group_sum<64>(acc[jw][e]);
      if (lane == 0 && e < nb && j0 + jw < M) out[static_cast<int64_t>(e) * M + j0 + jw] = s;
    }
  }
}

template <class D>
__global__ void __launch_bounds__(256)
skinny_sum_kernel(const D* __restrict__ P, D* __restrict__ out, int nb, int64_t M, int ksplit) {
  const int64_t o = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (o >= static_cast<int64_t>(nb) * M) return;
  const int64_t e = o / M, j = o % M;
  D s = P[e * M + j];
  for (int ks = 1; ks < ksplit; ++ks) s += P[(static_cast<int64_t>(ks) * kEpochBlock + e) * M + j];
  out[o] = s;
}

// Feature split of the skinny products: chunks of at least 512 features, at
// most kSkinnySplits of them.
constexpr int kSkinnySplits = 8;
inline int64_t skinny_chunk(int64_t d) {
  const int64_t c = (d + kSkinnySplits - 1) / kSkinnySplits;
  return c < 512 ? 512 : c;
}

template <class D>
hipError_t launch_skinny(const D* XB, const D* Y, D* out, D* P, int nb, int64_t M, int64_t d,
                         hipStream_t stream) {
  constexpr int JW = sizeof(D) == 4 ? 4 : 2;
  const int64_t kc = skinny_chunk(d);
  const int ksplit = static_cast<int>((d + kc - 1) / kc);
  const dim3 grid(static_cast<unsigned>((M + 4 * JW - 1) / (4 * JW)), static_cast<unsigned>(ksplit));
  hipLaunchKernelGGL((skinny_partial_kernel<D, JW>), grid, dim3(256), 0, stream, XB, Y, P, nb, M,
                     d, kc);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t total = static_cast<int64_t>(nb) * M;
  hipLaunchKernelGGL((skinny_sum_kernel<D>), dim3(static_cast<unsigned>((total + 255) / 256)),
                     dim3(256), 0, stream, P, out, nb, M, ksplit);
  return hipGetLastError();
}

// W -= delta_B' X_B: each element takes the block's rank-1 updates in order,
// w <- w - x_l delta_j (sdca_blas_ger with alpha -1).  Workgroup: 256
// consecutive features of kRankJ classes.
template <class D>
__global__ void __launch_bounds__(256)
rank_update_kernel(D* __restrict__ W, const D* __restrict__ Delta, const D* __restrict__ XB,
                   int nb, int64_t m, int64_t d) {
  __shared__ D dl[kEpochBlock][kRankJ];
  const int64_t j0 = static_cast<int64_t>(blockIdx.y) * kRankJ;
  for (int e = threadIdx.x; e < kEpochBlock * kRankJ; e += 256) {
    const int k = e / kRankJ, jj = e % kRankJ;
    dl[k][jj] = (k < nb && j0 + jj < m) ? Delta[static_cast<int64_t>(k) * m + j0 + jj] : D(0);
  }
  __syncthreads();
  const int64_t l = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (l >= d) return;
  D xk[kEpochBlock];
#pragma unroll
  for (int k = 0; k < kEpochBlock; ++k) xk[k] = (k < nb) ? XB[static_cast<int64_t>(k) * d + l] : D(0);
#pragma unroll
  for (int jj = 0; jj < kRankJ; ++jj) {
    const int64_t j = j0 + jj;
    if (j < m) {
      D w = W[j * d + l];
#pragma unroll
      for (int k = 0; k < kEpochBlock; ++k)
        if (k < nb) w = w - xk[k] * dl[k][jj];
      W[j * d + l] = w;
    }
  }
}

template <class D, class R, int C, int KM>
hipError_t launch_block(D* S, const D* Gm, const int64_t* idx, int nb, const D* norms,
                        const EpochLaunch& a, D* Delta, const EpochObj& ob, int* bad) {
  const int m = static_cast<int>(a.m);
  size_t lds = (static_cast<size_t>((m + 3) & ~3) + epoch_column_words(m, C) + kEpochThreads) *
               sizeof(D);
  // The block's scores in LDS where they fit (the running update then costs
  // LDS instead of global round trips).
  const size_t s_bytes = static_cast<size_t>(nb) * static_cast<size_t>(m) * sizeof(D);
  const int s_lds = lds + s_bytes <= kEpochLdsBytes ? 1 : 0;
  if (s_lds) lds += s_bytes;
  hipLaunchKernelGGL((epoch_block_kernel<D, R, C, KM>), dim3(1), dim3(kEpochThreads), lds,
                     a.stream, S, Gm, idx, nb, norms, a.labels, static_cast<D*>(a.A), Delta, ob,
                     m, s_lds, bad);
  return hipGetLastError();
}

// The block kernel's register form for m - 1 values and k (C = 0: the
// sorted-column form only).
template <class D, class R>
hipError_t launch_block_for(D* S, const D* Gm, const int64_t* idx, int nb, const D* norms,
                            const EpochLaunch& a, D* Delta, const EpochObj& ob, int* bad) {
  const int64_t mp = a.m - 1;
  const bool simplex = a.kind == SDCA_OBJ_HINGE_TOPK || a.kind == SDCA_OBJ_HINGE_TOPK_SMOOTH;
  const bool big_k = simplex && a.k > 8;
  if (mp > 2048 || big_k || a.kind > SDCA_OBJ_TOPK_HINGE_SMOOTH)
    return launch_block<D, R, 0, 5>(S, Gm, idx, nb, norms, a, Delta, ob, bad);
  if (!simplex || a.k <= 5) {
    if (mp <= 256) return launch_block<D, R, 1, 5>(S, Gm, idx, nb, norms, a, Delta, ob, bad);
    if (mp <= 1024) return launch_block<D, R, 4, 5>(S, Gm, idx, nb, norms, a, Delta, ob, bad);
    return launch_block<D, R, 8, 5>(S, Gm, idx, nb, norms, a, Delta, ob, bad);
  }
  if (mp <= 256) return launch_block<D, R, 1, 8>(S, Gm, idx, nb, norms, a, Delta, ob, bad);
  if (mp <= 1024) return launch_block<D, R, 4, 8>(S, Gm, idx, nb, norms, a, Delta, ob, bad);
  return launch_block<D, R, 8, 8>(S, Gm, idx, nb, norms, a, Delta, ob, bad);
}

template <class D, class R>
hipError_t launch_epoch_t(const EpochLaunch& a, int** flag_dev) {
  const int64_t d = a.d, m = a.m, n = a.n;
  const int64_t B = kEpochBlock;
  // Workspace: [flag (256 B) | idx | XB | S | G | Delta | norms]
  char* p = static_cast<char*>(a.ws);
  int* bad = reinterpret_cast<int*>(p);
  p += 256;
  int64_t* idx = reinterpret_cast<int64_t*>(p);
  p += B * sizeof(int64_t);
  D* XB = reinterpret_cast<D*>(p);
  D* S = XB + B * d;
  D* Gm = S + B * m;
  D* Delta = Gm + B * B;
  D* P = Delta + B * m;  // the skinny products' partial sums
  D* norms_ws = P + kSkinnySplits * B * (m > B ? m : B);
  *flag_dev = bad;
  hipError_t e = launch_clear(bad, 1, a.stream);
  if (e != hipSuccess) return e;
  const D* X = static_cast<const D*>(a.X);
  D* W = static_cast<D*>(a.W);
  const D* norms = static_cast<const D*>(a.norms);
  if (!norms) {
    hipLaunchKernelGGL((norms_kernel<D>), dim3(static_cast<unsigned>((n + 3) / 4)), dim3(256), 0,
                       a.stream, X, n, d, norms_ws);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    norms = norms_ws;
  }
  EpochObj ob;
  ob.kind = a.kind;
  ob.k = a.k;
  ob.c = a.c;
  ob.gamma = a.gamma;
  const dim3 rank_grid(static_cast<unsigned>((d + 255) / 256),
                       static_cast<unsigned>((m + kRankJ - 1) / kRankJ));
  for (int64_t q0 = 0; q0 < a.count; q0 += B) {
    const int nb = static_cast<int>(a.count - q0 < B ? a.count - q0 : B);
    hipLaunchKernelGGL((gather_kernel<D>), dim3(static_cast<unsigned>(nb)), dim3(256), 0, a.stream,
                       X, a.order, q0, n, d, XB, idx, bad);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if ((e = launch_skinny<D>(XB, W, S, P, nb, m, d, a.stream)) != hipSuccess) return e;
    if ((e = launch_skinny<D>(XB, XB, Gm, P, nb, nb, d, a.stream)) != hipSuccess) return e;
    if ((e = launch_block_for<D, R>(S, Gm, idx, nb, norms, a, Delta, ob, bad)) != hipSuccess)
      return e;
    hipLaunchKernelGGL((rank_update_kernel<D>), rank_grid, dim3(256), 0, a.stream, W, Delta, XB,
                       nb, m, d);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace

size_t epoch_workspace_bytes(int data, int64_t d, int64_t m, int64_t n, bool norms_given) {
  const size_t es = data == SDCA_F32 ? 4 : 8;
  const size_t B = kEpochBlock;
  const size_t mb = static_cast<size_t>(m) > B ? static_cast<size_t>(m) : B;
  return 256 + B * sizeof(int64_t) +
         es * (B * static_cast<size_t>(d) + 2 * B * static_cast<size_t>(m) + B * B +
               kSkinnySplits * B * mb + (norms_given ? 0 : static_cast<size_t>(n)));
}

int64_t epoch_max_m(int data) {
  // v and the thresholds' column, each m values, in at most 128 KiB of LDS
  return kMaxColumnBytes / (2 * (data == SDCA_F32 ? 4 : 8));
}

hipError_t launch_epoch(const EpochLaunch& a, int** flag_dev) {
  if (a.data == SDCA_F32 && a.result == SDCA_F32) return launch_epoch_t<float, float>(a, flag_dev);
  if (a.data == SDCA_F32 && a.result == SDCA_F64) return launch_epoch_t<float, double>(a, flag_dev);
  if (a.data == SDCA_F64 && a.result == SDCA_F64) return launch_epoch_t<double, double>(a, flag_dev);
  return hipErrorInvalidValue;
}

}  // namespace sdca_gpu
