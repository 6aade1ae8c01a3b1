// One SDCA epoch on feature input: the example loop of solver.h:39-51 over a
// given order, each step update_variables (update.h:52-85) with the
// objective's update_dual_variables, for the six multiclass objectives
//   l2_hinge_topk(_smooth)   prox_topk_simplex_biased  (l2_hinge_topk.h:44-68, 132-159)
//   l2_topk_hinge(_smooth)   prox_knapsack_le_biased   (l2_topk_hinge.h:46-69, 137-163)
//   l2_entropy               prox_two_entropy          (l2_entropy.h:48-74)
//   l2_entropy_topk          prox_topk_entropy_biased  (l2_entropy_topk.h:47-71)
// and the three multilabel ones, labels first (output.h:121-164):
//   l2_multilabel_hinge(_smooth)  prox_two_simplex  (l2_multilabel_hinge.h:40-66, 137-166)
//   l2_multilabel_entropy         prox_two_entropy  (l2_multilabel_entropy.h:43-69)
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
// The block kernel's objective families (one instantiation each, so that a
// kernel holds only its own solve): the multiclass hinges (kinds 0..3), the
// multiclass entropy, the top-k entropy, the multilabel hinges, the
// multilabel entropy.
constexpr int kFamHinge = 0, kFamEnt = 1, kFamTopkEnt = 2, kFamMlHinge = 3, kFamMlEnt = 4;
// LDS of the block kernel (gfx950: 160 KiB per workgroup), less the static
// arrays.
constexpr size_t kEpochLdsBytes = 144 * 1024;
constexpr int kRankJ = 8;  // classes per workgroup of the rank-B update
// Delta rows whose loads the score corrections issue together (their
// registers: kFixRows x PF values).
constexpr int kFixRows = 8;

struct EpochObj {
  int kind;
  int k;
  double c, gamma;
  // Kernel input: every update reaches the later examples' scores (the
  // reference reads A itself, update.h:88-107), not only those above
  // epsilon (the W update's test, update.h:78-84).
  int kernel;
};

// The block's delta rows in LDS: for the row sizes where kEpochBlock rows of
// m <= kEpochThreads PF values always fit next to the column buffers.
template <class D>
__host__ __device__ constexpr bool epoch_delta_in_lds(int PF) {
  return PF > 0 && (sizeof(D) == 4 ? PF <= 4 : PF <= 1);
}

// Words of the block's delta rows in LDS: kEpochBlock rows of m and the
// padding that the last row's unclamped slot reads run into (the thread
// slots cover kEpochThreads PF >= m columns).
__host__ __device__ inline int epoch_dx_words(int m, int PF) {
  return kEpochBlock * m + (kEpochThreads * PF > m ? kEpochThreads * PF - m : 0);
}

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

// Example index at position q of the order (q itself without one).  An
// index outside [0, n) reads as 0 (the block kernel raises the flag).
__device__ inline int64_t block_row(const int64_t* order, int64_t q, int64_t n) {
  const int64_t i = order ? order[q] : q;
  return (i >= 0 && i < n) ? i : 0;
}

// Kernel input (update.h:88-107), the training set's n x n kernel matrix K
// (row i = K_i, the reference's column i): norm2 = K_ii.
template <class D>
__global__ void __launch_bounds__(256)
kernel_diag_kernel(const D* __restrict__ K, int64_t n, D* __restrict__ norms) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) norms[i] = K[i * n + i];
}

// Kernel input: the block's Gram matrix is K itself, Gm[e][f] = K[i_e][i_f]
// (x_e . x_f of the feature form).
template <class D>
__global__ void __launch_bounds__(256)
kernel_gram_kernel(const D* __restrict__ K, const int64_t* __restrict__ order, int64_t q0,
                   int64_t n, int nb, D* __restrict__ Gm) {
  const int o = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
  if (o >= nb * nb) return;
  const int e = o / nb, f = o % nb;
  Gm[o] = K[block_row(order, q0 + e, n) * n + block_row(order, q0 + f, n)];
}

// Kernel input: the transposed copy At (m x n) that the score products read
// as their W takes the block's updated dual variables, At[c][i] = A[i][c].
template <class D>
__global__ void __launch_bounds__(256)
kernel_at_kernel(const D* __restrict__ A, D* __restrict__ At, const int64_t* __restrict__ order,
                 int64_t q0, int64_t n, int nb, int64_t m) {
  const int64_t o = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (o >= static_cast<int64_t>(nb) * m) return;
  const int64_t k = o / m, c = o % m;
  const int64_t i = block_row(order, q0 + k, n);
  At[c * n + i] = A[i * m + c];
}

// The thread's columns j = tid + G q for every q < PF (m <= G PF), with
// ok = j < m: the loops stay branch-free (exec-masked branches around each
// slot cost more than the slot's work), so loads read the clamped column
// j < m ? j : m - 1 and the stores of slots past m go to the thread's dummy
// word.  PF = 0: every j = tid (mod G) below m, q = 0, ok = true.
template <int PF, class F>
__device__ __forceinline__ void for_cols(int tid, int m, F&& f) {
  if constexpr (PF > 0) {
#pragma unroll
    for (int q = 0; q < PF; ++q) {
      const int j = tid + kEpochThreads * q;
      f(j, q, j < m);
    }
  } else {
    for (int j = tid; j < m; j += kEpochThreads) f(j, 0, true);
  }
}

// The block's examples in order (one workgroup of G threads, all of which
// run every step, including the thresholds).  S: nb x m scores at W_B;
// example k's scores are S_k - sum_{k' < k} G_{k'k} delta_{k'} over the
// earlier examples that changed W, in the order of the sequential updates
// (each thread owns the same classes j in every row, so the delta entries it
// reads are the ones it wrote).  The block's delta rows live in LDS where
// kEpochBlock rows always fit (DL), else in Delta (nb x m), which holds them
// for the rank update in any case.  Gm: nb x nb Gram matrix.  gdummy: G
// words of global memory, the threads' sinks for stores past m.  C, KM: the
// register form of the simplex / knapsack thresholds for m - 1 <= G C values
// (C = 0: the sorted-column form only) and k <= KM.  PF > 0 (m <= G PF):
// each thread keeps its entries of the example's vector, of a_i and of S_k
// in registers, the next example's a_i and S_k loaded while this one runs;
// PF = 0 keeps the vector in LDS and reads a_i and S_k as it goes.  GV
// (PF = 0, rows beyond the LDS): the vector, the thresholds' column and the
// labels live in gv (global memory, the workspace; L2-resident at the sizes
// where LDS ends), the same code reading them there.
template <class D, class R, int FK, int C, int KM, int PF, bool GV = false>
__global__ void __launch_bounds__(kEpochThreads)
epoch_block_kernel(const D* __restrict__ S, const D* __restrict__ Gm,
                   const int64_t* __restrict__ order, int64_t q0, int64_t n, int nb,
                   const D* __restrict__ norms, const int64_t* __restrict__ labels,
                   const int64_t* __restrict__ offsets, D* __restrict__ A,
                   D* __restrict__ Delta, D* __restrict__ gdummy, EpochObj ob, int m,
                   int* __restrict__ bad, D* __restrict__ gv) {
  constexpr int G = kEpochThreads;
  constexpr int PQ = PF > 0 ? PF : 1;
  constexpr bool DL = epoch_delta_in_lds<D>(PF);
  static_assert(!GV || (PF == 0 && !DL), "global vectors for the PF = 0 form");
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int cw = epoch_column_words(m, C);
  // the example's vector (PF = 0), m values
  D* const v = GV ? gv : reinterpret_cast<D*>(smem_raw);
  D* const cb = v + ((m + 3) & ~3);  // the column the thresholds read (cw words)
  // G per-thread dummy words (always in LDS)
  D* const dummy = GV ? reinterpret_cast<D*>(smem_raw) : cb + cw;
  D* const Dx = DL ? dummy + G : Delta;  // the block's delta rows
  // the example's labels (multilabel), m ints after the D words
  int* const lab = GV ? reinterpret_cast<int*>(cb + cw)
                      : reinterpret_cast<int*>(dummy + G + (DL ? epoch_dx_words(m, PF) : 0));
  __shared__ R sh_t, sh_lo, sh_hi;
  __shared__ int sh_slow;
  __shared__ D sh_vy;
  __shared__ D g_all[kEpochBlock * kEpochBlock];
  __shared__ D sh_norm[kEpochBlock];
  __shared__ int64_t sh_i[kEpochBlock];
  __shared__ int sh_y[kEpochBlock];   // multiclass: the label; multilabel: the label count
  __shared__ int64_t sh_off[kEpochBlock];
  __shared__ int sh_badex;
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & 63;
  D* const ld = dummy + tid;   // LDS sink
  D* const gd = gdummy + tid;  // global sink
  const int kind = ob.kind;
  const R c = static_cast<R>(ob.c), gamma = static_cast<R>(ob.gamma);
  constexpr bool hinge = FK == kFamHinge;
  constexpr bool ml = FK == kFamMlHinge || FK == kFamMlEnt;
  const bool smooth = kind == SDCA_OBJ_HINGE_TOPK_SMOOTH || kind == SDCA_OBJ_TOPK_HINGE_SMOOTH;
  const bool simplex = kind == SDCA_OBJ_HINGE_TOPK || kind == SDCA_OBJ_HINGE_TOPK_SMOOTH;
  const int op = simplex ? OP_TOPK_SIMPLEX_BIASED : OP_KNAPSACK_LE_BIASED;
  const R knap_hi = simplex ? R(0) : c / static_cast<R>(ob.k);
  // The block's indices, norms, labels and Gram matrix in LDS.
  // An index outside [0, n) or a label outside [0, m) raises *bad and is
  // read as 0; a multilabel example with a label count outside [1, m - 1]
  // (or, below, labels that are not distinct, sorted and in [0, m)) raises
  // it and is skipped (validate_labels_and_offsets, output.h:184-206).
  if (tid == 0) sh_badex = -1;
  if (tid < nb) {
    int64_t i = order ? order[q0 + tid] : q0 + tid;
    if (i < 0 || i >= n) {
      bad[0] = 1;
      i = 0;
    }
    int64_t yl;
    if (ml) {
      sh_off[tid] = offsets[i];
      yl = offsets[i + 1] - offsets[i];
      // a negative start is as broken as a bad count: skipped, never read
      if (yl < 1 || yl >= m || offsets[i] < 0) {
        bad[0] = 1;
        yl = 0;
      }
    } else {
      yl = labels[i];
      if (yl < 0 || yl >= m) {
        bad[0] = 1;
        yl = 0;
      }
    }
    sh_i[tid] = i;
    sh_norm[tid] = norms[i];
    sh_y[tid] = static_cast<int>(yl);
  }
  for (int e = tid; e < nb * nb; e += G) g_all[e] = Gm[e];
  __syncthreads();
  // PF > 0: the next example's a_i and S row are loaded into anext / snext
  // one example ahead and copied at the top of its step, where nothing newer
  // is in flight (so the wait for them waits for nothing else).
  D acur[PQ], anext[PQ], scur[PQ], snext[PQ], vr[PQ];
  if constexpr (PF > 0) {
    const D* a0 = A + sh_i[0] * m;
    for_cols<PF>(tid, m, [&](int j, int q, bool ok) {
      const int jc = ok ? j : m - 1;
      anext[q] = a0[jc];
      snext[q] = S[jc];
    });
  }
  // The example's vector entry of slot (j, q): registers or LDS.
  auto getv = [&](int j, int q) -> D {
    if constexpr (PF > 0) return vr[q];
    else return v[j];
  };
  auto setv = [&](int j, int q, D x) {
    if constexpr (PF > 0) vr[q] = x;
    else v[j] = x;
  };
  unsigned changed = 0;  // bit k': example k' changed W
  for (int k = 0; k < nb; ++k) {
    const int64_t i = sh_i[k];
    const D norm2 = sh_norm[k];
    const int y = sh_y[k];  // multilabel: the label count nl
    D* const arow = A + i * m;
    D* const drow = Delta + static_cast<int64_t>(k) * m;
    const D* const srow = S + static_cast<int64_t>(k) * m;
    const bool has_next = k + 1 < nb;
    if constexpr (PF > 0) {
#pragma unroll
      for (int q = 0; q < PF; ++q) {
        acur[q] = anext[q];
        scur[q] = snext[q];
      }
      // The next example's a as A holds it now (replaced below when it is
      // this example, the only one whose update is still to come).
      if (has_next) {
        const D* an = A + sh_i[k + 1] * m;
        const D* sn = srow + m;
        for_cols<PF>(tid, m, [&](int j, int q, bool ok) {
          const int jc = ok ? j : m - 1;
          anext[q] = an[jc];
          snext[q] = sn[jc];
        });
      }
    }
    if (ml && y > 0) {
      // The example's labels into LDS, checked distinct, sorted, in range.
      const int64_t o0 = sh_off[k];
      for (int q = tid; q < y; q += G) {
        const int64_t l = labels[o0 + q];
        const bool okl = l >= 0 && l < m && (q == 0 || l > labels[o0 + q - 1]);
        if (!okl) {
          bad[0] = 1;
          sh_badex = k;
        }
        lab[q] = okl ? static_cast<int>(l) : 0;
      }
    }
    if (!(norm2 > D(0)) || (ml && y == 0)) {  // update.h:62: the example changes nothing
      for_cols<PF>(tid, m, [&](int j, int q, bool ok) { *(ok ? drow + j : gd) = D(0); });
      continue;
    }
    // 1. The vector to project: axpby(pa, scores, pb, a_old).
    R rho = R(1);
    D pa = D(1), pb = -norm2;  // the entropic objectives
    if (hinge) {
      rho = smooth ? static_cast<R>(norm2) / (static_cast<R>(norm2) + gamma / c) : R(1);
      pa = smooth ? static_cast<D>(rho) / norm2 : D(1) / norm2;
      pb = smooth ? -static_cast<D>(rho) : D(-1);
    } else if (kind == SDCA_OBJ_MULTILABEL_HINGE) {  // l2_multilabel_hinge.h:50-54
      pa = D(1) / norm2;
      pb = D(-1);
    } else if (kind == SDCA_OBJ_MULTILABEL_HINGE_SMOOTH) {  // l2_multilabel_hinge.h:147-153
      const R gdc = gamma / c;
      pa = static_cast<D>(R(1) / (static_cast<R>(norm2) + gdc));
      pb = -static_cast<D>(static_cast<R>(norm2) / (static_cast<R>(norm2) + gdc));
    }
    if constexpr (PF > 0) {
      // The corrections row by row in increasing r, kFixRows rows' loads at
      // a time (the same sequence of subtractions per entry).  The row set
      // is uniform: readfirstlane keeps it and the row indices in scalar
      // registers, and G_rk comes from lane r's copy of column k of the Gram
      // matrix (one LDS read per example) by readlane.  Rows in LDS are read
      // unclamped (the padding after the last row holds the tail past m), so
      // a row's slots are one address with constant offsets.
      // Past the last row the index reads as 31 (ctz of the guard bit; row
      // 31 and lane 31 exist, and its values are not used).
      const D gk = g_all[(lane < nb ? lane : 0) * nb + k];
      unsigned rem = __builtin_amdgcn_readfirstlane(changed & ((1u << k) - 1u));
      const int nrows = __builtin_popcount(rem);
      for (int base = 0; base < nrows; base += kFixRows) {
        int rr[kFixRows];
        D g[kFixRows];
#pragma unroll
        for (int b = 0; b < kFixRows; ++b) {
          rr[b] = __builtin_ctz(rem | 0x80000000u);
          rem &= rem - 1u;
          g[b] = read_lane(gk, rr[b]);
        }
        D dv[kFixRows][PQ];
#pragma unroll
        for (int b = 0; b < kFixRows; ++b) {
          const D* drr = Dx + static_cast<int64_t>(rr[b]) * m;
          for_cols<PF>(tid, m, [&](int j, int q, bool ok) {
            dv[b][q] = drr[(DL || ok) ? j : m - 1];
          });
        }
#pragma unroll
        for (int b = 0; b < kFixRows; ++b) {
          if (base + b < nrows) {
#pragma unroll
            for (int q = 0; q < PF; ++q) scur[q] -= g[b] * dv[b][q];
          }
        }
      }
    }
    for_cols<PF>(tid, m, [&](int j, int q, bool ok) {
      D sc, ao;
      if constexpr (PF > 0) {
        sc = scur[q];
        ao = acur[q];
      } else {
        sc = srow[j];
        for (int r = 0; r < k; ++r)
          if ((changed >> r) & 1u) sc -= g_all[r * nb + k] * Dx[static_cast<int64_t>(r) * m + j];
        ao = arow[j];
      }
      const D x = pa * sc + pb * ao;
      setv(j, q, x);
      if constexpr (PF > 0) *((ok && j == y) ? &sh_vy : ld) = x;
    });
    __syncthreads();
    if (ml && sh_badex == k) {  // labels not valid: the example is skipped
      for_cols<PF>(tid, m, [&](int j, int q, bool ok) { *(ok ? drow + j : gd) = D(0); });
      __syncthreads();
      continue;
    }
    const D vy = PF > 0 ? sh_vy : v[y];
    if constexpr (ml) {
      // The labels first (output.h:121-164): label r of the example (the
      // r-th smallest) to row r, the other rows after them in index order;
      // the two-block prox, then the recovery.
      const int nl = y;
      auto rank_of = [&](int j, bool& is_lab) {
        int lo = 0, hi = nl;  // the count of labels below j
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (lab[mid] < j) lo = mid + 1;
          else hi = mid;
        }
        is_lab = lo < nl && lab[lo] == j;
        return lo;
      };
      constexpr bool ent = FK == kFamMlEnt;
      const D half = pa / D(2);
      for_cols<PF>(tid, m, [&](int j, int q, bool ok) {
        bool is_lab;
        const int r = rank_of(j, is_lab);
        const D x = getv(j, q);
        const D xx = ent ? x : (is_lab ? half - x : half + x);
        setv(j, q, xx);
        *(ok ? cb + (is_lab ? r : nl + j - r) : ld) = xx;
      });
      __syncthreads();
      if constexpr (ent) {  // prox_two_entropy, alpha = c norm2 (l2_multilabel_entropy.h:55-68)
        const R alpha = c * static_cast<R>(norm2);
        R t, c2;
        twoent_thresholds<D, R, G, true>(cb, m, nl, tid, alpha, t, c2);
        const D map_a = D(1) / static_cast<D>(alpha);
        const D ta = static_cast<D>(t), tb = static_cast<D>(t + c2);
        const D na = static_cast<D>(-c), nbias = static_cast<D>(c / static_cast<R>(nl));
        for_cols<PF>(tid, m, [&](int j, int q, bool ok) {
          bool is_lab;
          rank_of(j, is_lab);
          const D x = clamp_ref(map_a * lambert_w_exp_nb(getv(j, q) - (is_lab ? ta : tb)), D(0),
                                D(1));
          setv(j, q, is_lab ? na * x + nbias : na * x);
        });
      } else {  // prox_two_simplex, rhs c (l2_multilabel_hinge.h:59-65)
        D ta = D(0), tb = D(0);  // the two blocks' thresholds
        ProxParamsT<R> pp;
        pp.lo = R(0);
        pp.hi = c;
        pp.rhs = c;
        pp.rho = R(0);
        pp.k = 1;
        pp.op = OP_TWO_SIMPLEX;
        pp.p = nl;
        if constexpr (C > 0) {
          D vq[C];
          const int nvalid = (m - tid + G - 1) / G;
#pragma unroll
          for (int q = 0; q < C; ++q) {
            const D x = cb[tid + G * q];
            vq[q] = (q < nvalid) ? x : -num<D>::inf();
          }
          const ColThr<R> th = two_family_slots<G, C, C, D, R>(vq, m, nl, pp);
          ta = static_cast<D>(th.t);
          tb = static_cast<D>(th.t2);
        } else {
          // Rows beyond the register slots: the same passes over the LDS
          // column.
          const ColThr<R> th = two_family_array<G, D, R>(cb, m, nl, pp);
          ta = static_cast<D>(th.t);
          tb = static_cast<D>(th.t2);
        }
        const D hc = static_cast<D>(c);
        for_cols<PF>(tid, m, [&](int j, int q, bool ok) {
          bool is_lab;
          rank_of(j, is_lab);
          const D x = getv(j, q);
          setv(j, q, is_lab ? clamp_ref(x - ta, D(0), hc) : D(-1) * clamp_ref(x - tb, D(0), hc));
        });
      }
    } else if constexpr (FK == kFamEnt) {
      // prox_two_entropy over (label | the rest), alpha = c norm2
      for_cols<PF>(tid, m, [&](int j, int q, bool ok) {
        *(ok ? cb + (j == y ? 0 : (j < y ? j + 1 : j)) : ld) = getv(j, q);
      });
      __syncthreads();
      const R alpha = c * static_cast<R>(norm2);
      R t, c2;
      twoent_thresholds<D, R, G, true>(cb, m, 1, tid, alpha, t, c2);
      const D map_a = D(1) / static_cast<D>(alpha);
      const D ta = static_cast<D>(t), tb = static_cast<D>(t + c2);
      const D na = static_cast<D>(-c), nbias = static_cast<D>(c / R(1));
      for_cols<PF>(tid, m, [&](int j, int q, bool ok) {
        const D x = clamp_ref(map_a * lambert_w_exp_nb(getv(j, q) - (j == y ? ta : tb)), D(0), D(1));
        setv(j, q, (j == y) ? na * x + nbias : na * x);
      });
    } else {
      // The off-label entries shifted by (pa - v_y) (hinge) or -v_y (top-k
      // entropy), compacted into cb.
      const D shift = hinge ? pa - vy : -vy;
      for_cols<PF>(tid, m, [&](int j, int q, bool ok) {
        const bool off = j != y;
        const D x = getv(j, q) + shift;
        if (off) setv(j, q, x);
        *((ok && off) ? cb + (j < y ? j : j - 1) : ld) = x;
      });
      __syncthreads();
      const int mp = m - 1;
      if constexpr (hinge) {
        bool sorted_form = true;
        if constexpr (C > 0) {
          // The register form over the whole workgroup (slot c of thread g
          // = entry g + G c), which defers to the sorted form only where the
          // reference's biased cone search is needed
          // (topk_simplex_biased.h:57-66).
          D vq[C];
          const int nvalid = (mp - tid + G - 1) / G;
#pragma unroll
          for (int q = 0; q < C; ++q) {
            const D x = cb[tid + G * q];
            vq[q] = (q < nvalid) ? x : -num<D>::inf();
          }
          ProxParamsT<R> pp;
          pp.lo = R(0);
          pp.hi = knap_hi;
          pp.rhs = c;
          pp.rho = rho;
          pp.k = ob.k;
          pp.rhs_k = (ob.k > 0) ? c / static_cast<R>(ob.k) : R(0);
          pp.op = op;
          pp.p = 0;
          const ColThr<R> th = simplex
              ? topk_family<G, C, KM, D, R, false>(vq, mp, nvalid, pp, cb, ld)
              : knap_family<G, C, D, R>(vq, mp, nvalid, pp);
          if (tid == 0) {
            sh_slow = th.slow ? 1 : 0;
            sh_t = th.t;
            sh_lo = th.lo;
            sh_hi = th.hi;
          }
          __syncthreads();
          sorted_form = sh_slow != 0;
          if (sorted_form) {  // cb served as scratch: compact it again
            for_cols<PF>(tid, m, [&](int j, int q, bool ok) {
              *((ok && j != y) ? cb + (j < y ? j : j - 1) : ld) = getv(j, q);
            });
            __syncthreads();
          }
        }
        if (sorted_form) {
          sort_desc_unpadded(cb, mp);
          if (tid < 64) {
            R t, lo, hi;
            int branch, n_hi, n_mid;  // (not used by the epoch)
            thresholds_sorted<D, R>(cb, mp, op, R(0), knap_hi, c, rho, ob.k, t, lo, hi, branch,
                                    n_hi, n_mid);
            if (lane == 0) {
              sh_t = t;
              sh_lo = lo;
              sh_hi = hi;
            }
          }
        }
      } else {  // prox_topk_entropy_biased, alpha = c norm2
        R t, hi;
        entbias_thresholds<D, R, G, true>(cb, mp, tid, ob.k, c * static_cast<R>(norm2), t, hi);
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
      for_cols<PF>(tid, m, [&](int j, int q, bool ok) {
        const bool off = j != y;
        const D x0 = getv(j, q);
        const D x = hinge ? clamp_ref(x0 - t, lo, hi)
                          : clamp_ref(map_a * lambert_w_exp_nb(x0 - t), D(0), hi);
        if (off) setv(j, q, x);
        part += (ok && off) ? static_cast<R>(x) : R(0);
      });
      const R sum = group_sum<G>(part);
      // 3. Recover the variables: the label's entry from the sum, the others
      // negated (and scaled by c for the top-k entropy).
      const D scale = hinge ? D(-1) : static_cast<D>(-c);
      const D ay = hinge ? static_cast<D>(dmin(c, sum)) : static_cast<D>(c * dmin(R(1), sum));
      for_cols<PF>(tid, m, [&](int j, int q, bool ok) {
        setv(j, q, (j == y) ? ay : getv(j, q) * scale);
      });
    }
    // a_old - a_new (sdca_blas_axpy with -1), its 1-norm, a_i <- a_new.
    D part = 0;
    for_cols<PF>(tid, m, [&](int j, int q, bool ok) {
      const D an = getv(j, q);
      const D dl = (PF > 0 ? acur[q] : arow[j]) + D(-1) * an;
      *(ok ? drow + j : gd) = dl;
      *(ok ? arow + j : gd) = an;
      if constexpr (DL) *(ok ? Dx + static_cast<int64_t>(k) * m + j : ld) = dl;
      part += ok ? fabs(dl) : D(0);
    });
    const D asum = group_sum<G>(part);  // also orders v's last reads before the next writes
    if (asum > num<D>::eps() || ob.kernel) {
      changed |= 1u << k;  // the later examples' scores see this update
    } else {
      for_cols<PF>(tid, m, [&](int j, int q, bool ok) { *(ok ? drow + j : gd) = D(0); });
    }
    if constexpr (PF > 0) {
      if (has_next && sh_i[k + 1] == i) {
#pragma unroll
        for (int q = 0; q < PF; ++q) anext[q] = vr[q];
      }
    }
    __syncthreads();
  }
}

typedef float ep_f32x16 __attribute__((ext_vector_type(16)));
typedef double ep_f64x4 __attribute__((ext_vector_type(4)));

// The block's score and Gram products on the matrix cores.  Column c of the
// product is w_c (c < M) or x_{c - M} (M <= c < M + nb, the Gram matrix), row
// e is x_e, the block's e-th example.  Workgroup (tile, ks) takes 32 columns
// (tile tiles_w: the Gram matrix) over the features [ks kc, (ks + 1) kc),
// its four waves 32 features in turn; the waves' sums are added in wave
// order into P[ks][e][c] (Mt = M + nb columns), or, with one split, straight
// into S (nb x M) and Gm (nb x nb).
//   fp32: v_mfma_f32_32x32x2f32; lane l holds example / column l % 32 at
//         features 16 (l / 32) .. + 15 of the wave's 32;
//   fp64: 2 x 2 v_mfma_f64_16x16x4f64; lane l holds examples / columns
//         l % 16 and 16 + l % 16 at features 8 (l / 16) .. + 7.
template <class D>
__global__ void __launch_bounds__(256)
skinny_mfma_kernel(const D* __restrict__ X, const int64_t* __restrict__ order, int64_t q0,
                   int64_t n, const D* __restrict__ W, int nb, int64_t M, int64_t d, int64_t kc,
                   int tiles_w, int vec, D* __restrict__ P, D* __restrict__ S,
                   D* __restrict__ Gm) {
  constexpr int LD = 33;
  __shared__ D red[4][32 * LD];
  const int wave = static_cast<int>(threadIdx.x) >> 6, lane = static_cast<int>(threadIdx.x) & 63;
  const bool gram = static_cast<int>(blockIdx.x) == tiles_w;
  const int64_t j0 = gram ? 0 : static_cast<int64_t>(blockIdx.x) * 32;
  const int64_t cols = gram ? nb : M;
  const int64_t ks = blockIdx.y;
  const int64_t l0 = ks * kc;
  const int64_t l1 = (l0 + kc < d) ? l0 + kc : d;
  if constexpr (sizeof(D) == 4) {
    const int r = lane & 31, h = lane >> 5;
    const bool xr = r < nb, yr = j0 + r < cols;
    const D* xrow = X + (xr ? block_row(order, q0 + r, n) : 0) * d;
    const D* yrow = gram ? X + (yr ? block_row(order, q0 + r, n) : 0) * d
                         : W + (yr ? j0 + r : 0) * d;
    ep_f32x16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
    for (int64_t f0 = l0 + 32 * wave; f0 < l1; f0 += 128) {
      const int64_t fb = f0 + 16 * h;
      float a[16], b[16];
      if (vec && fb + 16 <= l1) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float4 xa = xr ? *reinterpret_cast<const float4*>(xrow + fb + 4 * u)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
          const float4 yb = yr ? *reinterpret_cast<const float4*>(yrow + fb + 4 * u)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
          a[4 * u] = xa.x; a[4 * u + 1] = xa.y; a[4 * u + 2] = xa.z; a[4 * u + 3] = xa.w;
          b[4 * u] = yb.x; b[4 * u + 1] = yb.y; b[4 * u + 2] = yb.z; b[4 * u + 3] = yb.w;
        }
      } else {
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const bool ok = fb + u < l1;
          a[u] = (xr && ok) ? xrow[fb + u] : 0.0f;
          b[u] = (yr && ok) ? yrow[fb + u] : 0.0f;
        }
      }
#pragma unroll
      for (int u = 0; u < 16; ++u) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[u], b[u], acc, 0, 0, 0);
    }
    // Accumulator i of lane l: row 8 (i / 4) + 4 (l / 32) + i % 4, column l % 32.
#pragma unroll
    for (int i = 0; i < 16; ++i) red[wave][(8 * (i >> 2) + 4 * h + (i & 3)) * LD + r] = acc[i];
  } else {
    const int r = lane & 15, g = lane >> 4;
    const D* xrow[2];
    const D* yrow[2];
    bool xr[2], yr[2];
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const int e = 16 * a + r;
      xr[a] = e < nb;
      yr[a] = j0 + e < cols;
      xrow[a] = X + (xr[a] ? block_row(order, q0 + e, n) : 0) * d;
      yrow[a] = gram ? X + (yr[a] ? block_row(order, q0 + e, n) : 0) * d
                     : W + (yr[a] ? j0 + e : 0) * d;
    }
    ep_f64x4 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[a][b][i] = 0.0;
    for (int64_t f0 = l0 + 32 * wave; f0 < l1; f0 += 128) {
      const int64_t fb = f0 + 8 * g;
      double xa[2][8], yb[2][8];
      if (vec && fb + 8 <= l1) {
#pragma unroll
        for (int a = 0; a < 2; ++a) {
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const double2 x2 = xr[a] ? *reinterpret_cast<const double2*>(xrow[a] + fb + 2 * u)
                                     : make_double2(0.0, 0.0);
            const double2 y2 = yr[a] ? *reinterpret_cast<const double2*>(yrow[a] + fb + 2 * u)
                                     : make_double2(0.0, 0.0);
            xa[a][2 * u] = x2.x; xa[a][2 * u + 1] = x2.y;
            yb[a][2 * u] = y2.x; yb[a][2 * u + 1] = y2.y;
          }
        }
      } else {
#pragma unroll
        for (int a = 0; a < 2; ++a) {
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const bool ok = fb + u < l1;
            xa[a][u] = (xr[a] && ok) ? xrow[a][fb + u] : 0.0;
            yb[a][u] = (yr[a] && ok) ? yrow[a][fb + u] : 0.0;
          }
        }
      }
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
          for (int b = 0; b < 2; ++b)
            acc[a][b] = __builtin_amdgcn_mfma_f64_16x16x4f64(xa[a][u], yb[b][u], acc[a][b], 0, 0, 0);
    }
    // Accumulator i of lane l: row l / 16 + 4 i, column l % 16 of its tile.
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave][(16 * a + g + 4 * i) * LD + 16 * b + r] = acc[a][b][i];
  }
  __syncthreads();
  const bool direct = gridDim.y == 1;
  const int64_t Mt = M + nb;
  for (int o = static_cast<int>(threadIdx.x); o < 32 * 32; o += 256) {
    const int e = o >> 5, cc = o & 31;
    D s = red[0][e * LD + cc];
    s += red[1][e * LD + cc];
    s += red[2][e * LD + cc];
    s += red[3][e * LD + cc];
    const int64_t col = j0 + cc;
    if (e < nb && col < cols) {
      if (direct) {
        if (gram) Gm[e * nb + col] = s;
        else S[e * M + col] = s;
      } else {
        P[(ks * kEpochBlock + e) * Mt + (gram ? M + col : col)] = s;
      }
    }
  }
}

// The splits' sums in split order, into S and Gm.
template <class D>
__global__ void __launch_bounds__(256)
skinny_sum_kernel(const D* __restrict__ P, D* __restrict__ S, D* __restrict__ Gm, int nb,
                  int64_t M, int ksplit) {
  const int64_t Mt = M + nb;
  const int64_t o = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (o >= static_cast<int64_t>(nb) * Mt) return;
  const int64_t e = o / Mt, c = o % Mt;
  D s = P[e * Mt + c];
  for (int ks = 1; ks < ksplit; ++ks) s += P[(static_cast<int64_t>(ks) * kEpochBlock + e) * Mt + c];
  if (c < M) S[e * M + c] = s;
  else Gm[e * nb + (c - M)] = s;
}

// Feature split of the skinny products: about kSkinnyGroups workgroups over
// the column tiles, splits of whole 128-feature steps, at most
// kSkinnyMaxSplits of them.
constexpr int kSkinnyGroups = 512;
constexpr int kSkinnyMaxSplits = 32;
struct SkinnyPlan {
  int tiles_w;
  int ksplit;
  int64_t kc;
};
inline SkinnyPlan skinny_plan(int64_t d, int64_t m) {
  SkinnyPlan p;
  p.tiles_w = static_cast<int>((m + 31) / 32);
  const int64_t tiles = p.tiles_w + 1;
  const int64_t steps = (d + 127) / 128;
  int64_t ks = (kSkinnyGroups + tiles - 1) / tiles;
  if (ks > steps) ks = steps;
  if (ks > kSkinnyMaxSplits) ks = kSkinnyMaxSplits;
  if (ks < 1) ks = 1;
  p.kc = ((steps + ks - 1) / ks) * 128;
  p.ksplit = static_cast<int>((d + p.kc - 1) / p.kc);
  if (p.ksplit < 1) p.ksplit = 1;
  return p;
}

template <class D>
hipError_t launch_skinny(const EpochLaunch& a, int64_t q0, int nb, D* S, D* Gm, D* P,
                         const SkinnyPlan& pl) {
  const D* X = static_cast<const D*>(a.X);
  const D* W = static_cast<const D*>(a.W);
  constexpr int64_t vw = 16 / sizeof(D);
  const int vec = (a.d % vw == 0) && (reinterpret_cast<uintptr_t>(X) % 16 == 0) &&
                  (reinterpret_cast<uintptr_t>(W) % 16 == 0);
  // Kernel input takes its Gram matrix from K (kernel_gram_kernel): no Gram
  // tile.
  const dim3 grid(static_cast<unsigned>(pl.tiles_w + (a.kernel ? 0 : 1)),
                  static_cast<unsigned>(pl.ksplit));
  hipLaunchKernelGGL((skinny_mfma_kernel<D>), grid, dim3(256), 0, a.stream, X, a.order, q0, a.n, W,
                     nb, a.m, a.d, pl.kc, pl.tiles_w, vec, P, S, Gm);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || pl.ksplit == 1) return e;
  // (With kernel input the sums of the absent Gram columns land in Gm and
  // are overwritten by the Gram matrix read from K after this.)
  const int64_t total = static_cast<int64_t>(nb) * (a.m + nb);
  hipLaunchKernelGGL((skinny_sum_kernel<D>), dim3(static_cast<unsigned>((total + 255) / 256)),
                     dim3(256), 0, a.stream, P, S, Gm, nb, a.m, pl.ksplit);
  return hipGetLastError();
}

// W -= delta_B' X_B: each element takes the block's rank-1 updates in order,
// w <- w - x_l delta_j (sdca_blas_ger with alpha -1).  Workgroup: 256
// consecutive features of kRankJ classes.
template <class D>
__global__ void __launch_bounds__(256)
rank_update_kernel(D* __restrict__ W, const D* __restrict__ Delta, const D* __restrict__ X,
                   const int64_t* __restrict__ order, int64_t q0, int64_t n, int nb, int64_t m,
                   int64_t d) {
  __shared__ D dl[kEpochBlock][kRankJ];
  __shared__ int64_t rows[kEpochBlock];
  const int64_t j0 = static_cast<int64_t>(blockIdx.y) * kRankJ;
  for (int e = threadIdx.x; e < kEpochBlock * kRankJ; e += 256) {
    const int k = e / kRankJ, jj = e % kRankJ;
    dl[k][jj] = (k < nb && j0 + jj < m) ? Delta[static_cast<int64_t>(k) * m + j0 + jj] : D(0);
  }
  if (threadIdx.x < kEpochBlock)
    rows[threadIdx.x] = threadIdx.x < nb ? block_row(order, q0 + threadIdx.x, n) : 0;
  __syncthreads();
  const int64_t l = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (l >= d) return;
  // Every load is issued before the arithmetic (the kRankJ elements of W
  // with the block's x values), so a thread waits for memory once.
  D xk[kEpochBlock];
#pragma unroll
  for (int k = 0; k < kEpochBlock; ++k) xk[k] = (k < nb) ? X[rows[k] * d + l] : D(0);
  D w[kRankJ];
#pragma unroll
  for (int jj = 0; jj < kRankJ; ++jj) w[jj] = (j0 + jj < m) ? W[(j0 + jj) * d + l] : D(0);
#pragma unroll
  for (int jj = 0; jj < kRankJ; ++jj) {
#pragma unroll
    for (int k = 0; k < kEpochBlock; ++k)
      if (k < nb) w[jj] = w[jj] - xk[k] * dl[k][jj];
  }
#pragma unroll
  for (int jj = 0; jj < kRankJ; ++jj)
    if (j0 + jj < m) W[(j0 + jj) * d + l] = w[jj];
}

// Dynamic LDS of the block kernel: the example's vector (m words), the
// thresholds' column, the per-thread dummy words, the block's delta rows
// where they always fit (the score corrections then read LDS instead of
// global memory) and, for the multilabel families, the example's labels.
__host__ inline size_t block_lds_bytes(size_t es, int m, int C, int PF, bool delta_in_lds,
                                      bool ml) {
  size_t lds = (static_cast<size_t>((m + 3) & ~3) + epoch_column_words(m, C) + kEpochThreads) * es;
  if (delta_in_lds) lds += static_cast<size_t>(epoch_dx_words(m, PF)) * es;
  if (ml) lds += static_cast<size_t>(m) * sizeof(int);
  return lds;
}

template <class D, class R, int FK, int C, int KM, int PF>
hipError_t launch_block(const D* S, const D* Gm, int64_t q0, int nb, const D* norms,
                        const EpochLaunch& a, D* Delta, D* gdummy, const EpochObj& ob, int* bad,
                        D* gv) {
  const int m = static_cast<int>(a.m);
  constexpr bool ml = FK == kFamMlHinge || FK == kFamMlEnt;
  const size_t lds = block_lds_bytes(sizeof(D), m, C, PF, epoch_delta_in_lds<D>(PF), ml);
  if (lds > kEpochLdsBytes) {
    // Rows beyond the LDS: the PF = 0 form with its vectors in gv (the
    // workspace holds epoch_gv_words(m) words there).
    if constexpr (PF == 0 && C == 0) {
      hipLaunchKernelGGL((epoch_block_kernel<D, R, FK, C, KM, PF, true>), dim3(1),
                         dim3(kEpochThreads), kEpochThreads * sizeof(D), a.stream, S, Gm,
                         a.order, q0, a.n, nb, norms, a.labels, a.offsets, static_cast<D*>(a.A),
                         Delta, gdummy, ob, m, bad, gv);
      return hipGetLastError();
    } else {
      return hipErrorInvalidValue;
    }
  }
  hipLaunchKernelGGL((epoch_block_kernel<D, R, FK, C, KM, PF>), dim3(1), dim3(kEpochThreads), lds,
                     a.stream, S, Gm, a.order, q0, a.n, nb, norms, a.labels, a.offsets,
                     static_cast<D*>(a.A), Delta, gdummy, ob, m, bad, gv);
  return hipGetLastError();
}

// The block kernel for the objective's family, m and k: register slots per
// thread PF from m (m <= 256, 1024, 2048), and the register forms (C = PF)
// of the multiclass hinges' simplex / knapsack thresholds (k <= 8 for the
// simplex) and of the multilabel hinges' two-block simplex.
template <class D, class R>
hipError_t launch_block_for(const D* S, const D* Gm, int64_t q0, int nb, const D* norms,
                            const EpochLaunch& a, D* Delta, D* gdummy, const EpochObj& ob,
                            int* bad, D* gv) {
  const int64_t m = a.m;
  const int pf = m <= 256 ? 1 : m <= 1024 ? 4 : m <= 2048 ? 8 : 0;
#define SDCA_EPOCH_BLOCK(FK, C, KM, PF) \
  launch_block<D, R, FK, C, KM, PF>(S, Gm, q0, nb, norms, a, Delta, gdummy, ob, bad, gv)
  // Families without a register form: one variant per PF.
#define SDCA_EPOCH_BY_PF(FK)                                      \
  (pf == 0 ? SDCA_EPOCH_BLOCK(FK, 0, 5, 0)                        \
           : pf == 1 ? SDCA_EPOCH_BLOCK(FK, 0, 5, 1)              \
                     : pf == 4 ? SDCA_EPOCH_BLOCK(FK, 0, 5, 4) : SDCA_EPOCH_BLOCK(FK, 0, 5, 8))
  hipError_t e;
  switch (a.kind) {
    case SDCA_OBJ_ENTROPY:
      e = SDCA_EPOCH_BY_PF(kFamEnt);
      break;
    case SDCA_OBJ_ENTROPY_TOPK:
      e = SDCA_EPOCH_BY_PF(kFamTopkEnt);
      break;
    case SDCA_OBJ_MULTILABEL_ENTROPY:
      e = SDCA_EPOCH_BY_PF(kFamMlEnt);
      break;
    case SDCA_OBJ_MULTILABEL_HINGE:
    case SDCA_OBJ_MULTILABEL_HINGE_SMOOTH:
      e = pf == 0 ? SDCA_EPOCH_BLOCK(kFamMlHinge, 0, 5, 0)
                  : pf == 1 ? SDCA_EPOCH_BLOCK(kFamMlHinge, 1, 5, 1)
                            : pf == 4 ? SDCA_EPOCH_BLOCK(kFamMlHinge, 4, 5, 4)
                                      : SDCA_EPOCH_BLOCK(kFamMlHinge, 8, 5, 8);
      break;
    default: {
      const bool simplex = a.kind == SDCA_OBJ_HINGE_TOPK || a.kind == SDCA_OBJ_HINGE_TOPK_SMOOTH;
      if (pf == 0 || (simplex && a.k > 8)) {
        e = SDCA_EPOCH_BY_PF(kFamHinge);
      } else if (!simplex || a.k <= 5) {
        e = pf == 1 ? SDCA_EPOCH_BLOCK(kFamHinge, 1, 5, 1)
                    : pf == 4 ? SDCA_EPOCH_BLOCK(kFamHinge, 4, 5, 4)
                              : SDCA_EPOCH_BLOCK(kFamHinge, 8, 5, 8);
      } else {
        e = pf == 1 ? SDCA_EPOCH_BLOCK(kFamHinge, 1, 8, 1)
                    : pf == 4 ? SDCA_EPOCH_BLOCK(kFamHinge, 4, 8, 4)
                              : SDCA_EPOCH_BLOCK(kFamHinge, 8, 8, 8);
      }
    }
  }
#undef SDCA_EPOCH_BY_PF
#undef SDCA_EPOCH_BLOCK
  return e;
}

template <class D, class R>
hipError_t launch_epoch_t(const EpochLaunch& a, int** flag_dev) {
  const int64_t d = a.d, m = a.m, n = a.n;
  const int64_t B = kEpochBlock;
  const SkinnyPlan pl = skinny_plan(d, m);
  // Workspace: [flag (256 B) | the threads' store sinks | S | G | Delta | P |
  // norms | At (kernel input)]
  char* p = static_cast<char*>(a.ws);
  int* bad = reinterpret_cast<int*>(p);
  p += 256;
  D* gdummy = reinterpret_cast<D*>(p);
  p += kEpochThreads * sizeof(double);
  D* S = reinterpret_cast<D*>(p);
  D* Gm = S + B * m;
  D* Delta = Gm + B * B;
  D* P = Delta + B * m;  // the skinny products' partial sums
  D* norms_ws = P + static_cast<int64_t>(pl.ksplit) * B * (m + B);
  D* At = norms_ws + n;
  // The block kernel's vectors when the rows exceed its LDS (16-byte aligned).
  D* gv = reinterpret_cast<D*>((reinterpret_cast<uintptr_t>(At + (a.kernel ? m * n : 0)) + 15) &
                               ~static_cast<uintptr_t>(15));
  *flag_dev = bad;
  hipError_t e = launch_clear(bad, 1, a.stream);
  if (e != hipSuccess) return e;
  const D* X = static_cast<const D*>(a.X);
  D* W = static_cast<D*>(a.W);
  const D* norms = static_cast<const D*>(a.norms);
  EpochLaunch ak = a;  // kernel input: the score products' W is At
  if (a.kernel) {
    hipLaunchKernelGGL((kernel_diag_kernel<D>), dim3(static_cast<unsigned>((n + 255) / 256)),
                       dim3(256), 0, a.stream, X, n, norms_ws);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    norms = norms_ws;
    if ((e = launch_transpose(a.data, a.A, At, n, m, a.stream)) != hipSuccess) return e;
    ak.W = At;
  } else if (!norms) {
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
  ob.kernel = a.kernel ? 1 : 0;
  const dim3 rank_grid(static_cast<unsigned>((d + 255) / 256),
                       static_cast<unsigned>((m + kRankJ - 1) / kRankJ));
  for (int64_t q0 = 0; q0 < a.count; q0 += B) {
    const int nb = static_cast<int>(a.count - q0 < B ? a.count - q0 : B);
    if ((e = launch_skinny<D>(ak, q0, nb, S, Gm, P, pl)) != hipSuccess) return e;
    if (a.kernel) {
      hipLaunchKernelGGL((kernel_gram_kernel<D>), dim3(static_cast<unsigned>((nb * nb + 255) / 256)),
                         dim3(256), 0, a.stream, X, a.order, q0, n, nb, Gm);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    if ((e = launch_block_for<D, R>(S, Gm, q0, nb, norms, a, Delta, gdummy, ob, bad, gv)) !=
        hipSuccess)
      return e;
    if (a.kernel) {
      const int64_t cnt = static_cast<int64_t>(nb) * m;
      hipLaunchKernelGGL((kernel_at_kernel<D>), dim3(static_cast<unsigned>((cnt + 255) / 256)),
                         dim3(256), 0, a.stream, static_cast<const D*>(a.A), At, a.order, q0, n,
                         nb, m);
    } else {
      hipLaunchKernelGGL((rank_update_kernel<D>), rank_grid, dim3(256), 0, a.stream, W, Delta, X,
                         a.order, q0, n, nb, m, d);
    }
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace

size_t epoch_workspace_bytes(int data, int64_t d, int64_t m, int64_t n, bool norms_given,
                             bool kernel) {
  const size_t es = data == SDCA_F32 ? 4 : 8;
  const size_t B = kEpochBlock;
  const size_t splits = static_cast<size_t>(skinny_plan(d, m).ksplit);
  (void)norms_given;  // the n norm words are kept in the layout either way
  const size_t mm = static_cast<size_t>((m + 3) & ~int64_t(3));
  // the block kernel's vectors beyond its LDS: the vector and the column
  // (mm values each) and the labels (m ints), 16-byte aligned
  const size_t gv = 16 + 2 * mm * es + 4 * static_cast<size_t>(m);
  return 256 + kEpochThreads * sizeof(double) + es * (2 * B * static_cast<size_t>(m) + B * B +
                     splits * B * (static_cast<size_t>(m) + B) + static_cast<size_t>(n) +
                     (kernel ? static_cast<size_t>(m) * static_cast<size_t>(n) : 0)) + gv;
}

int64_t epoch_max_m(int data, int kind) {
  // Rows beyond the block kernel's LDS run with its vectors in global
  // memory, so no row count is refused for the layout; the rank update's
  // grid (kRankJ classes per workgroup row, at most 65535 rows) sets the
  // bound.
  (void)data;
  (void)kind;
  return static_cast<int64_t>(65535) * kRankJ;
}

hipError_t launch_epoch(const EpochLaunch& a, int** flag_dev) {
  if (a.data == SDCA_F32 && a.result == SDCA_F32) return launch_epoch_t<float, float>(a, flag_dev);
  if (a.data == SDCA_F32 && a.result == SDCA_F64) return launch_epoch_t<float, double>(a, flag_dev);
  if (a.data == SDCA_F64 && a.result == SDCA_F64) return launch_epoch_t<double, double>(a, flag_dev);
  return hipErrorInvalidValue;
}

}  // namespace sdca_gpu
