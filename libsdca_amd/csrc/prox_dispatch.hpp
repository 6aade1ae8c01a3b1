// Launch of prox_columns_kernel for one family: picks the (G lanes per
// column, C slots per lane) configuration from m and the (Data, Result) pair.
#ifndef SDCA_HIP_PROX_DISPATCH_HPP
#define SDCA_HIP_PROX_DISPATCH_HPP

#include "prox_impl.hpp"

namespace sdca_gpu {

template <int FAM, int KM, class D, class R, int G, int C, int BT = 64>
hipError_t launch_one(const ProxLaunch& a) {
  // BT threads per workgroup: one wave, or (G = BT) one column per
  // workgroup.
  constexpr int B = BT / G;
  ProxParamsT<R> pp;
  pp.lo = static_cast<R>(a.lo);
  pp.hi = static_cast<R>(a.hi);
  pp.rhs = static_cast<R>(a.rhs);
  // rho enters the register kernel only through the biased simplex and
  // knapsack (the other operators take rho = 0).
  pp.rho = (a.op == OP_TOPK_SIMPLEX_BIASED || a.op == OP_TOPK_CONE_BIASED ||
            a.op == OP_KNAPSACK_LE_BIASED)
               ? static_cast<R>(a.rho) : R(0);
  pp.k = static_cast<int>(a.k);
  pp.rhs_k = (a.k > 0) ? pp.rhs / static_cast<R>(a.k) : R(0);
  pp.op = a.op;
  pp.p = static_cast<int>(a.p);
  const int64_t blocks = (a.n + B - 1) / B;
  // B*m tile, G*C - m words of slack for branch-free slot reads (slot c of
  // the last column's lane g is word (B - 1) m + g + G c <= B m + G C - m - 1),
  // BT dummy words.  Slack of G*C - m words rather than G*C keeps the LDS
  // per wave near the tile's own size when m is just below G*C (m = 1000 in
  // 64 x 16 slots: 8.7 KB instead of 16.7 KB), and with it the occupancy.
  if (a.m > static_cast<int64_t>(G) * C) return hipErrorInvalidValue;
  const bool full = a.m == static_cast<int64_t>(G) * C;
  const size_t slack = full ? 0 : static_cast<size_t>(G * C - a.m);
  // The entropic families store only to valid slots (with a branch) and
  // need no dummy words: at m = 1000 in fp64 that keeps a wave's LDS at
  // 8 KB, 5 waves per SIMD (the register limit) instead of 4.5.
  const size_t dummies = (FAM == FAM_ENT || FAM == FAM_TOPKENT) ? 0 : BT;
  size_t shmem =
      (static_cast<size_t>(B) * static_cast<size_t>(a.m) + slack + dummies) * sizeof(D);
  // The Lambert map keeps its last W values in an LDS array of R.
  if constexpr (FAM == FAM_ENT && KM == 1 && sizeof(R) >= sizeof(D) && BT == 64)
    shmem = w_lds_offset<D, R>(B, a.m, slack) +
            (static_cast<size_t>(B) * static_cast<size_t>(a.m) + slack) * sizeof(R);
  // The top-k cone streams its tiles with little work per column, and HBM
  // serves them faster with fewer tiles in flight: its workgroups reserve
  // LDS at 3.2x the tile, which caps a CU at ~50 KB of tiles (at m = 100 in
  // fp32, 2 waves per SIMD instead of 6: 68.3 -> 71.8 % of the HBM peak on
  // one box).  The top-k simplex keeps its natural 6 waves per SIMD: a cap
  // at 4 gained ~1.5 % in steady state but lost ~4 % over the first few
  // dozen launches after a cold start, when the shader clock is reduced and
  // the kernel, whose vector issue is ~78 % of its memory time, needs every
  // wave (cold starts measured in the first 25 launches: 0.59 ms per launch
  // with 6 waves, 0.61-0.62 ms with 4).  The biased operators and the
  // two-simplex, which compute more per column, keep their natural
  // occupancy too.
  if constexpr (FAM == FAM_TOPK && BT == 64) {
    const size_t tile = static_cast<size_t>(B) * static_cast<size_t>(a.m) * sizeof(D);
    if (a.op == OP_TOPK_CONE && shmem < tile * 16 / 5) shmem = tile * 16 / 5;
  }
  // m == G * C (the configuration's exact size) gets the variant without
  // per-slot validity tests (for one-wave workgroups: the wide
  // configurations are for rare sizes and keep one variant).
  if constexpr (BT == 64) {
    if (full) {
      hipLaunchKernelGGL((prox_columns_kernel<FAM, KM, D, R, G, C, BT, true>),
                         dim3(static_cast<unsigned>(blocks)), dim3(BT), shmem, a.stream,
                         static_cast<const D*>(a.in), static_cast<D*>(a.out), a.m, a.n, pp,
                         a.col_p, a.thr, a.slow, a.sets);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((prox_columns_kernel<FAM, KM, D, R, G, C, BT, false>),
                     dim3(static_cast<unsigned>(blocks)), dim3(BT), shmem, a.stream,
                     static_cast<const D*>(a.in), static_cast<D*>(a.out), a.m, a.n, pp,
                     a.col_p, a.thr, a.slow, a.sets);
  return hipGetLastError();
}

// Columns above kRegMaxM rows: one workgroup per column (kWideThreads
// threads, kMaxWideThreads for the largest fp32 columns), C slots per
// thread; the column (at most kMaxColumnBytes) is staged in LDS and the
// group reductions combine the waves through LDS.
template <int FAM, int KM, class D, class R>
hipError_t launch_wide(const ProxLaunch& a) {
  constexpr int G = kWideThreads, G2 = kMaxWideThreads;
  if (a.m <= 8 * G) return launch_one<FAM, KM, D, R, G, 8, G>(a);
  if (a.m <= 16 * G) return launch_one<FAM, KM, D, R, G, 16, G>(a);
  if (a.m <= 32 * G) return launch_one<FAM, KM, D, R, G, 32, G>(a);
  if constexpr (sizeof(D) == 4) return launch_one<FAM, KM, D, R, G2, 32, G2>(a);
  return hipErrorInvalidValue;
}

// m -> (G lanes per column, C slots per lane): the fewest lanes whose C
// slots hold the column (C = 25 fits m = 100 exactly on four lanes and
// m = 200 on eight).
template <int FAM, int KM, class D, class R>
hipError_t launch_by_m(const ProxLaunch& a) {
  // The knapsack and top-k families take the sorted-column kernel above
  // kRegMaxM rows.
  if constexpr (FAM == FAM_ENT || FAM == FAM_TOPKENT || FAM == FAM_TWO) {
    if (a.m > kRegMaxM) return launch_wide<FAM, KM, D, R>(a);
  }
  // The knapsack family's smallest columns (C1: m = 10) in exactly ten
  // slots: every pass of the variable fixing touches the column's own
  // values only.
  if constexpr (FAM == FAM_KNAP) {
    if (a.m <= 10) return launch_one<FAM, KM, D, R, 1, 10>(a);
  }
  if (a.m <= 16) return launch_one<FAM, KM, D, R, 1, 16>(a);
  if (a.m <= 64) return launch_one<FAM, KM, D, R, 4, 16>(a);
  if (a.m <= 100) return launch_one<FAM, KM, D, R, 4, 25>(a);
  if (a.m <= 128) return launch_one<FAM, KM, D, R, 4, 32>(a);
  if (a.m <= 200) return launch_one<FAM, KM, D, R, 8, 25>(a);
  if (a.m <= 256) return launch_one<FAM, KM, D, R, 16, 16>(a);
  if (a.m <= 512) return launch_one<FAM, KM, D, R, 16, 32>(a);
  if (a.m <= 1024) return launch_one<FAM, KM, D, R, 64, 16>(a);
  return launch_one<FAM, KM, D, R, 64, 32>(a);
}

template <int FAM, int KM>
hipError_t launch_by_type(const ProxLaunch& a) {
  if (a.data == SDCA_F32 && a.result == SDCA_F32) return launch_by_m<FAM, KM, float, float>(a);
  if (a.data == SDCA_F32 && a.result == SDCA_F64) return launch_by_m<FAM, KM, float, double>(a);
  if (a.data == SDCA_F64 && a.result == SDCA_F64) return launch_by_m<FAM, KM, double, double>(a);
  if (a.data == SDCA_F64 && a.result == SDCA_F32) return launch_by_m<FAM, KM, double, float>(a);
  return hipErrorInvalidValue;
}

}  // namespace sdca_gpu

#endif
