// Launch of prox_columns_kernel for one family: picks the (G lanes per
// column, C slots per lane) configuration from m and the (Data, Result) pair.
#ifndef SDCA_HIP_PROX_DISPATCH_HPP
#define SDCA_HIP_PROX_DISPATCH_HPP

#include "prox_impl.hpp"

namespace sdca_gpu {

template <int FAM, int KM, class D, class R, int G, int C>
hipError_t launch_one(const ProxLaunch& a) {
  constexpr int B = 256 / G;
  ProxParamsT<R> pp;
  pp.lo = static_cast<R>(a.lo);
  pp.hi = static_cast<R>(a.hi);
  pp.rhs = static_cast<R>(a.rhs);
  pp.k = static_cast<int>(a.k);
  pp.op = a.op;
  pp.p = static_cast<int>(a.p);
  const int64_t blocks = (a.n + B - 1) / B;
  const size_t shmem = static_cast<size_t>(B) * static_cast<size_t>(a.m) * sizeof(D);
  hipLaunchKernelGGL((prox_columns_kernel<FAM, KM, D, R, G, C>), dim3(static_cast<unsigned>(blocks)),
                     dim3(256), shmem, a.stream, static_cast<const D*>(a.in),
                     static_cast<D*>(a.out), a.m, a.n, pp, a.col_p, a.thr, a.slow);
  return hipGetLastError();
}

// m -> (G, C): the fewest lanes per column whose C slots hold the column.
template <int FAM, int KM, class D, class R>
hipError_t launch_by_m(const ProxLaunch& a) {
  if (a.m <= 16) return launch_one<FAM, KM, D, R, 1, 16>(a);
  if (a.m <= 64) return launch_one<FAM, KM, D, R, 4, 16>(a);
  if (a.m <= 128) return launch_one<FAM, KM, D, R, 4, 32>(a);
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
  return hipErrorInvalidValue;
}

}  // namespace sdca_gpu

#endif
