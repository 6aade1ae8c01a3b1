// Top-k family (topk_simplex, topk_cone and the biased simplex and cone) of
// the batched prox kernel; the register list length is chosen from k.
#include "prox_dispatch.hpp"

namespace sdca_gpu {
hipError_t launch_topk(const ProxLaunch& a) {
  // The biased cone scans the sorted list past the k largest: 16 entries.
  if (a.op == OP_TOPK_CONE_BIASED) return launch_by_type<FAM_TOPK, 15>(a);
  if (a.k <= 2) return launch_by_type<FAM_TOPK, 2>(a);
  if (a.k <= 5) return launch_by_type<FAM_TOPK, 5>(a);
  return launch_by_type<FAM_TOPK, 8>(a);
}
}  // namespace sdca_gpu
