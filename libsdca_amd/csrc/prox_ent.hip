// Entropic projection with the exp map (entropy) of the batched prox kernel;
// the Lambert-map variant (entropy_norm) is instantiated in prox_entnorm.hip.
#include "prox_dispatch.hpp"

namespace sdca_gpu {
hipError_t launch_ent(const ProxLaunch& a) {
  if (a.op == OP_ENTROPY_NORM) return launch_ent_norm(a);
  return launch_by_type<FAM_ENT, 0>(a);
}
}  // namespace sdca_gpu
