// Entropic projection with the Lambert W(exp) map (entropy_norm) of the
// batched prox kernel (family FAM_ENT with KM = 1).
#include "prox_dispatch.hpp"

namespace sdca_gpu {
hipError_t launch_ent_norm(const ProxLaunch& a) { return launch_by_type<FAM_ENT, 1>(a); }
}  // namespace sdca_gpu
