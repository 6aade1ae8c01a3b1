// Entropic family (entropy, entropy_norm) of the batched prox kernel.
#include "prox_dispatch.hpp"

namespace sdca_gpu {
hipError_t launch_ent(const ProxLaunch& a) { return launch_by_type<FAM_ENT, 0>(a); }
}  // namespace sdca_gpu
