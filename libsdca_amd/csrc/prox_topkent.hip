// Top-k entropy operator of the batched prox kernel.
#include "prox_dispatch.hpp"

namespace sdca_gpu {
hipError_t launch_topkent(const ProxLaunch& a) { return launch_by_type<FAM_TOPKENT, 0>(a); }
}  // namespace sdca_gpu
