// Two-block simplex operator of the batched prox kernel.
#include "prox_dispatch.hpp"

namespace sdca_gpu {
hipError_t launch_two(const ProxLaunch& a) { return launch_by_type<FAM_TWO, 0>(a); }
}  // namespace sdca_gpu
