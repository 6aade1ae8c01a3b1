// Knapsack family (knapsack_eq, knapsack_le) of the batched prox kernel.
#include "prox_dispatch.hpp"

namespace sdca_gpu {
hipError_t launch_knap(const ProxLaunch& a) { return launch_by_type<FAM_KNAP, 0>(a); }
}  // namespace sdca_gpu
