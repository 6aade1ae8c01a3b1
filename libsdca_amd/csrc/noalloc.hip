// sdca_prox_noalloc: the batched prox of sdca_prox without any device
// allocation, for callers that cannot allocate (code under HIP graph
// capture, serving loops, harnesses that forbid hipMalloc).
//
// The only device memory sdca_prox allocates beyond its inputs and outputs
// is the deferred-column list of the top-k, biased and sort-based
// two-simplex operators: [count, done, column ids...], n + 2 ints.  Here it
// lives in the file-scope array below, one copy per device, which each
// device holds until the process ends.  Its address on a device is looked up
// once (hipGetSymbolAddress, with that device current) and cached; kernels
// receive that address, never the array's host-side name.  Every call on a
// device shares its copy: the counters are cleared by a kernel at the start
// of each call, and calls that overlap on one device (concurrent streams or
// threads) race on it.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/sdca_hip.h"
#include "prox_launch.hpp"

namespace {

// Columns of the largest batch the fixed list holds (the C2 batch: 4M).
constexpr int64_t kNoAllocColumns = int64_t(1) << 22;
constexpr int64_t kScratchInts = kNoAllocColumns + 2;

__device__ __align__(256) int scratch[kScratchInts];

constexpr int kMaxDevices = 64;
std::mutex g_mutex;
int* g_scratch_ptr[kMaxDevices] = {};

// The device address of this device's scratch array (looked up once per
// device, with that device current), or NULL after a failure message.
int* scratch_on_current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    sdca_gpu::set_error(SDCA_ERR_HIP, "sdca_prox_noalloc: no current device");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_mutex);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      sdca_gpu::set_error(SDCA_ERR_HIP, "sdca_prox_noalloc: hipGetSymbolAddress(scratch) failed");
      return nullptr;
    }
    g_scratch_ptr[dev] = static_cast<int*>(ptr);
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" {

int64_t sdca_prox_noalloc_max_columns(void) { return kNoAllocColumns; }

int sdca_prox_noalloc(sdca_prox_op op, sdca_dtype data, sdca_dtype result, int64_t m, int64_t n,
                      const void* in, void* out, const sdca_prox_params* params,
                      const int64_t* col_p, sdca_thresholds* thresholds, void* stream) {
  int* list = scratch_on_current_device();
  if (!list) return SDCA_ERR_HIP;
  return sdca_gpu::prox_entry(op, data, result, m, n, in, out, params, col_p, thresholds,
                              SDCA_DEVICE_PTR, stream, list, kScratchInts);
}

}  // extern "C"
