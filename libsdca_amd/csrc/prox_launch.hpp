// Host-side launch interface of the prox kernels (internal to the library).
#ifndef SDCA_HIP_PROX_LAUNCH_HPP
#define SDCA_HIP_PROX_LAUNCH_HPP

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/sdca_hip.h"

namespace sdca_gpu {

enum {
  OP_KNAPSACK_EQ = SDCA_PROX_KNAPSACK_EQ,
  OP_KNAPSACK_LE = SDCA_PROX_KNAPSACK_LE,
  OP_TOPK_SIMPLEX = SDCA_PROX_TOPK_SIMPLEX,
  OP_TOPK_CONE = SDCA_PROX_TOPK_CONE,
  OP_ENTROPY = SDCA_PROX_ENTROPY,
  OP_ENTROPY_NORM = SDCA_PROX_ENTROPY_NORM,
  OP_TOPK_ENTROPY = SDCA_PROX_TOPK_ENTROPY,
  OP_TWO_SIMPLEX = SDCA_PROX_TWO_SIMPLEX,
  OP_LAMBERT_W_EXP = SDCA_PROX_LAMBERT_W_EXP,
  OP_KNAPSACK_LE_BIASED = SDCA_PROX_KNAPSACK_LE_BIASED,
  OP_TOPK_SIMPLEX_BIASED = SDCA_PROX_TOPK_SIMPLEX_BIASED,
  OP_TOPK_CONE_BIASED = SDCA_PROX_TOPK_CONE_BIASED,
  OP_TWO_SIMPLEX_SORT = SDCA_PROX_TWO_SIMPLEX_SORT
};

// Largest m handled by the one-wave register kernels.
constexpr int64_t kRegMaxM = 2048;
// Threads of the workgroup that holds one column above kRegMaxM rows, with
// up to 32 slots per thread (up to 16384 rows; 256 registers per thread at
// two waves per SIMD), and for the fp32 columns beyond that.
constexpr int kWideThreads = 512;
constexpr int kMaxWideThreads = 1024;
// Largest column (m times the element size) any kernel holds in LDS: the
// sorted-column, wave-per-column and workgroup-per-column kernels stage
// whole columns (160 KiB of LDS per workgroup on gfx950, less the dummy
// words and reduction scratch).
constexpr int64_t kMaxColumnBytes = 128 * 1024;
// Largest m of the prox operators (and of the evaluation) for an element
// type: 32768 rows in fp32, 16384 in fp64.
inline int64_t max_rows(int data) {
  return kMaxColumnBytes / (data == SDCA_F32 ? 4 : 8);
}
// Top-k operators keep k <= kTopkMaxK in registers; larger k takes the
// workgroup-per-column kernel.
constexpr int64_t kTopkMaxK = 8;

struct ProxLaunch {
  int op;
  int data;    // sdca_dtype of the elements
  int result;  // sdca_dtype of the internal arithmetic
  int64_t m, n;
  const void* in;
  void* out;
  double lo, hi, rhs, rho, alpha;
  int64_t k, p;
  const int64_t* col_p;     // device, or NULL
  sdca_thresholds* thr;     // device, or NULL
  sdca_prox_sets* sets;     // device, or NULL (one per threshold record)
  int* slow;                // device: [0] = count, [1..n] = column list
  hipStream_t stream;
};

// Register kernels, one per operator family (prox_*.hip).
hipError_t launch_knap(const ProxLaunch& a);
hipError_t launch_topk(const ProxLaunch& a);
hipError_t launch_ent(const ProxLaunch& a);
hipError_t launch_ent_norm(const ProxLaunch& a);
// Two-block simplex by sort and scan, one workgroup per column (prox_slow.hip).
hipError_t launch_two_sort(const ProxLaunch& a, bool all_columns);
// Biased top-k entropy, one wave per column (prox_entbias.hip).
hipError_t launch_ent_biased(const ProxLaunch& a);
// Two-block entropy, one wave per column (prox_entbias.hip).
hipError_t launch_two_ent(const ProxLaunch& a);
hipError_t launch_topkent(const ProxLaunch& a);
hipError_t launch_two(const ProxLaunch& a);
// Workgroup-per-column kernel over the flagged list (all_columns: every column).
hipError_t launch_slow(const ProxLaunch& a, bool all_columns);
// Columns beyond the LDS copy, every column: the sorted-column kernel with
// each workgroup's column sorted in a slice of scratch (device memory,
// scratch_bytes; at least one slice of the next power of two above m
// values), the sort-based two-block simplex likewise (slices of m values),
// and the two-block simplex with its passes over the column in device
// memory.
hipError_t launch_slow_global(const ProxLaunch& a, void* scratch, size_t scratch_bytes);
hipError_t launch_two_sort_global(const ProxLaunch& a, void* scratch, size_t scratch_bytes);
hipError_t launch_two_global(const ProxLaunch& a);
// The biased top-k entropy and the two-block entropy beyond the LDS: the
// wave-per-column kernels with each wave's column copy in a slice of
// scratch (device memory; slices of m rounded up to 4 values).
hipError_t launch_ent_biased_global(const ProxLaunch& a, void* scratch, size_t scratch_bytes);
hipError_t launch_two_ent_global(const ProxLaunch& a, void* scratch, size_t scratch_bytes);
// The top-k entropy beyond the LDS: one workgroup per column, its copy in a
// slice of scratch (m values).
hipError_t launch_topkent_global(const ProxLaunch& a, void* scratch, size_t scratch_bytes);
// Columns above max_rows(data) for the operators whose thresholds come from
// sweeps alone (knapsack_eq, knapsack_le, entropy, entropy_norm): one
// workgroup per column, the column re-read from global memory per sweep
// (prox_stream.hip).
bool stream_supported(int op);
hipError_t launch_stream(const ProxLaunch& a);
// Elementwise lambert_w_exp over m*n elements.
hipError_t launch_lambert(const ProxLaunch& a);
// Zero the slow-column counter.
hipError_t launch_clear(int* p, int count, hipStream_t stream);

// sdca_prox (capi.cpp) with an optional caller-provided deferred-column list
// of fixed_list_ints ints in place of the per-stream workspace: with it the
// call allocates nothing (device pointers only).
int prox_entry(int op, int data, int result, int64_t m, int64_t n, const void* in, void* out,
               const sdca_prox_params* params, const int64_t* col_p,
               sdca_thresholds* thresholds, unsigned flags, void* stream, int* fixed_list,
               int64_t fixed_list_ints, sdca_prox_sets* sets = nullptr);
// Records a failure message for sdca_last_error() on this thread; returns code.
int set_error(int code, const char* message);

}  // namespace sdca_gpu

#endif
