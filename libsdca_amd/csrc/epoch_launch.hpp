// Host-side launch interface of the SDCA epoch (internal to the library).
#ifndef SDCA_HIP_EPOCH_LAUNCH_HPP
#define SDCA_HIP_EPOCH_LAUNCH_HPP

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/sdca_hip.h"

namespace sdca_gpu {

// Examples per block of the blocked epoch: the block's scores and Gram
// matrix come from two GEMMs, its examples run in order in one workgroup.
constexpr int kEpochBlock = 32;

struct EpochLaunch {
  int data;    // sdca_dtype of X, W, A
  int result;  // sdca_dtype of the dual update's internal arithmetic
  int kind;    // sdca_objective_kind
  double c, gamma;
  int k;
  int64_t d, m, n;
  const void* X;          // n x d
  void* W;                // m x d, updated
  void* A;                // n x m, updated
  const int64_t* labels;  // n (multiclass), or offsets[n] (multilabel)
  const int64_t* offsets; // n + 1 CSR row starts into labels (multilabel), or NULL
  const int64_t* order;   // count example indices, or NULL for 0..count-1
  int64_t count;
  const void* norms;      // n squared norms, or NULL (computed into the workspace)
  bool kernel;            // kernel input: X is the n x n kernel matrix (d = n), W unused
  void* ws;               // epoch_workspace_bytes(...) bytes
  hipStream_t stream;
};

// Workspace bytes of one call (the block buffers, the norms when not given
// or taken from K's diagonal, the transposed dual variables for kernel
// input, the index list and the bad-input flag).
size_t epoch_workspace_bytes(int data, int64_t d, int64_t m, int64_t n, bool norms_given,
                             bool kernel = false);
// Enqueues the epoch; the bad-input flag (an example index or a label out of
// range: such entries are read as 0) is left in *flag_dev for the caller.
hipError_t launch_epoch(const EpochLaunch& a, int** flag_dev);
// Largest m of the epoch for an element type and objective kind (the block
// kernel's rows go to global memory beyond its LDS; the rank update's grid
// bounds m).
int64_t epoch_max_m(int data, int kind);

}  // namespace sdca_gpu

#endif
