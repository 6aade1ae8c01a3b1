// C ABI of the evaluation pass (include/sdca_hip.h).
#include <hip/hip_runtime.h>

#include "../../include/sdca_hip.h"

extern "C" {

int sdca_eval_features(const sdca_objective*, int, sdca_dtype, sdca_dtype, int64_t, int64_t,
                       int64_t, const void*, const void*, const void*, const void*,
                       const int64_t*, const int64_t*, sdca_eval_record*, double*, double*,
                       unsigned, void*) {
  return SDCA_ERR_NOT_IMPLEMENTED;
}

int sdca_eval_scores(const sdca_objective*, int, sdca_dtype, sdca_dtype, int64_t, int64_t,
                     const void*, const void*, const int64_t*, const int64_t*, double, double,
                     sdca_eval_record*, double*, double*, unsigned, void*) {
  return SDCA_ERR_NOT_IMPLEMENTED;
}

int sdca_scores(sdca_dtype, int64_t, int64_t, int64_t, const void*, const void*, void*,
                unsigned, void*) {
  return SDCA_ERR_NOT_IMPLEMENTED;
}

}  // extern "C"
