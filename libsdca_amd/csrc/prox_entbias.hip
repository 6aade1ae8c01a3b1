// Lambert-map operators solved one wave per column, with the column in LDS:
//
// * Biased top-k entropy (topk_entropy_biased.h:179-268):
//     x = clamp(W(exp(a - t)) / alpha, 0, s / k)
//   with (s, t) from the reference's two solves - the order-4 Householder
//   iteration on W(e^(alpha - t)) + sum_i W(e^(a_i - t)) = alpha while no
//   entry is capped (:9-61), then, while the feasibility test fails, the set
//   U of capped entries grows by the largest remaining entry and (s, t) come
//   from the Newton iteration on the two-equation system of :120-176.
// * Two-block entropy (two_entropy.h:109-231):
//     x = W(exp(a - t)) / alpha,  y = W(exp(b - t - alpha / p)) / alpha,
//   with t from the reference's two guesses, bisection and bracketed
//   Householder steps on sum W(e^(a - t)) + sum W(e^(b - t - c)) = alpha.
//
// Each pass of these iterations is a sum of W(e^(x_i + shift)) and its
// derivatives over the column: each lane sums a stride-64 share, and a
// butterfly reduction gives every lane the totals, so the scalar updates run
// uniformly on all 64 lanes and no barrier beyond the wave is needed.
// Entries moved into U are overwritten with -inf in LDS, where W(e^-inf) = 0
// drops them from every later sum; the final clamp reads the column again
// from global memory.
#include "common.hpp"
#include "prox_impl.hpp"
#include "prox_lambert_wave.hpp"
#include "prox_launch.hpp"

namespace sdca_gpu {

namespace {

constexpr int kEbMaxWaves = 4;

// reuse: each wave also has an LDS array of R (after the waves' columns)
// where the last pass leaves its W values, and the output map is a Taylor
// step from them (lambert_w_exp_shift) instead of a new evaluation.
//
// GV (columns beyond the LDS): each wave's column copy is its stride_elems
// slice of gscratch (device memory) instead; reuse is 0.  The wave's own
// accesses to it are ordered as its LDS accesses are (one wavefront).
template <class D, class R, bool GV = false>
__global__ void __launch_bounds__(64 * kEbMaxWaves)
entbias_kernel(const D* __restrict__ in, D* __restrict__ out, int64_t m64, int64_t n, int k,
               R alpha, sdca_thresholds* __restrict__ thr, int stride_elems, int reuse,
               sdca_prox_sets* __restrict__ sets, D* __restrict__ gscratch) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int waves = blockDim.x >> 6;
  D* s = GV ? gscratch + (static_cast<int64_t>(blockIdx.x) * waves + wave) * stride_elems
            : reinterpret_cast<D*>(smem_raw) + static_cast<int64_t>(wave) * stride_elems;
  R* const wl = reuse ? reinterpret_cast<R*>(smem_raw + static_cast<size_t>(waves) *
                                                            stride_elems * sizeof(D)) +
                            static_cast<int64_t>(wave) * stride_elems
                      : nullptr;
  const int m = static_cast<int>(m64);
  const D map_a = D(1) / static_cast<D>(alpha);  // a_lambert_w_exp_map (functor.h:33-38)
  for (int64_t j = static_cast<int64_t>(blockIdx.x) * waves + wave; j < n;
       j += static_cast<int64_t>(gridDim.x) * waves) {
    const D* col = in + j * m64;
    for (int i = lane; i < m; i += 64) s[i] = col[i];
    wave_lds_sync();
    R t, hi, tw = 0;
    int branch = SDCA_BRANCH_U_EMPTY;
    entbias_thresholds<D, R>(s, m, lane, k, alpha, t, hi, wl, &tw, &branch);
    if (thr && lane == 0) {
      thr[j].t = static_cast<double>(t);
      thr[j].lo = 0;
      thr[j].hi = static_cast<double>(hi);
    }
    // The reference's record keeps (first, last) in every branch
    // (topk_entropy_biased.h:224, 232, 269).
    if (sets && lane == 0) sets[j] = sdca_prox_sets{0, m, branch, 0};
    const D td = static_cast<D>(t), hd = static_cast<D>(hi);
    D* dst = out + j * m64;
    // Entries moved into U hold -inf in s (and W = 0 in wl): the map.
    const R dt = t - tw;
    const bool tay = wl && fabs(dt) <= R(kLambertShiftMax);
    for (int i = lane; i < m; i += 64) {
      const D y = (tay && s[i] != -num<D>::inf()) ? static_cast<D>(lambert_w_exp_shift(wl[i], dt))
                                                   : lambert_w_exp(col[i] - td);
      dst[i] = clamp_ref(map_a * y, D(0), hd);
    }
    wave_lds_sync();  // every lane is done with s before the next column's copy
  }
}

template <class D, class R, bool GV = false>
__global__ void __launch_bounds__(64 * kEbMaxWaves)
twoent_kernel(const D* __restrict__ in, D* __restrict__ out, int64_t m64, int64_t n,
              int64_t p_all, const int64_t* __restrict__ col_p, R alpha,
              sdca_thresholds* __restrict__ thr, int stride_elems, int reuse,
              sdca_prox_sets* __restrict__ sets, D* __restrict__ gscratch) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int waves = blockDim.x >> 6;
  // GV: as in entbias_kernel.
  D* s = GV ? gscratch + (static_cast<int64_t>(blockIdx.x) * waves + wave) * stride_elems
            : reinterpret_cast<D*>(smem_raw) + static_cast<int64_t>(wave) * stride_elems;
  R* const wl = reuse ? reinterpret_cast<R*>(smem_raw + static_cast<size_t>(waves) *
                                                            stride_elems * sizeof(D)) +
                            static_cast<int64_t>(wave) * stride_elems
                      : nullptr;
  const int m = static_cast<int>(m64);
  const D map_a = D(1) / static_cast<D>(alpha);  // a_lambert_w_exp_map (functor.h:33-38)
  for (int64_t j = static_cast<int64_t>(blockIdx.x) * waves + wave; j < n;
       j += static_cast<int64_t>(gridDim.x) * waves) {
    const int p = clamp_split(col_p ? col_p[j] : p_all, m);
    const D* col = in + j * m64;
    for (int i = lane; i < m; i += 64) s[i] = col[i];
    wave_lds_sync();
    R t, c, tw = 0;
    // The Householder steps end once f(t) is at the rounding level of its
    // sums (NOISE_STOP): the reference's own test, a step of at most
    // epsilon, then waits for t to stop moving between neighbouring floats
    // (about ten passes on N(0,1) columns at m = 200 against two or three),
    // and lands within that level too.
    twoent_thresholds<D, R, 64, true>(s, m, p, lane, alpha, t, c, wl, &tw);
    const R tb = t + c;
    if (thr && lane == 0) {
      thr[2 * j].t = static_cast<double>(t);
      thr[2 * j].lo = 0;
      thr[2 * j].hi = 1;
      thr[2 * j + 1].t = static_cast<double>(tb);
      thr[2 * j + 1].lo = 0;
      thr[2 * j + 1].hi = 1;
    }
    // Both blocks free in the reference's record (two_entropy.h:228-230).
    if (sets && lane == 0) {
      sets[2 * j] = sdca_prox_sets{0, p, SDCA_BRANCH_SEARCH, 0};
      sets[2 * j + 1] = sdca_prox_sets{0, m - p, SDCA_BRANCH_SEARCH, 0};
    }
    const D ta_d = static_cast<D>(t), tb_d = static_cast<D>(tb);
    D* dst = out + j * m64;
    const R dt = t - tw;  // both blocks' arguments moved by it
    const bool tay = wl && fabs(dt) <= lw_shift_max<R>();
    for (int i = lane; i < m; i += 64) {
      const D y = tay ? static_cast<D>(lambert_w_exp_shift(wl[i], dt))
                      : lambert_w_exp(col[i] - (i < p ? ta_d : tb_d));
      dst[i] = clamp_ref(map_a * y, D(0), D(1));
    }
    wave_lds_sync();
  }
}

// LDS per wave: the column in D and, where it fits (64 KiB per workgroup)
// and the Result type is at least as wide as the data (otherwise the map is
// evaluated in the data type), the array of W values in R.
template <class D, class R>
size_t eb_per_wave(int stride, bool& reuse) {
  const size_t col = static_cast<size_t>(stride) * sizeof(D);
  const size_t w = static_cast<size_t>(stride) * sizeof(R);
  reuse = sizeof(R) >= sizeof(D) && col + w <= 65536;
  return reuse ? col + w : col;
}

template <class D, class R>
hipError_t launch_twoent_t(const ProxLaunch& a) {
  const int stride = static_cast<int>((a.m + 3) & ~int64_t(3));
  bool reuse = false;
  const size_t per_wave = eb_per_wave<D, R>(stride, reuse);
  int waves = kEbMaxWaves;
  while (waves > 1 && waves * per_wave > 65536) waves >>= 1;
  int64_t grid = (a.n + waves - 1) / waves;
  if (grid > 16384) grid = 16384;
  if (grid < 1) grid = 1;
  hipLaunchKernelGGL((twoent_kernel<D, R>), dim3(static_cast<unsigned>(grid)), dim3(64 * waves),
                     waves * per_wave, a.stream, static_cast<const D*>(a.in),
                     static_cast<D*>(a.out), a.m, a.n, a.p, a.col_p, static_cast<R>(a.alpha),
                     a.thr, stride, reuse ? 1 : 0, a.sets, static_cast<D*>(nullptr));
  return hipGetLastError();
}

// Columns beyond the LDS: four waves per workgroup, each with a slice of
// scratch (as many workgroups as the scratch holds four slices, at most
// one wave per column).
template <class D>
int64_t eb_global_grid(const ProxLaunch& a, size_t scratch_bytes, int stride) {
  const int64_t slices = static_cast<int64_t>(scratch_bytes / (static_cast<size_t>(stride) *
                                                               sizeof(D)));
  int64_t grid = slices / kEbMaxWaves;
  const int64_t need = (a.n + kEbMaxWaves - 1) / kEbMaxWaves;
  if (grid > need) grid = need;
  if (grid > 16384) grid = 16384;
  return grid;
}

template <class D, class R>
hipError_t launch_twoent_global_t(const ProxLaunch& a, void* scratch, size_t scratch_bytes) {
  const int stride = static_cast<int>((a.m + 3) & ~int64_t(3));
  const int64_t grid = eb_global_grid<D>(a, scratch_bytes, stride);
  if (grid < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL((twoent_kernel<D, R, true>), dim3(static_cast<unsigned>(grid)),
                     dim3(64 * kEbMaxWaves), 0, a.stream, static_cast<const D*>(a.in),
                     static_cast<D*>(a.out), a.m, a.n, a.p, a.col_p, static_cast<R>(a.alpha),
                     a.thr, stride, 0, a.sets, static_cast<D*>(scratch));
  return hipGetLastError();
}

template <class D, class R>
hipError_t launch_entbias_global_t(const ProxLaunch& a, void* scratch, size_t scratch_bytes) {
  const int stride = static_cast<int>((a.m + 3) & ~int64_t(3));
  const int64_t grid = eb_global_grid<D>(a, scratch_bytes, stride);
  if (grid < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL((entbias_kernel<D, R, true>), dim3(static_cast<unsigned>(grid)),
                     dim3(64 * kEbMaxWaves), 0, a.stream, static_cast<const D*>(a.in),
                     static_cast<D*>(a.out), a.m, a.n, static_cast<int>(a.k),
                     static_cast<R>(a.alpha), a.thr, stride, 0, a.sets, static_cast<D*>(scratch));
  return hipGetLastError();
}

template <class D, class R>
hipError_t launch_t(const ProxLaunch& a) {
  const int stride = static_cast<int>((a.m + 3) & ~int64_t(3));  // 16-byte aligned slices
  bool reuse = false;
  const size_t per_wave = eb_per_wave<D, R>(stride, reuse);
  int waves = kEbMaxWaves;
  while (waves > 1 && waves * per_wave > 65536) waves >>= 1;
  int64_t grid = (a.n + waves - 1) / waves;
  if (grid > 16384) grid = 16384;
  if (grid < 1) grid = 1;
  hipLaunchKernelGGL((entbias_kernel<D, R>), dim3(static_cast<unsigned>(grid)), dim3(64 * waves),
                     waves * per_wave, a.stream, static_cast<const D*>(a.in),
                     static_cast<D*>(a.out), a.m, a.n, static_cast<int>(a.k),
                     static_cast<R>(a.alpha), a.thr, stride, reuse ? 1 : 0, a.sets,
                     static_cast<D*>(nullptr));
  return hipGetLastError();
}

}  // namespace

hipError_t launch_two_ent(const ProxLaunch& a) {
  if (a.data == SDCA_F32 && a.result == SDCA_F32) return launch_twoent_t<float, float>(a);
  if (a.data == SDCA_F32 && a.result == SDCA_F64) return launch_twoent_t<float, double>(a);
  if (a.data == SDCA_F64 && a.result == SDCA_F64) return launch_twoent_t<double, double>(a);
  if (a.data == SDCA_F64 && a.result == SDCA_F32) return launch_twoent_t<double, float>(a);
  return hipErrorInvalidValue;
}

hipError_t launch_two_ent_global(const ProxLaunch& a, void* scratch, size_t scratch_bytes) {
  if (a.data == SDCA_F32 && a.result == SDCA_F32)
    return launch_twoent_global_t<float, float>(a, scratch, scratch_bytes);
  if (a.data == SDCA_F32 && a.result == SDCA_F64)
    return launch_twoent_global_t<float, double>(a, scratch, scratch_bytes);
  if (a.data == SDCA_F64 && a.result == SDCA_F64)
    return launch_twoent_global_t<double, double>(a, scratch, scratch_bytes);
  if (a.data == SDCA_F64 && a.result == SDCA_F32)
    return launch_twoent_global_t<double, float>(a, scratch, scratch_bytes);
  return hipErrorInvalidValue;
}

hipError_t launch_ent_biased_global(const ProxLaunch& a, void* scratch, size_t scratch_bytes) {
  if (a.data == SDCA_F32 && a.result == SDCA_F32)
    return launch_entbias_global_t<float, float>(a, scratch, scratch_bytes);
  if (a.data == SDCA_F32 && a.result == SDCA_F64)
    return launch_entbias_global_t<float, double>(a, scratch, scratch_bytes);
  if (a.data == SDCA_F64 && a.result == SDCA_F64)
    return launch_entbias_global_t<double, double>(a, scratch, scratch_bytes);
  if (a.data == SDCA_F64 && a.result == SDCA_F32)
    return launch_entbias_global_t<double, float>(a, scratch, scratch_bytes);
  return hipErrorInvalidValue;
}

hipError_t launch_ent_biased(const ProxLaunch& a) {
  if (a.data == SDCA_F32 && a.result == SDCA_F32) return launch_t<float, float>(a);
  if (a.data == SDCA_F32 && a.result == SDCA_F64) return launch_t<float, double>(a);
  if (a.data == SDCA_F64 && a.result == SDCA_F64) return launch_t<double, double>(a);
  if (a.data == SDCA_F64 && a.result == SDCA_F32) return launch_t<double, float>(a);
  return hipErrorInvalidValue;
}

}  // namespace sdca_gpu
