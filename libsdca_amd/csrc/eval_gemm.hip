// Scores of the evaluation pass on the matrix cores: S = X W^T, i.e. for
// every example i and class j, S[i][j] = <x_i, w_j> - all the per-example
// gemv calls of eval_scores (eval/scores.h:21-26 -> cblas_sgemv) at once.
//
// Layout (column-major in the reference's terms = row-major here):
//   X: n rows (examples) of d contiguous features      (feature_input, data/input.h:14-18)
//   W: m rows (classes)  of d contiguous weights        (primal variables, context.h:36)
//   S: n rows (examples) of m contiguous scores
// Both operands are contiguous along the reduction dimension d.
//
// Tiling for gfx950: a 256-thread workgroup computes a 128 x 128 tile of S
// (128 examples x 128 classes) as 2 x 2 waves, each wave a 64 x 64 block of
// 2 x 2 v_mfma_f32_32x32x2f32 accumulators (64 fp32 accumulators per lane),
// or, when that pads m less, a 128 x 224 tile as 4 x 1 waves of 32 x 224
// (1 x 7 accumulators).
// K order (every fp32 score GEMM here, fused or not): k runs in groups of 8;
// MFMA step t (0..3) of group g sums k = 8g + t (lanes 0-31) and
// k = 8g + 4 + t (lanes 32-63), groups in increasing order, so every score
// is the same float whichever of these kernels forms it.  (From 2^32
// multiply-adds and 512 classes on, the unfused product goes to hipBLASLt:
// eval_blas.cpp.)
// Fast form (d % 16 == 0, 16-byte aligned operands; scores_gemm_fast_kernel):
// K advances in slabs of 16 held in LDS as [row][k] (rows padded to 20
// floats), so a lane's operands for four MFMA steps are one conflict-free
// ds_read_b128 and a 16-byte global load is one ds_write_b128.  The loads
// of slab s + 2 are issued as soon as slab s + 1 is in LDS (after the first
// half of slab s's MFMAs), so each has a whole slab of MFMAs to land, and
// the operand reads of the second half are interleaved with the first
// half's MFMAs.  Rows past n or m load the last row (their scores are not
// stored): no bounds branches in the loop.  83 % of the fp32 MFMA peak at
// d = 4096, m = 1000, n = 100,000 on MI355X.
// Generic form (any d, any alignment; scores_gemm_kernel): slabs of 16 read
// with bounds checks into registers while the previous slab is multiplied
// out of LDS, stored transposed to [k][row] so that the operand of lane l
// (row l % 32, k as above) is a conflict-free ds_read_b32.
// Both order the grid so that the 8 XCDs each own whole example blocks: the
// workgroups that share an X block run on one XCD and find it in that XCD's
// L2.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "eval_launch.hpp"

namespace sdca_gpu {

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int BK = 16;  // reduction slab

// Loads the slab [k0, k0 + BK) of rows [r0, r0 + ROWS) of a (rows x d)
// matrix into float4 registers (ROWS * 4 float4 per slab, NV per thread of
// NT); rows past `rows` and columns past d read as zero.
template <int ROWS, int NV, int NT>
__device__ inline void load_slab(const float* __restrict__ src, int64_t rows, int64_t d,
                                 int64_t r0, int64_t k0, bool vec, f32x4 (&r)[NV]) {
#pragma unroll
  for (int h = 0; h < NV; ++h) {
    const int f = static_cast<int>(threadIdx.x) + NT * h;  // float4 index in the slab
    const int row = f >> 2, q = f & 3;
    const int64_t gr = r0 + row;
    const int64_t gk = k0 + 4 * q;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (f < ROWS * 4 && gr < rows) {
      const float* p = src + gr * d + gk;
      if (vec && gk + 4 <= d) {
        v = *reinterpret_cast<const f32x4*>(p);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (gk + e < d) v[e] = p[e];
      }
    }
    r[h] = v;
  }
}

// Stores the float4 of a slab into LDS transposed to [k][row].
template <int ROWS, int NV, int NT>
__device__ inline void store_slab(float* __restrict__ lds, int ld, const f32x4 (&r)[NV]) {
#pragma unroll
  for (int h = 0; h < NV; ++h) {
    const int f = static_cast<int>(threadIdx.x) + NT * h;
    const int row = f >> 2, q = f & 3;
    if (f < ROWS * 4) {
#pragma unroll
      for (int e = 0; e < 4; ++e) lds[(4 * q + e) * ld + row] = r[h][e];
    }
  }
}

// One BM x BN tile of S per workgroup of WM x WN waves, each wave a
// (BM / WM) x (BN / WN) block of 32 x 32 accumulators.
template <int BM, int BN, int WM, int WN>
__global__ void __launch_bounds__(64 * WM * WN)
scores_gemm_kernel(const float* __restrict__ X, const float* __restrict__ W,
                   float* __restrict__ S, int64_t n, int64_t m, int64_t d,
                   int64_t tiles_m, int64_t tiles_n_padded, int vec) {
  constexpr int NT = 64 * WM * WN;           // threads
  constexpr int TM = BM / WM, TN = BN / WN;  // rows, columns of a wave's block
  static_assert(TM % 32 == 0 && TN % 32 == 0, "32 x 32 accumulators");
  constexpr int FM = TM / 32, FN = TN / 32;
  constexpr int LDA = BM + 4, LDB = BN + 4;  // padded LDS rows (floats)
  constexpr int NVA = (BM * 4 + NT - 1) / NT, NVB = (BN * 4 + NT - 1) / NT;
  __shared__ __align__(16) float As[2][BK * LDA];
  __shared__ __align__(16) float Bs[2][BK * LDB];

  // XCD-aware tile order: hardware places workgroup w on XCD w % 8.  Give
  // each XCD whole example blocks: consecutive workgroups on one XCD walk the
  // class tiles of the same example block.
  const int64_t w = blockIdx.x;
  const int64_t xcd = w % 8, slot = w / 8;
  const int64_t eb = (slot / tiles_m) * 8 + xcd;   // example block
  const int64_t cb = slot % tiles_m;                 // class block
  if (eb >= tiles_n_padded) return;
  const int64_t i0 = eb * BM, j0 = cb * BN;
  if (i0 >= n) return;

  const int lane = static_cast<int>(threadIdx.x) & 63;
  const int wave = static_cast<int>(threadIdx.x) >> 6;
  const int wr = wave / WN, wc = wave % WN;  // block of this wave
  const int lr = lane & 31, lk = lane >> 5;

  f32x16 acc[FM][FN];
#pragma unroll
  for (int a = 0; a < FM; ++a)
#pragma unroll
    for (int b = 0; b < FN; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;

  const bool vv = vec != 0;
  f32x4 ra[NVA], rb[NVB];
  load_slab<BM, NVA, NT>(X, n, d, i0, 0, vv, ra);
  load_slab<BN, NVB, NT>(W, m, d, j0, 0, vv, rb);
  store_slab<BM, NVA, NT>(As[0], LDA, ra);
  store_slab<BN, NVB, NT>(Bs[0], LDB, rb);
  __syncthreads();

  const int64_t nslabs = (d + BK - 1) / BK;
  for (int64_t s = 0; s < nslabs; ++s) {
    const int cur = static_cast<int>(s & 1);
    const bool more = s + 1 < nslabs;
    if (more) {
      load_slab<BM, NVA, NT>(X, n, d, i0, (s + 1) * BK, vv, ra);
      load_slab<BN, NVB, NT>(W, m, d, j0, (s + 1) * BK, vv, rb);
    }
    const float* as = As[cur];
    const float* bs = Bs[cur];
#pragma unroll
    for (int kk = 0; kk < BK; kk += 2) {
      const int kr = (kk & ~7) + 4 * lk + ((kk & 7) >> 1);  // the k order above
      float av[FM], bv[FN];
#pragma unroll
      for (int a = 0; a < FM; ++a) av[a] = as[kr * LDA + wr * TM + 32 * a + lr];
#pragma unroll
      for (int b = 0; b < FN; ++b) bv[b] = bs[kr * LDB + wc * TN + 32 * b + lr];
#pragma unroll
      for (int a = 0; a < FM; ++a)
#pragma unroll
        for (int b = 0; b < FN; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[a], bv[b], acc[a][b], 0, 0, 0);
    }
    if (more) {
      store_slab<BM, NVA, NT>(As[cur ^ 1], LDA, ra);
      store_slab<BN, NVB, NT>(Bs[cur ^ 1], LDB, rb);
    }
    __syncthreads();
  }

  // Accumulator r of lane l holds row 8 (r / 4) + 4 (l / 32) + r % 4 and
  // column l % 32 of its 32 x 32 block.
#pragma unroll
  for (int a = 0; a < FM; ++a) {
#pragma unroll
    for (int b = 0; b < FN; ++b) {
      const int64_t col = j0 + wc * TN + b * 32 + lr;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = i0 + wr * TM + a * 32 + 8 * (r / 4) + 4 * lk + (r % 4);
        if (row < n && col < m) S[row * m + col] = acc[a][b][r];
      }
    }
  }
}


// Loads rows [r0, r0 + ROWS) x k [k0, k0 + 16) of a (rows x d) matrix as
// float4 (NV per thread of NT); rows past `rows` load row rows - 1.
template <int ROWS, int NV, int NT>
__device__ inline void load_slab_fast(const float* __restrict__ src, int64_t rows, int64_t d,
                                      int64_t r0, int64_t k0, f32x4 (&r)[NV]) {
#pragma unroll
  for (int h = 0; h < NV; ++h) {
    const int f = static_cast<int>(threadIdx.x) + NT * h;  // float4 index in the slab
    if ((ROWS * 4) % NT == 0 || f < ROWS * 4) {
      int64_t gr = r0 + (f >> 2);
      gr = gr < rows ? gr : rows - 1;
      r[h] = *reinterpret_cast<const f32x4*>(src + gr * d + k0 + 4 * (f & 3));
    }
  }
}

// Stores a slab loaded by load_slab_fast as LDS rows [row][k] of LD floats.
template <int ROWS, int NV, int NT, int LD>
__device__ inline void store_slab_fast(float* __restrict__ lds, const f32x4 (&r)[NV]) {
#pragma unroll
  for (int h = 0; h < NV; ++h) {
    const int f = static_cast<int>(threadIdx.x) + NT * h;
    if ((ROWS * 4) % NT == 0 || f < ROWS * 4)
      *reinterpret_cast<f32x4*>(lds + (f >> 2) * LD + 4 * (f & 3)) = r[h];
  }
}

template <int BM, int BN, int WM, int WN>
__global__ void __launch_bounds__(64 * WM * WN)
scores_gemm_fast_kernel(const float* __restrict__ X, const float* __restrict__ W,
                        float* __restrict__ S, int64_t n, int64_t m, int64_t d,
                        int64_t tiles_m, int64_t tiles_n_padded) {
  constexpr int NT = 64 * WM * WN;           // threads
  constexpr int TM = BM / WM, TN = BN / WN;  // rows, columns of a wave's block
  static_assert(TM % 32 == 0 && TN % 32 == 0, "32 x 32 accumulators");
  constexpr int FM = TM / 32, FN = TN / 32;
  constexpr int LD = BK + 4;                 // padded LDS row (floats)
  constexpr int NVA = (BM * 4 + NT - 1) / NT, NVB = (BN * 4 + NT - 1) / NT;
  __shared__ __align__(16) float As[2][BM * LD];
  __shared__ __align__(16) float Bs[2][BN * LD];

  const int64_t w = blockIdx.x;  // XCD-aware tile order, as scores_gemm_kernel
  const int64_t xcd = w % 8, slot = w / 8;
  const int64_t eb = (slot / tiles_m) * 8 + xcd;
  const int64_t cb = slot % tiles_m;
  if (eb >= tiles_n_padded) return;
  const int64_t i0 = eb * BM, j0 = cb * BN;
  if (i0 >= n) return;

  const int lane = static_cast<int>(threadIdx.x) & 63;
  const int wave = static_cast<int>(threadIdx.x) >> 6;
  const int wr = wave / WN, wc = wave % WN;
  const int lr = lane & 31, lk = lane >> 5;

  f32x16 acc[FM][FN];
#pragma unroll
  for (int a = 0; a < FM; ++a)
#pragma unroll
    for (int b = 0; b < FN; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;

  const int64_t nslabs = d / BK;
  f32x4 ra[NVA], rb[NVB];
  load_slab_fast<BM, NVA, NT>(X, n, d, i0, 0, ra);
  load_slab_fast<BN, NVB, NT>(W, m, d, j0, 0, rb);
  store_slab_fast<BM, NVA, NT, LD>(As[0], ra);
  store_slab_fast<BN, NVB, NT, LD>(Bs[0], rb);
  if (nslabs > 1) {
    load_slab_fast<BM, NVA, NT>(X, n, d, i0, BK, ra);
    load_slab_fast<BN, NVB, NT>(W, m, d, j0, BK, rb);
  }
  __syncthreads();

  for (int64_t s = 0; s < nslabs; ++s) {
    const int cur = static_cast<int>(s & 1);
    // Lane l's operands: row l % 32 of each block, k 4 (l / 32) .. + 3 of
    // each group of 8.
    const float* as = As[cur] + (wr * TM + lr) * LD + 4 * lk;
    const float* bs = Bs[cur] + (wc * TN + lr) * LD + 4 * lk;
    f32x4 av[2][FM], bv[2][FN];
#pragma unroll
    for (int a = 0; a < FM; ++a) av[0][a] = *reinterpret_cast<const f32x4*>(as + 32 * a * LD);
#pragma unroll
    for (int b = 0; b < FN; ++b) bv[0][b] = *reinterpret_cast<const f32x4*>(bs + 32 * b * LD);
    // group 0: the second group's operands are read between its MFMAs
#pragma unroll
    for (int a = 0; a < FM; ++a) av[1][a] = *reinterpret_cast<const f32x4*>(as + 32 * a * LD + 8);
#pragma unroll
    for (int b = 0; b < FN; ++b) bv[1][b] = *reinterpret_cast<const f32x4*>(bs + 32 * b * LD + 8);
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int a = 0; a < FM; ++a)
#pragma unroll
        for (int b = 0; b < FN; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[0][a][t], bv[0][b][t], acc[a][b], 0, 0, 0);
#pragma unroll
    for (int u = 0; u < FM + FN; ++u) {
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // two MFMAs
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
    }
    // Slab s + 1 (in registers since the previous slab) goes to the other
    // buffer, which every wave finished reading before the last barrier;
    // then the loads of slab s + 2 start.
    if (s + 1 < nslabs) {
      store_slab_fast<BM, NVA, NT, LD>(As[cur ^ 1], ra);
      store_slab_fast<BN, NVB, NT, LD>(Bs[cur ^ 1], rb);
    }
    if (s + 2 < nslabs) {
      load_slab_fast<BM, NVA, NT>(X, n, d, i0, (s + 2) * BK, ra);
      load_slab_fast<BN, NVB, NT>(W, m, d, j0, (s + 2) * BK, rb);
    }
    // group 1
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int a = 0; a < FM; ++a)
#pragma unroll
        for (int b = 0; b < FN; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[1][a][t], bv[1][b][t], acc[a][b], 0, 0, 0);
    __syncthreads();
  }

  // Accumulator r of lane l holds row 8 (r / 4) + 4 (l / 32) + r % 4 and
  // column l % 32 of its 32 x 32 block.
#pragma unroll
  for (int a = 0; a < FM; ++a) {
#pragma unroll
    for (int b = 0; b < FN; ++b) {
      const int64_t col = j0 + wc * TN + b * 32 + lr;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = i0 + wr * TM + a * 32 + 8 * (r / 4) + 4 * lk + (r % 4);
        if (row < n && col < m) S[row * m + col] = acc[a][b][r];
      }
    }
  }
}

template <int BM, int BN, int WM, int WN>
hipError_t launch_tiles(const float* X, const float* W, float* S, int64_t n, int64_t m, int64_t d,
                        hipStream_t stream) {
  const int64_t tiles_m = (m + BN - 1) / BN;
  const int64_t tiles_n = (n + BM - 1) / BM;
  const int64_t tiles_n_padded = (tiles_n + 7) / 8 * 8;
  const int64_t grid = tiles_n_padded * tiles_m;
  const bool aligned = (reinterpret_cast<uintptr_t>(X) & 15) == 0 &&
                       (reinterpret_cast<uintptr_t>(W) & 15) == 0;
  if (aligned && d % BK == 0) {
    hipLaunchKernelGGL((scores_gemm_fast_kernel<BM, BN, WM, WN>), dim3(static_cast<unsigned>(grid)),
                       dim3(64 * WM * WN), 0, stream, X, W, S, n, m, d, tiles_m, tiles_n_padded);
    return hipGetLastError();
  }
  const int vec = (d % 4 == 0 && aligned) ? 1 : 0;
  hipLaunchKernelGGL((scores_gemm_kernel<BM, BN, WM, WN>), dim3(static_cast<unsigned>(grid)),
                     dim3(64 * WM * WN), 0, stream, X, W, S, n, m, d, tiles_m, tiles_n_padded, vec);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// fp64 scores on the matrix cores: v_mfma_f64_16x16x4f64 (78.6 TFLOP/s
// dense on MI355X, the same as the fp64 vector peak; the MFMA form needs no
// VALU issue).  A 256-thread workgroup computes a 64 x 64 tile of S as
// 2 x 2 waves of 32 x 32, each 2 x 2 accumulators of 16 x 16 (4 doubles per
// lane each).  K order (both fp64 kernels): k runs in groups of 8; MFMA step
// t (0, 1) of group g sums k = 8g + 2q + t over the lane quarters q = l / 16.
// Fast form (d % 16 == 0, 16-byte aligned operands;
// scores_gemm_f64_fast_kernel): slabs of 16 in LDS as [row][k] rows of 18
// doubles, 16-byte loads stored as one ds_write_b128, a lane's operands for
// two MFMA steps one ds_read_b128, loads of slab s + 2 issued once slab
// s + 1 is in LDS, rows past n or m clamped (80 % of the fp64 peak at
// d = 4096, m = 1000, n = 100,000).  Generic form (any d):
// slabs of 8 read with bounds checks into registers while the previous slab
// is multiplied out of LDS stored as [k][row] (+2 padding), where the
// operand of lane l (row l % 16, k as above) is a conflict-free ds_read_b64.
// ---------------------------------------------------------------------------
typedef double f64x4 __attribute__((ext_vector_type(4)));
typedef double f64x2 __attribute__((ext_vector_type(2)));
constexpr int BK64 = 8;

template <int ROWS>
__device__ inline void load_slab64(const double* __restrict__ src, int64_t rows, int64_t d,
                                   int64_t r0, int64_t k0, bool vec, f64x2 (&r)[ROWS * 4 / 256]) {
  constexpr int NV = ROWS * 4 / 256;  // (ROWS x 8 doubles) / 2 per load / 256 threads
#pragma unroll
  for (int h = 0; h < NV; ++h) {
    const int f = static_cast<int>(threadIdx.x) + 256 * h;  // double2 index in the slab
    const int row = f >> 2, q = f & 3;
    const int64_t gr = r0 + row;
    const int64_t gk = k0 + 2 * q;
    f64x2 v = {0.0, 0.0};
    if (gr < rows) {
      const double* p = src + gr * d + gk;
      if (vec && gk + 2 <= d) {
        v = *reinterpret_cast<const f64x2*>(p);
      } else {
#pragma unroll
        for (int e = 0; e < 2; ++e)
          if (gk + e < d) v[e] = p[e];
      }
    }
    r[h] = v;
  }
}

template <int ROWS>
__device__ inline void store_slab64(double* __restrict__ lds, int ld,
                                    const f64x2 (&r)[ROWS * 4 / 256]) {
  constexpr int NV = ROWS * 4 / 256;
#pragma unroll
  for (int h = 0; h < NV; ++h) {
    const int f = static_cast<int>(threadIdx.x) + 256 * h;
    const int row = f >> 2, q = f & 3;
#pragma unroll
    for (int e = 0; e < 2; ++e) lds[(2 * q + e) * ld + row] = r[h][e];
  }
}

__global__ void __launch_bounds__(256)
scores_gemm_f64_kernel(const double* __restrict__ X, const double* __restrict__ W,
                       double* __restrict__ S, int64_t n, int64_t m, int64_t d, int64_t tiles_m,
                       int64_t tiles_n_padded, int vec) {
  constexpr int BM = 64, BN = 64;
  constexpr int LD = 64 + 2;
  __shared__ __align__(16) double As[2][BK64 * LD];
  __shared__ __align__(16) double Bs[2][BK64 * LD];
  // XCD-aware order as in scores_gemm_kernel.
  const int64_t w = blockIdx.x;
  const int64_t xcd = w % 8, slot = w / 8;
  const int64_t eb = (slot / tiles_m) * 8 + xcd;
  const int64_t cb = slot % tiles_m;
  if (eb >= tiles_n_padded) return;
  const int64_t i0 = eb * BM, j0 = cb * BN;
  if (i0 >= n) return;
  const int lane = static_cast<int>(threadIdx.x) & 63;
  const int wave = static_cast<int>(threadIdx.x) >> 6;
  const int wr = wave >> 1, wc = wave & 1;
  const int lr = lane & 15, lk = lane >> 4;

  f64x4 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[a][b][e] = 0.0;

  const bool vv = vec != 0;
  f64x2 ra[BM * 4 / 256], rb[BN * 4 / 256];
  load_slab64<BM>(X, n, d, i0, 0, vv, ra);
  load_slab64<BN>(W, m, d, j0, 0, vv, rb);
  store_slab64<BM>(As[0], LD, ra);
  store_slab64<BN>(Bs[0], LD, rb);
  __syncthreads();
  const int64_t nslabs = (d + BK64 - 1) / BK64;
  for (int64_t s = 0; s < nslabs; ++s) {
    const int cur = static_cast<int>(s & 1);
    const bool more = s + 1 < nslabs;
    if (more) {
      load_slab64<BM>(X, n, d, i0, (s + 1) * BK64, vv, ra);
      load_slab64<BN>(W, m, d, j0, (s + 1) * BK64, vv, rb);
    }
    const double* as = As[cur];
    const double* bs = Bs[cur];
#pragma unroll
    for (int kk = 0; kk < BK64; kk += 4) {
      const int kr = 2 * lk + (kk >> 2);  // the k order above
      double av[2], bv[2];
#pragma unroll
      for (int a = 0; a < 2; ++a) av[a] = as[kr * LD + wr * 32 + 16 * a + lr];
#pragma unroll
      for (int b = 0; b < 2; ++b) bv[b] = bs[kr * LD + wc * 32 + 16 * b + lr];
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f64_16x16x4f64(av[a], bv[b], acc[a][b], 0, 0, 0);
    }
    if (more) {
      store_slab64<BM>(As[cur ^ 1], LD, ra);
      store_slab64<BN>(Bs[cur ^ 1], LD, rb);
    }
    __syncthreads();
  }
  // Accumulator e of lane l holds row l / 16 + 4 e and column l % 16 of its
  // 16 x 16 block (operands: lane l carries A[l % 16][l / 16] and
  // B[l / 16][l % 16]).
#pragma unroll
  for (int a = 0; a < 2; ++a) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int64_t col = j0 + wc * 32 + 16 * b + lr;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t row = i0 + wr * 32 + 16 * a + lk + 4 * e;
        if (row < n && col < m) S[row * m + col] = acc[a][b][e];
      }
    }
  }
}


// Loads rows [r0, r0 + ROWS) x k [k0, k0 + 16) of a (rows x d) double matrix
// as double2 (8 per row, NV per thread of 256); rows past `rows` load row
// rows - 1.
template <int ROWS, int NV>
__device__ inline void load_slab64_fast(const double* __restrict__ src, int64_t rows, int64_t d,
                                        int64_t r0, int64_t k0, f64x2 (&r)[NV]) {
#pragma unroll
  for (int h = 0; h < NV; ++h) {
    const int f = static_cast<int>(threadIdx.x) + 256 * h;
    int64_t gr = r0 + (f >> 3);
    gr = gr < rows ? gr : rows - 1;
    r[h] = *reinterpret_cast<const f64x2*>(src + gr * d + k0 + 2 * (f & 7));
  }
}

template <int ROWS, int NV, int LD>
__device__ inline void store_slab64_fast(double* __restrict__ lds, const f64x2 (&r)[NV]) {
#pragma unroll
  for (int h = 0; h < NV; ++h) {
    const int f = static_cast<int>(threadIdx.x) + 256 * h;
    *reinterpret_cast<f64x2*>(lds + (f >> 3) * LD + 2 * (f & 7)) = r[h];
  }
}

__global__ void __launch_bounds__(256)
scores_gemm_f64_fast_kernel(const double* __restrict__ X, const double* __restrict__ W,
                            double* __restrict__ S, int64_t n, int64_t m, int64_t d,
                            int64_t tiles_m, int64_t tiles_n_padded) {
  constexpr int BM = 64, BN = 64, KS = 16;  // tile, slab
  constexpr int LD = KS + 2;                // padded LDS row (doubles)
  constexpr int NV = BM * 8 / 256;          // double2 per thread and operand
  __shared__ __align__(16) double As[2][BM * LD];
  __shared__ __align__(16) double Bs[2][BN * LD];
  const int64_t w = blockIdx.x;  // XCD-aware order, as scores_gemm_kernel
  const int64_t xcd = w % 8, slot = w / 8;
  const int64_t eb = (slot / tiles_m) * 8 + xcd;
  const int64_t cb = slot % tiles_m;
  if (eb >= tiles_n_padded) return;
  const int64_t i0 = eb * BM, j0 = cb * BN;
  if (i0 >= n) return;
  const int lane = static_cast<int>(threadIdx.x) & 63;
  const int wave = static_cast<int>(threadIdx.x) >> 6;
  const int wr = wave >> 1, wc = wave & 1;
  const int lr = lane & 15, lk = lane >> 4;

  f64x4 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[a][b][e] = 0.0;

  const int64_t nslabs = d / KS;
  f64x2 ra[NV], rb[NV];
  load_slab64_fast<BM, NV>(X, n, d, i0, 0, ra);
  load_slab64_fast<BN, NV>(W, m, d, j0, 0, rb);
  store_slab64_fast<BM, NV, LD>(As[0], ra);
  store_slab64_fast<BN, NV, LD>(Bs[0], rb);
  if (nslabs > 1) {
    load_slab64_fast<BM, NV>(X, n, d, i0, KS, ra);
    load_slab64_fast<BN, NV>(W, m, d, j0, KS, rb);
  }
  __syncthreads();
  for (int64_t s = 0; s < nslabs; ++s) {
    const int cur = static_cast<int>(s & 1);
    // Lane l's operands: row l % 16 of each block, k 2 (l / 16), + 1 of
    // each group of 8.
    const double* as = As[cur] + (wr * 32 + lr) * LD + 2 * lk;
    const double* bs = Bs[cur] + (wc * 32 + lr) * LD + 2 * lk;
    f64x2 av[2][2], bv[2][2];
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        av[g][a] = *reinterpret_cast<const f64x2*>(as + 16 * a * LD + 8 * g);
        bv[g][a] = *reinterpret_cast<const f64x2*>(bs + 16 * a * LD + 8 * g);
      }
    // group 0; the second group's operand reads go between its MFMAs
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f64_16x16x4f64(av[0][a][t], bv[0][b][t], acc[a][b], 0, 0, 0);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // two MFMAs
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
    }
    // slab s + 1 to the other buffer (every wave finished reading it before
    // the last barrier), then the loads of slab s + 2
    if (s + 1 < nslabs) {
      store_slab64_fast<BM, NV, LD>(As[cur ^ 1], ra);
      store_slab64_fast<BN, NV, LD>(Bs[cur ^ 1], rb);
    }
    if (s + 2 < nslabs) {
      load_slab64_fast<BM, NV>(X, n, d, i0, (s + 2) * KS, ra);
      load_slab64_fast<BN, NV>(W, m, d, j0, (s + 2) * KS, rb);
    }
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f64_16x16x4f64(av[1][a][t], bv[1][b][t], acc[a][b], 0, 0, 0);
    __syncthreads();
  }
  // Accumulator e of lane l holds row l / 16 + 4 e and column l % 16 of its
  // 16 x 16 block.
#pragma unroll
  for (int a = 0; a < 2; ++a) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int64_t col = j0 + wc * 32 + 16 * b + lr;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t row = i0 + wr * 32 + 16 * a + lk + 4 * e;
        if (row < n && col < m) S[row * m + col] = acc[a][b][e];
      }
    }
  }
}

}  // namespace

hipError_t launch_scores_gemm_f64(const double* X, const double* W, double* S, int64_t n,
                                  int64_t m, int64_t d, hipStream_t stream) {
  const int64_t tiles_m = (m + 63) / 64;
  const int64_t tiles_n = (n + 63) / 64;
  const int64_t tiles_n_padded = (tiles_n + 7) / 8 * 8;
  const int64_t grid = tiles_n_padded * tiles_m;
  const bool aligned = (reinterpret_cast<uintptr_t>(X) & 15) == 0 &&
                       (reinterpret_cast<uintptr_t>(W) & 15) == 0;
  if (aligned && d % 16 == 0) {
    hipLaunchKernelGGL(scores_gemm_f64_fast_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                       stream, X, W, S, n, m, d, tiles_m, tiles_n_padded);
    return hipGetLastError();
  }
  const int vec = (d % 2 == 0 && aligned) ? 1 : 0;
  hipLaunchKernelGGL(scores_gemm_f64_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                     stream, X, W, S, n, m, d, tiles_m, tiles_n_padded, vec);
  return hipGetLastError();
}

hipError_t launch_scores_gemm_mfma(const float* X, const float* W, float* S, int64_t n,
                                   int64_t m, int64_t d, hipStream_t stream) {
  // Class tiles of 128 (2 x 2 waves of 64 x 64) or 224 (4 x 1 waves of
  // 32 x 224), whichever pads m less: m = 200 fills 89 % of one 224-wide
  // tile against 78 % of two 128-wide ones.
  const int64_t pad128 = (m + 127) / 128 * 128, pad224 = (m + 223) / 224 * 224;
  if (pad224 < pad128) return launch_tiles<128, 224, 4, 1>(X, W, S, n, m, d, stream);
  return launch_tiles<128, 128, 2, 2>(X, W, S, n, m, d, stream);
}

// Large products go to hipBLASLt (92.9 % of the fp32 MFMA peak at the C4
// shape against this file's 78-84 %); below kBlasMinMacs, and wherever the
// library declines, the MFMA kernel keeps the fused pass's k order, so the
// two-kernel pass gives the fused pass's bits there.
hipError_t launch_scores_gemm(const float* X, const float* W, float* S, int64_t n, int64_t m,
                              int64_t d, hipStream_t stream, void* blas_ws, size_t blas_ws_bytes) {
  if (blas_shape(n, m, d) && blas_scores_gemm(X, W, S, n, m, d, stream, blas_ws, blas_ws_bytes))
    return hipSuccess;
  return launch_scores_gemm_mfma(X, W, S, n, m, d, stream);
}

}  // namespace sdca_gpu
