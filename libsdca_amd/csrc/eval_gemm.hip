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
// 2 x 2 v_mfma_f32_32x32x2f32 accumulators (64 fp32 accumulators per lane).
// K advances in slabs of 16: every slab is read from global memory with
// 16-byte loads into registers while the previous slab is multiplied out of
// LDS, then stored into the other LDS buffer transposed to [k][row], so that
// the MFMA operand of lane l (row l % 32, k l / 32) is a conflict-free
// ds_read_b32.  The grid is ordered so that the 8 XCDs each own whole
// example blocks: the workgroups that share an X block run on one XCD and
// find it in that XCD's L2.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "eval_launch.hpp"

namespace sdca_gpu {

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 128;   // examples per tile
constexpr int BN = 128;   // classes per tile
constexpr int BK = 16;    // reduction slab
constexpr int LDA = BM + 4;  // padded LDS row (floats)
constexpr int LDB = BN + 4;

// Loads the slab [k0, k0 + BK) of rows [r0, r0 + 128) of a (rows x d) matrix
// into 2 float4 registers per thread (512 float4 per slab); rows past `rows`
// and columns past d read as zero.
__device__ inline void load_slab(const float* __restrict__ src, int64_t rows, int64_t d,
                                 int64_t r0, int64_t k0, bool vec, f32x4 (&r)[2]) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int f = static_cast<int>(threadIdx.x) + 256 * h;  // float4 index in the slab
    const int row = f >> 2, q = f & 3;
    const int64_t gr = r0 + row;
    const int64_t gk = k0 + 4 * q;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (gr < rows) {
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

// Stores the two float4 of a slab into LDS transposed to [k][row].
__device__ inline void store_slab(float* __restrict__ lds, int ld, const f32x4 (&r)[2]) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int f = static_cast<int>(threadIdx.x) + 256 * h;
    const int row = f >> 2, q = f & 3;
#pragma unroll
    for (int e = 0; e < 4; ++e) lds[(4 * q + e) * ld + row] = r[h][e];
  }
}

__global__ void __launch_bounds__(256)
scores_gemm_kernel(const float* __restrict__ X, const float* __restrict__ W,
                   float* __restrict__ S, int64_t n, int64_t m, int64_t d,
                   int64_t tiles_m, int64_t tiles_n_padded, int vec) {
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
  const int wr = wave >> 1, wc = wave & 1;  // 64 x 64 block of this wave
  const int lr = lane & 31, lk = lane >> 5;

  f32x16 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;

  const bool vv = vec != 0;
  f32x4 ra[2], rb[2];
  load_slab(X, n, d, i0, 0, vv, ra);
  load_slab(W, m, d, j0, 0, vv, rb);
  store_slab(As[0], LDA, ra);
  store_slab(Bs[0], LDB, rb);
  __syncthreads();

  const int64_t nslabs = (d + BK - 1) / BK;
  for (int64_t s = 0; s < nslabs; ++s) {
    const int cur = static_cast<int>(s & 1);
    const bool more = s + 1 < nslabs;
    if (more) {
      load_slab(X, n, d, i0, (s + 1) * BK, vv, ra);
      load_slab(W, m, d, j0, (s + 1) * BK, vv, rb);
    }
    const float* as = As[cur];
    const float* bs = Bs[cur];
#pragma unroll
    for (int kk = 0; kk < BK; kk += 2) {
      const int kr = kk + lk;
      const float a0 = as[kr * LDA + wr * 64 + lr];
      const float a1 = as[kr * LDA + wr * 64 + 32 + lr];
      const float b0 = bs[kr * LDB + wc * 64 + lr];
      const float b1 = bs[kr * LDB + wc * 64 + 32 + lr];
      acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b0, acc[0][0], 0, 0, 0);
      acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b1, acc[0][1], 0, 0, 0);
      acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b0, acc[1][0], 0, 0, 0);
      acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b1, acc[1][1], 0, 0, 0);
    }
    if (more) {
      store_slab(As[cur ^ 1], LDA, ra);
      store_slab(Bs[cur ^ 1], LDB, rb);
    }
    __syncthreads();
  }

  // Accumulator r of lane l holds row 8 (r / 4) + 4 (l / 32) + r % 4 and
  // column l % 32 of its 32 x 32 block.
#pragma unroll
  for (int a = 0; a < 2; ++a) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int64_t col = j0 + wc * 64 + b * 32 + lr;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = i0 + wr * 64 + a * 32 + 8 * (r / 4) + 4 * lk + (r % 4);
        if (row < n && col < m) S[row * m + col] = acc[a][b][r];
      }
    }
  }
}

}  // namespace

hipError_t launch_scores_gemm(const float* X, const float* W, float* S, int64_t n, int64_t m,
                              int64_t d, hipStream_t stream) {
  const int64_t tiles_m = (m + BN - 1) / BN;
  const int64_t tiles_n = (n + BM - 1) / BM;
  const int64_t tiles_n_padded = (tiles_n + 7) / 8 * 8;
  const int64_t grid = tiles_n_padded * tiles_m;
  const int vec = (d % 4 == 0 && (reinterpret_cast<uintptr_t>(X) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(W) & 15) == 0) ? 1 : 0;
  hipLaunchKernelGGL(scores_gemm_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0, stream,
                     X, W, S, n, m, d, tiles_m, tiles_n_padded, vec);
  return hipGetLastError();
}

}  // namespace sdca_gpu
