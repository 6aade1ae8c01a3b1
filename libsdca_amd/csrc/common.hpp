// Device-side building blocks shared by the prox and evaluation kernels
// (gfx950, wave64).  Numeric semantics follow libsdca v0.3.1: comparisons and
// threshold arithmetic in the Result type R, element storage and the final
// clamp in the Data type D.
#ifndef SDCA_HIP_COMMON_HPP
#define SDCA_HIP_COMMON_HPP

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sdca_gpu {

template <class T> struct num;
template <> struct num<float> {
  __device__ __host__ static constexpr float eps() { return 1.19209290e-07f; }
  __device__ __host__ static constexpr float inf() { return __builtin_huge_valf(); }
  __device__ __host__ static constexpr float quiet_nan() { return __builtin_nanf(""); }
  __device__ __host__ static constexpr float min_normal() { return 1.17549435082228750797e-38f; }
  __device__ __host__ static constexpr float max_finite() { return 3.40282346638528859812e+38f; }
  // exp_traits<float>::min_arg (math/log_exp.h:46-52)
  __device__ __host__ static constexpr float exp_min_arg() { return -8.733654022216796875000000e+01f; }
};
template <> struct num<double> {
  __device__ __host__ static constexpr double eps() { return 2.2204460492503131e-16; }
  __device__ __host__ static constexpr double inf() { return __builtin_huge_val(); }
  __device__ __host__ static constexpr double quiet_nan() { return __builtin_nan(""); }
  __device__ __host__ static constexpr double min_normal() { return 2.2250738585072013831e-308; }
  __device__ __host__ static constexpr double max_finite() { return 1.7976931348623157081e+308; }
  // exp_traits<double>::min_arg = log(DBL_MIN) (math/log_exp.h:27-34)
  __device__ __host__ static constexpr double exp_min_arg() { return -0x1.6232bdd7abcd2p+9; }
};

// e^x in double.  x = k ln2 + r with k = rint(x / ln2), by Cody and Waite's
// two-constant reduction (ln2 = L1 + L2, L1 holding 32 significant bits so
// that k L1 is exact for |k| < 2^21); e^r from its Taylor series to degree 13
// (|r| <= ln2 / 2 leaves a truncation error below 0.05 ulp), by Horner's rule
// in FMA; 2^k applied by ldexp, which also rounds the subnormal and
// overflowing results.  Within about 1 ulp of e^x, in 26 vector
// instructions against the device library's 47 (gfx950).  Clamping x to [-745.5, 709.9] keeps k in
// range (outside it e^x rounds to 0 or overflows anyway); NaN passes through.
//
// a * b + c with the constant c read from a scalar register pair.  Written
// as fma(), a constant addend is copied into a vector register pair (two
// moves) before each v_fmac_f64; as an operand of v_fma_f64 it costs two
// scalar moves instead.
__device__ inline double fma_sconst(double a, double b, double c) {
  double d;
  asm("v_fma_f64 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "s"(c));
  return d;
}

__device__ inline double exp_fast(double x) {
  const double xc = fmin(fmax(x, -745.5), 709.9);
  const double k = rint(xc * 0x1.71547652b82fep+0);
  double r = fma(-k, 0x1.62e42fee00000p-1, xc);
  r = fma(-k, 0x1.a39ef35793c76p-33, r);
  double p = r * (1.0 / 6227020800.0) + 1.0 / 479001600.0;  // 1 / 13!, 1 / 12!
  p = fma_sconst(p, r, 1.0 / 39916800.0);
  p = fma_sconst(p, r, 1.0 / 3628800.0);
  p = fma_sconst(p, r, 1.0 / 362880.0);
  p = fma_sconst(p, r, 1.0 / 40320.0);
  p = fma_sconst(p, r, 1.0 / 5040.0);
  p = fma_sconst(p, r, 1.0 / 720.0);
  p = fma_sconst(p, r, 1.0 / 120.0);
  p = fma_sconst(p, r, 1.0 / 24.0);
  p = fma_sconst(p, r, 1.0 / 6.0);
  p = fma(p, r, 0.5);
  p = fma(p, r, 1.0);
  p = fma(p, r, 1.0);
  const double y = ldexp(p, static_cast<int>(k));
  return x != x ? x : y;
}

__device__ inline float dexp(float x) { return expf(x); }
// The exp map's kernels keep the device library's exp: with exp_fast the
// C3-size exp map ran 2 % slower (its time is not in the exponentials),
// while the Lambert evaluations below gain 2-13 % from it.
__device__ inline double dexp(double x) { return exp(x); }
__device__ inline float dlog(float x) { return logf(x); }
__device__ inline double dlog(double x) { return log(x); }
__device__ inline float dlog1p(float x) { return log1pf(x); }
__device__ inline double dlog1p(double x) { return log1p(x); }
__device__ inline float dmax(float a, float b) { return fmaxf(a, b); }
__device__ inline double dmax(double a, double b) { return fmax(a, b); }
__device__ inline float dmin(float a, float b) { return fminf(a, b); }
__device__ inline double dmin(double a, double b) { return fmin(a, b); }

// std::max(lo, std::min(x, hi)) with the argument order of proxdef.h:177:
// min(x, hi) returns x unless hi < x; max(lo, y) returns lo unless lo < y.
// The split p of a two-block column: the C ABI requires 1 <= p <= m - 1;
// device-resident per-column splits are not read back by the host, so an
// out-of-range value is brought into that range here and no access leaves
// the column or its LDS copy.
__device__ inline int clamp_split(int64_t p, int m) {
  return static_cast<int>(p < 1 ? 1 : (p > m - 1 ? m - 1 : p));
}

template <class D>
__device__ inline D clamp_ref(D x, D lo, D hi) {
  D y = (hi < x) ? hi : x;
  return (lo < y) ? y : lo;
}

// clamp_ref for lo <= hi' with hi' = max(lo, hi) precomputed per column (then
// clamp_ref(x, lo, hi) == clamp_med3(x, lo, hi') for every x that is not NaN,
// including lo > hi, where both give lo): one v_med3_f32 for float.
__device__ inline float clamp_med3(float x, float lo, float hi_eff) {
  return __builtin_amdgcn_fmed3f(x, lo, hi_eff);
}
__device__ inline double clamp_med3(double x, double lo, double hi_eff) {
  return clamp_ref(x, lo, hi_eff);
}

// n / d from the hardware reciprocal plus one Newton step on the residual
// (four instructions instead of the IEEE division sequence); within an ulp of
// the rounded quotient for the normal-range operands of the threshold
// updates.  Double uses the IEEE division.
__device__ inline float div_near(float n, float d) {
  const float r = __builtin_amdgcn_rcpf(d);
  const float q = n * r;
  const float e = __builtin_fmaf(-d, q, n);
  return __builtin_fmaf(e, r, q);
}
// Double: reciprocal, one Newton step on it, then one on the quotient.
__device__ inline double div_near(double n, double d) {
  const double r0 = __builtin_amdgcn_rcp(d);
  const double r = __builtin_fma(__builtin_fma(-d, r0, 1.0), r0, r0);
  const double q = n * r;
  return __builtin_fma(__builtin_fma(-d, q, n), r, q);
}

// x log x with 0 log 0 = 0 (math/log_exp.h:76-80).
template <class T>
__device__ inline T x_log_x(T x) { return (x > 0) ? x * dlog(x) : T(0); }

// ---------------------------------------------------------------------------
// Lambert W(exp(x)) (math/lambert.h:31-157): same intervals, same
// initialisation and the same order-5 Householder step.  The step's
// quotient uses div_near: its error scales the (small) correction, so W keeps
// full precision.
// ---------------------------------------------------------------------------
template <class T>
__device__ inline T lw_step5(T w, T y) {
  T f0 = w - y, f1 = T(1) + y;
  T f11 = f1 * f1, f0y = f0 * y;
  T f00y = f0 * f0y;
  return w - div_near(T(4) * f0 * (T(6) * f1 * (f11 + f0y) + f00y),
                      f11 * (T(24) * f11 + T(36) * f0y) + f00y * (T(14) * y + f0 + T(8)));
}

template <class T>
__device__ inline T exp_approx(T x) {
  T y = T(1) + x / T(1024);
#pragma unroll
  for (int i = 0; i < 10; ++i) y *= y;
  return y;
}

// The reference's branches (lambert.h:81-105 float, :125-156 double) give
// every x an initial w (with at most one intermediate step) and then the
// same final step lw_step5(w, exp(x - w)), or a closed form at the extremes.
// Here only the initial part is branch-specific; the exponential and the
// final step are issued once for the whole wave, so a wave whose lanes span
// several intervals pays for the costly part once instead of per branch.
// Each lane still computes exactly its branch's sequence.
__device__ inline float lambert_w_exp(float x) {
  const int br = x > -1.0f ? (x <= 8.0f ? 0 : (x <= 536870912.0f ? 1 : 2))
                           : (x > -18.0f ? 3 : 4);
  float w = 0.0f;
  if (br == 0) {
    w = lw_step5(x, 1.0f);
  } else if (br == 1) {
    w = x - logf(x);  // (8, 2^29]: the result is lw_step5(x - log x, x)
  } else if (br == 3) {
    w = exp_approx(x);
  }
  const float e = expf(br == 4 ? x : x - w);
  const float r = lw_step5(w, br == 1 ? x : e);
  return br == 2 ? x : (br == 4 ? ((x > -104.0f) ? e : 0.0f) : r);
}

__device__ inline double lambert_w_exp(double x) {
  const int br = x > 0.0 ? (x <= 4.0 ? 0 : (x <= 576460752303423488.0 ? 1 : 2))
                         : (x > -20.0 ? 3 : (x > -36.0 ? 4 : 5));
  double w = 0.0;
  if (br == 0) {
    w = lw_step5(x, 1.0);
  } else if (br == 1) {
    w = lw_step5(x - log(x), x);
  } else if (br == 3 || br == 4) {
    w = exp_approx(x);
    if (br == 3) w = lw_step5(w, exp_approx(x - w));
  }
  const double e = exp_fast(br == 5 ? x : x - w);
  const double r = lw_step5(w, e);
  return br == 2 ? x : (br == 5 ? ((x > -746.0) ? e : 0.0) : r);
}

// The same values with every branch's initial part computed and the
// lane's own selected (no divergent branches): for callers that evaluate a
// few independent points per thread in one latency chain, where branches
// around each point would serialise them.
__device__ inline float lambert_w_exp_nb(float x) {
  const int br = x > -1.0f ? (x <= 8.0f ? 0 : (x <= 536870912.0f ? 1 : 2))
                           : (x > -18.0f ? 3 : 4);
  const float w0 = lw_step5(x, 1.0f);
  const float w1 = x - logf(x);
  const float w3 = exp_approx(x);
  const float w = br == 0 ? w0 : (br == 1 ? w1 : (br == 3 ? w3 : 0.0f));
  const float e = expf(br == 4 ? x : x - w);
  const float r = lw_step5(w, br == 1 ? x : e);
  return br == 2 ? x : (br == 4 ? ((x > -104.0f) ? e : 0.0f) : r);
}

__device__ inline double lambert_w_exp_nb(double x) {
  const int br = x > 0.0 ? (x <= 4.0 ? 0 : (x <= 576460752303423488.0 ? 1 : 2))
                         : (x > -20.0 ? 3 : (x > -36.0 ? 4 : 5));
  const double w0 = lw_step5(x, 1.0);
  const double w1 = lw_step5(x - log(x), x);
  const double w4 = exp_approx(x);
  const double w3 = lw_step5(w4, exp_approx(x - w4));
  const double w = br == 0 ? w0 : (br == 1 ? w1 : (br == 3 ? w3 : (br == 4 ? w4 : 0.0)));
  const double e = exp_fast(br == 5 ? x : x - w);
  const double r = lw_step5(w, e);
  return br == 2 ? x : (br == 5 ? ((x > -746.0) ? e : 0.0) : r);
}

// a * b + c, the constant c from a scalar register for double (fma_sconst).
__device__ inline double fma_c(double a, double b, double c) { return fma_sconst(a, b, c); }
__device__ inline float fma_c(float a, float b, float c) { return __builtin_fmaf(a, b, c); }

// W(z) for 0 <= z <= 0.06 by its series z - z^2 + 3/2 z^3 - 8/3 z^4
// + 125/24 z^5 (relative error below 11 z^5 < 1e-5): a start for lw_step5.
template <class R>
__device__ inline R lambert_w_series5(R z) {
  R p = fma_c(z, R(125.0 / 24.0), R(-8.0 / 3.0));
  p = fma_c(p, z, R(1.5));
  p = fma_c(p, z, R(-1));
  p = fma_c(p, z, R(1));
  return p * z;
}

// e^-v for 0 <= v <= 0.06: the Taylor polynomial of degree 9 (the omitted
// term is below 0.06^10 / 10! < 2e-19).
template <class R>
__device__ inline R exp_neg_small(R v) {
  R p = fma_c(v, R(-1.0 / 362880.0), R(1.0 / 40320.0));
  p = fma_c(p, v, R(-1.0 / 5040.0));
  p = fma_c(p, v, R(1.0 / 720.0));
  p = fma_c(p, v, R(-1.0 / 120.0));
  p = fma_c(p, v, R(1.0 / 24.0));
  p = fma_c(p, v, R(-1.0 / 6.0));
  p = fma_c(p, v, R(0.5));
  p = fma_c(p, v, R(-1));
  return fma_c(p, v, R(1));
}

// W(exp(y - dt)) from w = W(exp(y)) by the Taylor series in dt: the
// derivatives of W(e^y) are g1 = w / (1 + w), g2 = w / (1 + w)^3 and
// g3 = w (1 - 2w) / (1 + w)^5, so for |dt| <= 1e-4 the omitted fourth-order
// term is below 1e-17 w.  Callers keep |dt| within that.
template <class R>
__device__ inline R lambert_w_exp_shift(R w, R dt) {
  const R rd = div_near(R(1), R(1) + w);
  const R rd2 = rd * rd;
  const R g1 = w * rd;
  const R g2 = g1 * rd2;
  const R g3 = g2 * (R(1) - R(2) * w) * rd2;
  const R hdt2 = R(0.5) * dt * dt;
  return w - dt * g1 + hdt2 * g2 - (hdt2 * dt * R(1.0 / 3.0)) * g3;
}
constexpr double kLambertShiftMax = 1e-4;

// The same function for inputs spread over all the intervals (the elementwise
// map over arbitrary x): the branches (0, 4], (4, 2^59] and (-20, 0] each
// start with one step lw_step5(w0, y0) from their own (w0, y0) = (x, 1),
// (x - log x, x), (e0, exp_approx(x - e0)) with e0 = exp_approx(x); here that
// step has one call site with per-lane arguments, so a wave spanning several
// intervals pays for it once.  Each lane computes exactly the operations of
// lambert_w_exp, so the results are identical; inside the iterations, where
// a wave's arguments mostly share an interval, lambert_w_exp is faster.
__device__ inline double lambert_w_exp_mixed(double x) {
  const int br = x > 0.0 ? (x <= 4.0 ? 0 : (x <= 576460752303423488.0 ? 1 : 2))
                         : (x > -20.0 ? 3 : (x > -36.0 ? 4 : 5));
  double w0 = x, y0 = 1.0;
  if (br == 1) {
    w0 = x - log(x);
    y0 = x;
  } else if (br == 3 || br == 4) {
    w0 = exp_approx(x);
    if (br == 3) y0 = exp_approx(x - w0);
  }
  double w = (br == 4) ? w0 : 0.0;
  if (br == 0 || br == 1 || br == 3) w = lw_step5(w0, y0);
  const double e = exp_fast(br == 5 ? x : x - w);
  const double r = lw_step5(w, e);
  return br == 2 ? x : (br == 5 ? ((x > -746.0) ? e : 0.0) : r);
}
__device__ inline float lambert_w_exp_mixed(float x) { return lambert_w_exp(x); }

// ---------------------------------------------------------------------------
// Cross-lane exchange lane <-> lane ^ OFF inside a wave.  OFF = 1, 2: DPP
// quad permutations (a VALU operand modifier).  Beyond, two forms:
//  * VALU = false: ds_swizzle in xor mode for 4, 8, 16 and ds_bpermute for
//    32.  They run on the LDS pipe, beside the VALU work: the form for the
//    column kernels, whose many waves per SIMD are throughput-bound;
//  * VALU = true: DPP row shifts by 4 (left for lanes with bit 2 clear,
//    right for the others), DPP row rotation by 8, v_permlane16_swap /
//    v_permlane32_swap for 16 and 32.  No LDS round trip (67 against about
//    400 ns for a 64-lane sum chain): the form for one workgroup running a
//    column alone, one wave per SIMD, latency-bound.
// Both give lane ^ OFF, so a reduction has the same bits either way.
// ---------------------------------------------------------------------------
template <int OFF, bool VALU = false>
__device__ inline int xor_lane(int v) {
  // bound_ctrl (last argument) set: a lane whose source is outside its row
  // reads 0, as the old value 0 would give, and the compiler needs no move
  // of 0 into the destination first.
  if constexpr (OFF == 1) {
    return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, true);  // quad_perm [1,0,3,2]
  } else if constexpr (OFF == 2) {
    return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, true);  // quad_perm [2,3,0,1]
  } else if constexpr (!VALU) {
    if constexpr (OFF < 32) {
      return __builtin_amdgcn_ds_swizzle(v, (OFF << 10) | 0x1F);  // and 0x1F, xor OFF
    } else {
      return __shfl_xor(v, OFF, 64);
    }
  } else if constexpr (OFF == 4) {
    const int up = __builtin_amdgcn_update_dpp(0, v, 0x104, 0xF, 0xF, true);  // row_shl:4
    const int dn = __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);  // row_shr:4
    return (__lane_id() & 4) ? dn : up;
  } else if constexpr (OFF == 8) {
    return __builtin_amdgcn_update_dpp(0, v, 0x128, 0xF, 0xF, true);  // row_ror:8
  } else {
    // The swap with both operands v leaves rows (r0, r0, r2, r2) in the
    // first result and (r1, r1, r3, r3) in the second (16-lane rows; for
    // the 32-lane swap, halves (h0, h0) and (h1, h1)).
    static_assert(OFF == 16 || OFF == 32, "partner levels 1..32");
    const unsigned u = static_cast<unsigned>(v);
    const bool upper = (__lane_id() & OFF) != 0;
    if constexpr (OFF == 16) {
      const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
      return static_cast<int>(upper ? p[0] : p[1]);
    } else {
      const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
      return static_cast<int>(upper ? p[0] : p[1]);
    }
  }
}
template <int OFF, bool VALU = false>
__device__ inline float xor_lane(float v) {
  return __int_as_float(xor_lane<OFF, VALU>(__float_as_int(v)));
}
template <int OFF, bool VALU = false>
__device__ inline double xor_lane(double v) {
  const long long b = __double_as_longlong(v);
  const int lo = xor_lane<OFF, VALU>(static_cast<int>(b & 0xffffffffll));
  const int hi = xor_lane<OFF, VALU>(static_cast<int>(b >> 32));
  return __longlong_as_double((static_cast<long long>(hi) << 32) |
                              (static_cast<long long>(static_cast<unsigned>(lo))));
}

// ---------------------------------------------------------------------------
// Reductions over a group of G adjacent lanes of a wave (G a power of two,
// groups aligned to G).  Every lane of the group receives the result.
//
// G > 64: the group is the whole workgroup (blockDim.x == G, at most 16
// waves).  Each wave reduces in registers, lane 0 of every wave puts its
// result in LDS, and every thread combines the wave results in wave order,
// so all threads hold the same bits and branch alike on them.  Every thread
// of the workgroup must make the same sequence of these calls (they contain
// barriers).
// ---------------------------------------------------------------------------
constexpr int kMaxGroupWaves = 16;

// LDS words for the workgroup-wide reductions, one array per element type.
template <class T>
__device__ inline T* group_lds_words() {
  __shared__ T words[kMaxGroupWaves];
  return words;
}

// Make LDS writes of this wave visible to its own later reads.
__device__ inline void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
// Barrier between LDS writes and reads of a group: the wave's own ordering
// for groups inside a wave, a workgroup barrier for a workgroup-wide group.
template <int G>
__device__ inline void group_lds_sync() {
  if constexpr (G > 64) {
    __syncthreads();
  } else {
    wave_lds_sync();
  }
}

template <int G, class T, class Op>
__device__ inline T workgroup_combine(T x, Op op) {
  static_assert(G % 64 == 0 && G / 64 <= kMaxGroupWaves, "workgroup group of 2..16 waves");
  T* words = group_lds_words<T>();
  __syncthreads();  // the previous combine's readers are done with the words
  if ((threadIdx.x & 63) == 0) words[threadIdx.x >> 6] = x;
  __syncthreads();
  T r = words[0];
#pragma unroll
  for (int w = 1; w < G / 64; ++w) r = op(r, words[w]);
  return r;
}

// The lanes' part of a reduction over G <= 64 lanes (VALU: the exchange form).
template <int G, bool VALU, class T>
__device__ inline T lanes_sum(T x) {
  if constexpr (G >= 64) x += xor_lane<32, VALU>(x);
  if constexpr (G >= 32) x += xor_lane<16, VALU>(x);
  if constexpr (G >= 16) x += xor_lane<8, VALU>(x);
  if constexpr (G >= 8) x += xor_lane<4, VALU>(x);
  if constexpr (G >= 4) x += xor_lane<2, VALU>(x);
  if constexpr (G >= 2) x += xor_lane<1, VALU>(x);
  return x;
}
// The total of the 64 lanes of a wave by gfx9's DPP row reduction: pairs
// and quads by quad_perm, each 16-lane row by row_ror 4 and 8, rows 1 and 3
// add the last lane of rows 0 and 2 (row_bcast:15), rows 2 and 3 the last
// lane of the first half (row_bcast:31); lane 63 then holds the total and
// readlane gives every lane its bits.  Six DPP adds and a readlane against
// the butterfly's eighteen exchanges, moves and adds: the workgroup-wide
// reductions are latency-bound chains in one wave per SIMD.
template <int CTRL, int RM, bool B>
__device__ inline int dpp_bits(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, RM, 0xF, B);
}
template <int CTRL, int RM, bool B>
__device__ inline int dpp_add(int v) { return v + dpp_bits<CTRL, RM, B>(v); }
template <int CTRL, int RM, bool B>
__device__ inline float dpp_add(float v) {
  return v + __int_as_float(dpp_bits<CTRL, RM, B>(__float_as_int(v)));
}
template <int CTRL, int RM, bool B>
__device__ inline double dpp_add(double v) {
  const long long u = __double_as_longlong(v);
  const int lo = dpp_bits<CTRL, RM, B>(static_cast<int>(u & 0xffffffffll));
  const int hi = dpp_bits<CTRL, RM, B>(static_cast<int>(u >> 32));
  return v + __longlong_as_double((static_cast<long long>(hi) << 32) |
                                  static_cast<long long>(static_cast<unsigned>(lo)));
}
__device__ inline int lane63(int x) { return __builtin_amdgcn_readlane(x, 63); }
__device__ inline float lane63(float x) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63));
}
__device__ inline double lane63(double x) {
  const long long u = __double_as_longlong(x);
  const int lo = __builtin_amdgcn_readlane(static_cast<int>(u & 0xffffffffll), 63);
  const int hi = __builtin_amdgcn_readlane(static_cast<int>(u >> 32), 63);
  return __longlong_as_double((static_cast<long long>(hi) << 32) |
                              static_cast<long long>(static_cast<unsigned>(lo)));
}
// Lane l's value (l uniform) in every lane.
__device__ inline float read_lane(float x, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
}
__device__ inline double read_lane(double x, int l) {
  const long long u = __double_as_longlong(x);
  const int lo = __builtin_amdgcn_readlane(static_cast<int>(u & 0xffffffffll), l);
  const int hi = __builtin_amdgcn_readlane(static_cast<int>(u >> 32), l);
  return __longlong_as_double((static_cast<long long>(hi) << 32) |
                              static_cast<long long>(static_cast<unsigned>(lo)));
}
template <class T>
__device__ inline T wave_total(T x) {
  x = dpp_add<0xB1, 0xF, true>(x);    // quad_perm [1,0,3,2]
  x = dpp_add<0x4E, 0xF, true>(x);    // quad_perm [2,3,0,1]
  x = dpp_add<0x124, 0xF, true>(x);   // row_ror:4
  x = dpp_add<0x128, 0xF, true>(x);   // row_ror:8
  x = dpp_add<0x142, 0xA, false>(x);  // row_bcast:15 into rows 1 and 3
  x = dpp_add<0x143, 0xC, false>(x);  // row_bcast:31 into rows 2 and 3
  return lane63(x);
}

template <int G, class T>
__device__ inline T group_sum(T x) {
  if constexpr (G > 64) {
    return workgroup_combine<G>(wave_total(x), [](T a, T b) { return a + b; });
  } else {
    return lanes_sum<G, false>(x);
  }
}
// Several group sums in one exchange: each value reduced as group_sum<G>
// would, the workgroup-wide ones through one pair of barriers for all of
// them (the same wave-order sums, so the same bits as separate calls).
template <class T>
__device__ inline void slot_put(unsigned long long& slot, T x) {
  static_assert(sizeof(T) <= sizeof(unsigned long long), "8-byte slots");
  __builtin_memcpy(&slot, &x, sizeof(T));
}
template <class T>
__device__ inline T slot_get(const unsigned long long& slot) {
  T x;
  __builtin_memcpy(&x, &slot, sizeof(T));
  return x;
}
template <int G, class T>
__device__ inline T slot_sum(const unsigned long long (*slots)[8], int i) {
  T r = slot_get<T>(slots[0][i]);
#pragma unroll
  for (int w = 1; w < G / 64; ++w) r = r + slot_get<T>(slots[w][i]);
  return r;
}
template <int G, class... T>
__device__ inline void group_sums(T&... x) {
  static_assert(sizeof...(T) <= 8, "at most 8 values per exchange");
  if constexpr (G > 64) {
    __shared__ unsigned long long slots[kMaxGroupWaves][8];
    ((x = wave_total(x)), ...);
    __syncthreads();  // the previous exchange's readers are done with the slots
    if ((threadIdx.x & 63) == 0) {
      const int w = static_cast<int>(threadIdx.x) >> 6;
      int i = 0;
      ((slot_put(slots[w][i++], x)), ...);
    }
    __syncthreads();
    int i = 0;
    ((x = slot_sum<G, T>(slots, i++)), ...);
  } else {
    ((x = group_sum<G>(x)), ...);
  }
}

template <int OFF, bool VALU, class T>
__device__ inline T max_step(T x) {
  T y = xor_lane<OFF, VALU>(x);
  return (y > x) ? y : x;
}
template <int OFF, bool VALU, class T>
__device__ inline T min_step(T x) {
  T y = xor_lane<OFF, VALU>(x);
  return (y < x) ? y : x;
}
template <int G, bool VALU, class T>
__device__ inline T lanes_max(T x) {
  if constexpr (G >= 64) x = max_step<32, VALU>(x);
  if constexpr (G >= 32) x = max_step<16, VALU>(x);
  if constexpr (G >= 16) x = max_step<8, VALU>(x);
  if constexpr (G >= 8) x = max_step<4, VALU>(x);
  if constexpr (G >= 4) x = max_step<2, VALU>(x);
  if constexpr (G >= 2) x = max_step<1, VALU>(x);
  return x;
}
template <int G, bool VALU, class T>
__device__ inline T lanes_min(T x) {
  if constexpr (G >= 64) x = min_step<32, VALU>(x);
  if constexpr (G >= 32) x = min_step<16, VALU>(x);
  if constexpr (G >= 16) x = min_step<8, VALU>(x);
  if constexpr (G >= 8) x = min_step<4, VALU>(x);
  if constexpr (G >= 4) x = min_step<2, VALU>(x);
  if constexpr (G >= 2) x = min_step<1, VALU>(x);
  return x;
}
template <int G, class T>
__device__ inline T group_max(T x) {
  if constexpr (G > 64) {
    return workgroup_combine<G>(lanes_max<64, true>(x), [](T a, T b) { return (b > a) ? b : a; });
  } else {
    return lanes_max<G, false>(x);
  }
}
template <int G, class T>
__device__ inline T group_min(T x) {
  if constexpr (G > 64) {
    return workgroup_combine<G>(lanes_min<64, true>(x), [](T a, T b) { return (b < a) ? b : a; });
  } else {
    return lanes_min<G, false>(x);
  }
}
// Exclusive prefix sum over the wave by DPP alone: each 16-lane row by row
// shifts (a lane whose source lies before its row reads 0), then the row
// totals carried by row_bcast:15 (into rows 1 and 3) and row_bcast:31 (into
// rows 2 and 3).  For the workgroup-wide scan (latency-bound).
__device__ inline int wave_exclusive_scan_dpp(int x) {
  int incl = x;
  incl += __builtin_amdgcn_update_dpp(0, incl, 0x111, 0xF, 0xF, true);  // row_shr:1
  incl += __builtin_amdgcn_update_dpp(0, incl, 0x112, 0xF, 0xF, true);  // row_shr:2
  incl += __builtin_amdgcn_update_dpp(0, incl, 0x114, 0xF, 0xF, true);  // row_shr:4
  incl += __builtin_amdgcn_update_dpp(0, incl, 0x118, 0xF, 0xF, true);  // row_shr:8
  incl += __builtin_amdgcn_update_dpp(0, incl, 0x142, 0xA, 0xF, false);  // row_bcast:15
  incl += __builtin_amdgcn_update_dpp(0, incl, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return incl - x;
}

// Exclusive prefix sum over the group (lane order g = 0..G-1).
template <int G>
__device__ inline int group_exclusive_scan(int x, int g) {
  if constexpr (G > 64) {
    // The wave's own scan plus the totals of the waves before it.
    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const int ex = wave_exclusive_scan_dpp(x);
    int* words = group_lds_words<int>();
    __syncthreads();
    if (lane == 63) words[wave] = ex + x;
    __syncthreads();
    int base = 0;
    for (int w = 0; w < wave; ++w) base += words[w];
    return base + ex;
  }
  int incl = x;
  const int lane = static_cast<int>(threadIdx.x) & 63;
  if constexpr (G >= 2) { int y = xor_lane<1>(incl); if (g & 1) incl += y; }
  // After step s every lane holds the inclusive sum of its aligned block of
  // 2^(s+1) lanes restricted to lanes <= itself; the xor partner supplies the
  // lower half's total.
  if constexpr (G >= 4) { int t = __shfl(incl, (lane & ~3) | 1, 64); if (g & 2) incl += t; }
  if constexpr (G >= 8) { int t = __shfl(incl, (lane & ~7) | 3, 64); if (g & 4) incl += t; }
  if constexpr (G >= 16) { int t = __shfl(incl, (lane & ~15) | 7, 64); if (g & 8) incl += t; }
  if constexpr (G >= 32) { int t = __shfl(incl, (lane & ~31) | 15, 64); if (g & 16) incl += t; }
  if constexpr (G >= 64) { int t = __shfl(incl, 31, 64); if (g & 32) incl += t; }
  return incl - x;
}

// Sorted (descending) top list of L values, insertion of one value:
// new[i] = max(old[i], min(old[i-1], x)) = median(old[i-1], old[i], x), one
// v_med3_f32 per level for float.
// +inf in a register the compiler cannot see through: a median with it is
// max(), issued as v_med3_f32 instead of a v_max_f32 that needs its inputs
// canonicalised first (one extra instruction per loaded value).
__device__ inline float opaque_inf() {
  float x = __builtin_inff();
  asm("" : "+v"(x));
  return x;
}

template <int L>
__device__ inline void top_insert(float (&top)[L], float x, float pinf = opaque_inf()) {
#pragma unroll
  for (int i = L - 1; i >= 1; --i) top[i] = __builtin_amdgcn_fmed3f(top[i - 1], top[i], x);
  top[0] = __builtin_amdgcn_fmed3f(top[0], x, pinf);
}
template <int L>
__device__ inline void top_insert(double (&top)[L], double x, double = 0) {
#pragma unroll
  for (int i = L - 1; i >= 1; --i) {
    double lo = (top[i - 1] < x) ? top[i - 1] : x;
    top[i] = (top[i] < lo) ? lo : top[i];
  }
  top[0] = (top[0] < x) ? x : top[0];
}

// Insertion of the (N+1)-th value into a list whose entries N.. are still
// -inf: levels above N stay -inf and level N takes min(top[N-1], x), so the
// insertion costs N + 1 operations instead of L.
template <int N, int L>
__device__ inline void top_insert_first(float (&top)[L], float x, float pinf) {
  static_assert(N < L, "a level of the list");
  if constexpr (N > 0) {
    top[N] = __builtin_amdgcn_fmed3f(top[N - 1], x, -pinf);
#pragma unroll
    for (int i = N - 1; i >= 1; --i) top[i] = __builtin_amdgcn_fmed3f(top[i - 1], top[i], x);
  }
  top[0] = __builtin_amdgcn_fmed3f(top[0], x, pinf);
}
template <int N, int L>
__device__ inline void top_insert_first(double (&top)[L], double x, double) {
  static_assert(N < L, "a level of the list");
  if constexpr (N > 0) {
    top[N] = (top[N - 1] < x) ? top[N - 1] : x;
#pragma unroll
    for (int i = N - 1; i >= 1; --i) {
      double lo = (top[i - 1] < x) ? top[i - 1] : x;
      top[i] = (top[i] < lo) ? lo : top[i];
    }
  }
  top[0] = (top[0] < x) ? x : top[0];
}

// The top list (entries -inf on entry) of the slots v[N..C): the first L
// slots by top_insert_first, the rest by top_insert.
template <int N, int L, int C, class D>
__device__ inline void top_fill(D (&top)[L], const D (&v)[C], D pinf) {
  if constexpr (N < C) {
    if constexpr (N < L) {
      top_insert_first<N>(top, v[N], pinf);
    } else {
      top_insert(top, v[N], pinf);
    }
    top_fill<N + 1>(top, v, pinf);
  }
}

// Merge the top lists of the G lanes of a group (every lane ends with the
// top L values of the union, as a multiset).
// Max and min for the sorting networks: for float the median of (a, b, ±inf)
// with an opaque infinity (pinf, made once per network), one v_med3_f32 and
// no NaN-quieting of the operands (which fmaxf/fminf add).
__device__ inline float net_max(float a, float b, float pinf) {
  return __builtin_amdgcn_fmed3f(a, b, pinf);
}
__device__ inline float net_min(float a, float b, float pinf) {
  return __builtin_amdgcn_fmed3f(a, b, -pinf);
}
__device__ inline double net_max(double a, double b, double) { return (a < b) ? b : a; }
__device__ inline double net_min(double a, double b, double) { return (b < a) ? b : a; }
__device__ inline float net_inf(float) { return opaque_inf(); }
__device__ inline double net_inf(double) { return __builtin_inf(); }

// Sorts a bitonic sequence of L (a power of two) values descending by
// half-cleaner stages of max/min pairs.
template <int L, class D>
__device__ inline void bitonic_clean_desc(D (&x)[L]) {
  const D pinf = net_inf(D(0));
#pragma unroll
  for (int stride = L / 2; stride > 0; stride >>= 1) {
#pragma unroll
    for (int i = 0; i < L; ++i) {
      if ((i & stride) == 0) {
        const D a = x[i], b = x[i + stride];
        x[i] = net_max(a, b, pinf);
        x[i + stride] = net_min(a, b, pinf);
      }
    }
  }
}

// Sorts L (a power of two) values descending by Batcher's bitonic network.
template <int L, class D>
__device__ inline void bitonic_sort_desc(D (&x)[L]) {
  const D pinf = net_inf(D(0));
#pragma unroll
  for (int size = 2; size <= L; size <<= 1) {
#pragma unroll
    for (int stride = size / 2; stride > 0; stride >>= 1) {
#pragma unroll
      for (int i = 0; i < L; ++i) {
        if ((i & stride) == 0) {
          const D a = x[i], b = x[i + stride];
          // descending runs where (i & size) == 0, ascending otherwise, so
          // that each merge sees a bitonic sequence; the last pass (size = L)
          // is all descending.
          const bool desc = (i & size) == 0;
          x[i] = desc ? net_max(a, b, pinf) : net_min(a, b, pinf);
          x[i + stride] = desc ? net_min(a, b, pinf) : net_max(a, b, pinf);
        }
      }
    }
  }
}

template <int OFF, bool VALU, int L, class D>
__device__ inline void top_merge_step(D (&top)[L]) {
  D other[L];
#pragma unroll
  for (int i = 0; i < L; ++i) other[i] = xor_lane<OFF, VALU>(top[i]);
  if constexpr (L == 16) {
    // Two descending lists: c_i = max(a_i, b_(L-1-i)) holds the L largest of
    // both and falls then rises (bitonic); a bitonic half-cleaner network
    // sorts it descending.  80 max/min instead of the 256 med3 of inserting
    // the other list entry by entry.
    const D pinf = net_inf(D(0));
#pragma unroll
    for (int i = 0; i < L; ++i) top[i] = net_max(top[i], other[L - 1 - i], pinf);
    bitonic_clean_desc<L>(top);
  } else {
#pragma unroll
    for (int i = 0; i < L; ++i) top_insert(top, other[i]);
  }
}
template <int G, int L, class D>
__device__ inline void top_merge(D (&top)[L]) {
  if constexpr (G > 64) {
    // Each wave's list through LDS; every thread merges them in wave order.
    static_assert(G % 64 == 0 && G / 64 <= kMaxGroupWaves, "workgroup group of 2..16 waves");
    __shared__ D lists[kMaxGroupWaves][L];
    top_merge_step<32, true>(top);
    top_merge_step<16, true>(top);
    top_merge_step<8, true>(top);
    top_merge_step<4, true>(top);
    top_merge_step<2, true>(top);
    top_merge_step<1, true>(top);
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) {
#pragma unroll
      for (int i = 0; i < L; ++i) lists[wave][i] = top[i];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < L; ++i) top[i] = lists[0][i];
    for (int w = 1; w < G / 64; ++w) {
#pragma unroll
      for (int i = 0; i < L; ++i) top_insert(top, lists[w][i]);
    }
    return;
  }
  if constexpr (G >= 64) top_merge_step<32, false>(top);
  if constexpr (G >= 32) top_merge_step<16, false>(top);
  if constexpr (G >= 16) top_merge_step<8, false>(top);
  if constexpr (G >= 8) top_merge_step<4, false>(top);
  if constexpr (G >= 4) top_merge_step<2, false>(top);
  if constexpr (G >= 2) top_merge_step<1, false>(top);
}

}  // namespace sdca_gpu

#endif
