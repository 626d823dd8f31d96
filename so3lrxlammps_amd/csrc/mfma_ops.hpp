// fp64 MFMA operands shared by the fused kernels of evaluator.hip and
// generic.hip: the 16x16x4 fp64 MFMA and its chain over a 16-wide K chunk,
// weight fragments through buffer loads, the software-pipelined operand
// stream and the activations these kernels evaluate.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <type_traits>
#include <utility>

#include "radial_table.hpp"

namespace so3lr_amd {
namespace {

// fp64 MFMA V_MFMA_F64_16X16X4F64: D(16x16) += A(16x4) B(4x16) with
//   A[i][k] in lane i + 16k, B[k][j] in lane j + 16k,
//   D[i][j] in lane j + 16 (i % 4), register i / 4          (probed on gfx950).
// The filters run transposed: rows = features, columns = 16 pairs per
// wavefront.  A D tile then holds, in lane group g = lane / 16 and register r,
// feature 16 T + g + 4 r of pair lane % 16.  Taking the K index of the next
// layer in the same order (k = 16 T + g + 4 v) makes every layer's B operand
// the previous layer's D register, so activations never leave registers.
// Weights are pre-permuted on the host into that operand order, four K values
// per lane contiguous (permute_mfma).
typedef double v4d __attribute__((ext_vector_type(4)));
typedef double v2d __attribute__((ext_vector_type(2)));

__device__ __forceinline__ v4d mfma(double a, double b, v4d c) {
  return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}
// Weight fragments (one v4d per lane, 2 KiB per fragment) through buffer
// loads: the array base sits in a scalar buffer resource and the fragment
// offset in a scalar register, so a fragment costs two loads and no vector
// address arithmetic.  Descriptor word 3 = 0x00020000: raw 32-bit data
// format, as gfx9-family buffer loads expect.
typedef unsigned v4u __attribute__((ext_vector_type(4)));
__device__ __forceinline__ double u2_to_f64(unsigned lo, unsigned hi) {
  return __builtin_bit_cast(double, (unsigned long long)lo | ((unsigned long long)hi << 32));
}
__device__ __forceinline__ v4d frag_load(const double *P, int frag, int lane) {
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<double *>(P), 0, 0x7fffffff, 0x00020000);
  const v4u a = __builtin_amdgcn_raw_buffer_load_b128(rs, lane * 32, frag * 2048, 0);
  const v4u b = __builtin_amdgcn_raw_buffer_load_b128(rs, lane * 32 + 16, frag * 2048, 0);
  return v4d{u2_to_f64(a[0], a[1]), u2_to_f64(a[2], a[3]), u2_to_f64(b[0], b[1]), u2_to_f64(b[2], b[3])};
}
__device__ __forceinline__ v4d wload(const double *P, int KT, int mt, int T, int lane) {
  return frag_load(P, mt * KT + T, lane);
}
__device__ __forceinline__ v4d mfma4(const v4d &w, const v4d &b, v4d c) {
  c = mfma(w[0], b[0], c);
  c = mfma(w[1], b[1], c);
  c = mfma(w[2], b[2], c);
  return mfma(w[3], b[3], c);
}

// Compile-time loop: f(std::integral_constant<int, S>) for S = 0 .. N-1, so
// every register-array index below is a constant and nothing spills.
template <class F, int... S>
__device__ __forceinline__ void static_for_impl(F &f, std::integer_sequence<int, S...>) {
  (f(std::integral_constant<int, S>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F &&f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Software-pipelined operand stream: entry S (one v4d per lane: a weight
// fragment, a bias tile or a chunk of the incoming adjoint) is loaded PF
// entries before step S consumes it.  The scheduling fence after each step
// keeps the compiler from sinking the loads back next to their uses, so PF
// L2 round trips overlap the MFMAs of the steps in between.
template <int NS, int PF, class Load>
struct Stream {
  Load load;
  v4d buf[PF];
  __device__ __forceinline__ explicit Stream(Load l) : load(l) {}
  __device__ __forceinline__ void prime() {
    static_for<PF>([&](auto i) {
      constexpr int I = decltype(i)::value;
      if constexpr (I < NS) buf[I] = load(i);
    });
  }
  template <class Step>
  __device__ __forceinline__ void run(Step &&step) {
    static_for<NS>([&](auto si) {
      constexpr int S = decltype(si)::value;
      const v4d w = buf[S % PF];
      if constexpr (S + PF < NS) buf[S % PF] = load(std::integral_constant<int, S + PF>{});
      step(si, w);
      __builtin_amdgcn_sched_barrier(0);
    });
  }
};


// The same over a runtime loop of n iterations of NS entries each: entry S
// of iteration `it` (its kind and buffer slot fixed by S, its address by
// it) is loaded PF entries ahead, the last PF entries of an iteration
// loading the next iteration's first ones.  PF divides NS, so every buffer
// slot is a compile-time index.
template <int NS, int PF, class Load>
struct LoopStream {
  static_assert(NS % PF == 0 && PF <= NS, "stream depth must divide the loop body");
  Load load;  // load(std::integral_constant<int, S>, int it) -> v4d
  v4d buf[PF];
  __device__ __forceinline__ explicit LoopStream(Load l) : load(l) {}
  __device__ __forceinline__ void prime() {
    static_for<PF>([&](auto i) { buf[decltype(i)::value] = load(i, 0); });
  }
  template <class Step>
  __device__ __forceinline__ void run(int n, Step &&step) {
    for (int it = 0; it < n; ++it) {
      static_for<NS>([&](auto si) {
        constexpr int S = decltype(si)::value, N2 = S + PF;
        const v4d w = buf[S % PF];
        if constexpr (N2 < NS) buf[S % PF] = load(std::integral_constant<int, N2>{}, it);
        else if (it + 1 < n) buf[S % PF] = load(std::integral_constant<int, N2 - NS>{}, it + 1);
        step(si, it, w);
        __builtin_amdgcn_sched_barrier(0);
      });
    }
  }
};

// Activations of the MFMA filter kernels.  On gfx950 every VALU instruction a
// wavefront issues takes issue time from the fp64 MFMAs of its SIMD, so these
// are written for the fewest instructions: e^x = 2^m 2^(j/256) e^r with
// x = (256 m + j) ln2/256 + r, |r| <= ln2/512 (Cody-Waite, ln2/256 split into
// a 32-bit high part and a low part: exact reduction for |x| < 2800), 2^(j/256)
// from a 256-entry table in LDS and the degree-4 Taylor polynomial of e^r
// (truncation < 4e-17 relative).  The power 2^m is capped at 2^1000, which
// only matters for x > 693.
__device__ __forceinline__ double exp_tab(double x, const double *tab) {
  // t = x 256/ln2 + 1.5 2^52 rounds the product to an integer n held in the
  // low bits of t (exact for |n| < 2^51): n = t - 1.5 2^52, k = low word of t
  const double t = fma(x, 369.3299304675746, 6755399441055744.0);
  const double n = t - 6755399441055744.0;
  double r = fma(n, -0.00270760617331689, x);
  r = fma(n, -7.453964567463233e-13, r);
  const int k = int(unsigned(__builtin_bit_cast(unsigned long long, t)));
  double p = 1.0 / 24.0;
  p = fma(p, r, 1.0 / 6.0);
  p = fma(p, r, 0.5);
  p = fma(p, r, 1.0);
  p = fma(p, r, 1.0);
  return __builtin_ldexp(p * tab[k & 255], min(k >> 8, 1000));
}
// 1 / d from the hardware estimate (2^-24) and one Newton step: 2e-15
// relative, ample inside the activations
__device__ __forceinline__ double rcp_act(double d) {
  const double r = __builtin_amdgcn_rcp(d);
  return fma(fma(-d, r, 1.0), r, r);
}
__device__ __forceinline__ double silu_tab(double x, const double *tab) {
  return x * rcp_act(1.0 + exp_tab(-x, tab));
}
__device__ __forceinline__ double silu_prime_tab(double x, const double *tab) {
  const double s = rcp_act(1.0 + exp_tab(-x, tab));
  return s * (1.0 + x * (1.0 - s));
}
// The same for arguments of any size: the exponent is clamped to [-1000,
// 1000], where e^-x has long underflowed to 0 or reached the 2^1000 cap, so
// silu(x) = x (x > 1000) or 0 to within 1e-290 (x < -1000).  exp_tab's range
// ends near |x| = 5.8e6; the spherical filter branch takes the edge
// invariants of the equivariant features, whose size no weight bounds.
__device__ __forceinline__ double silu_tab_wide(double x, const double *tab) {
  return x * rcp_act(1.0 + exp_tab(-fmin(fmax(x, -1000.0), 1000.0), tab));
}
__device__ __forceinline__ double silu_prime_tab_wide(double x, const double *tab) {
  const double s = rcp_act(1.0 + exp_tab(-fmin(fmax(x, -1000.0), 1000.0), tab));
  return s * (1.0 + x * (1.0 - s));
}

// ---------------------------------------------------------------- radial tables
// Block 0's radial tables (evaluator.hip, generic.hip): per element pair
// {lo <= hi} (triangular index tri_key) and interval of r, one polynomial of
// degree kRadialDegree in t per logit, stored as kRadialCoefs / 2 coefficient
// pairs x L logits x 2: logit l's coefficients 2 kp and 2 kp + 1 at
// kp * 2 L + 2 l, so that the L lanes of a pair read 16 L contiguous bytes
// per load.
__device__ __forceinline__ int tri_key(int lo, int hi, int C) { return lo * C - lo * (lo - 1) / 2 + (hi - lo); }

// Interval and local coordinate t of r; below r0 the basis variable is
// clamped: the value at r0, slope 0 (inside = false).
__device__ __forceinline__ int radial_locate(double r, const RadialDomain &d, double &t, bool &inside) {
  inside = r >= d.r0;
  if (!inside) {
    t = -1.0;
    return 0;
  }
  const int i = int(fmin((r - d.r0) * (0.5 * d.scale), double(d.intervals - 1)));
  t = fma(r - fma(double(i), d.step, d.r0), d.scale, -1.0);
  return i;
}

// Logit l's polynomial at t from its record (L logits), Horner from the
// highest power.
template <int L>
__device__ __forceinline__ double radial_eval(const double *__restrict__ rec, int l, double t) {
  static_assert(kRadialCoefs % 2 == 0, "the table records hold coefficient pairs");
  double2 c[kRadialCoefs / 2];
#pragma unroll
  for (int kp = 0; kp < kRadialCoefs / 2; ++kp)
    c[kp] = *reinterpret_cast<const double2 *>(rec + kp * 2 * L + 2 * l);
  double v = c[kRadialCoefs / 2 - 1].y;
#pragma unroll
  for (int k = kRadialCoefs - 2; k >= 0; --k) v = fma(v, t, (k & 1) ? c[k >> 1].y : c[k >> 1].x);
  return v;
}

// A wavefront's 16 slots of an interval order (pairs bucketed by interval of
// r, each bucket padded with -1 to a multiple of 16 slots): the lane's pair p (-1:
// padding, whose lane works on the bucket's first pair and writes nothing),
// the interval i (the same in every lane), and the powers t^(16 c + g + 4 v)
// of chunk c in MFMA B-operand order (K index 16 c + g + 4 v).  False: the
// wavefront holds no pair.
__device__ __forceinline__ bool rint_slots(const int *n_slots, const int *order, const double *pr,
                                           const RadialDomain &d, int wave, int j, int g, int &p, int &i,
                                           bool &inside, v4d *tp) {
  const int q0 = wave * 16;
  if (wave < 0 || q0 >= *n_slots) return false;
  const int p0 = order[q0];
  if (p0 < 0) return false;  // a bucket's slots start with its pairs
  p = order[q0 + j];
  double t;
  i = __builtin_amdgcn_readfirstlane(radial_locate(pr[p >= 0 ? p : p0], d, t, inside));
  const double t2 = t * t, t4 = t2 * t2, t8 = t4 * t4, t16 = t8 * t8;
  tp[0][0] = g == 0 ? 1.0 : (g == 1 ? t : (g == 2 ? t2 : t2 * t));
  tp[0][1] = tp[0][0] * t4;
  tp[0][2] = tp[0][1] * t4;
  tp[0][3] = tp[0][2] * t4;
#pragma unroll
  for (int v = 0; v < 4; ++v) tp[1][v] = tp[0][v] * t16;
  return true;
}

}  // namespace
}  // namespace so3lr_amd
