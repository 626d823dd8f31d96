// Device-side closed forms shared by the gfx950 kernels (fp64 throughout).
//
//   spherical harmonics l=1..4 and their input VJP
//       src/kokkos_learned_energy_forces.cpp:14-139
//   PhysNet cutoff, Bernstein basis    src/kokkos_integrated_block0.cpp:138-163
//   exp-bump switch                    src/kokkos_physical_long_range.cpp:11-39
//   ZBL per directed edge              src/kokkos_physical_zbl.cpp:81-177
//   Coulomb + QDO dispersion pair      src/kokkos_physical_long_range.cpp:147-370
#pragma once

#include <hip/hip_runtime.h>

namespace so3lr_amd {

struct LrParams {
  double ke, sigma, cutoff, cuton_el, fine_factor, bohr, hartree, disp_scale, cuton_disp, full_scale;
  double shift, fshift;  // shifted-force constants at the cutoff
  // reciprocals of the constants above: 1/sigma, 1/bohr, 2/(sqrt(pi) sigma),
  // 1/(cutoff - cuton) of both switches
  double inv_sigma, inv_bohr, two_over_sqrtpi_sigma, inv_w_el, inv_w_disp;
  int n_ref;
};

struct ZblParams {
  double ke, rc, switch_off, p, d, a[4], c[4];
  // NLH repulsion (nlh_cap > 0): per element pair (min Z, max Z, from 1)
  // three amplitudes and rates in place of the screening sum
  const double *nlh_a, *nlh_b;
  int nlh_cap;
};

__device__ __forceinline__ double silu(double x) { return x / (1.0 + exp(-x)); }
__device__ __forceinline__ double silu_prime(double x) {
  const double s = 1.0 / (1.0 + exp(-x));
  return s * (1.0 + x * (1.0 - s));
}

// a * b + c as one three-operand v_fma_f64.  Where the scalar registers are
// full, the compiler keeps loop-invariant constants in vector registers and
// writes fma(p, r, c) as a copy of c plus the two-address v_fmac_f64; in a
// Horner loop that doubles the instruction count.
__device__ __forceinline__ double fma3(double a, double b, double c) {
  double d;
  asm("v_fma_f64 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
  return d;
}
// Lean forms for the long-range pair terms and the switch functions, which run
// once per long-range entry (about 900 per atom): the fewest VALU instructions
// at full fp64 accuracy (a few ulp), with no IEEE special-case handling:
//   e^x: Cody-Waite reduction x = n ln2 + r, |r| <= ln2 / 2, with ln2 split
//        into a 32-bit-exact high part and a low part, then the degree-13
//        Taylor polynomial of e^r (truncation < 4e-18 relative) and 2^n;
//        for -745 <= x <= 708 (below that the result underflows to 0);
//   1/d: the hardware reciprocal (2^-24) refined by two Newton steps
//        r <- r + r (1 - d r), each squaring the relative error.
// (The filter kernels' activations use a table-driven e^x in evaluator.hip.)
__device__ __forceinline__ double exp_lean(double x) {
  const double n = __builtin_rint(x * 1.4426950408889634074);
  double r = fma(n, -6.93147180369123816490e-01, x);
  r = fma(n, -1.90821492927058770002e-10, r);
  double p = 1.0 / 6227020800.0;  // 1/13!
  p = fma3(p, r, 1.0 / 479001600.0);
  p = fma3(p, r, 1.0 / 39916800.0);
  p = fma3(p, r, 1.0 / 3628800.0);
  p = fma3(p, r, 1.0 / 362880.0);
  p = fma3(p, r, 1.0 / 40320.0);
  p = fma3(p, r, 1.0 / 5040.0);
  p = fma3(p, r, 1.0 / 720.0);
  p = fma3(p, r, 1.0 / 120.0);
  p = fma3(p, r, 1.0 / 24.0);
  p = fma3(p, r, 1.0 / 6.0);
  p = fma3(p, r, 0.5);
  p = fma3(p, r, 1.0);
  p = fma3(p, r, 1.0);
  return __builtin_ldexp(p, int(n));
}
__device__ __forceinline__ double rcp_lean(double d) {
  double r = __builtin_amdgcn_rcp(d);
  r = fma(fma(-d, r, 1.0), r, r);
  return fma(fma(-d, r, 1.0), r, r);
}

// degree slot (0..3 for l = 1..4) of equivariant channel m in 0..23
__device__ __forceinline__ int degree_slot(int m) { return m < 3 ? 0 : (m < 8 ? 1 : (m < 15 ? 2 : 3)); }
// (-1)^l for the slot: the parity of Y_l under v -> -v
__device__ __forceinline__ double slot_parity(int slot) { return (slot & 1) ? 1.0 : -1.0; }

constexpr double kPi = 3.141592653589793238462643383279502884;

// One real harmonic Y_m(u), m in 0..23 (l=1: y z x; then l=2,3,4 in m=-l..l).
__device__ __forceinline__ double sh_component(int m, double x, double y, double z) {
  switch (m) {
    case 0: return 0.48860251190291992159 * y;   // sqrt(3/(4pi))
    case 1: return 0.48860251190291992159 * z;
    case 2: return 0.48860251190291992159 * x;
    case 3: return 1.09254843059207907054 * x * y;  // 0.5 sqrt(15/pi)
    case 4: return 1.09254843059207907054 * y * z;
    case 5: return 0.31539156525252000603 * (3.0 * z * z - 1.0);  // 0.25 sqrt(5/pi)
    case 6: return 1.09254843059207907054 * x * z;
    case 7: return 0.54627421529603953527 * (x * x - y * y);  // 0.25 sqrt(15/pi)
    case 8: return 0.59004358992664351035 * y * (3.0 * x * x - y * y);  // 0.25 sqrt(35/(2pi))
    case 9: return 2.89061144264055405538 * x * y * z;  // 0.5 sqrt(105/pi)
    case 10: return 0.45704579946446573616 * y * (5.0 * z * z - 1.0);  // 0.25 sqrt(21/(2pi))
    case 11: return 0.37317633259011539141 * (5.0 * z * z * z - 3.0 * z);  // 0.25 sqrt(7/pi)
    case 12: return 0.45704579946446573616 * x * (5.0 * z * z - 1.0);
    case 13: return 1.44530572132027702769 * (x * x - y * y) * z;  // 0.25 sqrt(105/pi)
    case 14: return 0.59004358992664351035 * x * (x * x - 3.0 * y * y);
    case 15: return 2.50334294179670453836 * x * y * (x * x - y * y);  // 0.75 sqrt(35/pi)
    case 16: return 1.77013076977993053104 * y * (3.0 * x * x - y * y) * z;  // 0.75 sqrt(35/(2pi))
    case 17: return 0.94617469575756001809 * x * y * (7.0 * z * z - 1.0);  // 0.75 sqrt(5/pi)
    case 18: return 0.66904654355728916795 * y * (7.0 * z * z * z - 3.0 * z);  // 0.75 sqrt(5/(2pi))
    case 19: return 0.10578554691520430380 * (35.0 * z * z * z * z - 30.0 * z * z + 3.0);  // 0.1875 sqrt(1/pi)
    case 20: return 0.66904654355728916795 * x * (7.0 * z * z * z - 3.0 * z);
    case 21: return 0.47308734787878000905 * (x * x - y * y) * (7.0 * z * z - 1.0);  // 0.375 sqrt(5/pi)
    case 22: return 1.77013076977993053104 * x * (x * x - 3.0 * y * y) * z;
    default: return 0.62583573544917613459 * (x * x * (x * x - 3.0 * y * y) - y * y * (3.0 * x * x - y * y));  // 0.1875 sqrt(35/pi)
  }
}

// d Y_m / d(x, y, z), u treated as a free 3-vector.
__device__ __forceinline__ void sh_component_grad(int m, double x, double y, double z, double &gx,
                                                  double &gy, double &gz) {
  gx = gy = gz = 0.0;
  switch (m) {
    case 0: gy = 0.48860251190291992159; break;
    case 1: gz = 0.48860251190291992159; break;
    case 2: gx = 0.48860251190291992159; break;
    case 3: { const double k = 1.09254843059207907054; gx = k * y; gy = k * x; break; }
    case 4: { const double k = 1.09254843059207907054; gy = k * z; gz = k * y; break; }
    case 5: gz = 0.31539156525252000603 * 6.0 * z; break;
    case 6: { const double k = 1.09254843059207907054; gx = k * z; gz = k * x; break; }
    case 7: { const double k = 0.54627421529603953527; gx = 2.0 * k * x; gy = -2.0 * k * y; break; }
    case 8: { const double k = 0.59004358992664351035; gx = 6.0 * k * x * y; gy = 3.0 * k * (x * x - y * y); break; }
    case 9: { const double k = 2.89061144264055405538; gx = k * y * z; gy = k * x * z; gz = k * x * y; break; }
    case 10: { const double k = 0.45704579946446573616; gy = k * (5.0 * z * z - 1.0); gz = 10.0 * k * y * z; break; }
    case 11: gz = 0.37317633259011539141 * (15.0 * z * z - 3.0); break;
    case 12: { const double k = 0.45704579946446573616; gx = k * (5.0 * z * z - 1.0); gz = 10.0 * k * x * z; break; }
    case 13: { const double k = 1.44530572132027702769; gx = 2.0 * k * x * z; gy = -2.0 * k * y * z; gz = k * (x * x - y * y); break; }
    case 14: { const double k = 0.59004358992664351035; gx = 3.0 * k * (x * x - y * y); gy = -6.0 * k * x * y; break; }
    case 15: { const double k = 2.50334294179670453836; gx = k * y * (3.0 * x * x - y * y); gy = k * x * (x * x - 3.0 * y * y); break; }
    case 16: { const double k = 1.77013076977993053104; gx = 6.0 * k * x * y * z; gy = 3.0 * k * (x * x - y * y) * z; gz = k * y * (3.0 * x * x - y * y); break; }
    case 17: { const double k = 0.94617469575756001809; gx = k * y * (7.0 * z * z - 1.0); gy = k * x * (7.0 * z * z - 1.0); gz = 14.0 * k * x * y * z; break; }
    case 18: { const double k = 0.66904654355728916795; gy = k * (7.0 * z * z * z - 3.0 * z); gz = k * y * (21.0 * z * z - 3.0); break; }
    case 19: gz = 0.10578554691520430380 * (140.0 * z * z * z - 60.0 * z); break;
    case 20: { const double k = 0.66904654355728916795; gx = k * (7.0 * z * z * z - 3.0 * z); gz = k * x * (21.0 * z * z - 3.0); break; }
    case 21: { const double k = 0.47308734787878000905; gx = 2.0 * k * x * (7.0 * z * z - 1.0); gy = -2.0 * k * y * (7.0 * z * z - 1.0); gz = 14.0 * k * z * (x * x - y * y); break; }
    case 22: { const double k = 1.77013076977993053104; gx = 3.0 * k * (x * x - y * y) * z; gy = -6.0 * k * x * y * z; gz = k * x * (x * x - 3.0 * y * y); break; }
    default: { const double k = 0.62583573544917613459; gx = 4.0 * k * x * (x * x - 3.0 * y * y); gy = 4.0 * k * y * (y * y - 3.0 * x * x); break; }
  }
}

// exp-bump switch: 1 at cuton, 0 at cutoff, value and d/dr
__device__ __forceinline__ void bump_switch(double r, double on, double off, double &val, double &der) {
  if (r >= off) { val = 0.0; der = 0.0; return; }
  const double w = off - on;
  const double c = (r - on) / w;
  const double left = 1.0 - c, right = c;
  const double sl = left > 1e-12 ? left : 1e-12, sr = right > 1e-12 ? right : 1e-12;
  const double el = left > 0.0 ? exp(-1.0 / sl) : 0.0;
  const double er = right > 0.0 ? exp(-1.0 / sr) : 0.0;
  const double den = el + er + 1e-12;
  val = el / den;
  const double dl = left > 0.0 ? -el / (sl * sl) : 0.0;
  const double dr = right > 0.0 ? er / (sr * sr) : 0.0;
  der = ((dl * den - el * (dl + dr)) / (den * den)) / w;
}

// Repulsion energy and d/dr of ONE directed edge (the value is symmetric in
// i, j): learned ZBL, or NLH tables (kokkos_physical_zbl.cpp:81-177).
__device__ __forceinline__ void zbl_directed(const ZblParams &P, double zi, double zj, double r,
                                             double &energy, double &grad) {
  energy = 0.0;
  grad = 0.0;
  if (!(r > 0.0) || r > P.rc * (1.0 + 1e-12)) return;
  const double xn = r / P.rc, x2 = xn * xn, x3 = x2 * xn;
  const double fc = r < P.rc ? 1.0 - 10.0 * x3 + 15.0 * x3 * xn - 6.0 * x3 * x2 : 0.0;
  const double dfc = r < P.rc ? (-30.0 * x2 + 60.0 * x3 - 30.0 * x3 * xn) / P.rc : 0.0;
  double sw, dsw;
  bump_switch(r, 0.0, P.switch_off, sw, dsw);
  const double zz = zi * zj;
  const double rs = r > 1e-6 ? r : 1e-6;
  const double inv = 1.0 / rs, dinv = r > 1e-6 ? -1.0 / (r * r) : 0.0;
  const double X = P.ke * fc * zz * inv;
  const double dX = P.ke * zz * (dfc * inv + fc * dinv);
  double Yv = 0.0, dY = 0.0;
  if (P.nlh_cap > 0) {
    const int za = int(zi < zj ? zi : zj), zb = int(zi < zj ? zj : zi);
    if (za >= 1 && zb <= P.nlh_cap) {
      const int base = ((za - 1) * P.nlh_cap + (zb - 1)) * 3;
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        const double amp = P.nlh_a[base + k], rt = P.nlh_b[base + k];
        const double ex = exp(-rt * r);
        Yv += amp * ex;
        dY -= rt * amp * ex;
      }
    }
  } else {
    const double rate = (pow(zi, P.p) + pow(zj, P.p)) * P.d;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const double ex = exp(-P.a[k] * r * rate);
      Yv += P.c[k] * ex;
      dY -= P.c[k] * P.a[k] * rate * ex;
    }
  }
  energy = 0.5 * sw * X * Yv;
  grad = 0.5 * (dsw * X * Yv + sw * dX * Yv + sw * X * dY);
}

struct LrPairTerms {
  double e_el, e_disp, pref, dh_self, radial;
  double dc_self;  // dE/dc_i of the C6 ratio (SEP_C6 only)
};

// bump_switch with 1 / (off - on) given, three reciprocals instead of seven
// divisions (same function; rounding differs in the last bits).
__device__ __forceinline__ void bump_switch_fast(double r, double on, double off, double inv_w, double &val,
                                                 double &der) {
  if (r >= off) { val = 0.0; der = 0.0; return; }
  const double c = (r - on) * inv_w;
  const double left = 1.0 - c, right = c;
  const double isl = rcp_lean(left > 1e-12 ? left : 1e-12), isr = rcp_lean(right > 1e-12 ? right : 1e-12);
  const double el = left > 0.0 ? exp_lean(-isl) : 0.0;
  const double er = right > 0.0 ? exp_lean(-isr) : 0.0;
  const double den = el + er + 1e-12, iden = rcp_lean(den);
  val = el * iden;
  const double dl = left > 0.0 ? -el * isl * isl : 0.0;
  const double dr = right > 0.0 ? er * isr * isr : 0.0;
  der = (dl * den - el * (dl + dr)) * iden * iden * inv_w;
}

// alpha^(1/7) for alpha > 0: a single-precision estimate refined by two
// Newton steps on x^7 = alpha, x <- (6 x + alpha / x^6) / 7 (each squares the
// relative error: 1e-7, 1e-13, below 1 ulp).
__device__ __forceinline__ double root7_lean(double a) {
  double x = double(__expf(__logf(float(a)) * (1.0f / 7.0f)));
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const double x3 = x * x * x;
    x = (6.0 * x + a * rcp_lean(x3 * x3)) * (1.0 / 7.0);
  }
  return x;
}

// erfcx(x) on [0, 3] in u = 2 x / 3 - 1, highest power first (gen_erfcx_poly.py)
// (in constant memory: read through the scalar cache, not held in registers)
static __constant__ double kErfcxPoly[26] = {
    -1.9285526545026629e-09, 5.7920154915414246e-09, -4.6119752723685525e-09,
    1.2374418534053267e-08, -6.8302916092557606e-08, 1.8960282584894505e-07,
    -4.5725982227457081e-07, 1.2076614734008636e-06, -3.1901620317342984e-06,
    8.1102004120020287e-06, -2.0126549072150048e-05, 4.8905112127983934e-05,
    -0.00011601010087456714, 0.00026818449435352847, -0.00060331955090763077,
    0.0013184708553075387, -0.0027932530866193999, 0.0057231897175237054,
    -0.011309695741544485, 0.021484255075844793, -0.039077115130126794,
    0.06772278857525682, -0.11114180538602185, 0.17133983967481778,
    -0.2454343765988401, 0.32158541645431754,
};
// erf(x) = 1 - e^{-x^2} erfcx(x) for 0 <= x <= 3 (absolute error < 4e-16),
// given e^{-x^2}.  Used when the model's cutoff / sigma is at most 3.
__device__ __forceinline__ double erf_lean(double x, double exp_mx2) {
  const double u = x * (2.0 / 3.0) - 1.0;
  double p = kErfcxPoly[0];
#pragma unroll
  for (int k = 1; k < 26; ++k) p = fma3(p, u, kErfcxPoly[k]);
  return fma(-exp_mx2, p, 1.0);
}

// Coulomb + QDO dispersion for one unique pair seen from atom "i" (self)
// (kokkos_physical_long_range.cpp:62-381).  dh_self = dE/dh_i; pref * q_j =
// dE/dq_i.  Returns false outside the cutoff.  Divisions are shared through
// reciprocals (1/r, 1/den, 1/s_fit, 1/(7 alpha), 1/d6, 1/d8, 1/d10; 1/gamma =
// 2 s_fit^2 exactly).  This runs once per long-range entry (about 900 per
// atom), so the reciprocals, e^x and alpha^(1/7) take the lean forms above.
// LEAN_ERF: erf(r / sigma) by erf_lean (the caller has checked cutoff / sigma <= 3)
// SEP_C6: the model's C6 head gives C6_i = C6_ref c_i (ci, cj); h then
// enters through the polarisabilities only (kokkos_physical_long_range.cpp:
// 217-285), and dc_self = dE/dc_i
template <bool LEAN_ERF, bool SEP_C6 = false>
__device__ __forceinline__ bool lr_pair_terms(const LrParams &P, const double *__restrict__ aref,
                                              const double *__restrict__ cref, int zi_, int zj_,
                                              double qi, double qj, double hi, double hj, double r,
                                              LrPairTerms &o, double ci = 0.0, double cj = 0.0) {
  if (!(r > 1e-12) || r >= P.cutoff) return false;
  const double ir = rcp_lean(r);
  double esw, desw;
  bump_switch_fast(r, P.cuton_el, P.cutoff, P.inv_w_el, esw, desw);
  const double ratio = r * P.inv_sigma;
  const double expt = exp_lean(-ratio * ratio), erft = LEAN_ERF ? erf_lean(ratio, expt) : erf(ratio);
  const double pot = erft * ir;
  const double dpot = (r * expt * P.two_over_sqrtpi_sigma - erft) * ir * ir;
  const double disp = r - P.cutoff;
  const double shifted = pot - P.shift - P.fshift * disp;
  const double kern = esw * (pot - P.shift) + (1.0 - esw) * shifted;
  const double dkern = dpot - (1.0 - esw) * P.fshift + desw * P.fshift * disp;
  const double sk = P.full_scale * P.ke;
  o.e_el = sk * qi * qj * kern;
  o.pref = sk * kern;
  o.radial = sk * qi * qj * dkern;
  o.e_disp = 0.0;
  o.dh_self = 0.0;
  o.dc_self = 0.0;
  const int zi = zi_ - 1, zj = zj_ - 1;
  if (zi < 0 || zj < 0 || zi >= P.n_ref || zj >= P.n_ref) return true;
  const double ai0 = aref[zi], aj0 = aref[zj], ci0 = cref[zi], cj0 = cref[zj];
  const double ai = ai0 * hi, aj = aj0 * hj;
  const double c6i = SEP_C6 ? ci0 * ci : ci0 * hi * hi, c6j = SEP_C6 ? cj0 * cj : cj0 * hj * hj;
  const double alpha = 0.5 * (ai + aj);
  const double num = 2.0 * c6i * c6j * aj * ai;
  const double den = ai * ai * c6j + aj * aj * c6i;
  if (!(alpha > 0.0 && den > 1e-30)) return true;
  const double iden = rcp_lean(den);
  const double c6 = num * iden;
  double dc6_dhi, dc6_dci = 0.0;
  if constexpr (SEP_C6) {
    dc6_dhi = (2.0 * c6i * c6j * aj * ai0 * den - num * 2.0 * ai * ai0 * c6j) * iden * iden;
    dc6_dci = (2.0 * ci0 * c6j * aj * ai * den - num * aj * aj * ci0) * iden * iden;
  } else {
    const double dc6i = 2.0 * ci0 * hi;
    const double dn_dhi = 2.0 * (dc6i * c6j * aj * ai + c6i * c6j * aj * ai0);
    const double dd_dhi = 2.0 * ai * ai0 * c6j + aj * aj * dc6i;
    dc6_dhi = (dn_dhi * den - num * dd_dhi) * iden * iden;
  }
  const double b0 = -0.00433008, b1 = 0.24428889, b2 = 0.04125273, b3 = -0.00078893;
  const double a7 = root7_lean(alpha);
  const double i7a = rcp_lean(7.0 * alpha);
  const double rvdw = P.fine_factor * a7;
  const double sfit = b3 * rvdw * rvdw * rvdw + b2 * rvdw * rvdw + b1 * rvdw + b0;
  const double isfit = rcp_lean(sfit);
  const double gam = 0.5 * isfit * isfit, igam = 2.0 * sfit * sfit;
  const double drvdw = rvdw * i7a;
  const double dsfit = (3.0 * b3 * rvdw * rvdw + 2.0 * b2 * rvdw + b1) * drvdw;
  const double dgam = -2.0 * gam * dsfit * isfit;
  const double c8 = 5.0 * c6 * igam, c10 = (245.0 / 8.0) * c6 * igam * igam;
  const double damp = P.disp_scale * 2.0 * 2.54 * a7;
  const double ddamp = damp * i7a;
  const double ra = r * P.inv_bohr;
  const double r2 = ra * ra, r4 = r2 * r2, r6 = r4 * r2, r8 = r4 * r4, r10 = r8 * r2;
  const double p2 = damp * damp, p4 = p2 * p2, p6 = p4 * p2, p8 = p4 * p4, p10 = p8 * p2;
  const double i6 = rcp_lean(r6 + p6), i8 = rcp_lean(r8 + p8), i10 = rcp_lean(r10 + p10);
  const double qdo = -c6 * i6 - c8 * i8 - c10 * i10;
  const double rad_au = (6.0 * c6 * r4 * i6 * i6 + 8.0 * c8 * r6 * i8 * i8 + 10.0 * c10 * r8 * i10 * i10) * ra;
  const double dc8 = -c8 * dgam * igam, dc10 = -2.0 * c10 * dgam * igam;
  const double dd6 = 6.0 * p4 * damp * ddamp, dd8 = 8.0 * p6 * damp * ddamp,
               dd10 = 10.0 * p8 * damp * ddamp;
  const double dqdo_da = c6 * dd6 * i6 * i6 - dc8 * i8 + c8 * dd8 * i8 * i8 - dc10 * i10 + c10 * dd10 * i10 * i10;
  const double dqdo_dc6 = -i6 - 5.0 * igam * i8 - (245.0 / 8.0) * igam * igam * i10;
  const double dpi = dqdo_dc6 * dc6_dhi + dqdo_da * 0.5 * ai0;
  double dsw, ddsw;
  bump_switch_fast(r, P.cuton_disp, P.cutoff, P.inv_w_disp, dsw, ddsw);
  const double sh = P.full_scale * P.hartree;
  o.e_disp = sh * qdo * dsw;
  o.radial += sh * (rad_au * dsw * P.inv_bohr + qdo * ddsw);
  o.dh_self = sh * dsw * dpi;
  if constexpr (SEP_C6) o.dc_self = sh * dsw * dqdo_dc6 * dc6_dci;
  return true;
}

// Walks the active incidence entries of a node, [beg, end), in list order:
// 64 entries per coalesced load of iact / iother, then the active ones two at
// a time as uniform values, body(e1, o1, e2, o2, two) (when one is left the
// second repeats the first and `two` is false), so a body may issue both
// entries' loads before it sums either and still keep the order of a
// sequential walk.  All 64 lanes of the wavefront take part.
template <class Body>
__device__ __forceinline__ void for_active_pairs(int beg, int end, const int *__restrict__ iact,
                                                 const int *__restrict__ iother, int lane, Body &&body) {
  for (int k0 = beg; k0 < end; k0 += 64) {
    const int k = k0 + lane;
    const int ent = k < end ? iact[k] : -1;
    const int oth = k < end ? iother[k] : 0;
    unsigned long long mask = __ballot(ent >= 0);
    while (mask) {
      const int l1 = __ffsll(mask) - 1;
      mask &= mask - 1;
      const bool two = mask != 0;
      const int l2 = two ? __ffsll(mask) - 1 : l1;
      if (two) mask &= mask - 1;
      body(__builtin_amdgcn_readlane(ent, l1), __builtin_amdgcn_readlane(oth, l1),
           __builtin_amdgcn_readlane(ent, l2), __builtin_amdgcn_readlane(oth, l2), two);
    }
  }
}

}  // namespace so3lr_amd
