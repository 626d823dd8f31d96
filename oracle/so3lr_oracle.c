/*
 * CPU fp64 oracle for SO3LR -- TEST INFRASTRUCTURE ONLY (see so3lr_oracle.h).
 *
 * The evaluation walks directed edges exactly as the reference pair style
 * does; the reference's atomic scatters become deterministic CSR gathers over
 * receivers and senders.  Reverse mode is hand-derived, as in the reference.
 */
#include "so3lr_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define HW ORC_HW
#define HH ORC_HH

int orc_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

static const double PI = 3.141592653589793238462643383279502884;

/* The widths of one model (so3lr_architecture.cpp:197-212, 246-293).  Slot s
 * (one equivariant head) holds channels off[s] .. off[s+1]-1, all of degree
 * deg[s]; channel c replicates the unique harmonic sh[c] (the unique
 * harmonics are l = 1..4 in order, 2l+1 each, so with degrees 1,2,3,4 the
 * map is the identity and slot_of is so3_conv_invariants.segment_ids). */
typedef struct {
  int F, NH, E, R, NI, FH, HK;
  int deg[ORC_MAXS], off[ORC_MAXS + 1];
  int slot_of[ORC_MAXE], sh[ORC_MAXE];
} dims_t;

/* 0, or a nonzero code for widths outside what the oracle takes. */
static int model_dims(const orc_model *m, dims_t *d) {
  d->F = m->F > 0 ? (int)m->F : 128;
  d->R = m->R > 0 ? (int)m->R : 32;
  if (d->F % HW != 0 || d->F > ORC_MAXF || d->R > ORC_MAXR) return 1;
  d->NH = d->F / HW;
  if (d->NH > ORC_MAXS) return 1;
  const int slots = m->n_slots > 0 ? (int)m->n_slots : 4;
  if (slots != d->NH) return 1;
  d->off[0] = 0;
  for (int s = 0; s < d->NH; ++s) {
    d->deg[s] = m->n_slots > 0 ? (int)m->degrees[s] : s + 1;
    if (d->deg[s] < 1 || d->deg[s] > 4 || (s > 0 && d->deg[s] < d->deg[s - 1])) return 1;
    d->off[s + 1] = d->off[s] + 2 * d->deg[s] + 1;
    const int base = d->deg[s] * d->deg[s] - 1; /* unique harmonics of l below: l^2 - 1 */
    for (int k = 0; k < 2 * d->deg[s] + 1; ++k) {
      d->slot_of[d->off[s] + k] = s;
      d->sh[d->off[s] + k] = base + k;
    }
  }
  d->E = d->off[d->NH];
  d->NI = d->F + d->NH;
  d->FH = d->F / 4;
  d->HK = m->head_hidden > 0 ? (int)m->head_hidden : d->F;
  if (d->HK > ORC_MAXK) return 1;
  return 0;
}

/* Compensated (Kahan-Babuska-Neumaier) accumulation of the extensive totals:
 * energy and virial of a 150,000-atom cell sum tens of millions of terms, and
 * a plain running sum carries a rounding error of order 1e-12 relative that
 * would be the checker's own.  sum_add keeps the lost low part in c; the
 * total is s + c. */
typedef struct {
  double s, c;
} csum_t;
static void sum_add(csum_t *a, double x) {
  const double t = a->s + x;
  if (fabs(a->s) >= fabs(x))
    a->c += (a->s - t) + x;
  else
    a->c += (x - t) + a->s;
  a->s = t;
}
static double sum_value(const csum_t *a) { return a->s + a->c; }

static double silu(double x) { return x / (1.0 + exp(-x)); }
static double silu_prime(double x) {
  const double s = 1.0 / (1.0 + exp(-x));
  return s * (1.0 + x * (1.0 - s));
}
static double softplus(double x) { return (x > 0.0 ? x : 0.0) + log1p(exp(-fabs(x))); }

/* y[o] = b[o] + sum_i W[o][i] x[i]   (torch (out, in) layout) */
static void matvec(const double *W, const double *b, int out, int in,
                   const double *x, double *y) {
  for (int o = 0; o < out; ++o) {
    const double *w = W + (size_t)o * in;
    double s = 0.0;
    for (int i = 0; i < in; ++i) s += w[i] * x[i];
    y[o] = s + (b ? b[o] : 0.0);
  }
}
/* gx[i] += sum_o W[o][i] g[o] */
static void matvecT_acc(const double *W, int out, int in, const double *g, double *gx) {
  for (int o = 0; o < out; ++o) {
    const double *w = W + (size_t)o * in;
    const double go = g[o];
    if (go == 0.0) continue;
    for (int i = 0; i < in; ++i) gx[i] += w[i] * go;
  }
}

/* ---------------------------------------------------------------------- */
/* Real spherical harmonics, l = 1..4, orthonormal, m = -l..l order.      */
/* Follows kokkos_learned_energy_forces.cpp:14-63 (same polynomials).     */
/* ---------------------------------------------------------------------- */
void orc_spherical_harmonics(double x, double y, double z, double *Y) {
  const double k1 = sqrt(3.0 / (4.0 * PI));
  Y[0] = k1 * y; Y[1] = k1 * z; Y[2] = k1 * x;
  const double k2a = 0.5 * sqrt(15.0 / PI), k2b = 0.25 * sqrt(5.0 / PI), k2c = 0.25 * sqrt(15.0 / PI);
  Y[3] = k2a * x * y; Y[4] = k2a * y * z; Y[5] = k2b * (3.0 * z * z - 1.0);
  Y[6] = k2a * x * z; Y[7] = k2c * (x * x - y * y);
  const double k3a = 0.25 * sqrt(35.0 / (2.0 * PI)), k3b = 0.5 * sqrt(105.0 / PI),
               k3c = 0.25 * sqrt(21.0 / (2.0 * PI)), k3d = 0.25 * sqrt(7.0 / PI),
               k3e = 0.25 * sqrt(105.0 / PI);
  Y[8] = k3a * y * (3.0 * x * x - y * y); Y[9] = k3b * x * y * z;
  Y[10] = k3c * y * (5.0 * z * z - 1.0); Y[11] = k3d * (5.0 * z * z * z - 3.0 * z);
  Y[12] = k3c * x * (5.0 * z * z - 1.0); Y[13] = k3e * (x * x - y * y) * z;
  Y[14] = k3a * x * (x * x - 3.0 * y * y);
  const double k4a = 0.75 * sqrt(35.0 / PI), k4b = 0.75 * sqrt(35.0 / (2.0 * PI)),
               k4c = 0.75 * sqrt(5.0 / PI), k4d = 0.75 * sqrt(5.0 / (2.0 * PI)),
               k4e = 0.1875 * sqrt(1.0 / PI), k4f = 0.375 * sqrt(5.0 / PI),
               k4g = 0.1875 * sqrt(35.0 / PI);
  Y[15] = k4a * x * y * (x * x - y * y); Y[16] = k4b * y * (3.0 * x * x - y * y) * z;
  Y[17] = k4c * x * y * (7.0 * z * z - 1.0); Y[18] = k4d * y * (7.0 * z * z * z - 3.0 * z);
  Y[19] = k4e * (35.0 * z * z * z * z - 30.0 * z * z + 3.0);
  Y[20] = k4d * x * (7.0 * z * z * z - 3.0 * z);
  Y[21] = k4f * (x * x - y * y) * (7.0 * z * z - 1.0);
  Y[22] = k4b * x * (x * x - 3.0 * y * y) * z;
  Y[23] = k4g * (x * x * (x * x - 3.0 * y * y) - y * y * (3.0 * x * x - y * y));
}

/* Gradient of sum_m g[m] Y_m(u) with respect to u treated as a free 3-vector
 * (the polynomials above, differentiated term by term). */
static void sh_vjp(double x, double y, double z, const double *g, double *gu) {
  double gx = 0, gy = 0, gz = 0;
  const double k1 = sqrt(3.0 / (4.0 * PI));
  gy += k1 * g[0]; gz += k1 * g[1]; gx += k1 * g[2];
  const double k2a = 0.5 * sqrt(15.0 / PI), k2b = 0.25 * sqrt(5.0 / PI), k2c = 0.25 * sqrt(15.0 / PI);
  gx += g[3] * k2a * y; gy += g[3] * k2a * x;
  gy += g[4] * k2a * z; gz += g[4] * k2a * y;
  gz += g[5] * k2b * 6.0 * z;
  gx += g[6] * k2a * z; gz += g[6] * k2a * x;
  gx += g[7] * k2c * 2.0 * x; gy -= g[7] * k2c * 2.0 * y;
  const double k3a = 0.25 * sqrt(35.0 / (2.0 * PI)), k3b = 0.5 * sqrt(105.0 / PI),
               k3c = 0.25 * sqrt(21.0 / (2.0 * PI)), k3d = 0.25 * sqrt(7.0 / PI),
               k3e = 0.25 * sqrt(105.0 / PI);
  gx += g[8] * k3a * 6.0 * x * y; gy += g[8] * k3a * (3.0 * x * x - 3.0 * y * y);
  gx += g[9] * k3b * y * z; gy += g[9] * k3b * x * z; gz += g[9] * k3b * x * y;
  gy += g[10] * k3c * (5.0 * z * z - 1.0); gz += g[10] * k3c * 10.0 * y * z;
  gz += g[11] * k3d * (15.0 * z * z - 3.0);
  gx += g[12] * k3c * (5.0 * z * z - 1.0); gz += g[12] * k3c * 10.0 * x * z;
  gx += g[13] * k3e * 2.0 * x * z; gy -= g[13] * k3e * 2.0 * y * z; gz += g[13] * k3e * (x * x - y * y);
  gx += g[14] * k3a * (3.0 * x * x - 3.0 * y * y); gy -= g[14] * k3a * 6.0 * x * y;
  const double k4a = 0.75 * sqrt(35.0 / PI), k4b = 0.75 * sqrt(35.0 / (2.0 * PI)),
               k4c = 0.75 * sqrt(5.0 / PI), k4d = 0.75 * sqrt(5.0 / (2.0 * PI)),
               k4e = 0.1875 * sqrt(1.0 / PI), k4f = 0.375 * sqrt(5.0 / PI),
               k4g = 0.1875 * sqrt(35.0 / PI);
  gx += g[15] * k4a * (3.0 * x * x * y - y * y * y); gy += g[15] * k4a * (x * x * x - 3.0 * x * y * y);
  gx += g[16] * k4b * 6.0 * x * y * z; gy += g[16] * k4b * (3.0 * x * x - 3.0 * y * y) * z;
  gz += g[16] * k4b * y * (3.0 * x * x - y * y);
  gx += g[17] * k4c * y * (7.0 * z * z - 1.0); gy += g[17] * k4c * x * (7.0 * z * z - 1.0);
  gz += g[17] * k4c * 14.0 * x * y * z;
  gy += g[18] * k4d * (7.0 * z * z * z - 3.0 * z); gz += g[18] * k4d * y * (21.0 * z * z - 3.0);
  gz += g[19] * k4e * (140.0 * z * z * z - 60.0 * z);
  gx += g[20] * k4d * (7.0 * z * z * z - 3.0 * z); gz += g[20] * k4d * x * (21.0 * z * z - 3.0);
  gx += g[21] * k4f * 2.0 * x * (7.0 * z * z - 1.0); gy -= g[21] * k4f * 2.0 * y * (7.0 * z * z - 1.0);
  gz += g[21] * k4f * 14.0 * z * (x * x - y * y);
  gx += g[22] * k4b * (3.0 * x * x - 3.0 * y * y) * z; gy -= g[22] * k4b * 6.0 * x * y * z;
  gz += g[22] * k4b * x * (x * x - 3.0 * y * y);
  gx += g[23] * k4g * (4.0 * x * x * x - 12.0 * x * y * y);
  gy += g[23] * k4g * (4.0 * y * y * y - 12.0 * x * x * y);
  gu[0] = gx; gu[1] = gy; gu[2] = gz;
}

/* ---------------------------------------------------------------------- */
/* Charge/spin embedding (so3lr_charge_spin.cpp:52-114)                   */
/* ---------------------------------------------------------------------- */
static void charge_spin_module(int F, const double *wq, const double *wk, const double *wv,
                               const double *m1, const double *m3,
                               const int64_t counts[119], double psi, double *table) {
  if (psi == 0.0) return;
  const int row = psi < 0.0 ? 1 : 0;
  const double *k = wk + row * F, *v = wv + row * F;
  double y[119] = {0};
  double denom = 0.0;
  for (int zz = 1; zz <= 118; ++zz) {
    if (counts[zz] <= 0) continue;
    double qk = 0.0;
    for (int c = 0; c < F; ++c) qk += wq[c * 118 + (zz - 1)] * k[c];
    y[zz] = softplus(qk / sqrt((double)F));
    denom += (double)counts[zz] * y[zz];
  }
  double x[ORC_MAXF], sx[ORC_MAXF], h[ORC_MAXF], sh[ORC_MAXF], g[ORC_MAXF];
  for (int zz = 1; zz <= 118; ++zz) {
    if (counts[zz] <= 0) continue;
    const double a = psi * y[zz] / denom;
    for (int c = 0; c < F; ++c) { x[c] = a * v[c]; sx[c] = silu(x[c]); }
    matvec(m1, NULL, F, F, sx, h);
    for (int c = 0; c < F; ++c) sh[c] = silu(h[c]);
    matvec(m3, NULL, F, F, sh, g);
    for (int c = 0; c < F; ++c) table[(zz - 1) * F + c] += x[c] + g[c];
  }
}

int orc_charge_spin_table(const orc_model *m, const int64_t counts[119],
                          double total_charge, double unpaired, double *table) {
  dims_t d;
  if (model_dims(m, &d) != 0) return 1;
  const int F = d.F;
  memset(table, 0, sizeof(double) * 118 * F);
  charge_spin_module(F, m->t[ORC_CE_WQ], m->t[ORC_CE_WK], m->t[ORC_CE_WV], m->t[ORC_CE_M1],
                     m->t[ORC_CE_M3], counts, total_charge, table);
  charge_spin_module(F, m->t[ORC_SE_WQ], m->t[ORC_SE_WK], m->t[ORC_SE_WV], m->t[ORC_SE_M1],
                     m->t[ORC_SE_M3], counts, unpaired, table);
  return 0;
}

int orc_charge_multiplicity_problem(const int64_t counts[119], double Q, double M) {
  if (!isfinite(Q) || round(Q) != Q) return 1;
  if (!isfinite(M) || round(M) != M || M < 1.0) return 2;
  int64_t protons = 0;
  for (int zz = 1; zz <= 118; ++zz) protons += counts[zz] * zz;
  const int64_t electrons = protons - (int64_t)Q;
  const int64_t unpaired = (int64_t)M - 1;
  if (electrons < 0) return 3;
  if (unpaired > electrons) return 4;
  if ((electrons - unpaired) % 2 != 0) return 5;
  return 0;
}

/* ---------------------------------------------------------------------- */
/* Smooth switch used by ZBL and LR: exp-bump, value 1 at cuton, 0 at     */
/* cutoff, with the 1e-12 stabilisers of the reference                    */
/* (kokkos_physical_long_range.cpp:11-39, kokkos_physical_zbl.cpp:110-131) */
/* ---------------------------------------------------------------------- */
static void smooth_switch(double r, double on, double off, double *val, double *der) {
  if (r >= off) { *val = 0.0; *der = 0.0; return; }
  const double w = off - on;
  const double c = (r - on) / w;
  const double left = 1.0 - c, right = c;
  const double sl = left > 1e-12 ? left : 1e-12, sr = right > 1e-12 ? right : 1e-12;
  const double el = left > 0.0 ? exp(-1.0 / sl) : 0.0;
  const double er = right > 0.0 ? exp(-1.0 / sr) : 0.0;
  const double den = el + er + 1e-12;
  *val = el / den;
  const double dl = left > 0.0 ? -el / (sl * sl) : 0.0;
  const double dr = right > 0.0 ? er / (sr * sr) : 0.0;
  *der = ((dl * den - el * (dl + dr)) / (den * den)) / w;
}

/* Repulsion for one directed edge (kokkos_physical_zbl.cpp:81-177): learned
 * ZBL, or the NLH pair tables indexed (min Z, max Z) from 1, whose pairs
 * outside the tables get no screening term. */
static void zbl_edge(const orc_model *m, double zi, double zj, double r,
                     double *energy, double *grad) {
  const double rc = m->s[ORC_S_RMAX];
  *energy = 0.0; *grad = 0.0;
  if (!(r > 0.0) || r > rc * (1.0 + 1e-12)) return;
  const double xn = r / rc, x2 = xn * xn, x3 = x2 * xn;
  const double fc = r < rc ? 1.0 - 10.0 * x3 + 15.0 * x3 * xn - 6.0 * x3 * x2 : 0.0;
  const double dfc = r < rc ? (-30.0 * x2 + 60.0 * x3 - 30.0 * x3 * xn) / rc : 0.0;
  /* switching_fn(r, 0, switch_off): the bump with cuton 0 */
  double sw, dsw;
  {
    const double off = m->s[ORC_S_ZBL_SWITCH_OFF];
    const double c = r / off, left = 1.0 - c, right = c;
    const double sl = left > 1e-12 ? left : 1e-12, sr = right > 1e-12 ? right : 1e-12;
    const double el = left > 0.0 ? exp(-1.0 / sl) : 0.0;
    const double er = right > 0.0 ? exp(-1.0 / sr) : 0.0;
    const double den = el + er + 1e-12;
    const double dl = left > 0.0 ? -el / (sl * sl) : 0.0;
    const double dr = right > 0.0 ? er / (sr * sr) : 0.0;
    sw = el / den;
    dsw = ((dl * den - el * (dl + dr)) / (den * den)) / off;
  }
  const double zz = zi * zj;
  const double rs = r > 1e-6 ? r : 1e-6;
  const double inv = 1.0 / rs, dinv = r > 1e-6 ? -1.0 / (r * r) : 0.0;
  const double ke = m->s[ORC_S_ZBL_KE];
  const double X = ke * fc * zz * inv;
  const double dX = ke * zz * (dfc * inv + fc * dinv);
  double Yv = 0.0, dY = 0.0;
  if (m->repulsion == ORC_REP_NLH) {
    const int64_t za = (int64_t)(zi < zj ? zi : zj), zb = (int64_t)(zi < zj ? zj : zi);
    if (za >= 1 && zb <= m->nlh_cap) {
      const size_t base = ((size_t)(za - 1) * (size_t)m->nlh_cap + (size_t)(zb - 1)) * 3;
      for (int k = 0; k < 3; ++k) {
        const double amp = m->nlh_a[base + k], rate = m->nlh_b[base + k];
        const double ex = exp(-rate * r);
        Yv += amp * ex;
        dY -= rate * amp * ex;
      }
    }
  } else {
    const double rate = (pow(zi, m->s[ORC_S_ZBL_P]) + pow(zj, m->s[ORC_S_ZBL_P])) * m->s[ORC_S_ZBL_D];
    for (int k = 0; k < 4; ++k) {
      const double a = m->s[ORC_S_ZBL_A1 + k], c = m->s[ORC_S_ZBL_C1 + k];
      const double ex = exp(-a * r * rate);
      Yv += c * ex;
      dY -= c * a * rate * ex;
    }
  }
  *energy = 0.5 * sw * X * Yv;
  *grad = 0.5 * (dsw * X * Yv + sw * dX * Yv + sw * X * dY);
}

/* One LR half pair (kokkos_physical_long_range.cpp:147-380).  C6 of an atom
 * is C6_ref h^2 (v1) or, with a C6 head (sep), C6_ref c with c its C6 ratio;
 * the polarisability is alpha_ref h either way.  dci, dcj: dE/dc (sep only). */
typedef struct {
  double e_elec, e_disp, charge_pref, dhi, dhj, dci, dcj, radial;
  int valid;
} lr_pair_t;

static lr_pair_t lr_pair(const orc_model *m, int64_t zi_, int64_t zj_, double qi, double qj,
                         double hi, double hj, int sep, double cri, double crj, double r) {
  lr_pair_t o = {0, 0, 0, 0, 0, 0, 0, 0, 0};
  const double cutoff = m->s[ORC_S_LR_CUTOFF], sigma = m->s[ORC_S_LR_SIGMA];
  const double ke = m->s[ORC_S_LR_KE];
  if (!(r > 1e-12) || r >= cutoff) return o;
  o.valid = 1;
  const double inv_sqrt_pi = 1.0 / sqrt(PI);
  const double cr = cutoff / sigma;
  const double cerf = erf(cr), cexp = exp(-cr * cr);
  const double shift = cerf / cutoff;
  const double fshift = (2.0 * cutoff * cexp * inv_sqrt_pi / sigma - cerf) / (cutoff * cutoff);
  double esw, desw;
  smooth_switch(r, m->s[ORC_S_LR_CUTON_EL], cutoff, &esw, &desw);
  const double ratio = r / sigma;
  const double erft = erf(ratio), expt = exp(-ratio * ratio);
  const double pot = erft / r;
  const double dpot = (2.0 * r * expt * inv_sqrt_pi / sigma - erft) / (r * r);
  const double disp = r - cutoff;
  const double shifted = pot - shift - fshift * disp;
  const double kern = esw * (pot - shift) + (1.0 - esw) * shifted;
  const double dkern = dpot - (1.0 - esw) * fshift + desw * fshift * disp;
  const double full = 2.0 * m->s[ORC_S_LR_PAIR_SCALE];
  o.e_elec = full * ke * qi * qj * kern;
  o.charge_pref = full * ke * kern;
  double radial = full * ke * qi * qj * dkern;

  const int64_t zi = zi_ - 1, zj = zj_ - 1;
  if (zi >= 0 && zj >= 0 && zi < m->n_alpha_ref && zj < m->n_alpha_ref) {
    const double *aref = m->t[ORC_ALPHA_REF], *cref = m->t[ORC_C6_REF];
    const double ai0 = aref[zi], aj0 = aref[zj], ci0 = cref[zi], cj0 = cref[zj];
    const double ai = ai0 * hi, aj = aj0 * hj;
    const double c6i = sep ? ci0 * cri : ci0 * hi * hi, c6j = sep ? cj0 * crj : cj0 * hj * hj;
    const double alpha = 0.5 * (ai + aj);
    const double num = 2.0 * c6i * c6j * aj * ai;
    const double den = ai * ai * c6j + aj * aj * c6i;
    if (alpha > 0.0 && den > 1e-30) {
      const double c6 = num / den;
      const double idd = 1.0 / (den * den);
      double dc6_dhi, dc6_dhj, dc6_dci = 0.0, dc6_dcj = 0.0;
      if (!sep) {
        const double dc6i = 2.0 * ci0 * hi, dc6j = 2.0 * cj0 * hj;
        const double dn_dhi = 2.0 * (dc6i * c6j * aj * ai + c6i * c6j * aj * ai0);
        const double dn_dhj = 2.0 * (c6i * dc6j * aj * ai + c6i * c6j * aj0 * ai);
        const double dd_dhi = 2.0 * ai * ai0 * c6j + aj * aj * dc6i;
        const double dd_dhj = ai * ai * dc6j + 2.0 * aj * aj0 * c6i;
        dc6_dhi = (dn_dhi * den - num * dd_dhi) * idd;
        dc6_dhj = (dn_dhj * den - num * dd_dhj) * idd;
      } else {
        /* h reaches C6 through the polarisabilities only, c through C6_i */
        dc6_dhi = (2.0 * c6i * c6j * aj * ai0 * den - num * 2.0 * ai * ai0 * c6j) * idd;
        dc6_dhj = (2.0 * c6i * c6j * aj0 * ai * den - num * 2.0 * aj * aj0 * c6i) * idd;
        dc6_dci = (2.0 * ci0 * c6j * aj * ai * den - num * aj * aj * ci0) * idd;
        dc6_dcj = (2.0 * c6i * cj0 * aj * ai * den - num * ai * ai * cj0) * idd;
      }
      const double b0 = -0.00433008, b1 = 0.24428889, b2 = 0.04125273, b3 = -0.00078893;
      const double a7 = pow(alpha, 1.0 / 7.0);
      const double rvdw = pow(m->s[ORC_S_LR_FINE], -4.0 / 21.0) * a7;
      const double sfit = b3 * rvdw * rvdw * rvdw + b2 * rvdw * rvdw + b1 * rvdw + b0;
      const double gam = 0.5 / (sfit * sfit);
      const double drvdw = rvdw / (7.0 * alpha);
      const double dsfit = (3.0 * b3 * rvdw * rvdw + 2.0 * b2 * rvdw + b1) * drvdw;
      const double dgam = -2.0 * gam * dsfit / sfit;
      const double c8 = 5.0 * c6 / gam, c10 = 245.0 * c6 / (8.0 * gam * gam);
      const double damp = m->s[ORC_S_LR_DISP_SCALE] * 2.0 * 2.54 * a7;
      const double ddamp = damp / (7.0 * alpha);
      const double ra = r / m->s[ORC_S_LR_BOHR];
      const double r2 = ra * ra, r4 = r2 * r2, r6 = r4 * r2, r8 = r4 * r4, r10 = r8 * r2;
      const double p2 = damp * damp, p4 = p2 * p2, p6 = p4 * p2, p8 = p4 * p4, p10 = p8 * p2;
      const double d6 = r6 + p6, d8 = r8 + p8, d10 = r10 + p10;
      const double qdo = -c6 / d6 - c8 / d8 - c10 / d10;
      const double rad_au = 6.0 * c6 * r4 * ra / (d6 * d6) + 8.0 * c8 * r6 * ra / (d8 * d8) +
                            10.0 * c10 * r8 * ra / (d10 * d10);
      const double dc8 = -c8 * dgam / gam, dc10 = -2.0 * c10 * dgam / gam;
      const double dd6 = 6.0 * p4 * damp * ddamp, dd8 = 8.0 * p6 * damp * ddamp,
                   dd10 = 10.0 * p8 * damp * ddamp;
      const double dqdo_da = c6 * dd6 / (d6 * d6) - dc8 / d8 + c8 * dd8 / (d8 * d8) - dc10 / d10 +
                             c10 * dd10 / (d10 * d10);
      const double dqdo_dc6 = -1.0 / d6 - (5.0 / gam) / d8 - (245.0 / (8.0 * gam * gam)) / d10;
      const double dpi = dqdo_dc6 * dc6_dhi + dqdo_da * 0.5 * ai0;
      const double dpj = dqdo_dc6 * dc6_dhj + dqdo_da * 0.5 * aj0;
      double dsw, ddsw;
      smooth_switch(r, m->s[ORC_S_LR_CUTON_DISP], cutoff, &dsw, &ddsw);
      const double hart = m->s[ORC_S_LR_HARTREE];
      o.e_disp = full * hart * qdo * dsw;
      radial += full * hart * (rad_au * dsw / m->s[ORC_S_LR_BOHR] + qdo * ddsw);
      o.dhi = full * hart * dsw * dpi;
      o.dhj = full * hart * dsw * dpj;
      o.dci = full * hart * dsw * dqdo_dc6 * dc6_dci;
      o.dcj = full * hart * dsw * dqdo_dc6 * dc6_dcj;
    }
  }
  o.radial = radial;
  return o;
}

/* CSR of edges grouped by a key array (counting sort, stable). */
static void build_csr(int64_t n, int64_t ne, const int64_t *key, int64_t *off, int64_t *idx) {
  for (int64_t i = 0; i <= n; ++i) off[i] = 0;
  for (int64_t e = 0; e < ne; ++e) off[key[e] + 1]++;
  for (int64_t i = 0; i < n; ++i) off[i + 1] += off[i];
  int64_t *fill = (int64_t *)malloc(sizeof(int64_t) * (size_t)(n + 1));
  memcpy(fill, off, sizeof(int64_t) * (size_t)(n + 1));
  for (int64_t e = 0; e < ne; ++e) idx[fill[key[e]]++] = e;
  free(fill);
}

void orc_rms_rows(int64_t rows, int64_t width, const double *x, double eps, double *y,
                  double *inv_rms) {
  for (int64_t i = 0; i < rows; ++i) {
    const double *xi = x + i * width;
    double ms = 0.0;
    for (int64_t c = 0; c < width; ++c) ms += xi[c] * xi[c];
    ms /= (double)width;
    const double r = 1.0 / sqrt(ms + eps);
    for (int64_t c = 0; c < width; ++c) y[i * width + c] = xi[c] * r;
    if (inv_rms) inv_rms[i] = r;
  }
}
/* d/dx of y = x * r(x), r = 1 / sqrt(mean(x^2) + eps), given gy and y:
 * r (gy - y mean(gy y)) */
static void rms_rows_bwd(int width, const double *gy, const double *y, double r, double *gx) {
  double m = 0.0;
  for (int c = 0; c < width; ++c) m += gy[c] * y[c];
  m /= (double)width;
  for (int c = 0; c < width; ++c) gx[c] = r * (gy[c] - y[c] * m);
}

/* The normalisation of one node row (kokkos_post_attention_block0.cpp:97-162):
 * affine LayerNorm with biased variance, RMSNorm without scale (xhat = y),
 * or none (xhat = y = x, is = 1). */
static void layer_norm(int mode, int F, const double *x, const double *w, const double *b, double eps,
                       double *y, double *xhat, double *inv_sigma) {
  if (mode == ORC_NORM_NONE) {
    *inv_sigma = 1.0;
    for (int c = 0; c < F; ++c) { xhat[c] = x[c]; y[c] = x[c]; }
    return;
  }
  if (mode == ORC_NORM_RMS) {
    orc_rms_rows(1, F, x, eps, xhat, inv_sigma);
    for (int c = 0; c < F; ++c) y[c] = xhat[c];
    return;
  }
  double mean = 0.0;
  for (int c = 0; c < F; ++c) mean += x[c];
  mean /= F;
  double var = 0.0;
  for (int c = 0; c < F; ++c) { const double d = x[c] - mean; var += d * d; }
  var /= F;
  const double is = 1.0 / sqrt(var + eps);
  *inv_sigma = is;
  for (int c = 0; c < F; ++c) { xhat[c] = (x[c] - mean) * is; y[c] = xhat[c] * w[c] + b[c]; }
}
/* gx = dL/dx given gy, for the normalisation above */
static void layer_norm_bwd(int mode, int F, const double *gy, const double *w, const double *xhat, double is,
                           double *gx) {
  if (mode == ORC_NORM_NONE) {
    for (int c = 0; c < F; ++c) gx[c] = gy[c];
    return;
  }
  if (mode == ORC_NORM_RMS) {
    rms_rows_bwd(F, gy, xhat, is, gx);
    return;
  }
  double mg = 0.0, mgx = 0.0;
  double gh[ORC_MAXF];
  for (int c = 0; c < F; ++c) { gh[c] = gy[c] * w[c]; mg += gh[c]; mgx += gh[c] * xhat[c]; }
  mg /= F; mgx /= F;
  for (int c = 0; c < F; ++c) gx[c] = is * (gh[c] - mg - xhat[c] * mgx);
}

/* per-block saved state for the reverse pass */
typedef struct {
  double *x_in, *ev_in;           /* n*F, n*E  block inputs */
  double *qkv;                    /* n*5F: q k v qe ke (q, k, qe, ke RMS-normalised per
                                     head with the QK normalisation) */
  double *qkis;                   /* n*4*NH: their 1/rms per (row, head), QK normalisation */
  double *s;                      /* ne*NH edge invariants, one per degree slot */
  double *finv, *fev;             /* ne*F filters */
  double *ainv_alpha, *aev_alpha; /* ne*NH */
  double *a_ev;                   /* n*E  ev + d_ev */
  double *n1, *n1hat, *n1is;      /* LN1 */
  double *hpre;                   /* n*F  MLP hidden preact */
  double *tout;                   /* n*NI interaction output (with bias) */
  double *pre2hat, *pre2is;       /* LN2 */
} block_state;

#define ALLOC(ptr, count) do { (ptr) = (double *)calloc((size_t)(count), sizeof(double)); if (!(ptr)) goto fail; } while (0)

int orc_evaluate(const orc_model *m, int64_t n, const int64_t *z,
                 const double *emb_offset, int64_t n_images,
                 const int64_t *image, const double *image_charge,
                 int64_t ne, const int64_t *snd, const int64_t *rcv,
                 const double *vec, int64_t np, const int64_t *pi,
                 const int64_t *pj, const double *pvec, orc_out *out) {
  int status = 1;
  if (n <= 0 || ne < 0 || np < 0) return 2;
  for (int64_t i = 0; i < n; ++i)
    if (z[i] < 1 || z[i] > 99) return 3;
  for (int64_t e = 0; e < ne; ++e)
    if (snd[e] < 0 || snd[e] >= n || rcv[e] < 0 || rcv[e] >= n) return 4;
  for (int64_t p = 0; p < np; ++p)
    if (pi[p] < 0 || pi[p] >= n || pj[p] < 0 || pj[p] >= n) return 4;
  if (n_images <= 0) return 5;
  dims_t D;
  if (model_dims(m, &D) != 0) return 7;
  /* ev heads are the degree slots: NH of each */
  const int F = D.F, NH = D.NH, E = D.E, R = D.R, NI = D.NI, FH = D.FH, HK = D.HK;

  const double gamma = m->s[ORC_S_GAMMA], rmax = m->s[ORC_S_RMAX];
  const double avg = m->s[ORC_S_AVG_NN], emb_scale = m->s[ORC_S_EMB_SCALE];
  const double eps = m->s[ORC_S_LN_EPS];
  const int L = m->n_blocks > 0 ? (int)m->n_blocks : 3;
  if (L > ORC_MAXL) return 6;
  const int has_c6 = m->t[ORC_C6_W1] != NULL;

  double *r = NULL, *Y = NULL, *fc = NULL, *rbf = NULL, *zbl_e = NULL, *zbl_g = NULL;
  double *x = NULL, *ev = NULL, *dinv = NULL, *dev = NULL;
  double *gx = NULL, *gev = NULL, *gr = NULL, *gY = NULL, *ge = NULL;
  double *he_pre = NULL, *hq_pre = NULL, *hh_pre = NULL, *hkey = NULL, *heff = NULL;
  double *eatom = NULL, *qraw = NULL, *q = NULL, *hir = NULL;
  double *x_emb = NULL, *c6_pre = NULL, *c6_key = NULL, *c6_eff = NULL, *c6r = NULL, *lr_dc = NULL;
  double *lr_e = NULL, *lr_dq = NULL, *lr_dh = NULL, *lr_f = NULL, *lr_pf = NULL;
  double *sr_f = NULL, *gqkv = NULL, *gfinv = NULL, *gfev = NULL, *gfc = NULL;
  double *img_sum = NULL, *img_cnt = NULL, *img_seed = NULL;
  csum_t elec_total = {0, 0}, disp_total = {0, 0};
  double *gs = NULL, *gainv = NULL, *gaev = NULL;
  int64_t *roff = NULL, *ridx = NULL, *soff = NULL, *sidx = NULL;
  lr_pair_t *lrp = NULL;
  block_state bs[ORC_MAXL];
  memset(bs, 0, sizeof(bs));

  ALLOC(r, ne); ALLOC(Y, ne * E); ALLOC(fc, ne); ALLOC(rbf, ne * R);
  ALLOC(zbl_e, ne); ALLOC(zbl_g, ne);
  ALLOC(x, n * F); ALLOC(ev, n * E); ALLOC(dinv, n * F); ALLOC(dev, n * E);
  roff = (int64_t *)malloc(sizeof(int64_t) * (size_t)(n + 1));
  soff = (int64_t *)malloc(sizeof(int64_t) * (size_t)(n + 1));
  ridx = (int64_t *)malloc(sizeof(int64_t) * (size_t)(ne > 0 ? ne : 1));
  sidx = (int64_t *)malloc(sizeof(int64_t) * (size_t)(ne > 0 ? ne : 1));
  if (!roff || !soff || !ridx || !sidx) goto fail;
  build_csr(n, ne, rcv, roff, ridx);
  build_csr(n, ne, snd, soff, sidx);

  /* ---- geometry + radial basis + ZBL per directed edge ---- */
  const int64_t *kk = m->rbf_k, *kr = m->rbf_krev;
  const double *bb = m->t[ORC_RBF_B];
#pragma omp parallel for schedule(static)
  for (int64_t e = 0; e < ne; ++e) {
    const double vx = vec[3 * e], vy = vec[3 * e + 1], vz = vec[3 * e + 2];
    const double rr = sqrt(vx * vx + vy * vy + vz * vz);
    r[e] = rr;
    const double inv = rr > 1e-14 ? 1.0 / rr : 0.0;
    double ysh[24];
    orc_spherical_harmonics(vx * inv, vy * inv, vz * inv, ysh);
    for (int c = 0; c < E; ++c) Y[E * e + c] = ysh[D.sh[c]];
    if (rr < rmax) {
      const double t = rr / rmax, t3 = t * t * t;
      fc[e] = 1.0 - 10.0 * t3 + 15.0 * t3 * t - 6.0 * t3 * t * t;
    } else {
      fc[e] = 0.0;
    }
    double xb = exp(-gamma * rr);
    if (xb < 1e-6) xb = 1e-6;
    if (xb > 1.0 - 1e-6) xb = 1.0 - 1e-6;
    const double lx = log(xb), l1x = log(1.0 - xb);
    for (int k = 0; k < R; ++k) rbf[e * R + k] = exp(bb[k] + (double)kk[k] * lx + (double)kr[k] * l1x);
    zbl_edge(m, (double)z[rcv[e]], (double)z[snd[e]], rr, &zbl_e[e], &zbl_g[e]);
  }

  /* ---- embedding: x0 = (W[:, Z-1] + offset) / scale, ev0 = 0 ---- */
  for (int64_t i = 0; i < n; ++i)
    for (int c = 0; c < F; ++c)
      x[i * F + c] = (m->t[ORC_EMB_W][c * 118 + (z[i] - 1)] + (emb_offset ? emb_offset[i * F + c] : 0.0)) / emb_scale;
  if (m->resid) {
    ALLOC(x_emb, n * F);
    memcpy(x_emb, x, sizeof(double) * (size_t)(n * F));
  }

  /* ---- interaction blocks, forward ---- */
  for (int b = 0; b < L; ++b) {
    const double *const *T = m->t + ORC_NGLOBAL + b * ORC_NBLOCK;
    block_state *S = &bs[b];
    ALLOC(S->x_in, n * F); ALLOC(S->ev_in, n * E); ALLOC(S->qkv, n * 5 * F); ALLOC(S->qkis, n * 4 * NH);
    ALLOC(S->s, ne * NH); ALLOC(S->finv, ne * F); ALLOC(S->fev, ne * F);
    ALLOC(S->ainv_alpha, ne * NH); ALLOC(S->aev_alpha, ne * NH); ALLOC(S->a_ev, n * E);
    ALLOC(S->n1, n * F); ALLOC(S->n1hat, n * F); ALLOC(S->n1is, n); ALLOC(S->hpre, n * F);
    ALLOC(S->tout, n * NI); ALLOC(S->pre2hat, n * F); ALLOC(S->pre2is, n);
    /* residual scalars (kokkos_local_energy_reverse.cpp:143-158): the block
     * input is resid[b] x + x0[b] x_emb, x the previous block's output (the
     * embedding itself for block 0) */
    if (m->resid)
      for (int64_t k = 0; k < n * F; ++k) x[k] = m->resid[b] * x[k] + m->x0l[b] * x_emb[k];
    memcpy(S->x_in, x, sizeof(double) * (size_t)(n * F));
    memcpy(S->ev_in, ev, sizeof(double) * (size_t)(n * E));
    const double *acg = T[ORC_B_ATT_CG], *icg = T[ORC_B_INT_CG];

    /* edge invariants + both filters (kokkos_integrated_block0.cpp:166-255) */
#pragma omp parallel for schedule(static)
    for (int64_t e = 0; e < ne; ++e) {
      double sv[ORC_MAXS] = {0};
      for (int c = 0; c < E; ++c) {
        const double d = ev[snd[e] * E + c] - ev[rcv[e] * E + c];
        sv[D.slot_of[c]] += d * d * acg[c];
      }
      for (int l = 0; l < NH; ++l) S->s[e * NH + l] = sv[l];
      for (int which = 0; which < 2; ++which) {
        const int base = which == 0 ? ORC_B_FI_RW0 : ORC_B_FE_RW0;
        double h[ORC_MAXF], h2[ORC_MAXF / 4], t1[ORC_MAXF], t2[ORC_MAXF];
        matvec(T[base + 0], T[base + 1], F, R, rbf + e * R, h);
        for (int c = 0; c < F; ++c) h[c] = silu(h[c]);
        matvec(T[base + 2], T[base + 3], F, F, h, t1);
        matvec(T[base + 4], T[base + 5], FH, NH, sv, h2);
        for (int c = 0; c < FH; ++c) h2[c] = silu(h2[c]);
        matvec(T[base + 6], T[base + 7], F, FH, h2, t2);
        double *dst = which == 0 ? S->finv + e * F : S->fev + e * F;
        for (int c = 0; c < F; ++c) dst[c] = t1[c] + t2[c];
      }
    }
    /* Q, K, V, Q_ev, K_ev: per-head x_h @ W[h], W stored (head, in, out) */
    const int wid[5] = {ORC_B_WQ, ORC_B_WK, ORC_B_WV, ORC_B_WQE, ORC_B_WKE};
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i)
      for (int w = 0; w < 5; ++w)
        for (int h = 0; h < NH; ++h)
          for (int o = 0; o < HW; ++o) {
            double s = 0.0;
            for (int k = 0; k < HW; ++k) s += x[i * F + h * HW + k] * T[wid[w]][(h * HW + k) * HW + o];
            S->qkv[i * 5 * F + w * F + h * HW + o] = s;
          }
    /* QK normalisation per (node, head) row of q, k, q_ev, k_ev, eps 1e-6
     * (kokkos_integrated_block0.cpp:288-328); v is left as it is */
    if (m->qk_norm) {
      const int rows[4] = {0, 1, 3, 4};
#pragma omp parallel for schedule(static)
      for (int64_t i = 0; i < n; ++i)
        for (int k = 0; k < 4; ++k)
          for (int h = 0; h < NH; ++h) {
            double *row = S->qkv + i * 5 * F + rows[k] * F + h * HW;
            orc_rms_rows(1, HW, row, 1e-6, row, S->qkis + (i * 4 + k) * NH + h);
          }
    }
    /* attention coefficients per (edge, head) */
#pragma omp parallel for schedule(static)
    for (int64_t e = 0; e < ne; ++e) {
      const double *qr = S->qkv + rcv[e] * 5 * F, *ks = S->qkv + snd[e] * 5 * F;
      for (int h = 0; h < NH; ++h) {
        double ai = 0.0, ae = 0.0;
        for (int c = h * HW; c < (h + 1) * HW; ++c) {
          ai += qr[c] * ks[F + c] * S->finv[e * F + c];
          ae += qr[3 * F + c] * ks[4 * F + c] * S->fev[e * F + c];
        }
        S->ainv_alpha[e * NH + h] = ai / avg;
        S->aev_alpha[e * NH + h] = ae / avg;
      }
    }
    /* receiver-side scatter, as a gather over the receiver CSR */
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
      double di[ORC_MAXF] = {0}, de[ORC_MAXE] = {0};
      for (int64_t k = roff[i]; k < roff[i + 1]; ++k) {
        const int64_t e = ridx[k];
        const double *vs = S->qkv + snd[e] * 5 * F + 2 * F;
        for (int c = 0; c < F; ++c) di[c] += fc[e] * S->ainv_alpha[e * NH + c / HW] * vs[c];
        for (int c = 0; c < E; ++c) de[c] += fc[e] * S->aev_alpha[e * NH + D.slot_of[c]] * Y[e * E + c];
      }
      memcpy(dinv + i * F, di, sizeof(double) * (size_t)F);
      memcpy(dev + i * E, de, sizeof(double) * (size_t)E);
    }
    /* post-attention (kokkos_post_attention_block0.cpp:165-300) */
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
      double ainv[ORC_MAXF], act[ORC_MAXF], hid[ORC_MAXF], mlp[ORC_MAXF], p[ORC_MAXF];
      double cat[ORC_MAXF + ORC_MAXS], pre2[ORC_MAXF], y2[ORC_MAXF];
      for (int c = 0; c < F; ++c) ainv[c] = x[i * F + c] + dinv[i * F + c];
      for (int c = 0; c < E; ++c) S->a_ev[i * E + c] = ev[i * E + c] + dev[i * E + c];
      layer_norm((int)m->norm1, F, ainv, T[ORC_B_LN1_W], T[ORC_B_LN1_B], eps, S->n1 + i * F, S->n1hat + i * F,
                 &S->n1is[i]);
      const double *n1 = S->n1 + i * F;
      for (int c = 0; c < F; ++c) act[c] = silu(n1[c]);
      matvec(T[ORC_B_M1_W], T[ORC_B_M1_B], F, F, act, S->hpre + i * F);
      for (int c = 0; c < F; ++c) hid[c] = silu(S->hpre[i * F + c]);
      matvec(T[ORC_B_M2_W], T[ORC_B_M2_B], F, F, hid, mlp);
      for (int c = 0; c < F; ++c) p[c] = n1[c] + mlp[c];
      for (int c = 0; c < F; ++c) cat[c] = p[c];
      for (int l = 0; l < NH; ++l) cat[F + l] = 0.0;
      for (int c = 0; c < E; ++c) cat[F + D.slot_of[c]] += S->a_ev[i * E + c] * S->a_ev[i * E + c] * icg[c];
      matvec(T[ORC_B_INT_W], T[ORC_B_INT_B], NI, NI, cat, S->tout + i * NI);
      const double *t = S->tout + i * NI;
      for (int c = 0; c < F; ++c) pre2[c] = p[c] + t[c];
      for (int c = 0; c < E; ++c) ev[i * E + c] = S->a_ev[i * E + c] * (1.0 + t[F + D.slot_of[c]]);
      layer_norm((int)m->norm2, F, pre2, T[ORC_B_LN2_W], T[ORC_B_LN2_B], eps, y2, S->pre2hat + i * F, &S->pre2is[i]);
      memcpy(x + i * F, y2, sizeof(double) * (size_t)F);
    }
  }

  /* ---- output heads (kokkos_output_heads.cpp:137-176,341-451) ---- */
  ALLOC(he_pre, n * HK); ALLOC(hq_pre, n * HK); ALLOC(hh_pre, n * HH); ALLOC(hkey, n * HH);
  ALLOC(heff, n); ALLOC(eatom, n); ALLOC(qraw, n); ALLOC(q, n); ALLOC(hir, n);
  if (has_c6) { ALLOC(c6_pre, n * HH); ALLOC(c6_key, n * HH); ALLOC(c6_eff, n); ALLOC(c6r, n); }
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    double t[ORC_MAXK], hh[HH];
    const int64_t zi = z[i];
    matvec(m->t[ORC_E_W1], m->t[ORC_E_B1], HK, F, x + i * F, he_pre + i * HK);
    for (int c = 0; c < HK; ++c) t[c] = silu(he_pre[i * HK + c]);
    double er = 0.0;
    for (int c = 0; c < HK; ++c) er += m->t[ORC_E_W2][c] * t[c];
    eatom[i] = (er + m->t[ORC_E_B2][0]) * m->t[ORC_E_SCALE][zi - 1] + m->t[ORC_E_SHIFT][zi - 1];
    matvec(m->t[ORC_Q_W1], m->t[ORC_Q_B1], HK, F, x + i * F, hq_pre + i * HK);
    for (int c = 0; c < HK; ++c) t[c] = silu(hq_pre[i * HK + c]);
    double qr = 0.0;
    for (int c = 0; c < HK; ++c) qr += m->t[ORC_Q_W2][c] * t[c];
    qraw[i] = qr + m->t[ORC_Q_B2][0] + m->t[ORC_Q_EMB][zi];
    matvec(m->t[ORC_H_W1], m->t[ORC_H_B1], HH, F, x + i * F, hh_pre + i * HH);
    for (int c = 0; c < HH; ++c) hh[c] = silu(hh_pre[i * HH + c]);
    matvec(m->t[ORC_H_W2], m->t[ORC_H_B2], HH, HH, hh, hkey + i * HH);
    double qk = 0.0;
    for (int c = 0; c < HH; ++c) qk += m->t[ORC_H_QEMB][zi * HH + c] * hkey[i * HH + c];
    heff[i] = m->t[ORC_H_VSHIFT][zi] + qk / sqrt((double)HH);
    hir[i] = fabs(heff[i]);
    if (has_c6) {
      /* the C6 ratio head: a second ratio head of the Hirshfeld form
       * (kokkos_output_heads.cpp:108-180) */
      matvec(m->t[ORC_C6_W1], m->t[ORC_C6_B1], HH, F, x + i * F, c6_pre + i * HH);
      for (int c = 0; c < HH; ++c) hh[c] = silu(c6_pre[i * HH + c]);
      matvec(m->t[ORC_C6_W2], m->t[ORC_C6_B2], HH, HH, hh, c6_key + i * HH);
      double ck = 0.0;
      for (int c = 0; c < HH; ++c) ck += m->t[ORC_C6_QEMB][zi * HH + c] * c6_key[i * HH + c];
      c6_eff[i] = m->t[ORC_C6_VSHIFT][zi] + ck / sqrt((double)HH);
      c6r[i] = fabs(c6_eff[i]);
    }
  }
  /* per-image charge conservation (kokkos_image_segments.cpp) */
  ALLOC(img_sum, n_images); ALLOC(img_cnt, n_images); ALLOC(img_seed, n_images);
  for (int64_t i = 0; i < n; ++i) {
    const int64_t im = image ? image[i] : 0;
    img_sum[im] += qraw[i];
    img_cnt[im] += 1.0;
  }
  for (int64_t i = 0; i < n; ++i) {
    const int64_t im = image ? image[i] : 0;
    const double Qi = image_charge ? image_charge[im] : 0.0;
    q[i] = qraw[i] + (Qi - img_sum[im]) / img_cnt[im];
  }

  /* ---- long range per unique half pair ---- */
  ALLOC(lr_e, n); ALLOC(lr_dq, n); ALLOC(lr_dh, n); ALLOC(lr_dc, n); ALLOC(lr_f, n * 3); ALLOC(lr_pf, (np > 0 ? np : 1) * 3);
  lrp = (lr_pair_t *)calloc((size_t)(np > 0 ? np : 1), sizeof(lr_pair_t));
  if (!lrp) goto fail;
#pragma omp parallel for schedule(static)
  for (int64_t p = 0; p < np; ++p) {
    const int64_t i = pi[p], j = pj[p];
    if (i == j) continue;
    const double dx = pvec[3 * p], dy = pvec[3 * p + 1], dz = pvec[3 * p + 2];
    const double rr = sqrt(dx * dx + dy * dy + dz * dz);
    lrp[p] = lr_pair(m, z[i], z[j], q[i], q[j], hir[i], hir[j], has_c6, has_c6 ? c6r[i] : 0.0,
                     has_c6 ? c6r[j] : 0.0, rr);
    if (lrp[p].valid) {
      const double inv = 1.0 / rr;
      lr_pf[3 * p] = lrp[p].radial * dx * inv;
      lr_pf[3 * p + 1] = lrp[p].radial * dy * inv;
      lr_pf[3 * p + 2] = lrp[p].radial * dz * inv;
    }
  }
  for (int64_t p = 0; p < np; ++p) {
    if (!lrp[p].valid) continue;
    const int64_t i = pi[p], j = pj[p];
    const double pe = lrp[p].e_elec + lrp[p].e_disp;
    sum_add(&elec_total, lrp[p].e_elec); sum_add(&disp_total, lrp[p].e_disp);
    lr_e[i] += 0.5 * pe; lr_e[j] += 0.5 * pe;
    lr_dq[i] += lrp[p].charge_pref * q[j]; lr_dq[j] += lrp[p].charge_pref * q[i];
    lr_dh[i] += lrp[p].dhi; lr_dh[j] += lrp[p].dhj;
    lr_dc[i] += lrp[p].dci; lr_dc[j] += lrp[p].dcj;
    for (int a = 0; a < 3; ++a) { lr_f[3 * i + a] += lr_pf[3 * p + a]; lr_f[3 * j + a] -= lr_pf[3 * p + a]; }
  }

  /* ---- seeds: energy 1, charge dE/dq - image mean, Hirshfeld dE/dh ---- */
  for (int64_t i = 0; i < n; ++i) img_seed[image ? image[i] : 0] += lr_dq[i];
  ALLOC(gx, n * F); ALLOC(gev, n * E);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    const int64_t zi = z[i];
    const int64_t im = image ? image[i] : 0;
    double gh[ORC_MAXK], ghh[HH], gk[HH];
    double *g = gx + i * F;
    memset(g, 0, sizeof(double) * F);
    for (int c = 0; c < HK; ++c)
      gh[c] = m->t[ORC_E_SCALE][zi - 1] * m->t[ORC_E_W2][c] * silu_prime(he_pre[i * HK + c]);
    matvecT_acc(m->t[ORC_E_W1], HK, F, gh, g);
    const double qseed = lr_dq[i] - img_seed[im] / img_cnt[im];
    for (int c = 0; c < HK; ++c) gh[c] = qseed * m->t[ORC_Q_W2][c] * silu_prime(hq_pre[i * HK + c]);
    matvecT_acc(m->t[ORC_Q_W1], HK, F, gh, g);
    const double sg = heff[i] > 0.0 ? 1.0 : (heff[i] < 0.0 ? -1.0 : 0.0);
    const double hs = lr_dh[i] * sg / sqrt((double)HH);
    for (int c = 0; c < HH; ++c) gk[c] = hs * m->t[ORC_H_QEMB][zi * HH + c];
    memset(ghh, 0, sizeof(ghh));
    matvecT_acc(m->t[ORC_H_W2], HH, HH, gk, ghh);
    for (int c = 0; c < HH; ++c) ghh[c] *= silu_prime(hh_pre[i * HH + c]);
    matvecT_acc(m->t[ORC_H_W1], HH, F, ghh, g);
    if (has_c6) {
      const double sc = c6_eff[i] > 0.0 ? 1.0 : (c6_eff[i] < 0.0 ? -1.0 : 0.0);
      const double cs = lr_dc[i] * sc / sqrt((double)HH);
      for (int c = 0; c < HH; ++c) gk[c] = cs * m->t[ORC_C6_QEMB][zi * HH + c];
      memset(ghh, 0, sizeof(ghh));
      matvecT_acc(m->t[ORC_C6_W2], HH, HH, gk, ghh);
      for (int c = 0; c < HH; ++c) ghh[c] *= silu_prime(c6_pre[i * HH + c]);
      matvecT_acc(m->t[ORC_C6_W1], HH, F, ghh, g);
    }
  }

  /* ---- interaction blocks, reverse ---- */
  ALLOC(gr, ne); ALLOC(gY, ne * E); ALLOC(gqkv, n * 5 * F); ALLOC(gfinv, ne * F);
  ALLOC(gfev, ne * F); ALLOC(gfc, ne); ALLOC(gs, ne * NH); ALLOC(gainv, n * F); ALLOC(gaev, n * E);
  for (int b = L - 1; b >= 0; --b) {
    const double *const *T = m->t + ORC_NGLOBAL + b * ORC_NBLOCK;
    block_state *S = &bs[b];
    const double *acg = T[ORC_B_ATT_CG], *icg = T[ORC_B_INT_CG];
    /* post-attention reverse (kokkos_post_attention_reverse.cpp) */
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
      double gpre2[ORC_MAXF], gt[ORC_MAXF + ORC_MAXS], gcat[ORC_MAXF + ORC_MAXS], gp[ORC_MAXF];
      double ghid[ORC_MAXF], gact[ORC_MAXF], gn1[ORC_MAXF];
      const double *t = S->tout + i * NI, *aev = S->a_ev + i * E;
      layer_norm_bwd((int)m->norm2, F, gx + i * F, T[ORC_B_LN2_W], S->pre2hat + i * F, S->pre2is[i], gpre2);
      for (int c = 0; c < F; ++c) { gt[c] = gpre2[c]; gp[c] = gpre2[c]; }
      for (int l = 0; l < NH; ++l) gt[F + l] = 0.0;
      double *ga = gaev + i * E;
      for (int c = 0; c < E; ++c) {
        gt[F + D.slot_of[c]] += gev[i * E + c] * aev[c];
        ga[c] = gev[i * E + c] * (1.0 + t[F + D.slot_of[c]]);
      }
      memset(gcat, 0, sizeof(double) * (size_t)NI);
      matvecT_acc(T[ORC_B_INT_W], NI, NI, gt, gcat);
      for (int c = 0; c < F; ++c) gp[c] += gcat[c];
      for (int c = 0; c < E; ++c) ga[c] += gcat[F + D.slot_of[c]] * 2.0 * aev[c] * icg[c];
      /* p = n1 + W2 silu(hpre) + b2,  hpre = W1 silu(n1) + b1 */
      memset(ghid, 0, sizeof(double) * (size_t)F);
      matvecT_acc(T[ORC_B_M2_W], F, F, gp, ghid);
      for (int c = 0; c < F; ++c) ghid[c] *= silu_prime(S->hpre[i * F + c]);
      memset(gact, 0, sizeof(double) * (size_t)F);
      matvecT_acc(T[ORC_B_M1_W], F, F, ghid, gact);
      for (int c = 0; c < F; ++c) gn1[c] = gp[c] + gact[c] * silu_prime(S->n1[i * F + c]);
      layer_norm_bwd((int)m->norm1, F, gn1, T[ORC_B_LN1_W], S->n1hat + i * F, S->n1is[i], gainv + i * F);
    }
    /* attention reverse per edge (kokkos_attention_scatter_reverse.cpp:280-500) */
#pragma omp parallel for schedule(static)
    for (int64_t e = 0; e < ne; ++e) {
      const int64_t ri = rcv[e], si = snd[e];
      const double *qr = S->qkv + ri * 5 * F, *ks = S->qkv + si * 5 * F;
      const double *gdi = gainv + ri * F, *gde = gaev + ri * E;
      double dfc = 0.0;
      for (int h = 0; h < NH; ++h) {
        double dai = 0.0, dae = 0.0, ci = 0.0, ce = 0.0;
        for (int c = h * HW; c < (h + 1) * HW; ++c) {
          dai += gdi[c] * fc[e] * ks[2 * F + c];
          ci += gdi[c] * ks[2 * F + c];
        }
        for (int c = D.off[h]; c < D.off[h + 1]; ++c) {
          dae += gde[c] * fc[e] * Y[e * E + c];
          ce += gde[c] * Y[e * E + c];
          gY[e * E + c] += gde[c] * fc[e] * S->aev_alpha[e * NH + h];
        }
        dfc += ci * S->ainv_alpha[e * NH + h] + ce * S->aev_alpha[e * NH + h];
        const double si_ = dai / avg, se_ = dae / avg;
        for (int c = h * HW; c < (h + 1) * HW; ++c) {
          gfinv[e * F + c] = si_ * qr[c] * ks[F + c];
          gfev[e * F + c] = se_ * qr[3 * F + c] * ks[4 * F + c];
        }
      }
      gfc[e] = dfc;
    }
    /* node gathers: dq at receivers, dk / dv at senders */
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
      double *g = gqkv + i * 5 * F;
      memset(g, 0, sizeof(double) * 5 * F);
      const double *qi = S->qkv + i * 5 * F;
      for (int64_t k = roff[i]; k < roff[i + 1]; ++k) {
        const int64_t e = ridx[k];
        const double *ks = S->qkv + snd[e] * 5 * F;
        const double *gdi = gainv + i * F, *gde = gaev + i * E;
        for (int h = 0; h < NH; ++h) {
          double dai = 0.0, dae = 0.0;
          for (int c = h * HW; c < (h + 1) * HW; ++c) dai += gdi[c] * fc[e] * ks[2 * F + c];
          for (int c = D.off[h]; c < D.off[h + 1]; ++c) dae += gde[c] * fc[e] * Y[e * E + c];
          for (int c = h * HW; c < (h + 1) * HW; ++c) {
            g[c] += dai / avg * ks[F + c] * S->finv[e * F + c];
            g[3 * F + c] += dae / avg * ks[4 * F + c] * S->fev[e * F + c];
          }
        }
      }
      for (int64_t k = soff[i]; k < soff[i + 1]; ++k) {
        const int64_t e = sidx[k];
        const double *qr = S->qkv + rcv[e] * 5 * F;
        const double *gdi = gainv + rcv[e] * F, *gde = gaev + rcv[e] * E;
        for (int h = 0; h < NH; ++h) {
          double dai = 0.0, dae = 0.0;
          for (int c = h * HW; c < (h + 1) * HW; ++c) dai += gdi[c] * fc[e] * qi[2 * F + c];
          for (int c = D.off[h]; c < D.off[h + 1]; ++c) dae += gde[c] * fc[e] * Y[e * E + c];
          for (int c = h * HW; c < (h + 1) * HW; ++c) {
            g[F + c] += dai / avg * qr[c] * S->finv[e * F + c];
            g[2 * F + c] += fc[e] * S->ainv_alpha[e * NH + h] * gdi[c];
            g[4 * F + c] += dae / avg * qr[3 * F + c] * S->fev[e * F + c];
          }
        }
      }
    }
    /* filter dgrad per edge (kokkos_block2_attention_input_reverse.cpp:198-240,301-336) */
#pragma omp parallel for schedule(static)
    for (int64_t e = 0; e < ne; ++e) {
      double grbf[ORC_MAXR] = {0}, gsv[ORC_MAXS] = {0};
      for (int which = 0; which < 2; ++which) {
        const int base = which == 0 ? ORC_B_FI_RW0 : ORC_B_FE_RW0;
        const double *gf = which == 0 ? gfinv + e * F : gfev + e * F;
        double pre[ORC_MAXF], gh[ORC_MAXF], pre2[ORC_MAXF / 4], gh2[ORC_MAXF / 4];
        matvec(T[base + 0], T[base + 1], F, R, rbf + e * R, pre);
        memset(gh, 0, sizeof(double) * (size_t)F);
        matvecT_acc(T[base + 2], F, F, gf, gh);
        for (int c = 0; c < F; ++c) gh[c] *= silu_prime(pre[c]);
        matvecT_acc(T[base + 0], F, R, gh, grbf);
        matvec(T[base + 4], T[base + 5], FH, NH, S->s + e * NH, pre2);
        memset(gh2, 0, sizeof(double) * (size_t)FH);
        matvecT_acc(T[base + 6], F, FH, gf, gh2);
        for (int c = 0; c < FH; ++c) gh2[c] *= silu_prime(pre2[c]);
        matvecT_acc(T[base + 4], FH, NH, gh2, gsv);
      }
      for (int l = 0; l < NH; ++l) gs[e * NH + l] = gsv[l];
      const double rr = r[e];
      double grad = 0.0;
      if (rr < rmax) {
        const double t = rr / rmax;
        grad += gfc[e] * (-30.0 * t * t * (1.0 - t) * (1.0 - t) / rmax);
      }
      const double xb = exp(-gamma * rr);
      if (xb > 1e-6 && xb < 1.0 - 1e-6)
        for (int k = 0; k < R; ++k)
          grad += grbf[k] * rbf[e * R + k] * (-gamma * (double)kk[k] + gamma * (double)kr[k] * xb / (1.0 - xb));
      gr[e] += grad;
    }
    /* node input adjoints: residual + QKV dgrad + edge-invariant adjoint */
    const int wid[5] = {ORC_B_WQ, ORC_B_WK, ORC_B_WV, ORC_B_WQE, ORC_B_WKE};
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
      double *g = gx + i * F;
      for (int c = 0; c < F; ++c) g[c] = gainv[i * F + c];
      if (m->qk_norm) {
        /* through the QK normalisation: the adjoints of the raw rows */
        const int rows[4] = {0, 1, 3, 4};
        for (int k = 0; k < 4; ++k)
          for (int h = 0; h < NH; ++h) {
            double *gr_ = gqkv + i * 5 * F + rows[k] * F + h * HW;
            double tmp[HW];
            rms_rows_bwd(HW, gr_, S->qkv + i * 5 * F + rows[k] * F + h * HW, S->qkis[(i * 4 + k) * NH + h], tmp);
            memcpy(gr_, tmp, sizeof(tmp));
          }
      }
      for (int w = 0; w < 5; ++w)
        for (int h = 0; h < NH; ++h)
          for (int k = 0; k < HW; ++k) {
            double s = 0.0;
            for (int o = 0; o < HW; ++o) s += T[wid[w]][(h * HW + k) * HW + o] * gqkv[i * 5 * F + w * F + h * HW + o];
            g[h * HW + k] += s;
          }
      double *ge_ = gev + i * E;
      for (int c = 0; c < E; ++c) ge_[c] = gaev[i * E + c];
      const double *evi = S->ev_in + i * E;
      for (int64_t k = soff[i]; k < soff[i + 1]; ++k) {
        const int64_t e = sidx[k];
        for (int c = 0; c < E; ++c)
          ge_[c] += gs[e * NH + D.slot_of[c]] * 2.0 * (evi[c] - S->ev_in[rcv[e] * E + c]) * acg[c];
      }
      for (int64_t k = roff[i]; k < roff[i + 1]; ++k) {
        const int64_t e = ridx[k];
        for (int c = 0; c < E; ++c)
          ge_[c] -= gs[e * NH + D.slot_of[c]] * 2.0 * (S->ev_in[snd[e] * E + c] - evi[c]) * acg[c];
      }
      /* residual scalars: d/d(previous output) = resid[b] d/d(input); the
       * embedding term does not depend on the positions */
      if (m->resid)
        for (int c = 0; c < F; ++c) g[c] *= m->resid[b];
    }
  }

  /* ---- geometry reverse (kokkos_learned_energy_forces.cpp:241-306) ---- */
  ALLOC(ge, ne * 3); ALLOC(sr_f, n * 3);
#pragma omp parallel for schedule(static)
  for (int64_t e = 0; e < ne; ++e) {
    const double vx = vec[3 * e], vy = vec[3 * e + 1], vz = vec[3 * e + 2];
    const double rr = r[e];
    if (rr <= 1e-14) { ge[3 * e] = ge[3 * e + 1] = ge[3 * e + 2] = 0.0; continue; }
    const double u[3] = {vx / rr, vy / rr, vz / rr};
    /* the feature channels' adjoints summed onto the unique harmonics they
     * replicate (kokkos_local_cartesian_forces.cpp) */
    double gu[3], gsh[24] = {0};
    for (int c = 0; c < E; ++c) gsh[D.sh[c]] += gY[e * E + c];
    sh_vjp(u[0], u[1], u[2], gsh, gu);
    const double radial = u[0] * gu[0] + u[1] * gu[1] + u[2] * gu[2];
    const double dr = gr[e] + zbl_g[e];
    for (int a = 0; a < 3; ++a) ge[3 * e + a] = dr * u[a] + (gu[a] - u[a] * radial) / rr;
  }
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    double f[3] = {0, 0, 0};
    for (int64_t k = soff[i]; k < soff[i + 1]; ++k)
      for (int a = 0; a < 3; ++a) f[a] += ge[3 * sidx[k] + a];
    for (int64_t k = roff[i]; k < roff[i + 1]; ++k)
      for (int a = 0; a < 3; ++a) f[a] -= ge[3 * ridx[k] + a];
    for (int a = 0; a < 3; ++a) sr_f[3 * i + a] = f[a];
  }

  /* ---- outputs ---- */
  /* W = -sum v (x) g over SR edges and LR pairs, symmetrised
   * (pair_so3lr_native_mpi.cpp:944-990), compensated */
  csum_t Wc[6] = {{0, 0}, {0, 0}, {0, 0}, {0, 0}, {0, 0}, {0, 0}};
  for (int64_t e = 0; e < ne; ++e) {
    const double *v = vec + 3 * e, *g = ge + 3 * e;
    sum_add(&Wc[0], -v[0] * g[0]); sum_add(&Wc[1], -v[1] * g[1]); sum_add(&Wc[2], -v[2] * g[2]);
    sum_add(&Wc[3], -0.5 * (v[0] * g[1] + v[1] * g[0]));
    sum_add(&Wc[4], -0.5 * (v[0] * g[2] + v[2] * g[0]));
    sum_add(&Wc[5], -0.5 * (v[1] * g[2] + v[2] * g[1]));
  }
  for (int64_t p = 0; p < np; ++p) {
    if (!lrp[p].valid) continue;
    const double *v = pvec + 3 * p, *g = lr_pf + 3 * p;
    sum_add(&Wc[0], -v[0] * g[0]); sum_add(&Wc[1], -v[1] * g[1]); sum_add(&Wc[2], -v[2] * g[2]);
    sum_add(&Wc[3], -0.5 * (v[0] * g[1] + v[1] * g[0]));
    sum_add(&Wc[4], -0.5 * (v[0] * g[2] + v[2] * g[0]));
    sum_add(&Wc[5], -0.5 * (v[1] * g[2] + v[2] * g[1]));
  }
  double W[6];
  for (int c = 0; c < 6; ++c) W[c] = sum_value(&Wc[c]);
  csum_t etot_c = {0, 0};
  for (int64_t i = 0; i < n; ++i) {
    double ez = 0.0;
    for (int64_t k = roff[i]; k < roff[i + 1]; ++k) ez += zbl_e[ridx[k]];
    const double ei = eatom[i] + ez + lr_e[i];
    sum_add(&etot_c, ei);
    if (out->e_learned) out->e_learned[i] = eatom[i];
    if (out->e_zbl) out->e_zbl[i] = ez;
    if (out->e_lr) out->e_lr[i] = lr_e[i];
    if (out->charges) out->charges[i] = q[i];
    if (out->hirshfeld) out->hirshfeld[i] = hir[i];
    if (out->c6_ratios && has_c6) out->c6_ratios[i] = c6r[i];
    if (out->forces)
      for (int a = 0; a < 3; ++a) out->forces[3 * i + a] = sr_f[3 * i + a] + lr_f[3 * i + a];
    if (out->image_energy) {
      if (i == 0) for (int64_t k = 0; k < n_images; ++k) out->image_energy[k] = 0.0;
      out->image_energy[image ? image[i] : 0] += ei;
    }
  }
  if (out->virial) memcpy(out->virial, W, sizeof(W));
  if (out->vatom) {
    /* the same terms as W, half to each endpoint of the edge or pair */
    memset(out->vatom, 0, sizeof(double) * 6 * (size_t)n);
    for (int64_t e = 0; e < ne; ++e) {
      const double *v = vec + 3 * e, *g = ge + 3 * e;
      const double w[6] = {-v[0] * g[0], -v[1] * g[1], -v[2] * g[2], -0.5 * (v[0] * g[1] + v[1] * g[0]),
                           -0.5 * (v[0] * g[2] + v[2] * g[0]), -0.5 * (v[1] * g[2] + v[2] * g[1])};
      for (int c = 0; c < 6; ++c) {
        out->vatom[6 * snd[e] + c] += 0.5 * w[c];
        out->vatom[6 * rcv[e] + c] += 0.5 * w[c];
      }
    }
    for (int64_t p = 0; p < np; ++p) {
      if (!lrp[p].valid) continue;
      const double *v = pvec + 3 * p, *g = lr_pf + 3 * p;
      const double w[6] = {-v[0] * g[0], -v[1] * g[1], -v[2] * g[2], -0.5 * (v[0] * g[1] + v[1] * g[0]),
                           -0.5 * (v[0] * g[2] + v[2] * g[0]), -0.5 * (v[1] * g[2] + v[2] * g[1])};
      for (int c = 0; c < 6; ++c) {
        out->vatom[6 * pi[p] + c] += 0.5 * w[c];
        out->vatom[6 * pj[p] + c] += 0.5 * w[c];
      }
    }
  }
  out->e_elec_total = sum_value(&elec_total);
  out->e_disp_total = sum_value(&disp_total);
  out->e_total = sum_value(&etot_c);
  status = 0;

fail:
  free(img_sum); free(img_cnt); free(img_seed);
  free(r); free(Y); free(fc); free(rbf); free(zbl_e); free(zbl_g);
  free(x); free(ev); free(dinv); free(dev); free(gx); free(gev); free(gr); free(gY); free(ge);
  free(he_pre); free(hq_pre); free(hh_pre); free(hkey); free(heff);
  free(eatom); free(qraw); free(q); free(hir);
  free(x_emb); free(c6_pre); free(c6_key); free(c6_eff); free(c6r); free(lr_dc);
  free(lr_e); free(lr_dq); free(lr_dh); free(lr_f); free(lr_pf); free(lrp);
  free(sr_f); free(gqkv); free(gfinv); free(gfev); free(gfc); free(gs); free(gainv); free(gaev);
  free(roff); free(ridx); free(soff); free(sidx);
  for (int b = 0; b < L; ++b) {
    block_state *S = &bs[b];
    free(S->x_in); free(S->ev_in); free(S->qkv); free(S->qkis); free(S->s); free(S->finv); free(S->fev);
    free(S->ainv_alpha); free(S->aev_alpha); free(S->a_ev); free(S->n1); free(S->n1hat);
    free(S->n1is); free(S->hpre); free(S->tout); free(S->pre2hat); free(S->pre2is);
  }
  return status;
}
