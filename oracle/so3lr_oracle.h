/*
 * CPU fp64 oracle for the SO3LR force evaluation -- TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of the reference algorithm (one directed edge
 * at a time, exactly as the reference pair style evaluates it) used to check
 * the HIP product path and, timed with OpenMP, as the CPU baseline.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it; the product library never links it.
 *
 * Reference files restated (paths under source/so3lr-lammps-native/):
 *   geometry / spherical harmonics  src/kokkos_learned_energy_forces.cpp:14-306
 *   cutoff, Bernstein RBF, filters,
 *   QKV, attention                  src/kokkos_integrated_block0.cpp:117-385
 *   post-attention block            src/kokkos_post_attention_block0.cpp:97-300
 *   embedding + block chaining      src/kokkos_local_energy_reverse.cpp:175-225
 *   output heads (+ reverse)        src/kokkos_output_heads.cpp:137-581
 *   ZBL repulsion                   src/kokkos_physical_zbl.cpp:31-179
 *   long range                      src/kokkos_physical_long_range.cpp:11-381
 *   charge/spin embedding           src/so3lr_charge_spin.cpp:46-141
 *   block reverse                   src/kokkos_attention_scatter_reverse.cpp:280-500,
 *                                   src/kokkos_block2_attention_input_reverse.cpp:144-390,
 *                                   src/kokkos_post_attention_reverse.cpp:107-449
 *   orchestration, charge
 *   correction, virial              plugins/lammps/pair_so3lr_native_mpi.cpp:944-990,1596-1878
 *   per-image charge correction     src/kokkos_image_segments.cpp
 *   architecture options            src/so3lr_architecture.cpp:300-392
 *     RMSNorm, norm positions       src/kokkos_post_attention_block0.cpp:126-162
 *     QK normalisation              src/kokkos_integrated_block0.cpp:288-328
 *     residual scalars              src/kokkos_local_energy_reverse.cpp:85-170
 *     NLH repulsion                 src/kokkos_physical_zbl.cpp:145-162
 *     C6 ratio head, C6 mixing      src/kokkos_output_heads.cpp:108-180,405-415,
 *                                   src/kokkos_physical_long_range.cpp:120-360
 *
 * Parity pins: every function here is checked in tests/test_oracle_*.py against
 * the reference's JAX golden vectors (tests/golden/refs), closed forms, finite
 * differences of the energy and invariances.  See the test files for which
 * check pins which function.  tests/test_model_file.py repeats the force
 * finite differences on a second, perturbed set of weights, so that the
 * reverse pass is not checked only on the shipped checkpoint's values.
 */
#ifndef SO3LR_ORACLE_H
#define SO3LR_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Widths.  The invariant width F, the radial basis R, the degree slots and
 * the energy/charge head width are model fields (so3lr_architecture.cpp:
 * 246-330, 420-450); the rest are fixed by the architecture:
 *   heads = F / 32, each 32 wide, one equivariant head per degree slot
 *   (so3lr_capabilities.cpp:62-69); slot s carries 2 l_s + 1 channels, the
 *   slots' degrees sorted, l in 1..4, a degree may repeat; equivariant width
 *   E = sum_s (2 l_s + 1); interaction width F + slots; spherical filter
 *   hidden width F / 4; Hirshfeld and C6 ratio heads 64 wide
 *   (kokkos_output_heads.cpp:16-20). */
#define ORC_HW 32    /* head width */
#define ORC_HH 64    /* Hirshfeld head width */
#define ORC_MAXL 8   /* interaction blocks, at most */
#define ORC_MAXF 256 /* invariant width, at most */
#define ORC_MAXR 64  /* radial basis, at most */
#define ORC_MAXS 8   /* degree slots (= heads), at most */
#define ORC_MAXE 72  /* equivariant channels, at most (8 slots of l = 4) */
#define ORC_MAXK 256 /* energy/charge head hidden width, at most */

/* Global tensors (pointer slots, filled by the caller from the .so3lr file). */
enum {
  ORC_EMB_W = 0,    /* (F,118) model.inv_feature_embedding.embedding.weight */
  ORC_RBF_B,        /* (R)       model.radial_embedding.radial_basis_fn.b */
  ORC_E_W1, ORC_E_B1, ORC_E_W2, ORC_E_B2, ORC_E_SCALE, ORC_E_SHIFT,
  ORC_Q_EMB, ORC_Q_W1, ORC_Q_B1, ORC_Q_W2, ORC_Q_B2,
  ORC_H_QEMB, ORC_H_W1, ORC_H_B1, ORC_H_W2, ORC_H_B2, ORC_H_VSHIFT,
  ORC_CE_WQ, ORC_CE_WK, ORC_CE_WV, ORC_CE_M1, ORC_CE_M3,
  ORC_SE_WQ, ORC_SE_WK, ORC_SE_WV, ORC_SE_M1, ORC_SE_M3,
  ORC_ALPHA_REF, ORC_C6_REF,
  /* optional C6 ratio head (NULL when the model has none), laid out as the
   * Hirshfeld head: (100,64) (64,F) (64) (64,64) (64) (100,1) */
  ORC_C6_QEMB, ORC_C6_W1, ORC_C6_B1, ORC_C6_W2, ORC_C6_B2, ORC_C6_VSHIFT,
  ORC_NGLOBAL
};

/* Per-block tensors: slot ORC_NGLOBAL + block * ORC_NBLOCK + id. */
enum {
  ORC_B_WQ = 0, ORC_B_WK, ORC_B_WV, ORC_B_WQE, ORC_B_WKE, /* (F/32,32,32) */
  ORC_B_FI_RW0, ORC_B_FI_RB0, ORC_B_FI_RW1, ORC_B_FI_RB1,
  ORC_B_FI_EW0, ORC_B_FI_EB0, ORC_B_FI_EW1, ORC_B_FI_EB1,
  ORC_B_FE_RW0, ORC_B_FE_RB0, ORC_B_FE_RW1, ORC_B_FE_RB1,
  ORC_B_FE_EW0, ORC_B_FE_EB0, ORC_B_FE_EW1, ORC_B_FE_EB1,
  ORC_B_ATT_CG, ORC_B_INT_CG,
  ORC_B_LN1_W, ORC_B_LN1_B, ORC_B_M1_W, ORC_B_M1_B, ORC_B_M2_W, ORC_B_M2_B,
  ORC_B_INT_W, ORC_B_INT_B, ORC_B_LN2_W, ORC_B_LN2_B,
  ORC_NBLOCK
};

#define ORC_NTENSOR (ORC_NGLOBAL + ORC_MAXL * ORC_NBLOCK)

/* Normalisation at the two positions of the post-attention block
 * (kokkos_post_attention_block0.cpp:97-162): affine LayerNorm, RMSNorm
 * without scale, or none (the second position only). */
enum { ORC_NORM_LAYER = 0, ORC_NORM_RMS = 1, ORC_NORM_NONE = 2 };
/* Short-range repulsion (kokkos_physical_zbl.cpp:81-177). */
enum { ORC_REP_ZBL = 0, ORC_REP_NLH = 1 };

/* Scalar slots. */
enum {
  ORC_S_GAMMA = 0, ORC_S_RMAX, ORC_S_AVG_NN, ORC_S_EMB_SCALE, ORC_S_LN_EPS,
  ORC_S_ZBL_KE, ORC_S_ZBL_SWITCH_OFF, ORC_S_ZBL_P, ORC_S_ZBL_D,
  ORC_S_ZBL_A1, ORC_S_ZBL_A2, ORC_S_ZBL_A3, ORC_S_ZBL_A4,
  ORC_S_ZBL_C1, ORC_S_ZBL_C2, ORC_S_ZBL_C3, ORC_S_ZBL_C4,
  ORC_S_LR_KE, ORC_S_LR_SIGMA, ORC_S_LR_CUTOFF, ORC_S_LR_CUTON_EL,
  ORC_S_LR_FINE, ORC_S_LR_BOHR, ORC_S_LR_HARTREE, ORC_S_LR_DISP_SCALE,
  ORC_S_LR_CUTON_DISP, ORC_S_LR_PAIR_SCALE,
  ORC_NSCALAR
};

typedef struct {
  const double *t[ORC_NTENSOR];
  const int64_t *rbf_k;     /* (R) */
  const int64_t *rbf_krev;  /* (R) */
  int64_t n_alpha_ref;      /* extent of the reference alpha/C6 tables */
  double s[ORC_NSCALAR];
  /* Architecture options; all zero/NULL is the v1 model with 3 blocks. */
  int64_t n_blocks;         /* interaction blocks (0 means 3) */
  int64_t norm1, norm2;     /* ORC_NORM_* of the two positions */
  int64_t qk_norm;          /* RMS-normalise the q, k, q_ev, k_ev head rows */
  int64_t repulsion;        /* ORC_REP_* */
  int64_t nlh_cap;          /* NLH tables: (cap, cap, 3) amplitudes and rates */
  const double *nlh_a, *nlh_b;
  const double *resid;      /* residual scalars per block (NULL: none) */
  const double *x0l;
  /* Widths; all zero is F = 128, R = 32, degrees 1,2,3,4, head width F. */
  int64_t F;                /* invariant features: a multiple of 32 up to ORC_MAXF */
  int64_t R;                /* radial basis, up to ORC_MAXR */
  int64_t n_slots;          /* degree slots = F / 32 */
  int64_t degrees[ORC_MAXS];/* degree of each slot, sorted, 1..4 */
  int64_t head_hidden;      /* energy and charge head hidden width */
} orc_model;

typedef struct {
  /* per-node outputs, each n long unless noted; any may be NULL */
  double *e_learned;   /* energy head (incl. per-element shift) */
  double *e_zbl;       /* ZBL repulsion, per receiver */
  double *e_lr;        /* Coulomb + dispersion, 0.5/0.5 split */
  double *charges;     /* corrected partial charges */
  double *hirshfeld;   /* Hirshfeld ratios */
  double *forces;      /* n*3, total force -dE/dx */
  double *virial;      /* 6: xx yy zz xy xz yz (-sum v (x) dE/dv, symmetrised) */
  double *image_energy;/* n_images: per-image total energy (packed mode) */
  double *vatom;       /* n*6 per-atom virial: each edge's and LR pair's
                          -v (x) dE/dv (symmetrised, as virial) split half to
                          each endpoint; sums to virial.  The reference has no
                          per-atom virial (pair_so3lr_native_mpi.cpp:1248-1251). */
  double *c6_ratios;   /* C6 head output (models with that head) */
  double e_elec_total; /* sum of electrostatic pair energies */
  double e_disp_total; /* sum of dispersion pair energies */
  double e_total;      /* sum of all per-node energies */
} orc_out;

/*
 * Charge/spin offset table (118 x F, row Z-1), to be added to the element
 * embedding before the embedding scale.  counts[z] is the number of atoms of
 * element z (index 0 unused).  psi is the total charge for the charge module
 * and multiplicity-1 for the spin module.  Follows so3lr_charge_spin.cpp:52-114.
 * Returns 0, or a nonzero code if a needed module is absent (never for v1).
 */
int orc_charge_spin_table(const orc_model *m, const int64_t counts[119],
                          double total_charge, double unpaired,
                          double *table);

/* (Q, M) validity per so3lr_charge_spin.cpp:116-141; 0 when consistent. */
int orc_charge_multiplicity_problem(const int64_t counts[119],
                                    double total_charge, double multiplicity);

/*
 * Full E + F + virial evaluation of one packed set of images.
 *   n nodes (all owned), atomic numbers z.
 *   emb_offset: n*F per-node charge/spin offsets (NULL = zero).
 *   image: n image ids in [0, n_images) (NULL = one image), image_charge:
 *   requested total charge per image.
 *   SR graph: ne directed edges, senders/receivers node indices, vectors
 *   v = x_receiver - x_sender (any order; the reference's order is
 *   receiver-major).
 *   LR graph: np unique half pairs (pi = sender, pj = receiver),
 *   vectors d = x_pj - x_pi.
 * Returns 0 on success.
 */
int orc_evaluate(const orc_model *m, int64_t n, const int64_t *z,
                 const double *emb_offset, int64_t n_images,
                 const int64_t *image, const double *image_charge,
                 int64_t ne, const int64_t *senders, const int64_t *receivers,
                 const double *vectors, int64_t np, const int64_t *pi,
                 const int64_t *pj, const double *pvectors, orc_out *out);

/* RMS normalisation of `rows` rows of `width` values:
 * y = x / sqrt(mean(x^2) + eps), inv_rms[row] = 1 / sqrt(mean(x^2) + eps)
 * (inv_rms may be NULL).  RMSNorm without scale
 * (kokkos_post_attention_block0.cpp:126-143, width F, eps of the model) and
 * the QK normalisation (kokkos_integrated_block0.cpp:288-328, width 32,
 * eps 1e-6) are this function. */
void orc_rms_rows(int64_t rows, int64_t width, const double *x, double eps, double *y,
                  double *inv_rms);

/* Real spherical harmonics l=1..4 at a unit vector (24 values). */
void orc_spherical_harmonics(double x, double y, double z, double *value);

/* Number of OpenMP threads the oracle runs with (1 without OpenMP). */
int orc_num_threads(void);

#ifdef __cplusplus
}
#endif

#endif
