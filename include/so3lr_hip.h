/*
 * so3lr_hip -- MI355X (gfx950) SO3LR force evaluator, C ABI.
 *
 * Drop-in replacement for the compute path behind
 *   pair_style so3lr/native/mpi MODEL [Q [M]]  /  pair_coeff * * E1 ... En
 * running as one LAMMPS rank on one GPU.  Ghost rows come from LAMMPS's own
 * communication and are collapsed onto their owners, so no GPU-to-GPU
 * exchange exists.  Each entry point names the reference interface it
 * replaces (paths under source/so3lr-lammps-native/).
 *
 * Threading: one context per rank; a context is not thread-safe.  All host
 * pointers are caller-owned and only read or written during the call.  All
 * device memory belongs to the context; capacities are retained across calls.
 * Every function returns SO3LR_OK (0) or a nonzero status; the message of the
 * last failure is available from so3lr_last_error().
 */
#ifndef SO3LR_HIP_H
#define SO3LR_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SO3LR_HIP_ABI_VERSION 1

/* status codes */
#define SO3LR_OK 0
#define SO3LR_ERR_ARGUMENT 1    /* bad pointer, size or flag */
#define SO3LR_ERR_MODEL 2       /* unreadable, corrupt or unsupported .so3lr */
#define SO3LR_ERR_SYSTEM 3      /* (charge, multiplicity) or element problem */
#define SO3LR_ERR_TOPOLOGY 4    /* neighbour lists inconsistent with the rows */
#define SO3LR_ERR_DEVICE 5      /* HIP runtime failure */
#define SO3LR_ERR_STATE 6       /* call made before its prerequisites */
#define SO3LR_ERR_UNSUPPORTED 7 /* request the path does not implement */

/* compute flags: LAMMPS eflag_global / eflag_atom / vflag_global / vflag_atom */
#define SO3LR_ENERGY 1
#define SO3LR_EATOM 2
#define SO3LR_VIRIAL 4
#define SO3LR_VATOM 8 /* accepted; values from so3lr_last_vatom (the reference refuses
                         per-atom virial, pair_so3lr_native_mpi.cpp:1248-1251) */

/* neighbour-list kinds accepted for the short-range list */
#define SO3LR_LIST_FULL 0 /* LAMMPS full list (the reference's SR request) */
#define SO3LR_LIST_HALF 1 /* LAMMPS newton-on half list */

typedef struct so3lr_ctx so3lr_ctx;

/*
 * Read and validate a .so3lr model, negotiate capabilities, upload weights to
 * HIP device `device`.  Replaces PairSO3LRNativeMPI::settings model loading
 * (plugins/lammps/pair_so3lr_native_mpi.cpp:1097-1137) and NativeModel::load
 * (src/native_model.cpp:325-406).  Accepts what the reference's MPI path
 * accepts (src/so3lr_capabilities.cpp:54-85): F = 128 or 256 features in
 * heads of 32, R = 32 or 64, sorted degree slots (repeats allowed), any
 * energy/charge head width and the optional operators; refusals return
 * SO3LR_ERR_MODEL with the rule in so3lr_last_error(NULL).
 */
int so3lr_create(const char *model_path, int device, so3lr_ctx **out);

/* Release all device and host resources. */
void so3lr_destroy(so3lr_ctx *ctx);

/* Message of the last failure on this context (or, when ctx is NULL, of the
 * calling thread's last failed so3lr_create or so3lr_check_system). */
const char *so3lr_last_error(const so3lr_ctx *ctx);

/* Short-range (which = 0) or long-range (which = 1) model cutoff in Angstrom;
 * PairSO3LRNativeMPI::init_one returns the SR cutoff (:1162-1172). */
double so3lr_cutoff(const so3lr_ctx *ctx, int which);

/* Element token (symbol in any case, or atomic number) -> Z in 1..99, 0 when
 * unknown.  Same rule as plugins/lammps/so3lr_element_map.h:15-49. */
int so3lr_atomic_number(const char *token);

/*
 * (Q, M) check of one composition, host only: no context and no device.
 * Returns SO3LR_OK, SO3LR_ERR_ARGUMENT (no atoms, Z outside 1..99) or
 * SO3LR_ERR_SYSTEM, with the reason in so3lr_last_error(NULL).  The rule of
 * charge_multiplicity_problem (src/so3lr_charge_spin.cpp:100-141), which
 * PairSO3LRTurbo::init_style runs for each image on its own rank
 * (plugins/lammps/pair_so3lr_turbo.cpp:208-219).
 */
int so3lr_check_system(int64_t n, const int32_t *z, double total_charge, double multiplicity);

/*
 * Owned atoms of the system: atomic numbers and the global (Q, M).  Validates
 * (Q, M) against the composition and builds the charge/spin embedding table.
 * Replaces PairSO3LRNativeMPI::setup_charge_spin (:1196-1235) and
 * charge_spin_offset_table / charge_multiplicity_problem
 * (src/so3lr_charge_spin.cpp:100-141).
 */
int so3lr_set_system(so3lr_ctx *ctx, int64_t n_owned, const int32_t *z,
                     double total_charge, double multiplicity);

/*
 * Packed independent images (turbo semantics,
 * src/kokkos_packed_so3lr_evaluator.cpp:180-286): owned atoms are grouped in
 * n_images contiguous ranges image_offsets[0..n_images] (image_offsets[0] = 0,
 * image_offsets[n_images] = n_owned); each image has its own total charge and
 * multiplicity, its own charge correction and its own charge/spin table
 * (src/kokkos_turbo_replica_bridge.cpp:122-145).  Call instead of
 * so3lr_set_system.  No periodic images may connect two images.
 */
int so3lr_set_images(so3lr_ctx *ctx, int64_t n_owned, const int32_t *z,
                     int64_t n_images, const int64_t *image_offsets,
                     const double *charges, const double *multiplicities);

/*
 * Candidate neighbour lists, given at every LAMMPS reneighbor (cut-off plus
 * skin).  Rows are LAMMPS atom rows: rows [0, n_owned) are owned, the rest are
 * ghosts; owner_of_row maps every row to its owned atom (tag collapse, the
 * one-rank periodic-image collapse of plugins/lammps/pair_so3lr_native.cpp:74-146).
 * Each list is CSR over receivers: ilist[k] is an owned row, its neighbours are
 * neigh[offsets[k] .. offsets[k+1]).
 *   SR list: full (SO3LR_LIST_FULL, the reference's request id 0) or newton-on
 *            half list; every directed edge of a full list must have its
 *            reverse.
 *   LR list: newton-on half list (the reference's request id 1).
 * Replaces snapshot_neighbor_list + build_lammps_native_candidate_topologies +
 * upload_device_candidate_graph (pair_so3lr_native_mpi.cpp:76-105,1297-1334;
 * src/lammps_neighbor_adapter.cpp:190-280).  A pair of an atom with its own
 * periodic image is refused, as the one-rank collapse refuses it.  For one
 * system (not packed images) the first evaluation on a new topology also puts
 * the owned atoms in a spatial order of its positions, inside the library;
 * results still come back in the caller's atom order.
 */
int so3lr_set_topology(so3lr_ctx *ctx, int64_t n_rows, const int32_t *owner_of_row,
                       int sr_kind, int64_t sr_inum, const int32_t *sr_ilist,
                       const int64_t *sr_offsets, const int32_t *sr_neigh,
                       int64_t lr_inum, const int32_t *lr_ilist,
                       const int64_t *lr_offsets, const int32_t *lr_neigh);

/*
 * One force evaluation.  x_rows: n_rows*3 host positions (owned + ghost rows,
 * LAMMPS atom->x).  Writes (overwrites) f_owned[n_owned*3] with the total force,
 * eatom[n_owned] when SO3LR_EATOM (may be NULL otherwise), *energy when
 * SO3LR_ENERGY and virial[6] (xx yy zz xy xz yz, the LAMMPS order) when
 * SO3LR_VIRIAL.  The caller adds them to atom->f, eatom, eng_vdwl and
 * virial as PairSO3LRNativeMPI::compute does (:1867-1878).
 * Replaces PairSO3LRNativeMPI::compute (:1246-1978).
 */
int so3lr_compute(so3lr_ctx *ctx, const double *x_rows, int flags, double *f_owned,
                  double *eatom, double *energy, double *virial);

/*
 * As so3lr_compute, with x_rows, f_owned and eatom in device memory (HBM
 * resident; no host copies of positions or forces).  energy and virial stay
 * host pointers.  Work is ordered on the context's stream (so3lr_set_stream).
 * When the same call (same pointers, flags, box, stream and topology) comes
 * twice in a row, its launch sequence is captured into a HIP graph and
 * replayed on later identical calls; the results are bit-identical to the
 * kernel-by-kernel launch (environment SO3LR_NO_GRAPH=1 turns replay off).
 */
int so3lr_compute_device(so3lr_ctx *ctx, const double *x_rows_dev, int flags,
                         double *f_owned_dev, double *eatom_dev, double *energy,
                         double *virial);

/*
 * As so3lr_compute_device, allocating nothing: no counterpart in the
 * reference; for callers that cannot allocate device memory (tight serving
 * loops, harnesses that forbid hipMalloc after set-up).  Every work buffer of
 * the evaluation is a slice of one static device array of 256 MiB that the
 * library holds on each device it runs on; a system that needs more work
 * space is refused with SO3LR_ERR_ARGUMENT (so3lr_compute_device has no such
 * limit).  The topology must have been set before (so3lr_set_topology or
 * so3lr_reneighbor_device, which allocate).  No graph is captured and no
 * event recorded; the call waits for its stream at the end (energy and
 * virial read-back), as so3lr_compute_device does.  All contexts on one
 * device share that device's array and the previous call's contents stay in
 * it: calls that overlap on one device race.  so3lr_last_terms and
 * so3lr_last_vatom refuse (SO3LR_ERR_STATE) after this call.
 */
int so3lr_compute_device_noalloc(so3lr_ctx *ctx, const double *x_rows_dev, int flags,
                                 double *f_owned_dev, double *eatom_dev, double *energy,
                                 double *virial);

/*
 * HBM-resident reneighbor (no counterpart in the reference, where LAMMPS
 * builds the lists on the host): builds the same candidate sets -- every
 * periodic image within cutoff + skin, SR and LR -- on the GPU from the owned
 * positions x_owned_dev (n_owned*3, device), after wrapping them in place into
 * the orthogonal box [lo, hi) along periodic axes (LAMMPS Domain::pbc).  Every
 * periodic length must exceed twice the long-range cutoff.  Afterwards
 * so3lr_compute_device takes owned positions (x_rows_dev = x_owned_dev, no
 * ghost rows) until the next so3lr_set_topology.
 */
int so3lr_reneighbor_device(so3lr_ctx *ctx, double *x_owned_dev, const double *lo,
                            const double *hi, const int *periodic, double skin);

/* Box of the device reneighbor path between rebuilds (NPT); same axes. */
int so3lr_set_box(so3lr_ctx *ctx, const double *lo, const double *hi);

/* Order all device work on `stream` (a hipStream_t; NULL = the context's own
 * stream).  The stream must have default priority. */
int so3lr_set_stream(so3lr_ctx *ctx, void *stream);

/*
 * Per-atom decomposition of the last evaluation, in owned-atom order; any
 * pointer may be NULL.  The analogue of SO3LR_NATIVE_DEBUG_DUMP
 * (pair_so3lr_native_mpi.cpp:1816-1865): learned energy (with the per-element
 * shift), ZBL energy, long-range energy, partial charges, Hirshfeld ratios;
 * totals[0] electrostatic and totals[1] dispersion energy.  image_energy
 * receives per-image totals in packed mode.
 */
int so3lr_last_terms(so3lr_ctx *ctx, double *learned, double *zbl, double *long_range,
                     double *charges, double *hirshfeld, double *totals,
                     double *image_energy);

/*
 * Per-atom virial of the last evaluation (no counterpart in the reference,
 * which refuses vflag_atom, pair_so3lr_native_mpi.cpp:1248-1251): vatom[6 * i
 * + c] for owned atom i, LAMMPS order xx yy zz xy xz yz.  Each pair's
 * -v (x) dE/dv (short range: the pair vector and its energy gradient, which
 * carries the whole network's dependence on that pair; long range: the
 * Coulomb and dispersion pair force), symmetrised as in the global virial,
 * goes half to each endpoint; the atoms' sum is the global virial.
 * on_device = 0: vatom is host memory; 1: device memory, written on the
 * context's stream.  The pair style adds it into vatom of its owned rows.
 */
int so3lr_last_vatom(so3lr_ctx *ctx, double *vatom, int on_device);

/* Number of short-range pairs inside the cutoff at the last evaluation, and
 * the candidate counts of the current topology (SR pairs, LR pairs). */
int so3lr_graph_stats(const so3lr_ctx *ctx, int64_t *sr_active, int64_t *sr_candidates,
                      int64_t *lr_candidates);

/*
 * Measurement hook (no counterpart in the reference, which times phases with
 * fenced host clocks, pair_so3lr_native_mpi.cpp:1681-1762): when enabled,
 * HIP events are recorded on the launch stream around the kernels
 * "filter_fwd", "filter_bwd", "attn_fwd", "attn_bwd" and "long_range".
 * Block 0 runs cheaper instantiations of the MFMA filters and of the reverse
 * attention (its ev input is zero); they are timed as "filter_fwd_block0",
 * "filter_bwd_block0" and "attn_bwd_block0".
 * Enabling clears the totals; disabling keeps them for reading.  While
 * enabled, evaluations are launched kernel by kernel (no graph replay).
 * _read returns the summed duration, the number of launches and the units
 * processed (active pairs for the filter kernels, owned atoms otherwise).
 */
int so3lr_kernel_timing(so3lr_ctx *ctx, int enable);
int so3lr_kernel_timing_read(so3lr_ctx *ctx, const char *kernel, double *total_ms,
                             int64_t *launches, int64_t *units);

/* Device bytes held by the context (weights + retained workspaces). */
int64_t so3lr_device_bytes(const so3lr_ctx *ctx);

#ifdef __cplusplus
}
#endif

#endif /* SO3LR_HIP_H */
