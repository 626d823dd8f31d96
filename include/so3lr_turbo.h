/*
 * so3lr_turbo -- independent-image batching over MPI onto one GPU, C ABI.
 *
 * Drop-in for the compute path behind
 *   pair_style so3lr/turbo MODEL [Q [M]]  /  pair_coeff * * E1 ... En
 * (plugins/lammps/pair_so3lr_turbo.cpp; paths under
 * source/so3lr-lammps-native/).  Every rank of the communicator is a one-rank
 * LAMMPS partition holding one non-periodic image (its own atoms, integrator,
 * charge and multiplicity).  The coordinator rank owns a so3lr_hip context on
 * its GPU, evaluates all images as one packed system (so3lr_set_images) and
 * hands every image back its own energy, forces, per-atom energies, charges
 * and Hirshfeld ratios.  Workers make no HIP call and hold no model.
 *
 * Communicators cross this ABI as Fortran handles (MPI_Comm_c2f), so the
 * header needs no mpi.h.  The library is built against MPICH (libmpi.so.12).
 * Status codes and flags are those of so3lr_hip.h.  Every function except
 * so3lr_turbo_last_error, so3lr_turbo_info and so3lr_turbo_stats is
 * collective over the communicator, and the calls that can fail return the
 * same status on every rank, so that one image's problem stops every image
 * rather than leaving the others waiting.
 */
#ifndef SO3LR_TURBO_H
#define SO3LR_TURBO_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct so3lr_turbo so3lr_turbo;

/*
 * For hosts without an MPI binding: MPI_Init when MPI is not yet initialised
 * (collective over MPI_COMM_WORLD), then *comm_f = MPI_Comm_c2f(MPI_COMM_WORLD),
 * *rank and *size of it (either pointer may be NULL).  LAMMPS passes
 * MPI_Comm_c2f(universe->uworld) to so3lr_turbo_create instead.
 */
int so3lr_turbo_mpi_world(int64_t *comm_f, int *rank, int *size);
/* MPI_Finalize, when this library initialised MPI. */
int so3lr_turbo_mpi_finalize(void);

/*
 * Per-image (Q, M) check (so3lr_check_system on every rank), combined over
 * the communicator: SO3LR_OK everywhere, or on every rank the status of the
 * lowest failing rank with the message "Pair style so3lr/turbo image K:
 * charge Q with multiplicity M: <reason>" in so3lr_turbo_last_error(NULL).
 * PairSO3LRTurbo::init_style (pair_so3lr_turbo.cpp:208-222), where the failing
 * image stops the universe (error->universe_one).
 */
int so3lr_turbo_check_images(int64_t comm_f, int64_t n, const int32_t *z, double total_charge,
                             double multiplicity);

/*
 * The broker: the coordinator loads `model_path` onto HIP device `device`;
 * the other ranks' model_path and device are ignored.  A coordinator failure
 * is returned on every rank with its message.  Replaces the coordinator model
 * load of PairSO3LRTurbo::settings (pair_so3lr_turbo.cpp:112-154) and
 * MpiTurboReplicaBroker::MpiTurboReplicaBroker (src/mpi_turbo_replica_broker.cpp:
 * 111-128).
 */
int so3lr_turbo_create(int64_t comm_f, int coordinator, const char *model_path, int device,
                       so3lr_turbo **out);

/* Release the broker and the coordinator's context.  It frees the broker's
 * duplicate of the communicator: call it on every rank, before MPI_Finalize. */
void so3lr_turbo_destroy(so3lr_turbo *t);

/* Message of the last failure on this broker (NULL: of the calling thread's
 * last failed so3lr_turbo_create, so3lr_turbo_check_images or
 * so3lr_turbo_mpi_world). */
const char *so3lr_turbo_last_error(const so3lr_turbo *t);

/* This rank, the number of images, the coordinator rank, and the model's SR
 * and LR cutoffs (Angstrom; broadcast from the coordinator: init_one returns
 * the LR cutoff, pair_so3lr_turbo.cpp:175-180).  Any pointer may be NULL. */
int so3lr_turbo_info(const so3lr_turbo *t, int *rank, int *size, int *coordinator,
                     double *sr_cutoff, double *lr_cutoff);

/*
 * One force evaluation of this rank's image, collective.
 *   n, z[n], x[n*3]: the image's owned atoms (a one-rank non-periodic
 *     partition has no ghost rows);
 *   total_charge, multiplicity: the image's (Q, M);
 *   lists_changed: nonzero when the lists differ from the previous call's
 *     (LAMMPS neighbor->ago == 0); an image sends its lists only then, on its
 *     first call, when its atom count changed, and after a failed call;
 *   SR list (sr_kind SO3LR_LIST_FULL as the style requests it, or
 *     SO3LR_LIST_HALF) and LR half list, CSR over receivers as in
 *     so3lr_set_topology, with NEIGHMASK already applied; every row index
 *     must be an owned atom of the image.
 * Writes f[n*3] (the image's forces, overwritten), and eatom, charges,
 * hirshfeld [n] and *energy (the image's total energy) where not NULL.
 * A malformed image anywhere returns SO3LR_ERR_TOPOLOGY on every rank, naming
 * the image; the broker stays usable.
 * Replaces PairSO3LRTurbo::compute (pair_so3lr_turbo.cpp:235-319),
 * MpiTurboReplicaBroker::evaluate (mpi_turbo_replica_broker.cpp:130-305) and
 * KokkosTurboReplicaBridge::evaluate (src/kokkos_turbo_replica_bridge.cpp:
 * 64-179).  The virial is LAMMPS's virial_fdotr_compute on the returned
 * forces, as in the reference.
 */
int so3lr_turbo_evaluate(so3lr_turbo *t, int64_t n, const int32_t *z, const double *x,
                         double total_charge, double multiplicity, int lists_changed, int sr_kind,
                         int64_t sr_inum, const int32_t *sr_ilist, const int64_t *sr_offsets,
                         const int32_t *sr_neigh, int64_t lr_inum, const int32_t *lr_ilist,
                         const int64_t *lr_offsets, const int32_t *lr_neigh, double *f, double *eatom,
                         double *charges, double *hirshfeld, double *energy);

/*
 * Figures of the last evaluation on this rank (measurement, no counterpart in
 * the reference beyond its broker_ms report, pair_so3lr_turbo.cpp:281-312):
 * packed atoms and images (coordinator; 0 elsewhere); lists_gathered: on the
 * coordinator whether any image's lists arrived, on a worker whether this
 * image sent its own; milliseconds: on the coordinator receiving every image
 * (which includes waiting for the slowest), the packed GPU evaluation and
 * sending the answers; on a worker the wait for its answer (as gather_ms);
 * and the whole call.
 */
int so3lr_turbo_stats(const so3lr_turbo *t, int64_t *packed_atoms, int64_t *images, int *lists_gathered,
                      double *gather_ms, double *evaluate_ms, double *scatter_ms, double *total_ms);

#ifdef __cplusplus
}
#endif

#endif /* SO3LR_TURBO_H */
