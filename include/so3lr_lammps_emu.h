/*
 * so3lr_lammps_emu -- host-side stand-in for the LAMMPS pieces the pair style
 * consumes (not part of the drop-in library): ghost atoms from periodic
 * images inside the communication cutoff (LAMMPS comm), and the neighbour
 * lists the pair style requests in init_style (pair_so3lr_native_mpi.cpp:
 * 1174-1192): a full short-range list (id 0) and a newton-on half long-range
 * list (id 1), both with cutoff + skin.  Used by the tests and by bench.py to
 * drive libso3lr_hip.so the way LAMMPS does.  Orthogonal boxes only.
 */
#ifndef SO3LR_LAMMPS_EMU_H
#define SO3LR_LAMMPS_EMU_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct so3lr_emu_lists so3lr_emu_lists;

/*
 * x: n owned positions inside [lo, hi) along periodic dimensions.
 * periodic[3]: 1 = periodic.  Ghosts are images within comm_cut of the box.
 * Lists hold rows within (cut + skin) of each owned receiver, in receiver
 * order 0..n-1.  sr_full = 1 builds the SR list full (both directions),
 * 0 builds it as a newton-on half list.  The LR list is always half.
 * Returns 0, or nonzero with a message in so3lr_emu_error().
 */
int so3lr_emu_build(int64_t n, const double *x, const double *lo, const double *hi,
                    const int *periodic, double sr_cut, double lr_cut, double skin,
                    double comm_cut, int sr_full, so3lr_emu_lists **out);
const char *so3lr_emu_error(void);
void so3lr_emu_free(so3lr_emu_lists *l);

int64_t so3lr_emu_rows(const so3lr_emu_lists *l);
/* owner of each row (identity on owned rows) and integer image flags (3 per
 * row): x_row = x_owner + flags * (hi - lo) */
const int32_t *so3lr_emu_owner(const so3lr_emu_lists *l);
const int32_t *so3lr_emu_image(const so3lr_emu_lists *l);
/* which = 0: SR list, 1: LR list.  inum = n; offsets has inum + 1 entries. */
int64_t so3lr_emu_inum(const so3lr_emu_lists *l, int which);
const int32_t *so3lr_emu_ilist(const so3lr_emu_lists *l, int which);
const int64_t *so3lr_emu_offsets(const so3lr_emu_lists *l, int which);
const int32_t *so3lr_emu_neigh(const so3lr_emu_lists *l, int which);

#ifdef __cplusplus
}
#endif

#endif
