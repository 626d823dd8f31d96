// A declaration of the subset of LAMMPS's API (src/lmptype.h) that the thin
// pair styles under lammps/ use -- test infrastructure, not LAMMPS.  Each
// name sits in the header where LAMMPS declares it, so a style that forgets
// an include fails to compile against these headers as it would against
// LAMMPS's own.
#pragma once
#include <cstdint>
#include <mpi.h>

namespace LAMMPS_NS {
typedef int tagint;         // LAMMPS's default (smallbig) integer sizes
typedef int64_t bigint;
}    // namespace LAMMPS_NS

#define NEIGHMASK 0x1FFFFFFF
#define FLERR __FILE__, __LINE__
