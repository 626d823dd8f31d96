// Test infrastructure: Universe (src/universe.h).
#pragma once
#include "pointers.h"

namespace LAMMPS_NS {
class Universe {
 public:
  MPI_Comm uworld = MPI_COMM_WORLD;
  int me = 0, nprocs = 1, nworlds = 1, iworld = 0;
};
}    // namespace LAMMPS_NS
