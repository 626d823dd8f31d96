// Test infrastructure: Comm (src/comm.h).
#pragma once
#include "pointers.h"

namespace LAMMPS_NS {
class Comm {
 public:
  int me = 0, nprocs = 1;
  double cutghostuser = 0.0;
  double get_comm_cutoff() { return cutghostuser; }
};
}    // namespace LAMMPS_NS
