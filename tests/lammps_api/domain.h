// Test infrastructure: Domain's periodicity flags (src/domain.h).
#pragma once
#include "pointers.h"

namespace LAMMPS_NS {
class Domain {
 public:
  int xperiodic = 0, yperiodic = 0, zperiodic = 0;
};
}    // namespace LAMMPS_NS
