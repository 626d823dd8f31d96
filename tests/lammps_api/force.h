// Test infrastructure: Force (src/force.h).
#pragma once
#include "pointers.h"

namespace LAMMPS_NS {
class Force {
 public:
  int newton_pair = 1;
};
}    // namespace LAMMPS_NS
