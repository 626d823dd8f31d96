// Test infrastructure: NeighList (src/neigh_list.h).
#pragma once
#include "pointers.h"

namespace LAMMPS_NS {
class NeighList {
 public:
  int inum = 0, gnum = 0;
  int *ilist = nullptr;
  int *numneigh = nullptr;
  int **firstneigh = nullptr;
};
}    // namespace LAMMPS_NS
