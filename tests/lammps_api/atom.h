// Test infrastructure: the per-atom arrays of Atom (src/atom.h).
#pragma once
#include "pointers.h"

namespace LAMMPS_NS {
class Atom {
 public:
  int nlocal = 0, nghost = 0, ntypes = 0;
  tagint *tag = nullptr;
  int *type = nullptr;
  double **x = nullptr, **f = nullptr;
};
}    // namespace LAMMPS_NS
