// Test infrastructure: the LAMMPS class's pointers (src/lammps.h), not LAMMPS.
#pragma once
#include <cstdio>

namespace LAMMPS_NS {
class Memory;
class Error;
class Universe;
class Atom;
class Neighbor;
class Comm;
class Domain;
class Force;

class LAMMPS {
 public:
  Memory *memory = nullptr;
  Error *error = nullptr;
  Universe *universe = nullptr;
  Atom *atom = nullptr;
  Neighbor *neighbor = nullptr;
  Comm *comm = nullptr;
  Domain *domain = nullptr;
  Force *force = nullptr;
  FILE *screen = nullptr, *logfile = nullptr;
};
}    // namespace LAMMPS_NS
