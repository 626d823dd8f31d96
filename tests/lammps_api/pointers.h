// Test infrastructure: the Pointers base class (src/pointers.h), not LAMMPS.
// Only forward declarations of the classes: their members need their own
// headers, as in LAMMPS.
#pragma once
#include "lmptype.h"
#include "lammps.h"
#include "utils.h"

namespace LAMMPS_NS {
class Pointers {
 public:
  explicit Pointers(LAMMPS *ptr)
      : lmp(ptr), memory(ptr->memory), error(ptr->error), universe(ptr->universe), atom(ptr->atom),
        neighbor(ptr->neighbor), comm(ptr->comm), domain(ptr->domain), force(ptr->force),
        screen(ptr->screen), logfile(ptr->logfile) {}
  virtual ~Pointers() = default;

 protected:
  LAMMPS *lmp;
  Memory *&memory;
  Error *&error;
  Universe *&universe;
  Atom *&atom;
  Neighbor *&neighbor;
  Comm *&comm;
  Domain *&domain;
  Force *&force;
  FILE *&screen;
  FILE *&logfile;
};
}    // namespace LAMMPS_NS
