// Test infrastructure: the Pair base class (src/pair.h) reduced to what a
// many-body pair style touches; ev_init follows LAMMPS's flag convention
// (eflag bit 1 global, 2 per atom; vflag bit 1/2 global, 4 per atom).
#pragma once
#include "pointers.h"

namespace LAMMPS_NS {
class NeighList;

class Pair : protected Pointers {
 public:
  explicit Pair(LAMMPS *lmp) : Pointers(lmp) {}
  ~Pair() override;

  double eng_vdwl = 0.0, eng_coul = 0.0;
  double virial[6] = {0, 0, 0, 0, 0, 0};
  double *eatom = nullptr;
  double **vatom = nullptr;
  int allocated = 0;
  int **setflag = nullptr;
  double **cutsq = nullptr;
  int manybody_flag = 0, one_coeff = 0, restartinfo = 1, single_enable = 1, no_virial_fdotr_compute = 0;
  int eflag_either = 0, eflag_global = 0, eflag_atom = 0;
  int vflag_either = 0, vflag_global = 0, vflag_atom = 0, vflag_fdotr = 0;

  virtual void compute(int, int) = 0;
  virtual void settings(int, char **) = 0;
  virtual void coeff(int, char **) = 0;
  virtual void init_style() {}
  virtual double init_one(int, int) { return 0.0; }
  virtual void init_list(int, NeighList *) {}

 protected:
  void ev_init(int eflag, int vflag);
  void virial_fdotr_compute();

 private:
  int maxeatom = 0, maxvatom = 0;
};
}    // namespace LAMMPS_NS
