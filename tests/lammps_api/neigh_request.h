// Test infrastructure: NeighRequest (src/neigh_request.h).
#pragma once
#include "pointers.h"

namespace LAMMPS_NS {
class NeighRequest {
 public:
  int id = 0, full = 0;
  double cutoff = 0.0;
  bool cut = false;
  void set_id(int i) { id = i; }
  void set_cutoff(double c) { cutoff = c; cut = true; }
};
}    // namespace LAMMPS_NS
