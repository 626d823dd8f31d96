// Test infrastructure: Neighbor and NeighConst (src/neighbor.h).  The
// requests are kept so the driver can check them; NeighRequest's members
// need neigh_request.h, as in LAMMPS.
#pragma once
#include "pointers.h"

#include <vector>

namespace LAMMPS_NS {
class NeighRequest;
class Pair;
namespace NeighConst {
enum { REQ_DEFAULT = 0, REQ_FULL = 1 << 0 };
}

class Neighbor {
 public:
  double skin = 1.0;
  int ago = -1;
  std::vector<NeighRequest *> requests;
  std::vector<int> request_flags;
  NeighRequest *add_request(Pair *, int flags = NeighConst::REQ_DEFAULT);
};
}    // namespace LAMMPS_NS
