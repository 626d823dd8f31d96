/* -*- c++ -*- ----------------------------------------------------------
   pair_style so3lr/native/mpi on libso3lr_hip (one LAMMPS rank per MI355X).

   The LAMMPS side of the drop-in: the commands, argument meaning and
   error->all messages of PairSO3LRNativeMPI
   (source/so3lr-lammps-native/plugins/lammps/pair_so3lr_native_mpi.{h,cpp}),
   with the evaluation behind the C ABI of include/so3lr_hip.h.  The Python
   mirror of this class is so3lrxlammps_amd/pair_style.py; a CPU test
   (tests/test_lammps_sources.py) holds the two to the same messages and rules.
------------------------------------------------------------------------- */

#ifdef PAIR_CLASS
// clang-format off
PairStyle(so3lr/native/mpi,PairSO3LRHip);
// clang-format on
#else

#ifndef LMP_PAIR_SO3LR_HIP_H
#define LMP_PAIR_SO3LR_HIP_H

#include "pair.h"

#include <cstdint>
#include <string>
#include <vector>

struct so3lr_ctx;

namespace LAMMPS_NS {

class PairSO3LRHip : public Pair {
 public:
  PairSO3LRHip(class LAMMPS *);
  ~PairSO3LRHip() override;
  void compute(int, int) override;
  void settings(int, char **) override;
  void coeff(int, char **) override;
  void init_style() override;
  double init_one(int, int) override;
  void init_list(int, class NeighList *) override;

 private:
  so3lr_ctx *ctx = nullptr;
  std::string model_path;
  double total_charge = 0.0, multiplicity = 1.0;
  double short_range_cutoff = 0.0, long_range_cutoff = 0.0;
  std::vector<int> type_z;  // LAMMPS type -> Z (index 0 unused)
  class NeighList *list_sr = nullptr, *list_lr = nullptr;
  // host snapshots handed to so3lr_set_topology at each reneighbor
  std::vector<int32_t> z_owned, owner, ilist_sr, neigh_sr, ilist_lr, neigh_lr;
  std::vector<int64_t> off_sr, off_lr;
  std::vector<double> f_owned, e_owned, v_owned;
  bool topology_stale = true;    // set_topology must follow the last set_system

  void allocate();
  void set_system();
  void upload_topology();
};

}    // namespace LAMMPS_NS

#endif
#endif
