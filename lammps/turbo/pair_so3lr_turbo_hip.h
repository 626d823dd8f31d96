/* -*- c++ -*- ----------------------------------------------------------
   pair_style so3lr/turbo on libso3lr_turbo: many one-rank, non-periodic
   LAMMPS partitions (one image each, its own charge and multiplicity)
   evaluated together on one GPU by universe rank 0.

   Commands and messages follow PairSO3LRTurbo
   (source/so3lr-lammps-native/plugins/lammps/pair_so3lr_turbo.{h,cpp}).  The
   Python mirror of this class is so3lrxlammps_amd/turbo.py.
------------------------------------------------------------------------- */

#ifdef PAIR_CLASS
// clang-format off
PairStyle(so3lr/turbo,PairSO3LRTurboHip);
// clang-format on
#else

#ifndef LMP_PAIR_SO3LR_TURBO_HIP_H
#define LMP_PAIR_SO3LR_TURBO_HIP_H

#include "pair.h"

#include <cstdint>
#include <vector>

struct so3lr_turbo;

namespace LAMMPS_NS {

class PairSO3LRTurboHip : public Pair {
 public:
  PairSO3LRTurboHip(class LAMMPS *);
  ~PairSO3LRTurboHip() override;
  void compute(int, int) override;
  void settings(int, char **) override;
  void coeff(int, char **) override;
  void init_style() override;
  double init_one(int, int) override;
  void init_list(int, class NeighList *) override;

 private:
  so3lr_turbo *broker = nullptr;
  double total_charge = 0.0, multiplicity = 1.0, short_range_cutoff = 0.0, long_range_cutoff = 0.0;
  std::vector<int> type_z;    // LAMMPS type -> Z (index 0 unused)
  class NeighList *list_sr = nullptr, *list_lr = nullptr;
  std::vector<int32_t> z, ilist_sr, neigh_sr, ilist_lr, neigh_lr;
  std::vector<int64_t> off_sr, off_lr;
  std::vector<double> x, f, ea;

  void allocate();
};

}    // namespace LAMMPS_NS

#endif
#endif
