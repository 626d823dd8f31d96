/* ----------------------------------------------------------------------
   LAMMPS plugin registering so3lr/turbo on libso3lr_turbo (many one-rank
   partitions batched onto one GPU; plugins/lammps/pair_so3lr_turbo.cpp).
   Load with:  plugin load so3lrturbohipplugin.so
------------------------------------------------------------------------- */

#include "lammpsplugin.h"
#include "version.h"

#include "pair_so3lr_turbo_hip.h"

using namespace LAMMPS_NS;

static Pair *so3lr_turbo_hip_creator(LAMMPS *lmp)
{
  return new PairSO3LRTurboHip(lmp);
}

extern "C" void lammpsplugin_init(void *lmp, void *handle, void *regfunc)
{
  auto register_plugin = reinterpret_cast<lammpsplugin_regfunc>(regfunc);
  lammpsplugin_t plugin;
  plugin.version = LAMMPS_VERSION;
  plugin.style = "pair";
  plugin.name = "so3lr/turbo";
  plugin.info = "SO3LR independent images batched onto one MI355X (libso3lr_turbo, fp64)";
  plugin.author = "so3lr-mi355x";
  plugin.creator.v1 = reinterpret_cast<lammpsplugin_factory1 *>(&so3lr_turbo_hip_creator);
  plugin.handle = handle;
  (*register_plugin)(&plugin, lmp);
}
