/* ----------------------------------------------------------------------
   LAMMPS plugin registering so3lr/native/mpi on libso3lr_hip, the plugin
   route of the reference (plugins/lammps/so3lrnativeplugin.cpp:17-36).
   Load with:  plugin load so3lrhipplugin.so
------------------------------------------------------------------------- */

#include "lammpsplugin.h"
#include "version.h"

#include "pair_so3lr_hip.h"

using namespace LAMMPS_NS;

static Pair *so3lr_hip_creator(LAMMPS *lmp)
{
  return new PairSO3LRHip(lmp);
}

extern "C" void lammpsplugin_init(void *lmp, void *handle, void *regfunc)
{
  auto register_plugin = reinterpret_cast<lammpsplugin_regfunc>(regfunc);
  lammpsplugin_t plugin;
  plugin.version = LAMMPS_VERSION;
  plugin.style = "pair";
  plugin.name = "so3lr/native/mpi";
  plugin.info = "SO3LR force field on one MI355X per rank (libso3lr_hip, fp64)";
  plugin.author = "so3lr-mi355x";
  plugin.creator.v1 = reinterpret_cast<lammpsplugin_factory1 *>(&so3lr_hip_creator);
  plugin.handle = handle;
  (*register_plugin)(&plugin, lmp);
}
