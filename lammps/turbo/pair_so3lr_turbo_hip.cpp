/* ----------------------------------------------------------------------
   pair_style so3lr/turbo MODEL [charge [multiplicity]] on libso3lr_turbo.

   Commands and messages follow PairSO3LRTurbo
   (source/so3lr-lammps-native/plugins/lammps/pair_so3lr_turbo.cpp): settings
   :112-154, coeff :156-173, init_one :175-180, init_style :182-223,
   init_list :225-233, compute :235-319.  Every partition is one rank with one
   non-periodic image; the broker (include/so3lr_turbo.h) gathers every
   image's atoms and lists to the coordinator, which evaluates them as packed
   images on its GPU and scatters forces and energies back.  Every failing
   broker call returns the same status on every rank, so error->universe_all
   is reached by all ranks together.
------------------------------------------------------------------------- */

#include "pair_so3lr_turbo_hip.h"

#include "atom.h"
#include "comm.h"
#include "domain.h"
#include "error.h"
#include "force.h"
#include "memory.h"
#include "neigh_list.h"
#include "neigh_request.h"
#include "neighbor.h"
#include "universe.h"
#include "utils.h"

#include "so3lr_hip.h"
#include "so3lr_turbo.h"

#include <cstring>
#include <string>

using namespace LAMMPS_NS;

static void snapshot(NeighList *l, std::vector<int32_t> &il, std::vector<int64_t> &off,
                     std::vector<int32_t> &nb)
{
  il.assign(l->ilist, l->ilist + l->inum);
  off.assign(1, 0);
  nb.clear();
  for (int ii = 0; ii < l->inum; ++ii) {
    const int i = l->ilist[ii];
    const int *jlist = l->firstneigh[i];
    for (int jj = 0; jj < l->numneigh[i]; ++jj) nb.push_back(jlist[jj] & NEIGHMASK);
    off.push_back(static_cast<int64_t>(nb.size()));
  }
}

PairSO3LRTurboHip::PairSO3LRTurboHip(LAMMPS *lmp) : Pair(lmp)
{
  manybody_flag = 1;
  one_coeff = 1;
  restartinfo = 0;
  single_enable = 0;
}

PairSO3LRTurboHip::~PairSO3LRTurboHip()
{
  so3lr_turbo_destroy(broker);    // every rank, before MPI_Finalize
  if (allocated) {
    memory->destroy(setflag);
    memory->destroy(cutsq);
  }
}

void PairSO3LRTurboHip::allocate()
{
  allocated = 1;
  const int n = atom->ntypes;
  memory->create(setflag, n + 1, n + 1, "so3lr/turbo:setflag");
  memory->create(cutsq, n + 1, n + 1, "so3lr/turbo:cutsq");
  for (int i = 1; i <= n; ++i)
    for (int j = i; j <= n; ++j) setflag[i][j] = 0;
}

void PairSO3LRTurboHip::settings(int narg, char **arg)
{
  if (narg < 1 || narg > 3)
    error->universe_all(FLERR,
                        "Illegal pair_style so3lr/turbo command: expected "
                        "'pair_style so3lr/turbo MODEL [charge [multiplicity]]'");
  // per image: each partition reads its own values (world-style variables)
  total_charge = narg > 1 ? utils::numeric(FLERR, arg[1], false, lmp) : 0.0;
  multiplicity = narg > 2 ? utils::numeric(FLERR, arg[2], false, lmp) : 1.0;
  so3lr_turbo_destroy(broker);
  broker = nullptr;
  // collective over the universe; the coordinator's failure ("Cannot
  // initialize the coordinator SO3LR model: ...") reaches every rank
  if (so3lr_turbo_create(static_cast<int64_t>(MPI_Comm_c2f(universe->uworld)), 0, arg[0], 0,
                         &broker) != SO3LR_OK)
    error->universe_all(FLERR, so3lr_turbo_last_error(nullptr));
  so3lr_turbo_info(broker, nullptr, nullptr, nullptr, &short_range_cutoff, &long_range_cutoff);
}

void PairSO3LRTurboHip::coeff(int narg, char **arg)
{
  if (!allocated) allocate();
  if (narg != atom->ntypes + 2 || std::strcmp(arg[0], "*") != 0 || std::strcmp(arg[1], "*") != 0)
    error->all(FLERR, "Pair coeff for so3lr/turbo must be '* * E1 ... Entypes'");
  type_z.assign(atom->ntypes + 1, 0);
  for (int t = 1; t <= atom->ntypes; ++t) {
    const int zt = so3lr_atomic_number(arg[t + 1]);
    if (zt == 0) error->all(FLERR, "Unknown SO3LR element '{}'", arg[t + 1]);
    type_z[t] = zt;
  }
  for (int i = 1; i <= atom->ntypes; ++i)
    for (int j = i; j <= atom->ntypes; ++j) setflag[i][j] = 1;
}

double PairSO3LRTurboHip::init_one(int i, int j)
{
  if (!setflag[i][j]) error->all(FLERR, "All so3lr/turbo coefficients are not set");
  return long_range_cutoff;
}

void PairSO3LRTurboHip::init_style()
{
  if (comm->nprocs != 1)
    error->universe_all(FLERR, "so3lr/turbo requires one MPI rank per LAMMPS partition");
  if (universe->nworlds != universe->nprocs || universe->nprocs < 2)
    error->universe_all(FLERR, "so3lr/turbo requires multiple one-rank partitions");
  if (domain->xperiodic || domain->yperiodic || domain->zperiodic)
    error->universe_all(FLERR, "so3lr/turbo requires non-periodic boundaries");
  if (!force->newton_pair) error->all(FLERR, "Pair style so3lr/turbo requires newton pair on");
  if (!broker) error->universe_all(FLERR, "SO3LR turbo broker was not initialized");
  if (type_z.size() != static_cast<std::size_t>(atom->ntypes) + 1)
    error->all(FLERR, "Pair style so3lr/turbo coefficients are missing");

  auto *sr = neighbor->add_request(this, NeighConst::REQ_FULL);
  sr->set_id(0);
  sr->set_cutoff(short_range_cutoff);
  auto *lr = neighbor->add_request(this);
  lr->set_id(1);
  lr->set_cutoff(long_range_cutoff);

  z.resize(atom->nlocal);
  for (int i = 0; i < atom->nlocal; ++i) z[i] = type_z[atom->type[i]];
  // collective: "Pair style so3lr/turbo image <k>: charge Q with
  // multiplicity M: <reason>" on every rank when any image is refused
  if (so3lr_turbo_check_images(static_cast<int64_t>(MPI_Comm_c2f(universe->uworld)), atom->nlocal,
                               z.data(), total_charge, multiplicity) != SO3LR_OK)
    error->universe_all(FLERR, so3lr_turbo_last_error(nullptr));
  utils::logmesg(lmp, "SO3LR turbo image {}: total charge {:g}, spin multiplicity {:g}\n",
                 universe->iworld, total_charge, multiplicity);
}

void PairSO3LRTurboHip::init_list(int which, NeighList *ptr)
{
  if (which == 0)
    list_sr = ptr;
  else if (which == 1)
    list_lr = ptr;
  else
    error->all(FLERR, "Unexpected so3lr/turbo neighbor-list ID");
}

void PairSO3LRTurboHip::compute(int eflag, int vflag)
{
  ev_init(eflag, vflag);
  if (vflag_atom) error->universe_all(FLERR, "so3lr/turbo does not provide per-atom virial");
  if (list_sr == nullptr || list_lr == nullptr)
    error->all(FLERR, "SO3LR turbo neighbor lists were not initialized");
  const int n = atom->nlocal;
  const bool changed = neighbor->ago == 0;
  if (changed) {
    snapshot(list_sr, ilist_sr, off_sr, neigh_sr);
    snapshot(list_lr, ilist_lr, off_lr, neigh_lr);
  }
  z.resize(n);
  x.resize(3 * static_cast<std::size_t>(n));
  f.resize(3 * static_cast<std::size_t>(n));
  ea.resize(n);
  for (int i = 0; i < n; ++i) {
    z[i] = type_z[atom->type[i]];
    for (int d = 0; d < 3; ++d) x[3 * static_cast<std::size_t>(i) + d] = atom->x[i][d];
  }
  double e = 0.0;
  if (so3lr_turbo_evaluate(broker, n, z.data(), x.data(), total_charge, multiplicity, changed ? 1 : 0,
                           SO3LR_LIST_FULL, static_cast<int64_t>(ilist_sr.size()), ilist_sr.data(),
                           off_sr.data(), neigh_sr.data(), static_cast<int64_t>(ilist_lr.size()),
                           ilist_lr.data(), off_lr.data(), neigh_lr.data(), f.data(),
                           eflag_atom ? ea.data() : nullptr, nullptr, nullptr, &e) != SO3LR_OK)
    error->universe_all(FLERR, std::string("SO3LR turbo LAMMPS evaluation failed: ") +
                                   so3lr_turbo_last_error(broker));
  for (int i = 0; i < n; ++i) {
    for (int d = 0; d < 3; ++d) atom->f[i][d] += f[3 * static_cast<std::size_t>(i) + d];
    if (eflag_atom) eatom[i] += ea[i];
  }
  if (eflag_global) eng_vdwl += e;
  // a turbo image has no ghost rows: the virial is LAMMPS's f.r sum
  if (vflag_fdotr) virial_fdotr_compute();
}
