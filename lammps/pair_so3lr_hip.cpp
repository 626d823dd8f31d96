/* ----------------------------------------------------------------------
   pair_style so3lr/native/mpi MODEL [charge [multiplicity]] on libso3lr_hip.

   Commands, argument meaning and messages follow PairSO3LRNativeMPI
   (source/so3lr-lammps-native/plugins/lammps/pair_so3lr_native_mpi.cpp):
   constructor flags :1058-1063, settings :1097-1137, coeff :1139-1160,
   init_one :1162-1172, init_style and the charge/spin setup :1174-1235,
   init_list :1237-1244, compute :1246-1978.  One LAMMPS rank drives one GPU;
   ghost rows come from LAMMPS's own communication (comm_modify cutoff >=
   long-range cutoff + skin) and the library folds them onto their owners,
   so no halo exchange runs between GPUs.
------------------------------------------------------------------------- */

#include "pair_so3lr_hip.h"

#include "atom.h"
#include "comm.h"
#include "domain.h"
#include "error.h"
#include "force.h"
#include "memory.h"
#include "neigh_list.h"
#include "neigh_request.h"
#include "neighbor.h"
#include "utils.h"

#include "so3lr_hip.h"

#include <cstring>
#include <unordered_map>

using namespace LAMMPS_NS;

PairSO3LRHip::PairSO3LRHip(LAMMPS *lmp) : Pair(lmp)
{
  manybody_flag = 1;
  one_coeff = 1;
  restartinfo = 0;
  single_enable = 0;
  no_virial_fdotr_compute = 1;    // the library returns the virial itself
}

PairSO3LRHip::~PairSO3LRHip()
{
  so3lr_destroy(ctx);
  if (allocated) {
    memory->destroy(setflag);
    memory->destroy(cutsq);
  }
}

void PairSO3LRHip::allocate()
{
  allocated = 1;
  const int n = atom->ntypes;
  memory->create(setflag, n + 1, n + 1, "so3lr/native/mpi:setflag");
  memory->create(cutsq, n + 1, n + 1, "so3lr/native/mpi:cutsq");
  for (int i = 1; i <= n; ++i)
    for (int j = i; j <= n; ++j) setflag[i][j] = 0;
}

void PairSO3LRHip::settings(int narg, char **arg)
{
  if (narg < 1 || narg > 3)
    error->all(FLERR,
               "Illegal pair_style so3lr/native/mpi command: expected "
               "'pair_style so3lr/native/mpi MODEL [charge [multiplicity]]'");
  model_path = arg[0];
  total_charge = narg > 1 ? utils::numeric(FLERR, arg[1], false, lmp) : 0.0;
  multiplicity = narg > 2 ? utils::numeric(FLERR, arg[2], false, lmp) : 1.0;
  so3lr_destroy(ctx);
  ctx = nullptr;
  z_owned.clear();    // a new context holds no system yet
  // the library's message reads "Cannot initialize MPI-native SO3LR model:
  // <reason>", the reference's own wording
  if (so3lr_create(model_path.c_str(), 0, &ctx) != SO3LR_OK)
    error->all(FLERR, "{}", so3lr_last_error(nullptr));
  short_range_cutoff = so3lr_cutoff(ctx, 0);
  long_range_cutoff = so3lr_cutoff(ctx, 1);
}

void PairSO3LRHip::coeff(int narg, char **arg)
{
  if (!allocated) allocate();
  if (narg != atom->ntypes + 2 || std::strcmp(arg[0], "*") != 0 || std::strcmp(arg[1], "*") != 0)
    error->all(FLERR,
               "Pair coeff for so3lr/native/mpi must be '* * E1 ... Entypes' "
               "where each E is an element symbol or atomic number");
  type_z.assign(atom->ntypes + 1, 0);
  for (int t = 1; t <= atom->ntypes; ++t) {
    const int z = so3lr_atomic_number(arg[t + 1]);
    if (z == 0)
      error->all(FLERR,
                 "Unknown SO3LR element '{}'; use a symbol or atomic number "
                 "from H/1 through Es/99",
                 arg[t + 1]);
    type_z[t] = z;
  }
  for (int i = 1; i <= atom->ntypes; ++i)
    for (int j = i; j <= atom->ntypes; ++j) setflag[i][j] = 1;
}

double PairSO3LRHip::init_one(int i, int j)
{
  if (!setflag[i][j]) error->all(FLERR, "All so3lr/native/mpi coefficients are not set");
  // the default (full) list carries the short-range cutoff; the half list
  // requested in init_style carries the long-range one
  return short_range_cutoff;
}

void PairSO3LRHip::init_style()
{
  if (!force->newton_pair) error->all(FLERR, "Pair style so3lr/native/mpi requires newton pair on");
  if (!ctx) error->all(FLERR, "Pair style so3lr/native/mpi model was not initialized");
  if (type_z.size() != static_cast<std::size_t>(atom->ntypes) + 1)
    error->all(FLERR, "Pair style so3lr/native/mpi coefficients are missing");
  if (comm->nprocs != 1)
    error->all(FLERR,
               "Pair style so3lr/native/mpi on libso3lr_hip runs one MPI rank per GPU "
               "(got {} ranks)",
               comm->nprocs);
  if (comm->get_comm_cutoff() < long_range_cutoff + neighbor->skin)
    error->all(FLERR,
               "Pair style so3lr/native/mpi needs comm_modify cutoff >= {:g} "
               "(long-range cutoff + skin)",
               long_range_cutoff + neighbor->skin);
  set_system();

  auto *sr = neighbor->add_request(this, NeighConst::REQ_FULL);
  sr->set_id(0);
  sr->set_cutoff(short_range_cutoff);
  auto *lr = neighbor->add_request(this);
  lr->set_id(1);
  lr->set_cutoff(long_range_cutoff);

  if (comm->me == 0) {
    utils::logmesg(lmp, "SO3LR: total charge {:g}, spin multiplicity {:g}\n", total_charge,
                   multiplicity);
    if (total_charge != 0.0 && (domain->xperiodic || domain->yperiodic || domain->zperiodic))
      error->warning(FLERR,
                     "SO3LR: net charge {:g} in a periodic cell. SO3LR's long range is "
                     "truncated real-space Coulomb, so the energy is defined, but there is "
                     "no neutralizing background",
                     total_charge);
  }
}

// The owned atoms' elements and the global (Q, M); the library checks (Q, M)
// against the composition and builds the charge/spin embedding.  Sent again
// only when LAMMPS has reordered or exchanged the owned atoms.
void PairSO3LRHip::set_system()
{
  const int nlocal = atom->nlocal;
  std::vector<int32_t> z(nlocal);
  for (int i = 0; i < nlocal; ++i) z[i] = type_z[atom->type[i]];
  if (z == z_owned && !z_owned.empty()) return;
  if (so3lr_set_system(ctx, nlocal, z.data(), total_charge, multiplicity) != SO3LR_OK)
    error->all(FLERR, "Pair style so3lr/native/mpi: {}", so3lr_last_error(ctx));
  z_owned.swap(z);
  topology_stale = true;    // a new system needs its topology again
}

void PairSO3LRHip::init_list(int which, NeighList *ptr)
{
  if (which == 0)
    list_sr = ptr;
  else if (which == 1)
    list_lr = ptr;
  else
    error->all(FLERR, "Unexpected so3lr/native/mpi neighbor-list ID");
}

// At each reneighbor: the owner of every row (ghost rows folded onto the
// owned atom with the same tag, as the one-rank collapse of
// pair_so3lr_native.cpp:74-146 does) and both lists as LAMMPS built them.
void PairSO3LRHip::upload_topology()
{
  set_system();
  const int nlocal = atom->nlocal, nall = nlocal + atom->nghost;
  std::unordered_map<tagint, int> local_of_tag;
  local_of_tag.reserve(nlocal);
  for (int i = 0; i < nlocal; ++i)
    if (!local_of_tag.emplace(atom->tag[i], i).second)
      error->all(FLERR, "SO3LR MPI-native LAMMPS evaluation failed: duplicate locally owned atom tag");
  owner.resize(nall);
  for (int i = 0; i < nlocal; ++i) owner[i] = i;
  for (int i = nlocal; i < nall; ++i) {
    const auto found = local_of_tag.find(atom->tag[i]);
    if (found == local_of_tag.end())
      error->all(FLERR, "SO3LR MPI-native LAMMPS evaluation failed: ghost tag has no owner");
    if (type_z[atom->type[i]] != z_owned[found->second])
      error->all(FLERR,
                 "SO3LR MPI-native LAMMPS evaluation failed: periodic image element differs "
                 "from owner");
    owner[i] = found->second;
  }
  auto snapshot = [](NeighList *l, std::vector<int32_t> &il, std::vector<int64_t> &off,
                     std::vector<int32_t> &nb) {
    il.assign(l->ilist, l->ilist + l->inum);
    off.assign(1, 0);
    nb.clear();
    for (int ii = 0; ii < l->inum; ++ii) {
      const int i = l->ilist[ii];
      const int *jlist = l->firstneigh[i];
      for (int jj = 0; jj < l->numneigh[i]; ++jj) nb.push_back(jlist[jj] & NEIGHMASK);
      off.push_back(static_cast<int64_t>(nb.size()));
    }
  };
  snapshot(list_sr, ilist_sr, off_sr, neigh_sr);
  snapshot(list_lr, ilist_lr, off_lr, neigh_lr);
  if (so3lr_set_topology(ctx, nall, owner.data(), SO3LR_LIST_FULL,
                         static_cast<int64_t>(ilist_sr.size()), ilist_sr.data(), off_sr.data(),
                         neigh_sr.data(), static_cast<int64_t>(ilist_lr.size()), ilist_lr.data(),
                         off_lr.data(), neigh_lr.data()) != SO3LR_OK)
    error->all(FLERR, "SO3LR MPI-native LAMMPS evaluation failed: {}", so3lr_last_error(ctx));
  topology_stale = false;
}

void PairSO3LRHip::compute(int eflag, int vflag)
{
  ev_init(eflag, vflag);
  if (list_sr == nullptr || list_lr == nullptr)
    error->all(FLERR, "SO3LR MPI neighbor lists were not initialized");
  if (neighbor->ago == 0 || topology_stale) upload_topology();
  const int nlocal = atom->nlocal;
  f_owned.resize(3 * static_cast<std::size_t>(nlocal));
  e_owned.resize(nlocal);
  int flags = SO3LR_ENERGY | SO3LR_VIRIAL;
  if (eflag_atom) flags |= SO3LR_EATOM;
  double e = 0.0, w[6] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
  // rows 0..nall-1 of atom->x (one contiguous block): owned, then ghosts
  if (so3lr_compute(ctx, &atom->x[0][0], flags, f_owned.data(), eflag_atom ? e_owned.data() : nullptr,
                    &e, w) != SO3LR_OK)
    error->all(FLERR, "SO3LR MPI-native LAMMPS evaluation failed: {}", so3lr_last_error(ctx));
  double **f = atom->f;
  for (int i = 0; i < nlocal; ++i)
    for (int d = 0; d < 3; ++d) f[i][d] += f_owned[3 * static_cast<std::size_t>(i) + d];
  if (eflag_global) eng_vdwl += e;
  if (eflag_atom)
    for (int i = 0; i < nlocal; ++i) eatom[i] += e_owned[i];
  if (vflag_global)
    for (int c = 0; c < 6; ++c) virial[c] += w[c];    // xx yy zz xy xz yz
  if (vflag_atom) {
    // an addition: the reference refuses per-atom virial (:1248-1251).  Each
    // pair's term goes half to each endpoint, ghosts already folded onto
    // their owners.
    v_owned.resize(6 * static_cast<std::size_t>(nlocal));
    if (so3lr_last_vatom(ctx, v_owned.data(), 0) != SO3LR_OK)
      error->all(FLERR, "SO3LR MPI-native LAMMPS evaluation failed: {}", so3lr_last_error(ctx));
    for (int i = 0; i < nlocal; ++i)
      for (int c = 0; c < 6; ++c) vatom[i][c] += v_owned[6 * static_cast<std::size_t>(i) + c];
  }
}
