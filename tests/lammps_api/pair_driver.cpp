// Test infrastructure: drives the thin LAMMPS pair style of lammps/ (compiled
// against the API subset in this directory) through a ctypes-callable C
// interface.  The caller supplies what LAMMPS would hold at each step -- the
// rows (owned atoms, then ghosts) with their tags and types, the full
// short-range and half long-range lists, neighbor->ago -- and reads back
// the forces, energies and virial the style added.  Not LAMMPS: the rows and
// lists come from the LAMMPS stand-in (libso3lr_lammps_emu.so).

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

#include "pair_so3lr_hip.h"

#include <cstring>
#include <memory>
#include <string>
#include <vector>

using namespace LAMMPS_NS;

// ---- the out-of-line parts of the API subset ----
Pair::~Pair() {
  delete[] eatom;
  if (vatom) {
    delete[] vatom[0];
    delete[] vatom;
  }
}

void Pair::ev_init(int eflag, int vflag) {
  eflag_global = eflag & 1;
  eflag_atom = eflag & 2;
  eflag_either = eflag_global || eflag_atom;
  vflag_global = vflag & 3;
  vflag_atom = vflag & 4;
  vflag_fdotr = (vflag & 2) && !no_virial_fdotr_compute;
  vflag_either = vflag_global || vflag_atom;
  eng_vdwl = eng_coul = 0.0;
  for (double &v : virial) v = 0.0;
  const int n = atom->nlocal + atom->nghost;
  if (eflag_atom) {
    if (n > maxeatom) {
      delete[] eatom;
      eatom = new double[n];
      maxeatom = n;
    }
    for (int i = 0; i < n; ++i) eatom[i] = 0.0;
  }
  if (vflag_atom) {
    if (n > maxvatom) {
      if (vatom) {
        delete[] vatom[0];
        delete[] vatom;
      }
      double *data = new double[6 * static_cast<std::size_t>(n)];
      vatom = new double *[n];
      for (int i = 0; i < n; ++i) vatom[i] = data + 6 * static_cast<std::size_t>(i);
      maxvatom = n;
    }
    for (int i = 0; i < n; ++i)
      for (int c = 0; c < 6; ++c) vatom[i][c] = 0.0;
  }
}

void Pair::virial_fdotr_compute() {
  const int n = atom->nlocal + atom->nghost;
  for (int i = 0; i < n; ++i) {
    const double *x = atom->x[i], *f = atom->f[i];
    virial[0] += f[0] * x[0];
    virial[1] += f[1] * x[1];
    virial[2] += f[2] * x[2];
    virial[3] += f[1] * x[0];
    virial[4] += f[2] * x[0];
    virial[5] += f[2] * x[1];
  }
}

NeighRequest *Neighbor::add_request(Pair *, int flags) {
  requests.push_back(new NeighRequest());
  requests.back()->full = (flags & NeighConst::REQ_FULL) ? 1 : 0;
  request_flags.push_back(flags);
  return requests.back();
}

std::string &utils::log_text() {
  static std::string text;
  return text;
}

// ---- the driver ----
namespace {
struct List {
  NeighList list;
  std::vector<int> ilist, numneigh, neigh;
  std::vector<int *> first;
};

struct Driver {
  LAMMPS lmp;
  Memory memory;
  Error error;
  Universe universe;
  Atom atom;
  Neighbor neighbor;
  Comm comm;
  Domain domain;
  Force force;
  std::unique_ptr<PairSO3LRHip> pair;
  std::vector<double> x, f;
  std::vector<tagint> tag;
  std::vector<int> type;
  std::vector<double *> xrow, frow;
  List lists[2];
  std::string message;

  Driver() {
    lmp.memory = &memory;
    lmp.error = &error;
    lmp.universe = &universe;
    lmp.atom = &atom;
    lmp.neighbor = &neighbor;
    lmp.comm = &comm;
    lmp.domain = &domain;
    lmp.force = &force;
    pair = std::make_unique<PairSO3LRHip>(&lmp);
  }
  ~Driver() {
    pair.reset();
    for (NeighRequest *r : neighbor.requests) delete r;
  }
};

// Run one command of the style; a LAMMPS abort becomes status 1 and its text.
template <class F> int run(Driver *d, F &&body) {
  try {
    body();
    d->message.clear();
    return 0;
  } catch (const std::exception &e) {
    d->message = e.what();
    return 1;
  }
}

std::vector<char *> argv(int narg, const char *const *args, std::vector<std::string> &keep) {
  keep.assign(args, args + narg);
  std::vector<char *> v;
  for (std::string &s : keep) v.push_back(&s[0]);
  return v;
}
}    // namespace

extern "C" {

void *pd_create(int ntypes, int newton_pair, int nprocs, double comm_cutoff, double skin, const int *periodic) {
  auto *d = new Driver();
  d->atom.ntypes = ntypes;
  d->force.newton_pair = newton_pair;
  d->comm.nprocs = nprocs;
  d->comm.cutghostuser = comm_cutoff;
  d->neighbor.skin = skin;
  d->domain.xperiodic = periodic[0];
  d->domain.yperiodic = periodic[1];
  d->domain.zperiodic = periodic[2];
  return d;
}

void pd_destroy(void *h) { delete static_cast<Driver *>(h); }

const char *pd_message(void *h) { return static_cast<Driver *>(h)->message.c_str(); }

int pd_warnings(void *h) { return int(static_cast<Driver *>(h)->error.warnings.size()); }

const char *pd_warning(void *h, int k) { return static_cast<Driver *>(h)->error.warnings[k].c_str(); }

const char *pd_log() { return utils::log_text().c_str(); }

int pd_settings(void *h, int narg, const char *const *args) {
  auto *d = static_cast<Driver *>(h);
  std::vector<std::string> keep;
  std::vector<char *> v = argv(narg, args, keep);
  return run(d, [&] { d->pair->settings(narg, v.data()); });
}

int pd_coeff(void *h, int narg, const char *const *args) {
  auto *d = static_cast<Driver *>(h);
  std::vector<std::string> keep;
  std::vector<char *> v = argv(narg, args, keep);
  return run(d, [&] { d->pair->coeff(narg, v.data()); });
}

// As Pair::init does before it calls init_one: no coefficients, no call.
int pd_init_one(void *h, int i, int j, double *cut) {
  auto *d = static_cast<Driver *>(h);
  return run(d, [&] {
    if (!d->pair->allocated) d->error.all(FLERR, "All pair coeffs are not set");
    *cut = d->pair->init_one(i, j);
  });
}

// The owned atoms (nlocal), the rows that follow them (nghost), one tag and
// type per row; positions are set by pd_positions.
int pd_set_atoms(void *h, int nlocal, int nghost, const int *tag, const int *type) {
  auto *d = static_cast<Driver *>(h);
  const int n = nlocal + nghost;
  d->atom.nlocal = nlocal;
  d->atom.nghost = nghost;
  d->tag.assign(tag, tag + n);
  d->type.assign(type, type + n);
  d->x.assign(3 * static_cast<std::size_t>(n), 0.0);
  d->f.assign(3 * static_cast<std::size_t>(n), 0.0);
  d->xrow.resize(n);
  d->frow.resize(n);
  for (int i = 0; i < n; ++i) {
    d->xrow[i] = &d->x[3 * static_cast<std::size_t>(i)];
    d->frow[i] = &d->f[3 * static_cast<std::size_t>(i)];
  }
  d->atom.tag = d->tag.data();
  d->atom.type = d->type.data();
  d->atom.x = d->xrow.data();
  d->atom.f = d->frow.data();
  return 0;
}

int pd_positions(void *h, const double *x) {
  auto *d = static_cast<Driver *>(h);
  std::memcpy(d->x.data(), x, d->x.size() * sizeof(double));
  return 0;
}

int pd_init_style(void *h) {
  auto *d = static_cast<Driver *>(h);
  return run(d, [&] {
    d->pair->init_style();
    // what Neighbor::init does with the requests: hand each its list
    for (std::size_t k = 0; k < d->neighbor.requests.size(); ++k)
      d->pair->init_list(d->neighbor.requests[k]->id, &d->lists[d->neighbor.requests[k]->id == 1 ? 1 : 0].list);
  });
}

// Request k of the last init_style: its id, full flag and cutoff.
int pd_request(void *h, int k, int *id, int *full, double *cutoff) {
  auto *d = static_cast<Driver *>(h);
  if (k < 0 || k >= int(d->neighbor.requests.size())) return 1;
  *id = d->neighbor.requests[k]->id;
  *full = d->neighbor.requests[k]->full;
  *cutoff = d->neighbor.requests[k]->cut ? d->neighbor.requests[k]->cutoff : -1.0;
  return 0;
}

// List `which` (0 full short range, 1 half long range) in the CSR form of
// the stand-in: inum receivers, offsets[inum + 1], neighbour rows.
int pd_set_list(void *h, int which, int inum, const int *ilist, const int64_t *offsets, const int *neigh) {
  auto *d = static_cast<Driver *>(h);
  List &L = d->lists[which];
  const int n = d->atom.nlocal + d->atom.nghost;
  L.ilist.assign(ilist, ilist + inum);
  L.numneigh.assign(n, 0);
  L.neigh.assign(neigh, neigh + (inum ? offsets[inum] : 0));
  L.first.assign(n, nullptr);
  for (int k = 0; k < inum; ++k) {
    L.numneigh[ilist[k]] = int(offsets[k + 1] - offsets[k]);
    L.first[ilist[k]] = L.neigh.data() + offsets[k];
  }
  L.list.inum = inum;
  L.list.ilist = L.ilist.data();
  L.list.numneigh = L.numneigh.data();
  L.list.firstneigh = L.first.data();
  return 0;
}

// One force evaluation as Verlet runs it: forces cleared, then pair->compute.
int pd_compute(void *h, int ago, int eflag, int vflag, double *f_owned, double *eatom, double *vatom,
               double *energy, double *virial) {
  auto *d = static_cast<Driver *>(h);
  d->neighbor.ago = ago;
  std::fill(d->f.begin(), d->f.end(), 0.0);
  return run(d, [&] {
    d->pair->compute(eflag, vflag);
    const int n = d->atom.nlocal;
    std::memcpy(f_owned, d->f.data(), 3 * static_cast<std::size_t>(n) * sizeof(double));
    if (eatom && d->pair->eflag_atom) std::memcpy(eatom, d->pair->eatom, n * sizeof(double));
    if (vatom && d->pair->vflag_atom)
      for (int i = 0; i < n; ++i)
        for (int c = 0; c < 6; ++c) vatom[6 * i + c] = d->pair->vatom[i][c];
    *energy = d->pair->eng_vdwl;
    for (int c = 0; c < 6; ++c) virial[c] = d->pair->virial[c];
  });
}

}    // extern "C"
