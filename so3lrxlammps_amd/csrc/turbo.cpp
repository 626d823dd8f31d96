// MPI broker of independent images onto one GPU (declared in
// include/so3lr_turbo.h).
//
// One call moves, per image: a small header (one MPI_Gather), the positions
// with (Q, M) and the atomic numbers (two MPI_Gatherv), the candidate lists
// only when some image reneighboured (one MPI_Gatherv of int64), one status
// broadcast, and one packed result block per image (one MPI_Scatterv).  The
// coordinator keeps the packed system between calls and calls
// so3lr_set_images / so3lr_set_topology only when the composition, (Q, M) or
// the lists change; otherwise a call is so3lr_compute on the new positions.
// The reference's broker (src/mpi_turbo_replica_broker.cpp:130-305) instead
// gathers every image's exact-cutoff edge vectors and uploads a fresh packed
// graph on every call.
#include "../../include/so3lr_turbo.h"
#include "../../include/so3lr_hip.h"

#include <mpi.h>

#include <climits>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

thread_local std::string g_error;
bool g_initialized_mpi = false;

// A failure with a status code; raised on the coordinator, returned on every rank.
struct Failure : std::runtime_error {
  int code;
  Failure(int c, const std::string &m) : std::runtime_error(m), code(c) {}
};

std::string num(double v) {
  char buf[64];
  std::snprintf(buf, sizeof(buf), "%.17g", v);
  return buf;
}

// Why the image's CSR list is unusable (empty when it is fine): every row an
// owned atom of the image and no self pair (pair_so3lr_turbo.cpp:53-73 refuses
// graphs that are not isolated owned graphs; kokkos_turbo_replica_bridge.cpp:
// 44-53 refuses self pairs).
std::string list_problem(const char *name, int64_t n, int64_t inum, const int32_t *il, const int64_t *off,
                         const int32_t *nb) {
  const std::string w = std::string(name) + " list: ";
  if (inum < 0 || inum > n) return w + "inum outside 0..n";
  if (inum == 0) return {};
  if (!il || !off) return w + "missing ilist or offsets";
  if (off[0] != 0) return w + "offsets[0] must be 0";
  for (int64_t k = 0; k < inum; ++k)
    if (off[k + 1] < off[k]) return w + "offsets decrease";
  if (off[inum] > 0 && !nb) return w + "missing neighbour array";
  for (int64_t k = 0; k < inum; ++k) {
    const int32_t i = il[k];
    if (i < 0 || i >= n) return w + "ilist entry outside the image's atoms";
    for (int64_t e = off[k]; e < off[k + 1]; ++e) {
      if (nb[e] < 0 || nb[e] >= n)
        return w + "neighbour row outside the image's owned atoms (a turbo image has no ghost rows)";
      if (nb[e] == i) return w + "an atom is its own neighbour";
    }
  }
  return {};
}

// Header of one image, gathered on every call.
enum { H_OK, H_N, H_CHANGED, H_KIND, H_SR_INUM, H_SR_NNZ, H_LR_INUM, H_LR_NNZ, H_SIZE };

// Broadcast a status and its message from `root`; returns the status, with
// the message in `out` on every rank.
int share_status(MPI_Comm comm, int root, int code, const std::string &mine, std::string &out) {
  int64_t st[2] = {code, code == SO3LR_OK ? 0 : int64_t(mine.size())};
  MPI_Bcast(st, 2, MPI_INT64_T, root, comm);
  out.clear();
  if (st[0] != SO3LR_OK && st[1] > 0) {
    std::vector<char> buf(static_cast<std::size_t>(st[1]));
    int rank = 0;
    MPI_Comm_rank(comm, &rank);
    if (rank == root) std::memcpy(buf.data(), mine.data(), buf.size());
    MPI_Bcast(buf.data(), int(st[1]), MPI_CHAR, root, comm);
    out.assign(buf.data(), buf.size());
  }
  return int(st[0]);
}

// Counts and displacements of one gathered buffer (coordinator side).
struct Layout {
  std::vector<int> cnt, dsp;
  bool fits = true;  // every count and the total fit MPI's int
  template <class F>
  void set(int size, F &&per) {
    cnt.assign(std::size_t(size), 0);
    dsp.assign(std::size_t(size), 0);
    int64_t at = 0;
    fits = true;
    for (int k = 0; k < size; ++k) {
      const int64_t c = per(k);
      if (c < 0 || c > INT_MAX || at > INT_MAX) fits = false;
      cnt[k] = int(c);
      dsp[k] = int(at);
      at += c;
    }
    if (at > INT_MAX) fits = false;
  }
  int64_t total() const { return cnt.empty() ? 0 : int64_t(dsp.back()) + cnt.back(); }
};

}  // namespace

struct so3lr_turbo {
  MPI_Comm comm = MPI_COMM_NULL;
  int rank = -1, size = 0, coord = 0;
  so3lr_ctx *ctx = nullptr;  // coordinator only
  double sr_cut = 0.0, lr_cut = 0.0;
  std::string error;

  // coordinator: the packed system, kept between calls
  bool full = true;  // the next call sets images and topology from scratch
  std::vector<int64_t> hdr, prev_hdr;
  Layout lay_d, lay_z, lay_l, lay_o;
  std::vector<double> xin;         // gathered [x (3 n), Q, M] per image
  std::vector<int32_t> zin;        // gathered atomic numbers
  std::vector<int64_t> lists_in;   // gathered lists
  std::vector<int64_t> node_off;   // image k: rows node_off[k] .. node_off[k + 1]
  std::vector<int32_t> z_all;
  std::vector<double> qm_all;
  std::vector<int32_t> owner, sr_il, sr_nb, lr_il, lr_nb;
  std::vector<int64_t> sr_off, lr_off;
  int sr_kind = SO3LR_LIST_FULL;
  std::vector<double> x_all, f_all, e_all, q_all, h_all, img_e, out;

  // every rank
  std::vector<double> send_d, recv_d;
  std::vector<int64_t> send_l;

  // figures of the last call
  int64_t packed = 0, images = 0;
  int gathered = 0;
  double t_gather = 0.0, t_eval = 0.0, t_scatter = 0.0, t_total = 0.0;

  bool coordinator() const { return rank == coord; }
  void run_packed(bool need_lists);
};

// The packed evaluation on the coordinator (KokkosTurboReplicaBridge::evaluate,
// kokkos_turbo_replica_bridge.cpp:64-179): image k's atoms are rows
// node_off[k] .. node_off[k + 1] of one system with per-image (Q, M), and its
// list rows are shifted by node_off[k].
void so3lr_turbo::run_packed(bool need_lists) {
  const std::size_t S = std::size_t(size);
  std::vector<int64_t> off(S + 1, 0);
  for (std::size_t k = 0; k < S; ++k) off[k + 1] = off[k] + hdr[k * H_SIZE + H_N];
  const int64_t N = off[S];
  std::vector<double> qm(2 * S);
  x_all.resize(std::size_t(3 * N));
  for (std::size_t k = 0; k < S; ++k) {
    const int64_t nk = off[k + 1] - off[k];
    const double *blk = xin.data() + lay_d.dsp[k];
    std::memcpy(x_all.data() + 3 * off[k], blk, sizeof(double) * std::size_t(3 * nk));
    qm[2 * k] = blk[3 * nk];
    qm[2 * k + 1] = blk[3 * nk + 1];
  }
  const bool images_changed = full || off != node_off || zin != z_all || qm != qm_all;
  if (images_changed) {
    full = true;  // until this call succeeds
    for (std::size_t k = 0; k < S; ++k) {
      const int rc = so3lr_check_system(off[k + 1] - off[k], zin.data() + off[k], qm[2 * k], qm[2 * k + 1]);
      if (rc != SO3LR_OK)
        throw Failure(rc, "image " + std::to_string(k) + ": charge " + num(qm[2 * k]) + " with multiplicity " +
                              num(qm[2 * k + 1]) + ": " + so3lr_last_error(nullptr));
    }
    std::vector<double> q(S), m(S);
    for (std::size_t k = 0; k < S; ++k) q[k] = qm[2 * k], m[k] = qm[2 * k + 1];
    const int rc = so3lr_set_images(ctx, N, zin.data(), int64_t(S), off.data(), q.data(), m.data());
    if (rc != SO3LR_OK) throw Failure(rc, so3lr_last_error(ctx));
    node_off = off;
    z_all = zin;
    qm_all = qm;
  }
  if (need_lists) {
    // per image [sr ilist, sr offsets, sr neigh, lr ilist, lr offsets, lr neigh]
    sr_il.clear(), sr_nb.clear(), lr_il.clear(), lr_nb.clear();
    sr_off.assign(1, 0), lr_off.assign(1, 0);
    for (std::size_t k = 0; k < S; ++k) {
      const int64_t *h = hdr.data() + k * H_SIZE;
      const int64_t base = off[k];
      const int64_t *p = lists_in.data() + lay_l.dsp[k];
      auto take = [&](int64_t inum, int64_t nnz, std::vector<int32_t> &il, std::vector<int64_t> &of,
                      std::vector<int32_t> &nb) {
        const int64_t e0 = of.back();
        for (int64_t i = 0; i < inum; ++i) il.push_back(int32_t(p[i] + base));
        p += inum;
        for (int64_t i = 1; i <= inum; ++i) of.push_back(e0 + p[i]);
        p += inum + 1;
        for (int64_t e = 0; e < nnz; ++e) nb.push_back(int32_t(p[e] + base));
        p += nnz;
      };
      take(h[H_SR_INUM], h[H_SR_NNZ], sr_il, sr_off, sr_nb);
      take(h[H_LR_INUM], h[H_LR_NNZ], lr_il, lr_off, lr_nb);
    }
    sr_kind = int(hdr[H_KIND]);
  }
  if (images_changed || need_lists) {
    owner.resize(std::size_t(N));
    for (int64_t i = 0; i < N; ++i) owner[i] = int32_t(i);
    const int rc = so3lr_set_topology(ctx, N, owner.data(), sr_kind, int64_t(sr_il.size()), sr_il.data(),
                                      sr_off.data(), sr_nb.data(), int64_t(lr_il.size()), lr_il.data(),
                                      lr_off.data(), lr_nb.data());
    if (rc != SO3LR_OK) throw Failure(rc, so3lr_last_error(ctx));
  }
  f_all.resize(std::size_t(3 * N));
  e_all.resize(std::size_t(N));
  q_all.resize(std::size_t(N));
  h_all.resize(std::size_t(N));
  img_e.resize(S);
  double etot = 0.0;
  int rc = so3lr_compute(ctx, x_all.data(), SO3LR_ENERGY | SO3LR_EATOM, f_all.data(), e_all.data(), &etot, nullptr);
  if (rc != SO3LR_OK) throw Failure(rc, so3lr_last_error(ctx));
  rc = so3lr_last_terms(ctx, nullptr, nullptr, nullptr, q_all.data(), h_all.data(), nullptr, img_e.data());
  if (rc != SO3LR_OK) throw Failure(rc, so3lr_last_error(ctx));
  // one result block per image: [energy, f (3 n), eatom, charges, hirshfeld]
  lay_o.set(size, [&](int k) { return 1 + 6 * (off[k + 1] - off[k]); });
  out.resize(std::size_t(lay_o.total()));
  for (std::size_t k = 0; k < S; ++k) {
    const int64_t a = off[k], nk = off[k + 1] - off[k];
    double *o = out.data() + lay_o.dsp[k];
    o[0] = img_e[k];
    std::memcpy(o + 1, f_all.data() + 3 * a, sizeof(double) * std::size_t(3 * nk));
    std::memcpy(o + 1 + 3 * nk, e_all.data() + a, sizeof(double) * std::size_t(nk));
    std::memcpy(o + 1 + 4 * nk, q_all.data() + a, sizeof(double) * std::size_t(nk));
    std::memcpy(o + 1 + 5 * nk, h_all.data() + a, sizeof(double) * std::size_t(nk));
  }
  full = false;
  packed = N;
  images = int64_t(S);
}

extern "C" {

int so3lr_turbo_mpi_world(int64_t *comm_f, int *rank, int *size) {
  int init = 0;
  MPI_Initialized(&init);
  if (!init) {
    if (MPI_Init(nullptr, nullptr) != MPI_SUCCESS) {
      g_error = "SO3LR turbo: MPI_Init failed";
      return SO3LR_ERR_DEVICE;
    }
    g_initialized_mpi = true;
  }
  if (comm_f) *comm_f = int64_t(MPI_Comm_c2f(MPI_COMM_WORLD));
  if (rank) MPI_Comm_rank(MPI_COMM_WORLD, rank);
  if (size) MPI_Comm_size(MPI_COMM_WORLD, size);
  return SO3LR_OK;
}

int so3lr_turbo_mpi_finalize(void) {
  int fin = 0;
  MPI_Finalized(&fin);
  if (g_initialized_mpi && !fin) MPI_Finalize();
  return SO3LR_OK;
}

int so3lr_turbo_check_images(int64_t comm_f, int64_t n, const int32_t *z, double total_charge,
                             double multiplicity) {
  const MPI_Comm comm = MPI_Comm_f2c(MPI_Fint(comm_f));
  int rank = 0;
  MPI_Comm_rank(comm, &rank);
  const int rc = so3lr_check_system(n, z, total_charge, multiplicity);
  std::string mine;
  if (rc != SO3LR_OK)
    mine = "Pair style so3lr/turbo image " + std::to_string(rank) + ": charge " + num(total_charge) +
           " with multiplicity " + num(multiplicity) + ": " + so3lr_last_error(nullptr);
  int bad = rc != SO3LR_OK ? rank : INT_MAX, first = INT_MAX;
  MPI_Allreduce(&bad, &first, 1, MPI_INT, MPI_MIN, comm);
  if (first == INT_MAX) return SO3LR_OK;
  return share_status(comm, first, rc, mine, g_error);
}

int so3lr_turbo_create(int64_t comm_f, int coordinator, const char *model_path, int device, so3lr_turbo **out) {
  if (!out) {
    g_error = "SO3LR turbo: null output handle";
    return SO3LR_ERR_ARGUMENT;
  }
  *out = nullptr;
  const MPI_Comm comm = MPI_Comm_f2c(MPI_Fint(comm_f));
  if (comm == MPI_COMM_NULL) {
    g_error = "SO3LR turbo broker communicator is null";
    return SO3LR_ERR_ARGUMENT;
  }
  auto *t = new so3lr_turbo();
  t->comm = comm;
  MPI_Comm_rank(comm, &t->rank);
  MPI_Comm_size(comm, &t->size);
  if (coordinator < 0 || coordinator >= t->size) {
    delete t;
    g_error = "SO3LR turbo coordinator rank is invalid";
    return SO3LR_ERR_ARGUMENT;
  }
  t->coord = coordinator;
  int rc = SO3LR_OK;
  std::string mine;
  if (t->coordinator()) {
    rc = model_path ? so3lr_create(model_path, device, &t->ctx) : SO3LR_ERR_ARGUMENT;
    if (rc != SO3LR_OK)
      mine = std::string("Cannot initialize the coordinator SO3LR model: ") +
             (model_path ? so3lr_last_error(nullptr) : "no model path");
  }
  rc = share_status(comm, coordinator, rc, mine, g_error);
  if (rc != SO3LR_OK) {
    if (t->ctx) so3lr_destroy(t->ctx);
    delete t;
    return rc;
  }
  double cut[2] = {0.0, 0.0};
  if (t->coordinator()) cut[0] = so3lr_cutoff(t->ctx, 0), cut[1] = so3lr_cutoff(t->ctx, 1);
  MPI_Bcast(cut, 2, MPI_DOUBLE, coordinator, comm);
  t->sr_cut = cut[0];
  t->lr_cut = cut[1];
  *out = t;
  return SO3LR_OK;
}

void so3lr_turbo_destroy(so3lr_turbo *t) {
  if (!t) return;
  if (t->ctx) so3lr_destroy(t->ctx);
  delete t;
}

const char *so3lr_turbo_last_error(const so3lr_turbo *t) { return t ? t->error.c_str() : g_error.c_str(); }

int so3lr_turbo_info(const so3lr_turbo *t, int *rank, int *size, int *coordinator, double *sr_cutoff,
                     double *lr_cutoff) {
  if (!t) return SO3LR_ERR_ARGUMENT;
  if (rank) *rank = t->rank;
  if (size) *size = t->size;
  if (coordinator) *coordinator = t->coord;
  if (sr_cutoff) *sr_cutoff = t->sr_cut;
  if (lr_cutoff) *lr_cutoff = t->lr_cut;
  return SO3LR_OK;
}

int so3lr_turbo_evaluate(so3lr_turbo *t, int64_t n, const int32_t *z, const double *x, double total_charge,
                         double multiplicity, int lists_changed, int sr_kind, int64_t sr_inum,
                         const int32_t *sr_ilist, const int64_t *sr_offsets, const int32_t *sr_neigh,
                         int64_t lr_inum, const int32_t *lr_ilist, const int64_t *lr_offsets,
                         const int32_t *lr_neigh, double *f, double *eatom, double *charges, double *hirshfeld,
                         double *energy) {
  if (!t) return SO3LR_ERR_ARGUMENT;  // no communicator to agree over
  const double t0 = MPI_Wtime();
  t->packed = t->images = 0;
  t->gathered = 0;
  t->t_eval = 0.0;

  // 1. this image's header; a malformed image sends zero sizes
  std::string why;
  if (n < 1 || n > INT_MAX / 8) why = "the image needs 1 .. 2^28 atoms";
  else if (!z || !x || !f) why = "missing atomic numbers, positions or force output";
  else if (sr_kind != SO3LR_LIST_FULL && sr_kind != SO3LR_LIST_HALF) why = "unknown short-range list kind";
  if (why.empty()) why = list_problem("SR", n, sr_inum, sr_ilist, sr_offsets, sr_neigh);
  if (why.empty()) why = list_problem("LR", n, lr_inum, lr_ilist, lr_offsets, lr_neigh);
  const bool ok = why.empty();
  int64_t h[H_SIZE] = {ok ? 1 : 0,
                       ok ? n : 0,
                       lists_changed ? 1 : 0,
                       ok ? sr_kind : -1,
                       ok ? sr_inum : 0,
                       ok && sr_inum > 0 ? sr_offsets[sr_inum] : 0,
                       ok ? lr_inum : 0,
                       ok && lr_inum > 0 ? lr_offsets[lr_inum] : 0};
  const bool coord = t->coordinator();
  if (coord) t->hdr.resize(std::size_t(t->size) * H_SIZE);
  MPI_Gather(h, H_SIZE, MPI_INT64_T, coord ? t->hdr.data() : nullptr, H_SIZE, MPI_INT64_T, t->coord, t->comm);

  // 2. the coordinator decides: the first malformed image, and whether the
  //    lists travel on this call
  int64_t ctl[2] = {-1, 0};
  std::string ctl_msg;
  if (coord) {
    const std::size_t S = std::size_t(t->size);
    bool need = t->full || t->prev_hdr.size() != t->hdr.size();
    for (std::size_t k = 0; k < S && ctl[0] < 0; ++k) {
      const int64_t *hk = t->hdr.data() + k * H_SIZE;
      if (!hk[H_OK]) ctl[0] = int64_t(k);
      else if (hk[H_KIND] != t->hdr[H_KIND]) {
        ctl[0] = int64_t(k);
        ctl_msg = "the short-range list kind differs from image 0's";
      }
      need = need || hk[H_CHANGED] || t->prev_hdr.empty() || t->prev_hdr[k * H_SIZE + H_N] != hk[H_N];
    }
    // gathered buffers must fit MPI's int counts
    if (ctl[0] < 0) {
      t->lay_d.set(t->size, [&](int k) { return 3 * t->hdr[k * H_SIZE + H_N] + 2; });
      t->lay_z.set(t->size, [&](int k) { return t->hdr[k * H_SIZE + H_N]; });
      t->lay_l.set(t->size, [&](int k) {
        const int64_t *hk = t->hdr.data() + std::size_t(k) * H_SIZE;
        return need ? 2 * hk[H_SR_INUM] + 1 + hk[H_SR_NNZ] + 2 * hk[H_LR_INUM] + 1 + hk[H_LR_NNZ] : 0;
      });
      t->lay_o.set(t->size, [&](int k) { return 1 + 6 * t->hdr[k * H_SIZE + H_N]; });
      if (!t->lay_d.fits || !t->lay_l.fits || !t->lay_o.fits) {
        ctl[0] = 0;
        ctl_msg = "the packed system exceeds MPI's int counts";
      }
    }
    ctl[1] = need ? 1 : 0;
  }
  MPI_Bcast(ctl, 2, MPI_INT64_T, t->coord, t->comm);
  if (ctl[0] >= 0) {
    // the reason travels from the rank that knows it
    const int root = ctl_msg.empty() ? int(ctl[0]) : t->coord;
    const std::string mine = t->rank == root ? (ctl_msg.empty() ? why : ctl_msg) : std::string();
    std::string reason;
    share_status(t->comm, root, SO3LR_ERR_TOPOLOGY, mine, reason);
    t->error = "SO3LR turbo broker received an invalid graph from image " + std::to_string(ctl[0]) + ": " + reason;
    if (coord) t->full = true;
    t->t_total = (MPI_Wtime() - t0) * 1e3;
    return SO3LR_ERR_TOPOLOGY;
  }
  const bool need_lists = ctl[1] != 0;

  // 3. positions with (Q, M), atomic numbers, and the lists when they travel
  t->send_d.resize(std::size_t(3 * n + 2));
  std::memcpy(t->send_d.data(), x, sizeof(double) * std::size_t(3 * n));
  t->send_d[3 * n] = total_charge;
  t->send_d[3 * n + 1] = multiplicity;
  if (coord) {
    t->xin.resize(std::size_t(t->lay_d.total()));
    t->zin.resize(std::size_t(t->lay_z.total()));
  }
  MPI_Gatherv(t->send_d.data(), int(3 * n + 2), MPI_DOUBLE, coord ? t->xin.data() : nullptr,
              coord ? t->lay_d.cnt.data() : nullptr, coord ? t->lay_d.dsp.data() : nullptr, MPI_DOUBLE, t->coord,
              t->comm);
  MPI_Gatherv(z, int(n), MPI_INT32_T, coord ? t->zin.data() : nullptr, coord ? t->lay_z.cnt.data() : nullptr,
              coord ? t->lay_z.dsp.data() : nullptr, MPI_INT32_T, t->coord, t->comm);
  if (need_lists) {
    std::vector<int64_t> &s = t->send_l;
    s.clear();
    auto put = [&](int64_t inum, const int32_t *il, const int64_t *of, const int32_t *nb) {
      for (int64_t i = 0; i < inum; ++i) s.push_back(il[i]);
      for (int64_t i = 0; i <= inum; ++i) s.push_back(inum > 0 ? of[i] : 0);
      const int64_t nnz = inum > 0 ? of[inum] : 0;
      for (int64_t e = 0; e < nnz; ++e) s.push_back(nb[e]);
    };
    put(sr_inum, sr_ilist, sr_offsets, sr_neigh);
    put(lr_inum, lr_ilist, lr_offsets, lr_neigh);
    if (coord) t->lists_in.resize(std::size_t(t->lay_l.total()));
    MPI_Gatherv(s.data(), int(s.size()), MPI_INT64_T, coord ? t->lists_in.data() : nullptr,
                coord ? t->lay_l.cnt.data() : nullptr, coord ? t->lay_l.dsp.data() : nullptr, MPI_INT64_T,
                t->coord, t->comm);
    t->gathered = 1;
  }
  const double t1 = MPI_Wtime();
  t->t_gather = (t1 - t0) * 1e3;

  // 4. the packed evaluation on the coordinator; its status on every rank
  int rc = SO3LR_OK;
  std::string mine;
  if (coord) {
    try {
      t->run_packed(need_lists);
      t->prev_hdr = t->hdr;
    } catch (const Failure &e) {
      rc = e.code;
      mine = e.what();
    } catch (const std::exception &e) {
      rc = SO3LR_ERR_DEVICE;
      mine = e.what();
    }
    if (rc != SO3LR_OK) t->full = true;
  }
  const double t2 = MPI_Wtime();
  if (coord) t->t_eval = (t2 - t1) * 1e3;
  std::string msg;
  rc = share_status(t->comm, t->coord, rc, mine, msg);
  if (rc != SO3LR_OK) {
    t->error = "SO3LR coordinator evaluation failed: " + msg;
    t->t_total = (MPI_Wtime() - t0) * 1e3;
    return rc;
  }

  // 5. this image's block back: [energy, f, eatom, charges, hirshfeld]
  t->recv_d.resize(std::size_t(1 + 6 * n));
  MPI_Scatterv(coord ? t->out.data() : nullptr, coord ? t->lay_o.cnt.data() : nullptr,
               coord ? t->lay_o.dsp.data() : nullptr, MPI_DOUBLE, t->recv_d.data(), int(1 + 6 * n), MPI_DOUBLE,
               t->coord, t->comm);
  const double *r = t->recv_d.data();
  if (energy) *energy = r[0];
  std::memcpy(f, r + 1, sizeof(double) * std::size_t(3 * n));
  if (eatom) std::memcpy(eatom, r + 1 + 3 * n, sizeof(double) * std::size_t(n));
  if (charges) std::memcpy(charges, r + 1 + 4 * n, sizeof(double) * std::size_t(n));
  if (hirshfeld) std::memcpy(hirshfeld, r + 1 + 5 * n, sizeof(double) * std::size_t(n));
  const double t3 = MPI_Wtime();
  t->t_scatter = (t3 - t2) * 1e3;
  t->t_total = (t3 - t0) * 1e3;
  t->error.clear();
  return SO3LR_OK;
}

int so3lr_turbo_stats(const so3lr_turbo *t, int64_t *packed_atoms, int64_t *images, int *lists_gathered,
                      double *gather_ms, double *evaluate_ms, double *scatter_ms, double *total_ms) {
  if (!t) return SO3LR_ERR_ARGUMENT;
  if (packed_atoms) *packed_atoms = t->packed;
  if (images) *images = t->images;
  if (lists_gathered) *lists_gathered = t->gathered;
  if (gather_ms) *gather_ms = t->t_gather;
  if (evaluate_ms) *evaluate_ms = t->t_eval;
  if (scatter_ms) *scatter_ms = t->t_scatter;
  if (total_ms) *total_ms = t->t_total;
  return SO3LR_OK;
}

}  // extern "C"
