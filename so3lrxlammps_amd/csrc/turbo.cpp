// MPI broker of independent images onto one GPU (declared in
// include/so3lr_turbo.h).
//
// Per call, point to point on a private duplicate of the caller's
// communicator: every worker posts its sends (a header; positions with (Q, M);
// atomic numbers; its candidate lists only when they changed since the
// coordinator last took them) and one receive for its result block, then
// waits politely (MPI_Testall with short sleeps), so idle workers leave the
// CPU to the coordinator and to the other images.  The coordinator receives
// the headers, then the data, evaluates all images as one packed system and
// answers each image with a status word and its block.  It keeps every
// image's lists between calls, and calls so3lr_set_images /
// so3lr_set_topology only when the composition, (Q, M) or some image's lists
// change; otherwise a call is so3lr_compute on the new positions.
//
// The reference's broker (src/mpi_turbo_replica_broker.cpp:130-305) runs a
// dozen blocking collectives per call and re-sends and re-uploads every
// image's exact-cutoff edge vectors each time; with MPICH's busy-polling
// collectives a box whose CPU share equals the number of images spends most of
// a step throttled.
#include "../../include/so3lr_turbo.h"
#include "../../include/so3lr_hip.h"

#include <mpi.h>
#include <sched.h>
#include <sys/prctl.h>
#include <time.h>

#include <climits>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

thread_local std::string g_error;
bool g_initialized_mpi = false;

// message tags on the broker's own communicator
enum { kTagHdr = 1, kTagX, kTagZ, kTagLists, kTagWhy, kTagRes, kTagMsg };

// A failure with a status code, found on the coordinator.
struct Failure : std::runtime_error {
  int code;
  Failure(int c, const std::string &m) : std::runtime_error(m), code(c) {}
};

std::string num(double v) {
  char buf[64];
  std::snprintf(buf, sizeof(buf), "%.17g", v);
  return buf;
}

// Complete the requests.  polite: sleep between tests (workers, whose wait
// covers the coordinator's GPU evaluation), with the thread's timer slack at
// 1 us for the wait (Linux's default 50 us slack makes a 20 us nap ~70 us);
// otherwise yield (the coordinator).
void settle(std::vector<MPI_Request> &reqs, bool polite) {
  if (reqs.empty()) return;
  int done = 0;
  for (int i = 0; i < 64 && !done; ++i) MPI_Testall(int(reqs.size()), reqs.data(), &done, MPI_STATUSES_IGNORE);
  if (!done) {
    const int slack = polite ? prctl(PR_GET_TIMERSLACK, 0, 0, 0, 0) : -1;
    if (slack > 0) prctl(PR_SET_TIMERSLACK, 1000UL, 0, 0, 0);
    const timespec nap{0, 20000};
    while (!done) {
      if (polite) nanosleep(&nap, nullptr);
      else sched_yield();
      MPI_Testall(int(reqs.size()), reqs.data(), &done, MPI_STATUSES_IGNORE);
    }
    if (slack > 0) prctl(PR_SET_TIMERSLACK, (unsigned long)slack, 0, 0, 0);
  }
  reqs.clear();
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
  if (off[inum] > int64_t(INT_MAX) / 4) return w + "too many neighbours";
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

// Header an image sends on every call.
enum { H_OK, H_N, H_LISTS, H_KIND, H_SR_INUM, H_SR_NNZ, H_LR_INUM, H_LR_NNZ, H_WHY, H_SIZE };
// Result block: status, resend-lists flag, message length, then (status OK)
// energy, f (3 n), eatom, charges, hirshfeld.
enum { R_STATUS, R_RESEND, R_MSGLEN, R_DATA };

int64_t lists_len(const int64_t *h) {
  return 2 * h[H_SR_INUM] + 1 + h[H_SR_NNZ] + 2 * h[H_LR_INUM] + 1 + h[H_LR_NNZ];
}

// Broadcast a status and its message from `root` (set-up calls only).
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

// The coordinator's copy of one image.
struct Image {
  int64_t hdr[H_SIZE] = {0};
  std::vector<double> xq;       // x (3 n), Q, M
  std::vector<int32_t> z;
  std::vector<int64_t> lists;   // [sr ilist, sr offsets, sr neigh, lr ilist, lr offsets, lr neigh]
  int64_t lists_hdr[H_SIZE] = {0};
  bool has_lists = false;
  std::vector<char> why;
  std::vector<double> res;      // result block
};

}  // namespace

struct so3lr_turbo {
  MPI_Comm comm = MPI_COMM_NULL;  // private duplicate
  int rank = -1, size = 0, coord = 0;
  so3lr_ctx *ctx = nullptr;       // coordinator only
  double sr_cut = 0.0, lr_cut = 0.0;
  std::string error;

  // worker side: whether the coordinator holds this image's current lists
  bool lists_synced = false;
  int64_t last_n = -1;
  std::vector<double> send_x, res;
  std::vector<int64_t> send_l;
  std::vector<MPI_Request> reqs;

  // coordinator side
  std::vector<Image> img;
  bool full = true;  // the next call sets images and topology from scratch
  std::vector<int64_t> node_off;
  std::vector<int32_t> z_all;
  std::vector<double> qm_all;
  std::vector<int32_t> owner, sr_il, sr_nb, lr_il, lr_nb;
  std::vector<int64_t> sr_off, lr_off;
  std::vector<double> x_all, f_all, e_all, q_all, h_all, img_e;

  // figures of the last call
  int64_t packed = 0, images = 0;
  int gathered = 0;
  double t_gather = 0.0, t_eval = 0.0, t_scatter = 0.0, t_total = 0.0;

  bool coordinator() const { return rank == coord; }
  void run_packed(bool lists_arrived);
};

// The packed evaluation on the coordinator (KokkosTurboReplicaBridge::evaluate,
// kokkos_turbo_replica_bridge.cpp:64-179): image k's atoms are rows
// node_off[k] .. node_off[k + 1] of one system with per-image (Q, M), and its
// list rows are shifted by node_off[k].
void so3lr_turbo::run_packed(bool lists_arrived) {
  const std::size_t S = std::size_t(size);
  std::vector<int64_t> off(S + 1, 0);
  for (std::size_t k = 0; k < S; ++k) off[k + 1] = off[k] + img[k].hdr[H_N];
  const int64_t N = off[S];
  std::vector<double> qm(2 * S);
  std::vector<int32_t> z(static_cast<std::size_t>(N));
  x_all.resize(std::size_t(3 * N));
  for (std::size_t k = 0; k < S; ++k) {
    const int64_t nk = off[k + 1] - off[k];
    std::memcpy(x_all.data() + 3 * off[k], img[k].xq.data(), sizeof(double) * std::size_t(3 * nk));
    std::memcpy(z.data() + off[k], img[k].z.data(), sizeof(int32_t) * std::size_t(nk));
    qm[2 * k] = img[k].xq[3 * nk];
    qm[2 * k + 1] = img[k].xq[3 * nk + 1];
  }
  for (std::size_t k = 0; k < S; ++k) {
    if (!img[k].has_lists || img[k].lists_hdr[H_N] != img[k].hdr[H_N])
      throw Failure(SO3LR_ERR_STATE, "image " + std::to_string(k) + " has no current lists");
    if (img[k].lists_hdr[H_KIND] != img[0].lists_hdr[H_KIND])
      throw Failure(SO3LR_ERR_TOPOLOGY,
                    "image " + std::to_string(k) + ": the short-range list kind differs from image 0's");
  }
  const bool images_changed = full || off != node_off || z != z_all || qm != qm_all;
  if (images_changed) {
    full = true;  // until this call succeeds
    for (std::size_t k = 0; k < S; ++k) {
      const int rc = so3lr_check_system(off[k + 1] - off[k], z.data() + off[k], qm[2 * k], qm[2 * k + 1]);
      if (rc != SO3LR_OK)
        throw Failure(rc, "image " + std::to_string(k) + ": charge " + num(qm[2 * k]) + " with multiplicity " +
                              num(qm[2 * k + 1]) + ": " + so3lr_last_error(nullptr));
    }
    std::vector<double> q(S), m(S);
    for (std::size_t k = 0; k < S; ++k) q[k] = qm[2 * k], m[k] = qm[2 * k + 1];
    const int rc = so3lr_set_images(ctx, N, z.data(), int64_t(S), off.data(), q.data(), m.data());
    if (rc != SO3LR_OK) throw Failure(rc, so3lr_last_error(ctx));
    node_off = off;
    z_all = z;
    qm_all = qm;
  }
  if (images_changed || lists_arrived) {
    sr_il.clear(), sr_nb.clear(), lr_il.clear(), lr_nb.clear();
    sr_off.assign(1, 0), lr_off.assign(1, 0);
    for (std::size_t k = 0; k < S; ++k) {
      const int64_t *h = img[k].lists_hdr;
      const int64_t base = off[k];
      const int64_t *p = img[k].lists.data();
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
    owner.resize(std::size_t(N));
    for (int64_t i = 0; i < N; ++i) owner[i] = int32_t(i);
    const int rc = so3lr_set_topology(ctx, N, owner.data(), int(img[0].lists_hdr[H_KIND]), int64_t(sr_il.size()),
                                      sr_il.data(), sr_off.data(), sr_nb.data(), int64_t(lr_il.size()),
                                      lr_il.data(), lr_off.data(), lr_nb.data());
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
  for (std::size_t k = 0; k < S; ++k) {
    const int64_t a = off[k], nk = off[k + 1] - off[k];
    std::vector<double> &o = img[k].res;
    o.assign(std::size_t(R_DATA + 1 + 6 * nk), 0.0);
    o[R_STATUS] = SO3LR_OK;
    o[R_DATA] = img_e[k];
    std::memcpy(&o[R_DATA + 1], f_all.data() + 3 * a, sizeof(double) * std::size_t(3 * nk));
    std::memcpy(&o[R_DATA + 1 + 3 * nk], e_all.data() + a, sizeof(double) * std::size_t(nk));
    std::memcpy(&o[R_DATA + 1 + 4 * nk], q_all.data() + a, sizeof(double) * std::size_t(nk));
    std::memcpy(&o[R_DATA + 1 + 5 * nk], h_all.data() + a, sizeof(double) * std::size_t(nk));
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
  const MPI_Comm user = MPI_Comm_f2c(MPI_Fint(comm_f));
  if (user == MPI_COMM_NULL) {
    g_error = "SO3LR turbo broker communicator is null";
    return SO3LR_ERR_ARGUMENT;
  }
  int rank = 0, size = 0;
  MPI_Comm_rank(user, &rank);
  MPI_Comm_size(user, &size);
  if (coordinator < 0 || coordinator >= size) {
    g_error = "SO3LR turbo coordinator rank is invalid";
    return SO3LR_ERR_ARGUMENT;
  }
  auto *t = new so3lr_turbo();
  MPI_Comm_dup(user, &t->comm);  // the broker's messages never meet the caller's
  t->rank = rank;
  t->size = size;
  t->coord = coordinator;
  int rc = SO3LR_OK;
  std::string mine;
  if (t->coordinator()) {
    rc = model_path ? so3lr_create(model_path, device, &t->ctx) : SO3LR_ERR_ARGUMENT;
    if (rc != SO3LR_OK)
      mine = std::string("Cannot initialize the coordinator SO3LR model: ") +
             (model_path ? so3lr_last_error(nullptr) : "no model path");
    t->img.resize(std::size_t(size));
  }
  rc = share_status(t->comm, coordinator, rc, mine, g_error);
  if (rc != SO3LR_OK) {
    so3lr_turbo_destroy(t);
    return rc;
  }
  double cut[2] = {0.0, 0.0};
  if (t->coordinator()) cut[0] = so3lr_cutoff(t->ctx, 0), cut[1] = so3lr_cutoff(t->ctx, 1);
  MPI_Bcast(cut, 2, MPI_DOUBLE, coordinator, t->comm);
  t->sr_cut = cut[0];
  t->lr_cut = cut[1];
  *out = t;
  return SO3LR_OK;
}

void so3lr_turbo_destroy(so3lr_turbo *t) {
  if (!t) return;
  if (t->ctx) so3lr_destroy(t->ctx);
  int fin = 0;
  MPI_Finalized(&fin);
  if (!fin && t->comm != MPI_COMM_NULL) MPI_Comm_free(&t->comm);
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

  // 1. this image: checks, header, the data in send form
  std::string why;
  if (n < 1 || n > INT_MAX / 8) why = "the image needs 1 .. 2^28 atoms";
  else if (!z || !x || !f) why = "missing atomic numbers, positions or force output";
  else if (sr_kind != SO3LR_LIST_FULL && sr_kind != SO3LR_LIST_HALF) why = "unknown short-range list kind";
  if (why.empty()) why = list_problem("SR", n, sr_inum, sr_ilist, sr_offsets, sr_neigh);
  if (why.empty()) why = list_problem("LR", n, lr_inum, lr_ilist, lr_offsets, lr_neigh);
  const bool ok = why.empty();
  const bool send_lists = ok && (lists_changed || !t->lists_synced || n != t->last_n);
  int64_t h[H_SIZE] = {ok ? 1 : 0,
                       ok ? n : 0,
                       send_lists ? 1 : 0,
                       ok ? sr_kind : -1,
                       ok ? sr_inum : 0,
                       ok && sr_inum > 0 ? sr_offsets[sr_inum] : 0,
                       ok ? lr_inum : 0,
                       ok && lr_inum > 0 ? lr_offsets[lr_inum] : 0,
                       ok ? 0 : int64_t(why.size())};
  if (ok) {
    t->send_x.resize(std::size_t(3 * n + 2));
    std::memcpy(t->send_x.data(), x, sizeof(double) * std::size_t(3 * n));
    t->send_x[3 * n] = total_charge;
    t->send_x[3 * n + 1] = multiplicity;
  }
  if (send_lists) {
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
  }
  if (lists_changed) t->lists_synced = false;

  int status = SO3LR_OK;
  bool resend = false;
  std::string msg;
  const double *block = nullptr;  // this image's result block

  if (!t->coordinator()) {
    // 2w. post everything, wait politely for the answer
    std::vector<MPI_Request> &r = t->reqs;
    r.assign(4, MPI_REQUEST_NULL);  // unused slots count as complete
    MPI_Isend(h, H_SIZE, MPI_INT64_T, t->coord, kTagHdr, t->comm, &r[0]);
    if (ok) {
      MPI_Isend(t->send_x.data(), int(3 * n + 2), MPI_DOUBLE, t->coord, kTagX, t->comm, &r[1]);
      MPI_Isend(z, int(n), MPI_INT32_T, t->coord, kTagZ, t->comm, &r[2]);
      if (send_lists)
        MPI_Isend(t->send_l.data(), int(t->send_l.size()), MPI_INT64_T, t->coord, kTagLists, t->comm, &r[3]);
    } else if (!why.empty()) {
      MPI_Isend(why.data(), int(why.size()), MPI_CHAR, t->coord, kTagWhy, t->comm, &r[1]);
    }
    t->res.resize(std::size_t(R_DATA + 1 + 6 * (ok ? n : 0)));
    MPI_Request rr;
    MPI_Irecv(t->res.data(), int(t->res.size()), MPI_DOUBLE, t->coord, kTagRes, t->comm, &rr);
    r.push_back(rr);
    settle(r, true);
    t->t_gather = (MPI_Wtime() - t0) * 1e3;
    status = int(t->res[R_STATUS]);
    resend = t->res[R_RESEND] != 0.0;
    if (status != SO3LR_OK && t->res[R_MSGLEN] > 0) {
      std::vector<char> buf(std::size_t(t->res[R_MSGLEN]));
      MPI_Irecv(buf.data(), int(buf.size()), MPI_CHAR, t->coord, kTagMsg, t->comm, &rr);
      r.push_back(rr);
      settle(r, true);
      msg.assign(buf.data(), buf.size());
    }
    block = t->res.data();
    t->gathered = send_lists ? 1 : 0;
  } else {
    // 2c. the coordinator: headers, then the data of every image
    const int S = t->size, me = t->rank;
    std::vector<MPI_Request> &r = t->reqs;
    std::memcpy(t->img[me].hdr, h, sizeof(h));
    for (int k = 0; k < S; ++k) {
      if (k == me) continue;
      MPI_Request q;
      MPI_Irecv(t->img[k].hdr, H_SIZE, MPI_INT64_T, k, kTagHdr, t->comm, &q);
      r.push_back(q);
    }
    settle(r, false);
    bool lists_arrived = false;
    for (int k = 0; k < S; ++k) {
      Image &im = t->img[k];
      const int64_t *hk = im.hdr;
      if (hk[H_OK]) {
        im.xq.resize(std::size_t(3 * hk[H_N] + 2));
        im.z.resize(std::size_t(hk[H_N]));
      } else {
        im.why.assign(std::size_t(hk[H_WHY]), '\0');
      }
      if (hk[H_LISTS]) {
        im.lists.resize(std::size_t(lists_len(hk)));
        std::memcpy(im.lists_hdr, hk, sizeof(im.hdr));
        im.has_lists = true;
        lists_arrived = true;
      }
      if (k == me) {
        if (ok) {
          std::memcpy(im.xq.data(), t->send_x.data(), im.xq.size() * sizeof(double));
          std::memcpy(im.z.data(), z, im.z.size() * sizeof(int32_t));
        } else {
          std::memcpy(im.why.data(), why.data(), why.size());
        }
        if (send_lists) std::memcpy(im.lists.data(), t->send_l.data(), im.lists.size() * sizeof(int64_t));
        continue;
      }
      MPI_Request q;
      if (hk[H_OK]) {
        MPI_Irecv(im.xq.data(), int(im.xq.size()), MPI_DOUBLE, k, kTagX, t->comm, &q);
        r.push_back(q);
        MPI_Irecv(im.z.data(), int(im.z.size()), MPI_INT32_T, k, kTagZ, t->comm, &q);
        r.push_back(q);
        if (hk[H_LISTS]) {
          MPI_Irecv(im.lists.data(), int(im.lists.size()), MPI_INT64_T, k, kTagLists, t->comm, &q);
          r.push_back(q);
        }
      } else if (hk[H_WHY] > 0) {
        MPI_Irecv(im.why.data(), int(im.why.size()), MPI_CHAR, k, kTagWhy, t->comm, &q);
        r.push_back(q);
      }
    }
    settle(r, false);
    const double t1 = MPI_Wtime();
    t->t_gather = (t1 - t0) * 1e3;
    t->gathered = lists_arrived ? 1 : 0;

    // 3c. evaluate, or name the first malformed image
    for (int k = 0; k < S && status == SO3LR_OK; ++k)
      if (!t->img[k].hdr[H_OK]) {
        status = SO3LR_ERR_TOPOLOGY;
        msg = "SO3LR turbo broker received an invalid graph from image " + std::to_string(k) + ": " +
              std::string(t->img[k].why.begin(), t->img[k].why.end());
      }
    if (status == SO3LR_OK) {
      try {
        t->run_packed(lists_arrived);
      } catch (const Failure &e) {
        status = e.code;
        msg = std::string("SO3LR coordinator evaluation failed: ") + e.what();
      } catch (const std::exception &e) {
        status = SO3LR_ERR_DEVICE;
        msg = std::string("SO3LR coordinator evaluation failed: ") + e.what();
      }
    }
    if (status != SO3LR_OK) {
      // every image sends its lists again on the next call
      t->full = true;
      for (Image &im : t->img) im.has_lists = false;
      resend = true;
    }
    const double t2 = MPI_Wtime();
    t->t_eval = (t2 - t1) * 1e3;

    // 4c. answers
    for (int k = 0; k < S; ++k) {
      Image &im = t->img[k];
      if (status != SO3LR_OK) im.res.assign(R_DATA, 0.0);
      im.res[R_STATUS] = status;
      im.res[R_RESEND] = resend ? 1.0 : 0.0;
      im.res[R_MSGLEN] = status != SO3LR_OK ? double(msg.size()) : 0.0;
      if (k == me) continue;
      MPI_Request q;
      MPI_Isend(im.res.data(), int(im.res.size()), MPI_DOUBLE, k, kTagRes, t->comm, &q);
      r.push_back(q);
      if (status != SO3LR_OK && !msg.empty()) {
        MPI_Isend(msg.data(), int(msg.size()), MPI_CHAR, k, kTagMsg, t->comm, &q);
        r.push_back(q);
      }
    }
    settle(r, false);
    t->t_scatter = (MPI_Wtime() - t2) * 1e3;
    block = t->img[me].res.data();
  }

  t->t_total = (MPI_Wtime() - t0) * 1e3;
  if (resend) t->lists_synced = false;
  if (status != SO3LR_OK) {
    t->error = msg;
    return status;
  }
  if (send_lists) t->lists_synced = true;
  t->last_n = n;
  const double *b = block + R_DATA;
  if (energy) *energy = b[0];
  std::memcpy(f, b + 1, sizeof(double) * std::size_t(3 * n));
  if (eatom) std::memcpy(eatom, b + 1 + 3 * n, sizeof(double) * std::size_t(n));
  if (charges) std::memcpy(charges, b + 1 + 4 * n, sizeof(double) * std::size_t(n));
  if (hirshfeld) std::memcpy(hirshfeld, b + 1 + 5 * n, sizeof(double) * std::size_t(n));
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
