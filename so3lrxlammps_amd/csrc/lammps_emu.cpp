// Host stand-in for LAMMPS ghost communication and neighbour lists (see
// include/so3lr_lammps_emu.h).  Cell lists over owned + ghost rows, OpenMP
// over receivers, two passes (count, fill) so the CSR is built in place.
#include "../../include/so3lr_lammps_emu.h"

#include <algorithm>
#include <cmath>
#include <stdexcept>
#include <string>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

struct so3lr_emu_lists {
  std::vector<int32_t> owner, image;
  std::vector<double> x;  // rows * 3
  int64_t n = 0;
  struct List {
    std::vector<int32_t> ilist, neigh;
    std::vector<int64_t> off;
  } sr, lr;
};

namespace {
thread_local std::string g_err;

void build(so3lr_emu_lists &L, int64_t n, const double *x, const double *lo, const double *hi,
           const int *per, double sr_cut, double lr_cut, double skin, double comm, bool sr_full) {
  if (n <= 0) throw std::invalid_argument("no atoms");
  const double len[3] = {hi[0] - lo[0], hi[1] - lo[1], hi[2] - lo[2]};
  const double rmax = std::max(sr_cut, lr_cut) + skin;
  if (comm < rmax) throw std::invalid_argument("communication cutoff is smaller than cutoff + skin");
  for (int d = 0; d < 3; ++d)
    if (per[d] && !(len[d] > 0)) throw std::invalid_argument("degenerate periodic box");
  L.n = n;
  L.owner.resize(n);
  L.image.assign(3 * n, 0);
  L.x.assign(x, x + 3 * n);
  for (int64_t i = 0; i < n; ++i) {
    L.owner[i] = int32_t(i);
    for (int d = 0; d < 3; ++d)
      if (per[d] && (x[3 * i + d] < lo[d] || x[3 * i + d] >= hi[d]))
        throw std::invalid_argument("owned atom outside the periodic box; wrap positions first");
  }
  // ghosts: every periodic image within `comm` of the box (LAMMPS comm cutoff)
  for (int sx = -1; sx <= 1; ++sx)
    for (int sy = -1; sy <= 1; ++sy)
      for (int sz = -1; sz <= 1; ++sz) {
        const int s[3] = {sx, sy, sz};
        if (!sx && !sy && !sz) continue;
        bool ok = true;
        for (int d = 0; d < 3; ++d)
          if (s[d] && !per[d]) ok = false;
        if (!ok) continue;
        for (int64_t i = 0; i < n; ++i) {
          double p[3];
          bool inside = true;
          for (int d = 0; d < 3; ++d) {
            p[d] = x[3 * i + d] + s[d] * len[d];
            if (per[d] && (p[d] < lo[d] - comm || p[d] >= hi[d] + comm)) inside = false;
          }
          if (!inside) continue;
          L.owner.push_back(int32_t(i));
          for (int d = 0; d < 3; ++d) { L.image.push_back(s[d]); L.x.push_back(p[d]); }
        }
      }
  const int64_t rows = int64_t(L.owner.size());
  if (rows >= (int64_t(1) << 31)) throw std::length_error("too many rows");
  // cell list over all rows, cell edge >= rmax
  double blo[3], bhi[3];
  for (int d = 0; d < 3; ++d) { blo[d] = 1e300; bhi[d] = -1e300; }
  for (int64_t r = 0; r < rows; ++r)
    for (int d = 0; d < 3; ++d) { blo[d] = std::min(blo[d], L.x[3 * r + d]); bhi[d] = std::max(bhi[d], L.x[3 * r + d]); }
  int nc[3];
  for (int d = 0; d < 3; ++d) nc[d] = std::max(1, int((bhi[d] - blo[d]) / rmax));
  const int64_t ncell = int64_t(nc[0]) * nc[1] * nc[2];
  auto cell_of = [&](const double *p, int *c) {
    for (int d = 0; d < 3; ++d) {
      int k = int((p[d] - blo[d]) / (bhi[d] - blo[d] + 1e-12) * nc[d]);
      c[d] = std::min(std::max(k, 0), nc[d] - 1);
    }
  };
  std::vector<int64_t> cstart(ncell + 1, 0);
  std::vector<int32_t> cell_rows(rows);
  std::vector<int> rc(3 * rows);
  for (int64_t r = 0; r < rows; ++r) {
    cell_of(&L.x[3 * r], &rc[3 * r]);
    ++cstart[(int64_t(rc[3 * r]) * nc[1] + rc[3 * r + 1]) * nc[2] + rc[3 * r + 2] + 1];
  }
  for (int64_t c = 0; c < ncell; ++c) cstart[c + 1] += cstart[c];
  {
    std::vector<int64_t> fill(cstart.begin(), cstart.end() - 1);
    for (int64_t r = 0; r < rows; ++r)
      cell_rows[fill[(int64_t(rc[3 * r]) * nc[1] + rc[3 * r + 1]) * nc[2] + rc[3 * r + 2]]++] = int32_t(r);
  }
  const double sr2 = (sr_cut + skin) * (sr_cut + skin), lr2 = (lr_cut + skin) * (lr_cut + skin);
  // pass 1: counts; pass 2: fill (same traversal order, so lists are deterministic)
  L.sr.ilist.resize(n); L.lr.ilist.resize(n);
  L.sr.off.assign(n + 1, 0); L.lr.off.assign(n + 1, 0);
  for (int pass = 0; pass < 2; ++pass) {
    if (pass == 1) {
      for (int64_t i = 0; i < n; ++i) { L.sr.off[i + 1] += L.sr.off[i]; L.lr.off[i + 1] += L.lr.off[i]; }
      L.sr.neigh.resize(L.sr.off[n]);
      L.lr.neigh.resize(L.lr.off[n]);
    }
#pragma omp parallel for schedule(dynamic, 64)
    for (int64_t i = 0; i < n; ++i) {
      L.sr.ilist[i] = L.lr.ilist[i] = int32_t(i);
      const double *pi = &L.x[3 * i];
      const int *ci = &rc[3 * i];
      int64_t ks = pass ? L.sr.off[i] : 0, kl = pass ? L.lr.off[i] : 0;
      for (int dx = -1; dx <= 1; ++dx)
        for (int dy = -1; dy <= 1; ++dy)
          for (int dz = -1; dz <= 1; ++dz) {
            const int cx = ci[0] + dx, cy = ci[1] + dy, cz = ci[2] + dz;
            if (cx < 0 || cy < 0 || cz < 0 || cx >= nc[0] || cy >= nc[1] || cz >= nc[2]) continue;
            const int64_t c = (int64_t(cx) * nc[1] + cy) * nc[2] + cz;
            for (int64_t k = cstart[c]; k < cstart[c + 1]; ++k) {
              const int32_t j = cell_rows[k];
              if (j == i) continue;
              const double ddx = pi[0] - L.x[3 * j], ddy = pi[1] - L.x[3 * j + 1], ddz = pi[2] - L.x[3 * j + 2];
              const double r2 = ddx * ddx + ddy * ddy + ddz * ddz;
              const int32_t oj = L.owner[j];
              const bool keep_half = oj > i;  // newton-on: one entry per unique pair
              if (r2 < sr2 && (sr_full || keep_half)) {
                if (pass) L.sr.neigh[ks] = j;
                ++ks;
              }
              if (r2 < lr2 && keep_half) {
                if (pass) L.lr.neigh[kl] = j;
                ++kl;
              }
            }
          }
      if (!pass) { L.sr.off[i + 1] = ks; L.lr.off[i + 1] = kl; }
    }
  }
}
}  // namespace

extern "C" {

int so3lr_emu_build(int64_t n, const double *x, const double *lo, const double *hi, const int *periodic,
                    double sr_cut, double lr_cut, double skin, double comm_cut, int sr_full,
                    so3lr_emu_lists **out) {
  if (!out || !x || !lo || !hi || !periodic) { g_err = "null argument"; return 1; }
  *out = nullptr;
  auto *L = new so3lr_emu_lists();
  try {
    build(*L, n, x, lo, hi, periodic, sr_cut, lr_cut, skin, comm_cut, sr_full != 0);
  } catch (const std::exception &e) {
    g_err = e.what();
    delete L;
    return 1;
  }
  *out = L;
  return 0;
}
const char *so3lr_emu_error(void) { return g_err.c_str(); }
void so3lr_emu_free(so3lr_emu_lists *l) { delete l; }
int64_t so3lr_emu_rows(const so3lr_emu_lists *l) { return int64_t(l->owner.size()); }
const int32_t *so3lr_emu_owner(const so3lr_emu_lists *l) { return l->owner.data(); }
const int32_t *so3lr_emu_image(const so3lr_emu_lists *l) { return l->image.data(); }
int64_t so3lr_emu_inum(const so3lr_emu_lists *l, int which) { return which ? int64_t(l->lr.ilist.size()) : int64_t(l->sr.ilist.size()); }
const int32_t *so3lr_emu_ilist(const so3lr_emu_lists *l, int which) { return which ? l->lr.ilist.data() : l->sr.ilist.data(); }
const int64_t *so3lr_emu_offsets(const so3lr_emu_lists *l, int which) { return which ? l->lr.off.data() : l->sr.off.data(); }
const int32_t *so3lr_emu_neigh(const so3lr_emu_lists *l, int which) { return which ? l->lr.neigh.data() : l->sr.neigh.data(); }

}  // extern "C"
