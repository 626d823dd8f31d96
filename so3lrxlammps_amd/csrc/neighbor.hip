// Device-side reneighbor for the HBM-resident path (no ghost rows).
//
// LAMMPS builds the reference's neighbour lists on the host and the pair
// style re-uploads them at every reneighbor (pair_so3lr_native_mpi.cpp:
// 1297-1334).  Here the same candidate sets -- every periodic image within
// cutoff + skin -- are built on the GPU from owned positions in an orthogonal
// box:
//   1. wrap positions into the box (LAMMPS Domain::pbc) and bin atoms into
//      cells of edge >= LR cutoff + skin (stable radix sort, deterministic);
//   2. one wavefront per atom walks the 27 neighbouring cells (periodic
//      wrap with an image code per cell) and emits, in a fixed order
//      (ballot prefix inside each 64-atom chunk), its full SR and LR lists;
//   3. the SR full list becomes the half-pair table (canonical direction:
//      smaller atom index first) and its own incidence list, the reverse
//      entry finding its pair by scanning its partner's list; the LR full
//      list is used as it is by the node-major LR kernel.
// Image code c in 0..26 stands for the shift ((c/9)-1, (c/3)%3-1, c%3-1)
// box lengths added to the neighbour's position.
//
// For a single system the evaluator's nodes follow a spatial (Morton) order
// of the wrapped positions, the device analogue of LAMMPS's periodic atom
// sort (atom_modify sort): node n is owned atom perm[n].  Neighbour gathers
// then stay within a compact region, which one XCD's L2 can serve.  Inputs
// are gathered into node order and forces scattered back, so callers keep
// their own atom order.
#include "evaluator.hpp"
#include "spatial_order.hpp"

#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <cmath>
#include <stdexcept>

namespace so3lr_amd {

#define NB_CHECK(expr)                                                                    \
  do {                                                                                    \
    hipError_t err_ = (expr);                                                             \
    if (err_ != hipSuccess)                                                               \
      throw DeviceError(std::string("HIP error in ") + #expr + ": " +             \
                               hipGetErrorString(err_));                                  \
  } while (0)

namespace {

// Entries of both candidate lists together (short and long range, each pair
// in both directions) that a device reneighbor accepts: list entries,
// incidence slots and their offsets are ints.  Water at 1 g/cm^3 with a 1 A
// skin holds about 990 entries per atom, so the limit is near 2.1 million
// atoms, above what 288 GB of HBM holds at the evaluation's ~200 KB per atom.
constexpr long long kMaxListEntries = (1LL << 31) - 2;

struct Grid {
  double lo[3], len[3];
  int nc[3];
  int per[3];
};

__global__ void k_wrap(int n, double *x, Grid G) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  for (int d = 0; d < 3; ++d) {
    if (!G.per[d]) continue;
    double v = x[3 * i + d] - G.lo[d];
    v -= floor(v / G.len[d]) * G.len[d];
    if (v >= G.len[d]) v -= G.len[d];
    if (v < 0.0) v = 0.0;
    x[3 * i + d] = G.lo[d] + v;
  }
}

__device__ __forceinline__ int cell_coord(double v, double lo, double len, int nc) {
  int c = int(floor((v - lo) / len * nc));
  return c < 0 ? 0 : (c >= nc ? nc - 1 : c);
}

__global__ void k_cell_keys(int n, const double *x, Grid G, int *key, int *idx) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int cx = cell_coord(x[3 * i], G.lo[0], G.len[0], G.nc[0]);
  const int cy = cell_coord(x[3 * i + 1], G.lo[1], G.len[1], G.nc[1]);
  const int cz = cell_coord(x[3 * i + 2], G.lo[2], G.len[2], G.nc[2]);
  key[i] = (cx * G.nc[1] + cy) * G.nc[2] + cz;
  idx[i] = i;
}

// cell_start[c] = first position of cell c in the sorted order
__global__ void k_cell_start(int n, int ncell, const int *skey, int *start) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i > n) return;
  const int prev = i == 0 ? -1 : skey[i - 1];
  const int cur = i == n ? ncell : skey[i];
  for (int c = prev + 1; c <= cur; ++c) start[c] = i;
}

// One wavefront per atom: count (FILL = false) or emit (FILL = true) every
// neighbour within the SR and LR radii, in stencil-cell order.
template <bool FILL>
__global__ __launch_bounds__(256) void k_nbr(int n, const double *x, Grid G, const int *cstart, const int *sidx,
                                             double sr2, double lr2, int *sr_cnt, int *lr_cnt,
                                             const int *sr_off, const int *lr_off, int *sr_list, int *lr_list,
                                             int *err) {
  const int lane = threadIdx.x & 63;
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= n) return;
  const double xi = x[3 * i], yi = x[3 * i + 1], zi = x[3 * i + 2];
  const int ci[3] = {cell_coord(xi, G.lo[0], G.len[0], G.nc[0]), cell_coord(yi, G.lo[1], G.len[1], G.nc[1]),
                     cell_coord(zi, G.lo[2], G.len[2], G.nc[2])};
  int ns = 0, nl = 0;
  int ws = FILL ? sr_off[i] : 0, wl = FILL ? lr_off[i] : 0;
  for (int s = 0; s < 27; ++s) {
    const int o[3] = {s / 9 - 1, (s / 3) % 3 - 1, s % 3 - 1};
    int c[3], img[3];
    bool ok = true;
    for (int d = 0; d < 3; ++d) {
      int cc = ci[d] + o[d];
      img[d] = 0;
      if (cc < 0) { if (!G.per[d]) { ok = false; break; } cc += G.nc[d]; img[d] = -1; }
      if (cc >= G.nc[d]) { if (!G.per[d]) { ok = false; break; } cc -= G.nc[d]; img[d] = 1; }
      c[d] = cc;
    }
    if (!ok) continue;
    // with fewer than 3 cells along a periodic axis two offsets reach the same
    // cell with different images; both are kept (distinct images)
    const int code = (img[0] + 1) * 9 + (img[1] + 1) * 3 + (img[2] + 1);
    const double sx = img[0] * G.len[0], sy = img[1] * G.len[1], sz = img[2] * G.len[2];
    const int cell = (c[0] * G.nc[1] + c[1]) * G.nc[2] + c[2];
    for (int k0 = cstart[cell]; k0 < cstart[cell + 1]; k0 += 64) {
      const int k = k0 + lane;
      bool in_sr = false, in_lr = false;
      int j = -1;
      if (k < cstart[cell + 1]) {
        j = sidx[k];
        const double dx = x[3 * j] + sx - xi, dy = x[3 * j + 1] + sy - yi, dz = x[3 * j + 2] + sz - zi;
        const double r2 = dx * dx + dy * dy + dz * dz;
        if (j == i && code == 13) {
          // the atom itself
        } else {
          in_lr = r2 < lr2;
          in_sr = r2 < sr2;
          if (j == i && in_lr && err) *err = 1;  // own periodic image inside the cutoff
        }
      }
      const unsigned long long bs = __ballot(in_sr), bl = __ballot(in_lr);
      const unsigned long long below = lane ? (~0ull >> (64 - lane)) : 0ull;
      if (FILL) {
        if (in_sr) sr_list[ws + __popcll(bs & below)] = j * 32 + code;
        if (in_lr) lr_list[wl + __popcll(bl & below)] = j * 32 + code;
        ws += __popcll(bs);
        wl += __popcll(bl);
      } else {
        ns += __popcll(bs);
        nl += __popcll(bl);
      }
    }
  }
  if (!FILL && lane == 0) {
    sr_cnt[i] = ns;
    lr_cnt[i] = nl;
  }
}

// exclusive scan of counts[0..n) into off[0..n] (one block, deterministic).
// The running total is carried in 64 bits and written to *total: the int
// offsets are valid only while it stays below 2^31, which the host checks
// before it reads or uses them.  A 1024-count tile sums in int (each count
// is one atom's neighbours: far below 2^21).
__global__ __launch_bounds__(1024) void k_scan_int(int n, const int *cnt, int *off, long long *total) {
  __shared__ int buf[1024];
  __shared__ long long carry;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  for (int start = 0; start < n; start += 1024) {
    const int i = start + threadIdx.x;
    const int v = i < n ? cnt[i] : 0;
    buf[threadIdx.x] = v;
    __syncthreads();
    for (int o = 1; o < 1024; o <<= 1) {
      const int t = int(threadIdx.x) >= o ? buf[threadIdx.x - o] : 0;
      __syncthreads();
      buf[threadIdx.x] += t;
      __syncthreads();
    }
    if (i < n) off[i] = int(carry + buf[threadIdx.x] - v);
    __syncthreads();
    if (threadIdx.x == 1023) carry += buf[1023];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    off[n] = int(carry);
    *total = carry;
  }
}

// canonical SR entries (i < j) per atom
__global__ void k_canon_count(int n, const int *off, const int *list, int *cnt) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  int c = 0;
  for (int k = off[i]; k < off[i + 1]; ++k)
    if ((list[k] >> 5) > i) ++c;
  cnt[i] = c;
}

// pairs in atom-major order of their canonical entry; incidence entries
// p * 2 + side in the same positions as the full list.  One wavefront per
// atom: canonical entries are numbered by ballot prefix in list order, and
// each lane finds the pair of one reverse entry in its partner's list.
__global__ __launch_bounds__(256) void k_pairs(int n, const int *off, const int *list, const int *poff, int *nodes,
                                               int *codes, int *inc, int *err) {
  const int lane = threadIdx.x & 63;
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= n) return;
  const int beg = off[i], end = off[i + 1];
  const unsigned long long below = lane ? (~0ull >> (64 - lane)) : 0ull;
  int p = poff[i];
  for (int k0 = beg; k0 < end; k0 += 64) {
    const int k = k0 + lane;
    const int e = k < end ? list[k] : 0;
    const bool canon = k < end && (e >> 5) > i;
    const unsigned long long mask = __ballot(canon);
    if (canon) {
      const int q = p + __popcll(mask & below);
      nodes[2 * q] = i;
      nodes[2 * q + 1] = e >> 5;
      codes[q] = e & 31;
      inc[k] = 2 * q;
    }
    p += __popcll(mask);
  }
  // reverse entries: find (i, -code) in j's list, whose canonical pair index
  // is poff[j] + (number of canonical entries before it)
  for (int k = beg + lane; k < end; k += 64) {
    const int e = list[k];
    const int j = e >> 5, code = e & 31;
    if (j > i) continue;
    const int want = i * 32 + (26 - code);  // negated image
    int q = poff[j], found = -1;
    for (int m = off[j]; m < off[j + 1]; ++m) {
      const int f = list[m];
      if ((f >> 5) > j) {
        if (f == want) { found = q; break; }
        ++q;
      }
    }
    if (found < 0) { if (err) *err = 2; inc[k] = 1; continue; }
    inc[k] = 2 * found + 1;
  }
}

}  // namespace

void Evaluator::build_topology_device(double *x, const double lo[3], const double hi[3], const int per[3],
                                      double skin) {
  if (!system_ready_) throw std::logic_error("SO3LR: set the system before the topology");
  hipStream_t s = stream_;
  const int n = int(n_);
  Grid G;
  const double rmax = std::max(rc_, lr_.cutoff) + skin;
  for (int d = 0; d < 3; ++d) {
    G.lo[d] = lo[d];
    G.len[d] = hi[d] - lo[d];
    G.per[d] = per[d] ? 1 : 0;
    if (!(G.len[d] > 0)) throw std::invalid_argument("SO3LR: degenerate box");
    if (G.per[d] && G.len[d] <= 2.0 * (lr_.cutoff + 0.0))
      throw std::invalid_argument("SO3LR: periodic box shorter than twice the long-range cutoff");
    G.nc[d] = std::max(1, int(std::floor(G.len[d] / rmax)));
  }
  const int ncell = G.nc[0] * G.nc[1] * G.nc[2];
  if (std::int64_t(ncell) > (std::int64_t(1) << 26)) throw std::invalid_argument("SO3LR: box too large for the cell grid");
  hipLaunchKernelGGL(k_wrap, dim3((n + 255) / 256), dim3(256), 0, s, n, x, G);
  int *key = ensure<int>(nb_key_, n), *idx = ensure<int>(nb_idx_, n);
  int *skey = ensure<int>(nb_skey_, n), *sidx = ensure<int>(nb_sidx_, n);
  int *cstart = ensure<int>(nb_cstart_, ncell + 1);
  const unsigned gb = unsigned((n + 255) / 256);
  auto sort_pairs = [&](int *k_in, int *k_out, int *v_in, int *v_out, int bits) {
    std::size_t tmp_bytes = 0;
    NB_CHECK(hipcub::DeviceRadixSort::SortPairs(nullptr, tmp_bytes, k_in, k_out, v_in, v_out, n, 0, bits, s));
    void *tmp = ensure<char>(nb_tmp_, tmp_bytes);
    NB_CHECK(hipcub::DeviceRadixSort::SortPairs(tmp, tmp_bytes, k_in, k_out, v_in, v_out, n, 0, bits, s));
  };
  // node order: Morton order of the wrapped positions (one system only: the
  // per-image charge correction of packed images needs contiguous images)
  const bool reorder = n_images_ == 1;
  if (reorder) {
    int *perm = ensure<int>(perm_, n);
    MortonBox B;
    for (int d = 0; d < 3; ++d) {
      B.lo[d] = G.lo[d];
      B.len[d] = G.len[d];
    }
    hipLaunchKernelGGL(k_morton, dim3(gb), dim3(256), 0, s, n, x, B, key, idx);
    sort_pairs(key, skey, idx, perm, 30);
    double *xn = ensure<double>(xn_, 3 * std::size_t(n));
    hipLaunchKernelGGL(k_gather_rows, dim3(unsigned((3 * std::size_t(n) + 255) / 256)), dim3(256), 0, s, n, 3, perm,
                       x, xn);
    hipLaunchKernelGGL(k_gather_int, dim3(gb), dim3(256), 0, s, n, perm, static_cast<const int *>(z_->p),
                       ensure<int>(nz_, n));
    hipLaunchKernelGGL(k_gather_rows, dim3(unsigned((std::size_t(n) * F_ + 255) / 256)), dim3(256), 0, s, n, F_,
                       perm, static_cast<const double *>(x0_->p), ensure<double>(nx0_, std::size_t(n) * F_));
    perm_host_.resize(n);
    NB_CHECK(hipMemcpyAsync(perm_host_.data(), perm, std::size_t(n) * sizeof(int), hipMemcpyDeviceToHost, s));
    x = xn;  // the lists below are built in node order
  }
  hipLaunchKernelGGL(k_cell_keys, dim3(gb), dim3(256), 0, s, n, x, G, key, idx);
  int bits = 1;
  while ((1 << bits) < ncell + 1) ++bits;
  sort_pairs(key, skey, idx, sidx, bits);
  hipLaunchKernelGGL(k_cell_start, dim3((n + 1 + 255) / 256), dim3(256), 0, s, n, ncell, skey, cstart);
  int *sr_cnt = ensure<int>(nb_srcnt_, n), *lr_cnt = ensure<int>(nb_lrcnt_, n);
  int *err = ensure<int>(nb_err_, 1);
  NB_CHECK(hipMemsetAsync(err, 0, sizeof(int), s));
  const double sr2 = (rc_ + skin) * (rc_ + skin), lr2 = (lr_.cutoff + skin) * (lr_.cutoff + skin);
  const int gw = (n + 3) / 4;
  hipLaunchKernelGGL(k_nbr<false>, dim3(gw), dim3(256), 0, s, n, x, G, cstart, sidx, sr2, lr2, sr_cnt, lr_cnt,
                     nullptr, nullptr, nullptr, nullptr, err);
  int *sr_off = ensure<int>(sr_inc_off_, n + 1), *lr_off = ensure<int>(lr_inc_off_, n + 1);
  long long *tot = ensure<long long>(nb_tot_, 4);
  hipLaunchKernelGGL(k_scan_int, dim3(1), dim3(1024), 0, s, n, sr_cnt, sr_off, tot);
  hipLaunchKernelGGL(k_scan_int, dim3(1), dim3(1024), 0, s, n, lr_cnt, lr_off, tot + 1);
  long long tot64[2] = {0, 0};
  NB_CHECK(hipMemcpyAsync(tot64, tot, sizeof(tot64), hipMemcpyDeviceToHost, s));
  NB_CHECK(hipStreamSynchronize(s));
  // the 64-bit totals decide before any int offset is read: every list entry
  // and incidence slot is addressed by an int
  if (tot64[0] + tot64[1] > kMaxListEntries)
    throw std::length_error("SO3LR: the neighbour lists of " + std::to_string(n) + " atoms hold " +
                            std::to_string(tot64[0] + tot64[1]) + " entries (short + long range); the limit is " +
                            std::to_string(kMaxListEntries) + " (about 2.1 million atoms of water)");
  const int totals[2] = {int(tot64[0]), int(tot64[1])};
  int *sr_list = ensure<int>(nb_srlist_, totals[0]);
  int *lr_list = ensure<int>(lr_inc_, totals[1]);
  hipLaunchKernelGGL(k_nbr<true>, dim3(gw), dim3(256), 0, s, n, x, G, cstart, sidx, sr2, lr2, nullptr, nullptr,
                     sr_off, lr_off, sr_list, lr_list, nullptr);
  // half-pair table of the SR list
  hipLaunchKernelGGL(k_canon_count, dim3((n + 255) / 256), dim3(256), 0, s, n, sr_off, sr_list, sr_cnt);
  int *poff = ensure<int>(nb_poff_, n + 1);
  hipLaunchKernelGGL(k_scan_int, dim3(1), dim3(1024), 0, s, n, sr_cnt, poff, tot + 2);  // at most totals[0]
  int npairs = 0, herr = 0;
  NB_CHECK(hipMemcpyAsync(&npairs, poff + n, sizeof(int), hipMemcpyDeviceToHost, s));
  NB_CHECK(hipStreamSynchronize(s));
  int *nodes = ensure<int>(sr_nodes_, 2 * std::size_t(std::max(npairs, 1)));
  int *codes = ensure<int>(sr_code_, std::max(npairs, 1));
  int *inc = ensure<int>(sr_inc_, std::max(totals[0], 1));
  hipLaunchKernelGGL(k_pairs, dim3(gw), dim3(256), 0, s, n, sr_off, sr_list, poff, nodes, codes, inc, err);
  NB_CHECK(hipMemcpyAsync(&herr, err, sizeof(int), hipMemcpyDeviceToHost, s));
  NB_CHECK(hipStreamSynchronize(s));
  if (herr == 1)
    throw std::invalid_argument("SO3LR: an atom sees its own periodic image within the cutoff; the box is too small");
  if (herr == 2) throw std::logic_error("SO3LR: internal error, short-range list not symmetric");
  if (2 * npairs != totals[0]) throw std::logic_error("SO3LR: internal error, short-range pair count");
  p_sr_ = npairs;
  p_lr_ = totals[1] / 2;
  lr_entries_ = totals[1];
  for (int d = 0; d < 3; ++d) box_len_[d] = G.len[d];
  permuted_ = reorder;
  rows_order_pending_ = false;
  shift_mode_ = true;
  topology_ready_ = true;
  ++topo_version_;
  evaluated_ = false;
  act_cap_ = 0;  // counted again by the next evaluation
}

}  // namespace so3lr_amd
