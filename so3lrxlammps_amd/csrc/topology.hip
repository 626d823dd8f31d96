// LAMMPS neighbour lists -> the evaluator's pair tables, on the GPU.
//
// At every LAMMPS reneighbor the pair style hands over its rows (owned +
// ghost atoms), the owner of every row and two candidate lists, receiver-major
// in ilist order: the full short-range list (request id 0) and the newton-on
// half long-range list (request id 1) (pair_so3lr_native_mpi.cpp:1174-1192,
// 1297-1334; src/lammps_neighbor_adapter.cpp:190-237).  The reference
// snapshots them on the host every reneighbor.  Here only the raw lists cross
// PCIe; the rest runs on the device:
//   1. owner-map check (identity on owned rows, ghosts map to owned atoms);
//   2. per list, one wavefront per ilist row counts the entries it keeps:
//      not the row itself, ghost images collapsed onto their owner (one-rank
//      collapse, plugins/lammps/pair_so3lr_native.cpp:74-146), and for a full
//      list only the direction whose receiver has the smaller owner index (the
//      other direction is counted, and the two counts must agree);
//   3. an exclusive scan over rows, then the same walk writes each kept entry
//      at its row offset + ballot prefix, so pairs keep list order;
//   4. the node-major incidence list: the pair endpoints (2 per pair) sorted
//      by node with a stable radix sort, so each node's entries stay in
//      increasing pair order, and the node offsets from the sorted keys.
// Results are identical to a sequential host walk of the lists.
#include "evaluator.hpp"
#include "spatial_order.hpp"

#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <stdexcept>
#include <string>

namespace so3lr_amd {

#define TOPO_CHECK(expr)                                                                             \
  do {                                                                                               \
    hipError_t err_ = (expr);                                                                        \
    if (err_ != hipSuccess) throw DeviceError(std::string("HIP error in ") + #expr + ": " + hipGetErrorString(err_)); \
  } while (0)

namespace {

enum TopoFault : int {
  kBadOwner = 1,    // owner_of_row not the identity on owned rows, or a ghost maps outside them
  kBadRow = 2,      // a neighbour row outside [0, n_rows)
  kSelfImage = 4,   // an atom paired with its own periodic image
};

__global__ void k_fill_ints(int n, int *p, int v) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t < n) p[t] = v;
}

__global__ void k_check_owner(int n_rows, int n, const int *owner, int *fault) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= n_rows) return;
  const int o = owner[r];
  if (o < 0 || o >= n || (r < n && o != r)) atomicOr(fault, kBadOwner);
}

// One wavefront per list row k.  COUNT: kept[k] = entries kept, and (FULL)
// the dropped reverse directions added to *dropped.  Otherwise: write the
// kept entries from poff[k] on, in list order.
template <bool FULL, bool COUNT>
__global__ __launch_bounds__(256) void k_list_walk(int inum, int n_rows, const int *ilist, const std::int64_t *off,
                                                   const int *neigh, const int *owner, int *kept,
                                                   unsigned long long *dropped, int *fault, const int *poff,
                                                   int *rows, int *nodes) {
  const int lane = threadIdx.x & 63;
  const int k = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (k >= inum) return;
  const int i = ilist[k];  // checked on the host: an owned row
  const std::int64_t beg = off[k], end = off[k + 1];
  const unsigned long long below = lane ? (~0ull >> (64 - lane)) : 0ull;
  int q = COUNT ? 0 : poff[k];
  int drop = 0;
  for (std::int64_t e0 = beg; e0 < end; e0 += 64) {
    const std::int64_t e = e0 + lane;
    bool keep = false;
    int j = 0, oj = 0;
    if (e < end) {
      j = neigh[e];
      if (j < 0 || j >= n_rows) {
        if (COUNT) atomicOr(fault, kBadRow);
      } else if (j != i) {
        oj = owner[j];
        if (oj == i) {
          if (COUNT) atomicOr(fault, kSelfImage);
        } else if (FULL && oj < i) {
          ++drop;
        } else {
          keep = true;
        }
      }
    }
    const unsigned long long mask = __ballot(keep);
    if (!COUNT && keep) {
      const int at = q + __popcll(mask & below);
      rows[2 * at] = i;
      rows[2 * at + 1] = j;
      nodes[2 * at] = i;
      nodes[2 * at + 1] = oj;
    }
    q += __popcll(mask);
  }
  if (COUNT) {
    if (FULL) {
      for (int o = 32; o > 0; o >>= 1) drop += __shfl_xor(drop, o, 64);
      if (lane == 0 && drop) atomicAdd(dropped, (unsigned long long)drop);
    }
    if (lane == 0) kept[k] = q;
  }
}

// Exclusive scan of cnt[0..n) into out[0..n] (one block; fixed order): the
// per-receiver pair counts.  The sum is at most
// the list's entry count, which set_topology refuses above 2^30 on the host
// before any upload, so every partial sum fits an int.
__global__ __launch_bounds__(1024) void k_scan_rows(int n, const int *cnt, int *out) {
  __shared__ int part[1024];
  __shared__ int base;
  if (threadIdx.x == 0) base = 0;
  __syncthreads();
  for (int s = 0; s < n; s += 1024) {
    const int i = s + threadIdx.x;
    const int v = i < n ? cnt[i] : 0;
    part[threadIdx.x] = v;
    __syncthreads();
    for (int d = 1; d < 1024; d <<= 1) {
      const int t = int(threadIdx.x) >= d ? part[threadIdx.x - d] : 0;
      __syncthreads();
      part[threadIdx.x] += t;
      __syncthreads();
    }
    if (i < n) out[i] = base + part[threadIdx.x] - v;
    __syncthreads();
    if (threadIdx.x == 1023) base += part[1023];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[n] = base;
}

__global__ void k_iota(int m, int *v) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t < m) v[t] = t;
}

// off[v] = first position of key v in the sorted keys (off[n] = m)
__global__ void k_segment_starts(int m, int n, const int *skey, int *off) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t > m) return;
  const int prev = t == 0 ? -1 : skey[t - 1];
  const int cur = t == m ? n : skey[t];
  for (int v = prev + 1; v <= cur; ++v) off[v] = t;
}

// Bounding box of the first n rows: out = {min x, y, z, max x, y, z}.  One
// block; the reduction order is fixed.
// min and max that keep a NaN once they have seen one (fmin/fmax drop it),
// so that a NaN coordinate reaches the host's finiteness check
__device__ __forceinline__ double min_keep_nan(double a, double b) { return (b < a || b != b) ? b : a; }
__device__ __forceinline__ double max_keep_nan(double a, double b) { return (b > a || b != b) ? b : a; }

__global__ __launch_bounds__(1024) void k_bbox(int n, const double *x, double *out) {
  __shared__ double sh[6][1024];
  const int t = threadIdx.x;
  double lo[3] = {HUGE_VAL, HUGE_VAL, HUGE_VAL}, hi[3] = {-HUGE_VAL, -HUGE_VAL, -HUGE_VAL};
  for (int i = t; i < n; i += 1024)
    for (int d = 0; d < 3; ++d) {
      lo[d] = min_keep_nan(lo[d], x[3 * i + d]);
      hi[d] = max_keep_nan(hi[d], x[3 * i + d]);
    }
  for (int d = 0; d < 3; ++d) {
    sh[d][t] = lo[d];
    sh[3 + d][t] = hi[d];
  }
  __syncthreads();
  for (int st = 512; st > 0; st >>= 1) {
    if (t < st)
      for (int d = 0; d < 3; ++d) {
        sh[d][t] = min_keep_nan(sh[d][t], sh[d][t + st]);
        sh[3 + d][t] = max_keep_nan(sh[3 + d][t], sh[3 + d][t + st]);
      }
    __syncthreads();
  }
  if (t < 6) out[t] = sh[t][0];
}

__global__ void k_invert(int n, const int *perm, int *inv) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) inv[perm[i]] = i;
}

// Per long-range incidence entry k (pair slot e = 2 c + side): the partner
// node, this endpoint's row and the partner's row, in three arrays of m.
__global__ void k_lr_records(int m, const int *inc, const int *rows, const int *nodes, int *rec) {
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= m) return;
  const int e = inc[k], c = e >> 1, side = e & 1;
  rec[k] = nodes[2 * c + 1 - side];
  rec[std::size_t(m) + k] = rows[2 * c + side];
  rec[2 * std::size_t(m) + k] = rows[2 * c + 1 - side];
}

// key = the first endpoint's node of pair c, value = c (the short-range
// pairs' spatial order)
__global__ void k_pair_keys(int np, const int *nodes, int *key, int *val) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= np) return;
  key[c] = nodes[2 * c];
  val[c] = c;
}

// dst[2 i + side] = src[2 order[i] + side]
__global__ void k_gather_pairs(int np, const int *order, const int *src, int *dst) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= 2 * np) return;
  dst[t] = src[2 * order[t >> 1] + (t & 1)];
}

__global__ void k_relabel(int m, const int *inv, int *nodes) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t < m) nodes[t] = inv[nodes[t]];
}

}  // namespace

void Evaluator::set_topology(std::int64_t n_rows, const std::int32_t *owner, int sr_kind, std::int64_t sr_inum,
                             const std::int32_t *sr_ilist, const std::int64_t *sr_off,
                             const std::int32_t *sr_neigh, std::int64_t lr_inum,
                             const std::int32_t *lr_ilist, const std::int64_t *lr_off,
                             const std::int32_t *lr_neigh) {
  if (!system_ready_) throw std::logic_error("SO3LR: set the system before the topology");
  const std::int64_t n = n_;
  if (n_rows < n || !owner) throw std::invalid_argument("SO3LR: fewer rows than owned atoms");
  if (n_rows >= (std::int64_t(1) << 31)) throw TopologyError("SO3LR: more than 2^31 rows");
  hipStream_t s = stream_;
  // host-side checks of the list shapes (O(inum)); the entries are checked on the device
  struct List {
    const char *what;
    bool full;
    std::int64_t inum;
    const std::int32_t *ilist;
    const std::int64_t *off;
    const std::int32_t *neigh;
    Buffer *d_ilist, *d_off, *d_neigh, *rows, *nodes, *inc_off, *inc;
    std::int64_t entries = 0, pairs = 0;
  };
  List lists[2] = {
      {"short-range", sr_kind == 0, sr_inum, sr_ilist, sr_off, sr_neigh, top_ilist_[0], top_off_[0], top_neigh_[0],
       sr_rows_, sr_nodes_, sr_inc_off_, sr_inc_},
      {"long-range", false, lr_inum, lr_ilist, lr_off, lr_neigh, top_ilist_[1], top_off_[1], top_neigh_[1], lr_rows_,
       lr_nodes_, lr_inc_off_, lr_inc_}};
  for (List &L : lists) {
    const std::string w = L.what;
    if (L.inum < 0 || (L.inum > 0 && (!L.ilist || !L.off || !L.neigh)))
      throw std::invalid_argument("SO3LR: invalid " + w + " neighbour list");
    if (L.inum > n) throw TopologyError("SO3LR: the " + w + " list has more receivers than owned atoms");
    if (L.inum == 0) continue;
    if (L.off[0] != 0) throw TopologyError("SO3LR: " + w + " offsets must start at 0");
    for (std::int64_t k = 0; k < L.inum; ++k) {
      if (L.off[k + 1] < L.off[k]) throw TopologyError("SO3LR: decreasing " + w + " offsets");
      if (L.ilist[k] < 0 || L.ilist[k] >= n) throw TopologyError("SO3LR: " + w + " receiver is not an owned row");
    }
    L.entries = L.off[L.inum];
    if (L.entries >= (std::int64_t(1) << 30))
      throw TopologyError("SO3LR: the " + w + " list exceeds 2^30 entries");
  }
  // the raw lists cross to the device once; everything else is built there
  int *d_owner = ensure<int>(top_owner_, std::size_t(n_rows));
  TOPO_CHECK(hipMemcpyAsync(d_owner, owner, std::size_t(n_rows) * sizeof(int), hipMemcpyHostToDevice, s));
  for (List &L : lists) {
    if (L.inum == 0) continue;
    TOPO_CHECK(hipMemcpyAsync(ensure<int>(L.d_ilist, std::size_t(L.inum)), L.ilist, std::size_t(L.inum) * sizeof(int),
                              hipMemcpyHostToDevice, s));
    TOPO_CHECK(hipMemcpyAsync(ensure<std::int64_t>(L.d_off, std::size_t(L.inum) + 1), L.off,
                              (std::size_t(L.inum) + 1) * sizeof(std::int64_t), hipMemcpyHostToDevice, s));
    TOPO_CHECK(hipMemcpyAsync(ensure<int>(L.d_neigh, std::size_t(std::max<std::int64_t>(L.entries, 1))), L.neigh,
                              std::size_t(L.entries) * sizeof(int), hipMemcpyHostToDevice, s));
  }
  // device-side fault word and counters: [0] fault bits, [1..2] dropped (u64)
  int *stat = ensure<int>(top_stat_, 8);
  hipLaunchKernelGGL(k_fill_ints, dim3(1), dim3(64), 0, s, 8, stat, 0);
  int *fault = stat;
  auto *dropped = reinterpret_cast<unsigned long long *>(stat + 2);
  hipLaunchKernelGGL(k_check_owner, dim3(unsigned((n_rows + 255) / 256)), dim3(256), 0, s, int(n_rows), int(n),
                     d_owner, fault);
  // pass 1: counts and row offsets of both lists, one read-back
  int *totals_dev[2] = {nullptr, nullptr};
  for (int w = 0; w < 2; ++w) {
    List &L = lists[w];
    if (L.inum == 0) continue;
    int *cnt = ensure<int>(top_cnt_[w], std::size_t(L.inum));
    int *poff = ensure<int>(top_poff_[w], std::size_t(L.inum) + 1);
    const dim3 grid(unsigned((L.inum + 3) / 4));
    const int *il = static_cast<const int *>(L.d_ilist->p);
    const std::int64_t *of = static_cast<const std::int64_t *>(L.d_off->p);
    const int *ng = static_cast<const int *>(L.d_neigh->p);
    if (L.full)
      hipLaunchKernelGGL((k_list_walk<true, true>), grid, dim3(256), 0, s, int(L.inum), int(n_rows), il, of, ng,
                         d_owner, cnt, dropped, fault, nullptr, nullptr, nullptr);
    else
      hipLaunchKernelGGL((k_list_walk<false, true>), grid, dim3(256), 0, s, int(L.inum), int(n_rows), il, of, ng,
                         d_owner, cnt, nullptr, fault, nullptr, nullptr, nullptr);
    hipLaunchKernelGGL(k_scan_rows, dim3(1), dim3(1024), 0, s, int(L.inum), cnt, poff);
    totals_dev[w] = poff + L.inum;
  }
  int host_stat[8] = {0}, host_tot[2] = {0, 0};
  TOPO_CHECK(hipMemcpyAsync(host_stat, stat, sizeof(host_stat), hipMemcpyDeviceToHost, s));
  for (int w = 0; w < 2; ++w)
    if (totals_dev[w]) TOPO_CHECK(hipMemcpyAsync(&host_tot[w], totals_dev[w], sizeof(int), hipMemcpyDeviceToHost, s));
  TOPO_CHECK(hipStreamSynchronize(s));
  const int bad = host_stat[0];
  if (bad & kBadOwner)
    throw TopologyError("SO3LR: owner_of_row must be the identity on owned rows and map ghosts to owned atoms");
  if (bad & kBadRow) throw TopologyError("SO3LR: a neighbour row is out of range");
  if (bad & kSelfImage)
    throw TopologyError("SO3LR: a neighbour list pairs an atom with its own periodic image; the box is too small "
                        "for the cutoff");
  unsigned long long host_dropped = 0;
  std::memcpy(&host_dropped, host_stat + 2, sizeof(host_dropped));
  if (lists[0].full && lists[0].inum > 0 && host_dropped != (unsigned long long)host_tot[0])
    throw TopologyError("SO3LR: the full short-range list is not symmetric (an edge lacks its reverse)");
  // pass 2: the pair tables, then the node-major incidence of each.  The
  // sort buffers are shared by both lists: sized for the larger one before
  // anything is launched, so no reallocation lands between the two sorts.
  int bits = 1;
  while ((std::int64_t(1) << bits) < n) ++bits;
  std::size_t m_max = 1, tmp_max = 1;
  for (int w = 0; w < 2; ++w) {
    const std::int64_t m = 2 * std::int64_t(host_tot[w]);
    if (m == 0) continue;
    std::size_t tmp_bytes = 0;
    TOPO_CHECK(hipcub::DeviceRadixSort::SortPairs(nullptr, tmp_bytes, static_cast<const int *>(nullptr),
                                                  static_cast<int *>(nullptr), static_cast<const int *>(nullptr),
                                                  static_cast<int *>(nullptr), int(m), 0, bits, s));
    m_max = std::max(m_max, std::size_t(m));
    tmp_max = std::max(tmp_max, tmp_bytes);
  }
  // the spatial node order of the first evaluation (order_rows_nodes) runs
  // on buffers sized here, so that evaluation allocates nothing: a single
  // system only (packed images keep their nodes contiguous per image)
  const bool reorder = n_images_ == 1 && n >= 2;
  if (reorder) {
    std::size_t tmp_bytes = 0;
    TOPO_CHECK(hipcub::DeviceRadixSort::SortPairs(nullptr, tmp_bytes, static_cast<const int *>(nullptr),
                                                  static_cast<int *>(nullptr), static_cast<const int *>(nullptr),
                                                  static_cast<int *>(nullptr), int(n), 0, 30, s));
    tmp_max = std::max(tmp_max, tmp_bytes);
    const std::size_t nz = std::size_t(n);
    ensure<int>(nb_key_, nz); ensure<int>(nb_idx_, nz); ensure<int>(nb_skey_, nz); ensure<int>(nb_sidx_, nz);
    ensure<int>(perm_, nz); ensure<int>(nz_, nz); ensure<double>(nx0_, nz * std::size_t(F_));
    ensure<double>(top_box_, 6);
    perm_host_.resize(nz);
  }
  int *slots = ensure<int>(top_slots_, m_max), *skeys = ensure<int>(top_skeys_, m_max);
  void *tmp = ensure<char>(top_tmp_, tmp_max);
  for (int w = 0; w < 2; ++w) {
    List &L = lists[w];
    L.pairs = host_tot[w];
    const std::size_t P = std::size_t(std::max<std::int64_t>(L.pairs, 1));
    ensure<int>(L.rows, 2 * P);
    ensure<int>(L.nodes, 2 * P);
    ensure<int>(L.inc_off, std::size_t(n) + 1);
    ensure<int>(L.inc, 2 * P);
  }
  for (int w = 0; w < 2; ++w) {
    List &L = lists[w];
    int *rows = static_cast<int *>(L.rows->p), *nodes = static_cast<int *>(L.nodes->p);
    int *inc_off = static_cast<int *>(L.inc_off->p), *inc = static_cast<int *>(L.inc->p);
    if (L.pairs == 0) {
      hipLaunchKernelGGL(k_fill_ints, dim3(unsigned((n + 1 + 255) / 256)), dim3(256), 0, s, int(n + 1), inc_off, 0);
      continue;
    }
    const dim3 grid(unsigned((L.inum + 3) / 4));
    const int *il = static_cast<const int *>(L.d_ilist->p);
    const std::int64_t *of = static_cast<const std::int64_t *>(L.d_off->p);
    const int *ng = static_cast<const int *>(L.d_neigh->p);
    const int *poff = static_cast<const int *>(top_poff_[w]->p);
    if (L.full)
      hipLaunchKernelGGL((k_list_walk<true, false>), grid, dim3(256), 0, s, int(L.inum), int(n_rows), il, of, ng,
                         d_owner, nullptr, nullptr, nullptr, poff, rows, nodes);
    else
      hipLaunchKernelGGL((k_list_walk<false, false>), grid, dim3(256), 0, s, int(L.inum), int(n_rows), il, of, ng,
                         d_owner, nullptr, nullptr, nullptr, poff, rows, nodes);
    // incidence: endpoint slots 2p + side sorted by their node (stable).
    // A topology that the first evaluation puts in spatial node order
    // (order_rows_nodes) gets its incidence there, from the relabelled nodes,
    // and no evaluation runs before that: it is not sorted twice.
    if (reorder) continue;
    const int m = int(2 * L.pairs);
    hipLaunchKernelGGL(k_iota, dim3(unsigned((m + 255) / 256)), dim3(256), 0, s, m, slots);
    std::size_t tmp_bytes = tmp_max;
    TOPO_CHECK(hipcub::DeviceRadixSort::SortPairs(tmp, tmp_bytes, static_cast<const int *>(nodes), skeys,
                                                  static_cast<const int *>(slots), inc, m, 0, bits, s));
    hipLaunchKernelGGL(k_segment_starts, dim3(unsigned((m + 1 + 255) / 256)), dim3(256), 0, s, m, int(n), skeys,
                       inc_off);
  }
  p_sr_ = lists[0].pairs;
  p_lr_ = lists[1].pairs;
  if (reorder)  // built by order_rows_nodes, on a buffer sized here
    ensure<int>(lr_rec_, 3 * std::size_t(std::max<std::int64_t>(2 * p_lr_, 1)));
  else
    build_lr_records();
  TOPO_CHECK(hipGetLastError());
  TOPO_CHECK(hipStreamSynchronize(s));
  n_rows_ = n_rows;
  shift_mode_ = false;
  permuted_ = false;
  rows_order_pending_ = reorder;
  topology_ready_ = true;
  ++topo_version_;
  evaluated_ = false;
  act_cap_ = 0;  // counted again by the next evaluation
}

// The nodes of a LAMMPS-list topology in the Morton order of the owned rows'
// positions (the first n rows), the analogue of LAMMPS's own periodic atom
// sort: the node-major gathers (attention, long range) then read partner rows
// from a compact region that one XCD's L2 serves, whatever order the caller
// keeps its atoms in.  The endpoint nodes are relabelled; the short-range
// pairs are put in the order of their first endpoint's new node (stable), so
// the pair-major filter kernels read endpoint rows of spatial neighbours as
// on the device reneighbor path (the long-range pairs, read node-major
// through their records, keep their list order); each incidence list is
// sorted again by node (stable, so a node's entries stay in increasing pair
// order).  Runs once per topology, at its first evaluation, on buffers
// set_topology sized.
void Evaluator::order_rows_nodes(const double *x) {
  // rows_order_pending_ stays set until the order is built: a refusal below
  // (non-finite positions) leaves the topology exactly as set_topology left
  // it, unsorted incidence and all, and the next evaluation orders it again
  const int n = int(n_);
  hipStream_t s = stream_;
  double *box = ensure<double>(top_box_, 6);
  hipLaunchKernelGGL(k_bbox, dim3(1), dim3(1024), 0, s, n, x, box);
  double hb[6];
  TOPO_CHECK(hipMemcpyAsync(hb, box, sizeof(hb), hipMemcpyDeviceToHost, s));
  TOPO_CHECK(hipStreamSynchronize(s));
  MortonBox B;
  for (int d = 0; d < 3; ++d) {
    if (!std::isfinite(hb[d]) || !std::isfinite(hb[3 + d]))
      throw std::invalid_argument("SO3LR: non-finite positions");
    B.lo[d] = hb[d];
    B.len[d] = std::max(hb[3 + d] - hb[d], 1e-6);
  }
  const std::size_t nz = std::size_t(n);
  int *key = ensure<int>(nb_key_, nz), *idx = ensure<int>(nb_idx_, nz), *skey = ensure<int>(nb_skey_, nz);
  int *inv = ensure<int>(nb_sidx_, nz), *perm = ensure<int>(perm_, nz);
  const unsigned gn = unsigned((n + 255) / 256);
  hipLaunchKernelGGL(k_morton, dim3(gn), dim3(256), 0, s, n, x, B, key, idx);
  void *tmp = top_tmp_->p;
  std::size_t tmp_bytes = top_tmp_->bytes;
  TOPO_CHECK(hipcub::DeviceRadixSort::SortPairs(tmp, tmp_bytes, static_cast<const int *>(key), skey,
                                                static_cast<const int *>(idx), perm, n, 0, 30, s));
  hipLaunchKernelGGL(k_invert, dim3(gn), dim3(256), 0, s, n, perm, inv);
  int bits = 1;
  while ((std::int64_t(1) << bits) < n) ++bits;
  struct Inc {
    Buffer *rows, *nodes, *inc_off, *inc;
    std::int64_t pairs;
    bool reorder_pairs;
  };
  const Inc lists[2] = {{sr_rows_, sr_nodes_, sr_inc_off_, sr_inc_, p_sr_, true},
                        {lr_rows_, lr_nodes_, lr_inc_off_, lr_inc_, p_lr_, false}};
  for (const Inc &L : lists) {
    const int m = int(2 * L.pairs);
    if (m == 0) continue;  // its node offsets are all zero already
    int *nodes = static_cast<int *>(L.nodes->p), *slots = static_cast<int *>(top_slots_->p),
        *skeys = static_cast<int *>(top_skeys_->p);
    const unsigned gm = unsigned((m + 255) / 256);
    hipLaunchKernelGGL(k_relabel, dim3(gm), dim3(256), 0, s, m, inv, nodes);
    if (L.reorder_pairs) {
      // the pairs in the order of their first node: keys and values in the
      // two halves of slots, sorted into those of skeys (both hold 2 P),
      // then rows and nodes gathered through slots
      const int np = m / 2;
      int *rows = static_cast<int *>(L.rows->p);
      const unsigned gp = unsigned((np + 255) / 256);
      hipLaunchKernelGGL(k_pair_keys, dim3(gp), dim3(256), 0, s, np, nodes, slots, slots + np);
      tmp_bytes = top_tmp_->bytes;
      TOPO_CHECK(hipcub::DeviceRadixSort::SortPairs(tmp, tmp_bytes, static_cast<const int *>(slots), skeys,
                                                    static_cast<const int *>(slots + np), skeys + np, np, 0, bits,
                                                    s));
      for (int *arr : {rows, nodes}) {
        hipLaunchKernelGGL(k_gather_pairs, dim3(gm), dim3(256), 0, s, np, skeys + np, arr, slots);
        TOPO_CHECK(hipMemcpyAsync(arr, slots, std::size_t(m) * sizeof(int), hipMemcpyDeviceToDevice, s));
      }
    }
    hipLaunchKernelGGL(k_iota, dim3(gm), dim3(256), 0, s, m, slots);
    tmp_bytes = top_tmp_->bytes;
    TOPO_CHECK(hipcub::DeviceRadixSort::SortPairs(tmp, tmp_bytes, static_cast<const int *>(nodes), skeys,
                                                  static_cast<const int *>(slots), static_cast<int *>(L.inc->p), m,
                                                  0, bits, s));
    hipLaunchKernelGGL(k_segment_starts, dim3(unsigned((m + 1 + 255) / 256)), dim3(256), 0, s, m, n, skeys,
                       static_cast<int *>(L.inc_off->p));
  }
  build_lr_records();
  hipLaunchKernelGGL(k_gather_int, dim3(gn), dim3(256), 0, s, n, perm, static_cast<const int *>(z_->p),
                     static_cast<int *>(nz_->p));
  hipLaunchKernelGGL(k_gather_rows, dim3(unsigned((nz * std::size_t(F_) + 255) / 256)), dim3(256), 0, s, n, F_, perm,
                     static_cast<const double *>(x0_->p), static_cast<double *>(nx0_->p));
  TOPO_CHECK(hipMemcpyAsync(perm_host_.data(), perm, nz * sizeof(int), hipMemcpyDeviceToHost, s));
  TOPO_CHECK(hipGetLastError());
  TOPO_CHECK(hipStreamSynchronize(s));
  permuted_ = true;
  rows_order_pending_ = false;
  ++topo_version_;
}

// The long-range records of the current LAMMPS-list incidence (its pairs,
// rows and nodes); after set_topology and after the nodes are relabelled.
void Evaluator::build_lr_records() {
  const int m = int(2 * p_lr_);
  lr_rec_len_ = m;
  int *rec = ensure<int>(lr_rec_, 3 * std::size_t(std::max(m, 1)));
  if (m == 0) return;
  hipLaunchKernelGGL(k_lr_records, dim3(unsigned((m + 255) / 256)), dim3(256), 0, stream_, m,
                     static_cast<const int *>(lr_inc_->p), static_cast<const int *>(lr_rows_->p),
                     static_cast<const int *>(lr_nodes_->p), rec);
}

}  // namespace so3lr_amd
