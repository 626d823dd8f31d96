// SO3LR E + F + virial evaluator on one gfx950 GPU (host side of the kernels).
//
// Pair-based, deterministic design.  The short-range graph is kept as unique
// pairs {a, b} (the reference evaluates both directed edges of a pair
// separately).  The filters depend on the pair only (distance and the
// symmetric equivariant invariant), so they are evaluated once per pair and
// shared by both directions; everything direction-dependent (attention
// coefficients, harmonics parity) is carried per direction.  Node sums that
// the reference forms with atomics are gathers over a node-major incidence
// list (each node sees every pair it belongs to), so results do not depend on
// thread timing.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "device_math.hpp"
#include "generic.hpp"
#include "model.hpp"

namespace so3lr_amd {

// A failure of the HIP runtime or of the device (allocation, launch, copy,
// device selection): reported as SO3LR_ERR_DEVICE at the C ABI.
struct DeviceError : std::runtime_error {
  explicit DeviceError(const std::string &what) : std::runtime_error(what) {}
};

// Neighbour lists inconsistent with the rows or with each other: reported as
// SO3LR_ERR_TOPOLOGY at the C ABI.
struct TopologyError : std::runtime_error {
  explicit TopologyError(const std::string &what) : std::runtime_error(what) {}
};

// Host-side weight layouts of the fp64 MFMA kernels (evaluator.hip): the
// transpose of a rows x cols row-major matrix; a bias of length M in MFMA
// accumulator order (a D tile starts from it); an M x K row-major matrix in
// MFMA A-operand order, 16-row tiles by 16-wide K chunks.
std::vector<double> transpose(const std::vector<double> &w, std::size_t rows, std::size_t cols);
std::vector<double> bias_acc(const std::vector<double> &b, std::size_t M);
std::vector<double> permute_mfma(const std::vector<double> &w, std::size_t M, std::size_t K);

// Device weight pointers for one interaction block.
struct BlockWeights {
  const double *wqkv;                   // (5, 4, 32, 32): q k v q_ev k_ev, (head, in, out)
  const double *fw0[2], *fb0[2];        // filter {inv, ev} radial layer 0 (128, 32), (128)
  const double *fw1[2], *fb1[2];        // radial layer 1 (128, 128), (128)
  const double *fw1t[2];                // its transpose (in, out)
  const double *fe0[2], *feb0[2];       // spherical layer 0 (32, 4), (32)
  const double *fe1[2], *feb1[2];       // spherical layer 1 (128, 32), (128)
  const double *fe1t[2];                // its transpose
  const double *att_cg, *int_cg;        // (24)
  const double *ln1w, *ln1b, *ln2w, *ln2b;
  const double *m1t, *m1b, *m2t, *m2b;  // MLP weights transposed (in, out)
  const double *m1w, *m2w;              // (out, in) for the reverse
  const double *intt, *intb, *intw;     // interaction (132x132): transposed and (out, in)
  // MFMA operand order of the filter weights (see permute_mfma in evaluator.hip)
  const double *w0p[2], *w1p[2], *e0p[2], *e1p[2];     // forward
  const double *w1tp[2], *w0tp[2], *e1tp[2], *e0tp[2];  // reverse (transposes)
  const double *b0p[2], *eb0p[2], *ob1p[2];             // biases in accumulator order
  const double *ob1p0[2];                               // ob1p with the ev = 0 spherical branch folded in (block 0) (ob1 = b1 + eb1)
  const double *ob10[2];                                // the same output bias in natural order (block 0's tables)
  const double *e0pk[2];                                // spherical layer 0, one v4d per lane
  // radial tables of the blocks after 0 (the RT filter kernels): per
  // interval and filter, the radial branch W1 silu(W0 rbf + b0) + ob1 as
  // 16 powers of t (an MFMA A operand of 128 x 16) and its r-derivative
  // (16 x 128); null without the tables
  const double *rrow, *rdr;
  // MFMA operand order of the node layers: forward and reverse (transpose)
  const double *qkvp, *qkvtp;           // per head (160 x 32) and (32 x 160)
  const double *m1p, *m2p, *m1tp, *m2tp;
  const double *intp, *inttp;           // 132 x 132, K padded to 144
  const double *m1bp, *m2bp, *intbp;    // node-layer biases in accumulator order
};

struct HeadWeights {
  int ho = 320;              // first-layer width: energy 128 | charge 128 | Hirshfeld 64 (| C6 64)
  const double *w1p, *w1tp;  // MFMA operand order: (ho x 128) and its transpose
  const double *b1p;         // first-layer bias (ho) in accumulator order
  const double *w1t;    // (128, 320): energy | charge | Hirshfeld first layers, transposed
  const double *w1;     // (320, 128)
  const double *b1;     // (320)
  const double *ew2, *qw2;  // (128)
  double eb2, qb2;
  const double *escale, *eshift;  // (118)
  const double *qemb;             // (100)
  const double *hkey_bwd;         // (100, 64): u[z][i] = sum_j hw2[j][i] hqemb[z][j]
  const double *hkey_c;           // (100): hqemb[z] . hb2
  const double *hqemb, *hvshift;  // (100, 64), (100)
  const double *ckey_bwd, *ckey_c, *cvshift;  // the C6 ratio head's, as hkey_bwd, hkey_c, hvshift (or null)
  const double *rbf_b, *rbf_k, *rbf_kr;  // (32) each
  const double *rbf_e;                   // (32) Bernstein recurrence factors (FilterMfma::rbf_e)
  const double *exp2_256;                // 2^(j/256), j < 256 (lean e^x of the filter kernels)
  const double *alpha_ref, *c6_ref;
  int n_ref;
};

class Evaluator {
 public:
  Evaluator(std::shared_ptr<Model> model, int device);
  ~Evaluator();

  const Model &model() const { return *model_; }
  void set_system(const std::vector<std::int32_t> &z, const std::vector<std::int64_t> &image_offsets,
                  const std::vector<double> &charges, const std::vector<double> &multiplicities);
  void set_topology(std::int64_t n_rows, const std::int32_t *owner_of_row, int sr_kind,
                    std::int64_t sr_inum, const std::int32_t *sr_ilist, const std::int64_t *sr_off,
                    const std::int32_t *sr_neigh, std::int64_t lr_inum, const std::int32_t *lr_ilist,
                    const std::int64_t *lr_off, const std::int32_t *lr_neigh);
  // x_rows_dev: device positions of all rows.  Forces/eatom to device
  // buffers (may be null); energy/virial to host.
  void compute_device(const double *x_rows_dev, int flags, double *f_dev, double *eatom_dev,
                      double *energy, double *virial);
  void compute_host(const double *x_rows, int flags, double *f, double *eatom, double *energy,
                    double *virial);
  // As compute_device, with every work buffer of the evaluation carved from
  // the library's static device scratch array (no allocation, no graph, no
  // events); throws std::invalid_argument when the system needs more than
  // scratch_capacity() bytes.  Per-atom terms and the per-atom virial are not
  // kept afterwards (last_terms / last_vatom refuse).
  void compute_device_noalloc(const double *x_rows_dev, int flags, double *f_dev, double *eatom_dev,
                              double *energy, double *virial);
  static std::size_t scratch_capacity();
  void last_terms(double *learned, double *zbl, double *lr, double *charges, double *hirshfeld,
                  double *totals, double *image_energy);
  // Per-atom virial of the last evaluation (n_owned x 6, atom order), to host
  // or device memory.
  void last_vatom(double *out, bool on_device);
  // HBM-resident reneighbor from owned positions (wrapped in place); after it,
  // compute_device takes owned positions.  Orthogonal box [lo, hi).
  void build_topology_device(double *x_owned, const double lo[3], const double hi[3], const int per[3],
                             double skin);
  void set_box(const double lo[3], const double hi[3]);
  bool shift_mode() const { return shift_mode_; }
  void set_stream(hipStream_t s) { stream_ = s ? s : own_stream_; }
  std::int64_t n_owned() const { return n_; }
  std::int64_t sr_active() const { return last_active_; }
  std::int64_t sr_candidates() const { return p_sr_; }
  std::int64_t lr_candidates() const { return p_lr_; }
  std::int64_t device_bytes() const { return bytes_; }
  // Kernel timing with HIP events on the launch stream (measurement hook).
  void set_timing(bool on) {  // enabling clears the totals; disabling keeps them for reading
    if (on) timings_.clear();
    timing_ = on;
  }
  bool timing_read(const std::string &kernel, double &total_ms, std::int64_t &launches,
                   std::int64_t &units) const;

 private:
  std::shared_ptr<Model> model_;
  int device_;
  hipStream_t own_stream_ = nullptr, stream_ = nullptr;
  std::int64_t bytes_ = 0;
  std::vector<void *> weight_allocs_;
  BlockWeights bw_[kMaxBlocks];
  HeadWeights hw_{};
  ZblParams zbl_{};
  LrParams lr_{};
  double gamma_ = 0, rc_ = 0, avg_ = 1, ln_eps_ = 1e-6;
  int layers_ = 0;
  // architecture options (Architecture in model.hpp)
  int norm1_ = 0, norm2_ = 0;   // NormMode of the two normalisation positions
  bool qk_norm_ = false, c6_ = false;
  std::vector<double> resid_, x0l_;  // residual scalars per block (empty: none)
  ChargeSpin charge_spin_;
  std::vector<double> emb_w_;  // (F, 118)
  int F_ = kF;                 // invariant features
  // the generic-width path (models other than the v1 widths) and its buffers
  std::unique_ptr<GenericPath> gen_;

  // system
  std::int64_t n_ = 0, n_images_ = 0, n_rows_ = 0;
  std::vector<std::int64_t> image_offsets_;
  bool system_ready_ = false, topology_ready_ = false, evaluated_ = false;
  std::int64_t p_sr_ = 0, p_lr_ = 0, last_active_ = 0;

  struct Buffer {
    void *p = nullptr;
    std::size_t bytes = 0;
  };
  std::vector<Buffer *> buffers_;
  Buffer *buf(const char *name);
  template <class T>
  T *ensure(Buffer *b, std::size_t count) {
    const std::size_t need = (count ? count : 1) * sizeof(T);
    if (b->bytes < need) {
      if (b->p) {
        if (hipFree(b->p) != hipSuccess) throw DeviceError("HIP error in hipFree");
        bytes_ -= std::int64_t(b->bytes);
      }
      b->p = nullptr;
      const std::size_t cap = need + need / 8;  // retained capacity with slack
      if (hipMalloc(&b->p, cap) != hipSuccess)
        throw DeviceError("HIP error in hipMalloc: out of device memory (" + std::to_string(cap) + " bytes)");
      b->bytes = cap;
      bytes_ += std::int64_t(cap);
      ++alloc_epoch_;  // a captured graph holds the old address
    }
    return static_cast<T *>(b->p);
  }
  void release_all();
  // Where the work buffers of the evaluation being set up come from: the
  // retained per-context buffers (ensure), a pass that only adds up their
  // sizes, or consecutive 256-byte aligned slices of the static scratch array.
  enum class Carve { Retained, Measure, Scratch };
  Carve carve_ = Carve::Retained;
  char *carve_base_ = nullptr;
  std::size_t carve_used_ = 0;
  template <class T>
  T *take(Buffer *b, std::size_t count) {
    if (carve_ == Carve::Retained) return ensure<T>(b, count);
    const std::size_t bytes = ((count ? count : 1) * sizeof(T) + 255) / 256 * 256;
    T *p = carve_ == Carve::Scratch ? reinterpret_cast<T *>(carve_base_ + carve_used_) : nullptr;
    carve_used_ += bytes;
    return p;
  }
  void compute_impl(const double *x, int flags, double *f_out, double *eatom_out, double *energy, double *virial,
                    bool from_scratch);
  // LAMMPS-list path: the nodes are put in the spatial order of the owned
  // rows' positions at the first evaluation after set_topology (the lists
  // carry no positions); rows_order_pending_ until then
  void order_rows_nodes(const double *x_rows);
  bool rows_order_pending_ = false;
  char *scratch_dev_ = nullptr;   // this device's copy of the static scratch array
  bool last_from_scratch_ = false;  // the last evaluation's buffers were scratch slices

  // node-sized device buffers (named members so the kernels' arguments read clearly)
  Buffer *z_, *x0_, *img_of_node_, *img_off_, *img_q_;
  Buffer *xs_, *evs_, *qkv_, *aev_, *n1_, *n1hat_, *n1is_, *hpre_, *tout_, *pre2hat_, *pre2is_;
  Buffer *ainv_, *act_;
  Buffer *hhead_, *heff_, *eatom_, *qraw_, *q_, *hir_, *qseed_;
  Buffer *elr_, *dq_, *dh_, *flr_, *vlr_, *elr_parts_, *ezbl_;
  Buffer *gx_, *gev_, *gainv_, *gaev_, *gqkv_, *ghead_;
  Buffer *qkis_, *c6eff_, *c6r_, *dc_;  // QK normalisation 1/rms; C6 head logit, ratio, dE/dratio
  Buffer *fout_, *etot_, *red_, *red_part_;
  // pair-sized buffers
  Buffer *owner_, *sr_rows_, *sr_nodes_, *sr_inc_off_, *sr_inc_, *lr_rows_, *lr_nodes_,
      *lr_inc_off_, *lr_inc_, *blk_count_, *n_active_, *cand2act_;
  // LAMMPS-list long range, per incidence entry: partner node, own row,
  // partner row (three arrays of lr_rec_len_ entries; build_lr_records)
  Buffer *lr_rec_;
  std::int64_t lr_rec_len_ = 0;
  void build_lr_records();
  Buffer *pa_, *pv_, *pr_, *pY_, *pfc_, *pzbl_, *ps_, *pf_, *palpha_;
  Buffer *df_, *dfc_, *psc_, *ds_, *dr_, *dY_, *pg_;
  Buffer *iact_, *iother_;  // per step: incidence entry -> active pair * 2 + side, partner node
  Buffer *gbuf_[GenericPath::kBuffers] = {};
  Buffer *probe_;           // the active-pair count of a new topology
  // capacity (pairs) of the active-pair buffers for the current topology; 0
  // until the first evaluation on it counts the active pairs
  std::int64_t act_cap_ = 0;
  Buffer *xrows_, *fhost_, *vatom_;
  // device reneighbor
  Buffer *nb_key_, *nb_idx_, *nb_skey_, *nb_sidx_, *nb_cstart_, *nb_tmp_, *nb_srcnt_, *nb_lrcnt_, *nb_err_,
      *nb_srlist_, *nb_poff_, *sr_code_, *nb_tot_;
  // spatial node order (device reneighbor, or the LAMMPS-list path after its
  // first evaluation): node n holds owned atom perm[n]; node-ordered copies
  // of the per-atom inputs (xn_: positions, device reneighbor path only)
  Buffer *perm_, *nz_, *nx0_, *xn_;
  // LAMMPS lists on the device (set_topology): the raw upload and the build's
  // work buffers; [0] short range, [1] long range
  Buffer *top_owner_, *top_ilist_[2], *top_off_[2], *top_neigh_[2], *top_cnt_[2], *top_poff_[2], *top_stat_,
      *top_slots_, *top_skeys_, *top_tmp_, *top_box_;
  std::vector<int> perm_host_;
  bool permuted_ = false;
  bool shift_mode_ = false;
  std::int64_t lr_entries_ = 0;
  double box_len_[3] = {0, 0, 0};
  double totals_[2] = {0.0, 0.0};
  struct Timing {
    double ms = 0;
    std::int64_t launches = 0, units = 0;
  };
  bool timing_ = false;
  bool naive_filters_ = false;  // SO3LR_NAIVE_FILTERS=1: scalar filter kernels (cross-check)
  // Small systems run the scalar filter kernels: with a few hundred active
  // pairs the fully unrolled MFMA filters are bound by fetching their code
  // into a cold instruction cache (30-40 us per launch).  Decided when a
  // topology's active pairs are counted: at most scalar_pairs_max_ of them
  // (SO3LR_SCALAR_FILTER_PAIRS; 0 never).
  std::int64_t scalar_pairs_max_ = 256;
  bool scalar_now_ = false;
  // Block 0 through element-pair tables (k_filter_fwd_class and
  // k_filter_bwd_class): a one-image system of at most 16 elements, whose
  // block-0 node rows depend on the element alone.  n_cls_ classes (0: the
  // full block-0 kernels); cls_lut_[z] = class of atomic number z; cls_rep0_[c]
  // = first atom of class c in the caller's order.  SO3LR_NO_CLASS_TABLES=1
  // runs the full kernels.
  int n_cls_ = 0;
  bool class_tables_ = true;
  Buffer *cls_lut_, *cls_rep0_, *cls_rep_, *cls_mt_, *cls_c0_, *cls_gv_, *cls_hist_, *cls_order_, *cls_rows_;
  // Block 0's radial tables (k_radial_tables, k_radial_fwd, k_radial_bwd): on
  // the element-pair path, every block-0 logit as a polynomial of r per
  // interval.  radial_ok_: both filters' radial hidden layers fit to the
  // bound (constructor); SO3LR_NO_RADIAL_TABLES=1 keeps the element-pair
  // MFMA kernels.  rad_tab_ holds the element pairs' value and slope tables,
  // sized by set_system and filled by the first evaluation after it
  // (rad_stale_).
  bool radial_tables_ = true, radial_ok_ = false, rad_stale_ = true;
  // the blocks after 0 on their radial tables (BlockWeights::rrow, rdr): every
  // such block's both radial branches fit to the bound; their pairs in
  // buckets of (spatial block, interval), each padded to a multiple of 16
  // slots (rint_order_, -1 in the padding), counted and placed per
  // evaluation (rint_hist_)
  bool radial_blocks_ = false;
  RadialDomain rbl_dom_{};
  Buffer *rint_order_, *rint_hist_;
  RadialDomain rad_dom_{};
  const double *rad_val_ = nullptr, *rad_slope_ = nullptr;  // [filter][interval][power][feature]
  Buffer *rad_tab_;
  // Graph replay of one evaluation: the launch sequence of compute_device is
  // captured when the same call (inputs, outputs, flags, box, stream,
  // topology and buffer addresses) comes twice in a row, and replayed while
  // it keeps coming.
  struct GraphKey {
    const void *x = nullptr, *f = nullptr, *eatom = nullptr;
    int flags = -1;
    double box[3] = {0, 0, 0};
    hipStream_t stream = nullptr;
    std::uint64_t topology = 0, epoch = 0;
    bool operator==(const GraphKey &o) const {
      return x == o.x && f == o.f && eatom == o.eatom && flags == o.flags && box[0] == o.box[0] &&
             box[1] == o.box[1] && box[2] == o.box[2] && stream == o.stream && topology == o.topology &&
             epoch == o.epoch;
    }
  };
  bool use_graphs_ = true;  // SO3LR_NO_GRAPH=1 turns replay off
  hipGraphExec_t graph_exec_ = nullptr;
  GraphKey graph_key_{}, last_key_{};
  std::uint64_t topo_version_ = 1, alloc_epoch_ = 0;
  double *host_out_ = nullptr;  // pinned: energy, virial, totals, active-pair count
  // compute_host's staging: pinned host buffers the library owns (positions
  // in; forces and per-atom energies out), grown as needed
  struct Pinned {
    double *p = nullptr;
    std::size_t count = 0;
  };
  Pinned pin_x_, pin_f_;
  double *pinned(Pinned &b, std::size_t count);
  // a device -> pinned copy that compute_impl enqueues after the evaluation's
  // kernels and before its one wait (compute_host's forces and energies)
  const double *stage_src_ = nullptr;
  double *stage_dst_ = nullptr;
  std::size_t stage_count_ = 0;
  void drop_graph();
  std::map<std::string, Timing> timings_;
  double *last_etot_ = nullptr;
};

}  // namespace so3lr_amd
