// The evaluation at any of the widths the reference's MPI path accepts
// (src/so3lr_capabilities.cpp:54-85): F = 128 or 256 invariant features in
// F / 32 heads of 32, one equivariant head per degree slot, slots of any
// sorted degrees 1..4 (a degree may repeat), R = 32 or 64 radial functions,
// an energy/charge head width of its own.  The v1 widths (F = 128, R = 32,
// degrees 1,2,3,4, head width 128) run on the fused kernels of evaluator.hip;
// every other model runs here.
//
// Same pair-based, deterministic design as the v1 path (and the same
// geometry, long-range, force and virial kernels around it): unique pairs
// {a, b} with both directions carried per pair, node sums as gathers over the
// node-major incidence, no atomics.  The filters over pairs are fused fp64
// MFMA kernels that keep each pair's hidden row in registers (block 0 of a
// one-image system through its element-pair tables); the node-side dense
// layers are one LDS-tiled fp64 GEMM with fused epilogues; the rest are
// node- or pair-major kernels in natural channel order.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <functional>
#include <vector>

#include "model.hpp"
#include "radial_table.hpp"

namespace so3lr_amd {

constexpr int kGMaxE = 72;  // equivariant channels, at most (8 slots of l = 4)

// The widths of one model.  Slot s (equivariant head s) holds channels
// off[s] .. off[s+1]-1 of degree deg[s]; channel c replicates the unique
// harmonic sh[c] (l = 1..4 in order, 2l + 1 each: the 24 values of a pair's
// harmonics row) and belongs to slot slot[c].
struct GDims {
  int F, NH, E, R, FH, HK, NI, HO;  // HO: energy HK | charge HK | Hirshfeld 64 (| C6 64)
  int c6;
  signed char slot[kGMaxE], sh[kGMaxE];
  signed char off[9];
  double par[8];  // (-1)^l of each slot: the harmonics of the reversed direction
  // the channels replicating unique harmonic m: shc[m][0 .. shn[m])
  signed char shn[24], shc[24][8];
};

// Device weights of one interaction block, in the model file's layouts.
struct GBlock {
  const double *wqkv;  // (5, NH, 32, 32): q k v q_ev k_ev, (head, in, out)
  const double *w0[2], *b0[2], *w1[2], *b1[2];    // radial layers (F, R) (F) (F, F) (F)
  const double *e0[2], *eb0[2], *e1[2], *eb1[2];  // spherical layers (FH, NH) (FH) (F, FH) (F)
  // both output layers side by side, (F, F + FH): [W1 | E1], and b1 + eb1,
  // so one GEMM over the hidden row [silu(W0 rbf + b0) | silu(E0 s + e0)]
  const double *wcat[2], *bcat[2];
  // the filters as MFMA operands (permute_mfma; biases in accumulator order,
  // bias_acc): W0 (F x R), E0 (FH x NH, K padded to 16), [W1 | E1], and their
  // transposes; b0, e0, b1 + e1
  const double *w0p[2], *e0p[2], *wcp[2], *w0tp[2], *e0tp[2], *wctp[2];
  const double *b0a[2], *eb0a[2], *bca[2];
  // blocks after 0 on their radial tables: per interval and filter the radial
  // branch W1 silu(W0 rbf + b0) + b1 + e1 as F x 32 powers of t (rows
  // permuted within each tile as wcp's), MFMA A operands; null without them
  const double *rrow;
  // and their slopes transposed, 32 powers x F (permute_mfma_kc, as wctp)
  const double *rdr;
  const double *att_cg, *int_cg;                  // (E)
  const double *ln1w, *ln1b, *ln2w, *ln2b;        // (F); RMSNorm and none: 1 and 0
  const double *m1, *m1b, *m2, *m2b;              // (F, F) (F)
  const double *wi, *bi;                          // (NI, NI) (NI)
};

struct GHeads {
  const double *w1, *b1;      // (HO, F) (HO): the first layers of all heads
  const double *hw2, *hb2;    // Hirshfeld key layer (64, 64) (64)
  const double *cw2, *cb2;    // C6 ratio head key layer (or null)
  const double *ew2, *qw2;    // (HK)
  double eb2, qb2;
  const double *escale, *eshift;  // (118)
  const double *qemb;             // (100)
  const double *hqemb, *hvshift;  // (100, 64) (100)
  const double *cqemb, *cvshift;  // C6 head's (or null)
  const double *rbf_b, *rbf_k, *rbf_kr;  // (R)
  const double *exp2_256;                // 2^(j/256), j < 256 (exp_tab)
};

// What one evaluation hands the generic path: the shared inputs (active
// pairs, incidence, embedding) and where its outputs go.
struct GContext {
  hipStream_t s;
  int N, cap;              // nodes; capacity of the active-pair buffers
  const int *nact;         // active pairs found (device)
  const int *pa;           // (cap, 2) endpoints a, b; v = x_a - x_b
  const double *pr, *pY, *pfc;  // distance, 24 harmonics of v / r, cutoff
  const int *inc_off, *iact, *iother;  // node-major incidence: pair * 2 + side, partner
  const int *z;
  const double *x0;        // (N, F) embedding
  double inv_avg, ln_eps, gamma, rc;
  int norm1, norm2, qk_norm;
  const std::vector<double> *resid, *x0l;
  // heads forward (outputs)
  double *eatom, *qraw, *heff, *hir, *c6eff, *c6r;
  // heads reverse (inputs): charge seed after the image mean, dE/dh, dE/dc
  const double *qseed, *dh, *dc;
  // reverse (outputs): dE/dY of the 24 harmonics per pair (side-0
  // orientation), dE/dr per pair (added to)
  double *dY, *dr;
  // when set, runs a launch sequence under a name for the evaluator's
  // per-kernel timing (HIP events around it; units: active pairs)
  std::function<void(const char *, const std::function<void()> &)> timed;
  // block 0 through element-pair tables (a one-image system, whose block-0
  // rows depend on the element alone): cls_C classes (0: the full filters),
  // the class of each atomic number, and the node that holds each class's
  // first atom (device)
  int cls_C = 0;
  const int *cls_lut = nullptr, *cls_rep = nullptr;
  // the active pairs in element-pair order (key min C + max), each bucket
  // padded with -1 to a multiple of kB0Pad slots: slot q holds pair
  // cls_order[q], the slots end at *cls_slots (device)
  const int *cls_order = nullptr, *cls_slots = nullptr;
  static constexpr int kB0Pad = 32;
  // block 0's radial tables (with the element-pair tables, when the model's
  // fits hold): the element pairs' value and slope tables (GenericPath::
  // radial_record() doubles per element pair and interval each), filled by
  // this evaluation when rad_build; null: the element-pair MFMA kernels
  double *rad_tab = nullptr;
  bool rad_build = false;
  // the blocks after 0 on their radial tables: the active pairs in buckets
  // of (spatial block, interval), padded with -1 to multiples of 16 slots;
  // the slots end at *rint_slots (device); null: the full forward filters
  const int *rint_order = nullptr, *rint_slots = nullptr;
  int rint_max = 0;  // slots at most
};

class GenericPath {
 public:
  // upload: copies a host vector to device memory the evaluator owns.
  // fit_radial: fit block 0's radial hidden layers for the radial tables.
  GenericPath(const Model &m, const std::function<const double *(const std::vector<double> &)> &upload,
              bool fit_radial);
  // block 0's radial tables: whether the fits hold, and the doubles of one
  // table record (element pair and interval: kRadialCoefs x 4 NH logits)
  bool radial_ok() const { return radial_ok_; }
  // the blocks after 0's radial tables: whether every fit holds, their domain
  bool radial_blocks_ok() const { return radial_blocks_ok_; }
  const RadialDomain &rbl_domain() const { return rbl_dom_; }
  std::size_t radial_record() const { return std::size_t(kRadialCoefs) * 4 * d_.NH; }
  const GDims &dims() const { return d_; }
  int F() const { return d_.F; }
  // The work buffers of one evaluation: take(id, doubles) returns buffer id's
  // memory (the evaluator's retained buffers or scratch slices).
  // C: the element classes of block 0's tables (0: none)
  static constexpr int kBuffers = 48;
  void carve(int N, int cap, int C, const std::function<double *(int, std::size_t)> &take);
  // Blocks and heads forward (to the heads' outputs), then, after the
  // evaluator's long-range step, heads and blocks in reverse.
  void forward(const GContext &c);
  void reverse(const GContext &c);
  double *pf_rows(const GContext &c, int b) const;

 private:
  GDims d_{};
  int layers_ = 0;
  GBlock bw_[kMaxBlocks];
  GHeads hw_{};
  double *b_[kBuffers] = {};
  // block 0's radial fits, [filter][interval][power][feature] (radial_table.hpp)
  bool radial_ok_ = false, radial_blocks_ok_ = false;
  RadialDomain rad_dom_{}, rbl_dom_{};
  const double *rad_val_ = nullptr, *rad_slope_ = nullptr;
};

}  // namespace so3lr_amd
