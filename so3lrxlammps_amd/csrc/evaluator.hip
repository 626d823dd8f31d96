// SO3LR E + F + virial on one gfx950 GPU: kernels and per-step orchestration.
//
// Data layout in HBM (N owned atoms, P candidate short-range pairs):
//   node state per block b:  x[b] N x 128, ev[b] N x 24, qkv[b] N x 640
//                            (q | k | v | q_ev | k_ev, head-major inside each)
//   pair state (active pairs compacted to the front each step):
//     nodes (a, b), v = x_a - x_b, r, Y(v/r) (24), fc, ZBL (e, de/dr)
//     per block: s (4 equivariant invariants), f (128 inv | 128 ev filters),
//     alpha (2 directions x (4 inv + 4 ev) attention coefficients)
//   reverse: df (256), dfc, ds (4), dr, dY (24), g = dE/dv (3)
// The directed edge "b -> a" (receiver a) uses Y(v/r); "a -> b" uses
// (-1)^l Y(v/r).  Node sums are gathers over a CSR incidence list.
#include "evaluator.hpp"
#include "mfma_ops.hpp"
#include "radial_table.hpp"

#include <algorithm>
#include <array>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <stdexcept>
#include <type_traits>
#include <utility>

namespace so3lr_amd {

// Work space of so3lr_compute_device_noalloc: one static array per device,
// present from the module's load on that device until the process ends (256
// MiB of its HBM).  Host code never names it as an address: the constructor
// looks up this device's copy once with hipGetSymbolAddress and keeps the
// pointer (scratch_dev_), which is what kernels and copies receive.  Every
// no-allocation evaluation on a device shares that device's copy; the
// contents of the previous call stay behind, and calls that overlap on one
// device race.
constexpr std::size_t kScratchBytes = std::size_t(256) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

#define HIP_CHECK(expr)                                                                   \
  do {                                                                                    \
    hipError_t err_ = (expr);                                                             \
    if (err_ != hipSuccess)                                                               \
      throw DeviceError(std::string("HIP error in ") + #expr + ": " +             \
                               hipGetErrorString(err_));                                  \
  } while (0)

namespace {

// Address of `device`'s copy of the scratch array, looked up once per device
// (the caller has made `device` current) and kept for the process.
char *scratch_on_device(int device) {
  static std::mutex mu;
  static std::vector<char *> table;
  std::lock_guard<std::mutex> lock(mu);
  if (std::size_t(device) >= table.size()) table.resize(std::size_t(device) + 1, nullptr);
  if (!table[device]) {
    void *sp = nullptr;
    const hipError_t se = hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch));
    if (se != hipSuccess || sp == nullptr)
      throw DeviceError(std::string("HIP error in hipGetSymbolAddress(scratch): ") + hipGetErrorString(se));
    table[device] = static_cast<char *>(sp);
  }
  return table[device];
}

constexpr int kWave = 64;
constexpr int kCompactPerBlock = 1024;  // candidates per compaction block (256 threads x 4)

// DPP lane permute of a double within the 16-lane rows of a wavefront (two
// 32-bit moves).  CTRL: 0xB1 quad_perm(1,0,3,2), 0x4E quad_perm(2,3,0,1),
// 0x141 row_half_mirror, 0x140 row_mirror.
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
  const unsigned lo = unsigned(__builtin_amdgcn_update_dpp(0, int(unsigned(b)), CTRL, 0xF, 0xF, false));
  const unsigned hi = unsigned(__builtin_amdgcn_update_dpp(0, int(unsigned(b >> 32)), CTRL, 0xF, 0xF, false));
  return __builtin_bit_cast(double, (unsigned long long)lo | ((unsigned long long)hi << 32));
}
// value of v in lane l (uniform)
__device__ __forceinline__ double lane_read(double v, int l) {
  const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
  const unsigned lo = unsigned(__builtin_amdgcn_readlane(int(unsigned(b)), l));
  const unsigned hi = unsigned(__builtin_amdgcn_readlane(int(unsigned(b >> 32)), l));
  return __builtin_bit_cast(double, (unsigned long long)lo | ((unsigned long long)hi << 32));
}
// Sum over the 16-lane row this lane belongs to (quads, then half-rows, then
// rows, each step adding the mirrored partner): every lane of the row ends
// with the same bits.  All 64 lanes must be active.
__device__ __forceinline__ double group_sum(double v) {
  v += dpp_f64<0xB1>(v);
  v += dpp_f64<0x4E>(v);
  v += dpp_f64<0x141>(v);
  v += dpp_f64<0x140>(v);
  return v;
}
// Sum over the wavefront: row sums combined in row order (uniform result).
__device__ __forceinline__ double wave_sum(double v) {
  v = group_sum(v);
  return ((lane_read(v, 0) + lane_read(v, 16)) + lane_read(v, 32)) + lane_read(v, 48);
}
__device__ __forceinline__ double pick4(int s, double a, double b, double c, double d) {
  return s == 0 ? a : (s == 1 ? b : (s == 2 ? c : d));
}

__global__ void k_fill(double *p, std::size_t n, double v) {
  const std::size_t i = std::size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// Residual scalars (kokkos_local_energy_reverse.cpp:124-170): a block's input
// x <- a x + c x0 (x0 the embedding), and the adjoint of the previous block's
// output g <- a g.
__global__ void k_axpby(std::size_t n, double a, double *x, double c, const double *x0) {
  const std::size_t i = std::size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) x[i] = a * x[i] + c * x0[i];
}
__global__ void k_scale(std::size_t n, double a, double *g) {
  const std::size_t i = std::size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) g[i] *= a;
}

// QK normalisation (kokkos_integrated_block0.cpp:288-328): each head row
// (32 channels) of q, k, q_ev, k_ev of a node divided by its RMS, eps 1e-6;
// v untouched.  One thread per (node, row); row r = 4 w + h, w = q, k, q_ev,
// k_ev at 0, 128, 384, 512 of the 640-wide node row (a head's 32 channels stay
// together in the tile-transposed order).  1/rms kept for the reverse.
__device__ __forceinline__ int qk_row(int r) { return (r < 8 ? 128 * (r >> 2) : 128 * ((r >> 2) + 1)) + 32 * (r & 3); }
__global__ __launch_bounds__(256) void k_qk_norm(int N, double *qkv, double *qkis) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= N * 16) return;
  double *row = qkv + std::size_t(t >> 4) * 640 + qk_row(t & 15);
  double ms = 0.0;
#pragma unroll 8
  for (int c = 0; c < 32; ++c) ms += row[c] * row[c];
  const double r = 1.0 / sqrt(ms / 32.0 + 1e-6);
#pragma unroll 8
  for (int c = 0; c < 32; ++c) row[c] *= r;
  qkis[t] = r;
}
// its reverse on the row adjoints: g <- r (g - y mean(g y)), y the normalised row
__global__ __launch_bounds__(256) void k_qk_norm_bwd(int N, const double *qkv, const double *qkis, double *gqkv) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= N * 16) return;
  const std::size_t o = std::size_t(t >> 4) * 640 + qk_row(t & 15);
  const double *y = qkv + o;
  double *g = gqkv + o;
  double m = 0.0;
#pragma unroll 8
  for (int c = 0; c < 32; ++c) m += g[c] * y[c];
  m /= 32.0;
  const double r = qkis[t];
#pragma unroll 8
  for (int c = 0; c < 32; ++c) g[c] = r * (g[c] - y[c] * m);
}

// ---------------------------------------------------------------- compaction
// Active short-range pairs are those with 0 < r^2 < rc^2, kept in candidate
// order (pair_so3lr_native_mpi.cpp:258-291,306-373 count + stable scan).
// Pair vector v = x_a - x_b of candidate c: LAMMPS rows (ghost rows carry
// the image displacement) or owned positions plus an image code (device
// reneighbor path; code c stands for ((c/9)-1, (c/3)%3-1, c%3-1) box lengths
// added to b).
struct RowsPos {
  const double *x;
  const int *rows;
  __device__ __forceinline__ void vec(int c, double &dx, double &dy, double &dz) const {
    const int ra = rows[2 * c], rb = rows[2 * c + 1];
    dx = x[3 * ra] - x[3 * rb];
    dy = x[3 * ra + 1] - x[3 * rb + 1];
    dz = x[3 * ra + 2] - x[3 * rb + 2];
  }
};
struct ShiftPos {
  const double *x;
  const int *nodes, *codes;
  double lx, ly, lz;
  __device__ __forceinline__ void vec(int c, double &dx, double &dy, double &dz) const {
    const int a = nodes[2 * c], b = nodes[2 * c + 1], code = codes[c];
    dx = x[3 * a] - x[3 * b] - (code / 9 - 1) * lx;
    dy = x[3 * a + 1] - x[3 * b + 1] - ((code / 3) % 3 - 1) * ly;
    dz = x[3 * a + 2] - x[3 * b + 2] - (code % 3 - 1) * lz;
  }
};

template <class Pos>
__device__ __forceinline__ bool sr_active(const Pos &pos, int c, double rc2, double &dx, double &dy, double &dz) {
  pos.vec(c, dx, dy, dz);
  const double r2 = dx * dx + dy * dy + dz * dz;
  return r2 > 0.0 && r2 < rc2;
}

template <class Pos>
__global__ __launch_bounds__(256) void k_sr_count(int P, Pos pos, double rc2, int *blk_count) {
  __shared__ int part[256];
  const int base = blockIdx.x * kCompactPerBlock + threadIdx.x * 4;
  int cnt = 0;
  for (int j = 0; j < 4; ++j) {
    const int c = base + j;
    double dx, dy, dz;
    if (c < P && sr_active(pos, c, rc2, dx, dy, dz)) ++cnt;
  }
  part[threadIdx.x] = cnt;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (int(threadIdx.x) < s) part[threadIdx.x] += part[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) blk_count[blockIdx.x] = part[0];
}

// exclusive scan of per-block counts in place; the total to *n_total and,
// clamped to the capacity of the active-pair buffers, to *n_active
__global__ __launch_bounds__(1024) void k_scan_counts(int nblk, int *cnt, int *n_active, int cap, int *n_total) {
  __shared__ int buf[1024];
  __shared__ int carry;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  for (int start = 0; start < nblk; start += 1024) {
    const int i = start + threadIdx.x;
    const int v = i < nblk ? cnt[i] : 0;
    buf[threadIdx.x] = v;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
      const int t = int(threadIdx.x) >= off ? buf[threadIdx.x - off] : 0;
      __syncthreads();
      buf[threadIdx.x] += t;
      __syncthreads();
    }
    if (i < nblk) cnt[i] = carry + buf[threadIdx.x] - v;
    __syncthreads();
    if (threadIdx.x == 1023) carry += buf[1023];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    *n_active = carry < cap ? carry : cap;
    if (n_total) *n_total = carry;
  }
}

template <class Pos>
__global__ __launch_bounds__(256) void k_sr_compact(
    int P, Pos pos, const int *nodes, double rc2, const int *blk_off, int cap,
    const int *z, ZblParams zp, int *cand2act, int *pa, double *pv, double *pr, double *pY,
    double *pfc, double *pzbl) {
  __shared__ int part[256];
  const int base = blockIdx.x * kCompactPerBlock + threadIdx.x * 4;
  int flags = 0, cnt = 0;
  for (int j = 0; j < 4; ++j) {
    const int c = base + j;
    double dx, dy, dz;
    if (c < P && sr_active(pos, c, rc2, dx, dy, dz)) { flags |= 1 << j; ++cnt; }
  }
  part[threadIdx.x] = cnt;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {
    const int t = int(threadIdx.x) >= off ? part[threadIdx.x - off] : 0;
    __syncthreads();
    part[threadIdx.x] += t;
    __syncthreads();
  }
  int at = blk_off[blockIdx.x] + part[threadIdx.x] - cnt;
  const double rc = sqrt(rc2);
  for (int j = 0; j < 4; ++j) {
    const int c = base + j;
    if (c >= P) break;
    if (!(flags & (1 << j))) { cand2act[c] = -1; continue; }
    double dx, dy, dz;
    sr_active(pos, c, rc2, dx, dy, dz);
    const int p = at++;
    if (p >= cap) {  // beyond the active-pair buffers: the host grows them and evaluates again
      cand2act[c] = -1;
      continue;
    }
    cand2act[c] = p;
    const int na = nodes[2 * c], nb = nodes[2 * c + 1];
    pa[2 * p] = na;
    pa[2 * p + 1] = nb;
    pv[3 * p] = dx; pv[3 * p + 1] = dy; pv[3 * p + 2] = dz;
    const double r = sqrt(dx * dx + dy * dy + dz * dz);
    pr[p] = r;
    const double inv = r > 1e-14 ? 1.0 / r : 0.0;
    const double ux = dx * inv, uy = dy * inv, uz = dz * inv;
    for (int m = 0; m < kE; ++m) pY[kE * p + m] = sh_component(m, ux, uy, uz);
    const double t = r / rc, t3 = t * t * t;
    pfc[p] = r < rc ? 1.0 - 10.0 * t3 + 15.0 * t3 * t - 6.0 * t3 * t * t : 0.0;
    double e, g;
    zbl_directed(zp, double(z[na]), double(z[nb]), r, e, g);
    pzbl[2 * p] = e;
    pzbl[2 * p + 1] = g;
  }
}

// Workgroups go to the 8 XCDs round-robin (block b on XCD b % 8).  Remapped
// so that each XCD walks one contiguous range of logical blocks: with nodes
// in spatial order, the neighbour rows a range gathers stay in its XCD's L2.
// A bijection of [0, gridDim.x) whatever the grid size.
__device__ __forceinline__ int xcd_block() {
#ifdef SO3LR_NO_XCD_MAP
  return blockIdx.x;
#endif
  const int G = gridDim.x, b = blockIdx.x;
  const int per = G >> 3, rem = G & 7, xcd = b & 7, i = b >> 3;
  return xcd * per + (xcd < rem ? xcd : rem) + i;
}
// The same for a grid sized for an upper bound of the work: only the first A
// logical blocks have work (A <= gridDim.x, known on the device only), and
// they are spread evenly over the XCDs; -1 for a block with none.
__device__ __forceinline__ int xcd_block_active(int A) {
  const int b = blockIdx.x;
  const int per = A >> 3, rem = A & 7, xcd = b & 7, i = b >> 3;
  if (i >= per + (xcd < rem ? 1 : 0)) return -1;
  return xcd * per + (xcd < rem ? xcd : rem) + i;
}

// ---------------------------------------------------------------- filters
// Per active pair: Bernstein basis and PhysNet cutoff of r, the equivariant
// invariant s_l = sum_{m in l} (ev_a - ev_b)^2 cg, and both filters
//   f = W1 silu(W0 rbf + b0) + b1 + E1 silu(E0 s + e0) + e1
// (kokkos_integrated_block0.cpp:138-255).  One 128-thread block per pair.
struct FilterArgs {
  const double *fw0[2], *fb0[2], *fw1t[2], *fb1[2], *fe0[2], *feb0[2], *fe1t[2], *feb1[2];
  const double *att_cg;
  const double *rbf_b, *rbf_k, *rbf_kr;
  double gamma;
};

__device__ __forceinline__ void bernstein(double r, double gamma, const double *b, const double *k,
                                          const double *kr, int ch, double &val) {
  double xb = exp(-gamma * r);
  xb = xb < 1e-6 ? 1e-6 : (xb > 1.0 - 1e-6 ? 1.0 - 1e-6 : xb);
  val = exp(b[ch] + k[ch] * log(xb) + kr[ch] * log(1.0 - xb));
}

// Position of filter channel c (0..127) inside its 128-wide half of a pair's
// filter row (pf) and of its adjoint (df): a 4 x 4 transpose inside each
// 16-channel tile, pos(c) = 16 (c / 16) + 4 (c % 4) + (c / 4) % 4.  The four
// accumulator values an MFMA filter lane holds for one output tile (channels
// 16 mt + g + 4 r, r = 0..3) are then adjacent, one 32-byte vector per lane,
// and every head's 32 channels stay contiguous for the attention kernels.
__host__ __device__ __forceinline__ int fpos(int c) { return (c & ~15) | ((c & 3) << 2) | ((c >> 2) & 3); }

__global__ __launch_bounds__(128) void k_filter_fwd(const int *n_active, const int *pa, const double *pr,
                                                    const double *ev, FilterArgs A, double *ps,
                                                    double *pf) {
  const int p = blockIdx.x;
  if (p >= *n_active) return;
  __shared__ double rbf[kR], s[4], h[kF], h2[kFH];
  const int c = threadIdx.x;
  const double r = pr[p];
  if (c < kR) bernstein(r, A.gamma, A.rbf_b, A.rbf_k, A.rbf_kr, c, rbf[c]);
  if (c < 4) {
    const int a = pa[2 * p], b = pa[2 * p + 1];
    const int lo = c == 0 ? 0 : (c == 1 ? 3 : (c == 2 ? 8 : 15));
    const int hi = c == 0 ? 3 : (c == 1 ? 8 : (c == 2 ? 15 : 24));
    double acc = 0.0;
    for (int m = lo; m < hi; ++m) {
      const double d = ev[std::size_t(a) * kE + m] - ev[std::size_t(b) * kE + m];
      acc += d * d * A.att_cg[m];
    }
    s[c] = acc;
    ps[4 * std::size_t(p) + c] = acc;
  }
  __syncthreads();
  for (int which = 0; which < 2; ++which) {
    double acc = A.fb0[which][c];
    const double *w0 = A.fw0[which] + c * kR;
    for (int k = 0; k < kR; ++k) acc += w0[k] * rbf[k];
    h[c] = silu(acc);
    if (c < kFH) {
      const double *e0 = A.fe0[which] + c * 4;
      h2[c] = silu(A.feb0[which][c] + e0[0] * s[0] + e0[1] * s[1] + e0[2] * s[2] + e0[3] * s[3]);
    }
    __syncthreads();
    double f = A.fb1[which][c] + A.feb1[which][c];
    const double *w1t = A.fw1t[which];
    for (int k = 0; k < kF; ++k) f += w1t[k * kF + c] * h[k];
    const double *e1t = A.fe1t[which];
    for (int j = 0; j < kFH; ++j) f += e1t[j * kF + c] * h2[j];
    pf[256 * std::size_t(p) + which * kF + fpos(c)] = f;
    __syncthreads();
  }
}

// Reverse of the filters and of the radial basis / cutoff
// (kokkos_block2_attention_input_reverse.cpp:198-240,301-336).
__global__ __launch_bounds__(128) void k_filter_bwd(const int *n_active, const double *pr,
                                                    const double *pfc_unused, const double *ps,
                                                    const double *df, const double *dfc, FilterArgs A,
                                                    double rc, double *ds, double *dr) {
  const int p = blockIdx.x;
  if (p >= *n_active) return;
  __shared__ double rbf[kR], s[4], g[2 * kF], dh[kF], dh2[kFH], drbf[kR], dsv[4];
  const int c = threadIdx.x;
  const double r = pr[p];
  if (c < kR) { bernstein(r, A.gamma, A.rbf_b, A.rbf_k, A.rbf_kr, c, rbf[c]); drbf[c] = 0.0; }
  if (c < 4) { s[c] = ps[4 * std::size_t(p) + c]; dsv[c] = 0.0; }
  g[c] = df[256 * std::size_t(p) + fpos(c)];
  g[kF + c] = df[256 * std::size_t(p) + kF + fpos(c)];
  __syncthreads();
  for (int which = 0; which < 2; ++which) {
    const double *gf = g + which * kF;
    double pre = A.fb0[which][c];
    const double *w0 = A.fw0[which] + c * kR;
    for (int k = 0; k < kR; ++k) pre += w0[k] * rbf[k];
    double acc = 0.0;
    const double *w1 = A.fw1t[which];  // (in, out): column c of W1 is row c here
    for (int o = 0; o < kF; ++o) acc += w1[c * kF + o] * gf[o];
    dh[c] = acc * silu_prime(pre);
    if (c < kFH) {
      const double *e0 = A.fe0[which] + c * 4;
      const double pre2 = A.feb0[which][c] + e0[0] * s[0] + e0[1] * s[1] + e0[2] * s[2] + e0[3] * s[3];
      const double *e1t = A.fe1t[which];
      double a2 = 0.0;
      for (int o = 0; o < kF; ++o) a2 += e1t[c * kF + o] * gf[o];
      dh2[c] = a2 * silu_prime(pre2);
    }
    __syncthreads();
    if (c < kR) {
      double a = 0.0;
      for (int q = 0; q < kF; ++q) a += A.fw0[which][q * kR + c] * dh[q];
      drbf[c] += a;
    }
    if (c < 4) {
      double a = 0.0;
      for (int j = 0; j < kFH; ++j) a += A.fe0[which][j * 4 + c] * dh2[j];
      dsv[c] += a;
    }
    __syncthreads();
  }
  if (c == 0) {
    for (int l = 0; l < 4; ++l) ds[4 * std::size_t(p) + l] = dsv[l];
    double grad = 0.0;
    if (r < rc) {
      const double t = r / rc;
      grad += dfc[p] * (-30.0 * t * t * (1.0 - t) * (1.0 - t) / rc);
    }
    const double xb = exp(-A.gamma * r);
    if (xb > 1e-6 && xb < 1.0 - 1e-6)
      for (int k = 0; k < kR; ++k)
        grad += drbf[k] * rbf[k] * (-A.gamma * A.rbf_k[k] + A.gamma * A.rbf_kr[k] * xb / (1.0 - xb));
    dr[p] += grad;
  }
}


// ---------------------------------------------------------------- MFMA filters
struct FilterMfma {
  const double *w0p[2], *w1p[2], *e1p[2];              // forward operands
  const double *w1tp[2], *w0tp[2], *e1tp[2], *e0tp[2];  // reverse operands (transposes)
  const double *b0p[2], *eb0p[2], *ob1p[2];             // biases in accumulator order
  const double *ob1p0[2];                               // output bias with the ev = 0 spherical branch folded in
  const double *e0pk[2];                                // spherical layer 0: one v4d per lane {tile 0, tile 1, 0, 0}
  const double *att_cg;
  const double *rbf_b, *rbf_k, *rbf_kr;
  const double *rbf_e;     // Bernstein factors: e^{b_c} (c < 4), e^{b_c - b_{c-4}} (c >= 4)
  const double *exp2_256;  // 2^(j/256), j < 256
  double gamma;
};

// The table into LDS: call at kernel start, before any wavefront returns.
#define SO3LR_EXP2_TABLE(A)                                               \
  __shared__ double exp2_lds[256];                                        \
  if (threadIdx.x < 256) exp2_lds[threadIdx.x] = (A).exp2_256[threadIdx.x]; \
  __syncthreads();

// Stream entries in flight per wavefront (measured at config 3: 4 for the
// forward filter of blocks after 0, which 3, 5 or 6 slow by 3-18%; 6 for
// block 0's forward and for the reverse filters, 1-2% faster than 4 there).
#ifndef SO3LR_FILTER_PF
#define SO3LR_FILTER_PF 4
#endif
constexpr int kFilterPF = SO3LR_FILTER_PF;
#ifndef SO3LR_FILTER_FWD0_PF
#define SO3LR_FILTER_FWD0_PF 6
#endif
#ifndef SO3LR_FILTER_BWD_PF
#define SO3LR_FILTER_BWD_PF 6
#endif
// Two wavefronts per SIMD (<= 256 registers per lane): measured faster than
// one wavefront with a deeper prefetch, since the second wave's MFMAs cover
// the first one's VALU phases (RBF, SiLU).
#ifndef SO3LR_FILTER_WAVES
#define SO3LR_FILTER_WAVES 2
#endif
#define FILTER_OCCUPANCY __attribute__((amdgpu_waves_per_eu(SO3LR_FILTER_WAVES, SO3LR_FILTER_WAVES)))
#ifndef SO3LR_FILTER_FWD_WAVES
#define SO3LR_FILTER_FWD_WAVES SO3LR_FILTER_WAVES
#endif
#define FILTER_FWD_OCCUPANCY __attribute__((amdgpu_waves_per_eu(SO3LR_FILTER_FWD_WAVES, SO3LR_FILTER_FWD_WAVES)))

__device__ __forceinline__ v4d tile_load(const double *P, int t, int lane) { return frag_load(P, t, lane); }

// first equivariant channel of degree slot h (l = h + 1): 0, 3, 8, 15
__device__ __forceinline__ int ev_offset(int h) { return h == 0 ? 0 : (h == 1 ? 3 : (h == 2 ? 8 : 15)); }

// Bernstein basis b_c(x) = e^{b_c} x^c (1 - x)^(31 - c), x = e^{-gamma r}
// clamped to [1e-6, 1 - 1e-6] (kokkos_integrated_block0.cpp:117-160; the
// exponents k_c = c, 31 - c are checked at load), at the lane's channels
// c = g + 4 t, t < 8 (register t & 3 of tile t >> 2).  The first from powers
// of x and y = 1 - x, each next one by the ratio b_{c+4} / b_c =
// e^{b_{c+4} - b_c} (x / y)^4: no logarithm and one exponential (x itself)
// per lane instead of eight.  rbf_e holds e^{b_c} for c < 4 and
// e^{b_c - b_{c-4}} for c >= 4.  rho = x / y.
__device__ __forceinline__ void bernstein8(double x, int g, const double *__restrict__ rbf_e, v4d *rb,
                                           double &rho) {
  const double y = 1.0 - x;
  const double y2 = y * y, y4 = y2 * y2, y8 = y4 * y4;
  const double y28 = (y8 * y8) * (y8 * y4);
  const double x2 = x * x;
  // x^g y^(3 - g)
  const double lead = g == 0 ? y2 * y : (g == 1 ? x * y2 : (g == 2 ? x2 * y : x2 * x));
  double v = rbf_e[g] * lead * y28;
  rho = x * rcp_act(y);
  const double r2 = rho * rho, r4 = r2 * r2;
  rb[0][0] = v;
#pragma unroll
  for (int t = 1; t < 8; ++t) {
    v = v * r4 * rbf_e[g + 4 * t];
    rb[t >> 2][t & 3] = v;
  }
}

// The basis and, in db, d b_c / dr at those channels (zero where the clamp of
// x is active): b_c (-gamma c + gamma (31 - c) x / (1 - x)).
__device__ __forceinline__ void rbf8_with_grad(double r, int g, const FilterMfma &A, const double *tab, v4d *rb,
                                               v4d *db) {
  double x = exp_tab(-A.gamma * r, tab);
  bool clamped = false;
  if (x < 1e-6) { x = 1e-6; clamped = true; }
  if (x > 1.0 - 1e-6) { x = 1.0 - 1e-6; clamped = true; }
  double rho;
  bernstein8(x, g, A.rbf_e, rb, rho);
  const double q = clamped ? 0.0 : A.gamma * rho, gk = clamped ? 0.0 : -A.gamma;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const double k = double(g + 4 * t);
    db[t >> 2][t & 3] = rb[t >> 2][t & 3] * (gk * k + (31.0 - k) * q);
  }
}

// The basis alone (forward filter).
__device__ __forceinline__ void rbf8(double r, int g, const FilterMfma &A, const double *tab, v4d *rb) {
  double x = exp_tab(-A.gamma * r, tab);
  if (x < 1e-6) x = 1e-6;
  if (x > 1.0 - 1e-6) x = 1.0 - 1e-6;
  double rho;
  bernstein8(x, g, A.rbf_e, rb, rho);
}

// Both filters of one block for 16 pairs per wavefront, 4 wavefronts per block.
// Per filter the stream holds 96 weight fragments: W0 (s < 16: tile s % 8,
// K chunk s / 8), W1 (16 <= s < 80) and E1 (80 <= s < 96), tile-minor.
// The RT reverse (blocks after 0 on their radial tables, in interval order):
// operand-stream depth and wavefronts per SIMD.
#ifndef SO3LR_RT_BWD_PF
#define SO3LR_RT_BWD_PF 6
#endif
#ifndef SO3LR_RT_BWD_WAVES
#define SO3LR_RT_BWD_WAVES 2
#endif
template <bool EV0>
__global__ __launch_bounds__(256) FILTER_FWD_OCCUPANCY void k_filter_fwd_mfma(const int *n_active, const int *pa,
                                                                     const double *pr, const double *ev,
                                                                     const double *__restrict__ qkv, double inv_avg,
                                                                     FilterMfma A, double *ps, double *pf,
                                                                     double *palpha) {
  SO3LR_EXP2_TABLE(A)
  const int nact = *n_active;
  const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
  // consecutive pairs on one XCD: the endpoint rows they read are
  // spatial neighbours, so they share that XCD's L2
  const int blk = xcd_block_active((nact + 63) / 64);
  if (blk < 0) return;
  const int wave = blk * 4 + (threadIdx.x >> 6);
  if (wave * 16 >= nact) return;  // whole wavefront idle
  const int p = wave * 16 + j;
  const bool valid = p < nact;
  const int pp = valid ? p : nact - 1;
  const int a = pa[2 * pp], b = pa[2 * pp + 1];
  // q k v q_ev k_ev rows of both endpoints (tile-transposed channel order):
  // the lane's four channels of an output tile are one 32-byte vector
  const double *qa = qkv + std::size_t(a) * 640 + 4 * g, *qb = qkv + std::size_t(b) * 640 + 4 * g;

  // Per filter the stream holds: the layer-0 bias tiles (8), the spherical
  // layer-0 bias tiles (2) and operand (1), W0 (16: tile s % 8, K chunk
  // s / 8), then per output tile mt its bias, the endpoint rows q_a, k_b,
  // q_b, k_a of its channels, the 8 W1 chunks and the 2 E1 chunks (15
  // each): 147 entries.  The rows come first so that their loads (from L2,
  // or HBM where a partner's row has left it) are issued a whole tile of
  // MFMAs before the logits need them; q_a k_b and q_b k_a are multiplied as
  // they arrive.  The output is built one tile at a time and stored as
  // soon as it is complete, so only one output accumulator is live; the
  // attention logits of both directions are reduced from it on the spot.
  // EV0 (block 0, ev = 0): the spherical branch sees s = 0 for every pair,
  // so it is the constant E1 silu(e0) + e1, folded into the output bias
  // (ob1p0); its entries are left out (13 per tile, 128 in all).
  constexpr int TS = EV0 ? 24 : 27, PT = EV0 ? 13 : 15;
  constexpr int UW = 5, UE = 13;  // first W1 and first E1 entry of a tile
  constexpr int NF = TS + 8 * PT;
  auto load = [&](auto si) -> v4d {
    constexpr int S = decltype(si)::value, which = S / NF, s = S % NF;
    if constexpr (s < 8) return tile_load(A.b0p[which], s, lane);
    else if constexpr (!EV0 && s < 10) return tile_load(A.eb0p[which], s - 8, lane);
    else if constexpr (!EV0 && s == 10) return tile_load(A.e0pk[which], 0, lane);
    else if constexpr (s < TS) return wload(A.w0p[which], 2, (s - TS + 16) % 8, (s - TS + 16) / 8, lane);
    else {
      constexpr int mt = (s - TS) / PT, u = (s - TS) % PT;
      constexpr int qoff = which ? 384 : 0, koff = which ? 512 : 128;  // q, k (invariant) or q_ev, k_ev
      if constexpr (u == 0) return tile_load(EV0 ? A.ob1p0[which] : A.ob1p[which], mt, lane);
      else if constexpr (u == 1) return *reinterpret_cast<const v4d *>(qa + qoff + 16 * mt);
      else if constexpr (u == 2) return *reinterpret_cast<const v4d *>(qb + koff + 16 * mt);
      else if constexpr (u == 3) return *reinterpret_cast<const v4d *>(qb + qoff + 16 * mt);
      else if constexpr (u == 4) return *reinterpret_cast<const v4d *>(qa + koff + 16 * mt);
      else if constexpr (u < UE) return wload(A.w1p[which], 8, mt, u - UW, lane);
      else return wload(A.e1p[which], 2, mt, u - UE, lane);
    }
  };
  Stream<2 * NF, EV0 ? SO3LR_FILTER_FWD0_PF : kFilterPF, decltype(load)> st(load);
  st.prime();

  v4d rb[2];
  rbf8(pr[pp], g, A, exp2_lds, rb);
  // equivariant invariant of degree slot g (K = 4 operand of the spherical filter)
  double sg = 0.0;
  if constexpr (!EV0) {
    // slot g's 2 g + 3 channels, as nine loads per endpoint with the channels
    // past the slot weighted by zero, so that all of them are in flight at
    // once (the endpoints' rows are far apart in interval order)
    const int lo = g == 0 ? 0 : (g == 1 ? 3 : (g == 2 ? 8 : 15)), n = 2 * g + 3;
    const double *ea = ev + std::size_t(a) * kE, *eb = ev + std::size_t(b) * kE;
    double va[9], vb[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) {
      const int m = min(lo + k, kE - 1);
      va[k] = ea[m];
      vb[k] = eb[m];
    }
#pragma unroll
    for (int k = 0; k < 9; ++k) {
      const double d = va[k] - vb[k];
      sg += k < n ? d * d * A.att_cg[lo + k] : 0.0;
    }
    if (valid) ps[4 * std::size_t(p) + g] = sg;
  }
  // tile mt of filter `which`: its four values per lane are adjacent (fpos)
  v4d *const rowv = EV0 ? nullptr : reinterpret_cast<v4d *>(pf + 256 * std::size_t(p) + 4 * g);
  v4d h[8], h2[2], e0, o, qv, qk0, qk1;
  double t0 = 0.0, t1 = 0.0;  // per-head partial logits: a <- b (side 0), b <- a (side 1)

  st.run([&](auto si, const v4d &w) {
    constexpr int S = decltype(si)::value, which = S / NF, s = S % NF;
    if constexpr (s < 8) {
      h[s] = w;
    } else if constexpr (!EV0 && s < 10) {
      h2[s - 8] = w;
    } else if constexpr (!EV0 && s == 10) {
      e0 = w;
    } else if constexpr (s < TS) {
      constexpr int i = s - TS + 16;  // W0 entry 0..15
      h[i % 8] = mfma4(w, rb[i / 8], h[i % 8]);
      // each hidden tile's SiLU is taken one step before its first use,
      // behind the MFMAs just issued (tile 0 here, tile t at W1 step t)
      if constexpr (i == 15) {
#pragma unroll
        for (int r = 0; r < 4; ++r) h[0][r] = silu_tab(h[0][r], exp2_lds);
      }
    } else {
      constexpr int mt = (s - TS) / PT, u = (s - TS) % PT;
      if constexpr (u == 0) {
        o = w;
      } else if constexpr (u == 1 || u == 3) {
        qv = w;
      } else if constexpr (u == 2) {
        qk0 = qv * w;  // q_a k_b: edge b -> a
      } else if constexpr (u == 4) {
        qk1 = qv * w;  // q_b k_a: edge a -> b
      } else {
        if constexpr (u < UE) {
          constexpr int i = u - UW;  // W1 chunk
          o = mfma4(w, h[i], o);
          if constexpr (mt == 0 && i < 7) {
#pragma unroll
            for (int r = 0; r < 4; ++r) h[i + 1][r] = silu_tab(h[i + 1][r], exp2_lds);
          }
          if constexpr (!EV0 && mt == 0 && i == 7) {
#pragma unroll
            for (int t = 0; t < 2; ++t) {
              h2[t] = mfma(e0[t], sg, h2[t]);
#pragma unroll
              for (int r = 0; r < 4; ++r) h2[t][r] = silu_tab_wide(h2[t][r], exp2_lds);
            }
          }
          // (block 0, EV0: the rows are not stored; its reverse has no
          // node-major attention kernel to read them, and the messages use alpha)
        } else {
          o = mfma4(w, h2[u - UE], o);
        }
        if constexpr (u == PT - 1) {
          // the output tile is complete
          if constexpr (!EV0) {
            if (valid) __builtin_nontemporal_store(o, rowv + which * 32 + 4 * mt);
          }
          // <q_recv, k_send (.) f> over the lane's four channels of this tile
          t0 += ((qk0[0] * o[0] + qk0[1] * o[1]) + qk0[2] * o[2]) + qk0[3] * o[3];
          t1 += ((qk1[0] * o[0] + qk1[1] * o[1]) + qk1[2] * o[2]) + qk1[3] * o[3];
          if constexpr (mt & 1) {
            // head mt / 2 complete: sum its 32 channels over the four lane
            // groups; the alpha of edge b -> a belongs to side 0 (a receives)
            t0 += __shfl_xor(t0, 16, kWave);
            t0 += __shfl_xor(t0, 32, kWave);
            t1 += __shfl_xor(t1, 16, kWave);
            t1 += __shfl_xor(t1, 32, kWave);
            constexpr int hd = mt / 2;
            if (valid && g == hd) {
              double *al = palpha + 16 * std::size_t(p) + 4 * which + hd;
              al[0] = t0 * inv_avg;
              al[8] = t1 * inv_avg;
            }
            t0 = 0.0;
            t1 = 0.0;
          }
        }
      }
    }
  });
}

// The forward filters of the blocks after 0 on their radial tables, in
// bucket order (16 slots of one bucket, spatial block and interval, per
// wavefront; -1 in the padding).  Per filter the stream holds the spherical
// layer-0 biases and operand (3), then per output tile the interval's
// coefficient tile (128 channels x 32 powers: two K chunks, against the
// pairs' powers of t in place of the W0 and W1 chains), the endpoint rows
// q_a, k_b, q_b, k_a of its channels (from L2: a spatial block's buckets
// run together on one XCD) and the 2 E1 chunks.  The rows go to pf and the
// logits of both directions to palpha as in k_filter_fwd_mfma.  Measured
// as two passes (the rows in bucket order, the logits in pair order) it
// took 0.79 against 0.70 ms.
#ifndef SO3LR_RT_FWD_PF
#define SO3LR_RT_FWD_PF 6
#endif
__global__ __launch_bounds__(256) FILTER_FWD_OCCUPANCY void k_radial_fwd_rows(
    const int *n_slots, const int *order, const int *pa, const double *pr, const double *__restrict__ ev,
    const double *__restrict__ qkv, const double *__restrict__ rtab, RadialDomain rd, double inv_avg, FilterMfma A,
    double *ps, double *pf, double *palpha) {
  SO3LR_EXP2_TABLE(A)
  const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
  const int blk = xcd_block_active((*n_slots + 63) / 64);
  const int wave = blk < 0 ? -1 : blk * 4 + (threadIdx.x >> 6);
  int p, ri;
  bool inside;
  v4d tp[2];
  if (!rint_slots(n_slots, order, pr, rd, wave, j, g, p, ri, inside, tp)) return;
  const bool valid = p >= 0;
  const int pp = valid ? p : order[wave * 16];
  const int a = pa[2 * pp], b = pa[2 * pp + 1];
  const double *qa = qkv + std::size_t(a) * 640 + 4 * g, *qb = qkv + std::size_t(b) * 640 + 4 * g;
  const double *coef = rtab + std::size_t(ri) * 2 * 16 * 256;
  constexpr int TS = 3, PT = 8, NF = TS + 8 * PT;
  auto load = [&](auto si) -> v4d {
    constexpr int S = decltype(si)::value, which = S / NF, s = S % NF;
    if constexpr (s < 2) return tile_load(A.eb0p[which], s, lane);
    else if constexpr (s == 2) return tile_load(A.e0pk[which], 0, lane);
    else {
      constexpr int mt = (s - TS) / PT, u = (s - TS) % PT;
      constexpr int qoff = which ? 384 : 0, koff = which ? 512 : 128;
      if constexpr (u < 2) return wload(coef + which * 16 * 256, 2, mt, u, lane);
      else if constexpr (u == 2) return *reinterpret_cast<const v4d *>(qa + qoff + 16 * mt);
      else if constexpr (u == 3) return *reinterpret_cast<const v4d *>(qb + koff + 16 * mt);
      else if constexpr (u == 4) return *reinterpret_cast<const v4d *>(qb + qoff + 16 * mt);
      else if constexpr (u == 5) return *reinterpret_cast<const v4d *>(qa + koff + 16 * mt);
      else return wload(A.e1p[which], 2, mt, u - 6, lane);
    }
  };
  Stream<2 * NF, SO3LR_RT_FWD_PF, decltype(load)> st(load);
  st.prime();
  // equivariant invariant of degree slot g, all loads in flight at once
  double sg = 0.0;
  {
    const int lo = g == 0 ? 0 : (g == 1 ? 3 : (g == 2 ? 8 : 15)), n = 2 * g + 3;
    const double *ea = ev + std::size_t(a) * kE, *eb = ev + std::size_t(b) * kE;
    double va[9], vb[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) {
      const int m = min(lo + k, kE - 1);
      va[k] = ea[m];
      vb[k] = eb[m];
    }
#pragma unroll
    for (int k = 0; k < 9; ++k) {
      const double d = va[k] - vb[k];
      sg += k < n ? d * d * A.att_cg[lo + k] : 0.0;
    }
    if (valid) ps[4 * std::size_t(p) + g] = sg;
  }
  v4d *const rowv = reinterpret_cast<v4d *>(pf + 256 * std::size_t(pp) + 4 * g);
  const v4d zero = v4d{0.0, 0.0, 0.0, 0.0};
  v4d h2[2], o, qv, qk0, qk1;
  double t0 = 0.0, t1 = 0.0;
  st.run([&](auto si, const v4d &w) {
    constexpr int S = decltype(si)::value, which = S / NF, s = S % NF;
    if constexpr (s < 2) {
      h2[s] = w;
    } else if constexpr (s == 2) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        h2[t] = mfma(w[t], sg, h2[t]);
#pragma unroll
        for (int r = 0; r < 4; ++r) h2[t][r] = silu_tab_wide(h2[t][r], exp2_lds);
      }
    } else {
      constexpr int mt = (s - TS) / PT, u = (s - TS) % PT;
      if constexpr (u == 0) {
        o = mfma4(w, tp[0], zero);
      } else if constexpr (u == 1) {
        o = mfma4(w, tp[1], o);
      } else if constexpr (u == 2 || u == 4) {
        qv = w;
      } else if constexpr (u == 3) {
        qk0 = qv * w;  // q_a k_b: edge b -> a
      } else if constexpr (u == 5) {
        qk1 = qv * w;  // q_b k_a: edge a -> b
      } else {
        o = mfma4(w, h2[u - 6], o);
        if constexpr (u == PT - 1) {
          if (valid) __builtin_nontemporal_store(o, rowv + which * 32 + 4 * mt);
          t0 += ((qk0[0] * o[0] + qk0[1] * o[1]) + qk0[2] * o[2]) + qk0[3] * o[3];
          t1 += ((qk1[0] * o[0] + qk1[1] * o[1]) + qk1[2] * o[2]) + qk1[3] * o[3];
          if constexpr (mt & 1) {
            t0 += __shfl_xor(t0, 16, kWave);
            t0 += __shfl_xor(t0, 32, kWave);
            t1 += __shfl_xor(t1, 16, kWave);
            t1 += __shfl_xor(t1, 32, kWave);
            constexpr int hd = mt / 2;
            if (valid && g == hd) {
              double *al = palpha + 16 * std::size_t(p) + 4 * which + hd;
              al[0] = t0 * inv_avg;
              al[8] = t1 * inv_avg;
            }
            t0 = 0.0;
            t1 = 0.0;
          }
        }
      }
    }
  });
}

// Operand schedule of the reverse filter's first section (per filter).
// Entry kinds: P, a term of the invariant head scalars (q = 0..3: gainv_a,
// v_b, gainv_b, v_a of chunk T, head h; `last` completes the head); R, a row
// chunk of the df of chunk T (u = 0..3: q_a, k_b, q_b, k_a); M, the MFMA
// entry `tile` of chunk T (W1^T tiles 0..7, then E1^T tiles 8..9); S, the
// head-h scalar record written by the node-major attention reverse.  The
// loads that carry no MFMA work (P, S and R) ride between the M entries of
// the previous chunk, so every one of them is covered by MFMA time: chunk
// T's rows arrive during chunk T - 1, and head h + 1's scalars during head
// h's chunks (scalar riders before row riders, so a head's scalars are
// complete before its first df is formed).
// SRC: 0 = P entries (block 0, invariant filter), 1 = S entries (blocks
// after 0, whose node-major reverse wrote the scalars), 2 = neither (block 0,
// equivariant filter: the scalars are lane shuffles).
struct BwdEntry {
  int kind, q, T, h, last;
};
constexpr int kBwdP = 0, kBwdR = 1, kBwdM = 2, kBwdS = 3;
template <int NM, int SRC>
constexpr int bwd_section_len() {
  return (SRC == 0 ? 8 + 24 : SRC == 1 ? 4 : 0) + 4 + 8 * NM + 28;
}
template <int NM, int SRC>
constexpr std::array<BwdEntry, bwd_section_len<NM, SRC>()> bwd_schedule() {
  std::array<BwdEntry, bwd_section_len<NM, SRC>()> out{};
  int n = 0;
  auto put = [&](int kind, int q, int T, int h, int last) { out[n++] = BwdEntry{kind, q, T, h, last}; };
  if (SRC == 0)  // lead-in: head 0's scalars
    for (int T = 0; T < 2; ++T)
      for (int q = 0; q < 4; ++q) put(kBwdP, q, T, 0, T == 1 && q == 3);
  if (SRC == 1) put(kBwdS, 0, 0, 0, 1);
  for (int u = 0; u < 4; ++u) put(kBwdR, u, 0, 0, 0);  // lead-in: chunk 0's rows
  for (int T = 0; T < 8; ++T) {
    BwdEntry riders[9] = {};
    int nr = 0;
    const int h = T / 2;
    if (SRC == 0 && h + 1 < 4)
      for (int q = 0; q < 4; ++q)
        riders[nr++] = BwdEntry{kBwdP, q, 2 * (h + 1) + (T & 1), h + 1, (T & 1) == 1 && q == 3};
    if (SRC == 1 && T + 1 < 8 && ((T + 1) & 1) == 0) riders[nr++] = BwdEntry{kBwdS, 0, T + 1, (T + 1) / 2, 1};
    if (T + 1 < 8)
      for (int u = 0; u < 4; ++u) riders[nr++] = BwdEntry{kBwdR, u, T + 1, (T + 1) / 2, 0};
    // one rider after each M entry; riders beyond the M entries follow them
    for (int m = 0; m < (NM > nr ? NM : nr); ++m) {
      if (m < NM) put(kBwdM, m, T, h, 0);
      if (m < nr) out[n++] = riders[m];
    }
  }
  return out;
}
template <int NM, int SRC>
constexpr BwdEntry bwd_entry(int s) {
  return bwd_schedule<NM, SRC>()[s];
}
// Compile-time check of a schedule: every slot filled (one M entry per MFMA
// tile of each chunk), the four row entries of chunk T before its first M
// entry, each head's scalars complete before the first row entry that uses
// them.
template <int NM, int SRC>
constexpr bool bwd_schedule_ok() {
  const auto sc = bwd_schedule<NM, SRC>();
  int rows_seen[8] = {}, m_seen[8] = {}, head_done = SRC == 2 ? 3 : -1;
  for (const BwdEntry &e : sc) {
    if ((e.kind == kBwdP || e.kind == kBwdS) && e.last) head_done = e.h;
    if (e.kind == kBwdR) {
      if (e.q == 1 && e.h > head_done) return false;
      if (m_seen[e.T]) return false;
      ++rows_seen[e.T];
    }
    if (e.kind == kBwdM) {
      if (rows_seen[e.T] != 4) return false;
      ++m_seen[e.T];
    }
  }
  for (int T = 0; T < 8; ++T)
    if (m_seen[T] != NM || rows_seen[T] != 4) return false;
  return true;
}
static_assert(bwd_schedule_ok<10, 1>() && bwd_schedule_ok<8, 0>() && bwd_schedule_ok<8, 2>() &&
                  bwd_schedule_ok<4, 1>(),
              "reverse-filter operand schedule out of order");

// Reverse of the attention's pair terms, of both filters, of the Bernstein
// basis and of the cutoff, for 16 pairs per wavefront
// (kokkos_attention_scatter_reverse.cpp:280-500 for the pair adjoints;
// kokkos_block2_attention_input_reverse.cpp:198-240,301-336 for the rest).
//
// The adjoint of the filter outputs, df, is formed here in registers and
// never stored.  For pair {a, b} (a receives along b -> a, b along a -> b)
// and head h, with g the attention-residual adjoints (gainv, gaev) of the
// block and fc the cutoff:
//   ci_h = <g_a, v_b>_h,  co_h = <g_b, v_a>_h        (invariant channels of h)
//   ce_h = <gev_a, Y>_h,  coe_h = (-1)^(h+1) <gev_b, Y>_h   (degree h + 1)
//   df_inv[c] = fc/avg (ci_h q_a[c] k_b[c] + co_h q_b[c] k_a[c])
//   df_ev[c]  = fc/avg (ce_h qe_a[c] ke_b[c] + coe_h qe_b[c] ke_a[c])
//   dE/dfc    = sum_h alpha(a<-b)_h ci_h + alpha_ev(a<-b)_h ce_h
//                     + alpha(b<-a)_h co_h + alpha_ev(b<-a)_h coe_h
//   dE/dY[m] += fc (alpha_ev(a<-b) gev_a[m] + (-1)^l alpha_ev(b<-a) gev_b[m])
// For blocks after 0 the node-major reverse (k_attn_bwd_nodes) has formed
// the head sums, dE/dfc and dE/dY already, and this kernel reads the sums'
// record; block 0 has no node-major reverse (its inputs do not depend on the
// positions), so its instantiation (EV0) forms all three here (FIRST, when
// block 0 is also the first block of the reverse pass, writes dE/dY without
// reading it).  The node rows (q, k, v, q_ev, k_ev of both endpoints and
// their gainv) arrive through the operand stream in the tile-transposed
// channel order, so a lane's four channels of a tile are one 32-byte vector.
//
// Per filter the stream holds the first section (bwd_schedule: the head
// scalars, the df rows and d hidden = W^T df over W1^T and E1^T), then:
//   per tile mt (8): the layer-0 bias, then W0 chunks 0, 1 (pre-activation
//             recomputed tile by tile, then d hidden *= silu');
//   the spherical layer-0 biases and operand (the same, 4 -> 32);
//   W0^T (16): d rbf = W0^T d hidden;
//   E0^T (2):  d s = E0^T d hidden_s.
// EV0 (block 0, ev = 0): the spherical branch is a constant (folded into the
// output bias by the forward kernel) and s has no adjoint to give, so its
// entries are left out.
// RT (blocks after 0 on their radial tables): pairs in bucket order as in
// k_radial_fwd_rows; the first section keeps E1^T (2 entries per chunk) and takes
// the interval's slope tile against each chunk's df (third entry), whose
// sum over the powers of t is the radial branches' dE/dr; the layer-0
// recompute, W0^T and the Bernstein basis are left out.
template <bool EV0, bool FIRST, bool RT = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(RT ? SO3LR_RT_BWD_WAVES : SO3LR_FILTER_WAVES,
                                                                     RT ? SO3LR_RT_BWD_WAVES : SO3LR_FILTER_WAVES))) void
k_filter_bwd_mfma(
    const int *n_active, const int *pa, const double *pr, const double *ps, const double *pfc, const double *pY,
    const double *palpha, const double *__restrict__ qkv, const double *__restrict__ gainv,
    const double *__restrict__ gaev, const double *__restrict__ psc, const double *__restrict__ pdfc, double inv_avg,
    FilterMfma A, double rc, double *ds, double *dr, double *dY, const int *n_slots = nullptr,
    const int *order = nullptr, const double *__restrict__ rtab = nullptr, RadialDomain rd = {}) {
  static_assert(!(EV0 && RT), "block 0 has its own tables");
  SO3LR_EXP2_TABLE(A)
  const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
  int p, pp, ri = 0;
  bool valid, inside = false;
  v4d tp[2];
  if constexpr (RT) {
    // consecutive slots on one XCD: a spatial block's buckets share its L2
    const int blk = xcd_block_active((*n_slots + 63) / 64);
    const int wave = blk < 0 ? -1 : blk * 4 + (threadIdx.x >> 6);
    if (!rint_slots(n_slots, order, pr, rd, wave, j, g, p, ri, inside, tp)) return;
    valid = p >= 0;
    pp = valid ? p : order[wave * 16];
  } else {
    const int nact = *n_active;
    // consecutive pairs on one XCD: the node rows they gather are spatial
    // neighbours, so they share that XCD's L2
    const int blk = xcd_block_active((nact + 63) / 64);
    if (blk < 0) return;
    const int wave = blk * 4 + (threadIdx.x >> 6);
    if (wave * 16 >= nact) return;
    p = wave * 16 + j;
    valid = p < nact;
    pp = valid ? p : nact - 1;
  }
  const int a = pa[2 * pp], b = pa[2 * pp + 1];
  // node rows, tile-transposed: chunk T of this lane at +16 T
  const double *ra = qkv + std::size_t(a) * 640 + 4 * g, *rb = qkv + std::size_t(b) * 640 + 4 * g;
  const double *gaa = gainv + std::size_t(a) * kF + 4 * g, *gab = gainv + std::size_t(b) * kF + 4 * g;
  auto row = [](const double *r, int off) { return *reinterpret_cast<const v4d *>(r + off); };

  // head scalars: block 0 forms them here (SRC 0 and 2), later blocks read
  // the node-major reverse's record (SRC 1)
  constexpr int NM = RT ? 4 : (EV0 ? 8 : 10), SRC0 = EV0 ? 0 : 1, SRC1 = EV0 ? 2 : 1;
  constexpr int A_END0 = bwd_section_len<NM, SRC0>(), A_END1 = bwd_section_len<NM, SRC1>();
  const double *rec = psc + 16 * std::size_t(pp);
  constexpr int B_LEN = RT ? 0 : 24, C_LEN = EV0 ? 0 : 3, D_LEN = RT ? 0 : 16, E_LEN = EV0 ? 0 : 2;
  constexpr int TAIL = B_LEN + C_LEN + D_LEN + E_LEN;
  constexpr int NB0 = A_END0 + TAIL, NB1 = A_END1 + TAIL;
  auto load = [&](auto si) -> v4d {
    constexpr int S = decltype(si)::value, which = S < NB0 ? 0 : 1, s = which ? S - NB0 : S;
    constexpr int A_END = which ? A_END1 : A_END0;
    constexpr int qoff = which ? 384 : 0, koff = which ? 512 : 128;
    if constexpr (s < A_END) {
      constexpr BwdEntry e = bwd_entry<NM, which ? SRC1 : SRC0>(s);
      if constexpr (e.kind == kBwdS) {
        return *reinterpret_cast<const v4d *>(rec + 4 * e.h);
      } else if constexpr (e.kind == kBwdP) {
        if constexpr (e.q == 0) return row(gaa, 16 * e.T);
        else if constexpr (e.q == 1) return row(rb, 256 + 16 * e.T);
        else if constexpr (e.q == 2) return row(gab, 16 * e.T);
        else return row(ra, 256 + 16 * e.T);
      } else if constexpr (e.kind == kBwdR) {
        if constexpr (e.q == 0) return row(ra, qoff + 16 * e.T);
        else if constexpr (e.q == 1) return row(rb, koff + 16 * e.T);
        else if constexpr (e.q == 2) return row(rb, qoff + 16 * e.T);
        else return row(ra, koff + 16 * e.T);
      } else {
        if constexpr (RT && e.q >= 2) return wload(rtab + (std::size_t(ri) * 2 + which) * 16 * 256, 8, e.q - 2, e.T, lane);
        else if constexpr (RT) return wload(A.e1tp[which], 8, e.q, e.T, lane);
        else if constexpr (e.q < 8) return wload(A.w1tp[which], 8, e.q, e.T, lane);
        else return wload(A.e1tp[which], 8, e.q - 8, e.T, lane);
      }
    } else if constexpr (s < A_END + B_LEN) {
      constexpr int mt = (s - A_END) / 3, u = (s - A_END) % 3;
      if constexpr (u == 0) return tile_load(A.b0p[which], mt, lane);
      else return wload(A.w0p[which], 2, mt, u - 1, lane);
    } else if constexpr (s < A_END + B_LEN + C_LEN) {
      constexpr int c = s - A_END - B_LEN;
      if constexpr (c < 2) return tile_load(A.eb0p[which], c, lane);
      else return reinterpret_cast<const v4d *>(A.e0pk[which])[lane];
    } else if constexpr (s < A_END + B_LEN + C_LEN + D_LEN) {
      constexpr int d = s - A_END - B_LEN - C_LEN;
      return wload(A.w0tp[which], 8, d % 2, d / 2, lane);
    } else {
      return wload(A.e0tp[which], 2, 0, s - A_END - B_LEN - C_LEN - D_LEN, lane);
    }
  };
  Stream<NB0 + NB1, RT ? SO3LR_RT_BWD_PF : SO3LR_FILTER_BWD_PF, decltype(load)> st(load);
  st.prime();

  const double r = pr[pp];
  const double fcs = pfc[pp] * inv_avg;  // fc / avg
  const double *al = palpha + 16 * std::size_t(pp);
  // Equivariant pair terms: lane group g takes degree slot g (channels
  // off(g) .. off(g) + 2g + 2, contiguous in the natural ev order): its
  // <gev_a, Y>, <gev_b, Y> and its share of dE/dY.
  double ce_mine = 0.0, coe_mine = 0.0;
  if constexpr (EV0) {
    const int lo = ev_offset(g), n_m = 2 * g + 3;
    const double par = slot_parity(g);
    const double ain_e = al[4 + g], aout_e = al[12 + g];
    const double *gea = gaev + std::size_t(a) * kE, *geb = gaev + std::size_t(b) * kE;
    const double *y = pY + kE * std::size_t(pp);
    double *dy = dY + kE * std::size_t(pp);
    const double fc = pfc[pp];
    for (int k = 0; k < n_m; ++k) {
      const int m = lo + k;
      const double ea = gea[m], eb = geb[m], ym = y[m];
      ce_mine += ea * ym;
      coe_mine += eb * ym;
      if (valid) dy[m] = (FIRST ? 0.0 : dy[m]) + fc * (ain_e * ea + par * aout_e * eb);
    }
    coe_mine *= par;
  }
  // dE/dfc: the equivariant terms of this lane group's slot now, the
  // invariant ones head by head below (every lane ends with the whole sum)
  double dfc = 0.0;
  if constexpr (EV0) {
    dfc = al[4 + g] * ce_mine + al[12 + g] * coe_mine;
    dfc += __shfl_xor(dfc, 16, kWave);
    dfc += __shfl_xor(dfc, 32, kWave);
  }
  // The running sums (dfc, part, ds_acc) are needed only at the end; an empty
  // asm on each update keeps the compiler from sinking the updates to that
  // use, which would hold every head's terms in registers until then.
  auto pin = [](double &v) { asm volatile("" : "+v"(v)); };
  pin(dfc);

  const v4d zero = v4d{0, 0, 0, 0};
  const double sg = EV0 ? 0.0 : ps[4 * std::size_t(pp) + g];
  // the Bernstein basis is formed where the layer-0 recompute starts (once
  // per filter), not held through the df / W^T section
  v4d rb8[2], db8[2];
  v4d dh[8], dh2[2], bT, bTn, t2, hold, pre, prev, pre2[2];
  // d rbf and d s of one filter, folded into scalars at the end of their
  // sections (dE/dr is linear in d rbf), so neither is held through the next
  // filter's df section
  v4d drb[2], dsa, accdr[2];
  double part = 0.0, ds_acc = 0.0;
  double ci = 0.0, co = 0.0, s_in = 0.0, s_out = 0.0;

  st.run([&](auto si, const v4d &w) {
    constexpr int S = decltype(si)::value, which = S < NB0 ? 0 : 1, s = which ? S - NB0 : S;
    constexpr int A_END = which ? A_END1 : A_END0;
    constexpr int B_END = A_END + B_LEN, C_END = B_END + C_LEN, D_END = C_END + D_LEN;
    if constexpr (s == 0) {
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) dh[mt] = zero;
      dh2[0] = zero;
      dh2[1] = zero;
      if constexpr (RT && which == 0) {
        accdr[0] = zero;
        accdr[1] = zero;
      }
    }
    if constexpr (s < A_END) {
      constexpr BwdEntry e = bwd_entry<NM, which ? SRC1 : SRC0>(s);
      if constexpr (e.kind == kBwdS) {
        // fc/avg-scaled head scalars of this pair: {in, out, in_ev, out_ev}
        s_in = which ? w[2] : w[0];
        s_out = which ? w[3] : w[1];
      } else if constexpr (e.kind == kBwdP) {
        // <gainv_a, v_b> and <gainv_b, v_a> over the lane's channels of head e.h
        if constexpr (e.q == 0 || e.q == 2) {
          hold = w;
        } else {
          const double d = ((hold[0] * w[0] + hold[1] * w[1]) + hold[2] * w[2]) + hold[3] * w[3];
          if constexpr (e.q == 1) ci += d;
          else co += d;
        }
        if constexpr (e.last) {
          // the head is complete: sum over the four lane groups
          ci += __shfl_xor(ci, 16, kWave);
          ci += __shfl_xor(ci, 32, kWave);
          co += __shfl_xor(co, 16, kWave);
          co += __shfl_xor(co, 32, kWave);
          dfc += al[e.h] * ci + al[8 + e.h] * co;
          pin(dfc);
          s_in = fcs * ci;
          s_out = fcs * co;
          ci = 0.0;
          co = 0.0;
        }
      } else if constexpr (e.kind == kBwdR) {
        // the df of chunk e.T, built while the previous chunk's MFMAs run
        if constexpr (EV0 && which == 1 && e.q == 0 && (e.T & 1) == 0) {
          // the slot-h sums live in lane group h
          s_in = fcs * __shfl(ce_mine, j + 16 * e.h, kWave);
          s_out = fcs * __shfl(coe_mine, j + 16 * e.h, kWave);
        }
        if constexpr (e.q == 0) {
          bTn = w;  // q_a
        } else if constexpr (e.q == 1) {
          bTn = s_in * (bTn * w);  // (a <- b): q_a k_b
        } else if constexpr (e.q == 2) {
          t2 = w;  // q_b
        } else {
          bTn += s_out * (t2 * w);  // (b <- a): q_b k_a
        }
      } else {
        if constexpr (e.q == 0) bT = bTn;
        if constexpr (RT) {
          if constexpr (e.q < 2) dh2[e.q] = mfma4(w, bT, dh2[e.q]);
          else accdr[e.q - 2] = mfma4(w, bT, accdr[e.q - 2]);  // slopes . df, rows = powers of t
        } else if constexpr (e.q < 8) {
          dh[e.q] = mfma4(w, bT, dh[e.q]);
        } else {
          dh2[e.q - 8] = mfma4(w, bT, dh2[e.q - 8]);
        }
      }
    } else if constexpr (s < B_END) {
      constexpr int mt = (s - A_END) / 3, u = (s - A_END) % 3;
      if constexpr (s == A_END) {
        // each filter forms its own copy: an opaque copy of the inputs keeps
        // the compiler from merging the two computations into one that stays
        // live across the second filter's df section
        double rr = r;
        int gg = g;
        asm volatile("" : "+v"(rr), "+v"(gg));
        rbf8_with_grad(rr, gg, A, exp2_lds, rb8, db8);
      }
      if constexpr (u == 0) {
        pre = w;
      } else {
        pre = mfma4(w, rb8[u - 1], pre);
        // silu' of the previous tile's pre-activation (complete by now) runs
        // while this tile's MFMAs do
        if constexpr (u == 1 && mt > 0) {
#pragma unroll
          for (int q = 0; q < 4; ++q) dh[mt - 1][q] *= silu_prime_tab(prev[q], exp2_lds);
        }
        if constexpr (u == 2) prev = pre;
      }
    } else if constexpr (s < C_END) {
      if constexpr (s < C_END - 1) {
        pre2[s - B_END] = w;
      } else {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          pre2[mt] = mfma(w[mt], sg, pre2[mt]);
#pragma unroll
          for (int q = 0; q < 4; ++q) dh2[mt][q] *= silu_prime_tab_wide(pre2[mt][q], exp2_lds);
        }
      }
    } else if constexpr (s < D_END) {
      if constexpr (s == C_END) {
        drb[0] = zero;
        drb[1] = zero;
      }
      drb[(s - C_END) % 2] = mfma4(w, dh[(s - C_END) / 2], drb[(s - C_END) % 2]);
      if constexpr (s == D_END - 1) {
        // dE/dr through the Bernstein basis
#pragma unroll
        for (int t = 0; t < 8; ++t) part += drb[t >> 2][t & 3] * db8[t >> 2][t & 3];
        pin(part);
      }
    } else {
      if constexpr (s == D_END) dsa = zero;
      dsa = mfma4(w, dh2[s - D_END], dsa);
      if constexpr (s == D_END + E_LEN - 1) {
        ds_acc += dsa[0];  // rows 0..3 of the padded tile: lane group g, register 0
        pin(ds_acc);
      }
    }
    // the last tile's silu' (it is needed from the last two W0^T steps on)
    if constexpr (!RT && s == B_END) {
#pragma unroll
      for (int q = 0; q < 4; ++q) dh[7][q] *= silu_prime_tab(prev[q], exp2_lds);
    }
  });

  // RT: the radial branches' dE/dr, sum over the powers of t (tile m, row
  // g + 4 r: power 16 m + g + 4 r)
  if constexpr (RT) {
    double sum = 0.0;
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) sum += accdr[m][r] * tp[m][r];
    part = inside ? sum : 0.0;
  }
  // dE/dr: the Bernstein part of both filters + the cutoff
  part += __shfl_xor(part, 16, kWave);
  part += __shfl_xor(part, 32, kWave);
  if (valid) {
    if constexpr (!EV0) ds[4 * std::size_t(p) + g] = ds_acc;
    if (g == 0) {
      if constexpr (!EV0) dfc = pdfc[pp];
      double grad = part;
      if (r < rc) {
        const double t = r / rc;
        grad += dfc * (-30.0 * t * t * (1.0 - t) * (1.0 - t) / rc);
      }
      dr[p] += grad;
    }
  }
}

// ---------------------------------------------------------------- block 0 through element-pair tables
// Block 0's node rows (q, k, v, q_ev, k_ev) are projections of the embedding
// x0, which in a one-image system is a function of the atomic number alone
// (x0[i] = (emb[z_i] + charge/spin table[z_i]) / scale): the rows take one
// value per element present, its class.  Block 0 uses its filter outputs f
// only inside the attention logits <q_a (.) k_b, f>_h, with
// f = W1 silu(W0 rbf + b0) + ob1 (the ev = 0 spherical branch folded into
// ob1).  With the element-pair tables, for filter w, classes A, B, head h,
//   M[w][A][B][h] = W1_w^T (q_A (.) k_B on the 32 channels of head h)   (128)
//   c0[w][A][B][h] = <q_A (.) k_B, ob1_w>_h
// a logit is <M[w][A][B][h], hidden> + c0[w][A][B][h], and the reverse's
// W1^T df is sum_h s_in_h M[w][A][B][h] + s_out_h M[w][B][A][h]; the head
// sums <gainv_a, v_b>_h are Gv[a][class(b)][h] (k_class_gv).  The W1 and E1
// products (two thirds of block 0's filter MFMAs) and the node-row gathers
// drop out.  Same algebra as k_filter_fwd_mfma<true> / k_filter_bwd_mfma<true,
// .>, different rounding.
//
// Table rows hold the 128 hidden features in the MFMA register order: the
// coefficient of feature f at tpos(f), so that a lane's four features of
// tile t (16 t + g + 4 r) are the 32-byte vector at 16 t + 4 g.  The node
// rows use the same order for their channels.
constexpr int kMaxClasses = 16;
__host__ __device__ constexpr int tpos(int c) { return 16 * (c / 16) + 4 * (c % 4) + (c % 16) / 4; }

// rep[c] = the node that holds class c's first atom (rep0[c], caller's order);
// also clears the class-pair histogram of k_cls_count (nkeys entries)
__global__ void k_class_reps(int n, const int *z, const int *cls, const int *perm, const int *rep0, int *rep,
                             int nkeys, int *hist) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < nkeys) hist[i] = 0;
  if (i >= n) return;
  const int c = cls[z[i]];
  if ((perm ? perm[i] : i) == rep0[c]) rep[c] = i;
}

// Block 0's input rows of the classes (rep[c]'s row of x), for their q k v
// rows (k_qkv_mfma on C rows): the only block-0 node rows the table path reads.
__global__ void k_class_rows(int C, const int *rep, const double *__restrict__ x, double *__restrict__ xc) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= C * kF) return;
  xc[t] = x[std::size_t(rep[t / kF]) * kF + t % kF];
}

// One block per (A, B) and (w, h); thread f = hidden feature.  qkv: the
// classes' rows (k_class_rows).
__global__ __launch_bounds__(128) void k_class_tables(int C, const double *__restrict__ qkv,
                                                      const double *__restrict__ w1_0,
                                                      const double *__restrict__ w1_1,
                                                      const double *__restrict__ ob_0,
                                                      const double *__restrict__ ob_1, double *Mt, double *c0) {
  const int A = blockIdx.x / C, B = blockIdx.x % C, w = blockIdx.y / 4, h = blockIdx.y % 4;
  const int f = threadIdx.x;
  const double *W1 = w ? w1_1 : w1_0;  // (out, in)
  const double *qa = qkv + std::size_t(A) * 640 + (w ? 384 : 0);
  const double *kb = qkv + std::size_t(B) * 640 + (w ? 512 : 128);
  __shared__ double qk[32];
  if (f < 32) {
    const int pc = tpos(32 * h + f);
    qk[f] = qa[pc] * kb[pc];
  }
  __syncthreads();
  const std::size_t row = ((std::size_t(w) * C + A) * C + B) * 4 + h;
  double acc = 0.0;
  for (int k = 0; k < 32; ++k) acc += W1[std::size_t(32 * h + k) * kF + f] * qk[k];
  Mt[row * kF + tpos(f)] = acc;
  if (f == 0) {
    const double *ob = w ? ob_1 : ob_0;
    double s = 0.0;
    for (int k = 0; k < 32; ++k) s += ob[32 * h + k] * qk[k];
    c0[row] = s;
  }
}

// Gv[a][B][h] = <gainv_a, v_B>_h over positions 32 h .. 32 h + 31 (one
// head's two tiles) of both rows: one wavefront per node, lane l holding
// positions 2 l and 2 l + 1, so its 16-lane row is head l / 16; qkv: the
// classes' rows.
__global__ __launch_bounds__(256) void k_class_gv(int n, int C, const double *__restrict__ gainv,
                                                  const double *__restrict__ qkv, double *Gv) {
  const int lane = threadIdx.x & 63;
  const int a = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (a >= n) return;  // the whole wavefront
  const double2 ga = *reinterpret_cast<const double2 *>(gainv + std::size_t(a) * kF + 2 * lane);
  for (int B = 0; B < C; ++B) {
    const double2 v = *reinterpret_cast<const double2 *>(qkv + std::size_t(B) * 640 + 256 + 2 * lane);
    const double sum = group_sum(ga.x * v.x + ga.y * v.y);
    if ((lane & 15) == 0) Gv[(std::size_t(a) * C + B) * 4 + (lane >> 4)] = sum;
  }
}

// A lane's 32 bytes of a table row through buffer loads: the lane's row
// start in a vector offset, the row and tile part (the same for every lane)
// in a scalar offset, so the 64 rows of a filter need no vector addresses.
// The offset passes through an empty asm, which keeps the compiler from
// hoisting every row's load to the start of the section (the rows' uses
// carry no MFMA dependence that would hold them in their stream slots).
__device__ __forceinline__ v4d table_load(__amdgpu_buffer_rsrc_t rs, int voff, int soff) {
  asm volatile("" : "+v"(voff));
  const v4u x = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, 0);
  const v4u y = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + 16, soff, 0);
  return v4d{u2_to_f64(x[0], x[1]), u2_to_f64(x[2], x[3]), u2_to_f64(y[0], y[1]), u2_to_f64(y[2], y[3])};
}

// The active pairs in order of their element pair {min, max} (key
// min * C + max), for the table kernels: a wavefront's 16 pairs then read the
// same table rows, which the vector L1 serves once.  A counting sort: counts
// (k_cls_count), bucket starts (k_cls_scan), placement (k_cls_place).  Within
// a bucket the order depends on the atomics' timing; every pair's results go
// to its own slots, so the kernels' outputs do not.
__device__ __forceinline__ int cls_key(int ca, int cb, int C) { return ca < cb ? ca * C + cb : cb * C + ca; }

// One LDS atomic per distinct key in a wavefront: the lanes of each key are
// found with a ballot, the first of them adds their count.  Returns, in
// every lane with a key, the value the atomic returned for its key plus the
// lane's rank among that key's lanes; key < 0: no key (returns 0).
__device__ __forceinline__ int wave_key_add(int key, int *counters) {
  const int lane = threadIdx.x & 63;
  const unsigned long long below = (1ull << lane) - 1ull;
  unsigned long long left = __ballot(key >= 0);
  int out = 0;
  while (left) {
    const int leader = __ffsll((long long)left) - 1;
    const int lk = __shfl(key, leader, kWave);
    const unsigned long long m = __ballot(key == lk);
    int base = 0;
    if (lane == leader) base = atomicAdd(&counters[lk], __popcll(m));
    base = __shfl(base, leader, kWave);
    if (key == lk) out = base + __popcll(m & below);
    left &= ~m;
  }
  return out;
}

// Each block takes kClsChunk consecutive pairs (16 per thread), so the
// global counters see one atomic per key and block.
constexpr int kClsPer = 16, kClsChunk = 256 * kClsPer;

__global__ __launch_bounds__(256) void k_cls_count(const int *n_active, const int *pa, const int *z, const int *cls,
                                                   int C, int *hist) {
  __shared__ int lc[kMaxClasses * kMaxClasses];
  const int nact = *n_active;
  const int p0 = blockIdx.x * kClsChunk;
  if (p0 >= nact) return;  // the whole block
  for (int t = threadIdx.x; t < C * C; t += 256) lc[t] = 0;
  __syncthreads();
  for (int it = 0; it < kClsPer; ++it) {
    const int p = p0 + it * 256 + threadIdx.x;
    const int key = p < nact ? cls_key(cls[z[pa[2 * p]]], cls[z[pa[2 * p + 1]]], C) : -1;
    (void)wave_key_add(key, lc);
  }
  __syncthreads();
  for (int t = threadIdx.x; t < C * C; t += 256)
    if (lc[t]) atomicAdd(&hist[t], lc[t]);
}

// bucket starts into cursor (advanced by the placement), each bucket padded
// to a multiple of pad slots; the slots' end into *total when given
__global__ void k_cls_scan(int nkeys, const int *hist, int *cursor, int pad, int *total) {
  if (threadIdx.x != 0) return;
  int run = 0;
  for (int t = 0; t < nkeys; ++t) {
    cursor[t] = run;
    run += (hist[t] + pad - 1) / pad * pad;
  }
  if (total) *total = run;
}

__global__ __launch_bounds__(256) void k_cls_place(const int *n_active, const int *pa, const int *z, const int *cls,
                                                   int C, int *cursor, int *order) {
  __shared__ int lc[kMaxClasses * kMaxClasses], lb[kMaxClasses * kMaxClasses];
  const int nact = *n_active;
  const int p0 = blockIdx.x * kClsChunk;
  if (p0 >= nact) return;
  for (int t = threadIdx.x; t < C * C; t += 256) lc[t] = 0;
  __syncthreads();
  int key[kClsPer], rank[kClsPer];
#pragma unroll
  for (int it = 0; it < kClsPer; ++it) {
    const int p = p0 + it * 256 + threadIdx.x;
    key[it] = p < nact ? cls_key(cls[z[pa[2 * p]]], cls[z[pa[2 * p + 1]]], C) : -1;
    rank[it] = wave_key_add(key[it], lc);
  }
  __syncthreads();
  for (int t = threadIdx.x; t < C * C; t += 256) lb[t] = lc[t] ? atomicAdd(&cursor[t], lc[t]) : 0;
  __syncthreads();
#pragma unroll
  for (int it = 0; it < kClsPer; ++it)
    if (key[it] >= 0) order[lb[key[it]] + rank[it]] = p0 + it * 256 + threadIdx.x;
}

// Block 0's forward filter through the tables: per filter the stream holds
// the layer-0 bias tiles (8), W0 (16: tile s % 8, K chunk s / 8), the table
// rows of both directions (64: direction, head, tile; the lane's four
// features of each) and the two c0 vectors (heads 0..3).  Writes the logits
// (palpha) of both directions and filters, as k_filter_fwd_mfma<true>.
// Three wavefronts per SIMD with four stream entries in flight (160
// registers): 0.356 against 0.369 ms at config 3 for two wavefronts and six.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 3))) void k_filter_fwd_class(
    const int *n_active, const int *order, const int *pa, const double *pr, const int *__restrict__ z,
    const int *__restrict__ cls, int C, const double *__restrict__ Mt, const double *__restrict__ c0, double inv_avg,
    FilterMfma A, double *palpha) {
  SO3LR_EXP2_TABLE(A)
  const int nact = *n_active;
  const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
  const int blk = xcd_block_active((nact + 63) / 64);
  if (blk < 0) return;
  const int wave = blk * 4 + (threadIdx.x >> 6);
  if (wave * 16 >= nact) return;
  // slot q of the element-pair order holds pair p
  const int q = wave * 16 + j;
  const bool valid = q < nact;
  const int p = order[valid ? q : nact - 1];
  const int ca = cls[z[pa[2 * p]]], cb = cls[z[pa[2 * p + 1]]];
  const int tw = C * C * 4 * kF * 8, cw = C * C * 4;  // one filter's tables (bytes; entries)
  // direction 0 reads the rows of (lo, hi), direction 1 those of (hi, lo),
  // the same in every lane of a bucket; with ca > cb direction 0 is b <- a
  const bool sw = ca > cb;
  const int lo = sw ? cb : ca, hi = sw ? ca : cb;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<double *>(Mt), 0, 0x7fffffff, 0x00020000);
  const int vab = ((lo * C + hi) * 4 * kF + 4 * g) * 8, vba = ((hi * C + lo) * 4 * kF + 4 * g) * 8;
  const double *cab = c0 + std::size_t(lo * C + hi) * 4, *cba = c0 + std::size_t(hi * C + lo) * 4;
  constexpr int NF = 24 + 64 + 2;
  auto load = [&](auto si) -> v4d {
    constexpr int S = decltype(si)::value, which = S / NF, s = S % NF;
    if constexpr (s < 8) return tile_load(A.b0p[which], s, lane);
    else if constexpr (s < 24) return wload(A.w0p[which], 2, (s - 8) % 8, (s - 8) / 8, lane);
    else if constexpr (s < 88) {
      constexpr int k = s - 24, dir = k / 32, hd = (k / 8) % 4, t = k % 8;
      return table_load(rs, dir ? vba : vab, which * tw + (hd * kF + 16 * t) * 8);
    } else {
      return *reinterpret_cast<const v4d *>((s == 88 ? cab : cba) + which * cw);
    }
  };
  Stream<2 * NF, 4, decltype(load)> st(load);
  st.prime();

  v4d rb[2];
  rbf8(pr[p], g, A, exp2_lds, rb);
  v4d h[8], cv0;
  double acc[8];  // [direction * 4 + head]: this lane's part of the logits
  st.run([&](auto si, const v4d &w) {
    constexpr int S = decltype(si)::value, which = S / NF, s = S % NF;
    if constexpr (s < 8) {
      h[s] = w;
    } else if constexpr (s < 24) {
      constexpr int i = s - 8;
      h[i % 8] = mfma4(w, rb[i / 8], h[i % 8]);
    } else if constexpr (s < 88) {
      constexpr int k = s - 24, dir = k / 32, hd = (k / 8) % 4, t = k % 8;
      if constexpr (k < 8) {  // each hidden tile's SiLU at its first use
#pragma unroll
        for (int r = 0; r < 4; ++r) h[t][r] = silu_tab(h[t][r], exp2_lds);
      }
      const double d = ((w[0] * h[t][0] + w[1] * h[t][1]) + w[2] * h[t][2]) + w[3] * h[t][3];
      if constexpr (t == 0) acc[dir * 4 + hd] = d;
      else acc[dir * 4 + hd] += d;
    } else if constexpr (s == 88) {
      cv0 = w;
    } else {
      // sums over the four lane groups; lane group g writes head g
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        acc[q] += __shfl_xor(acc[q], 16, kWave);
        acc[q] += __shfl_xor(acc[q], 32, kWave);
      }
      if (valid) {
        const double d0 = (pick4(g, acc[0], acc[1], acc[2], acc[3]) + pick4(g, cv0[0], cv0[1], cv0[2], cv0[3])) * inv_avg;
        const double d1 = (pick4(g, acc[4], acc[5], acc[6], acc[7]) + pick4(g, w[0], w[1], w[2], w[3])) * inv_avg;
        double *al = palpha + 16 * std::size_t(p) + 4 * which;
        al[g] = sw ? d1 : d0;  // a <- b
        al[8 + g] = sw ? d0 : d1;  // b <- a
      }
    }
  });
}

// Block 0's reverse filter through the tables (k_filter_bwd_mfma<true, FIRST>
// with the df section replaced): per filter the stream holds the table rows
// (64: direction, head, tile), then per tile the layer-0 bias and W0 chunks
// (24: the pre-activation recomputed, d hidden *= silu'), then W0^T (16:
// d rbf = W0^T d hidden).  The head sums of the invariant filter come from
// Gv, those of the equivariant filter from <gev, Y> as in the full kernel.
template <bool FIRST>
__global__ __launch_bounds__(256) FILTER_OCCUPANCY void k_filter_bwd_class(
    const int *n_active, const int *order, const int *pa, const double *pr, const double *pfc, const double *pY,
    const double *palpha, const double *__restrict__ gaev, const int *__restrict__ z,
    const int *__restrict__ cls, int C, const double *__restrict__ Mt, const double *__restrict__ Gv,
    double inv_avg, FilterMfma A, double rc, double *dr, double *dY) {
  SO3LR_EXP2_TABLE(A)
  const int nact = *n_active;
  const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
  const int blk = xcd_block_active((nact + 63) / 64);
  if (blk < 0) return;
  const int wave = blk * 4 + (threadIdx.x >> 6);
  if (wave * 16 >= nact) return;
  // slot q of the element-pair order holds pair pp
  const int q = wave * 16 + j;
  const bool valid = q < nact;
  const int pp = order[valid ? q : nact - 1];
  const int a = pa[2 * pp], b = pa[2 * pp + 1];
  const int ca = cls[z[a]], cb = cls[z[b]];
  const int tw = C * C * 4 * kF * 8;  // one filter's tables, bytes
  // direction 0 reads (lo, hi), direction 1 (hi, lo); with ca > cb direction
  // 0 carries the b <- a coefficients
  const bool sw = ca > cb;
  const int lo = sw ? cb : ca, hi = sw ? ca : cb;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<double *>(Mt), 0, 0x7fffffff, 0x00020000);
  const int vab = ((lo * C + hi) * 4 * kF + 4 * g) * 8, vba = ((hi * C + lo) * 4 * kF + 4 * g) * 8;
  constexpr int NB = 64 + 24 + 16;
  auto load = [&](auto si) -> v4d {
    constexpr int S = decltype(si)::value, which = S / NB, s = S % NB;
    if constexpr (s < 64) {
      constexpr int dir = s / 32, hd = (s / 8) % 4, t = s % 8;
      return table_load(rs, dir ? vba : vab, which * tw + (hd * kF + 16 * t) * 8);
    } else if constexpr (s < 88) {
      constexpr int mt = (s - 64) / 3, u = (s - 64) % 3;
      if constexpr (u == 0) return tile_load(A.b0p[which], mt, lane);
      else return wload(A.w0p[which], 2, mt, u - 1, lane);
    } else {
      constexpr int d = s - 88;
      return wload(A.w0tp[which], 8, d % 2, d / 2, lane);
    }
  };
  Stream<2 * NB, SO3LR_FILTER_BWD_PF, decltype(load)> st(load);
  st.prime();

  // the invariant filter's head sums: <gainv_a, v_b>_h and <gainv_b, v_a>_h
  const v4d gin = *reinterpret_cast<const v4d *>(Gv + (std::size_t(a) * C + cb) * 4);
  const v4d gout = *reinterpret_cast<const v4d *>(Gv + (std::size_t(b) * C + ca) * 4);
  const double r = pr[pp];
  const double fcs = pfc[pp] * inv_avg;  // fc / avg
  const double *al = palpha + 16 * std::size_t(pp);
  // equivariant pair terms: lane group g takes degree slot g, as in
  // k_filter_bwd_mfma: its <gev_a, Y>, <gev_b, Y> and its share of dE/dY
  double ce_mine = 0.0, coe_mine = 0.0;
  {
    const int lo = ev_offset(g), n_m = 2 * g + 3;
    const double par = slot_parity(g);
    const double ain_e = al[4 + g], aout_e = al[12 + g];
    const double *gea = gaev + std::size_t(a) * kE, *geb = gaev + std::size_t(b) * kE;
    const double *y = pY + kE * std::size_t(pp);
    double *dy = dY + kE * std::size_t(pp);
    const double fc = pfc[pp];
    for (int k = 0; k < n_m; ++k) {
      const int m = lo + k;
      const double ea = gea[m], eb = geb[m], ym = y[m];
      ce_mine += ea * ym;
      coe_mine += eb * ym;
      if (valid) dy[m] = (FIRST ? 0.0 : dy[m]) + fc * (ain_e * ea + par * aout_e * eb);
    }
    coe_mine *= par;
  }
  double dfc = al[4 + g] * ce_mine + al[12 + g] * coe_mine;
  dfc += __shfl_xor(dfc, 16, kWave);
  dfc += __shfl_xor(dfc, 32, kWave);
#pragma unroll
  for (int hd = 0; hd < 4; ++hd) dfc += al[hd] * gin[hd] + al[8 + hd] * gout[hd];
  auto pin = [](double &v) { asm volatile("" : "+v"(v)); };
  pin(dfc);

  const v4d zero = v4d{0, 0, 0, 0};
  // coefficients of the direction-0 and direction-1 rows
  double s_in[4], s_out[4];
#pragma unroll
  for (int hd = 0; hd < 4; ++hd) {
    s_in[hd] = fcs * (sw ? gout[hd] : gin[hd]);
    s_out[hd] = fcs * (sw ? gin[hd] : gout[hd]);
  }
  v4d rb8[2], db8[2], dh[8], pre, prev, drb[2];
  double part = 0.0;
  st.run([&](auto si, const v4d &w) {
    constexpr int S = decltype(si)::value, which = S / NB, s = S % NB;
    if constexpr (which == 1 && s == 0) {
      // the equivariant filter's head sums: slot h lives in lane group h
#pragma unroll
      for (int hd = 0; hd < 4; ++hd) {
        const double ci = fcs * __shfl(ce_mine, j + 16 * hd, kWave);
        const double co = fcs * __shfl(coe_mine, j + 16 * hd, kWave);
        s_in[hd] = sw ? co : ci;
        s_out[hd] = sw ? ci : co;
      }
    }
    if constexpr (s < 64) {
      constexpr int dir = s / 32, hd = (s / 8) % 4, t = s % 8;
      const double c = dir ? s_out[hd] : s_in[hd];
      if constexpr (s < 8) dh[t] = c * w;
      else dh[t] += c * w;
      // held here: sunk to its use, every row would stay live until then
      asm volatile("" : "+v"(dh[t]));
    } else if constexpr (s < 88) {
      constexpr int mt = (s - 64) / 3, u = (s - 64) % 3;
      if constexpr (s == 64) {
        // an opaque copy per filter, as in k_filter_bwd_mfma
        double rr = r;
        int gg = g;
        asm volatile("" : "+v"(rr), "+v"(gg));
        rbf8_with_grad(rr, gg, A, exp2_lds, rb8, db8);
      }
      if constexpr (u == 0) {
        pre = w;
      } else {
        pre = mfma4(w, rb8[u - 1], pre);
        if constexpr (u == 1 && mt > 0) {
#pragma unroll
          for (int q = 0; q < 4; ++q) dh[mt - 1][q] *= silu_prime_tab(prev[q], exp2_lds);
        }
        if constexpr (u == 2) prev = pre;
      }
    } else {
      constexpr int d = s - 88;
      if constexpr (d == 0) {
#pragma unroll
        for (int q = 0; q < 4; ++q) dh[7][q] *= silu_prime_tab(prev[q], exp2_lds);
        drb[0] = zero;
        drb[1] = zero;
      }
      drb[d % 2] = mfma4(w, dh[d / 2], drb[d % 2]);
      if constexpr (d == 15) {
#pragma unroll
        for (int t = 0; t < 8; ++t) part += drb[t >> 2][t & 3] * db8[t >> 2][t & 3];
        pin(part);
      }
    }
  });

  part += __shfl_xor(part, 16, kWave);
  part += __shfl_xor(part, 32, kWave);
  if (valid && g == 0) {
    double grad = part;
    if (r < rc) {
      const double t = r / rc;
      grad += dfc * (-30.0 * t * t * (1.0 - t) * (1.0 - t) / rc);
    }
    dr[pp] += grad;
  }
}

// ---------------------------------------------------------------- block 0, radial tables
// With the element-pair tables, each of block 0's logits is a fixed function
// of r per element pair: <M[w][A][B][h], h_w(r)> + c0[w][A][B][h], h_w the
// filter's radial hidden layer.  fit_radial_hidden (radial_table.cpp) fits
// h_w and dh_w/dr per interval of [r0, rc] as polynomials of degree 13 in
// t in [-1, 1] (monomial coefficients, [w][interval][power][feature]);
// k_radial_tables contracts them with the element pairs' M rows into one
// polynomial per logit and its r-derivative.  The forward then evaluates 16
// polynomials per pair instead of both filters' MFMA chains, the reverse 16
// derivatives instead of recomputing the pre-activations.
//
// Table records (mfma_ops.hpp) of 16 logits: l = 8 w + 4 dir + h, dir 0:
// lo <- hi, the M rows of (lo, hi).
constexpr int kRadRecord = kRadialCoefs * 16;

// One block per (element pair, interval), thread (power k, logit l):
// coefficient k of logit l's polynomial and of its derivative.  c0 joins
// the constant coefficient of the value.
__global__ __launch_bounds__(256) void k_radial_tables(int C, const double *__restrict__ Mt,
                                                       const double *__restrict__ c0,
                                                       const double *__restrict__ gval,
                                                       const double *__restrict__ gslope, RadialDomain d,
                                                       double *tval, double *tslope) {
  const int key = blockIdx.x / d.intervals, i = blockIdx.x % d.intervals;
  const int t = threadIdx.x;
  if (t >= 16 * kRadialCoefs) return;
  int lo = 0, start = 0;
  while (start + (C - lo) <= key) start += C - lo++;
  const int hi = lo + (key - start);
  const int l = t & 15, k = t >> 4;
  const int w = l >> 3, dir = (l >> 2) & 1, h = l & 3;
  const int A = dir ? hi : lo, B = dir ? lo : hi;
  const std::size_t row = ((std::size_t(w) * C + A) * C + B) * 4 + h;
  const double *m = Mt + row * kF;
  const std::size_t g = ((std::size_t(w) * d.intervals + i) * kRadialCoefs + k) * kF;
  double av = 0.0, as = 0.0;
  for (int f = 0; f < kF; ++f) {
    const double mf = m[tpos(f)];
    av += mf * gval[g + f];
    as += mf * gslope[g + f];
  }
  if (k == 0) av += c0[row];
  const std::size_t o = (std::size_t(key) * d.intervals + i) * kRadRecord + (k >> 1) * 32 + 2 * l + (k & 1);
  tval[o] = av;
  tslope[o] = as;
}

// Block 0's forward through the radial tables: 16 lanes per pair (lane l =
// logit 8 w + 4 dir + h), 16 pairs per block in pair order (no element-pair
// sort: the tables of a few elements stay in L2).  Writes the logits as
// k_filter_fwd_class.
__global__ __launch_bounds__(256) void k_radial_fwd(const int *n_active, const int *pa,
                                                    const double *pr, const int *__restrict__ z,
                                                    const int *__restrict__ cls, int C,
                                                    const double *__restrict__ tval, RadialDomain d, double inv_avg,
                                                    double *palpha) {
  const int nact = *n_active;
  const int blk = xcd_block_active((nact + 15) / 16);
  if (blk < 0) return;
  const int q = blk * 16 + (threadIdx.x >> 4), l = threadIdx.x & 15;
  if (q >= nact) return;  // the pair's 16 lanes
  const int p = q;
  const int ca = cls[z[pa[2 * p]]], cb = cls[z[pa[2 * p + 1]]];
  const bool sw = ca > cb;
  const int lo = sw ? cb : ca, hi = sw ? ca : cb;
  double t;
  bool inside;
  const int i = radial_locate(pr[p], d, t, inside);
  const double *rec = tval + (std::size_t(tri_key(lo, hi, C)) * d.intervals + i) * kRadRecord;
  const double v = radial_eval<16>(rec, l, t);
  // lo <- hi is a <- b unless the classes are swapped
  const int dir = (l >> 2) & 1;
  palpha[16 * std::size_t(p) + (((dir ^ int(sw)) << 3) | ((l >> 3) << 2) | (l & 3))] = v * inv_avg;
}

// Block 0's reverse through the radial tables (k_filter_bwd_class's result):
// lane l of a pair holds logit l's head sum S (invariant filter: Gv; the
// equivariant filter's degree slot h: <gev, Y>), adds al * S to dE/dfc and
// fc/avg * S * d logit/dr to dE/dr; the pair's lanes share its 24 channels of
// dE/dY.
template <bool FIRST>
__global__ __launch_bounds__(256) void k_radial_bwd(const int *n_active, const int *pa,
                                                    const double *pr, const double *pfc, const double *pY,
                                                    const double *palpha, const double *__restrict__ gaev,
                                                    const int *__restrict__ z, const int *__restrict__ cls, int C,
                                                    const double *__restrict__ tslope, const double *__restrict__ Gv,
                                                    RadialDomain d, double inv_avg, double rc, double *dr,
                                                    double *dY) {
  const int nact = *n_active;
  const int blk = xcd_block_active((nact + 15) / 16);
  if (blk < 0) return;
  const int q = blk * 16 + (threadIdx.x >> 4), l = threadIdx.x & 15;
  if (q >= nact) return;  // the pair's 16 lanes
  const int p = q;
  const int a = pa[2 * p], b = pa[2 * p + 1];
  const int ca = cls[z[a]], cb = cls[z[b]];
  const bool sw = ca > cb;
  const int lo = sw ? cb : ca, hi = sw ? ca : cb;
  const double r = pr[p];
  double t;
  bool inside;
  const int i = radial_locate(r, d, t, inside);
  const double *rec = tslope + (std::size_t(tri_key(lo, hi, C)) * d.intervals + i) * kRadRecord;
  const double slope = inside ? radial_eval<16>(rec, l, t) : 0.0;
  const int w = l >> 3, h = l & 3, dd = ((l >> 2) & 1) ^ int(sw);  // dd 0: a <- b
  const double *al = palpha + 16 * std::size_t(p);
  const double al_m = al[(dd << 3) | (w << 2) | h];
  const double fc = pfc[p];
  // the equivariant pair terms channel by channel: lane l takes channels l
  // and 16 + l (l < 8) of dE/dY and of the slot sums <gev_a, Y>_s (es[s])
  // and <gev_b, Y>_s (es[4 + s]), summed over the pair's lanes below
  const double *gea = gaev + std::size_t(a) * kE, *geb = gaev + std::size_t(b) * kE;
  const double *y = pY + kE * std::size_t(p);
  double *dy = dY + kE * std::size_t(p);
  double es[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int m = l + 16 * c;
    if (m < kE) {
      const int hs = m < 3 ? 0 : (m < 8 ? 1 : (m < 15 ? 2 : 3));
      const double ea = gea[m], eb = geb[m], ym = y[m];
      dy[m] = (FIRST ? 0.0 : dy[m]) + fc * (al[4 + hs] * ea + slot_parity(hs) * al[12 + hs] * eb);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        es[s] += hs == s ? ea * ym : 0.0;
        es[4 + s] += hs == s ? eb * ym : 0.0;
      }
    }
  }
#pragma unroll
  for (int o = 1; o < 16; o <<= 1)
#pragma unroll
    for (int k = 0; k < 8; ++k) es[k] += __shfl_xor(es[k], o, 16);
  // head sum of this lane's logit: invariant filter from Gv, equivariant
  // filter (slot h) from the slot sums
  double S;
  if (w == 0) S = Gv[(std::size_t(dd ? b : a) * C + (dd ? ca : cb)) * 4 + h];
  else S = dd ? slot_parity(h) * pick4(h, es[4], es[5], es[6], es[7]) : pick4(h, es[0], es[1], es[2], es[3]);
  double part = fc * inv_avg * S * slope, dfc = al_m * S;
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) {
    part += __shfl_xor(part, o, 16);
    dfc += __shfl_xor(dfc, o, 16);
  }
  if (l == 0) {
    double grad = part;
    if (r < rc) {
      const double u = r / rc;
      grad += dfc * (-30.0 * u * u * (1.0 - u) * (1.0 - u) / rc);
    }
    dr[p] += grad;
  }
}

// ---------------------------------------------------------------- blocks after 0, radial tables
// A filter's radial branch W1 silu(W0 rbf + b0) + ob1 (the whole output bias
// included) depends on r alone in every block: fit_radial_hidden fits its
// 128 outputs and their r-derivatives per interval of r (32 intervals of
// degree 31 for the blocks after 0), and those blocks evaluate the fits as
// MFMA products over a wavefront's 16 pairs, which therefore lie in one
// interval.  The active pairs are bucketed by (spatial block of kRintAtoms
// nodes of their first endpoint, interval), each bucket padded to a multiple
// of 16 slots (-1 in the padding): counts (k_rint_count), bucket starts (k_rint_scan),
// placement (k_rint_place).  The nodes are in spatial order, so a block's
// buckets, run one after another on one XCD, read one region's node rows
// from L2.  Within a bucket the order depends on the atomics' timing; each
// pair's results go to its own rows, so the results do not.
__device__ __forceinline__ int rint_key(int a, double r, const RadialDomain &d) {
  double t;
  bool inside;
  return (a / kRintAtoms) * kBlockIntervals + radial_locate(r, d, t, inside);
}

// one active pair per thread: hist[key] += 1
__global__ __launch_bounds__(256) void k_rint_count(const int *n_active, const int *pa, const double *pr,
                                                    RadialDomain d, int *hist) {
  const int p = blockIdx.x * 256 + threadIdx.x;
  if (p < *n_active) atomicAdd(&hist[rint_key(pa[2 * p], pr[p], d)], 1);
}

// bucket starts, each bucket padded to a multiple of 16 slots, into cursor;
// the slots' end into *total (one block: a run of keys per thread)
__global__ __launch_bounds__(1024) void k_rint_scan(int nkeys, const int *hist, int *cursor, int *total) {
  __shared__ int v[1024];
  const int t = threadIdx.x, per = (nkeys + 1023) / 1024, k0 = t * per, k1 = min(nkeys, k0 + per);
  int own = 0;
  for (int k = k0; k < k1; ++k) own += (hist[k] + 15) / 16 * 16;
  v[t] = own;
  __syncthreads();
  for (int o = 1; o < 1024; o <<= 1) {
    const int add = t >= o ? v[t - o] : 0;
    __syncthreads();
    v[t] += add;
    __syncthreads();
  }
  int run = v[t] - own;
  for (int k = k0; k < k1; ++k) {
    cursor[k] = run;
    run += (hist[k] + 15) / 16 * 16;
  }
  if (t == 1023) *total = v[t];
}

// one active pair per thread: its slot from its bucket's cursor
__global__ __launch_bounds__(256) void k_rint_place(const int *n_active, const int *pa, const double *pr,
                                                    RadialDomain d, int *cursor, int *order) {
  const int p = blockIdx.x * 256 + threadIdx.x;
  if (p < *n_active) order[atomicAdd(&cursor[rint_key(pa[2 * p], pr[p], d)], 1)] = p;
}

// ---------------------------------------------------------------- MFMA node GEMMs
// out[n][o] = sum_k W[o][k] X[n][k] (+ epilogue), 16 nodes per wavefront as the
// MFMA column block, output features as rows.  K is read from the node rows in
// the permuted order k = 16 T + g + 4 v (zero beyond K); W is pre-permuted
// (permute_mfma) and zero-padded to 16-row tiles and 16-column K chunks.
// EPI 0: out = acc + bias; 1: out = pre, out2 = silu(pre).  The bias comes in accumulator order
// (bias_acc) and starts the accumulators.  Output tiles are taken MG at a
// time; per tile group the operand stream holds, per K chunk, the X chunk and
// the MG weight fragments.
template <int EPI, int KT, int MT, int MG>
__global__ __launch_bounds__(256) void k_gemm(int rows, int K, int O, const double *__restrict__ X, int ldx,
                                              const double *__restrict__ Wp, const double *__restrict__ biasp,
                                              double *__restrict__ out, int ldo, double *__restrict__ out2) {
  // one group of MG output tiles per wavefront (the group is blockIdx.y), so
  // a few thousand node rows still give every SIMD several wavefronts
  static_assert(MT % MG == 0, "output tiles must split into equal groups");
  constexpr int PER_T = 1 + MG, PER_G = KT * PER_T;
  const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
  const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (w * 16 >= rows) return;
  const int grp = blockIdx.y;
  const int n = w * 16 + j;
  const bool valid = n < rows;
  const int nn = valid ? n : rows - 1;
  const double *xr = X + std::size_t(nn) * ldx;
  const v4d zero = v4d{0, 0, 0, 0};

  auto load = [&](auto si) -> v4d {
    constexpr int s = decltype(si)::value, T = s / PER_T, u = s % PER_T;
    if constexpr (u == 0) {
      v4d b;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int k = 16 * T + g + 4 * v;
        b[v] = (16 * T + 16 <= K || k < K) ? xr[k] : 0.0;
      }
      return b;
    } else {
      return wload(Wp, KT, grp * MG + u - 1, T, lane);
    }
  };
  Stream<PER_G, kFilterPF, decltype(load)> st(load);
  v4d acc[MG];
#pragma unroll
  for (int q = 0; q < MG; ++q) acc[q] = biasp ? tile_load(biasp, grp * MG + q, lane) : zero;
  st.prime();
  v4d bT = zero;
  st.run([&](auto si, const v4d &wv) {
    constexpr int s = decltype(si)::value, u = s % PER_T;
    if constexpr (u == 0) {
      bT = wv;
    } else {
      acc[u - 1] = mfma4(wv, bT, acc[u - 1]);
    }
  });
  if (!valid) return;
#pragma unroll
  for (int q = 0; q < MG; ++q)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int o = 16 * (grp * MG + q) + g + 4 * r;
      if (o >= O) continue;
      const std::size_t io = std::size_t(n) * ldo + o;
      const double v = acc[q][r];
      if constexpr (EPI == 0) out[io] = v;
      if constexpr (EPI == 1) { out[io] = v; out2[io] = silu(v); }
    }
}

// Block-diagonal projections: per head h, the 160 outputs (q k v q_ev k_ev,
// 32 each) depend on x[h*32 .. h*32+32).  Wp holds, per head, the permuted
// (160 x 32) matrix; out[n][w*128 + h*32 + o].  Stream per head: the two
// input chunks, then the 10 x 2 weight fragments (tile-major).
__global__ __launch_bounds__(256) void k_qkv_mfma(int rows, const double *__restrict__ X,
                                                  const double *__restrict__ Wp, double *__restrict__ out) {
  const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
  const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (w * 16 >= rows) return;
  const int n = w * 16 + j;
  const bool valid = n < rows;
  const double *xr = X + std::size_t(valid ? n : rows - 1) * kF;
  const int h = blockIdx.y;  // one head per wavefront
  constexpr int PER_H = 2 + 20;
  auto load = [&](auto si) -> v4d {
    constexpr int s = decltype(si)::value;
    if constexpr (s < 2) {
      return v4d{xr[h * kHW + 16 * s + g], xr[h * kHW + 16 * s + g + 4], xr[h * kHW + 16 * s + g + 8],
                 xr[h * kHW + 16 * s + g + 12]};
    } else {
      return wload(Wp + std::size_t(h) * 160 * kHW, 2, (s - 2) / 2, (s - 2) % 2, lane);
    }
  };
  Stream<PER_H, kFilterPF, decltype(load)> st(load);
  st.prime();
  const v4d zero = v4d{0, 0, 0, 0};
  v4d b[2] = {zero, zero}, acc[10];
  st.run([&](auto si, const v4d &wv) {
    constexpr int s = decltype(si)::value;
    if constexpr (s < 2) {
      b[s] = wv;
      if constexpr (s == 0) {
#pragma unroll
        for (int mt = 0; mt < 10; ++mt) acc[mt] = zero;
      }
    } else {
      constexpr int mt = (s - 2) / 2, T = (s - 2) % 2;
      acc[mt] = mfma4(wv, b[T], acc[mt]);
    }
    if constexpr (s == PER_H - 1) {
      if (valid) {
        // tile mt is projection mt / 2, channels 32 h + 16 (mt % 2) + [0, 16):
        // one 16-channel tile of the row, stored in the tile-transposed order
        // (fpos), so each lane writes its four values as one vector
        double *row = out + std::size_t(n) * 640 + h * kHW + 4 * g;
#pragma unroll
        for (int mt = 0; mt < 10; ++mt)
          *reinterpret_cast<v4d *>(row + (mt >> 1) * kF + 16 * (mt & 1)) = acc[mt];
      }
    }
  });
}

// dx[n][h*32 + k] = base[n][.] + sum_{w,o} W[w][h][k][o] g[n][w*128 + h*32 + o];
// per head the permuted transpose (32 x 160), K read in the permuted order
// from the 160 gradient entries of that head.  Stream per head and K chunk:
// the gradient chunk, then the two weight fragments.
__global__ __launch_bounds__(256) void k_qkv_bwd_mfma(int rows, const double *__restrict__ G,
                                                      const double *__restrict__ Wtp, const double *__restrict__ base,
                                                      double *__restrict__ dx) {
  const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
  const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (w * 16 >= rows) return;
  const int n = w * 16 + j;
  const bool valid = n < rows;
  const double *gr = G + std::size_t(valid ? n : rows - 1) * 640;
  const int h = blockIdx.y;  // one head per wavefront
  constexpr int PER_H = 10 * 3;
  auto load = [&](auto si) -> v4d {
    constexpr int s = decltype(si)::value, T = s / 3, u = s % 3;
    if constexpr (u == 0) {
      // K entries 16 T + g + 4 v: projection T / 2, channels 32 h + 16 (T % 2)
      // + g + 4 v, adjacent in the tile-transposed row order (fpos)
      return *reinterpret_cast<const v4d *>(gr + (T >> 1) * kF + h * kHW + 16 * (T & 1) + 4 * g);
    } else {
      return wload(Wtp + std::size_t(h) * kHW * 160, 10, u - 1, T, lane);
    }
  };
  Stream<PER_H, kFilterPF, decltype(load)> st(load);
  st.prime();
  const v4d zero = v4d{0, 0, 0, 0};
  v4d bT = zero, acc[2];
  st.run([&](auto si, const v4d &wv) {
    constexpr int s = decltype(si)::value, u = s % 3;
    if constexpr (s == 0) { acc[0] = zero; acc[1] = zero; }
    if constexpr (u == 0) bT = wv;
    else acc[u - 1] = mfma4(wv, bT, acc[u - 1]);
    if constexpr (s == PER_H - 1) {
      if (valid) {
        // base (the attention-residual adjoint) is stored in the
        // tile-transposed order: channels 16 mt + g + 4 r at 16 mt + 4 g + r
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const v4d bv = *reinterpret_cast<const v4d *>(base + std::size_t(n) * kF + h * kHW + 16 * mt + 4 * g);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int c = h * kHW + 16 * mt + g + 4 * r;
            dx[std::size_t(n) * kF + c] = bv[r] + acc[mt][r];
          }
        }
      }
    }
  });
}

// ---------------------------------------------------------------- attention
// 16-byte load / store of two adjacent doubles (16-byte aligned)
__device__ __forceinline__ double2 ld2(const double *p) { return *reinterpret_cast<const double2 *>(p); }
__device__ __forceinline__ void st2(double *p, double a, double b) { *reinterpret_cast<double2 *>(p) = double2{a, b}; }
// Node-major, one wavefront per node.  Lane l works for head h = l / 16: it
// holds the invariant channels 32 h + t and 32 h + 16 + t (t = l % 16) and the
// equivariant channel off[h] + t of degree h + 1 when t < 2 h + 3, so every
// per-head sum is a 16-lane group reduction.


// Active incidence of this step: entry k of a node's list as active pair
// index * 2 + side (-1 for a candidate beyond the cutoff) and its partner
// node, so the node-major kernels read their pairs with one coalesced load
// per 64 entries instead of a chain of dependent lookups.
__global__ void k_inc_active(int E, const int *inc, const int *cand2act, const int *pa, int *iact, int *iother) {
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= E) return;
  const int e = inc[k];
  const int p = cand2act[e >> 1];
  iact[k] = p < 0 ? -1 : (p << 1 | (e & 1));
  iother[k] = p < 0 ? 0 : pa[2 * p + 1 - (e & 1)];
}

// Attention forward, node-major (kokkos_integrated_block0.cpp:330-385): for
// node n and every incident active pair p = {n, o}, the edge o -> n gives
// alpha = <q_n, k_o (.) f_p> / avg (per head) and the messages
// fc alpha v_o (invariant) and fc alpha_ev Y (equivariant, (-1)^l Y when n is
// the pair's second endpoint).  Lanes: 16 per head, two channels each.
// This full form runs with the scalar filter kernels; the MFMA filter forms
// alpha itself and k_attn_msg does the rest.
__global__ __launch_bounds__(256) void k_attn_fwd(int N, const int *inc_off, const int *__restrict__ iact,
                                                  const int *__restrict__ iother, const double *__restrict__ x,
                                                  const double *__restrict__ ev, const double *__restrict__ qkv,
                                                  const double *__restrict__ pf, const double *__restrict__ pY,
                                                  const double *__restrict__ pfc, double inv_avg,
                                                  double *__restrict__ palpha, double *__restrict__ ainv,
                                                  double *__restrict__ aev) {
  const int lane = threadIdx.x & 63;
  const int n = xcd_block() * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const int h = lane >> 4, t = lane & 15;
  // the lane's two channels sit next to each other in the tile-transposed
  // rows (filters, q k v): positions 32 h + 2 t and + 1, read as one 16-byte
  // vector; fpos is its own inverse, so the channels are fpos(position)
  const int p0 = 32 * h + 2 * t, p1 = p0 + 1;
  const int c0 = fpos(p0), c1 = fpos(p1);  // c1 = c0 + 4
  const bool evv = t < 2 * h + 3;
  const int m = evv ? ev_offset(h) + t : 0;
  const double par = slot_parity(h);
  const double *qn = qkv + std::size_t(n) * 640;
  const double2 qv = ld2(qn + p0), qev = ld2(qn + 384 + p0);
  const double q0 = qv.x, q1 = qv.y, qe0 = qev.x, qe1 = qev.y;
  double acc0 = 0.0, acc1 = 0.0, acce = 0.0;
  struct Terms { double ai, ae, d0, d1, de; };
  auto terms = [&](int e, int o) {
    const int p = e >> 1, side = e & 1;
    const double *ko = qkv + std::size_t(o) * 640;
    const double *fp = pf + 256 * std::size_t(p);
    const double2 kv = ld2(ko + 128 + p0), vv = ld2(ko + 256 + p0), kev = ld2(ko + 512 + p0);
    const double2 fv = ld2(fp + p0), fev = ld2(fp + 128 + p0);
    const double k0 = kv.x, k1 = kv.y, v0 = vv.x, v1 = vv.y, ke0 = kev.x, ke1 = kev.y;
    const double f0 = fv.x, f1 = fv.y, fe0 = fev.x, fe1 = fev.y;
    const double fc = pfc[p];
    const double y = pY[kE * std::size_t(p) + m] * (side == 0 ? 1.0 : par);
    Terms T;
    T.ai = group_sum(q0 * k0 * f0 + q1 * k1 * f1) * inv_avg;
    T.ae = group_sum(qe0 * ke0 * fe0 + qe1 * ke1 * fe1) * inv_avg;
    T.d0 = fc * T.ai * v0;
    T.d1 = fc * T.ai * v1;
    T.de = fc * T.ae * y;
    return T;
  };
  for_active_pairs(inc_off[n], inc_off[n + 1], iact, iother, lane, [&](int e1, int o1, int e2, int o2, bool two) {
    const Terms A = terms(e1, o1);
    const Terms B = terms(e2, o2);
    acc0 += A.d0; acc1 += A.d1; acce += A.de;
    if (two) { acc0 += B.d0; acc1 += B.d1; acce += B.de; }
    if (t == 0) {
      double *al = palpha + 16 * std::size_t(e1 >> 1) + 8 * (e1 & 1);
      al[h] = A.ai;
      al[4 + h] = A.ae;
      if (two) {
        double *bl = palpha + 16 * std::size_t(e2 >> 1) + 8 * (e2 & 1);
        bl[h] = B.ai;
        bl[4 + h] = B.ae;
      }
    }
  });
  const std::size_t i = std::size_t(n) * kF;
  ainv[i + c0] = x[i + c0] + acc0;
  ainv[i + c1] = x[i + c1] + acc1;
  if (evv) aev[std::size_t(n) * kE + m] = ev[std::size_t(n) * kE + m] + acce;
}

// LayerNorm over 128 channels held two per lane (biased variance), the
// lane's two channels having weights w0, w1 and biases b0, b1.
// mode (NormMode): 0 affine LayerNorm; 1 RMSNorm without scale (no mean
// removed; the caller passes w = 1, b = 0); 2 none (h = y = v, is = 1)
__device__ __forceinline__ void wave_layer_norm_pair(double v0, double v1, double w0, double w1, double b0,
                                                     double b1, double eps, int mode, double &y0, double &y1,
                                                     double &h0, double &h1, double &is) {
  const double mean = mode == 0 ? wave_sum(v0 + v1) / kF : 0.0;
  const double d0 = v0 - mean, d1 = v1 - mean;
  is = mode == 2 ? 1.0 : 1.0 / sqrt(wave_sum(d0 * d0 + d1 * d1) / kF + eps);
  h0 = d0 * is;
  h1 = d1 * is;
  y0 = h0 * w0 + b0;
  y1 = h1 * w1 + b1;
}

// Attention forward messages, node-major, with the per-direction logits the
// forward MFMA filter computed (same lane layout as k_attn_fwd): for node n
// and every incident active pair, fc alpha v_o (invariant) and fc alpha_ev Y
// (equivariant, (-1)^l Y when n is the pair's second endpoint).
__global__ __launch_bounds__(256) void k_attn_msg(int N, const int *inc_off, const int *__restrict__ iact,
                                                  const int *__restrict__ iother, const double *__restrict__ x,
                                                  const double *__restrict__ ev, const double *__restrict__ qkv,
                                                  const double *__restrict__ pY, const double *__restrict__ pfc,
                                                  const double *__restrict__ palpha, const double *__restrict__ lnw,
                                                  const double *__restrict__ lnb, double eps, int lnmode,
                                                  double *__restrict__ n1, double *__restrict__ n1hat,
                                                  double *__restrict__ n1is, double *__restrict__ act,
                                                  double *__restrict__ aev, const int *__restrict__ z,
                                                  const int *__restrict__ cls) {
  const int lane = threadIdx.x & 63;
  const int n = xcd_block() * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const int h = lane >> 4, t = lane & 15;
  const int p0 = 32 * h + 2 * t;
  const int c0 = fpos(p0), c1 = c0 + 4;
  const bool evv = t < 2 * h + 3;
  const int m = evv ? ev_offset(h) + t : 0;
  const double par = slot_parity(h);
  double acc0 = 0.0, acc1 = 0.0, acce = 0.0;
  struct Terms { double d0, d1, de; };
  auto terms = [&](int e, int o) {
    const int p = e >> 1, side = e & 1;
    // block 0 on the table path: qkv holds one row per element class
    const double2 vv = ld2(qkv + std::size_t(cls ? cls[z[o]] : o) * 640 + 256 + p0);
    const double *al = palpha + 16 * std::size_t(p) + 8 * side;
    const double ai = al[h], ae = al[4 + h];
    const double fc = pfc[p];
    const double y = pY[kE * std::size_t(p) + m] * (side == 0 ? 1.0 : par);
    return Terms{fc * ai * vv.x, fc * ai * vv.y, fc * ae * y};
  };
  for_active_pairs(inc_off[n], inc_off[n + 1], iact, iother, lane, [&](int e1, int o1, int e2, int o2, bool two) {
    const Terms A = terms(e1, o1);
    const Terms B = terms(e2, o2);
    acc0 += A.d0; acc1 += A.d1; acce += A.de;
    if (two) { acc0 += B.d0; acc1 += B.d1; acce += B.de; }
  });
  // the residual, then the post-attention block's LayerNorm 1 and the silu
  // of it (the MLP input), with the whole node row in this wavefront
  const std::size_t i = std::size_t(n) * kF;
  double y0, y1, h0, h1, is;
  wave_layer_norm_pair(x[i + c0] + acc0, x[i + c1] + acc1, lnw[c0], lnw[c1], lnb[c0], lnb[c1], eps, lnmode, y0, y1,
                       h0, h1, is);
  n1[i + c0] = y0;
  n1[i + c1] = y1;
  n1hat[i + c0] = h0;
  n1hat[i + c1] = h1;
  if (lane == 0) n1is[n] = is;
  act[i + c0] = silu(y0);
  act[i + c1] = silu(y1);
  if (evv) aev[std::size_t(n) * kE + m] = ev[std::size_t(n) * kE + m] + acce;
}

// LayerNorm over 128 channels held two per lane: channels lane and 64 + lane.
__device__ __forceinline__ void wave_layer_norm(double v0, double v1, const double *w, const double *b,
                                                double eps, int mode, int lane, double &y0, double &y1,
                                                double &h0, double &h1, double &is) {
  wave_layer_norm_pair(v0, v1, w[lane], w[64 + lane], b[lane], b[64 + lane], eps, mode, y0, y1, h0, h1, is);
}

// LN1 of the attention residual, and silu of it for the MLP input
__global__ __launch_bounds__(256) void k_post1(int N, const double *ainv, const double *w, const double *b,
                                               double eps, int mode, double *n1, double *n1hat, double *n1is,
                                               double *act) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const std::size_t i = std::size_t(n) * kF;
  double y0, y1, h0, h1, is;
  wave_layer_norm(ainv[i + lane], ainv[i + 64 + lane], w, b, eps, mode, lane, y0, y1, h0, h1, is);
  n1[i + lane] = y0; n1[i + 64 + lane] = y1;
  n1hat[i + lane] = h0; n1hat[i + 64 + lane] = h1;
  if (lane == 0) n1is[n] = is;
  act[i + lane] = silu(y0);
  act[i + 64 + lane] = silu(y1);
}


// The post-attention node chain of one block with every activation in MFMA
// registers (kokkos_post_attention_block0.cpp:302-333):
//   hpre = W1 silu(n1) + b1 (kept for the reverse), hid = silu(hpre),
//   p = n1 + W2 hid + b2,
//   t = Wint [p, inv(aev)] + bint (132 wide, kept), inv_l = sum_{m in l} aev_m^2 cg_m,
//   x' = LN2(p + t[0:128]) (statistics kept), ev' = aev (1 + t[128 + slot]).
// An MFMA output tile (rows 16 mt + 4 r + g of node j in lane j + 16 g,
// register r) is the B operand of the next layer as it stands, so the layers
// chain without memory round trips.
struct NodeChainArgs {
  const double *m1p, *m1bp, *m2p, *m2bp, *intp, *intbp;  // MFMA operand order
  const double *int_cg, *ln2w, *ln2b, *exp2_256;
  double eps;
  int mode2;  // NormMode of the second position (RMSNorm, none: w = 1, b = 0 given)
};
// Two wavefronts per 16 atoms (four per block: two 16-atom tiles), so that a
// 24k-atom system fills the chip: half h of a tile computes the output tiles
// 4 h .. 4 h + 3 of each layer (and the gate tile 8 in half 0), and the layer inputs are exchanged through LDS in the operand
// order (chunk T of lane l at buf[tile][T][l]).  LayerNorm 2's row sums are
// combined across the halves through LDS as well.
__global__ __launch_bounds__(256) void k_node_fwd(int N, const double *__restrict__ act,
                                                   const double *__restrict__ n1, const double *__restrict__ aev,
                                                   NodeChainArgs A, double *__restrict__ hpre,
                                                   double *__restrict__ tout, double *__restrict__ xout,
                                                   double *__restrict__ evout, double *__restrict__ pre2hat,
                                                   double *__restrict__ pre2is) {
  __shared__ double exp2_lds[256];
  __shared__ v4d buf[2][8][64];         // one 16-atom tile's layer input, operand order (16 KB per tile)
  __shared__ double stat[2][2][2][64];  // [tile][half][sum, sum of squares][lane]
  if (threadIdx.x < 256) exp2_lds[threadIdx.x] = A.exp2_256[threadIdx.x];
  const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
  const int wl = threadIdx.x >> 6, tile = wl >> 1, h = wl & 1;
  // every wavefront runs to the end (the barriers); rows beyond N are clamped
  const int n = blockIdx.x * 32 + tile * 16 + j;
  const bool valid = n < N;
  const std::size_t nn = std::size_t(valid ? n : N - 1);
  __syncthreads();
  auto chunk = [&](const double *rows, int T) {
    const double *r = rows + nn * kF + 16 * T + g;
    return v4d{r[0], r[4], r[8], r[12]};
  };
  // stream: MLP-1 biases (4), per T the act chunk and 4 W1 fragments (40);
  // MLP-2 biases (4), 8 x 4 W2 fragments (32), the 4 n1 chunks of the
  // residual; the interaction biases (5: the 5th is the gate tile, used by
  // half 0 only) and per T (9) 5 fragments
  constexpr int P1 = 4 + 40, P2 = P1 + 4 + 32 + 4, NS = P2 + 5 + 45;
  const int o0 = 4 * h;  // first output tile of this half
  auto tmt = [&](int q) { return q < 4 ? o0 + q : 8; };  // interaction output tile q of this half
  auto load = [&](auto si) -> v4d {
    constexpr int s = decltype(si)::value;
    if constexpr (s < 4) {
      return tile_load(A.m1bp, o0 + s, lane);
    } else if constexpr (s < P1) {
      constexpr int T = (s - 4) / 5, u = (s - 4) % 5;
      if constexpr (u == 0) return chunk(act, T);
      else return wload(A.m1p, 8, o0 + u - 1, T, lane);
    } else if constexpr (s < P1 + 4) {
      return tile_load(A.m2bp, o0 + s - P1, lane);
    } else if constexpr (s < P2 - 4) {
      constexpr int i = s - P1 - 4;
      return wload(A.m2p, 8, o0 + i % 4, i / 4, lane);
    } else if constexpr (s < P2) {
      return chunk(n1, o0 + s - (P2 - 4));
    } else if constexpr (s < P2 + 5) {
      return tile_load(A.intbp, tmt(s - P2), lane);
    } else {
      constexpr int i = s - P2 - 5;
      return wload(A.intp, 9, tmt(i % 5), i / 5, lane);
    }
  };
  // two operands in flight measured best here (88 against 94 us with four)
  Stream<NS, 2, decltype(load)> st(load);
  st.prime();

  double inv = 0.0;
  {
    const int lo = g == 0 ? 0 : (g == 1 ? 3 : (g == 2 ? 8 : 15));
    const int hi = g == 0 ? 3 : (g == 1 ? 8 : (g == 2 ? 15 : 24));
    for (int m = lo; m < hi; ++m) {
      const double a = aev[nn * kE + m];
      inv += a * a * A.int_cg[m];
    }
  }
  const v4d inv4 = v4d{inv, 0.0, 0.0, 0.0};
  v4d acc[5], pb[4], xT;
  st.run([&](auto si, const v4d &wv) {
    constexpr int s = decltype(si)::value;
    if constexpr (s < 4) {
      acc[s] = wv;
    } else if constexpr (s < P1) {
      constexpr int u = (s - 4) % 5;
      if constexpr (u == 0) xT = wv;
      else acc[u - 1] = mfma4(wv, xT, acc[u - 1]);
      if constexpr (s == P1 - 1) {
        // hpre (kept) and silu(hpre) into LDS for both halves
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          v4d hd;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            if (valid) hpre[nn * kF + 16 * (o0 + q) + 4 * r + g] = acc[q][r];
            hd[r] = silu_tab(acc[q][r], exp2_lds);
          }
          buf[tile][o0 + q][lane] = hd;
        }
        __syncthreads();
      }
    } else if constexpr (s < P1 + 4) {
      acc[s - P1] = wv;
    } else if constexpr (s < P2 - 4) {
      constexpr int i = s - P1 - 4;
      acc[i % 4] = mfma4(wv, buf[tile][i / 4][lane], acc[i % 4]);
      if constexpr (s == P2 - 5) __syncthreads();  // every half has read the MLP-2 input
    } else if constexpr (s < P2) {
      constexpr int q = s - (P2 - 4);
      pb[q] = acc[q] + wv;  // p = n1 + W2 hid + b2
      buf[tile][o0 + q][lane] = pb[q];
      if constexpr (q == 3) __syncthreads();
    } else if constexpr (s < P2 + 5) {
      acc[s - P2] = wv;
    } else {
      constexpr int i = s - P2 - 5, T = i / 5, q = i % 5;
      if (q < 4 || h == 0) {
        if constexpr (T < 8) acc[q] = mfma4(wv, buf[tile][T][lane], acc[q]);
        else acc[q] = mfma4(wv, inv4, acc[q]);
      }
    }
  });

  // interaction output (kept); LayerNorm 2 of p + t over the row, the two
  // halves' sums combined through LDS
#pragma unroll
  for (int q = 0; q < 5; ++q) {
    if (q == 4 && h != 0) break;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int c = 16 * tmt(q) + 4 * r + g;
      if (valid && c < kNI) tout[nn * kNI + c] = acc[q][r];
    }
  }
  double sum = 0.0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    pb[q] += acc[q];
#pragma unroll
    for (int r = 0; r < 4; ++r) sum += pb[q][r];
  }
  sum += __shfl_xor(sum, 16, kWave);
  sum += __shfl_xor(sum, 32, kWave);
  stat[tile][h][0][lane] = sum;
  __syncthreads();
  const double mean = A.mode2 == 0 ? (stat[tile][0][0][lane] + stat[tile][1][0][lane]) / kF : 0.0;
  double var = 0.0;
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const double d = pb[q][r] - mean;
      var += d * d;
    }
  var += __shfl_xor(var, 16, kWave);
  var += __shfl_xor(var, 32, kWave);
  stat[tile][h][1][lane] = var;
  __syncthreads();
  const double is = A.mode2 == 2 ? 1.0 : 1.0 / sqrt((stat[tile][0][1][lane] + stat[tile][1][1][lane]) / kF + A.eps);
  if (valid) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int c = 16 * (o0 + q) + 4 * r + g;
        const double hh = (pb[q][r] - mean) * is;
        pre2hat[nn * kF + c] = hh;
        xout[nn * kF + c] = hh * A.ln2w[c] + A.ln2b[c];
      }
    if (h == 0 && g == 0) pre2is[nn] = is;
  }
  if (h == 0) {
    // ev' = aev (1 + gate[slot]); gate l = t[128 + l] in lane j + 16 l of half 0
    const double gate[4] = {__shfl(acc[4][0], j, kWave), __shfl(acc[4][0], j + 16, kWave),
                            __shfl(acc[4][0], j + 32, kWave), __shfl(acc[4][0], j + 48, kWave)};
    if (valid) {
#pragma unroll
      for (int k = 0; k < 6; ++k) {
        const int m = g + 4 * k;
        evout[nn * kE + m] = aev[nn * kE + m] * (1.0 + pick4(degree_slot(m), gate[0], gate[1], gate[2], gate[3]));
      }
    }
  }
}

// Reverse of the post-attention node chain, the adjoints in MFMA registers
// (kokkos_post_attention_reverse.cpp:328-449):
//   LayerNorm 2 reverse: d = LN2^T gx, the adjoint of p and of t[0:128];
//   t[128 + l] (gates): sum_{m in l} gev_m aev_m; aev: gev (1 + gate);
//   interaction reverse: gcat = Wint^T gt; p += gcat[0:128];
//   aev += 2 aev cg gcat[128 + slot];
//   MLP reverse: ghid = (W2^T p) silu'(hpre), gact = W1^T ghid;
//   LayerNorm 1 reverse of g = p + gact silu'(n1): the adjoint of the
//   attention residual, gainv.
struct NodeChainBwdArgs {
  const double *inttp, *m2tp, *m1tp;  // MFMA operand order (transposes)
  const double *int_cg, *ln1w, *ln2w;
  int mode1, mode2;  // NormMode of the two positions: RMSNorm drops the mean term, none both
};
// Two wavefronts per 16 atoms (four per block: two 16-atom tiles): half h
// owns the feature tiles 4 h .. 4 h + 3 of every 128-wide adjoint (and the
// gate tile 8 in half 0); each layer's input adjoint is exchanged through LDS
// in the operand order, and the LayerNorm row sums are combined across the
// halves through LDS.
__global__ __launch_bounds__(256) void k_node_bwd(int N, const double *__restrict__ gx,
                                                   const double *__restrict__ gev, const double *__restrict__ t,
                                                   const double *__restrict__ aev, const double *__restrict__ pre2hat,
                                                   const double *__restrict__ pre2is, const double *__restrict__ hpre,
                                                   const double *__restrict__ n1, const double *__restrict__ n1hat,
                                                   const double *__restrict__ n1is, NodeChainBwdArgs A,
                                                   double *__restrict__ gainv, double *__restrict__ gaev) {
  __shared__ v4d buf[2][8][64];         // one tile's layer-input adjoint, operand order (16 KB per tile)
  __shared__ double stat[2][2][2][64];  // [tile][half][two sums][lane]
  const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
  const int wl = threadIdx.x >> 6, tile = wl >> 1, h = wl & 1;
  const int n = blockIdx.x * 32 + tile * 16 + j;
  const bool valid = n < N;
  const std::size_t nn = std::size_t(valid ? n : N - 1);
  const int o0 = 4 * h;
  auto chunk = [&](const double *rows, int T) {
    const double *r = rows + nn * kF + 16 * T + g;
    return v4d{r[0], r[4], r[8], r[12]};
  };
  auto tmt = [&](int q) { return q < 4 ? o0 + q : 8; };
  // both halves' two sums of a row, combined (one barrier)
  auto row_sums = [&](double a, double b, double &ta, double &tb) {
    a += __shfl_xor(a, 16, kWave);
    a += __shfl_xor(a, 32, kWave);
    b += __shfl_xor(b, 16, kWave);
    b += __shfl_xor(b, 32, kWave);
    stat[tile][h][0][lane] = a;
    stat[tile][h][1][lane] = b;
    __syncthreads();
    ta = stat[tile][0][0][lane] + stat[tile][1][0][lane];
    tb = stat[tile][0][1][lane] + stat[tile][1][1][lane];
  };
  // stream: the 4 gx and 4 LN2-normalised chunks of this half; Wint^T for
  // the 5 output tiles (the 5th, the gate tile, for half 0) over 9 K chunks;
  // W2^T for 4 tiles over 8 chunks and the 4 hpre chunks; W1^T likewise and
  // the 4 n1 and 4 LN1-normalised chunks
  constexpr int SA = 8, SB = SA + 45, SD = SB + 32 + 4, NS = SD + 32 + 8;
  auto load = [&](auto si) -> v4d {
    constexpr int s = decltype(si)::value;
    if constexpr (s < 4) return chunk(gx, o0 + s);
    else if constexpr (s < SA) return chunk(pre2hat, o0 + s - 4);
    else if constexpr (s < SB) return wload(A.inttp, 9, tmt((s - SA) % 5), (s - SA) / 5, lane);
    else if constexpr (s < SD - 4) return wload(A.m2tp, 8, o0 + (s - SB) % 4, (s - SB) / 4, lane);
    else if constexpr (s < SD) return chunk(hpre, o0 + s - (SD - 4));
    else if constexpr (s < NS - 8) return wload(A.m1tp, 8, o0 + (s - SD) % 4, (s - SD) / 4, lane);
    else if constexpr (s < NS - 4) return chunk(n1, o0 + s - (NS - 8));
    else return chunk(n1hat, o0 + s - (NS - 4));
  };
  Stream<NS, kFilterPF, decltype(load)> st(load);
  st.prime();

  const double *ger = gev + nn * kE, *aer = aev + nn * kE;
  double ga[6] = {0, 0, 0, 0, 0, 0};
  if (h == 0) {
    const double gates[4] = {t[nn * kNI + kF], t[nn * kNI + kF + 1], t[nn * kNI + kF + 2], t[nn * kNI + kF + 3]};
#pragma unroll
    for (int k = 0; k < 6; ++k) {
      const int m = g + 4 * k;
      ga[k] = ger[m] * (1.0 + pick4(degree_slot(m), gates[0], gates[1], gates[2], gates[3]));
    }
  }
  double gsum = 0.0;
  {
    const int lo = g == 0 ? 0 : (g == 1 ? 3 : (g == 2 ? 8 : 15));
    const int hi = g == 0 ? 3 : (g == 1 ? 8 : (g == 2 ? 15 : 24));
    for (int m = lo; m < hi; ++m) gsum += ger[m] * aer[m];
  }
  const v4d gt8 = v4d{gsum, 0.0, 0.0, 0.0};
  const double is2 = pre2is[nn], is1 = n1is[nn];

  v4d d[4], acc[5], hat[4];
  double mg = 0.0, mgx = 0.0;
  st.run([&](auto si, const v4d &wv) {
    constexpr int s = decltype(si)::value;
    if constexpr (s < 4) {
#pragma unroll
      for (int r = 0; r < 4; ++r) d[s][r] = wv[r] * A.ln2w[16 * (o0 + s) + 4 * r + g];
    } else if constexpr (s < SA) {
      constexpr int q = s - 4;
      hat[q] = wv;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        mg += d[q][r];
        mgx += d[q][r] * wv[r];
      }
      if constexpr (q == 3) {
        // LayerNorm 2 reverse; the adjoint of p and t[0:128] into LDS
        double tm, tx;
        row_sums(mg, mgx, tm, tx);
        tm = A.mode2 == 0 ? tm / kF : 0.0;
        tx = A.mode2 == 2 ? 0.0 : tx / kF;
#pragma unroll
        for (int q2 = 0; q2 < 4; ++q2) {
#pragma unroll
          for (int r = 0; r < 4; ++r) d[q2][r] = is2 * (d[q2][r] - tm - hat[q2][r] * tx);
          buf[tile][o0 + q2][lane] = d[q2];
        }
#pragma unroll
        for (int q2 = 0; q2 < 5; ++q2) acc[q2] = v4d{0.0, 0.0, 0.0, 0.0};
        __syncthreads();
      }
    } else if constexpr (s < SB) {
      // gcat = Wint^T [d, gate adjoints]
      constexpr int i = s - SA, T = i / 5, q = i % 5;
      if (q < 4 || h == 0) {
        if constexpr (T < 8) acc[q] = mfma4(wv, buf[tile][T][lane], acc[q]);
        else acc[q] = mfma4(wv, gt8, acc[q]);
      }
      if constexpr (s == SB - 1) {
        // p += gcat[own]; the aev adjoint gains 2 aev cg gcat[128 + slot]
        if (h == 0) {
          const double gc[4] = {__shfl(acc[4][0], j, kWave), __shfl(acc[4][0], j + 16, kWave),
                                __shfl(acc[4][0], j + 32, kWave), __shfl(acc[4][0], j + 48, kWave)};
#pragma unroll
          for (int k = 0; k < 6; ++k) {
            const int m = g + 4 * k;
            ga[k] += pick4(degree_slot(m), gc[0], gc[1], gc[2], gc[3]) * 2.0 * aer[m] * A.int_cg[m];
          }
        }
        __syncthreads();  // every half has read d
#pragma unroll
        for (int q2 = 0; q2 < 4; ++q2) {
          d[q2] += acc[q2];
          buf[tile][o0 + q2][lane] = d[q2];
          acc[q2] = v4d{0.0, 0.0, 0.0, 0.0};
        }
        __syncthreads();
      }
    } else if constexpr (s < SD - 4) {
      // W2^T p
      constexpr int i = s - SB;
      acc[i % 4] = mfma4(wv, buf[tile][i / 4][lane], acc[i % 4]);
    } else if constexpr (s < SD) {
      // ghid = (W2^T p) silu'(hpre), own tiles
      constexpr int q = s - (SD - 4);
#pragma unroll
      for (int r = 0; r < 4; ++r) hat[q][r] = acc[q][r] * silu_prime(wv[r]);
      if constexpr (q == 3) {
        __syncthreads();  // every half has read p
#pragma unroll
        for (int q2 = 0; q2 < 4; ++q2) {
          buf[tile][o0 + q2][lane] = hat[q2];
          acc[q2] = v4d{0.0, 0.0, 0.0, 0.0};
        }
        __syncthreads();
      }
    } else if constexpr (s < NS - 8) {
      // gact = W1^T ghid
      constexpr int i = s - SD;
      acc[i % 4] = mfma4(wv, buf[tile][i / 4][lane], acc[i % 4]);
    } else if constexpr (s < NS - 4) {
      // g = p + gact silu'(n1), then gh = g * w1
      constexpr int q = s - (NS - 8);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        acc[q][r] = (d[q][r] + acc[q][r] * silu_prime(wv[r])) * A.ln1w[16 * (o0 + q) + 4 * r + g];
    } else {
      hat[s - (NS - 4)] = wv;  // LayerNorm 1 normalised input
    }
  });

  // LayerNorm 1 reverse
  double m1 = 0.0, m1x = 0.0;
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      m1 += acc[q][r];
      m1x += acc[q][r] * hat[q][r];
    }
  double tm, tx;
  row_sums(m1, m1x, tm, tx);
  tm = A.mode1 == 0 ? tm / kF : 0.0;
  tx = A.mode1 == 2 ? 0.0 : tx / kF;
  if (valid) {
    // tile-transposed channel order (fpos): channels 16 T + g + 4 r, r = 0..3,
    // of this lane are one 32-byte vector at 16 T + 4 g
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v4d out;
#pragma unroll
      for (int r = 0; r < 4; ++r) out[r] = is1 * (acc[q][r] - tm - hat[q][r] * tx);
      *reinterpret_cast<v4d *>(gainv + nn * kF + 16 * (o0 + q) + 4 * g) = out;
    }
    if (h == 0) {
#pragma unroll
      for (int k = 0; k < 6; ++k) gaev[nn * kE + g + 4 * k] = ga[k];
    }
  }
}

// ---------------------------------------------------------------- heads
struct HeadArgs {
  const double *ew2, *qw2, *escale, *eshift, *qemb, *hqemb, *hvshift, *hkey_bwd, *hkey_c;
  double eb2, qb2;
  const double *ckey_bwd, *ckey_c, *cvshift;  // C6 ratio head (null: none); its hidden units at 320
  int ho;                                     // head activation row width (320, or 384 with the C6 head)
};

// energy, raw charge, Hirshfeld key and ratio (kokkos_output_heads.cpp:137-176,341-451)
// (and, with the C6 head, its logit and ratio: the same form as Hirshfeld's,
// kokkos_output_heads.cpp:108-180)
__global__ __launch_bounds__(256) void k_heads(int N, const int *z, const double *act, HeadArgs H,
                                               double *eatom, double *qraw, double *heff, double *hir,
                                               double *c6eff, double *c6r) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const double *a = act + std::size_t(n) * H.ho;
  const int zz = z[n];
  const double e = wave_sum(H.ew2[lane] * a[lane] + H.ew2[64 + lane] * a[64 + lane]);
  const double q = wave_sum(H.qw2[lane] * a[128 + lane] + H.qw2[64 + lane] * a[192 + lane]);
  // Hirshfeld logit q_emb[z] . (W2 a + b2), contracted through the element's
  // row u[z] = W2^T q_emb[z]
  const double qk = H.hkey_c[zz] + wave_sum(H.hkey_bwd[zz * kHH + lane] * a[256 + lane]);
  const double ck = H.ckey_bwd ? H.ckey_c[zz] + wave_sum(H.ckey_bwd[zz * kHH + lane] * a[320 + lane]) : 0.0;
  if (lane == 0) {
    eatom[n] = (e + H.eb2) * H.escale[zz - 1] + H.eshift[zz - 1];
    qraw[n] = q + H.qb2 + H.qemb[zz];
    const double ef = H.hvshift[zz] + qk / 8.0;  // sqrt(64)
    heff[n] = ef;
    hir[n] = fabs(ef);
    if (H.ckey_bwd) {
      const double ce = H.cvshift[zz] + ck / 8.0;
      c6eff[n] = ce;
      c6r[n] = fabs(ce);
    }
  }
}

// per-image mean removal: out = in + (target - sum_image(in)) / count  (sign = +1)
// or out = in - mean_image(in) (target ignored, sign = -1).  One block per image.
__global__ __launch_bounds__(1024) void k_image_center(const std::int64_t *img_off, const double *target,
                                                       const double *in, double *out, int mode) {
  __shared__ double part[1024];
  const std::int64_t lo = img_off[blockIdx.x], hi = img_off[blockIdx.x + 1];
  double s = 0.0;
  for (std::int64_t i = lo + threadIdx.x; i < hi; i += 1024) s += in[i];
  part[threadIdx.x] = s;
  __syncthreads();
  for (int st = 512; st > 0; st >>= 1) {
    if (int(threadIdx.x) < st) part[threadIdx.x] += part[threadIdx.x + st];
    __syncthreads();
  }
  const double cnt = double(hi - lo);
  const double shift = mode == 0 ? (target[blockIdx.x] - part[0]) / cnt : -part[0] / cnt;
  for (std::int64_t i = lo + threadIdx.x; i < hi; i += 1024) out[i] = in[i] + shift;
}

// seeds -> d/d(x_final): energy 1, charge (dE/dq - mean), Hirshfeld dE/dh
// (and dE/dc of the C6 head into its hidden units)
__global__ __launch_bounds__(256) void k_heads_bwd(int N, const int *z, const double *pre, const double *qseed,
                                                   const double *dh, const double *heff, const double *dc,
                                                   const double *c6eff, HeadArgs H, double *ghead) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const double *pr = pre + std::size_t(n) * H.ho;
  double *g = ghead + std::size_t(n) * H.ho;
  const int zz = z[n];
  const double sc = H.escale[zz - 1];
  g[lane] = sc * H.ew2[lane] * silu_prime(pr[lane]);
  g[64 + lane] = sc * H.ew2[64 + lane] * silu_prime(pr[64 + lane]);
  const double qs = qseed[n];
  g[128 + lane] = qs * H.qw2[lane] * silu_prime(pr[128 + lane]);
  g[192 + lane] = qs * H.qw2[64 + lane] * silu_prime(pr[192 + lane]);
  const double ef = heff[n];
  const double sg = ef > 0.0 ? 1.0 : (ef < 0.0 ? -1.0 : 0.0);
  const double hs = dh[n] * sg / 8.0;
  // ghh[i] = sum_j hw2[j][i] gk[j] with gk[j] = hs * hqemb[z][j] = hs * u[z][i]
  g[256 + lane] = hs * H.hkey_bwd[zz * kHH + lane] * silu_prime(pr[256 + lane]);
  if (H.ckey_bwd) {
    const double ce = c6eff[n];
    const double cs = dc[n] * (ce > 0.0 ? 1.0 : (ce < 0.0 ? -1.0 : 0.0)) / 8.0;
    g[320 + lane] = cs * H.ckey_bwd[zz * kHH + lane] * silu_prime(pr[320 + lane]);
  }
}

// ---------------------------------------------------------------- long range
// Node-major over the node's long-range entries (kokkos_physical_long_range.cpp:
// 147-380, each pair seen from both endpoints): d = x_n - x_other; F_n =
// -dE/dr d/r; half of every pair energy and of its virial goes to each
// endpoint.  SEP: the C6 ratios c6r of the model's C6 head set C6 (dE/dc into
// dcv).  The lists carry a skin (about a fifth of the entries lie beyond the
// cutoff), so the wavefront first finds the entries inside it, 64 at a time,
// queues them in LDS, and evaluates only full wavefronts of them (and one
// partial at the end): the pair terms are the kernel's whole cost.
// Src gives an entry's partner node and displacement:
//   LrRows: LAMMPS half pairs, one record per incidence entry k (the entry is
//   k itself): the partner node, this endpoint's row and the partner's row,
//   three arrays of the incidence's length (lr_rec, built with the incidence),
//   so the scan reads them in order instead of through the pair table;
//   LrImages: the device reneighbor's full list (entry = node * 32 + image code).
struct LrRows {
  static constexpr bool kByIndex = true;
  const int *o, *row_self, *row_other;
  const double *x;
  __device__ __forceinline__ int other(int e) const { return o[e]; }
  __device__ __forceinline__ void disp(int e, int, double &dx, double &dy, double &dz) const {
    const int ra = row_self[e], rb = row_other[e];
    dx = x[3 * ra] - x[3 * rb];
    dy = x[3 * ra + 1] - x[3 * rb + 1];
    dz = x[3 * ra + 2] - x[3 * rb + 2];
  }
};
struct LrImages {
  static constexpr bool kByIndex = false;
  const double *x;
  const double *shift;  // LDS: 27 x 4 image shifts (box multiples)
  __device__ __forceinline__ int other(int e) const { return e >> 5; }
  __device__ __forceinline__ void disp(int e, int n, double &dx, double &dy, double &dz) const {
    const int o = e >> 5, code = e & 31;
    const double *sh = shift + 4 * code;
    dx = x[3 * n] - x[3 * o] - sh[0];
    dy = x[3 * n + 1] - x[3 * o + 1] - sh[1];
    dz = x[3 * n + 2] - x[3 * o + 2] - sh[2];
  }
};
#ifndef SO3LR_LR_WAVES
#define SO3LR_LR_WAVES 2
#endif
#define LR_OCCUPANCY __attribute__((amdgpu_waves_per_eu(SO3LR_LR_WAVES)))
template <class Src, bool LEAN_ERF, bool SEP>
__global__ __launch_bounds__(256) LR_OCCUPANCY void k_lr(int N, const int *inc_off, const int *inc, Src S,
                                                         double lx, double ly, double lz, const int *z,
                                                         const double *q, const double *hir, const double *c6r,
                                                         LrParams P, const double *aref, const double *cref,
                                                         double *elr, double *dq, double *dhv, double *dcv,
                                                         double *flr, double *vlr, double *parts) {
  // per wavefront, up to 127 queued entries inside the cutoff: displacement,
  // partner charge, Hirshfeld ratio, C6 ratio and element (all gathered in
  // the scan, so the evaluation reads LDS only)
  struct Queue {
    double dx[128], dy[128], dz[128], qo[128], ho[128], co[SEP ? 128 : 1];
    int zo[128];
  };
  __shared__ double shift[27 * 4];
  __shared__ Queue queue[4];
  if (threadIdx.x < 27) {  // the image shift of code c: ((c/9) - 1, (c/3)%3 - 1, c%3 - 1) box lengths
    const int c = threadIdx.x;
    shift[4 * c] = (c / 9 - 1) * lx;
    shift[4 * c + 1] = ((c / 3) % 3 - 1) * ly;
    shift[4 * c + 2] = (c % 3 - 1) * lz;
    shift[4 * c + 3] = 0.0;
  }
  __syncthreads();
  if constexpr (std::is_same<Src, LrImages>::value) S.shift = shift;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int n = xcd_block() * 4 + wv;
  if (n >= N) return;
  Queue &Q = queue[wv];
  const unsigned long long below = lane ? (~0ull >> (64 - lane)) : 0ull;
  const int zn = z[n];
  const double qn = q[n], hn = hir[n], cn = SEP ? c6r[n] : 0.0;
  // the cutoff test of lr_pair_terms, widened by a relative 1e-12 so that no
  // entry it would evaluate is dropped here (it tests r < cutoff itself)
  const double rc2 = P.cutoff * P.cutoff * (1.0 + 1e-12);
  double e_el = 0, e_d = 0, sdq = 0, sdh = 0, sdc = 0, f0 = 0, f1 = 0, f2 = 0;
  double w0 = 0, w1 = 0, w2 = 0, w3 = 0, w4 = 0, w5 = 0;
  auto evaluate = [&](int i) {
    const double dx = Q.dx[i], dy = Q.dy[i], dz = Q.dz[i], qo = Q.qo[i];
    const double r = sqrt(dx * dx + dy * dy + dz * dz);
    LrPairTerms t;
    if (!lr_pair_terms<LEAN_ERF, SEP>(P, aref, cref, zn, Q.zo[i], qn, qo, hn, Q.ho[i], r, t, cn,
                                      SEP ? Q.co[SEP ? i : 0] : 0.0))
      return;
    e_el += 0.5 * t.e_el;
    e_d += 0.5 * t.e_disp;
    sdq += t.pref * qo;
    sdh += t.dh_self;
    if constexpr (SEP) sdc += t.dc_self;
    const double s = t.radial / r;
    f0 -= s * dx; f1 -= s * dy; f2 -= s * dz;
    // W = -sum_pairs d (x) f_pair, f_pair = radial d / r; half per endpoint
    w0 -= 0.5 * s * dx * dx; w1 -= 0.5 * s * dy * dy; w2 -= 0.5 * s * dz * dz;
    w3 -= 0.5 * s * dx * dy; w4 -= 0.5 * s * dx * dz; w5 -= 0.5 * s * dy * dz;
  };
  int pending = 0;  // queued entries, the same in every lane (< 64 between scans)
  const int beg = inc_off[n], end = inc_off[n + 1];
  for (int k0 = beg; k0 < end; k0 += kWave) {
    const int k = k0 + lane;
    bool in = false;
    int e = 0;
    double dx = 0, dy = 0, dz = 0;
    if (k < end) {
      e = Src::kByIndex ? k : inc[k];
      S.disp(e, n, dx, dy, dz);
      const double r2 = dx * dx + dy * dy + dz * dz;
      in = r2 > 1e-24 && r2 < rc2;
    }
    const unsigned long long m = __ballot(in);
    if (in) {
      const int i = pending + __popcll(m & below);  // at most 126
      const int o = S.other(e);
      Q.dx[i] = dx; Q.dy[i] = dy; Q.dz[i] = dz;
      Q.qo[i] = q[o]; Q.ho[i] = hir[o]; Q.zo[i] = z[o];
      if constexpr (SEP) Q.co[i] = c6r[o];
    }
    pending += __popcll(m);
    // the wavefront's LDS writes are complete before any lane reads them
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
    if (pending >= kWave) {
      evaluate(lane);
      // move the overflow (pending - 64 < 64 entries) to the front
      const int rest = pending - kWave;
      const int src = kWave + (lane < rest ? lane : 0);
      const double mx = Q.dx[src], my = Q.dy[src], mz = Q.dz[src], mq = Q.qo[src], mh = Q.ho[src];
      const double mc = SEP ? Q.co[SEP ? src : 0] : 0.0;
      const int mzo = Q.zo[src];
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
      if (lane < rest) {
        Q.dx[lane] = mx; Q.dy[lane] = my; Q.dz[lane] = mz; Q.qo[lane] = mq; Q.ho[lane] = mh; Q.zo[lane] = mzo;
        if constexpr (SEP) Q.co[lane] = mc;
      }
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
      pending = rest;
    }
  }
  if (lane < pending) evaluate(lane);
  e_el = wave_sum(e_el); e_d = wave_sum(e_d); sdq = wave_sum(sdq); sdh = wave_sum(sdh);
  if constexpr (SEP) sdc = wave_sum(sdc);
  f0 = wave_sum(f0); f1 = wave_sum(f1); f2 = wave_sum(f2);
  w0 = wave_sum(w0); w1 = wave_sum(w1); w2 = wave_sum(w2);
  w3 = wave_sum(w3); w4 = wave_sum(w4); w5 = wave_sum(w5);
  if (lane == 0) {
    elr[n] = e_el + e_d;
    dq[n] = sdq;
    dhv[n] = sdh;
    if constexpr (SEP) dcv[n] = sdc;
    flr[3 * n] = f0; flr[3 * n + 1] = f1; flr[3 * n + 2] = f2;
    double *v = vlr + 6 * std::size_t(n);
    v[0] = w0; v[1] = w1; v[2] = w2; v[3] = w3; v[4] = w4; v[5] = w5;
    parts[2 * n] = e_el;
    parts[2 * n + 1] = e_d;
  }
}

// ---------------------------------------------------------------- block reverse
// LN2 reverse, gate adjoint, start of the interaction reverse

// gp += gcat[:128]; g_aev += gcat[128 + l] 2 a_ev cg

// g_n1 = gp + gact silu'(n1); LN1 reverse -> d/d(x + d_inv)

// Attention reverse, node-major (kokkos_attention_scatter_reverse.cpp:280-500).
// For node n and each active pair p = {n, o}: the incoming edge o -> n gives
// dq_n, the outgoing edge n -> o gives dk_n, dv_n (sender-side terms,
// gathered here instead of scattered).  The endpoint with side 0 also writes
// the per-pair adjoints df (both directions), dfc and accumulates dY (the
// first reverse block, FIRST, writes it without reading).  Lane
// layout as in k_attn_fwd.
// NODE_ADJ false (block 0): only the pair adjoints are needed, not dq, dk, dv.
template <bool NODE_ADJ, bool FIRST>
__global__ __launch_bounds__(256) void k_attn_bwd(int N, const int *inc_off, const int *__restrict__ iact,
                                                  const int *__restrict__ iother, const double *__restrict__ qkv,
                                                  const double *__restrict__ pf, const double *__restrict__ pY,
                                                  const double *__restrict__ pfc, const double *__restrict__ palpha,
                                                  const double *__restrict__ gainv, const double *__restrict__ gaev,
                                                  double inv_avg, double *__restrict__ gqkv,
                                                  double *__restrict__ df, double *__restrict__ dfc,
                                                  double *__restrict__ dY) {
  const int lane = threadIdx.x & 63;
  const int n = xcd_block() * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const int h = lane >> 4, t = lane & 15;
  // the lane's two channels sit next to each other in the tile-transposed
  // rows (filters, q k v): positions 32 h + 2 t and + 1, read as one 16-byte
  // vector; fpos is its own inverse, so the channels are fpos(position)
  const int p0 = 32 * h + 2 * t;
  const bool evv = t < 2 * h + 3;
  const int m = evv ? ev_offset(h) + t : 0;
  const double par = slot_parity(h);
  const double *me = qkv + std::size_t(n) * 640;
  const double2 mqv = ld2(me + p0), mkv = ld2(me + 128 + p0), mvv = ld2(me + 256 + p0);
  const double2 mqev = ld2(me + 384 + p0), mkev = ld2(me + 512 + p0);
  const double mq0 = mqv.x, mq1 = mqv.y, mk0 = mkv.x, mk1 = mkv.y, mv0 = mvv.x, mv1 = mvv.y;
  const double mqe0 = mqev.x, mqe1 = mqev.y, mke0 = mkev.x, mke1 = mkev.y;
  const double2 mgv = ld2(gainv + std::size_t(n) * kF + p0);  // fpos rows: channels c0, c1
  const double mg0 = mgv.x, mg1 = mgv.y;
  const double mge = evv ? gaev[std::size_t(n) * kE + m] : 0.0;
  double dq0 = 0, dq1 = 0, dk0 = 0, dk1 = 0, dv0 = 0, dv1 = 0, dqe0 = 0, dqe1 = 0, dke0 = 0, dke1 = 0;
  struct Terms {
    double dq0, dq1, dqe0, dqe1, dk0, dk1, dke0, dke1, dv0, dv1;  // node-side contributions
    double g0, g1, ge0, ge1, fcg, dy;                             // pair adjoints (side 0 only); dy: new dY
  };
  auto terms = [&](int e, int o) {
    const int p = e >> 1, side = e & 1;
    const double *ot = qkv + std::size_t(o) * 640;
    const double2 oqv = ld2(ot + p0), okv = ld2(ot + 128 + p0), ovv = ld2(ot + 256 + p0);
    const double2 oqev = ld2(ot + 384 + p0), okev = ld2(ot + 512 + p0);
    const double oq0 = oqv.x, oq1 = oqv.y, ok0 = okv.x, ok1 = okv.y, ov0 = ovv.x, ov1 = ovv.y;
    const double oqe0 = oqev.x, oqe1 = oqev.y, oke0 = okev.x, oke1 = okev.y;
    // every load of the pair unconditional (m = 0 on lanes without an
    // equivariant channel: a valid address, the value is masked below), so
    // one wait covers the whole iteration
    const double2 ogv = ld2(gainv + std::size_t(o) * kF + p0);
    const double og0 = ogv.x, og1 = ogv.y;
    const double oge_ld = gaev[std::size_t(o) * kE + m];
    const double *fp = pf + 256 * std::size_t(p);
    const v2d fiv = __builtin_nontemporal_load(reinterpret_cast<const v2d *>(fp + p0));
    const v2d fev = __builtin_nontemporal_load(reinterpret_cast<const v2d *>(fp + 128 + p0));
    const double fi0 = fiv.x, fi1 = fiv.y, fe0 = fev.x, fe1 = fev.y;
    const double fc = pfc[p];
    const double y_ld = pY[kE * std::size_t(p) + m];
    const double dy_old = FIRST ? 0.0 : dY[kE * std::size_t(p) + m];  // used by the side-0 endpoint only
    const double *al = palpha + 16 * std::size_t(p);
    const double ain_i = al[8 * side + h], ain_e = al[8 * side + 4 + h];
    const double aout_i = al[8 * (1 - side) + h], aout_e = al[8 * (1 - side) + 4 + h];
    const double oge = evv ? oge_ld : 0.0;
    const double y = evv ? y_ld : 0.0;
    const double y_n = side == 0 ? y : par * y;  // harmonics of edge o -> n
    const double y_o = side == 0 ? par * y : y;  // harmonics of edge n -> o
    // per-head sums for the incoming (o -> n) and outgoing (n -> o) edges
    const double ci = group_sum(mg0 * ov0 + mg1 * ov1);
    const double ce = group_sum(mge * y_n);
    const double co = group_sum(og0 * mv0 + og1 * mv1);
    const double coe = group_sum(oge * y_o);
    const double sin_ = fc * ci * inv_avg, sine = fc * ce * inv_avg;
    const double sout = fc * co * inv_avg, soute = fc * coe * inv_avg;
    Terms T;
    T.dq0 = sin_ * ok0 * fi0; T.dq1 = sin_ * ok1 * fi1;
    T.dqe0 = sine * oke0 * fe0; T.dqe1 = sine * oke1 * fe1;
    T.dk0 = sout * oq0 * fi0; T.dk1 = sout * oq1 * fi1;
    T.dke0 = soute * oqe0 * fe0; T.dke1 = soute * oqe1 * fe1;
    T.dv0 = fc * aout_i * og0; T.dv1 = fc * aout_i * og1;
    T.g0 = sin_ * mq0 * ok0 + sout * oq0 * mk0;
    T.g1 = sin_ * mq1 * ok1 + sout * oq1 * mk1;
    T.ge0 = sine * mqe0 * oke0 + soute * oqe0 * mke0;
    T.ge1 = sine * mqe1 * oke1 + soute * oqe1 * mke1;
    // d/d fc: every head's sum appears in its 16 lanes; take one lane per head
    const double part = ain_i * ci + ain_e * ce + aout_i * co + aout_e * coe;
    T.fcg = lane_read(part, 0) + lane_read(part, 16) + lane_read(part, 32) + lane_read(part, 48);
    // dE/dY_p: edge o->n via y_n (= Y_p), edge n->o via y_o (parity)
    T.dy = dy_old + (fc * ain_e * mge + par * fc * aout_e * oge);
    return T;
  };
  auto apply = [&](const Terms &T, int e) {
    if constexpr (NODE_ADJ) {
      dq0 += T.dq0; dq1 += T.dq1;
      dqe0 += T.dqe0; dqe1 += T.dqe1;
      dk0 += T.dk0; dk1 += T.dk1;
      dke0 += T.dke0; dke1 += T.dke1;
      dv0 += T.dv0; dv1 += T.dv1;
    }
    if ((e & 1) == 0) {
      const std::size_t p = std::size_t(e >> 1);
      double *d = df + 256 * p;
      __builtin_nontemporal_store(v2d{T.g0, T.g1}, reinterpret_cast<v2d *>(d + p0));
      __builtin_nontemporal_store(v2d{T.ge0, T.ge1}, reinterpret_cast<v2d *>(d + 128 + p0));
      if (lane == 0) dfc[p] = T.fcg;
      if (evv) dY[kE * p + m] = T.dy;
    }
  };
  // one pair at a time: two in flight need ~190 registers and lose occupancy
  for_active_pairs(inc_off[n], inc_off[n + 1], iact, iother, lane, [&](int e1, int o1, int e2, int o2, bool two) {
    apply(terms(e1, o1), e1);
    if (two) apply(terms(e2, o2), e2);
  });
  if constexpr (!NODE_ADJ) return;
  double *g = gqkv + std::size_t(n) * 640;
  st2(g + p0, dq0, dq1);
  st2(g + 128 + p0, dk0, dk1);
  st2(g + 256 + p0, dv0, dv1);
  st2(g + 384 + p0, dqe0, dqe1);
  st2(g + 512 + p0, dke0, dke1);
}


// Attention reverse, node-major (kokkos_attention_scatter_reverse.cpp:
// 280-500): for node n and each active pair p = {n, o}, the incoming edge
// o -> n gives dq_n, dq_ev_n and the outgoing edge n -> o gives dk_n,
// dk_ev_n, dv_n (sender-side terms gathered, not scattered).  The endpoint
// with side 0 also writes the pair's terms for the reverse filter, which
// forms df from them and the node rows: per head h the record
//   {fc/avg ci_h, fc/avg co_h, fc/avg ce_h, fc/avg coe_h}
// (32 bytes, psc + 16 p + 4 h), dE/dfc and dE/dY (FIRST, the first block of
// the reverse pass, writes dE/dY without reading it).  Lane layout as in
// k_attn_fwd; gainv in the tile-transposed order.
template <bool FIRST>
__global__ __launch_bounds__(256) void k_attn_bwd_nodes(int N, const int *inc_off, const int *__restrict__ iact,
                                                        const int *__restrict__ iother, const double *__restrict__ qkv,
                                                        const double *__restrict__ pf, const double *__restrict__ pY,
                                                        const double *__restrict__ pfc,
                                                        const double *__restrict__ palpha,
                                                        const double *__restrict__ gainv,
                                                        const double *__restrict__ gaev, double inv_avg,
                                                        double *__restrict__ gqkv, double *__restrict__ psc,
                                                        double *__restrict__ pdfc, double *__restrict__ dY) {
  const int lane = threadIdx.x & 63;
  const int n = xcd_block() * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const int h = lane >> 4, t = lane & 15;
  const int p0 = 32 * h + 2 * t;
  const bool evv = t < 2 * h + 3;
  const int m = evv ? ev_offset(h) + t : 0;
  const double par = slot_parity(h);
  const double *me = qkv + std::size_t(n) * 640;
  const double2 mvv = ld2(me + 256 + p0);
  const double2 mgv = ld2(gainv + std::size_t(n) * kF + p0);
  const double mge = evv ? gaev[std::size_t(n) * kE + m] : 0.0;
  double dq0 = 0, dq1 = 0, dk0 = 0, dk1 = 0, dv0 = 0, dv1 = 0, dqe0 = 0, dqe1 = 0, dke0 = 0, dke1 = 0;
  auto visit = [&](int e, int o) {
    const int p = e >> 1, side = e & 1;
    const double *ot = qkv + std::size_t(o) * 640;
    const double2 oqv = ld2(ot + p0), okv = ld2(ot + 128 + p0), ovv = ld2(ot + 256 + p0);
    const double2 oqev = ld2(ot + 384 + p0), okev = ld2(ot + 512 + p0);
    const double2 ogv = ld2(gainv + std::size_t(o) * kF + p0);
    const double oge_ld = gaev[std::size_t(o) * kE + m];  // m = 0 off the ev lanes: valid, masked below
    const double *fp = pf + 256 * std::size_t(p);
    const v2d fiv = __builtin_nontemporal_load(reinterpret_cast<const v2d *>(fp + p0));
    const v2d fev = __builtin_nontemporal_load(reinterpret_cast<const v2d *>(fp + 128 + p0));
    const double fc = pfc[p];
    const double y_ld = pY[kE * std::size_t(p) + m];
    const double *al = palpha + 16 * std::size_t(p);
    const double aout_i = al[8 * (1 - side) + h];
    const double oge = evv ? oge_ld : 0.0;
    const double y = evv ? y_ld : 0.0;
    const double y_n = side == 0 ? y : par * y;  // harmonics of edge o -> n
    const double y_o = side == 0 ? par * y : y;  // harmonics of edge n -> o
    const double ci = group_sum(mgv.x * ovv.x + mgv.y * ovv.y);
    const double ce = group_sum(mge * y_n);
    const double co = group_sum(ogv.x * mvv.x + ogv.y * mvv.y);
    const double coe = group_sum(oge * y_o);
    const double sin_ = fc * ci * inv_avg, sine = fc * ce * inv_avg;
    const double sout = fc * co * inv_avg, soute = fc * coe * inv_avg;
    dq0 += sin_ * okv.x * fiv.x; dq1 += sin_ * okv.y * fiv.y;
    dqe0 += sine * okev.x * fev.x; dqe1 += sine * okev.y * fev.y;
    dk0 += sout * oqv.x * fiv.x; dk1 += sout * oqv.y * fiv.y;
    dke0 += soute * oqev.x * fev.x; dke1 += soute * oqev.y * fev.y;
    dv0 += fc * aout_i * ogv.x; dv1 += fc * aout_i * ogv.y;
    // the pair's terms, once per pair (its side-0 endpoint; side is uniform
    // across the wavefront): every head's sums appear in that head's 16 lanes
    if (side == 0) {
      const double ain_i = al[h], ain_e = al[4 + h], aout_e = al[12 + h];
      const double part = ain_i * ci + ain_e * ce + aout_i * co + aout_e * coe;
      const double fcg = lane_read(part, 0) + lane_read(part, 16) + lane_read(part, 32) + lane_read(part, 48);
      if (t == 0) *reinterpret_cast<v4d *>(psc + 16 * std::size_t(p) + 4 * h) = v4d{sin_, sout, sine, soute};
      if (lane == 0) pdfc[p] = fcg;
      if (evv) {
        double *dy = dY + kE * std::size_t(p) + m;
        *dy = (FIRST ? 0.0 : *dy) + fc * (ain_e * mge + par * aout_e * oge);
      }
    }
  };
  for_active_pairs(inc_off[n], inc_off[n + 1], iact, iother, lane, [&](int e1, int o1, int e2, int o2, bool two) {
    visit(e1, o1);
    if (two) visit(e2, o2);
  });
  double *gq = gqkv + std::size_t(n) * 640;
  st2(gq + p0, dq0, dq1);
  st2(gq + 128 + p0, dk0, dk1);
  st2(gq + 256 + p0, dv0, dv1);
  st2(gq + 384 + p0, dqe0, dqe1);
  st2(gq + 512 + p0, dke0, dke1);
}

// g_ev_in = g_aev + sum_pairs 2 (ev_n - ev_o) cg ds[slot]
__global__ __launch_bounds__(256) void k_ev_bwd(int N, const int *inc_off, const int *__restrict__ iact,
                                                const int *__restrict__ iother, const double *__restrict__ ev,
                                                const double *__restrict__ cg, const double *__restrict__ ds,
                                                const double *__restrict__ gaev, double *__restrict__ gev) {
  const int lane = threadIdx.x & 63;
  const int n = xcd_block() * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const int c = lane < kE ? lane : 0;
  const int slot = degree_slot(c);
  const double en = ev[std::size_t(n) * kE + c];
  double acc = gaev[std::size_t(n) * kE + c];
  auto term = [&](int e, int o) { return 2.0 * (en - ev[std::size_t(o) * kE + c]) * cg[c] * ds[4 * std::size_t(e >> 1) + slot]; };
  for_active_pairs(inc_off[n], inc_off[n + 1], iact, iother, lane, [&](int e1, int o1, int e2, int o2, bool two) {
    const double a = term(e1, o1), b = term(e2, o2);
    acc += a;
    if (two) acc += b;
  });
  if (lane < kE) gev[std::size_t(n) * kE + lane] = acc;
}

// ---------------------------------------------------------------- geometry
// g = dE/dv for v = x_a - x_b (kokkos_learned_energy_forces.cpp:241-306)
__global__ __launch_bounds__(256) void k_geom_bwd(const int *n_active, const double *pv, const double *pr,
                                                  const double *dr, const double *pzbl, const double *dY,
                                                  double *pg) {
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= *n_active) return;
  const double r = pr[p];
  if (r <= 1e-14) { pg[3 * p] = pg[3 * p + 1] = pg[3 * p + 2] = 0.0; return; }
  const double ux = pv[3 * p] / r, uy = pv[3 * p + 1] / r, uz = pv[3 * p + 2] / r;
  double gx = 0, gy = 0, gz = 0;
  for (int m = 0; m < kE; ++m) {
    double ax, ay, az;
    sh_component_grad(m, ux, uy, uz, ax, ay, az);
    const double w = dY[kE * std::size_t(p) + m];
    gx += w * ax; gy += w * ay; gz += w * az;
  }
  const double rad = ux * gx + uy * gy + uz * gz;
  // the ZBL energy is carried by both directed edges of the pair
  const double d = dr[p] + 2.0 * pzbl[2 * p + 1];
  pg[3 * p] = d * ux + (gx - ux * rad) / r;
  pg[3 * p + 1] = d * uy + (gy - uy * rad) / r;
  pg[3 * p + 2] = d * uz + (gz - uz * rad) / r;
}

// forces and per-atom energies: F_a = -g, F_b = +g; each endpoint receives the
// ZBL energy of the directed edge it receives
__global__ void k_fill_int(int *p, int n, int v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}
// the active-pair count next to the reduced energy and virial, for one read-back
__global__ void k_copy_count(const int *n_active, double *dst) {
  if (threadIdx.x == 0) dst[0] = double(*n_active);
}

// xn[n] = x[perm[n]] (positions into node order)
__global__ void k_gather_pos(int N, const int *perm, const double *x, double *xn) {
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k < 3 * N) xn[k] = x[3 * perm[k / 3] + k % 3];
}

__global__ __launch_bounds__(256) void k_forces(int N, const int *inc_off, const int *inc, const int *cand2act,
                                                const double *pg, const double *pzbl, const double *flr,
                                                const double *eatom, const double *elr, const int *perm,
                                                double *f, double *ezbl, double *etot) {
  const int lane = threadIdx.x & 63;
  const int n = xcd_block() * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  double f0 = 0, f1 = 0, f2 = 0, ez = 0;
  for (int k = inc_off[n] + lane; k < inc_off[n + 1]; k += kWave) {
    const int e = inc[k];
    const int p = cand2act[e >> 1];
    if (p < 0) continue;
    const double s = (e & 1) ? 1.0 : -1.0;
    f0 += s * pg[3 * p]; f1 += s * pg[3 * p + 1]; f2 += s * pg[3 * p + 2];
    ez += pzbl[2 * p];
  }
  f0 = wave_sum(f0); f1 = wave_sum(f1); f2 = wave_sum(f2); ez = wave_sum(ez);
  if (lane == 0) {
    const int a = perm ? perm[n] : n;  // caller's atom index (node order -> atom order)
    f[3 * a] = f0 + flr[3 * n];
    f[3 * a + 1] = f1 + flr[3 * n + 1];
    f[3 * a + 2] = f2 + flr[3 * n + 2];
    ezbl[n] = ez;
    etot[a] = eatom[n] + ez + elr[n];
  }
}

// Per-atom virial (no counterpart in the reference, which refuses it): each
// active SR pair's -v (x) dE/dv, symmetrised as in the global virial, split
// half to each endpoint, plus the node's long-range halves.  The atoms' sum is
// the global virial.  Node-major over the incidence lists, fixed order.
__global__ __launch_bounds__(256) void k_vatom(int N, const int *inc_off, const int *inc, const int *cand2act,
                                               const double *pv, const double *pg, const double *vlr,
                                               const int *perm, double *vatom) {
  const int lane = threadIdx.x & 63;
  const int n = xcd_block() * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  double w[6] = {0, 0, 0, 0, 0, 0};
  for (int k = inc_off[n] + lane; k < inc_off[n + 1]; k += kWave) {
    const int p = cand2act[inc[k] >> 1];
    if (p < 0) continue;
    const double *v = pv + 3 * std::size_t(p), *g = pg + 3 * std::size_t(p);
    w[0] -= 0.5 * v[0] * g[0];
    w[1] -= 0.5 * v[1] * g[1];
    w[2] -= 0.5 * v[2] * g[2];
    w[3] -= 0.25 * (v[0] * g[1] + v[1] * g[0]);
    w[4] -= 0.25 * (v[0] * g[2] + v[2] * g[0]);
    w[5] -= 0.25 * (v[1] * g[2] + v[2] * g[1]);
  }
#pragma unroll
  for (int c = 0; c < 6; ++c) w[c] = wave_sum(w[c]);
  if (lane == 0) {
    const int a = perm ? perm[n] : n;
#pragma unroll
    for (int c = 0; c < 6; ++c) vatom[6 * std::size_t(a) + c] = w[c] + vlr[6 * std::size_t(n) + c];
  }
}

// energy, virial (SR pairs + LR per-node halves), electrostatic and dispersion
// totals: red[0] E, red[1..6] W, red[7] E_el, red[8] E_disp.  One block.
// Energy, virial and energy parts: fixed-order two-stage reduction.  Block b
// sums a contiguous range of nodes and of active pairs into partial[b][0..9);
// one block then sums the partials in block order.
constexpr int kReduceBlocks = 240;

__device__ __forceinline__ void block_sum9(double *acc, double *sh, double *dst) {
  for (int c = 0; c < 9; ++c) {
    sh[threadIdx.x] = acc[c];
    __syncthreads();
    for (int st = 128; st > 0; st >>= 1) {
      if (int(threadIdx.x) < st) sh[threadIdx.x] += sh[threadIdx.x + st];
      __syncthreads();
    }
    if (threadIdx.x == 0) dst[c] = sh[0];
    __syncthreads();
  }
}

__global__ __launch_bounds__(256) void k_reduce_part(int N, const int *n_active, const double *etot,
                                                     const double *pv, const double *pg, const double *vlr,
                                                     const double *parts, double *partial) {
  __shared__ double sh[256];
  double acc[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
  const int B = gridDim.x, b = blockIdx.x;
  const int nper = (N + B - 1) / B, n0 = b * nper, n1 = min(N, n0 + nper);
  for (int i = n0 + threadIdx.x; i < n1; i += 256) {
    acc[0] += etot[i];
    for (int c = 0; c < 6; ++c) acc[1 + c] += vlr[6 * std::size_t(i) + c];
    acc[7] += parts[2 * i];
    acc[8] += parts[2 * i + 1];
  }
  const int P = *n_active;
  const int pper = (P + B - 1) / B, p0 = b * pper, p1 = min(P, p0 + pper);
  for (int p = p0 + threadIdx.x; p < p1; p += 256) {
    const double *v = pv + 3 * std::size_t(p), *g = pg + 3 * std::size_t(p);
    acc[1] -= v[0] * g[0]; acc[2] -= v[1] * g[1]; acc[3] -= v[2] * g[2];
    acc[4] -= 0.5 * (v[0] * g[1] + v[1] * g[0]);
    acc[5] -= 0.5 * (v[0] * g[2] + v[2] * g[0]);
    acc[6] -= 0.5 * (v[1] * g[2] + v[2] * g[1]);
  }
  block_sum9(acc, sh, partial + 9 * std::size_t(b));
}

__global__ __launch_bounds__(256) void k_reduce_final(int B, const double *partial, double *red) {
  __shared__ double sh[256];
  double acc[9];
  for (int c = 0; c < 9; ++c) acc[c] = int(threadIdx.x) < B ? partial[9 * threadIdx.x + c] : 0.0;
  block_sum9(acc, sh, red);
}

int ceil_div(std::int64_t a, std::int64_t b) { return int((a + b - 1) / b); }

}  // namespace

// ====================================================================== host
Evaluator::Buffer *Evaluator::buf(const char *) {
  buffers_.push_back(new Buffer());
  return buffers_.back();
}

void Evaluator::release_all() {
  for (Buffer *b : buffers_) {
    if (b->p) (void)hipFree(b->p);
    delete b;
  }
  buffers_.clear();
  for (void *p : weight_allocs_) (void)hipFree(p);
  weight_allocs_.clear();
}

void Evaluator::drop_graph() {
  if (graph_exec_) (void)hipGraphExecDestroy(graph_exec_);
  graph_exec_ = nullptr;
  graph_key_ = GraphKey{};
}

Evaluator::~Evaluator() {
  if (stream_) (void)hipStreamSynchronize(stream_);
  drop_graph();
  if (host_out_) (void)hipHostFree(host_out_);
  for (Pinned *b : {&pin_x_, &pin_f_})
    if (b->p) (void)hipHostFree(b->p);
  release_all();
  if (own_stream_) (void)hipStreamDestroy(own_stream_);
}

// (declared in evaluator.hpp: the generic path uses them too)
std::vector<double> transpose(const std::vector<double> &w, std::size_t rows, std::size_t cols) {
  std::vector<double> t(w.size());
  for (std::size_t r = 0; r < rows; ++r)
    for (std::size_t c = 0; c < cols; ++c) t[c * rows + r] = w[r * cols + c];
  return t;
}

// MFMA A-operand order of an (M x K) row-major matrix used as D = W X^T:
// P[mt][T][lane][v] = W[16 mt + lane % 16][16 T + lane / 16 + 4 v] (K a
// multiple of 16), or P[mt][lane] = W[16 mt + lane % 16][lane / 16] for K = 4.
// Rows beyond M (padding to a multiple of 16) are zero.
// Bias b (length M) in MFMA accumulator order: P[mt][lane][r] = b[16 mt +
// lane / 16 + 4 r] (zero beyond M), so a D tile starts from its bias.
std::vector<double> bias_acc(const std::vector<double> &b, std::size_t M) {
  const std::size_t MT = (M + 15) / 16;
  std::vector<double> p(MT * 64 * 4, 0.0);
  for (std::size_t mt = 0; mt < MT; ++mt)
    for (std::size_t lane = 0; lane < 64; ++lane)
      for (std::size_t r = 0; r < 4; ++r) {
        const std::size_t row = 16 * mt + lane / 16 + 4 * r;
        if (row < M) p[(mt * 64 + lane) * 4 + r] = b[row];
      }
  return p;
}

std::vector<double> permute_mfma(const std::vector<double> &w, std::size_t M, std::size_t K) {
  const std::size_t MT = (M + 15) / 16;
  if (K == 4) {
    std::vector<double> p(MT * 64, 0.0);
    for (std::size_t mt = 0; mt < MT; ++mt)
      for (std::size_t lane = 0; lane < 64; ++lane) {
        const std::size_t row = 16 * mt + lane % 16;
        if (row < M) p[mt * 64 + lane] = w[row * K + lane / 16];
      }
    return p;
  }
  if (K % 16 != 0) {  // zero-pad K to the next multiple of 16
    const std::size_t Kp = (K + 15) / 16 * 16;
    std::vector<double> wp(M * Kp, 0.0);
    for (std::size_t r = 0; r < M; ++r)
      for (std::size_t c = 0; c < K; ++c) wp[r * Kp + c] = w[r * K + c];
    return permute_mfma(wp, M, Kp);
  }
  const std::size_t KT = K / 16;
  std::vector<double> p(MT * KT * 64 * 4, 0.0);
  for (std::size_t mt = 0; mt < MT; ++mt)
    for (std::size_t T = 0; T < KT; ++T)
      for (std::size_t lane = 0; lane < 64; ++lane)
        for (std::size_t v = 0; v < 4; ++v) {
          const std::size_t row = 16 * mt + lane % 16, col = 16 * T + lane / 16 + 4 * v;
          if (row < M) p[((mt * KT + T) * 64 + lane) * 4 + v] = w[row * K + col];
        }
  return p;
}


Evaluator::Evaluator(std::shared_ptr<Model> model, int device) : model_(std::move(model)), device_(device) {
  int count = 0;
  HIP_CHECK(hipGetDeviceCount(&count));
  if (device < 0 || device >= count) throw DeviceError("SO3LR: HIP device index out of range");
  HIP_CHECK(hipSetDevice(device));
  HIP_CHECK(hipStreamCreateWithFlags(&own_stream_, hipStreamNonBlocking));
  if (const char *nv = std::getenv("SO3LR_NAIVE_FILTERS")) naive_filters_ = nv[0] == '1';
  if (const char *sp = std::getenv("SO3LR_SCALAR_FILTER_PAIRS")) scalar_pairs_max_ = std::atoll(sp);
  // SO3LR_NO_GRAPH=1: always launch the kernels one by one (no graph replay)
  if (const char *ng = std::getenv("SO3LR_NO_GRAPH")) use_graphs_ = ng[0] != '1';
  if (const char *nc = std::getenv("SO3LR_NO_CLASS_TABLES")) class_tables_ = nc[0] != '1';
  // SO3LR_NO_RADIAL_TABLES=1: block 0 on the element-pair MFMA kernels
  if (const char *nr = std::getenv("SO3LR_NO_RADIAL_TABLES")) radial_tables_ = nr[0] != '1';
  HIP_CHECK(hipHostMalloc(reinterpret_cast<void **>(&host_out_), 16 * sizeof(double), hipHostMallocDefault));
  scratch_dev_ = scratch_on_device(device);
  stream_ = own_stream_;
  const Model &m = *model_;
  const Architecture &a = m.arch();
  layers_ = a.layers;
  gamma_ = a.gamma;
  rc_ = a.sr_cutoff;
  avg_ = a.attention_norm;
  ln_eps_ = a.ln_eps;
  norm1_ = int(a.norm1);
  norm2_ = int(a.norm2);
  qk_norm_ = a.qk_norm;
  c6_ = a.c6_head;
  if (a.residual_scalars) {
    resid_ = m.f64("model.resid_lambdas", {std::size_t(a.layers)});
    x0l_ = m.f64("model.x0_lambdas", {std::size_t(a.layers)});
  }
  auto up = [&](const std::vector<double> &v) -> const double * {
    void *p = nullptr;
    HIP_CHECK(hipMalloc(&p, v.size() * sizeof(double)));
    HIP_CHECK(hipMemcpy(p, v.data(), v.size() * sizeof(double), hipMemcpyHostToDevice));
    weight_allocs_.push_back(p);
    bytes_ += std::int64_t(v.size() * sizeof(double));
    return static_cast<const double *>(p);
  };
  // models of other widths than v1's run on the generic kernels, which hold
  // their own weights; the fused v1 kernels' weights are laid out below
  if (a.generic) gen_ = std::make_unique<GenericPath>(m, up, radial_tables_ && class_tables_);
  F_ = a.F;
  const std::size_t F = kF, R = kR, FH = kFH, NI = kNI, HW = kHW;
  for (int b = 0; b < (a.generic ? 0 : layers_); ++b) {
    const std::string p = "model.euclidean_transformers." + std::to_string(b) + ".";
    const std::string at = p + "euclidean_attention_block.";
    BlockWeights &B = bw_[b];
    std::vector<double> qkv;
    for (const char *nm : {"W_q_inv", "W_k_inv", "W_v_inv", "W_q_ev", "W_k_ev"}) {
      const auto w = m.f64(at + nm, {4, HW, HW});
      qkv.insert(qkv.end(), w.begin(), w.end());
    }
    B.wqkv = up(qkv);
    {
      std::vector<double> fwdp, bwdp;
      for (int h = 0; h < 4; ++h) {
        std::vector<double> Mh(160 * HW);  // [w*32 + o][k] = W[w][h][k][o]
        for (int w = 0; w < 5; ++w)
          for (std::size_t k = 0; k < HW; ++k)
            for (std::size_t o = 0; o < HW; ++o)
              Mh[(w * HW + o) * HW + k] = qkv[((std::size_t(w) * 4 + h) * HW + k) * HW + o];
        const auto pf = permute_mfma(Mh, 160, HW);
        const auto pb = permute_mfma(transpose(Mh, 160, HW), HW, 160);
        fwdp.insert(fwdp.end(), pf.begin(), pf.end());
        bwdp.insert(bwdp.end(), pb.begin(), pb.end());
      }
      B.qkvp = up(fwdp);
      B.qkvtp = up(bwdp);
    }
    for (int k = 0; k < 2; ++k) {
      // the reference evaluates the transformer-level filter nets
      // (kokkos_integrated_block0.cpp:507-512)
      const std::string f = p + (k == 0 ? "filter_net_inv." : "filter_net_ev.");
      B.fw0[k] = up(m.f64(f + "mlp_rbf.0.weight", {F, R}));
      B.fb0[k] = up(m.f64(f + "mlp_rbf.0.bias", {F}));
      const auto w1 = m.f64(f + "mlp_rbf.mlp_rbf_layer_1.0.weight", {F, F});
      B.fw1[k] = up(w1);
      B.fw1t[k] = up(transpose(w1, F, F));
      B.fb1[k] = up(m.f64(f + "mlp_rbf.mlp_rbf_layer_1.0.bias", {F}));
      B.fe0[k] = up(m.f64(f + "mlp_ev.0.weight", {FH, 4}));
      B.feb0[k] = up(m.f64(f + "mlp_ev.0.bias", {FH}));
      const auto e1 = m.f64(f + "mlp_ev.mlp_ev_layer_1.0.weight", {F, FH});
      B.fe1[k] = up(e1);
      B.fe1t[k] = up(transpose(e1, F, FH));
      B.feb1[k] = up(m.f64(f + "mlp_ev.mlp_ev_layer_1.0.bias", {F}));
      const auto w0 = m.f64(f + "mlp_rbf.0.weight", {F, R});
      const auto e0 = m.f64(f + "mlp_ev.0.weight", {FH, 4});
      B.w0p[k] = up(permute_mfma(w0, F, R));
      B.w1p[k] = up(permute_mfma(w1, F, F));
      B.e0p[k] = up(permute_mfma(e0, FH, 4));
      B.e1p[k] = up(permute_mfma(e1, F, FH));
      B.w1tp[k] = up(permute_mfma(transpose(w1, F, F), F, F));
      B.w0tp[k] = up(permute_mfma(transpose(w0, F, R), R, F));
      B.e1tp[k] = up(permute_mfma(transpose(e1, F, FH), FH, F));
      B.e0tp[k] = up(permute_mfma(transpose(e0, FH, 4), 4, FH));
      const auto b0 = m.f64(f + "mlp_rbf.0.bias", {F});
      const auto eb0 = m.f64(f + "mlp_ev.0.bias", {FH});
      auto ob1 = m.f64(f + "mlp_rbf.mlp_rbf_layer_1.0.bias", {F});
      const auto eb1 = m.f64(f + "mlp_ev.mlp_ev_layer_1.0.bias", {F});
      for (int c = 0; c < F; ++c) ob1[c] += eb1[c];  // both branches add into one output
      B.b0p[k] = up(bias_acc(b0, F));
      B.eb0p[k] = up(bias_acc(eb0, FH));
      B.ob1p[k] = up(bias_acc(ob1, F));
      // with ev = 0 (block 0) the spherical branch is E1 silu(e0) + e1 for
      // every pair: one more constant in the output bias
      std::vector<double> ob10(ob1);
      for (int c = 0; c < F; ++c) {
        double acc = 0.0;
        for (int jj = 0; jj < FH; ++jj) acc += e1[std::size_t(c) * FH + jj] * (eb0[jj] / (1.0 + std::exp(-eb0[jj])));
        ob10[c] += acc;
      }
      B.ob1p0[k] = up(bias_acc(ob10, F));
      B.ob10[k] = up(ob10);
      const auto e0p = permute_mfma(e0, FH, 4);  // two tiles, one value per lane each
      std::vector<double> e0pk(64 * 4, 0.0);
      for (int lane = 0; lane < 64; ++lane) {
        e0pk[lane * 4 + 0] = e0p[lane];
        e0pk[lane * 4 + 1] = e0p[64 + lane];
      }
      B.e0pk[k] = up(e0pk);
    }
    B.att_cg = up(m.f64(at + "so3_conv_invariants.cg_rep", {24}));
    B.int_cg = up(m.f64(p + "interaction_block.so3_conv_invariants.cg_rep", {24}));
    // an affine LayerNorm has parameters; RMSNorm and no normalisation run
    // the same kernels with w = 1, b = 0
    const std::vector<double> ones(F, 1.0), zeros(F, 0.0);
    const bool ln1 = a.norm1 == NormMode::Layer, ln2 = a.norm2 == NormMode::Layer;
    B.ln1w = up(ln1 ? m.f64(p + "layer_norm_inv_1.weight", {F}) : ones);
    B.ln1b = up(ln1 ? m.f64(p + "layer_norm_inv_1.bias", {F}) : zeros);
    B.ln2w = up(ln2 ? m.f64(p + "layer_norm_inv_2.weight", {F}) : ones);
    B.ln2b = up(ln2 ? m.f64(p + "layer_norm_inv_2.bias", {F}) : zeros);
    const auto m1 = m.f64(p + "mlp_1.1.weight", {F, F}), m2 = m.f64(p + "mlp_1.3.weight", {F, F});
    B.m1w = up(m1); B.m1t = up(transpose(m1, F, F));
    B.m2w = up(m2); B.m2t = up(transpose(m2, F, F));
    B.m1p = up(permute_mfma(m1, F, F)); B.m2p = up(permute_mfma(m2, F, F));
    B.m1tp = up(permute_mfma(transpose(m1, F, F), F, F)); B.m2tp = up(permute_mfma(transpose(m2, F, F), F, F));
    B.m1b = up(m.f64(p + "mlp_1.1.bias", {F}));
    B.m2b = up(m.f64(p + "mlp_1.3.bias", {F}));
    B.m1bp = up(bias_acc(m.f64(p + "mlp_1.1.bias", {F}), F));
    B.m2bp = up(bias_acc(m.f64(p + "mlp_1.3.bias", {F}), F));
    const auto iw = m.f64(p + "interaction_block.linear_layer.weight", {NI, NI});
    B.intw = up(iw); B.intt = up(transpose(iw, NI, NI));
    B.intp = up(permute_mfma(iw, NI, NI));
    B.inttp = up(permute_mfma(transpose(iw, NI, NI), NI, NI));
    B.intb = up(m.f64(p + "interaction_block.linear_layer.bias", {NI}));
    B.intbp = up(bias_acc(m.f64(p + "interaction_block.linear_layer.bias", {NI}), NI));
  }
  // block 0's radial hidden layers as piecewise polynomials (radial tables),
  // used when both filters fit to within 1e-14 (values) and 1e-13 (slopes)
  // of their largest magnitudes at the check points
  if (!a.generic && radial_tables_ && class_tables_) {
    const auto bb = m.f64("model.radial_embedding.radial_basis_fn.b", {R});
    std::vector<double> val, slope;
    bool ok = true;
    for (int k = 0; k < 2 && ok; ++k) {
      const std::string f = std::string("model.euclidean_transformers.0.") + (k ? "filter_net_ev." : "filter_net_inv.");
      try {
        const RadialFit fit = fit_radial_hidden(m.f64(f + "mlp_rbf.0.weight", {F, R}), m.f64(f + "mlp_rbf.0.bias", {F}),
                                                int(F), int(R), bb, gamma_, rc_, kRadialIntervals, kRadialDegree);
        ok = fit.value_error <= 1e-14 && fit.slope_error <= 1e-13;
        val.insert(val.end(), fit.value.begin(), fit.value.end());
        slope.insert(slope.end(), fit.slope.begin(), fit.slope.end());
        rad_dom_ = RadialDomain{fit.r0, fit.step, fit.scale, fit.intervals};
      } catch (const std::invalid_argument &) {
        ok = false;
      }
    }
    if (ok) {
      rad_val_ = up(val);
      rad_slope_ = up(slope);
      radial_ok_ = true;
    }
  }
  // the blocks after 0: each filter's whole radial branch W1 h(r) + ob1 as
  // piecewise polynomials (32 intervals of degree 31, the same bound), laid
  // out as MFMA operands: per interval and filter the coefficients (128 x 32
  // powers) and the slope coefficients transposed (32 x 128)
  if (!a.generic && radial_tables_ && layers_ > 1) {
    const auto bb = m.f64("model.radial_embedding.radial_basis_fn.b", {R});
    bool ok = true;
    std::vector<std::vector<double>> rows(layers_), drs(layers_);
    for (int b = 1; b < layers_ && ok; ++b) {
      std::vector<RadialFit> fits;
      for (int k = 0; k < 2 && ok; ++k) {
        const std::string f = "model.euclidean_transformers." + std::to_string(b) + "." +
                              (k ? "filter_net_ev." : "filter_net_inv.");
        const auto w1 = m.f64(f + "mlp_rbf.mlp_rbf_layer_1.0.weight", {F, F});
        auto ob1 = m.f64(f + "mlp_rbf.mlp_rbf_layer_1.0.bias", {F});
        const auto eb1 = m.f64(f + "mlp_ev.mlp_ev_layer_1.0.bias", {F});
        for (std::size_t c = 0; c < F; ++c) ob1[c] += eb1[c];
        try {
          fits.push_back(fit_radial_hidden(m.f64(f + "mlp_rbf.0.weight", {F, R}), m.f64(f + "mlp_rbf.0.bias", {F}),
                                           int(F), int(R), bb, gamma_, rc_, kBlockIntervals, kBlockDegree, &w1,
                                           &ob1, int(F)));
          ok = fits.back().value_error <= 1e-14 && fits.back().slope_error <= 1e-13;
        } catch (const std::invalid_argument &) {
          ok = false;
        }
      }
      if (!ok) break;
      const std::size_t n = kBlockPowers;
      for (int i = 0; i < kBlockIntervals; ++i)
        for (int k = 0; k < 2; ++k) {
          const RadialFit &ft = fits[std::size_t(k)];
          std::vector<double> cv(F * n), st(n * F);
          for (std::size_t c = 0; c < F; ++c)
            for (std::size_t kk = 0; kk < n; ++kk) {
              cv[c * n + kk] = ft.value[(std::size_t(i) * n + kk) * F + c];
              st[kk * F + c] = ft.slope[(std::size_t(i) * n + kk) * F + c];
            }
          const auto pr = permute_mfma(cv, F, n), pd = permute_mfma(st, n, F);
          rows[std::size_t(b)].insert(rows[std::size_t(b)].end(), pr.begin(), pr.end());
          drs[std::size_t(b)].insert(drs[std::size_t(b)].end(), pd.begin(), pd.end());
        }
      rbl_dom_ = RadialDomain{fits[0].r0, fits[0].step, fits[0].scale, fits[0].intervals};
    }
    if (ok) {
      for (int b = 1; b < layers_; ++b) {
        bw_[b].rrow = up(rows[std::size_t(b)]);
        bw_[b].rdr = up(drs[std::size_t(b)]);
      }
      radial_blocks_ = true;
    }
  }
  if (!a.generic) {
    const std::string e = "model.atomic_energy_output_block.", q = "model.partial_charges_output_block.",
                      h = "model.hirshfeld_output_block.";
    const std::string c6h = "model.c6_ratios_output_block.";
    const std::size_t HH = kHH;
    std::vector<double> w1 = m.f64(e + "layers.0.weight", {F, F});
    const auto qw1 = m.f64(q + "transform_inv_features.0.weight", {F, F});
    const auto hw1 = m.f64(h + "transform_features.0.weight", {HH, F});
    w1.insert(w1.end(), qw1.begin(), qw1.end());
    w1.insert(w1.end(), hw1.begin(), hw1.end());
    std::vector<double> b1 = m.f64(e + "layers.0.bias", {F});
    const auto qb1 = m.f64(q + "transform_inv_features.0.bias", {F});
    const auto hb1 = m.f64(h + "transform_features.0.bias", {HH});
    b1.insert(b1.end(), qb1.begin(), qb1.end());
    b1.insert(b1.end(), hb1.begin(), hb1.end());
    if (c6_) {  // the C6 head's first layer: 64 more hidden units at 320
      const auto cw1 = m.f64(c6h + "transform_features.0.weight", {HH, F});
      const auto cb1 = m.f64(c6h + "transform_features.0.bias", {HH});
      w1.insert(w1.end(), cw1.begin(), cw1.end());
      b1.insert(b1.end(), cb1.begin(), cb1.end());
    }
    const int HO = c6_ ? 384 : 320;
    hw_.ho = HO;
    hw_.w1 = up(w1);
    hw_.w1t = up(transpose(w1, HO, F));
    hw_.w1p = up(permute_mfma(w1, HO, F));
    hw_.w1tp = up(permute_mfma(transpose(w1, HO, F), F, HO));
    hw_.b1 = up(b1);
    hw_.b1p = up(bias_acc(b1, HO));
    hw_.ew2 = up(m.f64(e + "final_layer.weight", {1, F}));
    hw_.eb2 = m.f64(e + "final_layer.bias", {1})[0];
    hw_.escale = up(m.f64(e + "energy_scales.weight", {1, 118}));
    hw_.eshift = up(m.f64(e + "energy_shifts", {118}));
    hw_.qw2 = up(m.f64(q + "transform_inv_features.2.weight", {1, F}));
    hw_.qb2 = m.f64(q + "transform_inv_features.2.bias", {1})[0];
    hw_.qemb = up(m.f64(q + "atomic_embedding.weight", {100, 1}));
    // reverse of a ratio head's key layer seeded by the element's query:
    // u[z][i] = sum_j W2[j][i] q_emb[z][j] depends on the element only, and
    // the logit q_emb[z] . (W2 a + b2) = u[z] . a + q_emb[z] . b2, so the key
    // vector itself is never needed
    auto ratio_head = [&](const std::string &pre, const double *&kbwd, const double *&kc, const double *&vsh) {
      const auto w2 = m.f64(pre + "transform_features.2.weight", {HH, HH});
      const auto qe = m.f64(pre + "q_embedding.weight", {100, HH});
      const auto b2 = m.f64(pre + "transform_features.2.bias", {HH});
      std::vector<double> u(100 * HH, 0.0), c(100, 0.0);
      for (std::size_t zz = 0; zz < 100; ++zz) {
        for (std::size_t i = 0; i < HH; ++i) {
          double acc = 0.0;
          for (std::size_t j = 0; j < HH; ++j) acc += w2[j * HH + i] * qe[zz * HH + j];
          u[zz * HH + i] = acc;
        }
        for (std::size_t j = 0; j < HH; ++j) c[zz] += qe[zz * HH + j] * b2[j];
      }
      kbwd = up(u);
      kc = up(c);
      vsh = up(m.f64(pre + "v_shift_embedding.weight", {100, 1}));
      return qe;
    };
    hw_.hqemb = up(ratio_head(h, hw_.hkey_bwd, hw_.hkey_c, hw_.hvshift));
    hw_.ckey_bwd = hw_.ckey_c = hw_.cvshift = nullptr;
    if (c6_) ratio_head(c6h, hw_.ckey_bwd, hw_.ckey_c, hw_.cvshift);
    const auto bb = m.f64("model.radial_embedding.radial_basis_fn.b", {R});
    const auto kk = m.i64("model.radial_embedding.radial_basis_fn.k", {R});
    const auto kr = m.i64("model.radial_embedding.radial_basis_fn.k_rev", {R});
    hw_.rbf_b = up(bb);
    hw_.rbf_k = up(std::vector<double>(kk.begin(), kk.end()));
    hw_.rbf_kr = up(std::vector<double>(kr.begin(), kr.end()));
    {
      std::vector<double> e(R);
      for (std::size_t c = 0; c < R; ++c)
        e[c] = double(std::exp(static_cast<long double>(bb[c]) - (c >= 4 ? static_cast<long double>(bb[c - 4]) : 0.0L)));
      hw_.rbf_e = up(e);
    }
    {
      std::vector<double> t(256);
      for (int j = 0; j < 256; ++j) t[j] = double(std::exp2(static_cast<long double>(j) / 256.0L));
      hw_.exp2_256 = up(t);
    }
  }
  {
    const auto &al = m.tensor("physical.reference_alphas");
    if (al.shape.size() != 1 || al.shape[0] < 8) throw std::runtime_error("SO3LR physical reference-table contract changed");
    hw_.n_ref = int(al.shape[0]);
    hw_.alpha_ref = up(m.f64("physical.reference_alphas", al.shape));
    hw_.c6_ref = up(m.f64("physical.reference_c6", al.shape));
  }
  emb_w_ = m.f64("model.inv_feature_embedding.embedding.weight", {std::size_t(F_), 118});
  charge_spin_.load(m);
  zbl_.ke = a.zbl_ke; zbl_.rc = a.sr_cutoff; zbl_.switch_off = a.zbl_switch_off;
  zbl_.p = a.zbl_p; zbl_.d = a.zbl_d;
  for (int k = 0; k < 4; ++k) { zbl_.a[k] = a.zbl_a[k]; zbl_.c[k] = a.zbl_c[k]; }
  zbl_.nlh_a = zbl_.nlh_b = nullptr;
  zbl_.nlh_cap = 0;
  if (a.nlh) {
    const auto &ta = m.tensor("physical.nlh_a");
    zbl_.nlh_a = up(m.f64("physical.nlh_a", ta.shape));
    zbl_.nlh_b = up(m.f64("physical.nlh_b", ta.shape));
    zbl_.nlh_cap = int(ta.shape[0]);
  }
  lr_.ke = a.lr_ke; lr_.sigma = a.lr_sigma; lr_.cutoff = a.lr_cutoff; lr_.cuton_el = a.lr_cuton_el;
  lr_.fine_factor = std::pow(a.lr_fine, -4.0 / 21.0);
  lr_.bohr = a.lr_bohr; lr_.hartree = a.lr_hartree; lr_.disp_scale = a.lr_disp_scale;
  lr_.cuton_disp = a.lr_cuton_disp; lr_.full_scale = 2.0 * a.lr_pair_scale;
  {
    const double cr = lr_.cutoff / lr_.sigma;
    const double cerf = std::erf(cr), cexp = std::exp(-cr * cr);
    lr_.shift = cerf / lr_.cutoff;
    lr_.fshift = (2.0 * lr_.cutoff * cexp * 0.56418958354775628695 / lr_.sigma - cerf) / (lr_.cutoff * lr_.cutoff);
  }
  lr_.n_ref = hw_.n_ref;
  lr_.inv_sigma = 1.0 / lr_.sigma;
  lr_.inv_bohr = 1.0 / lr_.bohr;
  lr_.two_over_sqrtpi_sigma = 2.0 * 0.56418958354775628695 / lr_.sigma;
  lr_.inv_w_el = 1.0 / (lr_.cutoff - lr_.cuton_el);
  lr_.inv_w_disp = 1.0 / (lr_.cutoff - lr_.cuton_disp);

  z_ = buf("z"); x0_ = buf("x0"); img_of_node_ = buf("img"); img_off_ = buf("img_off"); img_q_ = buf("img_q");
  xs_ = buf("xs"); evs_ = buf("evs"); qkv_ = buf("qkv"); aev_ = buf("aev"); n1_ = buf("n1");
  n1hat_ = buf("n1hat"); n1is_ = buf("n1is"); hpre_ = buf("hpre"); tout_ = buf("tout");
  pre2hat_ = buf("pre2hat"); pre2is_ = buf("pre2is"); ainv_ = buf("ainv"); act_ = buf("act");
  hhead_ = buf("hhead");
  heff_ = buf("heff"); eatom_ = buf("eatom"); qraw_ = buf("qraw"); q_ = buf("q"); hir_ = buf("hir");
  qseed_ = buf("qseed"); elr_ = buf("elr"); dq_ = buf("dq"); dh_ = buf("dh"); flr_ = buf("flr");
  vlr_ = buf("vlr"); elr_parts_ = buf("elr_parts"); ezbl_ = buf("ezbl"); gx_ = buf("gx");
  gev_ = buf("gev"); gainv_ = buf("gainv"); gaev_ = buf("gaev"); gqkv_ = buf("gqkv");
  ghead_ = buf("ghead"); fout_ = buf("fout"); etot_ = buf("etot"); red_ = buf("red");
  qkis_ = buf("qkis"); c6eff_ = buf("c6eff"); c6r_ = buf("c6r"); dc_ = buf("dc");
  owner_ = buf("owner"); sr_rows_ = buf("sr_rows"); sr_nodes_ = buf("sr_nodes");
  sr_inc_off_ = buf("sr_inc_off"); sr_inc_ = buf("sr_inc"); lr_rows_ = buf("lr_rows");
  lr_nodes_ = buf("lr_nodes"); lr_inc_off_ = buf("lr_inc_off"); lr_inc_ = buf("lr_inc");
  lr_rec_ = buf("lr_rec");
  blk_count_ = buf("blk"); n_active_ = buf("nact"); cand2act_ = buf("c2a"); pa_ = buf("pa");
  psc_ = buf("psc"); pv_ = buf("pv"); pr_ = buf("pr"); pY_ = buf("pY"); pfc_ = buf("pfc"); pzbl_ = buf("pzbl");
  ps_ = buf("ps"); pf_ = buf("pf"); palpha_ = buf("palpha"); df_ = buf("df"); dfc_ = buf("dfc");
  ds_ = buf("ds"); dr_ = buf("dr"); dY_ = buf("dY"); pg_ = buf("pg"); xrows_ = buf("xrows");
  fhost_ = buf("fhost"); vatom_ = buf("vatom");
  nb_key_ = buf("nb_key"); nb_idx_ = buf("nb_idx"); nb_skey_ = buf("nb_skey"); nb_sidx_ = buf("nb_sidx");
  nb_cstart_ = buf("nb_cstart"); nb_tmp_ = buf("nb_tmp"); nb_srcnt_ = buf("nb_srcnt"); nb_lrcnt_ = buf("nb_lrcnt");
  nb_err_ = buf("nb_err"); nb_srlist_ = buf("nb_srlist"); nb_poff_ = buf("nb_poff"); sr_code_ = buf("sr_code");
  nb_tot_ = buf("nb_tot");
  perm_ = buf("perm"); nz_ = buf("nz"); nx0_ = buf("nx0"); xn_ = buf("xn");
  cls_lut_ = buf("cls_lut"); cls_rep0_ = buf("cls_rep0"); cls_rep_ = buf("cls_rep"); cls_mt_ = buf("cls_mt");
  cls_c0_ = buf("cls_c0"); cls_gv_ = buf("cls_gv"); cls_hist_ = buf("cls_hist"); cls_order_ = buf("cls_order");
  cls_rows_ = buf("cls_rows"); rad_tab_ = buf("rad_tab"); rint_order_ = buf("rint_order"); rint_hist_ = buf("rint_hist");
  iact_ = buf("iact"); iother_ = buf("iother"); red_part_ = buf("red_part"); probe_ = buf("probe");
  top_owner_ = buf("top_owner"); top_stat_ = buf("top_stat"); top_slots_ = buf("top_slots");
  top_skeys_ = buf("top_skeys"); top_tmp_ = buf("top_tmp"); top_box_ = buf("top_box");
  for (int w = 0; w < 2; ++w) {
    top_ilist_[w] = buf("top_ilist"); top_off_[w] = buf("top_off"); top_neigh_[w] = buf("top_neigh");
    top_cnt_[w] = buf("top_cnt"); top_poff_[w] = buf("top_poff");
  }
  if (gen_)
    for (int i = 0; i < GenericPath::kBuffers; ++i) gbuf_[i] = buf("generic");
}

void Evaluator::set_box(const double lo[3], const double hi[3]) {
  if (!shift_mode_) throw std::logic_error("SO3LR: the box is set by the device reneighbor path only");
  for (int d = 0; d < 3; ++d) {
    const double l = hi[d] - lo[d];
    if (!(l > 2.0 * lr_.cutoff)) throw std::invalid_argument("SO3LR: box shorter than twice the long-range cutoff");
    box_len_[d] = l;
  }
}

void Evaluator::set_system(const std::vector<std::int32_t> &z, const std::vector<std::int64_t> &image_offsets,
                           const std::vector<double> &charges, const std::vector<double> &multiplicities) {
  const std::int64_t n = std::int64_t(z.size());
  if (n <= 0) throw std::invalid_argument("SO3LR: the system has no atoms");
  for (auto zz : z)
    if (zz < 1 || zz > 99) throw std::invalid_argument("SO3LR: atomic numbers must lie in 1..99");
  const std::int64_t ni = std::int64_t(charges.size());
  if (ni < 1 || std::int64_t(multiplicities.size()) != ni || std::int64_t(image_offsets.size()) != ni + 1 ||
      image_offsets.front() != 0 || image_offsets.back() != n)
    throw std::invalid_argument("SO3LR: inconsistent image description");
  // every offset is used as an index below: 0 = off[0] < off[1] < ... < off[ni] = n
  for (std::int64_t k = 0; k < ni; ++k)
    if (!(image_offsets[k + 1] > image_offsets[k]))
      throw std::invalid_argument("SO3LR: image offsets must increase strictly from 0 to the atom count "
                                  "(every image needs at least one atom)");
  const int F = F_;
  std::vector<double> x0(std::size_t(n) * F);
  std::vector<int> img(n);
  for (std::int64_t k = 0; k < ni; ++k) {
    const std::int64_t lo = image_offsets[k], hi = image_offsets[k + 1];
    std::int64_t counts[119] = {0};
    for (std::int64_t i = lo; i < hi; ++i) ++counts[z[i]];
    const std::string why = charge_multiplicity_problem(counts, charges[k], multiplicities[k]);
    if (!why.empty())
      throw std::domain_error("charge " + std::to_string(charges[k]) + " with multiplicity " +
                              std::to_string(multiplicities[k]) + ": " + why);
    const std::vector<double> tab = charge_spin_.table(counts, charges[k], multiplicities[k] - 1.0);
    const double inv = 1.0 / model_->arch().embedding_scale;
    for (std::int64_t i = lo; i < hi; ++i) {
      img[i] = int(k);
      for (int c = 0; c < F; ++c)
        x0[std::size_t(i) * F + c] = (emb_w_[c * 118 + (z[i] - 1)] + tab[(z[i] - 1) * F + c]) * inv;
    }
  }
  n_ = n;
  n_images_ = ni;
  image_offsets_ = image_offsets;
  HIP_CHECK(hipMemcpyAsync(ensure<int>(z_, n), z.data(), n * sizeof(int), hipMemcpyHostToDevice, stream_));
  HIP_CHECK(hipMemcpyAsync(ensure<double>(x0_, x0.size()), x0.data(), x0.size() * sizeof(double),
                           hipMemcpyHostToDevice, stream_));
  HIP_CHECK(hipMemcpyAsync(ensure<std::int64_t>(img_off_, ni + 1), image_offsets.data(),
                           (ni + 1) * sizeof(std::int64_t), hipMemcpyHostToDevice, stream_));
  HIP_CHECK(hipMemcpyAsync(ensure<double>(img_q_, ni), charges.data(), ni * sizeof(double),
                           hipMemcpyHostToDevice, stream_));
  // block 0's element classes: with one image x0 depends on z alone
  n_cls_ = 0;
  std::vector<int> lut(128, 0), rep0;
  if (ni == 1) {
    std::vector<int> seen(128, -1);
    for (std::int64_t i = 0; i < n; ++i)
      if (seen[z[i]] < 0) {
        seen[z[i]] = int(rep0.size());
        rep0.push_back(int(i));
      }
    if (int(rep0.size()) <= kMaxClasses) {
      for (int zz = 0; zz < 128; ++zz) lut[zz] = std::max(seen[zz], 0);
      rep0.resize(kMaxClasses, 0);
      HIP_CHECK(hipMemcpyAsync(ensure<int>(cls_lut_, 128), lut.data(), 128 * sizeof(int), hipMemcpyHostToDevice,
                               stream_));
      HIP_CHECK(hipMemcpyAsync(ensure<int>(cls_rep0_, kMaxClasses), rep0.data(), kMaxClasses * sizeof(int),
                               hipMemcpyHostToDevice, stream_));
      n_cls_ = int(std::count_if(seen.begin(), seen.end(), [](int c) { return c >= 0; }));
    }
  }
  // block 0's radial tables: sized here (no allocation in the evaluation),
  // filled by the next evaluation
  rad_stale_ = true;
  const std::size_t rad_rec = gen_ ? (gen_->radial_ok() ? gen_->radial_record() : 0) : (radial_ok_ ? kRadRecord : 0);
  if (rad_rec && n_cls_ > 0)
    (void)ensure<double>(rad_tab_, 2 * std::size_t(n_cls_) * (n_cls_ + 1) / 2 * kRadialIntervals * rad_rec);
  HIP_CHECK(hipStreamSynchronize(stream_));
  system_ready_ = true;
  topology_ready_ = false;
  ++topo_version_;
  evaluated_ = false;
}

double *Evaluator::pinned(Pinned &b, std::size_t count) {
  if (b.count < count) {
    if (b.p) HIP_CHECK(hipHostFree(b.p));
    b.p = nullptr;
    b.count = 0;
    const std::size_t cap = count + count / 8;
    HIP_CHECK(hipHostMalloc(reinterpret_cast<void **>(&b.p), cap * sizeof(double), hipHostMallocDefault));
    b.count = cap;
  }
  return b.p;
}

void Evaluator::compute_host(const double *x_rows, int flags, double *f, double *eatom, double *energy,
                             double *virial) {
  if (!topology_ready_) throw std::logic_error("SO3LR: compute called before set_topology");
  if (shift_mode_)
    throw std::logic_error("SO3LR: the topology came from so3lr_reneighbor_device; call so3lr_compute_device "
                           "with owned positions");
  const std::size_t nx = std::size_t(n_rows_) * 3, n = std::size_t(n_);
  double *xd = ensure<double>(xrows_, nx);
  double *fd = ensure<double>(fhost_, n * 4);
  double *px = pinned(pin_x_, nx), *pf = pinned(pin_f_, n * 4);
  // positions in: copied into pinned memory slice by slice, each slice's DMA
  // running while the next slice is copied (the stream is idle here: every
  // evaluation ends waiting for it)
  constexpr std::size_t kSlice = std::size_t(1) << 16;  // doubles, 512 KiB
  for (std::size_t a = 0; a < nx; a += kSlice) {
    const std::size_t c = std::min(kSlice, nx - a);
    std::memcpy(px + a, x_rows + a, c * sizeof(double));
    HIP_CHECK(hipMemcpyAsync(xd + a, px + a, c * sizeof(double), hipMemcpyHostToDevice, stream_));
  }
  // forces (and per-atom energies, which follow them in fd) out: one copy to
  // pinned memory, enqueued by the evaluation ahead of its one wait
  struct StageReset {
    Evaluator *e;
    ~StageReset() { e->stage_count_ = 0; }
  } stage_reset{this};
  stage_src_ = fd;
  stage_dst_ = pf;
  stage_count_ = n * ((flags & 2) ? 4 : 3);
  compute_device(xd, flags, fd, (flags & 2) ? fd + 3 * n_ : nullptr, energy, virial);
  if (f) std::memcpy(f, pf, n * 3 * sizeof(double));
  if (eatom && (flags & 2)) std::memcpy(eatom, pf + 3 * n, n * sizeof(double));
}

namespace {
FilterMfma filter_mfma(const BlockWeights &B, const HeadWeights &H, double gamma) {
  FilterMfma FM;
  for (int k = 0; k < 2; ++k) {
    FM.w0p[k] = B.w0p[k]; FM.w1p[k] = B.w1p[k]; FM.e1p[k] = B.e1p[k];
    FM.w1tp[k] = B.w1tp[k]; FM.w0tp[k] = B.w0tp[k]; FM.e1tp[k] = B.e1tp[k]; FM.e0tp[k] = B.e0tp[k];
    FM.b0p[k] = B.b0p[k]; FM.eb0p[k] = B.eb0p[k]; FM.ob1p[k] = B.ob1p[k]; FM.e0pk[k] = B.e0pk[k];
    FM.ob1p0[k] = B.ob1p0[k];
  }
  FM.att_cg = B.att_cg; FM.rbf_b = H.rbf_b; FM.rbf_k = H.rbf_k; FM.rbf_kr = H.rbf_kr; FM.gamma = gamma;
  FM.rbf_e = H.rbf_e;
  FM.exp2_256 = H.exp2_256;
  return FM;
}
}  // namespace

void Evaluator::compute_device(const double *x, int flags, double *f_out, double *eatom_out, double *energy,
                               double *virial) {
  compute_impl(x, flags, f_out, eatom_out, energy, virial, false);
}

void Evaluator::compute_device_noalloc(const double *x, int flags, double *f_out, double *eatom_out,
                                       double *energy, double *virial) {
  compute_impl(x, flags, f_out, eatom_out, energy, virial, true);
}

std::size_t Evaluator::scratch_capacity() { return kScratchBytes; }

void Evaluator::compute_impl(const double *x, int flags, double *f_out, double *eatom_out, double *energy,
                             double *virial, bool from_scratch) {
  if (!topology_ready_) throw std::logic_error("SO3LR: compute called before set_topology");
  const std::int64_t N = n_, P = p_sr_, L = layers_;
  const std::size_t Nz = std::size_t(N), Pz = std::size_t(std::max<std::int64_t>(P, 1));
  hipStream_t s = stream_;
  const double rc2 = rc_ * rc_;
  const int nblk = std::max(1, ceil_div(P, kCompactPerBlock));
  // --- node-order inputs: the spatial order of the device reneighbor path
  // (positions gathered into node order as well), or of a LAMMPS-list
  // topology, set at its first evaluation (positions stay in row order) ---
  if (rows_order_pending_ && !shift_mode_) order_rows_nodes(x);
  const int *perm = permuted_ ? static_cast<const int *>(perm_->p) : nullptr;
  const int *z = static_cast<const int *>((permuted_ ? nz_ : z_)->p);
  const double *x0 = static_cast<const double *>((permuted_ ? nx0_ : x0_)->p);
  const double *x_in = x;
  const bool gather_pos = permuted_ && shift_mode_;
  if (gather_pos) x = static_cast<const double *>(xn_->p);
  // --- capacity of the active-pair buffers: the pairs inside the cutoff
  // (about 60% of the candidates with a 1 A skin), counted once per topology
  // and given 1/8 of margin; an evaluation that finds more grows it and runs
  // again (see the end of this function) ---
  if (act_cap_ == 0 && P > 0) {
    int *cnt = from_scratch ? reinterpret_cast<int *>(scratch_dev_) : ensure<int>(probe_, std::size_t(nblk) + 2);
    if (gather_pos)
      hipLaunchKernelGGL(k_gather_pos, dim3(unsigned((3 * Nz + 255) / 256)), dim3(256), 0, s, int(N), perm, x_in,
                         const_cast<double *>(x));
    if (shift_mode_) {
      const ShiftPos pos{x, static_cast<const int *>(sr_nodes_->p), static_cast<const int *>(sr_code_->p),
                         box_len_[0], box_len_[1], box_len_[2]};
      hipLaunchKernelGGL(k_sr_count<ShiftPos>, dim3(nblk), dim3(256), 0, s, int(P), pos, rc2, cnt);
    } else {
      const RowsPos pos{x, static_cast<const int *>(sr_rows_->p)};
      hipLaunchKernelGGL(k_sr_count<RowsPos>, dim3(nblk), dim3(256), 0, s, int(P), pos, rc2, cnt);
    }
    hipLaunchKernelGGL(k_scan_counts, dim3(1), dim3(1024), 0, s, nblk, cnt, cnt + nblk, 0x7fffffff, cnt + nblk + 1);
    int total = 0;
    HIP_CHECK(hipMemcpyAsync(&total, cnt + nblk + 1, sizeof(int), hipMemcpyDeviceToHost, s));
    HIP_CHECK(hipStreamSynchronize(s));
    act_cap_ = std::min<std::int64_t>(P, std::int64_t(total) + total / 8 + 256);
    scalar_now_ = std::int64_t(total) <= scalar_pairs_max_;
  }
  if (P == 0) scalar_now_ = false;
  const bool scalar = naive_filters_ || scalar_now_;
  const std::int64_t PA = std::max<std::int64_t>(std::min(act_cap_, P), 1);
  const std::size_t Pa = std::size_t(PA);
  // --- buffers (retained capacity; all allocation happens before any work
  // is enqueued, so the sequence below can be captured into a graph) ---
  const std::size_t HO = std::size_t(hw_.ho);
  double *qkis = nullptr, *c6eff = nullptr, *c6r = nullptr, *dc = nullptr;
  double *xs = nullptr;
  double *evs = nullptr;
  double *qkv = nullptr;
  double *aev = nullptr;
  double *n1 = nullptr;
  double *n1hat = nullptr;
  double *n1is = nullptr;
  double *hpre = nullptr;
  double *tout = nullptr;
  double *pre2hat = nullptr;
  double *pre2is = nullptr;
  double *ainv = nullptr;
  double *act = nullptr;
  double *hhead = nullptr;
  double *heff = nullptr;
  double *eatom = nullptr;
  double *qraw = nullptr;
  double *q = nullptr;
  double *hir = nullptr;
  double *qseed = nullptr;
  double *elr = nullptr;
  double *dq = nullptr;
  double *dh = nullptr;
  double *flr = nullptr;
  double *vlr = nullptr;
  double *parts = nullptr;
  double *ezbl = nullptr;
  double *gx = nullptr;
  double *gev = nullptr;
  double *gainv = nullptr;
  double *gaev = nullptr;
  double *gqkv = nullptr;
  double *ghead = nullptr;
  double *fo = nullptr;
  double *etot = nullptr;
  double *red = nullptr;
  int *blk = nullptr;
  int *nact = nullptr;
  int *c2a = nullptr;
  int *pa = nullptr;
  double *pv = nullptr;
  double *pr = nullptr;
  double *pY = nullptr;
  double *pfc = nullptr;
  double *pzbl = nullptr;
  double *ps = nullptr;
  double *pf = nullptr;
  double *palpha = nullptr;
  double *df = nullptr;
  double *dfc = nullptr;
  double *psc = nullptr;
  double *ds = nullptr;
  double *dr = nullptr;
  double *dY = nullptr;
  double *pg = nullptr;
  int *iact = nullptr, *iother = nullptr;
  double *partial = nullptr;
  // block 0 through element-pair tables (k_filter_fwd_class, k_filter_bwd_class)
  const bool use_cls = !gen_ && !scalar && class_tables_ && n_cls_ > 0;
  // and with the radial tables (k_radial_fwd, k_radial_bwd)
  const bool use_rad = use_cls && radial_ok_;
  // the blocks after 0 on their radial tables (k_radial_fwd_rows,
  // k_filter_bwd_mfma<false, false, true>)
  const bool use_rt = !gen_ && !scalar && radial_blocks_ && L > 1;
  // and the generic path's (g_radial_fwd_rows)
  const bool use_grt = gen_ && gen_->radial_blocks_ok() && L > 1;
  int *rord = nullptr, *rhist = nullptr;
  // buckets of the blocks after 0: (spatial block of kRintAtoms nodes, interval)
  const int rkeys = int(ceil_div(N, kRintAtoms)) * kBlockIntervals;
  // (the generic path's: g_cls_tables, g_b0_fwd, g_b0_bwd)
  const bool gen_cls = gen_ && class_tables_ && n_cls_ > 0;
  const int C = use_cls ? n_cls_ : 0;
  int *crep = nullptr, *chist = nullptr, *ccur = nullptr, *cord = nullptr;
  double *cmt = nullptr, *cc0 = nullptr, *cgv = nullptr, *cxr = nullptr, *cqkv = nullptr, *cqis = nullptr;
  auto carve_all = [&] {
    if (!gen_) {
    xs = take<double>(xs_, (L + 1) * Nz * kF);
    evs = take<double>(evs_, (L + 1) * Nz * kE);
    qkv = take<double>(qkv_, L * Nz * 640);
    aev = take<double>(aev_, L * Nz * kE);
    n1 = take<double>(n1_, L * Nz * kF);
    n1hat = take<double>(n1hat_, L * Nz * kF);
    n1is = take<double>(n1is_, L * Nz);
    hpre = take<double>(hpre_, L * Nz * kF);
    tout = take<double>(tout_, L * Nz * kNI);
    pre2hat = take<double>(pre2hat_, L * Nz * kF);
    pre2is = take<double>(pre2is_, L * Nz);
    ainv = take<double>(ainv_, Nz * kF);
    act = take<double>(act_, Nz * HO); // MLP input (128 wide) and head activations (HO)
    hhead = take<double>(hhead_, Nz * HO);
    gx = take<double>(gx_, Nz * kF);
    gev = take<double>(gev_, Nz * kE);
    gainv = take<double>(gainv_, Nz * kF);
    gaev = take<double>(gaev_, Nz * kE);
    gqkv = take<double>(gqkv_, Nz * 640);
    ghead = take<double>(ghead_, Nz * HO);
    qkis = qk_norm_ ? take<double>(qkis_, L * Nz * 16) : nullptr;
    ps = take<double>(ps_, L * 4 * Pa);
    // filter rows of every block for the scalar cross-check path; of blocks
    // after 0 only on the MFMA path (block 0's are never read there)
    pf = take<double>(pf_, std::size_t(scalar ? L : L - 1) * 256 * Pa);
    palpha = take<double>(palpha_, L * 16 * Pa);
    // the pair adjoints of the filters stay in registers on the MFMA path;
    // it passes the head scalars (16 per pair) and dE/dfc between its kernels
    df = scalar ? take<double>(df_, 256 * Pa) : nullptr;
    dfc = take<double>(dfc_, Pa);
    psc = scalar ? nullptr : take<double>(psc_, 16 * Pa);
    ds = take<double>(ds_, 4 * Pa);
    if (use_rt) {
      // counts, bucket cursors and the slots' end; the bucket order
      rhist = take<int>(rint_hist_, 2 * std::size_t(rkeys) + 1);
      rord = take<int>(rint_order_, Pa + 16 * std::size_t(rkeys));
    }
    if (use_cls) {
      crep = take<int>(cls_rep_, kMaxClasses);
      chist = take<int>(cls_hist_, 2 * kMaxClasses * kMaxClasses);  // counts, then bucket cursors
      ccur = chist + kMaxClasses * kMaxClasses;
      cord = take<int>(cls_order_, Pa);
      // the classes' block-0 input rows, q k v rows and QK-norm factors
      cxr = take<double>(cls_rows_, kMaxClasses * std::size_t(kF + 640 + 16));
      cqkv = cxr + kMaxClasses * kF;
      cqis = cqkv + kMaxClasses * 640;
      cmt = take<double>(cls_mt_, 2 * std::size_t(C) * C * 4 * kF);
      cc0 = take<double>(cls_c0_, 2 * std::size_t(C) * C * 4);
      cgv = take<double>(cls_gv_, Nz * C * 4);
    }
    } else {
      gen_->carve(int(N), int(PA), gen_cls ? n_cls_ : 0,
                  [&](int i, std::size_t cnt) { return take<double>(gbuf_[i], cnt); });
      if (use_grt) {
        rhist = take<int>(rint_hist_, 2 * std::size_t(rkeys) + 1);
        rord = take<int>(rint_order_, Pa + 16 * std::size_t(rkeys));
      }
      if (gen_cls) {
        crep = take<int>(cls_rep_, kMaxClasses);
        // class-pair counts and cursors, then the slot count; the pairs in
        // element-pair order, each bucket padded with -1
        chist = take<int>(cls_hist_, 2 * kMaxClasses * kMaxClasses + 1);
        ccur = chist + kMaxClasses * kMaxClasses;
        cord = take<int>(cls_order_, Pa + std::size_t(GContext::kB0Pad) * n_cls_ * n_cls_);
      }
    }
    heff = take<double>(heff_, Nz);
    eatom = take<double>(eatom_, Nz);
    qraw = take<double>(qraw_, Nz);
    q = take<double>(q_, Nz);
    hir = take<double>(hir_, Nz);
    qseed = take<double>(qseed_, Nz);
    elr = take<double>(elr_, Nz);
    dq = take<double>(dq_, Nz);
    dh = take<double>(dh_, Nz);
    flr = take<double>(flr_, Nz * 3);
    vlr = take<double>(vlr_, Nz * 6);
    parts = take<double>(elr_parts_, Nz * 2);
    ezbl = take<double>(ezbl_, Nz);
    c6eff = c6_ ? take<double>(c6eff_, Nz) : nullptr;
    c6r = c6_ ? take<double>(c6r_, Nz) : nullptr;
    dc = c6_ ? take<double>(dc_, Nz) : nullptr;
    fo = f_out ? f_out : take<double>(fout_, Nz * 3);
    etot = eatom_out ? eatom_out : take<double>(etot_, Nz);
    red = take<double>(red_, 16);
    blk = take<int>(blk_count_, nblk);
    nact = take<int>(n_active_, 2);  // [0] active pairs kept, [1] active pairs found
    c2a = take<int>(cand2act_, Pz);
    // per active pair (the candidate-indexed map c2a and the incidence stay
    // sized by candidates)
    pa = take<int>(pa_, 2 * Pa);
    pv = take<double>(pv_, 3 * Pa);
    pr = take<double>(pr_, Pa);
    pY = take<double>(pY_, kE * Pa);
    pfc = take<double>(pfc_, Pa);
    pzbl = take<double>(pzbl_, 2 * Pa);
    dr = take<double>(dr_, Pa);
    dY = take<double>(dY_, kE * Pa);
    pg = take<double>(pg_, 3 * Pa);
    iact = take<int>(iact_, 2 * Pz);
    iother = take<int>(iother_, 2 * Pz);
    partial = take<double>(red_part_, 9 * kReduceBlocks);
  };
  struct CarveReset {  // the work-buffer source goes back to the retained buffers
    Evaluator *e;
    ~CarveReset() { e->carve_ = Carve::Retained; }
  } carve_reset{this};
  if (from_scratch) {
    carve_ = Carve::Measure;
    carve_used_ = 0;
    carve_all();
    if (carve_used_ > kScratchBytes)
      throw std::invalid_argument("SO3LR: this system needs " + std::to_string(carve_used_) +
                                  " bytes of work space; so3lr_compute_device_noalloc has " +
                                  std::to_string(kScratchBytes) + " (use so3lr_compute_device)");
    carve_ = Carve::Scratch;
    carve_base_ = scratch_dev_;
    carve_used_ = 0;
  }
  carve_all();
  double *hact = act;
  const int *sr_rows = static_cast<const int *>(sr_rows_->p);
  const int *sr_nodes = static_cast<const int *>(sr_nodes_->p);
  const int *sr_off = static_cast<const int *>(sr_inc_off_->p);
  const int *sr_inc = static_cast<const int *>(sr_inc_->p);
  // LAMMPS-list long range: per incidence entry the partner node, own row and
  // partner row (lr_rec_, three arrays of lr_rec_len_ entries)
  const int *lr_rec = static_cast<const int *>(lr_rec_->p);
  const std::size_t lr_m = std::size_t(lr_rec_len_);
  const int *lr_off = static_cast<const int *>(lr_inc_off_->p);
  const int *lr_inc = static_cast<const int *>(lr_inc_->p);
  const std::int64_t *img_off = static_cast<const std::int64_t *>(img_off_->p);
  const double *img_q = static_cast<const double *>(img_q_->p);

  const int gN4 = ceil_div(N, 4);
  // per-launch HIP events for the measured kernels; units: 0 = active pairs, 1 = nodes
  struct Pending { const char *name; hipEvent_t a, b; int unit_kind; };
  std::vector<Pending> pending;
  auto timed = [&](const char *name, int unit_kind, auto &&launch) {
    if (!timing_ || from_scratch) { launch(); return; }  // events are created: not in the no-allocation call
    Pending pd{name, nullptr, nullptr, unit_kind};
    HIP_CHECK(hipEventCreate(&pd.a));
    HIP_CHECK(hipEventCreate(&pd.b));
    HIP_CHECK(hipEventRecord(pd.a, s));
    launch();
    HIP_CHECK(hipEventRecord(pd.b, s));
    pending.push_back(pd);
  };
  auto fill = [&](double *p, std::size_t cnt) {
    if (cnt) hipLaunchKernelGGL(k_fill, dim3(unsigned((cnt + 255) / 256)), dim3(256), 0, s, p, cnt, 0.0);
  };
  // node GEMM shapes (K, O) of the heads: 128->320 and its reverse 320->128;
  // output tiles per wavefront: MT / MG groups run as separate wavefronts
#ifndef SO3LR_MG8
#define SO3LR_MG8 4
#endif
  auto gemm = [&](int epi, int rows, int K, int O, const double *X, int ldx, const double *Wp, const double *bias,
                  double *out, int ldo, double *out2) {
    const dim3 grid(unsigned(ceil_div(rows, 64)));
#define SO3LR_GEMM(E, KT, MT, MG)                                                                             \
  if (epi == E && (K + 15) / 16 == KT && (O + 15) / 16 == MT) {                                              \
    hipLaunchKernelGGL((k_gemm<E, KT, MT, MG>), dim3(grid.x, MT / MG), dim3(256), 0, s, rows, K, O, X, ldx, Wp, \
                       bias, out, ldo, out2);                                                                 \
    return;                                                                                                   \
  }
    SO3LR_GEMM(0, 20, 8, SO3LR_MG8) SO3LR_GEMM(1, 8, 20, 4)
    SO3LR_GEMM(0, 24, 8, SO3LR_MG8) SO3LR_GEMM(1, 8, 24, 4)  // with the C6 head (384 hidden units)
#undef SO3LR_GEMM
    throw std::logic_error("SO3LR: internal error, no node GEMM for this shape");
  };
  const unsigned gN64 = unsigned(std::max(1, ceil_div(N, 64)));

  // Everything from here to the read-back is one sequence on stream s: run
  // directly, or captured once into a graph and replayed.
  auto enqueue = [&] {
  if (gather_pos)
    hipLaunchKernelGGL(k_gather_pos, dim3(unsigned((3 * Nz + 255) / 256)), dim3(256), 0, s, int(N), perm, x_in,
                       const_cast<double *>(x));
  // --- active short-range pairs, geometry, ZBL ---
  const int cap = int(PA);
  if (P > 0 && !shift_mode_) {
    const RowsPos pos{x, sr_rows};
    hipLaunchKernelGGL(k_sr_count<RowsPos>, dim3(nblk), dim3(256), 0, s, int(P), pos, rc2, blk);
    hipLaunchKernelGGL(k_scan_counts, dim3(1), dim3(1024), 0, s, nblk, blk, nact, cap, nact + 1);
    hipLaunchKernelGGL(k_sr_compact<RowsPos>, dim3(nblk), dim3(256), 0, s, int(P), pos, sr_nodes, rc2, blk, cap, z,
                       zbl_, c2a, pa, pv, pr, pY, pfc, pzbl);
  } else if (P > 0) {
    const ShiftPos pos{x, sr_nodes, static_cast<const int *>(sr_code_->p), box_len_[0], box_len_[1], box_len_[2]};
    hipLaunchKernelGGL(k_sr_count<ShiftPos>, dim3(nblk), dim3(256), 0, s, int(P), pos, rc2, blk);
    hipLaunchKernelGGL(k_scan_counts, dim3(1), dim3(1024), 0, s, nblk, blk, nact, cap, nact + 1);
    hipLaunchKernelGGL(k_sr_compact<ShiftPos>, dim3(nblk), dim3(256), 0, s, int(P), pos, sr_nodes, rc2, blk, cap, z,
                       zbl_, c2a, pa, pv, pr, pY, pfc, pzbl);
  } else {
    hipLaunchKernelGGL(k_fill_int, dim3(1), dim3(64), 0, s, nact, 2, 0);  // no memset nodes in graphs
  }
  // active incidence of this step (2 entries per candidate pair)
  if (P > 0)
    hipLaunchKernelGGL(k_inc_active, dim3(unsigned((2 * Pz + 255) / 256)), dim3(256), 0, s, int(2 * P), sr_inc, c2a,
                       pa, iact, iother);
  fill(dr, Pa);
  // erf(r / sigma) by the polynomial of erf_lean when r / sigma stays within [0, 3]
  const bool lean_erf = lr_.cutoff * lr_.inv_sigma <= 3.0;
  auto long_range = [&] { timed("long_range", 1, [&] {
#define SO3LR_LR(FULL, LEAN, SEP)                                                                                     \
  if (FULL)                                                                                                          \
    hipLaunchKernelGGL((k_lr<LrImages, LEAN, SEP>), dim3(gN4), dim3(256), 0, s, int(N), lr_off, lr_inc,              \
                       LrImages{x, nullptr}, box_len_[0], box_len_[1], box_len_[2], z, q, hir, c6r, lr_,             \
                       hw_.alpha_ref, hw_.c6_ref, elr, dq, dh, dc, flr, vlr, parts);                                 \
  else                                                                                                               \
    hipLaunchKernelGGL((k_lr<LrRows, LEAN, SEP>), dim3(gN4), dim3(256), 0, s, int(N), lr_off, lr_inc,                \
                       LrRows{lr_rec, lr_rec + lr_m, lr_rec + 2 * lr_m, x}, 0.0, 0.0, 0.0, z, q, hir, c6r, lr_,     \
                       hw_.alpha_ref, hw_.c6_ref,                                                                    \
                       elr, dq, dh, dc, flr, vlr, parts);
    if (c6_) {
      if (lean_erf) { SO3LR_LR(shift_mode_, true, true) } else { SO3LR_LR(shift_mode_, false, true) }
    } else {
      if (lean_erf) { SO3LR_LR(shift_mode_, true, false) } else { SO3LR_LR(shift_mode_, false, false) }
    }
#undef SO3LR_LR
  }); };
  if (gen_) {
    // generic widths: blocks and heads forward, the long range and the charge
    // seeds as below, then heads and blocks in reverse to dE/dY, dE/dr
    GContext G{s, int(N), int(PA), nact, pa, pr, pY, pfc, sr_off, iact, iother, z, x0, 1.0 / avg_, ln_eps_,
               gamma_, rc_, norm1_, norm2_, qk_norm_ ? 1 : 0, &resid_, &x0l_, eatom, qraw, heff, hir, c6eff, c6r,
               qseed, dh, dc, dY, dr, nullptr};
    if (timing_ && !from_scratch)
      G.timed = [&](const char *name, const std::function<void()> &f) { timed(name, 0, f); };
    if (gen_cls) {
      const int C = n_cls_;
      const int slots_max = int(Pa) + GContext::kB0Pad * C * C;
      int *cslots = ccur + kMaxClasses * kMaxClasses;
      G.cls_C = C;
      G.cls_lut = static_cast<const int *>(cls_lut_->p);
      G.cls_rep = crep;
      G.cls_order = cord;
      G.cls_slots = cslots;
      hipLaunchKernelGGL(k_class_reps, dim3(unsigned(ceil_div(std::max<std::int64_t>(N, C * C), 256))), dim3(256), 0, s,
                         int(N), z, G.cls_lut, perm, static_cast<const int *>(cls_rep0_->p), crep, C * C, chist);
      if (gen_->radial_ok()) {
        // block 0 through the radial tables (filled once after set_system), in pair order
        G.rad_tab = static_cast<double *>(rad_tab_->p);
        G.rad_build = rad_stale_;
        rad_stale_ = false;
      } else {
        // the element-pair kernels' slot order
        hipLaunchKernelGGL(k_fill_int, dim3(unsigned(ceil_div(slots_max, 256))), dim3(256), 0, s, cord, slots_max, -1);
        const dim3 gsort(unsigned(ceil_div(PA, kClsChunk)));
        hipLaunchKernelGGL(k_cls_count, gsort, dim3(256), 0, s, nact, pa, z, G.cls_lut, C, chist);
        hipLaunchKernelGGL(k_cls_scan, dim3(1), dim3(64), 0, s, C * C, chist, ccur, GContext::kB0Pad, cslots);
        hipLaunchKernelGGL(k_cls_place, gsort, dim3(256), 0, s, nact, pa, z, G.cls_lut, C, ccur, cord);
      }
    }
    if (use_grt) {
      // the blocks after 0 on their radial tables: the active pairs in bucket order
      const int slots_max = PA + 16 * rkeys;
      const RadialDomain &dom = gen_->rbl_domain();
      const dim3 gpair(unsigned(std::max(1, ceil_div(PA, 256))));
      hipLaunchKernelGGL(k_fill_int, dim3(unsigned(ceil_div(rkeys, 256))), dim3(256), 0, s, rhist, rkeys, 0);
      hipLaunchKernelGGL(k_fill_int, dim3(unsigned(ceil_div(slots_max, 256))), dim3(256), 0, s, rord, slots_max, -1);
      hipLaunchKernelGGL(k_rint_count, gpair, dim3(256), 0, s, nact, pa, pr, dom, rhist);
      hipLaunchKernelGGL(k_rint_scan, dim3(1), dim3(1024), 0, s, rkeys, rhist, rhist + rkeys, rhist + 2 * rkeys);
      hipLaunchKernelGGL(k_rint_place, gpair, dim3(256), 0, s, nact, pa, pr, dom, rhist + rkeys, rord);
      G.rint_order = rord;
      G.rint_slots = rhist + 2 * rkeys;
      G.rint_max = slots_max;
    }
    gen_->forward(G);
    hipLaunchKernelGGL(k_image_center, dim3(unsigned(n_images_)), dim3(1024), 0, s, img_off, img_q, qraw, q, 0);
    long_range();
    hipLaunchKernelGGL(k_image_center, dim3(unsigned(n_images_)), dim3(1024), 0, s, img_off, img_q, dq, qseed, 1);
    gen_->reverse(G);
  } else {
  HIP_CHECK(hipMemcpyAsync(xs, x0, Nz * kF * sizeof(double), hipMemcpyDeviceToDevice, s));
  const unsigned gNF = unsigned((Nz * kF + 255) / 256);
  // residual scalars: block b's input is resid[b] x + x0[b] x0, x the block
  // below's output (block 0: the embedding itself)
  if (!resid_.empty()) hipLaunchKernelGGL(k_axpby, dim3(gNF), dim3(256), 0, s, Nz * kF, resid_[0], xs, x0l_[0], x0);
  fill(evs, Nz * kE);
  const double inv_avg = 1.0 / avg_;
  const unsigned gP = unsigned(PA);
  const unsigned gP64 = unsigned(std::max(1, ceil_div(PA, 64)));  // 64 pairs per MFMA block
  const unsigned gP16 = unsigned(std::max(1, ceil_div(PA, 16)));  // 16 pairs per radial-table block
  // slots of the bucket order: every bucket padded by fewer than 16
  const int rslots_max = PA + 16 * rkeys;
  const unsigned gR = unsigned(ceil_div(rslots_max, 64));  // 16 slots per wavefront
  const int *rslots = rhist ? rhist + 2 * rkeys : nullptr;

  // --- interaction blocks, forward ---
  for (int b = 0; b < L; ++b) {
    const BlockWeights &B = bw_[b];
    double *xb = xs + b * Nz * kF, *evb = evs + b * Nz * kE;
    double *qb = qkv + b * Nz * 640, *aevb = aev + b * Nz * kE;
    double *n1b = n1 + b * Nz * kF, *n1hb = n1hat + b * Nz * kF, *n1ib = n1is + b * Nz;
    double *hpb = hpre + b * Nz * kF, *tb = tout + b * Nz * kNI;
    double *p2h = pre2hat + b * Nz * kF, *p2i = pre2is + b * Nz;
    double *psb = ps + b * 4 * Pa, *pab = palpha + b * 16 * Pa;
    double *pfb = scalar ? pf + b * 256 * Pa : (b > 0 ? pf + (b - 1) * 256 * Pa : nullptr);
    FilterArgs A;
    for (int k = 0; k < 2; ++k) {
      A.fw0[k] = B.fw0[k]; A.fb0[k] = B.fb0[k]; A.fw1t[k] = B.fw1t[k]; A.fb1[k] = B.fb1[k];
      A.fe0[k] = B.fe0[k]; A.feb0[k] = B.feb0[k]; A.fe1t[k] = B.fe1t[k]; A.feb1[k] = B.feb1[k];
    }
    A.att_cg = B.att_cg; A.rbf_b = hw_.rbf_b; A.rbf_k = hw_.rbf_k; A.rbf_kr = hw_.rbf_kr; A.gamma = gamma_;
    const FilterMfma FM = filter_mfma(B, hw_, gamma_);
    if (use_rt && b == 1) {
      // the active pairs in bucket order, for every block after 0 and the reverse
      const dim3 gpair(unsigned(std::max(1, ceil_div(PA, 256))));
      hipLaunchKernelGGL(k_fill_int, dim3(unsigned(ceil_div(rkeys, 256))), dim3(256), 0, s, rhist, rkeys, 0);
      hipLaunchKernelGGL(k_fill_int, dim3(unsigned(ceil_div(rslots_max, 256))), dim3(256), 0, s, rord, rslots_max, -1);
      hipLaunchKernelGGL(k_rint_count, gpair, dim3(256), 0, s, nact, pa, pr, rbl_dom_, rhist);
      hipLaunchKernelGGL(k_rint_scan, dim3(1), dim3(1024), 0, s, rkeys, rhist, rhist + rkeys, rhist + 2 * rkeys);
      hipLaunchKernelGGL(k_rint_place, gpair, dim3(256), 0, s, nact, pa, pr, rbl_dom_, rhist + rkeys, rord);
    }
    // the MFMA filter also forms the attention logits of both directions
    // from the filter tiles it holds; the scalar cross-check path leaves them
    // to the full attention kernel
    // block 0 runs cheaper instantiations (ev = 0): timed under their own names
    const bool blk0 = b == 0 && !scalar;
    if (blk0 && use_cls) {
      // block 0's q k v rows of the element classes only, the element-pair
      // tables from them, and the active pairs in element-pair order (used
      // again by the reverse)
      const int *lut = static_cast<const int *>(cls_lut_->p);
      hipLaunchKernelGGL(k_class_reps, dim3(unsigned(ceil_div(std::max<std::int64_t>(N, C * C), 256))), dim3(256), 0, s,
                         int(N), z, lut, perm, static_cast<const int *>(cls_rep0_->p), crep, C * C, chist);
      hipLaunchKernelGGL(k_class_rows, dim3(unsigned(ceil_div(C * kF, 256))), dim3(256), 0, s, C, crep, xb, cxr);
      hipLaunchKernelGGL(k_qkv_mfma, dim3(1, kHeads), dim3(256), 0, s, C, cxr, B.qkvp, cqkv);
      if (qk_norm_)
        hipLaunchKernelGGL(k_qk_norm, dim3(unsigned(ceil_div(16 * C, 256))), dim3(256), 0, s, C, cqkv, cqis);
      if (!use_rad || rad_stale_)  // with the radial tables filled, nothing reads these
        hipLaunchKernelGGL(k_class_tables, dim3(unsigned(C * C), 8), dim3(128), 0, s, C, cqkv, B.fw1[0], B.fw1[1],
                           B.ob10[0], B.ob10[1], cmt, cc0);
      if (use_rad && rad_stale_) {  // the classes' rows are those of the system: once after set_system
        const std::size_t keys = std::size_t(C) * (C + 1) / 2, half = keys * kRadialIntervals * kRadRecord;
        double *tab = static_cast<double *>(rad_tab_->p);
        hipLaunchKernelGGL(k_radial_tables, dim3(unsigned(keys * kRadialIntervals)), dim3(256), 0, s, C, cmt, cc0,
                           rad_val_, rad_slope_, rad_dom_, tab, tab + half);
        rad_stale_ = false;
      }
      if (!use_rad) {  // the element-pair kernels' pair order
        const dim3 gsort(unsigned(ceil_div(PA, kClsChunk)));
        hipLaunchKernelGGL(k_cls_count, gsort, dim3(256), 0, s, nact, pa, z, lut, C, chist);
        hipLaunchKernelGGL(k_cls_scan, dim3(1), dim3(64), 0, s, C * C, chist, ccur, 1, nullptr);
        hipLaunchKernelGGL(k_cls_place, gsort, dim3(256), 0, s, nact, pa, z, lut, C, ccur, cord);
      }
    } else {
      hipLaunchKernelGGL(k_qkv_mfma, dim3(gN64, kHeads), dim3(256), 0, s, int(N), xb, B.qkvp, qb);
      if (qk_norm_)
        hipLaunchKernelGGL(k_qk_norm, dim3(unsigned(ceil_div(16 * N, 256))), dim3(256), 0, s, int(N), qb,
                           qkis + b * Nz * 16);
    }
    timed(blk0 ? (use_rad ? "filter_fwd_block0_radial" : use_cls ? "filter_fwd_block0_tables" : "filter_fwd_block0")
               : (use_rt ? "filter_fwd_radial" : "filter_fwd"),
          0, [&] {
      if (blk0 && use_rad)
        hipLaunchKernelGGL(k_radial_fwd, dim3(gP16), dim3(256), 0, s, nact, pa, pr, z,
                           static_cast<const int *>(cls_lut_->p), C, static_cast<const double *>(rad_tab_->p),
                           rad_dom_, inv_avg, pab);
      else if (blk0 && use_cls)
        hipLaunchKernelGGL(k_filter_fwd_class, dim3(gP64), dim3(256), 0, s, nact, cord, pa, pr, z,
                           static_cast<const int *>(cls_lut_->p), C, cmt, cc0, inv_avg, FM, pab);
      else if (scalar)
        hipLaunchKernelGGL(k_filter_fwd, dim3(gP), dim3(128), 0, s, nact, pa, pr, evb, A, psb, pfb);
      else if (b == 0)  // ev = 0: the spherical branch is a constant
        hipLaunchKernelGGL(k_filter_fwd_mfma<true>, dim3(gP64), dim3(256), 0, s, nact, pa, pr, evb, qb, inv_avg, FM,
                           psb, pfb, pab);
      else if (use_rt)  // rows and logits in bucket order, the radial branches from the tables
        hipLaunchKernelGGL(k_radial_fwd_rows, dim3(gR), dim3(256), 0, s, rslots, rord, pa, pr, evb, qb, B.rrow,
                           rbl_dom_, inv_avg, FM, psb, pfb, pab);
      else
        hipLaunchKernelGGL(k_filter_fwd_mfma<false>, dim3(gP64), dim3(256), 0, s, nact, pa, pr, evb, qb, inv_avg, FM,
                           psb, pfb, pab);
    });
    timed("attn_fwd", 1, [&] {
      if (scalar)
        hipLaunchKernelGGL(k_attn_fwd, dim3(gN4), dim3(256), 0, s, int(N), sr_off, iact, iother, xb, evb, qb,
                           pfb, pY, pfc, inv_avg, pab, ainv, aevb);
      else
        hipLaunchKernelGGL(k_attn_msg, dim3(gN4), dim3(256), 0, s, int(N), sr_off, iact, iother, xb, evb,
                           blk0 && use_cls ? cqkv : qb, pY, pfc, pab, B.ln1w, B.ln1b, ln_eps_, norm1_, n1b, n1hb,
                           n1ib, act, aevb, z, blk0 && use_cls ? static_cast<const int *>(cls_lut_->p) : nullptr);
    });
    if (scalar)  // the MFMA path's k_attn_msg has done LayerNorm 1 already
      hipLaunchKernelGGL(k_post1, dim3(gN4), dim3(256), 0, s, int(N), ainv, B.ln1w, B.ln1b, ln_eps_, norm1_, n1b,
                         n1hb, n1ib, act);
    // the post-attention node chain in one kernel (MLP, interaction, LayerNorm 2, ev gate)
    const NodeChainArgs NC{B.m1p, B.m1bp, B.m2p, B.m2bp, B.intp, B.intbp, B.int_cg, B.ln2w, B.ln2b, hw_.exp2_256,
                           ln_eps_, norm2_};
    hipLaunchKernelGGL(k_node_fwd, dim3(unsigned(ceil_div(N, 32))), dim3(256), 0, s, int(N), act, n1b, aevb, NC, hpb, tb,
                       xs + (b + 1) * Nz * kF, evs + (b + 1) * Nz * kE, p2h, p2i);
    if (!resid_.empty() && b + 1 < L)
      hipLaunchKernelGGL(k_axpby, dim3(gNF), dim3(256), 0, s, Nz * kF, resid_[b + 1], xs + (b + 1) * Nz * kF,
                         x0l_[b + 1], x0);
  }

  // --- heads, charge correction, long range ---
  HeadArgs H{hw_.ew2, hw_.qw2, hw_.escale, hw_.eshift, hw_.qemb, hw_.hqemb, hw_.hvshift,
             hw_.hkey_bwd, hw_.hkey_c, hw_.eb2, hw_.qb2, hw_.ckey_bwd, hw_.ckey_c, hw_.cvshift, hw_.ho};
  const double *xf = xs + L * Nz * kF;
  gemm(1, int(N), kF, int(HO), xf, kF, hw_.w1p, hw_.b1p, hhead, int(HO), hact);
  hipLaunchKernelGGL(k_heads, dim3(gN4), dim3(256), 0, s, int(N), z, hact, H, eatom, qraw, heff, hir, c6eff, c6r);
  hipLaunchKernelGGL(k_image_center, dim3(unsigned(n_images_)), dim3(1024), 0, s, img_off, img_q, qraw, q, 0);
  long_range();
  hipLaunchKernelGGL(k_image_center, dim3(unsigned(n_images_)), dim3(1024), 0, s, img_off, img_q, dq, qseed, 1);
  hipLaunchKernelGGL(k_heads_bwd, dim3(gN4), dim3(256), 0, s, int(N), z, hhead, qseed, dh, heff, dc, c6eff, H,
                     ghead);
  gemm(0, int(N), int(HO), kF, ghead, int(HO), hw_.w1tp, nullptr, gx, kF, nullptr);
  fill(gev, Nz * kE);

  // --- interaction blocks, reverse ---
  for (int b = L - 1; b >= 0; --b) {
    const BlockWeights &B = bw_[b];
    double *evb = evs + b * Nz * kE;
    double *qb = qkv + b * Nz * 640, *aevb = aev + b * Nz * kE;
    double *n1b = n1 + b * Nz * kF, *n1hb = n1hat + b * Nz * kF, *n1ib = n1is + b * Nz;
    double *hpb = hpre + b * Nz * kF, *tb = tout + b * Nz * kNI;
    double *p2h = pre2hat + b * Nz * kF, *p2i = pre2is + b * Nz;
    double *psb = ps + b * 4 * Pa, *pab = palpha + b * 16 * Pa;
    double *pfb = scalar ? pf + b * 256 * Pa : (b > 0 ? pf + (b - 1) * 256 * Pa : nullptr);
    FilterArgs A;
    for (int k = 0; k < 2; ++k) {
      A.fw0[k] = B.fw0[k]; A.fb0[k] = B.fb0[k]; A.fw1t[k] = B.fw1t[k]; A.fb1[k] = B.fb1[k];
      A.fe0[k] = B.fe0[k]; A.feb0[k] = B.feb0[k]; A.fe1t[k] = B.fe1t[k]; A.feb1[k] = B.feb1[k];
    }
    A.att_cg = B.att_cg; A.rbf_b = hw_.rbf_b; A.rbf_k = hw_.rbf_k; A.rbf_kr = hw_.rbf_kr; A.gamma = gamma_;
    // the post-attention node chain in reverse in one kernel: gainv, gaev
    const NodeChainBwdArgs NB{B.inttp, B.m2tp, B.m1tp, B.int_cg, B.ln1w, B.ln2w, norm1_, norm2_};
    hipLaunchKernelGGL(k_node_bwd, dim3(unsigned(ceil_div(N, 32))), dim3(256), 0, s, int(N), gx, gev, tb, aevb, p2h,
                       p2i, hpb, n1b, n1hb, n1ib, NB, gainv, gaev);
    if (scalar) {
      // scalar cross-check path: the attention reverse writes the pair
      // adjoints (df, dE/dfc, dE/dY) and the scalar filter reverse reads them
      timed(b == 0 ? "attn_bwd_block0" : "attn_bwd", 1, [&] {
#define SO3LR_ATTN_BWD(ADJ, FIRST)                                                                              \
  hipLaunchKernelGGL((k_attn_bwd<ADJ, FIRST>), dim3(gN4), dim3(256), 0, s, int(N), sr_off, iact, iother, qb, pfb, pY, \
                     pfc, pab, gainv, gaev, inv_avg, gqkv, df, dfc, dY)
        // the first reverse block (L - 1) writes dY, the others add to it
        if (b > 0 && b == L - 1) SO3LR_ATTN_BWD(true, true);
        else if (b > 0) SO3LR_ATTN_BWD(true, false);
        else if (L == 1) SO3LR_ATTN_BWD(false, true);
        else SO3LR_ATTN_BWD(false, false);
#undef SO3LR_ATTN_BWD
      });
      timed(b == 0 ? "filter_bwd_block0" : "filter_bwd", 0, [&] {
        hipLaunchKernelGGL(k_filter_bwd, dim3(gP), dim3(128), 0, s, nact, pr, pfc, psb, df, dfc, A, rc_, ds, dr);
      });
    } else {
      // node adjoints (dq, dk, dv; not needed in block 0, whose inputs do not
      // depend on the positions), then the pair adjoints and the filter
      // reverse in one pair-major kernel
      const bool first = b == L - 1;
      if (b > 0)
        timed("attn_bwd", 1, [&] {
          if (first)
            hipLaunchKernelGGL(k_attn_bwd_nodes<true>, dim3(gN4), dim3(256), 0, s, int(N), sr_off, iact, iother, qb,
                               pfb, pY, pfc, pab, gainv, gaev, inv_avg, gqkv, psc, dfc, dY);
          else
            hipLaunchKernelGGL(k_attn_bwd_nodes<false>, dim3(gN4), dim3(256), 0, s, int(N), sr_off, iact, iother, qb,
                               pfb, pY, pfc, pab, gainv, gaev, inv_avg, gqkv, psc, dfc, dY);
        });
      const FilterMfma FM = filter_mfma(B, hw_, gamma_);
      if (b == 0 && use_cls) {
        hipLaunchKernelGGL(k_class_gv, dim3(unsigned(ceil_div(N, 4))), dim3(256), 0, s, int(N), C, gainv, cqkv, cgv);
        timed(use_rad ? "filter_bwd_block0_radial" : "filter_bwd_block0_tables", 0, [&] {
          const int *lut = static_cast<const int *>(cls_lut_->p);
          const double *slope =
              use_rad ? static_cast<const double *>(rad_tab_->p) +
                            std::size_t(C) * (C + 1) / 2 * kRadialIntervals * kRadRecord
                      : nullptr;
          if (use_rad && first)
            hipLaunchKernelGGL(k_radial_bwd<true>, dim3(gP16), dim3(256), 0, s, nact, pa, pr, pfc, pY, pab, gaev, z,
                               lut, C, slope, cgv, rad_dom_, inv_avg, rc_, dr, dY);
          else if (use_rad)
            hipLaunchKernelGGL(k_radial_bwd<false>, dim3(gP16), dim3(256), 0, s, nact, pa, pr, pfc, pY, pab, gaev,
                               z, lut, C, slope, cgv, rad_dom_, inv_avg, rc_, dr, dY);
          else if (first)
            hipLaunchKernelGGL(k_filter_bwd_class<true>, dim3(gP64), dim3(256), 0, s, nact, cord, pa, pr, pfc, pY, pab,
                               gaev, z, lut, C, cmt, cgv, inv_avg, FM, rc_, dr, dY);
          else
            hipLaunchKernelGGL(k_filter_bwd_class<false>, dim3(gP64), dim3(256), 0, s, nact, cord, pa, pr, pfc, pY,
                               pab, gaev, z, lut, C, cmt, cgv, inv_avg, FM, rc_, dr, dY);
        });
      } else {
        timed(b == 0 ? "filter_bwd_block0" : (use_rt ? "filter_bwd_radial" : "filter_bwd"), 0, [&] {
#define SO3LR_FILTER_BWD(E0, FIRST)                                                                                \
  hipLaunchKernelGGL((k_filter_bwd_mfma<E0, FIRST>), dim3(gP64), dim3(256), 0, s, nact, pa, pr, psb, pfc, pY, pab,  \
                     qb, gainv, gaev, psc, dfc, inv_avg, FM, rc_, ds, dr, dY)
          if (b == 0 && first) SO3LR_FILTER_BWD(true, true);
          else if (b == 0) SO3LR_FILTER_BWD(true, false);
          else if (use_rt)  // in interval order, the radial branches' dE/dr from the slope tables
            hipLaunchKernelGGL((k_filter_bwd_mfma<false, false, true>), dim3(gR), dim3(256), 0, s, nact, pa, pr, psb,
                               pfc, pY, pab, qb, gainv, gaev, psc, dfc, inv_avg, FM, rc_, ds, dr, dY, rslots, rord,
                               B.rdr, rbl_dom_);
          else SO3LR_FILTER_BWD(false, false);  // dE/dY of blocks after 0: the node-major reverse
#undef SO3LR_FILTER_BWD
        });
      }
    }
    // the adjoints of a block's inputs x_b, ev_b feed the block below; block
    // 0's inputs (the embedding and ev = 0) do not depend on the positions
    if (b > 0) {
      if (qk_norm_)  // through the QK normalisation to the raw projections
        hipLaunchKernelGGL(k_qk_norm_bwd, dim3(unsigned(ceil_div(16 * N, 256))), dim3(256), 0, s, int(N), qb,
                           qkis + b * Nz * 16, gqkv);
      hipLaunchKernelGGL(k_qkv_bwd_mfma, dim3(gN64, kHeads), dim3(256), 0, s, int(N), gqkv, B.qkvtp, gainv, gx);
      // residual scalars: the adjoint of the block below's output
      if (!resid_.empty()) hipLaunchKernelGGL(k_scale, dim3(gNF), dim3(256), 0, s, Nz * kF, resid_[b], gx);
      hipLaunchKernelGGL(k_ev_bwd, dim3(gN4), dim3(256), 0, s, int(N), sr_off, iact, iother, evb, B.att_cg, ds,
                         gaev, gev);
    }
  }

  }  // v1 widths

  // --- geometry reverse, forces, energies, virial ---
  hipLaunchKernelGGL(k_geom_bwd, dim3(ceil_div(PA, 256)), dim3(256), 0, s, nact, pv, pr,
                     dr, pzbl, dY, pg);
  hipLaunchKernelGGL(k_forces, dim3(gN4), dim3(256), 0, s, int(N), sr_off, sr_inc, c2a, pg, pzbl, flr, eatom, elr,
                     perm, fo, ezbl, etot);
  hipLaunchKernelGGL(k_reduce_part, dim3(kReduceBlocks), dim3(256), 0, s, int(N), nact, etot, pv, pg, vlr, parts,
                     partial);
  hipLaunchKernelGGL(k_reduce_final, dim3(1), dim3(256), 0, s, kReduceBlocks, partial, red);
  hipLaunchKernelGGL(k_copy_count, dim3(1), dim3(64), 0, s, nact + 1, red + 9);  // the pairs found
  HIP_CHECK(hipGetLastError());
  HIP_CHECK(hipMemcpyAsync(host_out_, red, 10 * sizeof(double), hipMemcpyDeviceToHost, s));
  };  // enqueue

  const GraphKey key{x_in, fo, etot, flags, {box_len_[0], box_len_[1], box_len_[2]}, s, topo_version_,
                     alloc_epoch_};
  if (from_scratch) {
    enqueue();  // instantiating a graph allocates: never here
  } else if (timing_ || !use_graphs_) {
    enqueue();
  } else if (graph_exec_ && key == graph_key_) {
    HIP_CHECK(hipGraphLaunch(graph_exec_, s));
  } else if (key == last_key_) {
    // the same call twice in a row: capture it once and replay from now on
    drop_graph();
    hipGraph_t graph = nullptr;
    HIP_CHECK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    enqueue();
    HIP_CHECK(hipStreamEndCapture(s, &graph));
    const hipError_t ierr = hipGraphInstantiate(&graph_exec_, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (ierr != hipSuccess) {
      graph_exec_ = nullptr;
      throw DeviceError(std::string("HIP error in hipGraphInstantiate: ") + hipGetErrorString(ierr));
    }
    graph_key_ = key;
    HIP_CHECK(hipGraphLaunch(graph_exec_, s));
  } else {
    enqueue();
  }
  if (!from_scratch) last_key_ = key;
  if (stage_count_)  // compute_host's read-back, ahead of the one wait
    HIP_CHECK(hipMemcpyAsync(stage_dst_, stage_src_, stage_count_ * sizeof(double), hipMemcpyDeviceToHost, s));
  HIP_CHECK(hipStreamSynchronize(s));
  const double *host_red = host_out_;
  const std::int64_t host_nact = std::int64_t(host_out_[9]);
  last_active_ = host_nact;
  if (host_nact > PA) {
    // more active pairs than the buffers hold (atoms moved closer since the
    // count): nothing beyond the capacity was written; grow and evaluate again
    for (Pending &pd : pending) {
      (void)hipEventDestroy(pd.a);
      (void)hipEventDestroy(pd.b);
    }
    act_cap_ = std::min<std::int64_t>(P, host_nact + host_nact / 8 + 256);
    compute_impl(x_in, flags, f_out, eatom_out, energy, virial, from_scratch);
    return;
  }
  for (Pending &pd : pending) {
    float ms = 0.f;
    HIP_CHECK(hipEventElapsedTime(&ms, pd.a, pd.b));
    Timing &t = timings_[pd.name];
    t.ms += ms;
    t.launches += 1;
    t.units += pd.unit_kind == 0 ? host_nact : N;
    (void)hipEventDestroy(pd.a);
    (void)hipEventDestroy(pd.b);
  }
  if (energy) *energy = host_red[0];
  if (virial) for (int c = 0; c < 6; ++c) virial[c] = host_red[1 + c];
  totals_[0] = host_red[7];
  totals_[1] = host_red[8];
  last_etot_ = etot;
  evaluated_ = true;
  last_from_scratch_ = from_scratch;
  (void)flags;
}

void Evaluator::last_vatom(double *out, bool on_device) {
  if (!evaluated_) throw std::logic_error("SO3LR: no evaluation yet");
  if (last_from_scratch_)
    throw std::logic_error("SO3LR: so3lr_compute_device_noalloc keeps no per-atom virial; use so3lr_compute_device");
  const std::int64_t N = n_;
  const std::size_t Nz = std::size_t(N);
  double *dst = on_device ? out : ensure<double>(vatom_, Nz * 6);
  const int *perm = permuted_ ? static_cast<const int *>(perm_->p) : nullptr;
  // the evaluation's own buffers, as it left them
  hipLaunchKernelGGL(k_vatom, dim3(ceil_div(N, 4)), dim3(256), 0, stream_, int(N),
                     static_cast<const int *>(sr_inc_off_->p), static_cast<const int *>(sr_inc_->p),
                     static_cast<const int *>(cand2act_->p), static_cast<const double *>(pv_->p),
                     static_cast<const double *>(pg_->p), static_cast<const double *>(vlr_->p), perm, dst);
  HIP_CHECK(hipGetLastError());
  if (!on_device) HIP_CHECK(hipMemcpyAsync(out, dst, Nz * 6 * sizeof(double), hipMemcpyDeviceToHost, stream_));
  HIP_CHECK(hipStreamSynchronize(stream_));
}

bool Evaluator::timing_read(const std::string &kernel, double &total_ms, std::int64_t &launches,
                            std::int64_t &units) const {
  const auto it = timings_.find(kernel);
  if (it == timings_.end()) return false;
  total_ms = it->second.ms;
  launches = it->second.launches;
  units = it->second.units;
  return true;
}

void Evaluator::last_terms(double *learned, double *zbl, double *lr, double *charges, double *hirshfeld,
                           double *totals, double *image_energy) {
  if (!evaluated_) throw std::logic_error("SO3LR: no evaluation yet");
  if (last_from_scratch_)
    throw std::logic_error("SO3LR: so3lr_compute_device_noalloc keeps no per-atom terms; use so3lr_compute_device");
  const std::size_t Nz = std::size_t(n_);
  // node-ordered buffers come back in the caller's atom order
  std::vector<std::vector<double>> staged;
  std::vector<double *> dests;
  auto get = [&](double *dst, Buffer *b) {
    if (!dst) return;
    double *into = dst;
    if (permuted_) {
      staged.emplace_back(Nz);
      into = staged.back().data();
      dests.push_back(dst);
    }
    HIP_CHECK(hipMemcpyAsync(into, b->p, Nz * sizeof(double), hipMemcpyDeviceToHost, stream_));
  };
  get(learned, eatom_); get(zbl, ezbl_); get(lr, elr_); get(charges, q_); get(hirshfeld, hir_);
  std::vector<double> et;
  if (image_energy) {
    et.resize(Nz);
    HIP_CHECK(hipMemcpyAsync(et.data(), last_etot_, Nz * sizeof(double), hipMemcpyDeviceToHost, stream_));
  }
  HIP_CHECK(hipStreamSynchronize(stream_));
  for (std::size_t k = 0; k < dests.size(); ++k)
    for (std::size_t i = 0; i < Nz; ++i) dests[k][perm_host_[i]] = staged[k][i];
  if (totals) { totals[0] = totals_[0]; totals[1] = totals_[1]; }
  if (image_energy)
    for (std::int64_t k = 0; k < n_images_; ++k) {
      double s = 0.0;
      for (std::int64_t i = image_offsets_[k]; i < image_offsets_[k + 1]; ++i) s += et[i];
      image_energy[k] = s;
    }
}

}  // namespace so3lr_amd
