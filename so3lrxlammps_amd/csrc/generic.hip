// The generic-width evaluation (see generic.hpp): kernels and host side.
//
// Data layout in HBM (N nodes, P active-pair capacity, L blocks), natural
// channel order throughout:
//   node state per block b:  x[b] N x F, ev[b] N x E, qkv[b] N x 5F
//                            (q | k | v | q_ev | k_ev, head-major inside each)
//   pair state per block b:  s (NH slot invariants), f (F inv | F ev filters;
//                            none for block 0 on the element-pair tables),
//                            alpha (2 directions x (NH inv + NH ev))
//   per evaluation:          rbf (R), and the reverse's logit adjoints psc
//                            (4 NH), dE/dfc, ds (NH), dE/dr and dE/dY (24)
// Pair p = {a, b}, v = x_a - x_b: direction 0 is the edge b -> a (receiver a,
// harmonics Y(v/r)), direction 1 the edge a -> b ((-1)^l Y(v/r)).
#include "generic.hpp"
#include "evaluator.hpp"
#include "mfma_ops.hpp"

#include <algorithm>
#include <array>
#include <cmath>
#include <stdexcept>
#include <string>

namespace so3lr_amd {

#define G_CHECK(expr)                                                                                    \
  do {                                                                                                   \
    hipError_t err_ = (expr);                                                                            \
    if (err_ != hipSuccess) throw DeviceError(std::string("HIP error in ") + #expr + ": " + hipGetErrorString(err_)); \
  } while (0)

namespace {

__device__ __forceinline__ double gsilu(double x) { return x / (1.0 + exp(-x)); }
__device__ __forceinline__ double gsilu_prime(double x) {
  const double s = 1.0 / (1.0 + exp(-x));
  return s * (1.0 + x * (1.0 - s));
}
// Sum over the 64 lanes of a wavefront, the same value in every lane (lane
// 0's butterfly result, broadcast).  All lanes must be active.
__device__ __forceinline__ double wsum(double v) {
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return __shfl(v, 0, 64);
}

// ------------------------------------------------------------------ GEMM
// Y (rows x O, leading dimension ldy) = epilogue(X (rows x K, ldx) op(W) + bias)
// with op(W) = W^T for W (O x K) row-major (the model file's (out, in)
// layout) or, WKO, W itself for W (K x O) row-major (the adjoint of a layer:
// X W).  rows = min(*rows_dev, rows) when rows_dev is given (the active-pair
// count on the device).
enum { EPI_STORE = 0, EPI_SILU, EPI_ACCUM, EPI_ADD, EPI_DSILU, EPI_DSILU_ADD };
struct GemmArgs {
  int rows;
  const int *rows_dev;
  int K, O;
  const double *X;
  int ldx;
  const double *W;
  const double *bias;
  double *Y;
  int ldy;
  double *Y2;         // EPI_SILU: the pre-activation as well (may be null)
  int ldy2;
  const double *aux;  // EPI_DSILU*: silu' of aux
  int ldaux;
  const double *res;  // EPI_ADD, EPI_DSILU_ADD: added
  int ldres;
  // batches (grid z = nby * nbx, z = zy * nbx + zx): X, Y and res move by
  // zy * (..)0 + zx * (..)1 elements, W by z * wbs
  int nbx;
  long xbs0, xbs1, ybs0, ybs1, rbs0, rbs1, wbs;
  int ldw;  // WKO: the weight's row length (its full output width); 0: O
};

typedef double gv4d __attribute__((ext_vector_type(4)));

// 64 x BN output tiles (BN = 32 NT, up to 320 columns: a filter or node
// layer's whole output row in one workgroup, so X is read once) on fp64 MFMA
// 16x16x4: four wavefronts in 2 x 2, each 32 rows x BN/2 columns (2 x NT
// MFMA tiles).
// D[i][j] += sum_k A[i][k] B[k][j] with A[i][k] = X[row i][k] (lane l gives
// i = l % 16, k = l / 16) and B[k][j] = op(W)[k][col j] (lane l gives
// k = l / 16, j = l % 16); lane l holds D[l / 16 + 4 r][l % 16] in register
// r, so sixteen lanes write sixteen adjacent columns of one row.  K runs in
// chunks of 16 through LDS; the next chunk's global loads are issued before
// the current chunk's MFMAs.
#ifndef SO3LR_GEMM_WAVES
#define SO3LR_GEMM_WAVES 3
#endif
template <int EPI, bool WKO, int NT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(SO3LR_GEMM_WAVES))) void g_gemm(GemmArgs A) {
  constexpr int BN = 32 * NT;      // output columns per workgroup (NT MFMA column tiles per wavefront)
  constexpr int WPT = BN / 16;     // W chunk values per thread (BN x 16 / 256)
  __shared__ double xs[64][17];
  __shared__ double ws[BN][17];
  const int rows = A.rows_dev ? min(*A.rows_dev, A.rows) : A.rows;
  // With several column blocks the grid's x is a multiple of 8 and the
  // blocks are taken in dispatch order, (row block, column block) such that
  // the column blocks of one row block run one after another on one XCD
  // (dispatch goes round-robin over the 8 XCDs): the later ones read that
  // row block's X from the XCD's L2, not HBM.
  int rb = blockIdx.x, cb = blockIdx.y;
  if (gridDim.y > 1) {
    const unsigned lin = blockIdx.y * gridDim.x + blockIdx.x, k = lin >> 3;
    rb = int((k / gridDim.y) * 8 + (lin & 7));
    cb = int(k % gridDim.y);
  }
  const int row0 = rb * 64, col0 = cb * BN;
  if (row0 >= rows) return;  // uniform over the block
  {
    const long zx = long(blockIdx.z) % A.nbx, zy = long(blockIdx.z) / A.nbx;
    A.X += zy * A.xbs0 + zx * A.xbs1;
    A.Y += zy * A.ybs0 + zx * A.ybs1;
    if (A.res) A.res += zy * A.rbs0 + zx * A.rbs1;
    A.W += long(blockIdx.z) * A.wbs;
  }
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wr0 = (wv >> 1) * 32, wc0 = (wv & 1) * (BN / 2);
  const int li = lane & 15, lk = lane >> 4;
  double xreg[4], wreg[WPT];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int idx = tid + 256 * q, kk = idx & 15, rr = idx >> 4;
      const int row = row0 + rr, k = k0 + kk;
      xreg[q] = (row < rows && k < A.K) ? A.X[std::size_t(row) * A.ldx + k] : 0.0;
    }
#pragma unroll
    for (int q = 0; q < WPT; ++q) {
      const int idx = tid + 256 * q;
      if (WKO) {
        const int cc = idx % BN, kk = idx / BN, col = col0 + cc, k = k0 + kk;
        wreg[q] = (col < A.O && k < A.K) ? A.W[std::size_t(k) * (A.ldw ? A.ldw : A.O) + col] : 0.0;
      } else {
        const int kk = idx & 15, cc = idx >> 4, col = col0 + cc, k = k0 + kk;
        wreg[q] = (col < A.O && k < A.K) ? A.W[std::size_t(col) * A.K + k] : 0.0;
      }
    }
  };
  auto stash = [&] {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int idx = tid + 256 * q;
      xs[idx >> 4][idx & 15] = xreg[q];
    }
#pragma unroll
    for (int q = 0; q < WPT; ++q) {
      const int idx = tid + 256 * q;
      if (WKO) ws[idx % BN][idx / BN] = wreg[q];
      else ws[idx >> 4][idx & 15] = wreg[q];
    }
  };
  gv4d acc[2][NT];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < NT; ++b) acc[a][b] = gv4d{0.0, 0.0, 0.0, 0.0};
  fetch(0);
  stash();
  __syncthreads();
  for (int k0 = 0; k0 < A.K; k0 += 16) {
    const bool more = k0 + 16 < A.K;
    if (more) fetch(k0 + 16);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int kk = lk + 4 * v;
      double av[2], bv[NT];
#pragma unroll
      for (int a = 0; a < 2; ++a) av[a] = xs[wr0 + 16 * a + li][kk];
#pragma unroll
      for (int b = 0; b < NT; ++b) bv[b] = ws[wc0 + 16 * b + li][kk];
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < NT; ++b) acc[a][b] = __builtin_amdgcn_mfma_f64_16x16x4f64(av[a], bv[b], acc[a][b], 0, 0, 0);
    }
    __syncthreads();
    if (more) {
      stash();
      __syncthreads();
    }
  }
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < NT; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = row0 + wr0 + 16 * a + lk + 4 * r;
        const int col = col0 + wc0 + 16 * b + li;
        if (row >= rows || col >= A.O) continue;
        const double dot = acc[a][b][r];
        const double pre = dot + (A.bias ? A.bias[col] : 0.0);
        double *y = A.Y + std::size_t(row) * A.ldy + col;
        if (EPI == EPI_STORE) {
          *y = pre;
        } else if (EPI == EPI_SILU) {
          if (A.Y2) A.Y2[std::size_t(row) * A.ldy2 + col] = pre;
          *y = gsilu(pre);
        } else if (EPI == EPI_ACCUM) {
          *y += pre;
        } else if (EPI == EPI_ADD) {
          *y = pre + A.res[std::size_t(row) * A.ldres + col];
        } else if (EPI == EPI_DSILU) {
          *y = dot * gsilu_prime(A.aux[std::size_t(row) * A.ldaux + col]);
        } else {
          *y = A.res[std::size_t(row) * A.ldres + col] + dot * gsilu_prime(A.aux[std::size_t(row) * A.ldaux + col]);
        }
      }
}

// ------------------------------------------------------------- node kernels
// QK normalisation: each 32-wide head row of q, k, q_ev, k_ev scaled to unit
// RMS (eps 1e-6; kokkos_integrated_block0.cpp:288-328), 1/rms kept.
__device__ __forceinline__ int qk_row(int k) { return k < 2 ? k : k + 1; }  // q k (v) qe ke
__global__ __launch_bounds__(256) void g_qk_norm(int N, int F, int NH, double *__restrict__ qkv,
                                                 double *__restrict__ qkis) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= N * 4 * NH) return;
  const int n = t / (4 * NH), k = (t / NH) % 4, h = t % NH;
  double *row = qkv + std::size_t(n) * 5 * F + std::size_t(qk_row(k)) * F + 32 * h;
  double ms = 0.0;
  for (int c = 0; c < 32; ++c) ms += row[c] * row[c];
  const double r = 1.0 / sqrt(ms / 32.0 + 1e-6);
  for (int c = 0; c < 32; ++c) row[c] *= r;
  qkis[t] = r;
}
// Through the normalisation: g <- r (g - y mean(g y)), y the normalised row.
__global__ __launch_bounds__(256) void g_qk_norm_bwd(int N, int F, int NH, const double *__restrict__ qkv,
                                                     const double *__restrict__ qkis, double *__restrict__ gqkv) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= N * 4 * NH) return;
  const int n = t / (4 * NH), k = (t / NH) % 4, h = t % NH;
  const std::size_t o = std::size_t(n) * 5 * F + std::size_t(qk_row(k)) * F + 32 * h;
  double m = 0.0;
  for (int c = 0; c < 32; ++c) m += gqkv[o + c] * qkv[o + c];
  m /= 32.0;
  const double r = qkis[t];
  for (int c = 0; c < 32; ++c) gqkv[o + c] = r * (gqkv[o + c] - qkv[o + c] * m);
}

__global__ void g_axpby(std::size_t n, double a, double *x, double c, const double *x0) {
  const std::size_t i = std::size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) x[i] = a * x[i] + c * x0[i];
}
__global__ void g_scale(std::size_t n, double a, double *g) {
  const std::size_t i = std::size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) g[i] *= a;
}
__global__ void g_fill(double *p, std::size_t n) {
  const std::size_t i = std::size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.0;
}

// The normalisation of one node row held 4 channels per lane (c = lane + 64 j,
// j < F / 64; kokkos_post_attention_block0.cpp:97-162): mode 0 affine
// LayerNorm (biased variance), 1 RMSNorm without scale (w = 1, b = 0
// given), 2 none.  h = normalised row, y = h w + b, is = 1 / sigma.
__device__ __forceinline__ void g_norm_row(int F, int mode, const double *v, const double *w, const double *b,
                                           double eps, int lane, double *y, double *h, double &is) {
  const int J = F >> 6;
  double s = 0.0;
  for (int j = 0; j < J; ++j) s += v[j];
  const double mean = mode == 0 ? wsum(s) / F : 0.0;
  double q = 0.0;
  for (int j = 0; j < J; ++j) q += (v[j] - mean) * (v[j] - mean);
  is = mode == 2 ? 1.0 : 1.0 / sqrt(wsum(q) / F + eps);
  for (int j = 0; j < J; ++j) {
    const int c = lane + 64 * j;
    h[j] = (v[j] - mean) * is;
    y[j] = mode == 2 ? v[j] : h[j] * w[c] + b[c];
  }
}
// Its adjoint: gx given gy, the normalised row h and 1 / sigma.
__device__ __forceinline__ void g_norm_row_bwd(int F, int mode, const double *gy, const double *w,
                                               const double *h, double is, int lane, double *gx) {
  const int J = F >> 6;
  if (mode == 2) {
    for (int j = 0; j < J; ++j) gx[j] = gy[j];
    return;
  }
  double gh[4], a = 0.0, bsum = 0.0;
  for (int j = 0; j < J; ++j) {
    gh[j] = mode == 0 ? gy[j] * w[lane + 64 * j] : gy[j];
    a += gh[j];
    bsum += gh[j] * h[j];
  }
  const double mg = mode == 0 ? wsum(a) / F : 0.0, mgx = wsum(bsum) / F;
  for (int j = 0; j < J; ++j) gx[j] = is * (gh[j] - mg - h[j] * mgx);
}

// Dispatch block b (round-robin over the 8 XCDs) to logical block: each XCD
// takes a contiguous run of the `active` blocks, so consecutive pairs or
// nodes (spatially sorted: they share endpoints and partners) share that
// XCD's L2.  -1: beyond the active blocks.  The grid is a multiple of 8 and
// holds at least `active` blocks.
__device__ __forceinline__ int g_xcd_block(int active) {
  const int b = blockIdx.x;
  const int per = active >> 3, rem = active & 7, xcd = b & 7, i = b >> 3;
  if (i >= per + (xcd < rem ? 1 : 0)) return -1;
  return xcd * per + (xcd < rem ? xcd : rem) + i;
}

// Attention messages, node-major (kokkos_integrated_block0.cpp:330-385):
// node n receives from each incident pair's partner o the invariant message
// fc alpha v_o and the equivariant fc alpha_ev Y (parity of the direction),
// then the residual and the first normalisation (and silu of it, the MLP
// input).  One wavefront per node.
__global__ __launch_bounds__(256) void g_attn_msg(GDims d, int N, const int *__restrict__ inc_off,
                                                  const int *__restrict__ iact, const int *__restrict__ iother,
                                                  const double *__restrict__ x, const double *__restrict__ ev,
                                                  const double *__restrict__ qkv, const double *__restrict__ pY,
                                                  const double *__restrict__ pfc, const double *__restrict__ palpha,
                                                  const double *__restrict__ lnw, const double *__restrict__ lnb,
                                                  double eps, int mode, double *__restrict__ n1,
                                                  double *__restrict__ n1hat, double *__restrict__ n1is,
                                                  double *__restrict__ act, double *__restrict__ aev) {
  const int lane = threadIdx.x & 63;
  const int blk = g_xcd_block((N + 3) / 4);
  if (blk < 0) return;
  const int n = blk * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const int F = d.F, NH = d.NH, E = d.E, J = F >> 6;
  double di[4] = {0, 0, 0, 0}, de[2] = {0, 0};
  // this lane's channels: invariant c = lane + 64 j (head c / 32), and
  // equivariant c = lane + 64 j below E (slot, harmonic, parity)
  int sl[2] = {0, 0}, sh[2] = {0, 0};
  double par[2] = {1.0, 1.0};
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int c = lane + 64 * j;
    if (c < E) {
      sl[j] = d.slot[c];
      sh[j] = d.sh[c];
      par[j] = d.par[sl[j]];
    }
  }
  struct Terms {
    double v[4], a[4], y[2], ae[2], fc;
  };
  auto load = [&](int e, int o) {
    Terms T;
    const int p = e >> 1, side = e & 1;
    T.fc = pfc[p];
    const double *al = palpha + std::size_t(p) * 4 * NH + side * 2 * NH;
    const double *vo = qkv + std::size_t(o) * 5 * F + 2 * F;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = lane + 64 * (j < J ? j : 0);
      T.v[j] = vo[c];
      T.a[j] = al[c >> 5];
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int c = lane + 64 * j;
      const bool on = c < E;
      T.y[j] = on ? pY[std::size_t(p) * 24 + sh[j]] * (side ? par[j] : 1.0) : 0.0;
      T.ae[j] = on ? al[NH + sl[j]] : 0.0;
    }
    return T;
  };
  auto add = [&](const Terms &T) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (j < J) di[j] += T.fc * T.a[j] * T.v[j];
#pragma unroll
    for (int j = 0; j < 2; ++j)
      if (lane + 64 * j < E) de[j] += T.fc * T.ae[j] * T.y[j];
  };
  for_active_pairs(inc_off[n], inc_off[n + 1], iact, iother, lane, [&](int e1, int o1, int e2, int o2, bool two) {
    const Terms A = load(e1, o1), B = load(e2, o2);
    add(A);
    if (two) add(B);
  });
  double v[4], y[4], h[4], is;
  for (int j = 0; j < J; ++j) v[j] = x[std::size_t(n) * F + lane + 64 * j] + di[j];
  g_norm_row(F, mode, v, lnw, lnb, eps, lane, y, h, is);
  for (int j = 0; j < J; ++j) {
    const std::size_t i = std::size_t(n) * F + lane + 64 * j;
    n1[i] = y[j];
    n1hat[i] = h[j];
    act[i] = gsilu(y[j]);
  }
  if (lane == 0) n1is[n] = is;
  for (int j = 0; j < 2; ++j) {
    const int c = lane + 64 * j;
    if (c < E) aev[std::size_t(n) * E + c] = ev[std::size_t(n) * E + c] + de[j];
  }
}

// Interaction input: cat[n][F + s] = sum_{c in slot s} aev_c^2 cg_c
// (kokkos_post_attention_block0.cpp:302-333).
__global__ void g_cat_inv(GDims d, int N, const double *__restrict__ aev, const double *__restrict__ cg,
                          double *__restrict__ cat) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= N * d.NH) return;
  const int n = t / d.NH, s = t % d.NH;
  double acc = 0.0;
  for (int c = d.off[s]; c < d.off[s + 1]; ++c) {
    const double a = aev[std::size_t(n) * d.E + c];
    acc += a * a * cg[c];
  }
  cat[std::size_t(n) * d.NI + d.F + s] = acc;
}

// Block output: x' = norm2(p + t[0:F]), ev' = aev (1 + t[F + slot]).
__global__ __launch_bounds__(256) void g_node_post(GDims d, int N, const double *__restrict__ cat,
                                                   const double *__restrict__ tout, const double *__restrict__ aev,
                                                   const double *__restrict__ lnw, const double *__restrict__ lnb,
                                                   double eps, int mode, double *__restrict__ xout,
                                                   double *__restrict__ evout, double *__restrict__ pre2hat,
                                                   double *__restrict__ pre2is) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const int F = d.F, J = F >> 6;
  const std::size_t r = std::size_t(n) * d.NI;
  double v[4], y[4], h[4], is;
  for (int j = 0; j < J; ++j) v[j] = cat[r + lane + 64 * j] + tout[r + lane + 64 * j];
  g_norm_row(F, mode, v, lnw, lnb, eps, lane, y, h, is);
  for (int j = 0; j < J; ++j) {
    const std::size_t i = std::size_t(n) * F + lane + 64 * j;
    xout[i] = y[j];
    pre2hat[i] = h[j];
  }
  if (lane == 0) pre2is[n] = is;
  for (int j = 0; j < 2; ++j) {
    const int c = lane + 64 * j;
    if (c < d.E) evout[std::size_t(n) * d.E + c] = aev[std::size_t(n) * d.E + c] * (1.0 + tout[r + F + d.slot[c]]);
  }
}

// Output heads from their hidden activations (kokkos_output_heads.cpp:137-176):
// energy (HK), charge (HK), Hirshfeld and C6 ratio keys (64 each).
__global__ __launch_bounds__(256) void g_heads(GDims d, int N, const int *__restrict__ z, const double *__restrict__ hact,
                                               const double *__restrict__ hkey, GHeads H, double *__restrict__ eatom,
                                               double *__restrict__ qraw, double *__restrict__ heff,
                                               double *__restrict__ hir, double *__restrict__ c6eff,
                                               double *__restrict__ c6r) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const double *a = hact + std::size_t(n) * d.HO;
  double e = 0.0, q = 0.0;
  for (int c = lane; c < d.HK; c += 64) {
    e += H.ew2[c] * a[c];
    q += H.qw2[c] * a[d.HK + c];
  }
  e = wsum(e);
  q = wsum(q);
  const int zz = z[n];
  const double hk = wsum(H.hqemb[zz * 64 + lane] * hkey[std::size_t(n) * 128 + lane]);
  const double ck = d.c6 ? wsum(H.cqemb[zz * 64 + lane] * hkey[std::size_t(n) * 128 + 64 + lane]) : 0.0;
  if (lane == 0) {
    eatom[n] = (e + H.eb2) * H.escale[zz - 1] + H.eshift[zz - 1];
    qraw[n] = q + H.qb2 + H.qemb[zz];
    const double hv = H.hvshift[zz] + hk / 8.0;  // q . k / sqrt(64)
    heff[n] = hv;
    hir[n] = fabs(hv);
    if (d.c6) {
      const double cv = H.cvshift[zz] + ck / 8.0;
      c6eff[n] = cv;
      c6r[n] = fabs(cv);
    }
  }
}

// Heads in reverse to the adjoint of their hidden pre-activations
// (kokkos_output_heads.cpp:182-220): energy seed 1, charge seed qseed,
// Hirshfeld dE/dh, C6 dE/dc.
__global__ __launch_bounds__(256) void g_heads_bwd(GDims d, int N, const int *__restrict__ z,
                                                   const double *__restrict__ hpre, const double *__restrict__ qseed,
                                                   const double *__restrict__ dh, const double *__restrict__ heff,
                                                   const double *__restrict__ dc, const double *__restrict__ c6eff,
                                                   GHeads H, double *__restrict__ ghead) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const int zz = z[n], HK = d.HK;
  const double *pre = hpre + std::size_t(n) * d.HO;
  double *g = ghead + std::size_t(n) * d.HO;
  const double es = H.escale[zz - 1], qs = qseed[n];
  for (int c = lane; c < HK; c += 64) {
    g[c] = es * H.ew2[c] * gsilu_prime(pre[c]);
    g[HK + c] = qs * H.qw2[c] * gsilu_prime(pre[HK + c]);
  }
  auto ratio = [&](double seed, double logit, const double *qemb, const double *w2, int at) {
    const double sg = logit > 0.0 ? 1.0 : (logit < 0.0 ? -1.0 : 0.0);
    const double s = seed * sg / 8.0;
    double acc = 0.0;  // sum_j W2[j][lane] q_emb[z][j] s
    for (int j = 0; j < 64; ++j) acc += w2[j * 64 + lane] * (s * qemb[zz * 64 + j]);
    g[at + lane] = acc * gsilu_prime(pre[at + lane]);
  };
  ratio(dh[n], heff[n], H.hqemb, H.hw2, 2 * HK);
  if (d.c6) ratio(dc[n], c6eff[n], H.cqemb, H.cw2, 2 * HK + 64);
}

// Reverse of the second normalisation and the ev gate (kokkos_post_attention_reverse.cpp):
// gt[0:F] = dnorm2, gt[F + s] = sum_{c in s} gev_c aev_c, ga = gev (1 + t[F + slot]).
__global__ __launch_bounds__(256) void g_ln2_bwd(GDims d, int N, const double *__restrict__ gx,
                                                 const double *__restrict__ gev, const double *__restrict__ tout,
                                                 const double *__restrict__ aev, const double *__restrict__ pre2hat,
                                                 const double *__restrict__ pre2is, const double *__restrict__ lnw,
                                                 int mode, double *__restrict__ gt, double *__restrict__ ga) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const int F = d.F, J = F >> 6;
  double gy[4], h[4], gxo[4];
  for (int j = 0; j < J; ++j) {
    gy[j] = gx[std::size_t(n) * F + lane + 64 * j];
    h[j] = pre2hat[std::size_t(n) * F + lane + 64 * j];
  }
  g_norm_row_bwd(F, mode, gy, lnw, h, pre2is[n], lane, gxo);
  const std::size_t r = std::size_t(n) * d.NI;
  for (int j = 0; j < J; ++j) gt[r + lane + 64 * j] = gxo[j];
  if (lane < d.NH) {
    double acc = 0.0;
    for (int c = d.off[lane]; c < d.off[lane + 1]; ++c) acc += gev[std::size_t(n) * d.E + c] * aev[std::size_t(n) * d.E + c];
    gt[r + F + lane] = acc;
  }
  for (int j = 0; j < 2; ++j) {
    const int c = lane + 64 * j;
    if (c < d.E) ga[std::size_t(n) * d.E + c] = gev[std::size_t(n) * d.E + c] * (1.0 + tout[r + F + d.slot[c]]);
  }
}

// gp = gt[0:F] + gcat[0:F]; ga += gcat[F + slot] 2 aev cg.
__global__ void g_cat_bwd(GDims d, int N, const double *__restrict__ gt, const double *__restrict__ gcat,
                          const double *__restrict__ aev, const double *__restrict__ cg, double *__restrict__ gp,
                          double *__restrict__ ga) {
  const std::size_t t = std::size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int W = d.F + d.E;
  if (t >= std::size_t(N) * W) return;
  const int n = int(t / W), c = int(t % W);
  const std::size_t r = std::size_t(n) * d.NI;
  if (c < d.F) {
    gp[std::size_t(n) * d.F + c] = gt[r + c] + gcat[r + c];
  } else {
    const int m = c - d.F;
    const std::size_t i = std::size_t(n) * d.E + m;
    ga[i] += gcat[r + d.F + d.slot[m]] * 2.0 * aev[i] * cg[m];
  }
}

__global__ __launch_bounds__(256) void g_ln1_bwd(int F, int N, const double *__restrict__ gn1,
                                                 const double *__restrict__ lnw, const double *__restrict__ n1hat,
                                                 const double *__restrict__ n1is, int mode, double *__restrict__ gainv) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const int J = F >> 6;
  double gy[4], h[4], go[4];
  for (int j = 0; j < J; ++j) {
    gy[j] = gn1[std::size_t(n) * F + lane + 64 * j];
    h[j] = n1hat[std::size_t(n) * F + lane + 64 * j];
  }
  g_norm_row_bwd(F, mode, gy, lnw, h, n1is[n], lane, go);
  for (int j = 0; j < J; ++j) gainv[std::size_t(n) * F + lane + 64 * j] = go[j];
}

// The attention reverse's node gathers (kokkos_attention_scatter_reverse.cpp:280-500):
// dq at the receiver, dk and dv at the sender of each direction.  One
// wavefront per node and 64 channels (F / 64 wavefronts per node, in one
// workgroup): a lane holds one channel's five sums, so a wavefront needs
// few registers and many are in flight to cover the entries' loads.
__global__ __launch_bounds__(256) void g_attn_bwd_node(GDims d, int N, const int *__restrict__ inc_off,
                                                       const int *__restrict__ iact, const int *__restrict__ iother,
                                                       const double *__restrict__ qkv, const double *__restrict__ pf,
                                                       const double *__restrict__ pfc,
                                                       const double *__restrict__ palpha,
                                                       const double *__restrict__ psc,
                                                       const double *__restrict__ gainv, double *__restrict__ gqkv) {
  const int lane = threadIdx.x & 63;
  const int F = d.F, NH = d.NH, NQ = F >> 6;
  const int blk = g_xcd_block((N * NQ + 3) / 4);
  if (blk < 0) return;
  const int wq = blk * 4 + (threadIdx.x >> 6), n = wq / NQ;
  if (n >= N) return;
  const int c = 64 * (wq % NQ) + lane, h = c >> 5;
  double gq = 0.0, gk = 0.0, gv = 0.0, gqe = 0.0, gke = 0.0;
  // per entry: n receives along direction sn from o and sends along
  // so = 1 - sn to o
  struct Terms {
    double si, sie, so, soe, ao, fi, fe, qo, ko, qeo, keo, go, fc;
  };
  auto load = [&](int e, int o) {
    Terms T;
    const int p = e >> 1, sn = e & 1, so = 1 - sn;
    T.fc = pfc[p];
    const double *sc = psc + std::size_t(p) * 4 * NH;
    const double *al = palpha + std::size_t(p) * 4 * NH;
    const double *fi = pf + std::size_t(p) * 2 * F;
    const double *qo = qkv + std::size_t(o) * 5 * F;
    T.si = sc[sn * 2 * NH + h];
    T.sie = sc[sn * 2 * NH + NH + h];
    T.so = sc[so * 2 * NH + h];
    T.soe = sc[so * 2 * NH + NH + h];
    T.ao = al[so * 2 * NH + h];
    T.fi = fi[c];
    T.fe = fi[F + c];
    T.qo = qo[c];
    T.ko = qo[F + c];
    T.qeo = qo[3 * F + c];
    T.keo = qo[4 * F + c];
    T.go = gainv[std::size_t(o) * F + c];
    return T;
  };
  auto add = [&](const Terms &T) {
    gq += T.si * T.ko * T.fi;
    gqe += T.sie * T.keo * T.fe;
    gk += T.so * T.qo * T.fi;
    gv += T.fc * T.ao * T.go;
    gke += T.soe * T.qeo * T.fe;
  };
  for_active_pairs(inc_off[n], inc_off[n + 1], iact, iother, lane, [&](int e1, int o1, int e2, int o2, bool two) {
    const Terms A = load(e1, o1), B = load(e2, o2);
    add(A);
    if (two) add(B);
  });
  double *g = gqkv + std::size_t(n) * 5 * F + c;
  g[0] = gq;
  g[F] = gk;
  g[2 * F] = gv;
  g[3 * F] = gqe;
  g[4 * F] = gke;
}

// gev = ga + sum over incident pairs of 2 (ev_n - ev_o) cg ds[slot]: the
// edge invariants' adjoint (kokkos_block2_attention_input_reverse.cpp:144-196).
__global__ __launch_bounds__(256) void g_ev_bwd(GDims d, int N, const int *__restrict__ inc_off,
                                                const int *__restrict__ iact, const int *__restrict__ iother,
                                                const double *__restrict__ ev, const double *__restrict__ cg,
                                                const double *__restrict__ ds, const double *__restrict__ ga,
                                                double *__restrict__ gev) {
  const int lane = threadIdx.x & 63;
  const int blk = g_xcd_block((N + 3) / 4);
  if (blk < 0) return;
  const int n = blk * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const int E = d.E;
  for (int j = 0; j < 2; ++j) {
    const int c = lane + 64 * j;
    if (c >= E) continue;
    const int sl = d.slot[c];
    const double en = ev[std::size_t(n) * E + c];
    double acc = ga[std::size_t(n) * E + c];
    for (int k = inc_off[n]; k < inc_off[n + 1]; ++k) {
      const int e = iact[k];
      if (e < 0) continue;
      acc += 2.0 * (en - ev[std::size_t(iother[k]) * E + c]) * cg[c] * ds[std::size_t(e >> 1) * d.NH + sl];
    }
    gev[std::size_t(n) * E + c] = acc;
  }
}

// ------------------------------------------------------------- pair kernels
// Bernstein basis of the distance (kokkos_integrated_block0.cpp:117-164), one
// thread per active pair.
__global__ void g_rbf(int R, const int *nact, int cap, const double *__restrict__ pr, double gamma,
                      const double *__restrict__ b, const double *__restrict__ kk, const double *__restrict__ kr,
                      double *__restrict__ rbf) {
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= min(*nact, cap)) return;
  double xb = exp(-gamma * pr[p]);
  xb = xb < 1e-6 ? 1e-6 : (xb > 1.0 - 1e-6 ? 1.0 - 1e-6 : xb);
  const double lx = log(xb), l1x = log(1.0 - xb);
  for (int k = 0; k < R; ++k) rbf[std::size_t(p) * R + k] = exp(b[k] + kk[k] * lx + kr[k] * l1x);
}

// Equivariant invariants per slot: s = sum_{c in slot} (ev_a - ev_b)^2 cg
// (kokkos_integrated_block0.cpp:166-195).
__global__ void g_pair_inv(GDims d, const int *nact, int cap, const int *__restrict__ pa,
                           const double *__restrict__ ev, const double *__restrict__ cg, double *__restrict__ ps) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  const int p = t / d.NH, s = t % d.NH;
  if (p >= min(*nact, cap)) return;
  const double *ea = ev + std::size_t(pa[2 * p]) * d.E, *eb = ev + std::size_t(pa[2 * p + 1]) * d.E;
  double acc = 0.0;
  for (int c = d.off[s]; c < d.off[s + 1]; ++c) {
    const double x = ea[c] - eb[c];
    acc += x * x * cg[c];
  }
  ps[std::size_t(p) * d.NH + s] = acc;
}

// M sums over each 32-lane half of a wavefront at once (M = 2, 4, 8 or 16
// values per lane, v[0..M)): at each of the first log2 M butterfly steps a
// lane keeps half of its values, sends the other half to its partner and adds
// the partner's copy of the half it kept (lane bit 4, then 3, ...: a set bit
// keeps the upper half); the remaining steps add the single value left.
// Lane l of half H = l / 32 ends with the sum of value index
// (l % 32) >> (5 - log2 M) of its half, the same in each run of 32 / M lanes;
// M - 1 + 5 - log2 M exchanges instead of 5 M.
template <int W, int MASK, int M>
__device__ __forceinline__ void half_sums_step(double (&v)[M], int lane) {
  if constexpr (W > 1) {
    constexpr int H = W / 2;
    const bool up = (lane & MASK) != 0;
#pragma unroll
    for (int i = 0; i < H; ++i) {
      const double send = up ? v[i] : v[H + i];
      const double keep = up ? v[H + i] : v[i];
      v[i] = keep + __shfl_xor(send, MASK, 64);
    }
    half_sums_step<H, MASK / 2, M>(v, lane);
  } else if constexpr (MASK > 0) {
    v[0] += __shfl_xor(v[0], MASK, 64);
    half_sums_step<1, MASK / 2, M>(v, lane);
  }
}
template <int M>
__device__ __forceinline__ double half_sums(double (&v)[M], int lane) {
  static_assert(M == 2 || M == 4 || M == 8 || M == 16, "half_sums takes 2, 4, 8 or 16 values");
  half_sums_step<M, 16, M>(v, lane);
  return v[0];
}

// Attention reverse, pair side (kokkos_attention_scatter_reverse.cpp:280-500),
// one wavefront per pair, both directions: with r the receiver and s the
// sender of a direction,
//   ci_h = <gainv_r, v_s>_head h,  ce_h = <gaev_r, Y'>_slot h  (Y' the
//   direction's harmonics), psc = fc c norm (the logits' adjoints, kept for
//   the node gathers and the filters' reverse, which forms the filter
//   adjoint df = sum_dir psc q_r k_s (inv) and psc_ev q_ev_r k_ev_s (ev)),
//   dE/dfc = sum ci alpha + ce alpha_ev,
//   dE/dY_m = sum_dir sum_{c: sh(c) = m} gaev_r,c fc alpha_ev par (side-0
//   orientation); the first reverse block writes dY, the others add.
// The head sums ci come from half_sums over the 2 J products of a lane
// (direction, j); the slot sums ce from the wavefront's own LDS rows, one
// lane per direction and slot.  Each wavefront uses only its own LDS rows, so
// a wavefront-level fence orders them and an idle wavefront leaves at once.
template <int J>
__global__ __launch_bounds__(256) void g_attn_bwd_pairs(GDims d, const int *nact, int cap, const int *__restrict__ pa,
                                                        const double *__restrict__ qkv, const double *__restrict__ pY,
                                                        const double *__restrict__ pfc,
                                                        const double *__restrict__ palpha,
                                                        const double *__restrict__ gainv,
                                                        const double *__restrict__ ga, double inv_avg, int first,
                                                        double *__restrict__ psc, double *__restrict__ dY,
                                                        double *__restrict__ dfc) {
  __shared__ double lt[4][2][kGMaxE];   // per wavefront: dE/dY terms per direction and channel
  __shared__ double lte[4][2][kGMaxE];  // per wavefront: gaev_r Y' per direction and channel
  __shared__ double lps[4][32];         // per wavefront: psc of the pair
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int blk = g_xcd_block((min(*nact, cap) + 3) / 4);
  if (blk < 0) return;
  const int p = blk * 4 + wv;
  if (p >= min(*nact, cap)) return;
  const int NH = d.NH, F = d.F, E = d.E;
  const double fc = pfc[p];
  const double *al = palpha + std::size_t(p) * 4 * NH;
  double v[2 * J];
#pragma unroll
  for (int side = 0; side < 2; ++side) {
    const int rcv = pa[2 * p + side], snd = pa[2 * p + 1 - side];
    const double *g = gainv + std::size_t(rcv) * F, *vs = qkv + std::size_t(snd) * 5 * F + 2 * F;
#pragma unroll
    for (int j = 0; j < J; ++j) v[side * J + j] = g[lane + 64 * j] * vs[lane + 64 * j];
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int c = lane + 64 * jj;
      if (c < E) {
        const int sl = d.slot[c];
        const double pr = side ? d.par[sl] : 1.0;
        const double gr = ga[std::size_t(rcv) * E + c];
        lte[wv][side][c] = gr * pY[std::size_t(p) * 24 + d.sh[c]] * pr;
        lt[wv][side][c] = gr * fc * al[side * 2 * NH + NH + sl] * pr;
      }
    }
  }
  const double ci = half_sums<2 * J>(v, lane);
  constexpr int RUN = 32 >> (J == 2 ? 2 : 3);
  double part = 0.0;  // this lane's terms of dE/dfc
  if (lane % RUN == 0) {
    const int m = (lane & 31) / RUN, j = m % J, side = m / J, h = 2 * j + (lane >> 5);
    part = ci * al[side * 2 * NH + h];
    lps[wv][side * 2 * NH + h] = fc * ci * inv_avg;
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  if (lane < 2 * NH) {
    const int side = lane / NH, sl = lane % NH;
    double ce = 0.0;
    for (int c = d.off[sl]; c < d.off[sl + 1]; ++c) ce += lte[wv][side][c];
    part += ce * al[side * 2 * NH + NH + sl];
    lps[wv][side * 2 * NH + NH + sl] = fc * ce * inv_avg;
  }
  const double dsum = wsum(part);
  if (lane == 0) dfc[p] = dsum;
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  if (lane < 4 * NH) psc[std::size_t(p) * 4 * NH + lane] = lps[wv][lane];
  if (lane < 24) {
    double acc = 0.0;
    for (int side = 0; side < 2; ++side)
      for (int t = 0; t < d.shn[lane]; ++t) acc += lt[wv][side][d.shc[lane][t]];
    double *y = dY + std::size_t(p) * 24 + lane;
    *y = first ? acc : *y + acc;
  }
}

// Block 0 through element-pair tables (the algebra of evaluator.hip's
// k_class_tables, at generic widths): block 0's q, k rows depend on the
// element alone in a one-image system, and its filter outputs enter only the
// logits <q_a (.) k_b, f>_h, f = W1 hidden + bias with s = 0 (the spherical
// hidden row is silu(eb0) for every pair).  Per filter w and key (lo, hi)
// (key lo C + hi; the keys with lo > hi go unused) the 2 NH table rows
//   M[r][f] = sum_{c in head h} W1_w[c][f] q_A[c] k_B[c]
//   cb[r]   = sum_{c in head h} (b1 + e1 + E1 silu(e0))[c] q_A[c] k_B[c]
// with (A, B, h) = (lo, hi, r) for r < NH and (hi, lo, r - NH) after make
// the logits of a pair M hidden + cb, and its hidden adjoint M^T times the
// logits' adjoints.  The rows go out as MFMA A operands, zero-padded to 16
// rows (2 NH = F / 16 <= 16):
//   tf[w][key][T][lane][v] = M[lane % 16][16 T + lane / 16 + 4 v]  (rows r)
//   tr[w][key][T][lane][v] = M[lane / 16 + 4 v][16 T + lane % 16]  (rows f)
// and cb[w][key][r].  One block per (key, r < 16) and filter; thread f.
__global__ __launch_bounds__(256) void g_cls_tables(int F, int NH, int FH, int C, const double *__restrict__ qkv,
                                                    const int *__restrict__ rep, const double *__restrict__ wcat0,
                                                    const double *__restrict__ wcat1,
                                                    const double *__restrict__ bcat0,
                                                    const double *__restrict__ bcat1,
                                                    const double *__restrict__ eb00,
                                                    const double *__restrict__ eb01, double *__restrict__ tf,
                                                    double *__restrict__ tr, double *__restrict__ cb) {
  const int w = blockIdx.y, key = blockIdx.x / 16, r = blockIdx.x % 16;
  const int lo = key / C, hi = key % C, h = r % NH;
  const int A = r < NH ? lo : hi, B = r < NH ? hi : lo;
  const bool live = r < 2 * NH;
  const int f = threadIdx.x, HW = F + FH, FT = F / 16;
  const double *wc = w ? wcat1 : wcat0;
  __shared__ double qk[32], tb[32];
  if (live && f < 32) {
    const double *qa = qkv + std::size_t(rep[A]) * 5 * F + (w ? 3 * F : 0);
    const double *kb = qkv + std::size_t(rep[B]) * 5 * F + (w ? 4 * F : F);
    const int c = 32 * h + f;
    qk[f] = qa[c] * kb[c];
    // the output bias of channel c with the spherical branch at s = 0
    const double *eb0 = w ? eb01 : eb00;
    double bias = (w ? bcat1 : bcat0)[c];
    for (int j = 0; j < FH; ++j) bias += wc[std::size_t(c) * HW + F + j] * gsilu(eb0[j]);
    tb[f] = bias * qk[f];
  }
  __syncthreads();
  const std::size_t wk = std::size_t(w) * C * C + key;
  if (f < F) {
    double acc = 0.0;
    if (live)
      for (int k = 0; k < 32; ++k) acc += wc[std::size_t(32 * h + k) * HW + f] * qk[k];
    const int T = f / 16, fi = f % 16;
    tf[((wk * FT + T) * 64 + r + 16 * (fi % 4)) * 4 + fi / 4] = acc;
    tr[((wk * FT + T) * 64 + fi + 16 * (r % 4)) * 4 + r / 4] = acc;
  }
  if (live && f == 0) {
    double sum = 0.0;
    for (int k = 0; k < 32; ++k) sum += tb[k];
    cb[wk * 2 * NH + r] = sum;
  }
}

// Block 0's filters through the tables, fused: per pair and filter the
// hidden row silu(W0 rbf + b0) stays in registers, its logits are one MFMA
// chain per hidden tile against the table rows; in reverse the hidden
// adjoint is the table rows times the logits' adjoints, then through
// silu'(pre) (pre recomputed) and W0^T to the basis adjoint, and dE/dr from
// it and the cutoff's adjoint.  The layout of evaluator.hip's MFMA filters: features
// as rows, 16 pairs per column tile, a tile's D registers the next layer's B
// operand (feature 16 T + g + 4 r of pair lane % 16 in lane group g,
// register r).  FT = F / 16 hidden tiles, RT = R / 16 basis chunks, NH =
// FT / 2 heads (F = 32 NH), so the 2 NH table rows fit one MFMA tile.
// The slots run in element-pair order, each bucket padded with -1 to a
// multiple of 32: a wavefront's CT column tiles (16 CT <= 32 slots) are of
// one key, whose table rows every lane reads, and its first slot holds a
// pair unless the whole wavefront is padding.
struct B0Args {
  const int *slots, *order, *pa, *z, *cls;
  int C;
  const double *pr, *rbf;               // distance; basis rows (R per pair)
  const double *w0p[2], *w0tp[2], *b0a[2];
  const double *tf, *tr, *cb;           // g_cls_tables
  const double *exp2_256, *kk, *kr;
  double gamma, rc, inv_avg;
  double *palpha;                       // forward: the logits (4 NH per pair)
  const double *psc, *dfc;              // reverse: the logits' and the cutoff's adjoints
  double *dr;                           // reverse: dE/dr (added to)
};

// The wavefront's slots: pair p[ct] of column tile ct (padding: the first
// slot's pair, with ok false), its orientation sw[ct] (classes (hi, lo)),
// the key, and the lane's basis values rb[ct][Kc][v] = rbf_k,
// k = 16 Kc + g + 4 v.  False: no pair in the wavefront.
template <int RT, int CT>
__device__ __forceinline__ bool b0_slots(const B0Args &A, int wave, int j, int g, int *p, bool *ok, bool *sw,
                                         int &key, v4d (*rb)[RT]) {
  const int q0 = wave * 16 * CT;
  if (q0 >= *A.slots) return false;
  const int p0 = __builtin_amdgcn_readfirstlane(A.order[q0]);
  if (p0 < 0) return false;
  const int ca = A.cls[A.z[A.pa[2 * p0]]], cbb = A.cls[A.z[A.pa[2 * p0 + 1]]];
  key = __builtin_amdgcn_readfirstlane(ca < cbb ? ca * A.C + cbb : cbb * A.C + ca);
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const int e = A.order[q0 + 16 * ct + j];
    ok[ct] = e >= 0;
    p[ct] = ok[ct] ? e : p0;
    sw[ct] = A.cls[A.z[A.pa[2 * p[ct]]]] > A.cls[A.z[A.pa[2 * p[ct] + 1]]];
    const double *row = A.rbf + std::size_t(p[ct]) * 16 * RT + g;
#pragma unroll
    for (int Kc = 0; Kc < RT; ++Kc)
#pragma unroll
      for (int v = 0; v < 4; ++v) rb[ct][Kc][v] = row[16 * Kc + 4 * v];
  }
  return true;
}

#ifndef SO3LR_B0_FWD_CT
#define SO3LR_B0_FWD_CT 2
#endif
#ifndef SO3LR_B0_BWD_CT
#define SO3LR_B0_BWD_CT 1
#endif
#ifndef SO3LR_B0_PF
#define SO3LR_B0_PF 6
#endif

// Forward: per filter the stream holds, per hidden tile T, the bias tile,
// the RT W0 chunks and the table rows of tile T - 1 (whose SiLU runs after
// tile T's first MFMA, off the critical path), then the last tile's rows.
template <int FT, int RT, int CT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void g_b0_fwd(B0Args A) {
  constexpr int NH = FT / 2, NT = FT * (RT + 2);
  __shared__ double tab[256];
  tab[threadIdx.x] = A.exp2_256[threadIdx.x];
  __syncthreads();
  const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(int(blockIdx.x) * 4 + int(threadIdx.x >> 6));
  int p[CT], key = 0;
  bool ok[CT], sw[CT];
  v4d rb[CT][RT];
  if (!b0_slots<RT, CT>(A, wave, j, g, p, ok, sw, key, rb)) return;
  const std::size_t NK = std::size_t(A.C) * A.C;
  const double *tfw[2] = {A.tf + std::size_t(key) * FT * 256, A.tf + (NK + key) * FT * 256};
  auto load = [&](auto si) -> v4d {
    constexpr int S = decltype(si)::value, w = S / NT, s = S % NT;
    constexpr int T = s < RT + 1 ? 0 : 1 + (s - RT - 1) / (RT + 2);
    constexpr int u = s < RT + 1 ? s : (s - RT - 1) % (RT + 2);
    if constexpr (T == FT) return frag_load(tfw[w], FT - 1, lane);
    else if constexpr (u == 0) return frag_load(A.b0a[w], T, lane);
    else if constexpr (u <= RT) return frag_load(A.w0p[w], T * RT + u - 1, lane);
    else return frag_load(tfw[w], T - 1, lane);
  };
  Stream<2 * NT, SO3LR_B0_PF, decltype(load)> st(load);
  st.prime();
  v4d pre[2][CT], h[CT], lg[CT];
  st.run([&](auto si, const v4d &wv) {
    constexpr int S = decltype(si)::value, w = S / NT, s = S % NT;
    constexpr int T = s < RT + 1 ? 0 : 1 + (s - RT - 1) / (RT + 2);
    constexpr int u = s < RT + 1 ? s : (s - RT - 1) % (RT + 2);
    if constexpr (s == 0) {
      // the logits start from the table biases (rows r = g + 4 rr)
      const double *cbw = A.cb + (w * NK + key) * 2 * NH;
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) lg[ct][rr] = g + 4 * rr < 2 * NH ? cbw[g + 4 * rr] : 0.0;
    }
    if constexpr (T == FT) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) h[ct][rr] = silu_tab(pre[(FT - 1) % 2][ct][rr], tab);
        lg[ct] = mfma4(wv, h[ct], lg[ct]);
      }
      // row r < NH: the logit of (lo, hi) head r, the receiver's side unless
      // the pair runs (hi, lo)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int r = g + 4 * rr;
          if (r < 2 * NH && ok[ct]) {
            const int side = (r >= NH) != sw[ct] ? 1 : 0;
            A.palpha[std::size_t(p[ct]) * 4 * NH + side * 2 * NH + w * NH + r % NH] = lg[ct][rr] * A.inv_avg;
          }
        }
    } else if constexpr (u == 0) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) pre[T % 2][ct] = wv;
    } else if constexpr (u <= RT) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) pre[T % 2][ct] = mfma4(wv, rb[ct][u - 1], pre[T % 2][ct]);
      if constexpr (u == 1 && T > 0) {
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) h[ct][rr] = silu_tab(pre[(T - 1) % 2][ct][rr], tab);
      }
    } else {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) lg[ct] = mfma4(wv, h[ct], lg[ct]);
    }
  });
}

// Reverse: per filter the stream holds, per hidden tile T, the bias tile,
// the table rows (d hidden = rows^T coefficients), the RT W0 chunks (pre
// again; silu' of tile T - 1 after the first) and the RT W0^T chunks of tile
// T - 1 (d rbf += W0^T d hidden), then the last tile's W0^T chunks.
template <int FT, int RT, int CT>
// Two wavefronts per SIMD, 16 pairs each: at F = 256, R = 64 (config 3)
// 1.25 ms, against 1.38 for 32 pairs at one wavefront per SIMD.
#ifndef SO3LR_B0_BWD_WAVES
#define SO3LR_B0_BWD_WAVES 2
#endif
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(SO3LR_B0_BWD_WAVES, SO3LR_B0_BWD_WAVES))) void
g_b0_bwd(B0Args A) {
  constexpr int NH = FT / 2, NB = FT * (2 + 2 * RT);
  __shared__ double tab[256];
  tab[threadIdx.x] = A.exp2_256[threadIdx.x];
  __syncthreads();
  const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(int(blockIdx.x) * 4 + int(threadIdx.x >> 6));
  int p[CT], key = 0;
  bool ok[CT], sw[CT];
  v4d rb[CT][RT];
  if (!b0_slots<RT, CT>(A, wave, j, g, p, ok, sw, key, rb)) return;
  const std::size_t NK = std::size_t(A.C) * A.C;
  const double *trw[2] = {A.tr + std::size_t(key) * FT * 256, A.tr + (NK + key) * FT * 256};
  // the B operand of the table product: row r = g + 4 v's logit adjoint
  v4d cf[2][CT];
#pragma unroll
  for (int w = 0; w < 2; ++w)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int r = g + 4 * v;
        const int side = (r >= NH) != sw[ct] ? 1 : 0;
        cf[w][ct][v] = r < 2 * NH ? A.psc[std::size_t(p[ct]) * 4 * NH + side * 2 * NH + w * NH + r % NH] : 0.0;
      }
  auto load = [&](auto si) -> v4d {
    constexpr int S = decltype(si)::value, w = S / NB, s = S % NB;
    constexpr int T = s < RT + 2 ? 0 : 1 + (s - RT - 2) / (2 * RT + 2);
    constexpr int u = s < RT + 2 ? s : (s - RT - 2) % (2 * RT + 2);
    if constexpr (T == FT) return frag_load(A.w0tp[w], u * FT + FT - 1, lane);
    else if constexpr (u == 0) return frag_load(A.b0a[w], T, lane);
    else if constexpr (u == 1) return frag_load(trw[w], T, lane);
    else if constexpr (u < RT + 2) return frag_load(A.w0p[w], T * RT + u - 2, lane);
    else return frag_load(A.w0tp[w], (u - RT - 2) * FT + T - 1, lane);
  };
  Stream<2 * NB, SO3LR_B0_PF, decltype(load)> st(load);
  st.prime();
  const v4d zero = v4d{0.0, 0.0, 0.0, 0.0};
  v4d pre[2][CT], gh[2][CT], drb[CT][RT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct)
#pragma unroll
    for (int Kc = 0; Kc < RT; ++Kc) drb[ct][Kc] = zero;
  auto dsilu = [&](int t) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) gh[t][ct][rr] *= silu_prime_tab(pre[t][ct][rr], tab);
  };
  st.run([&](auto si, const v4d &wv) {
    constexpr int S = decltype(si)::value, w = S / NB, s = S % NB;
    constexpr int T = s < RT + 2 ? 0 : 1 + (s - RT - 2) / (2 * RT + 2);
    constexpr int u = s < RT + 2 ? s : (s - RT - 2) % (2 * RT + 2);
    if constexpr (T == FT) {
      if constexpr (u == 0) dsilu((FT - 1) % 2);
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) drb[ct][u] = mfma4(wv, gh[(FT - 1) % 2][ct], drb[ct][u]);
    } else if constexpr (u == 0) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) pre[T % 2][ct] = wv;
    } else if constexpr (u == 1) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        // rows r >= 2 NH are zero: two MFMAs cover the 8 rows of NH = 4
        v4d acc = mfma(wv[0], cf[w][ct][0], zero);
        acc = mfma(wv[1], cf[w][ct][1], acc);
        if constexpr (2 * NH > 8) {
          acc = mfma(wv[2], cf[w][ct][2], acc);
          acc = mfma(wv[3], cf[w][ct][3], acc);
        }
        gh[T % 2][ct] = acc;
      }
    } else if constexpr (u < RT + 2) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) pre[T % 2][ct] = mfma4(wv, rb[ct][u - 2], pre[T % 2][ct]);
      if constexpr (u == 2 && T > 0) dsilu((T - 1) % 2);
    } else {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
        drb[ct][u - RT - 2] = mfma4(wv, gh[(T - 1) % 2][ct], drb[ct][u - RT - 2]);
    }
  });
  // dE/dr: the basis adjoint against d rbf / dr (zero where the basis
  // variable is clamped), plus the cutoff's
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const double r = A.pr[p[ct]];
    const double xb = exp(-A.gamma * r);
    double part = 0.0;
    if (xb > 1e-6 && xb < 1.0 - 1e-6) {
      const double ratio = xb / (1.0 - xb);
#pragma unroll
      for (int Kc = 0; Kc < RT; ++Kc)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int k = 16 * Kc + g + 4 * rr;
          part += drb[ct][Kc][rr] * rb[ct][Kc][rr] * (-A.gamma * A.kk[k] + A.gamma * ratio * A.kr[k]);
        }
    }
    part += __shfl_xor(part, 16, 64);
    part += __shfl_xor(part, 32, 64);
    if (ok[ct] && g == 0) {
      double grad = part;
      if (r < A.rc) {
        const double t = r / A.rc;
        grad += A.dfc[p[ct]] * (-30.0 * t * t * (1.0 - t) * (1.0 - t) / A.rc);
      }
      A.dr[p[ct]] += grad;
    }
  }
}

// ------------------------------------------------------ block 0, radial tables
// Block 0's logits as polynomials of r per element pair (the algebra of
// evaluator.hip's k_radial_* at generic widths): each filter's radial hidden
// layer h_w(r) is fitted per interval of r (fit_radial_hidden), and the
// 4 NH logits of a pair are <M row, h_w(r)> + cb with g_cls_tables' rows and
// biases.  Table records (mfma_ops.hpp) of L = 4 NH logits, l = 2 NH w + r
// with g_cls_tables' row r (r < NH: lo <- hi, head r; else hi <- lo, head
// r - NH); the value table, then the slope table.

// One block per (element pair {lo <= hi}, interval); threads over (power k,
// logit l): coefficient k of logit l's value and slope polynomials.
__global__ __launch_bounds__(256) void g_radial_tables(int F, int NH, int C, const double *__restrict__ tf,
                                                       const double *__restrict__ cb,
                                                       const double *__restrict__ gval,
                                                       const double *__restrict__ gslope, RadialDomain d,
                                                       double *tval, double *tslope) {
  const int key = int(blockIdx.x) / d.intervals, i = int(blockIdx.x) % d.intervals;
  int lo = 0, start = 0;
  while (start + (C - lo) <= key) start += C - lo++;
  const int hi = lo + (key - start);
  const int L = 4 * NH, FT = F / 16;
  const std::size_t rec = std::size_t(kRadialCoefs) * L;
  for (int t = threadIdx.x; t < kRadialCoefs * L; t += blockDim.x) {
    const int l = t % L, k = t / L;
    const int w = l / (2 * NH), r = l % (2 * NH);
    const std::size_t wk = std::size_t(w) * C * C + std::size_t(lo) * C + hi;
    const double *m = tf + wk * FT * 256;  // row r of (lo, hi) in g_cls_tables' tf order
    const std::size_t g = ((std::size_t(w) * d.intervals + i) * kRadialCoefs + k) * F;
    double av = 0.0, as = 0.0;
    for (int f = 0; f < F; ++f) {
      const int T = f / 16, fi = f % 16;
      const double mf = m[(T * 64 + r + 16 * (fi % 4)) * 4 + fi / 4];
      av += mf * gval[g + f];
      as += mf * gslope[g + f];
    }
    if (k == 0) av += cb[wk * 2 * NH + r];
    const std::size_t o = (std::size_t(key) * d.intervals + i) * rec + (k >> 1) * 2 * L + 2 * l + (k & 1);
    tval[o] = av;
    tslope[o] = as;
  }
}

// Forward: L = 4 NH lanes per pair (logit l), 256 / L pairs per block in
// pair order; the logits (times 1 / avg) where g_b0_fwd writes them.
template <int L>
__global__ __launch_bounds__(256) void g_radial_fwd(const int *n_active, const int *pa, const double *pr,
                                                    const int *__restrict__ z, const int *__restrict__ cls, int C,
                                                    const double *__restrict__ tval, RadialDomain d, double inv_avg,
                                                    double *palpha) {
  constexpr int NH = L / 4, PB = 256 / L;
  const int q = int(blockIdx.x) * PB + int(threadIdx.x) / L, l = int(threadIdx.x) % L;
  if (q >= *n_active) return;  // the pair's L lanes
  const int ca = cls[z[pa[2 * q]]], cb = cls[z[pa[2 * q + 1]]];
  const bool sw = ca > cb;
  double t;
  bool inside;
  const int i = radial_locate(pr[q], d, t, inside);
  const double *rec = tval + (std::size_t(tri_key(sw ? cb : ca, sw ? ca : cb, C)) * d.intervals + i) *
                                 (std::size_t(kRadialCoefs) * L);
  const double v = radial_eval<L>(rec, l, t);
  const int w = l / (2 * NH), r = l % (2 * NH);
  const int side = (r >= NH) != sw ? 1 : 0;  // 0: a <- b
  palpha[std::size_t(q) * 4 * NH + side * 2 * NH + w * NH + r % NH] = v * inv_avg;
}

// Reverse: dE/dr += sum over the pair's logits of their adjoints (psc) times
// the slopes, plus the cutoff's adjoint (dfc) times fc'(r).
template <int L>
__global__ __launch_bounds__(256) void g_radial_bwd(const int *n_active, const int *pa, const double *pr,
                                                    const int *__restrict__ z, const int *__restrict__ cls, int C,
                                                    const double *__restrict__ tslope, RadialDomain d,
                                                    const double *__restrict__ psc, const double *__restrict__ dfc,
                                                    double rc, double *dr) {
  constexpr int NH = L / 4, PB = 256 / L;
  const int q = int(blockIdx.x) * PB + int(threadIdx.x) / L, l = int(threadIdx.x) % L;
  if (q >= *n_active) return;  // the pair's L lanes
  const int ca = cls[z[pa[2 * q]]], cb = cls[z[pa[2 * q + 1]]];
  const bool sw = ca > cb;
  const double r = pr[q];
  double t;
  bool inside;
  const int i = radial_locate(r, d, t, inside);
  const double *rec = tslope + (std::size_t(tri_key(sw ? cb : ca, sw ? ca : cb, C)) * d.intervals + i) *
                                   (std::size_t(kRadialCoefs) * L);
  const double slope = inside ? radial_eval<L>(rec, l, t) : 0.0;
  const int w = l / (2 * NH), row = l % (2 * NH);
  const int side = (row >= NH) != sw ? 1 : 0;
  double part = psc[std::size_t(q) * 4 * NH + side * 2 * NH + w * NH + row % NH] * slope;
#pragma unroll
  for (int o = 1; o < L; o <<= 1) part += __shfl_xor(part, o, L);
  if (l == 0) {
    double grad = part;
    if (r < rc) {
      const double u = r / rc;
      grad += dfc[q] * (-30.0 * u * u * (1.0 - u) * (1.0 - u) / rc);
    }
    dr[q] += grad;
  }
}

// ------------------------------------------------------ fused filters
// Both filters of a block for 16 pairs per wavefront, on fp64 MFMA in the
// layout of the table kernels above (features as rows, the pairs as the 16
// columns, a tile's D registers the next layer's B operand)
// (kokkos_integrated_block0.cpp:198-255 forward,
// kokkos_block2_attention_input_reverse.cpp:198-336 reverse).  FT = F / 16
// hidden tiles of the radial branch and FT / 4 of the spherical one (FH =
// F / 4), RT = R / 16 basis chunks, NH = FT / 2 slots.
//   forward: the hidden row [silu(W0 rbf + b0) | silu(E0 s + e0)] (HT = FT +
//            FT / 4 tiles) in registers, then f = [W1 | E1] hidden + b1 + e1
//            one output tile at a time, stored as the pair's filter row, and
//            the attention logits <q_r, k_s (.) f>_h / avg from each tile;
//   reverse: d hidden = [W1 | E1]^T df, df = psc_0 q_a k_b + psc_1 q_b k_a
//            formed from the logits' adjoints psc (g_attn_bwd_pairs) and the
//            endpoint rows, TG hidden tiles at a time (all of them unless
//            set lower); each group then times silu'(pre) (pre again) and
//            through W0^T to the basis adjoint or E0^T to dE/ds; last dE/dr
//            from the basis adjoint and the cutoff's.
struct FiltArgs {
  const int *nact;
  int cap;
  const int *pa;
  const double *pr, *rbf, *ps, *qkv;                                   // distance, basis rows, s, node rows
  const double *w0p[2], *b0a[2], *e0p[2], *eb0a[2], *wcp[2], *bca[2];  // forward operands
  const double *w0tp[2], *e0tp[2], *wctp[2];                           // reverse operands
  const double *exp2_256, *kk, *kr;
  double gamma, rc, inv_avg;
  double *pf, *palpha;      // forward: filter rows (2 F per pair), logits (4 NH)
  const double *psc, *dfc;  // reverse: the logits' and the cutoff's adjoints
  double *ds, *dr;          // reverse: dE/ds (NH per pair), dE/dr (added to)
};

#ifndef SO3LR_FILT_PF
#define SO3LR_FILT_PF 6
#endif

// the lane's pair (padding lanes: the last active pair, valid false);
// false: the wavefront has no pair
__device__ __forceinline__ bool filt_pair(const FiltArgs &A, int j, int &pp, bool &valid) {
  const int nact = min(*A.nact, A.cap);
  const int blk = g_xcd_block((nact + 63) / 64);
  if (blk < 0) return false;
  const int wave = blk * 4 + int(threadIdx.x >> 6);
  if (wave * 16 >= nact) return false;
  const int p = wave * 16 + j;
  valid = p < nact;
  pp = valid ? p : nact - 1;
  return true;
}
// the pair's basis values rb[Kc][v] = rbf_k (k = 16 Kc + g + 4 v) and
// invariants sv[v] = s_{g + 4 v} (0 beyond NH), the B operands of the
// hidden row's layer 0; loaded where each pass over the hidden row starts
// (from L2 after the first), so they hold no registers in between
template <int RT, int NH>
__device__ __forceinline__ void filt_inputs(const FiltArgs &A, int pp, int g, v4d *rb, v4d &sv) {
  // an opaque copy of the pair index: the loads of one pass are not merged
  // with those of another (which would keep the values live throughout)
  asm volatile("" : "+v"(pp));
  const double *row = A.rbf + std::size_t(pp) * 16 * RT + g;
#pragma unroll
  for (int Kc = 0; Kc < RT; ++Kc)
#pragma unroll
    for (int v = 0; v < 4; ++v) rb[Kc][v] = row[16 * Kc + 4 * v];
#pragma unroll
  for (int v = 0; v < 4; ++v) sv[v] = g + 4 * v < NH ? A.ps[std::size_t(pp) * NH + g + 4 * v] : 0.0;
}

// One wavefront per SIMD: at two, F = 256 overflows the registers (the
// hidden row alone takes 160); measured at config 3, F = 256: 3.56 ms per
// block (logits included) against 5.11 ms at two wavefronts with spills.
#ifndef SO3LR_FILT_FWD_WAVES
#define SO3LR_FILT_FWD_WAVES 1
#endif
#ifndef SO3LR_FILT_PFB
#define SO3LR_FILT_PFB 10
#endif
template <int FT, int RT>
// At F = 128 (a 10-tile hidden row) two wavefronts per SIMD fit with five
// chunks in flight: 1.10 against 1.17 ms per block at one wavefront (slots
// 1,1,2,3, R = 32, config 3).
#ifndef SO3LR_FILT_FWD_WAVES_F128
#define SO3LR_FILT_FWD_WAVES_F128 2
#endif
#ifndef SO3LR_FILT_PFB_F128
#define SO3LR_FILT_PFB_F128 5
#endif
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(
    FT == 8 ? SO3LR_FILT_FWD_WAVES_F128 : SO3LR_FILT_FWD_WAVES, FT == 8 ? SO3LR_FILT_FWD_WAVES_F128 : SO3LR_FILT_FWD_WAVES))) void
g_filt_fwd(FiltArgs A) {
  constexpr int FHT = FT / 4, NH = FT / 2, HT = FT + FHT, F = 16 * FT;
  constexpr int NA = FT * (1 + RT) + 2 * FHT;  // hidden row: per tile the bias and its weight chunks
  constexpr int NB = HT;                       // output tile: its HT weight chunks
  constexpr int PFS = FT == 8 ? SO3LR_FILT_PFB_F128 : SO3LR_FILT_PFB;
  constexpr int PFB = NB % PFS == 0 ? PFS : NB;
  __shared__ double tab[256];
  tab[threadIdx.x] = A.exp2_256[threadIdx.x];
  __syncthreads();
  const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
  int pp = 0;
  bool valid = false;
  if (!filt_pair(A, j, pp, valid)) return;
  const int a = A.pa[2 * pp], b = A.pa[2 * pp + 1];
  // the output rows of [W1 | E1] come permuted within each tile (row 16 mt +
  // i is channel 16 mt + 4 (i % 4) + i / 4), so register r of lane group g
  // holds channel 16 mt + 4 g + r: a lane's four channels are contiguous
  const double *ra = A.qkv + std::size_t(a) * 5 * F + 4 * g, *rr = A.qkv + std::size_t(b) * 5 * F + 4 * g;
  double *frow = A.pf + std::size_t(pp) * 2 * F + 4 * g;
  double *al = A.palpha + std::size_t(pp) * 4 * NH;
  v4d h[HT];
  static_for<2>([&](auto wi) {
    constexpr int w = decltype(wi)::value;
    const double *b0a = A.b0a[w], *w0p = A.w0p[w], *eb0a = A.eb0a[w], *e0p = A.e0p[w], *bca = A.bca[w],
                 *wcp = A.wcp[w];
    v4d rb[RT], sv;
    filt_inputs<RT, NH>(A, pp, g, rb, sv);
    auto la = [&](auto si) -> v4d {
      constexpr int S = decltype(si)::value;
      if constexpr (S < FT * (1 + RT)) {
        constexpr int T = S / (1 + RT), u = S % (1 + RT);
        if constexpr (u == 0) return frag_load(b0a, T, lane);
        else return frag_load(w0p, T * RT + u - 1, lane);
      } else {
        constexpr int t = (S - FT * (1 + RT)) / 2, u = (S - FT * (1 + RT)) % 2;
        if constexpr (u == 0) return frag_load(eb0a, t, lane);
        else return frag_load(e0p, t, lane);
      }
    };
    Stream<NA, SO3LR_FILT_PF, decltype(la)> sa(la);
    sa.prime();
    sa.run([&](auto si, const v4d &wv) {
      constexpr int S = decltype(si)::value;
      constexpr bool RAD = S < FT * (1 + RT);
      constexpr int T = RAD ? S / (1 + RT) : FT + (S - FT * (1 + RT)) / 2;
      constexpr int u = RAD ? S % (1 + RT) : (S - FT * (1 + RT)) % 2;
      if constexpr (u == 0) {
        h[T] = wv;
      } else {
        if constexpr (RAD) {
          h[T] = mfma4(wv, rb[u - 1], h[T]);
        } else {
          h[T] = mfma(wv[0], sv[0], h[T]);
          if constexpr (NH > 4) h[T] = mfma(wv[1], sv[1], h[T]);
        }
        // the tile before: its SiLU behind the MFMA just issued
        if constexpr (u == 1 && T > 0) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            if constexpr (T - 1 < FT) h[T - 1][r] = silu_tab(h[T - 1][r], tab);
            else h[T - 1][r] = silu_tab_wide(h[T - 1][r], tab);
          }
        }
      }
    });
#pragma unroll
    for (int r = 0; r < 4; ++r) h[HT - 1][r] = silu_tab_wide(h[HT - 1][r], tab);
    auto lb = [&](auto si, int mt) -> v4d { return frag_load(wcp, mt * HT + decltype(si)::value, lane); };
    LoopStream<NB, PFB, decltype(lb)> sb(lb);
    sb.prime();
    constexpr int qo = w ? 3 * F : 0, ko = w ? 4 * F : F;  // q, k or q_ev, k_ev
    v4d o, qa, kb, qb, ka, bn = frag_load(bca, 0, lane);  // bn: the next tile's bias
    double t0 = 0.0, t1 = 0.0;  // the lane's part of the head's logits: a <- b, b <- a
    sb.run(FT, [&](auto si, int mt, const v4d &wv) {
      constexpr int u = decltype(si)::value;
      if constexpr (u == 0) {
        o = mfma4(wv, h[0], bn);
        bn = frag_load(bca, min(mt + 1, FT - 1), lane);
        // the endpoint rows at the tile's channels, used when it is complete
        qa = *reinterpret_cast<const v4d *>(ra + qo + 16 * mt);
        kb = *reinterpret_cast<const v4d *>(rr + ko + 16 * mt);
        qb = *reinterpret_cast<const v4d *>(rr + qo + 16 * mt);
        ka = *reinterpret_cast<const v4d *>(ra + ko + 16 * mt);
      } else {
        o = mfma4(wv, h[u], o);
      }
      if constexpr (u == NB - 1) {
        if (valid) *reinterpret_cast<v4d *>(frow + w * F + 16 * mt) = o;
        // alpha = <q_receiver, k_sender (.) f>_h / avg (kokkos_integrated_block0.cpp:330-360)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          t0 += qa[r] * kb[r] * o[r];
          t1 += qb[r] * ka[r] * o[r];
        }
        if (mt & 1) {  // head mt / 2 complete: sum over the lane groups
          t0 += __shfl_xor(t0, 16, 64);
          t0 += __shfl_xor(t0, 32, 64);
          t1 += __shfl_xor(t1, 16, 64);
          t1 += __shfl_xor(t1, 32, 64);
          if (valid && g == 0) {
            al[w * NH + (mt >> 1)] = t0 * A.inv_avg;
            al[2 * NH + w * NH + (mt >> 1)] = t1 * A.inv_avg;
          }
          t0 = 0.0;
          t1 = 0.0;
        }
      }
    });
  });
}

// The reverse's second part for hidden tiles T0 .. T0 + TG - 1: per tile
// its bias (kind 0), forward chunks (kind 1: W0 K chunks or E0) and, one
// tile behind, the previous tile's transposed chunks (kind 2: W0^T row tiles
// or E0^T), then the last tile's transposed chunks.
struct FEntry {
  int kind, T, k;
};
template <int FT, int RT>
constexpr int filt_chunks(int T) { return T < FT ? RT : 1; }
template <int FT, int RT, int T0, int TG>
constexpr int filt_sched_len() {
  int n = 0;
  for (int T = T0; T < T0 + TG; ++T) n += 1 + filt_chunks<FT, RT>(T) + (T > T0 ? filt_chunks<FT, RT>(T - 1) : 0);
  return n + filt_chunks<FT, RT>(T0 + TG - 1);
}
template <int FT, int RT, int T0, int TG>
constexpr std::array<FEntry, filt_sched_len<FT, RT, T0, TG>()> filt_sched() {
  std::array<FEntry, filt_sched_len<FT, RT, T0, TG>()> out{};
  int n = 0;
  for (int T = T0; T < T0 + TG; ++T) {
    out[n++] = FEntry{0, T, 0};
    for (int k = 0; k < filt_chunks<FT, RT>(T); ++k) out[n++] = FEntry{1, T, k};
    if (T > T0)
      for (int k = 0; k < filt_chunks<FT, RT>(T - 1); ++k) out[n++] = FEntry{2, T - 1, k};
  }
  for (int k = 0; k < filt_chunks<FT, RT>(T0 + TG - 1); ++k) out[n++] = FEntry{2, T0 + TG - 1, k};
  return out;
}
template <int FT, int RT, int T0, int TG>
constexpr FEntry filt_entry(int s) {
  return filt_sched<FT, RT, T0, TG>()[s];
}

// The whole hidden row's adjoint in one group (TG = HT, its accumulators in
// the accumulation registers) at one wavefront per SIMD: measured at F = 256
// (config 3) 4.59 ms per block against 5.72 for groups of 5 at two
// wavefronts per SIMD, whose endpoint rows are read once per group.
#ifndef SO3LR_FILT_TG
#define SO3LR_FILT_TG 20
#endif

#ifndef SO3LR_FILT_BWD_WAVES
#define SO3LR_FILT_BWD_WAVES 1
#endif
template <int FT, int RT>
// At F = 128 the hidden row's adjoint (10 tiles) leaves room for two
// wavefronts per SIMD: 1.07 against 1.25 ms per block (slots 1,1,2,3, R =
// 32, config 3), 1.40 against 1.61 at R = 64.
#ifndef SO3LR_FILT_BWD_WAVES_F128
#define SO3LR_FILT_BWD_WAVES_F128 2
#endif
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(
    FT == 8 ? SO3LR_FILT_BWD_WAVES_F128 : SO3LR_FILT_BWD_WAVES, FT == 8 ? SO3LR_FILT_BWD_WAVES_F128 : SO3LR_FILT_BWD_WAVES))) void
g_filt_bwd(FiltArgs A) {
  constexpr int FHT = FT / 4, NH = FT / 2, HT = FT + FHT, F = 16 * FT;
  constexpr int TG = HT % SO3LR_FILT_TG == 0 ? SO3LR_FILT_TG : HT, NG = HT / TG;  // hidden tiles per group
  constexpr int N1 = 4 + TG;  // per output tile: four endpoint rows, then TG weight chunks
#ifndef SO3LR_FILT_PF1
#define SO3LR_FILT_PF1 8
#endif
  __shared__ double tab[256];
  tab[threadIdx.x] = A.exp2_256[threadIdx.x];
  __syncthreads();
  const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
  int pp = 0;
  bool valid = false;
  if (!filt_pair(A, j, pp, valid)) return;
  const int a = A.pa[2 * pp], b = A.pa[2 * pp + 1];
  const double *ra = A.qkv + std::size_t(a) * 5 * F + 4 * g, *rr = A.qkv + std::size_t(b) * 5 * F + 4 * g;
  const double *ps = A.psc + std::size_t(pp) * 4 * NH;
  const v4d zero = v4d{0.0, 0.0, 0.0, 0.0};
  v4d drb[RT], dsa = zero;
#pragma unroll
  for (int Kc = 0; Kc < RT; ++Kc) drb[Kc] = zero;
  // one filter at a time, a loop: unrolled, the two filters' code overflows
  // the registers
#pragma unroll 1
  for (int w = 0; w < 2; ++w) {
    const int qo = w ? 3 * F : 0, ko = w ? 4 * F : F;
    const double *b0a = w ? A.b0a[1] : A.b0a[0], *w0p = w ? A.w0p[1] : A.w0p[0], *w0tp = w ? A.w0tp[1] : A.w0tp[0];
    const double *eb0a = w ? A.eb0a[1] : A.eb0a[0], *e0p = w ? A.e0p[1] : A.e0p[0], *e0tp = w ? A.e0tp[1] : A.e0tp[0];
    const double *wctp = w ? A.wctp[1] : A.wctp[0];
    static_for<NG>([&](auto gi) {
      constexpr int T0 = decltype(gi)::value * TG;
      v4d dh[TG];
#pragma unroll
      for (int t = 0; t < TG; ++t) dh[t] = zero;
      // d hidden (tiles T0..) = sum over output tiles mt of [W1 | E1]^T df_mt,
      // df_mt = psc_0 q_a k_b + psc_1 q_b k_a at the lane's channels
      // 16 mt + 4 g + v (side 0: a receives from b): [W1 | E1]^T comes with
      // its K chunks in that order (permute_mfma_kc), so a lane's four
      // channels of a row are one 32-byte load.  Unrolled over the output
      // tiles: as a loop, the accumulators' registers rotate from one
      // iteration to the next and cost eight moves per chain (measured 4.50
      // against 3.95 ms at F = 256, config 3).
      auto l1 = [&](auto si) -> v4d {
        constexpr int u = decltype(si)::value % N1, mt = decltype(si)::value / N1;
        if constexpr (u < 4) {
          const double *row = (u == 0 ? ra + qo : (u == 1 ? rr + ko : (u == 2 ? rr + qo : ra + ko))) + 16 * mt;
          return *reinterpret_cast<const v4d *>(row);
        } else {
          return frag_load(wctp, (T0 + u - 4) * FT + mt, lane);
        }
      };
      double c0 = ps[w * NH], c1 = ps[2 * NH + w * NH];  // head 0
      v4d qv, df;
      Stream<N1 * FT, SO3LR_FILT_PF1, decltype(l1)> s1(l1);
      s1.prime();
      s1.run([&](auto si, const v4d &wv) {
        constexpr int u = decltype(si)::value % N1, mt = decltype(si)::value / N1;
        if constexpr (u == 0 || u == 2) {
          qv = wv;
        } else if constexpr (u == 1) {
          df = c0 * (qv * wv);
        } else if constexpr (u == 3) {
          df += c1 * (qv * wv);
          // the coefficients of the next tile's head (a tile lies in one head)
          const int hn = min(mt + 1, FT - 1) >> 1;
          c0 = ps[w * NH + hn];
          c1 = ps[2 * NH + w * NH + hn];
        } else {
          dh[u - 4] = mfma4(wv, df, dh[u - 4]);
        }
      });
      // per tile: pre again, d hidden *= silu'(pre), then through W0^T / E0^T
      v4d rb[RT], sv;
      filt_inputs<RT, NH>(A, pp, g, rb, sv);
      auto l2 = [&](auto si) -> v4d {
        constexpr FEntry e = filt_entry<FT, RT, T0, TG>(decltype(si)::value);
        if constexpr (e.kind == 0) {
          if constexpr (e.T < FT) return frag_load(b0a, e.T, lane);
          else return frag_load(eb0a, e.T - FT, lane);
        } else if constexpr (e.kind == 1) {
          if constexpr (e.T < FT) return frag_load(w0p, e.T * RT + e.k, lane);
          else return frag_load(e0p, e.T - FT, lane);
        } else {
          if constexpr (e.T < FT) return frag_load(w0tp, e.k * FT + e.T, lane);
          else return frag_load(e0tp, e.T - FT, lane);
        }
      };
      constexpr int N2 = filt_sched_len<FT, RT, T0, TG>();
      Stream<N2, SO3LR_FILT_PF, decltype(l2)> s2(l2);
      s2.prime();
      v4d pre[2];
      auto dsilu = [&](auto ti) {
        constexpr int T = decltype(ti)::value;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if constexpr (T < FT) dh[T - T0][r] *= silu_prime_tab(pre[T % 2][r], tab);
          else dh[T - T0][r] *= silu_prime_tab_wide(pre[T % 2][r], tab);
        }
      };
      s2.run([&](auto si, const v4d &wv) {
        constexpr FEntry e = filt_entry<FT, RT, T0, TG>(decltype(si)::value);
        constexpr int T = e.T;
        if constexpr (e.kind == 0) {
          pre[T % 2] = wv;
        } else if constexpr (e.kind == 1) {
          if constexpr (T < FT) {
            pre[T % 2] = mfma4(wv, rb[e.k], pre[T % 2]);
          } else {
            pre[T % 2] = mfma(wv[0], sv[0], pre[T % 2]);
            if constexpr (NH > 4) pre[T % 2] = mfma(wv[1], sv[1], pre[T % 2]);
          }
          if constexpr (e.k == 0 && T > T0) dsilu(std::integral_constant<int, T - 1>{});
        } else {
          if constexpr (e.k == 0 && T == T0 + TG - 1) dsilu(std::integral_constant<int, T>{});
          if constexpr (T < FT) drb[e.k] = mfma4(wv, dh[T - T0], drb[e.k]);
          else dsa = mfma4(wv, dh[T - T0], dsa);
        }
      });
    });
  }
  // dE/ds of the pair's slots (rows g + 4 r of the E0^T tile), summed over
  // both filters
  if (valid) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (g + 4 * r < NH) A.ds[std::size_t(pp) * NH + g + 4 * r] = dsa[r];
  }
  // dE/dr: the basis adjoint against d rbf / dr (zero where the basis
  // variable is clamped), plus the cutoff's
  const double r = A.pr[pp];
  const double xb = exp(-A.gamma * r);
  double part = 0.0;
  if (xb > 1e-6 && xb < 1.0 - 1e-6) {
    const double ratio = xb / (1.0 - xb);
    const double *row = A.rbf + std::size_t(pp) * 16 * RT + g;
#pragma unroll
    for (int Kc = 0; Kc < RT; ++Kc)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int k = 16 * Kc + g + 4 * q;
        part += drb[Kc][q] * row[k - g] * (-A.gamma * A.kk[k] + A.gamma * ratio * A.kr[k]);
      }
  }
  part += __shfl_xor(part, 16, 64);
  part += __shfl_xor(part, 32, 64);
  if (valid && g == 0) {
    double grad = part;
    if (r < A.rc) {
      const double t = r / A.rc;
      grad += A.dfc[pp] * (-30.0 * t * t * (1.0 - t) * (1.0 - t) / A.rc);
    }
    A.dr[pp] += grad;
  }
}

unsigned blocks_for(std::size_t n, int per) { return unsigned((n + std::size_t(per) - 1) / std::size_t(per)); }

}  // namespace

// ------------------------------------------------------------------ host side
namespace {
enum Buf {
  XS = 0, EVS, QKV, QKIS, AEV, N1, N1HAT, N1IS, HPRE, TOUT, PRE2HAT, PRE2IS,
  ACT, HID, CAT, HACT, HHPRE, HKEY, GHEAD,
  GX, GEV, GT, GCAT, GA, GP, GHID, GN1, GAINV, GQKV,
  RBF, PS, PF, PALPHA, PSC, DFC, DS, CLS_M, CLS_B,
  NBUF
};
static_assert(NBUF <= GenericPath::kBuffers, "generic path buffer table");

#ifndef SO3LR_GEMM_MAX_NT
#define SO3LR_GEMM_MAX_NT 4
#endif
constexpr int kGemmMaxNT = SO3LR_GEMM_MAX_NT;

template <int EPI, bool WKO>
void gemm(hipStream_t s, int rows, const int *rows_dev, int K, int O, const double *X, int ldx, const double *W,
          const double *bias, double *Y, int ldy, const double *aux = nullptr, int ldaux = 0,
          const double *res = nullptr, int ldres = 0, double *Y2 = nullptr, int ldy2 = 0) {
  if (rows <= 0) return;
  GemmArgs A{rows, rows_dev, K, O, X, ldx, W, bias, Y, ldy, Y2, ldy2, aux, ldaux, res, ldres,
             1, 0, 0, 0, 0, 0, 0, 0, 0};
  // column blocks of 32 kGemmMaxNT columns, and the rest (O not a multiple
  // of that, e.g. 320 = 2 x 128 + 64) as a launch of its own on the columns
  // left, so no block computes padded columns; NT = 32-column tiles per
  // wavefront
  const int cmax = 32 * kGemmMaxNT;
  const dim3 gr(blocks_for(std::size_t(rows), 64));
  auto launch = [&](GemmArgs B, int nb, int tiles) {
    const dim3 grid(nb > 1 ? (gr.x + 7) / 8 * 8 : gr.x, unsigned(nb));
#define G_GEMM_NT(NT)                                                              \
  if (tiles <= NT) {                                                               \
    hipLaunchKernelGGL((g_gemm<EPI, WKO, NT>), grid, dim3(256), 0, s, B);          \
    return;                                                                        \
  }
    G_GEMM_NT(2) G_GEMM_NT(4) G_GEMM_NT(6) G_GEMM_NT(8) G_GEMM_NT(10)
#undef G_GEMM_NT
    throw std::logic_error("SO3LR: generic GEMM with more than 320 columns per block");
  };
  const int full = O / cmax, rest = O - full * cmax;
  if (full == 0 || rest == 0) {
    const int nb = (O + cmax - 1) / cmax, cols = (O + nb - 1) / nb;
    launch(A, nb, (cols + 31) / 32);
    return;
  }
  GemmArgs M = A;
  M.O = full * cmax;
  if (WKO) M.ldw = O;
  launch(M, full, kGemmMaxNT);
  GemmArgs R = A;
  const int c0 = full * cmax;
  R.O = rest;
  if (WKO) {
    R.W = W + c0;
    R.ldw = O;
  } else {
    R.W = W + std::size_t(c0) * K;
  }
  if (bias) R.bias = bias + c0;
  R.Y = Y + c0;
  if (Y2) R.Y2 = Y2 + c0;
  if (aux) R.aux = aux + c0;
  if (res) R.res = res + c0;
  launch(R, 1, (rest + 31) / 32);
}
// Per-head 32 x 32 projections as one batched launch (O = K = 32).
template <int EPI, bool WKO>
void gemm_heads(hipStream_t s, int rows, int nby, int nbx, const double *X, int ldx, long xbs0, long xbs1,
                const double *W, long wbs, double *Y, int ldy, long ybs0, long ybs1, const double *res = nullptr,
                int ldres = 0, long rbs0 = 0, long rbs1 = 0) {
  if (rows <= 0) return;
  GemmArgs A{rows, nullptr, 32, 32, X, ldx, W, nullptr, Y, ldy, nullptr, 0, nullptr, 0, res, ldres,
             nbx, xbs0, xbs1, ybs0, ybs1, rbs0, rbs1, wbs, 0};
  hipLaunchKernelGGL((g_gemm<EPI, WKO, 2>), dim3(blocks_for(std::size_t(rows), 64), 1, unsigned(nby * nbx)),
                     dim3(256), 0, s, A);
}
}  // namespace

namespace {
bool cls_on(const GContext &c) { return c.cls_C > 0; }

// Slots of block 0's element-pair order, at most: every nonempty bucket
// padded by fewer than kB0Pad
std::size_t b0_slot_bound(const GContext &c) {
  return std::size_t(std::max(c.cap, 1)) + std::size_t(GContext::kB0Pad) * c.cls_C * c.cls_C;
}

// g_b0_fwd / g_b0_bwd at F = 16 FT, R = 16 RT over `slots` slots (one
// wavefront per 16 CT)
template <bool FWD>
void launch_b0(hipStream_t s, int F, int R, std::size_t slots, const B0Args &A) {
  constexpr int CT = FWD ? SO3LR_B0_FWD_CT : SO3LR_B0_BWD_CT;
  static_assert(GContext::kB0Pad % (16 * CT) == 0, "a wavefront's slots lie in one bucket");
  const dim3 grid(blocks_for(slots, 64 * CT));
#define G_B0(FT, RT)                                                                        \
  if (F == 16 * FT && R == 16 * RT) {                                                       \
    if constexpr (FWD) hipLaunchKernelGGL((g_b0_fwd<FT, RT, CT>), grid, dim3(256), 0, s, A); \
    else hipLaunchKernelGGL((g_b0_bwd<FT, RT, CT>), grid, dim3(256), 0, s, A);              \
    return;                                                                                 \
  }
  G_B0(8, 2) G_B0(8, 4) G_B0(16, 2) G_B0(16, 4)
#undef G_B0
  throw std::logic_error("SO3LR: block 0's table kernels at widths other than F = 128, 256 and R = 32, 64");
}

// The forward filters of the blocks after 0 on their radial tables (the
// algebra of evaluator.hip's k_radial_fwd_rows at generic widths): the pairs
// in bucket order (16 slots of one bucket, spatial block and interval, per
// wavefront), per filter the spherical hidden tiles silu(E0 s + e0), then
// per output tile the interval's coefficient tile (two K chunks against the
// pairs' powers of t, in place of the W0 and W1 chains), the E1 chunks and
// the endpoint rows; the rows go to pf and the logits to palpha as in
// g_filt_fwd.
struct GRadArgs {
  const int *slots, *order, *pa;
  const double *pr, *ps, *qkv, *rtab;
  RadialDomain d;
  const double *eb0a[2], *e0p[2], *wcp[2];
  const double *exp2_256;
  double inv_avg;
  double *pf, *palpha;
  // reverse (g_radial_bwd_rows): rtab holds the slope tiles
  const double *e0tp[2], *wctp[2], *psc, *dfc;
  double rc;
  double *ds, *dr;
};

template <int FT>
__global__ __launch_bounds__(256) void g_radial_fwd_rows(GRadArgs A) {
  constexpr int FHT = FT / 4, NH = FT / 2, HT = FT + FHT, F = 16 * FT, NE = 6 + FHT;
  __shared__ double tab[256];
  tab[threadIdx.x] = A.exp2_256[threadIdx.x];
  __syncthreads();
  const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
  const int blk = g_xcd_block((*A.slots + 63) / 64);
  const int wave = blk < 0 ? -1 : blk * 4 + int(threadIdx.x >> 6);
  int p, ri;
  bool inside;
  v4d tp[2];
  if (!rint_slots(A.slots, A.order, A.pr, A.d, wave, j, g, p, ri, inside, tp)) return;
  const bool valid = p >= 0;
  const int pp = valid ? p : A.order[wave * 16];
  const int a = A.pa[2 * pp], b = A.pa[2 * pp + 1];
  const double *ra = A.qkv + std::size_t(a) * 5 * F + 4 * g, *rr = A.qkv + std::size_t(b) * 5 * F + 4 * g;
  double *frow = A.pf + std::size_t(pp) * 2 * F + 4 * g;
  double *al = A.palpha + std::size_t(pp) * 4 * NH;
  v4d sv;
#pragma unroll
  for (int v = 0; v < 4; ++v) sv[v] = g + 4 * v < NH ? A.ps[std::size_t(pp) * NH + g + 4 * v] : 0.0;
  const v4d zero = v4d{0.0, 0.0, 0.0, 0.0};
  static_for<2>([&](auto wi) {
    constexpr int w = decltype(wi)::value;
    v4d he[FHT];
#pragma unroll
    for (int t = 0; t < FHT; ++t) {
      const v4d e0 = frag_load(A.e0p[w], t, lane);
      he[t] = mfma(e0[0], sv[0], frag_load(A.eb0a[w], t, lane));
      if constexpr (NH > 4) he[t] = mfma(e0[1], sv[1], he[t]);
#pragma unroll
      for (int r = 0; r < 4; ++r) he[t][r] = silu_tab_wide(he[t][r], tab);
    }
    const double *coef = A.rtab + (std::size_t(ri) * 2 + w) * FT * 2 * 256;
    constexpr int qo = w ? 3 * F : 0, ko = w ? 4 * F : F;  // q, k or q_ev, k_ev
    auto ld = [&](auto si) -> v4d {
      constexpr int S = decltype(si)::value, mt = S / NE, u = S % NE;
      if constexpr (u < 2) return frag_load(coef, mt * 2 + u, lane);
      else if constexpr (u < 2 + FHT) return frag_load(A.wcp[w], mt * HT + FT + u - 2, lane);
      else if constexpr (u == 2 + FHT) return *reinterpret_cast<const v4d *>(ra + qo + 16 * mt);
      else if constexpr (u == 3 + FHT) return *reinterpret_cast<const v4d *>(rr + ko + 16 * mt);
      else if constexpr (u == 4 + FHT) return *reinterpret_cast<const v4d *>(rr + qo + 16 * mt);
      else return *reinterpret_cast<const v4d *>(ra + ko + 16 * mt);
    };
    Stream<FT * NE, 6, decltype(ld)> st(ld);
    st.prime();
    v4d o, qv, qk0, qk1;
    double t0 = 0.0, t1 = 0.0;
    st.run([&](auto si, const v4d &wv) {
      constexpr int S = decltype(si)::value, mt = S / NE, u = S % NE;
      if constexpr (u == 0) {
        o = mfma4(wv, tp[0], zero);
      } else if constexpr (u == 1) {
        o = mfma4(wv, tp[1], o);
      } else if constexpr (u < 2 + FHT) {
        o = mfma4(wv, he[u - 2], o);
      } else if constexpr (u == 2 + FHT || u == 4 + FHT) {
        qv = wv;
      } else if constexpr (u == 3 + FHT) {
        qk0 = qv * wv;  // q_a k_b: edge b -> a
      } else {
        qk1 = qv * wv;  // q_b k_a: edge a -> b
        if (valid) *reinterpret_cast<v4d *>(frow + w * F + 16 * mt) = o;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          t0 += qk0[r] * o[r];
          t1 += qk1[r] * o[r];
        }
        if constexpr (mt & 1) {  // head mt / 2 complete: sum over the lane groups
          t0 += __shfl_xor(t0, 16, 64);
          t0 += __shfl_xor(t0, 32, 64);
          t1 += __shfl_xor(t1, 16, 64);
          t1 += __shfl_xor(t1, 32, 64);
          if (valid && g == 0) {
            al[w * NH + (mt >> 1)] = t0 * A.inv_avg;
            al[2 * NH + w * NH + (mt >> 1)] = t1 * A.inv_avg;
          }
          t0 = 0.0;
          t1 = 0.0;
        }
      }
    });
  });
}

// The reverse filters of the blocks after 0 on their radial tables, in
// bucket order: per filter and output tile mt, df from the logits' adjoints
// and the endpoint rows as in g_filt_bwd, then the spherical hidden row's
// adjoint (E1^T chunks) and the slope tiles against df, whose sum over the
// powers of t is the radial branches' dE/dr; the spherical branch goes on
// through silu' and E0^T to dE/ds.  No W1^T, no layer-0 recompute.
template <int FT>
__global__ __launch_bounds__(256) void g_radial_bwd_rows(GRadArgs A) {
  constexpr int FHT = FT / 4, NH = FT / 2, F = 16 * FT, NE = 4 + FHT + 2;
  __shared__ double tab[256];
  tab[threadIdx.x] = A.exp2_256[threadIdx.x];
  __syncthreads();
  const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
  const int blk = g_xcd_block((*A.slots + 63) / 64);
  const int wave = blk < 0 ? -1 : blk * 4 + int(threadIdx.x >> 6);
  int p, ri;
  bool inside;
  v4d tp[2];
  if (!rint_slots(A.slots, A.order, A.pr, A.d, wave, j, g, p, ri, inside, tp)) return;
  const bool valid = p >= 0;
  const int pp = valid ? p : A.order[wave * 16];
  const int a = A.pa[2 * pp], b = A.pa[2 * pp + 1];
  const double *ra = A.qkv + std::size_t(a) * 5 * F + 4 * g, *rr = A.qkv + std::size_t(b) * 5 * F + 4 * g;
  const double *ps = A.psc + std::size_t(pp) * 4 * NH;
  v4d sv;
#pragma unroll
  for (int v = 0; v < 4; ++v) sv[v] = g + 4 * v < NH ? A.ps[std::size_t(pp) * NH + g + 4 * v] : 0.0;
  const v4d zero = v4d{0.0, 0.0, 0.0, 0.0};
  v4d dsa = zero, accdr[2] = {zero, zero};
  static_for<2>([&](auto wi) {
    constexpr int w = decltype(wi)::value;
    constexpr int qo = w ? 3 * F : 0, ko = w ? 4 * F : F;
    const double *slope = A.rtab + (std::size_t(ri) * 2 + w) * 2 * FT * 256;
    v4d dh[FHT];
#pragma unroll
    for (int t = 0; t < FHT; ++t) dh[t] = zero;
    auto ld = [&](auto si) -> v4d {
      constexpr int S = decltype(si)::value, mt = S / NE, u = S % NE;
      if constexpr (u < 4) {
        const double *row = (u == 0 ? ra + qo : (u == 1 ? rr + ko : (u == 2 ? rr + qo : ra + ko))) + 16 * mt;
        return *reinterpret_cast<const v4d *>(row);
      } else if constexpr (u < 4 + FHT) {
        return frag_load(A.wctp[w], (FT + u - 4) * FT + mt, lane);
      } else {
        return frag_load(slope, (u - 4 - FHT) * FT + mt, lane);
      }
    };
    double c0 = ps[w * NH], c1 = ps[2 * NH + w * NH];  // head 0
    v4d qv, df;
    Stream<NE * FT, 6, decltype(ld)> st(ld);
    st.prime();
    st.run([&](auto si, const v4d &wv) {
      constexpr int S = decltype(si)::value, mt = S / NE, u = S % NE;
      if constexpr (u == 0 || u == 2) {
        qv = wv;
      } else if constexpr (u == 1) {
        df = c0 * (qv * wv);
      } else if constexpr (u == 3) {
        df += c1 * (qv * wv);
        const int hn = min(mt + 1, FT - 1) >> 1;  // the next tile's head
        c0 = ps[w * NH + hn];
        c1 = ps[2 * NH + w * NH + hn];
      } else if constexpr (u < 4 + FHT) {
        dh[u - 4] = mfma4(wv, df, dh[u - 4]);
      } else {
        accdr[u - 4 - FHT] = mfma4(wv, df, accdr[u - 4 - FHT]);
      }
    });
    // the spherical branch: pre again, d hidden *= silu'(pre), E0^T
#pragma unroll
    for (int t = 0; t < FHT; ++t) {
      const v4d e0 = frag_load(A.e0p[w], t, lane);
      v4d pre = mfma(e0[0], sv[0], frag_load(A.eb0a[w], t, lane));
      if constexpr (NH > 4) pre = mfma(e0[1], sv[1], pre);
#pragma unroll
      for (int r = 0; r < 4; ++r) dh[t][r] *= silu_prime_tab_wide(pre[r], tab);
      dsa = mfma4(frag_load(A.e0tp[w], t, lane), dh[t], dsa);
    }
  });
  if (valid) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (g + 4 * r < NH) A.ds[std::size_t(pp) * NH + g + 4 * r] = dsa[r];
  }
  // dE/dr: the radial branches' (powers 16 m + g + 4 r), plus the cutoff's
  double part = 0.0;
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int r = 0; r < 4; ++r) part += accdr[m][r] * tp[m][r];
  if (!inside) part = 0.0;
  part += __shfl_xor(part, 16, 64);
  part += __shfl_xor(part, 32, 64);
  if (valid && g == 0) {
    const double r = A.pr[pp];
    double grad = part;
    if (r < A.rc) {
      const double t = r / A.rc;
      grad += A.dfc[pp] * (-30.0 * t * t * (1.0 - t) * (1.0 - t) / A.rc);
    }
    A.dr[pp] += grad;
  }
}

// g_radial_fwd / g_radial_bwd at NH = 4 or 8 heads over cap pairs
template <bool FWD>
void launch_radial(hipStream_t s, int NH, const GContext &c, const double *tab, RadialDomain d, double *palpha,
                   const double *psc, const double *dfc) {
#define G_RAD(L)                                                                                                    \
  if (4 * NH == L) {                                                                                                \
    const dim3 grid(blocks_for(std::size_t(std::max(c.cap, 1)), 256 / L));                                         \
    if constexpr (FWD)                                                                                              \
      hipLaunchKernelGGL(g_radial_fwd<L>, grid, dim3(256), 0, s, c.nact, c.pa, c.pr, c.z, c.cls_lut, c.cls_C, tab, \
                         d, c.inv_avg, palpha);                                                                     \
    else                                                                                                            \
      hipLaunchKernelGGL(g_radial_bwd<L>, grid, dim3(256), 0, s, c.nact, c.pa, c.pr, c.z, c.cls_lut, c.cls_C, tab, \
                         d, psc, dfc, c.rc, c.dr);                                                                  \
    return;                                                                                                         \
  }
  G_RAD(16) G_RAD(32)
#undef G_RAD
  throw std::logic_error("SO3LR: block 0's radial tables at other than 4 or 8 heads");
}

// g_filt_fwd / g_filt_bwd at F = 16 FT, R = 16 RT over cap pairs (one
// wavefront per 16, the grid a multiple of 8: g_xcd_block)
template <bool FWD>
void launch_filt(hipStream_t s, int F, int R, std::size_t cap, const FiltArgs &A) {
  const dim3 grid((blocks_for(cap, 64) + 7) / 8 * 8);
#define G_FILT(FT, RT)                                                                \
  if (F == 16 * FT && R == 16 * RT) {                                                 \
    if constexpr (FWD) hipLaunchKernelGGL((g_filt_fwd<FT, RT>), grid, dim3(256), 0, s, A); \
    else hipLaunchKernelGGL((g_filt_bwd<FT, RT>), grid, dim3(256), 0, s, A);          \
    return;                                                                           \
  }
  G_FILT(8, 2) G_FILT(8, 4) G_FILT(16, 2) G_FILT(16, 4)
#undef G_FILT
  throw std::logic_error("SO3LR: fused filters at widths other than F = 128, 256 and R = 32, 64");
}

// the fused filters' arguments (the reverse adds its inputs and outputs)
FiltArgs filt_args(const GContext &c, const GBlock &B, const GHeads &H, const double *rbf, const double *ps,
                   const double *qkv, double *pf) {
  FiltArgs A{};
  A.nact = c.nact;
  A.cap = c.cap;
  A.pa = c.pa;
  A.pr = c.pr;
  A.rbf = rbf;
  A.ps = ps;
  A.qkv = qkv;
  for (int w = 0; w < 2; ++w) {
    A.w0p[w] = B.w0p[w];
    A.b0a[w] = B.b0a[w];
    A.e0p[w] = B.e0p[w];
    A.eb0a[w] = B.eb0a[w];
    A.wcp[w] = B.wcp[w];
    A.bca[w] = B.bca[w];
    A.w0tp[w] = B.w0tp[w];
    A.e0tp[w] = B.e0tp[w];
    A.wctp[w] = B.wctp[w];
  }
  A.exp2_256 = H.exp2_256;
  A.kk = H.rbf_k;
  A.kr = H.rbf_kr;
  A.gamma = c.gamma;
  A.rc = c.rc;
  A.inv_avg = c.inv_avg;
  A.pf = pf;
  return A;
}

// block 0's table kernels' arguments (the reverse adds its inputs and dr)
B0Args b0_args(const GContext &c, const GBlock &B, const GHeads &H, const double *rbf, const double *tables,
               const double *cb, int F, double *palpha) {
  const std::size_t NK = std::size_t(c.cls_C) * c.cls_C;
  B0Args A{};
  A.slots = c.cls_slots;
  A.order = c.cls_order;
  A.pa = c.pa;
  A.z = c.z;
  A.cls = c.cls_lut;
  A.C = c.cls_C;
  A.pr = c.pr;
  A.rbf = rbf;
  for (int w = 0; w < 2; ++w) {
    A.w0p[w] = B.w0p[w];
    A.w0tp[w] = B.w0tp[w];
    A.b0a[w] = B.b0a[w];
  }
  A.tf = tables;
  A.tr = tables + NK * 32 * std::size_t(F);
  A.cb = cb;
  A.exp2_256 = H.exp2_256;
  A.kk = H.rbf_k;
  A.kr = H.rbf_kr;
  A.gamma = c.gamma;
  A.rc = c.rc;
  A.inv_avg = c.inv_avg;
  A.palpha = palpha;
  return A;
}

// permute_mfma with each K chunk's columns in the order k = 16 T + 4 (lane
// / 16) + v: the B operand of MFMA v then holds, in lane group g, channel
// 16 T + 4 g + v, so a lane's four values of a chunk are contiguous in a row
// (K a multiple of 16)
std::vector<double> permute_mfma_kc(const std::vector<double> &w, std::size_t M, std::size_t K) {
  const std::size_t MT = (M + 15) / 16, KT = K / 16;
  std::vector<double> p(MT * KT * 64 * 4, 0.0);
  for (std::size_t mt = 0; mt < MT; ++mt)
    for (std::size_t T = 0; T < KT; ++T)
      for (std::size_t lane = 0; lane < 64; ++lane)
        for (std::size_t v = 0; v < 4; ++v) {
          const std::size_t row = 16 * mt + lane % 16, col = 16 * T + 4 * (lane / 16) + v;
          if (row < M) p[((mt * KT + T) * 64 + lane) * 4 + v] = w[row * K + col];
        }
  return p;
}

// run f, under c.timed when the evaluator is timing kernels
void section(const GContext &c, const char *name, const std::function<void()> &f) {
  if (c.timed) c.timed(name, f);
  else f();
}
}  // namespace

GenericPath::GenericPath(const Model &m, const std::function<const double *(const std::vector<double> &)> &up,
                         bool fit_radial) {
  const Architecture &a = m.arch();
  GDims &d = d_;
  d.F = a.F;
  d.NH = a.heads;
  d.R = a.R;
  d.FH = a.F / 4;
  d.HK = a.head_hidden;
  d.NI = a.F + a.heads;
  d.c6 = a.c6_head ? 1 : 0;
  d.HO = 2 * d.HK + 64 + (d.c6 ? 64 : 0);
  if ((d.F != 128 && d.F != 256) || d.NH * 32 != d.F)
    throw std::logic_error("SO3LR: generic path given widths other than F = 128 or 256 in heads of 32");
  int off = 0;
  d.off[0] = 0;
  for (int s = 0; s < d.NH; ++s) {
    const int l = a.degrees[std::size_t(s)];
    for (int k = 0; k < 2 * l + 1; ++k) {
      d.slot[off + k] = static_cast<signed char>(s);
      d.sh[off + k] = static_cast<signed char>(l * l - 1 + k);  // unique harmonics of l start at l^2 - 1
    }
    off += 2 * l + 1;
    d.off[s + 1] = static_cast<signed char>(off);
    d.par[s] = (l & 1) ? -1.0 : 1.0;
  }
  d.E = off;
  for (int m = 0; m < 24; ++m) d.shn[m] = 0;
  for (int c = 0; c < d.E; ++c) {
    const int m = d.sh[c];
    d.shc[m][int(d.shn[m])] = static_cast<signed char>(c);
    d.shn[m] = static_cast<signed char>(d.shn[m] + 1);
  }
  layers_ = a.layers;
  const std::size_t F = std::size_t(d.F), R = std::size_t(d.R), FH = std::size_t(d.FH), NH = std::size_t(d.NH),
                    NI = std::size_t(d.NI), E = std::size_t(d.E), HK = std::size_t(d.HK), HH = 64;
  for (int b = 0; b < layers_; ++b) {
    const std::string p = "model.euclidean_transformers." + std::to_string(b) + ".";
    const std::string at = p + "euclidean_attention_block.";
    GBlock &B = bw_[b];
    std::vector<double> qkv;
    for (const char *nm : {"W_q_inv", "W_k_inv", "W_v_inv", "W_q_ev", "W_k_ev"}) {
      const auto w = m.f64(at + nm, {NH, 32, 32});
      qkv.insert(qkv.end(), w.begin(), w.end());
    }
    B.wqkv = up(qkv);
    for (int k = 0; k < 2; ++k) {
      // the transformer-level filter nets (kokkos_integrated_block0.cpp:507-512)
      const std::string f = p + (k == 0 ? "filter_net_inv." : "filter_net_ev.");
      B.w0[k] = up(m.f64(f + "mlp_rbf.0.weight", {F, R}));
      B.b0[k] = up(m.f64(f + "mlp_rbf.0.bias", {F}));
      {
        // the fused kernels' operands (g_filt_fwd, g_filt_bwd, g_b0_fwd, g_b0_bwd)
        const auto w0 = m.f64(f + "mlp_rbf.0.weight", {F, R});
        const auto e0 = m.f64(f + "mlp_ev.0.weight", {FH, NH});
        std::vector<double> e0k(FH * 16, 0.0);  // K (the NH slots) padded to 16
        for (std::size_t o = 0; o < FH; ++o)
          for (std::size_t i = 0; i < NH; ++i) e0k[o * 16 + i] = e0[o * NH + i];
        B.w0p[k] = up(permute_mfma(w0, F, R));
        B.w0tp[k] = up(permute_mfma(transpose(w0, F, R), R, F));
        B.e0p[k] = up(permute_mfma(e0k, FH, 16));
        B.e0tp[k] = up(permute_mfma(transpose(e0, FH, NH), NH, FH));
        B.b0a[k] = up(bias_acc(m.f64(f + "mlp_rbf.0.bias", {F}), F));
        B.eb0a[k] = up(bias_acc(m.f64(f + "mlp_ev.0.bias", {FH}), FH));
      }
      B.w1[k] = up(m.f64(f + "mlp_rbf.mlp_rbf_layer_1.0.weight", {F, F}));
      B.b1[k] = up(m.f64(f + "mlp_rbf.mlp_rbf_layer_1.0.bias", {F}));
      B.e0[k] = up(m.f64(f + "mlp_ev.0.weight", {FH, NH}));
      B.eb0[k] = up(m.f64(f + "mlp_ev.0.bias", {FH}));
      B.e1[k] = up(m.f64(f + "mlp_ev.mlp_ev_layer_1.0.weight", {F, FH}));
      B.eb1[k] = up(m.f64(f + "mlp_ev.mlp_ev_layer_1.0.bias", {F}));
      {
        const auto w1 = m.f64(f + "mlp_rbf.mlp_rbf_layer_1.0.weight", {F, F});
        const auto e1 = m.f64(f + "mlp_ev.mlp_ev_layer_1.0.weight", {F, FH});
        auto bc = m.f64(f + "mlp_rbf.mlp_rbf_layer_1.0.bias", {F});
        const auto eb1 = m.f64(f + "mlp_ev.mlp_ev_layer_1.0.bias", {F});
        std::vector<double> wc(F * (F + FH));
        for (std::size_t o = 0; o < F; ++o) {
          for (std::size_t i = 0; i < F; ++i) wc[o * (F + FH) + i] = w1[o * F + i];
          for (std::size_t i = 0; i < FH; ++i) wc[o * (F + FH) + F + i] = e1[o * FH + i];
          bc[o] += eb1[o];
        }
        B.wcat[k] = up(wc);
        B.bcat[k] = up(bc);
        // the forward's output rows permuted within each tile (g_filt_fwd)
        std::vector<double> wcr(wc.size()), bcr(F);
        for (std::size_t o = 0; o < F; ++o) {
          const std::size_t src = 16 * (o / 16) + 4 * (o % 4) + (o % 16) / 4;
          std::copy(wc.begin() + std::ptrdiff_t(src * (F + FH)), wc.begin() + std::ptrdiff_t((src + 1) * (F + FH)),
                    wcr.begin() + std::ptrdiff_t(o * (F + FH)));
          bcr[o] = bc[src];
        }
        B.wcp[k] = up(permute_mfma(wcr, F, F + FH));
        B.bca[k] = up(bias_acc(bcr, F));
        B.wctp[k] = up(permute_mfma_kc(transpose(wc, F, F + FH), F + FH, F));
      }
    }
    B.att_cg = up(m.f64(at + "so3_conv_invariants.cg_rep", {E}));
    B.int_cg = up(m.f64(p + "interaction_block.so3_conv_invariants.cg_rep", {E}));
    const std::vector<double> ones(F, 1.0), zeros(F, 0.0);
    const bool ln1 = a.norm1 == NormMode::Layer, ln2 = a.norm2 == NormMode::Layer;
    B.ln1w = up(ln1 ? m.f64(p + "layer_norm_inv_1.weight", {F}) : ones);
    B.ln1b = up(ln1 ? m.f64(p + "layer_norm_inv_1.bias", {F}) : zeros);
    B.ln2w = up(ln2 ? m.f64(p + "layer_norm_inv_2.weight", {F}) : ones);
    B.ln2b = up(ln2 ? m.f64(p + "layer_norm_inv_2.bias", {F}) : zeros);
    B.m1 = up(m.f64(p + "mlp_1.1.weight", {F, F}));
    B.m1b = up(m.f64(p + "mlp_1.1.bias", {F}));
    B.m2 = up(m.f64(p + "mlp_1.3.weight", {F, F}));
    B.m2b = up(m.f64(p + "mlp_1.3.bias", {F}));
    B.wi = up(m.f64(p + "interaction_block.linear_layer.weight", {NI, NI}));
    B.bi = up(m.f64(p + "interaction_block.linear_layer.bias", {NI}));
  }
  const std::string e = "model.atomic_energy_output_block.", q = "model.partial_charges_output_block.",
                    h = "model.hirshfeld_output_block.", c6h = "model.c6_ratios_output_block.";
  std::vector<double> w1 = m.f64(e + "layers.0.weight", {HK, F});
  std::vector<double> b1 = m.f64(e + "layers.0.bias", {HK});
  auto append = [](std::vector<double> &dst, const std::vector<double> &src) { dst.insert(dst.end(), src.begin(), src.end()); };
  append(w1, m.f64(q + "transform_inv_features.0.weight", {HK, F}));
  append(b1, m.f64(q + "transform_inv_features.0.bias", {HK}));
  append(w1, m.f64(h + "transform_features.0.weight", {HH, F}));
  append(b1, m.f64(h + "transform_features.0.bias", {HH}));
  if (d.c6) {
    append(w1, m.f64(c6h + "transform_features.0.weight", {HH, F}));
    append(b1, m.f64(c6h + "transform_features.0.bias", {HH}));
  }
  hw_.w1 = up(w1);
  hw_.b1 = up(b1);
  hw_.hw2 = up(m.f64(h + "transform_features.2.weight", {HH, HH}));
  hw_.hb2 = up(m.f64(h + "transform_features.2.bias", {HH}));
  hw_.hqemb = up(m.f64(h + "q_embedding.weight", {100, HH}));
  hw_.hvshift = up(m.f64(h + "v_shift_embedding.weight", {100, 1}));
  hw_.cw2 = hw_.cb2 = hw_.cqemb = hw_.cvshift = nullptr;
  if (d.c6) {
    hw_.cw2 = up(m.f64(c6h + "transform_features.2.weight", {HH, HH}));
    hw_.cb2 = up(m.f64(c6h + "transform_features.2.bias", {HH}));
    hw_.cqemb = up(m.f64(c6h + "q_embedding.weight", {100, HH}));
    hw_.cvshift = up(m.f64(c6h + "v_shift_embedding.weight", {100, 1}));
  }
  hw_.ew2 = up(m.f64(e + "final_layer.weight", {1, HK}));
  hw_.eb2 = m.f64(e + "final_layer.bias", {1})[0];
  hw_.qw2 = up(m.f64(q + "transform_inv_features.2.weight", {1, HK}));
  hw_.qb2 = m.f64(q + "transform_inv_features.2.bias", {1})[0];
  hw_.escale = up(m.f64(e + "energy_scales.weight", {1, 118}));
  hw_.eshift = up(m.f64(e + "energy_shifts", {118}));
  hw_.qemb = up(m.f64(q + "atomic_embedding.weight", {100, 1}));
  hw_.rbf_b = up(m.f64("model.radial_embedding.radial_basis_fn.b", {R}));
  const auto kk = m.i64("model.radial_embedding.radial_basis_fn.k", {R});
  const auto kr = m.i64("model.radial_embedding.radial_basis_fn.k_rev", {R});
  hw_.rbf_k = up(std::vector<double>(kk.begin(), kk.end()));
  hw_.rbf_kr = up(std::vector<double>(kr.begin(), kr.end()));
  std::vector<double> t(256);
  for (int j = 0; j < 256; ++j) t[std::size_t(j)] = double(std::exp2(static_cast<long double>(j) / 256.0L));
  hw_.exp2_256 = up(t);
  // block 0's radial hidden layers as piecewise polynomials (radial tables),
  // used when both filters fit to within 1e-14 (values) and 1e-13 (slopes)
  // of their largest magnitudes at the check points
  if (fit_radial) {
    const auto bb = m.f64("model.radial_embedding.radial_basis_fn.b", {R});
    std::vector<double> val, slope;
    bool ok = true;
    for (int k = 0; k < 2 && ok; ++k) {
      const std::string f = std::string("model.euclidean_transformers.0.") + (k ? "filter_net_ev." : "filter_net_inv.");
      try {
        const RadialFit fit = fit_radial_hidden(m.f64(f + "mlp_rbf.0.weight", {F, R}), m.f64(f + "mlp_rbf.0.bias", {F}),
                                                int(F), int(R), bb, a.gamma, a.sr_cutoff, kRadialIntervals,
                                                kRadialDegree);
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
  // the blocks after 0: each filter's radial branch W1 h(r) + b1 + e1 as
  // piecewise polynomials (32 intervals of degree 31, the same bound), per
  // interval and filter an F x 32 coefficient tile with the output rows
  // permuted within each tile as wcp's (g_filt_fwd's channel order)
  if (fit_radial && layers_ > 1) {
    const auto bb = m.f64("model.radial_embedding.radial_basis_fn.b", {R});
    bool ok = true;
    std::vector<std::vector<double>> rows(static_cast<std::size_t>(layers_)), drs(static_cast<std::size_t>(layers_));
    RadialDomain dom{};
    for (int b = 1; b < layers_ && ok; ++b) {
      std::vector<RadialFit> fits;
      for (int k = 0; k < 2 && ok; ++k) {
        const std::string f = "model.euclidean_transformers." + std::to_string(b) + "." +
                              (k ? "filter_net_ev." : "filter_net_inv.");
        const auto w1 = m.f64(f + "mlp_rbf.mlp_rbf_layer_1.0.weight", {F, F});
        auto bc = m.f64(f + "mlp_rbf.mlp_rbf_layer_1.0.bias", {F});
        const auto eb1 = m.f64(f + "mlp_ev.mlp_ev_layer_1.0.bias", {F});
        for (std::size_t c = 0; c < F; ++c) bc[c] += eb1[c];
        try {
          fits.push_back(fit_radial_hidden(m.f64(f + "mlp_rbf.0.weight", {F, R}), m.f64(f + "mlp_rbf.0.bias", {F}),
                                           int(F), int(R), bb, a.gamma, a.sr_cutoff, kBlockIntervals, kBlockDegree,
                                           &w1, &bc, int(F)));
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
          std::vector<double> cv(F * n);
          for (std::size_t o = 0; o < F; ++o) {
            const std::size_t src = 16 * (o / 16) + 4 * (o % 4) + (o % 16) / 4;
            for (std::size_t kk = 0; kk < n; ++kk) cv[o * n + kk] = ft.value[(std::size_t(i) * n + kk) * F + src];
          }
          const auto pr = permute_mfma(cv, F, n);
          rows[std::size_t(b)].insert(rows[std::size_t(b)].end(), pr.begin(), pr.end());
          // the slopes transposed, channels in natural order (the reverse's df)
          std::vector<double> st(n * F);
          for (std::size_t kk = 0; kk < n; ++kk)
            for (std::size_t o = 0; o < F; ++o) st[kk * F + o] = ft.slope[(std::size_t(i) * n + kk) * F + o];
          const auto pd = permute_mfma_kc(st, n, F);
          drs[std::size_t(b)].insert(drs[std::size_t(b)].end(), pd.begin(), pd.end());
        }
      dom = RadialDomain{fits[0].r0, fits[0].step, fits[0].scale, fits[0].intervals};
    }
    if (ok) {
      for (int b = 1; b < layers_; ++b) {
        bw_[b].rrow = up(rows[std::size_t(b)]);
        bw_[b].rdr = up(drs[std::size_t(b)]);
      }
      rbl_dom_ = dom;
      radial_blocks_ok_ = true;
    }
  }
}

void GenericPath::carve(int N, int cap, int C, const std::function<double *(int, std::size_t)> &take) {
  const std::size_t n = std::size_t(N), P = std::size_t(std::max(cap, 1)), L = std::size_t(layers_);
  const std::size_t F = std::size_t(d_.F), E = std::size_t(d_.E), NH = std::size_t(d_.NH), NI = std::size_t(d_.NI),
                    R = std::size_t(d_.R), HO = std::size_t(d_.HO);
  const std::size_t sizes[NBUF] = {
      (L + 1) * n * F, (L + 1) * n * E, L * n * 5 * F, L * n * 4 * NH, L * n * E, L * n * F, L * n * F, L * n,
      L * n * F, L * n * NI, L * n * F, L * n,
      n * F, n * F, n * NI, n * HO, n * HO, n * 128, n * HO,
      n * F, n * E, n * NI, n * NI, n * E, n * F, n * F, n * F, n * F, n * 5 * F,
      // the pairs' basis rows, s, filter rows (none for block 0 on the
      // element-pair tables), logits, the logits' adjoints, dE/dfc, dE/ds
      P * R, L * P * NH, (L - (C > 0 ? 1 : 0)) * P * 2 * F, L * P * 4 * NH, P * 4 * NH, P, P * NH,
      // block 0's element-pair tables (g_cls_tables): per filter and key the
      // rows as 16 x F operands of both orientations, and their biases
      std::size_t(C) * C * 64 * F, std::size_t(C) * C * 4 * NH};
  for (int i = 0; i < NBUF; ++i) b_[i] = take(i, sizes[i]);
}

// block b's filter rows (2 F per pair); block 0 on the element-pair tables
// has none
double *GenericPath::pf_rows(const GContext &c, int b) const {
  const int first = cls_on(c) ? 1 : 0;
  return b < first ? nullptr : b_[PF] + std::size_t(b - first) * std::size_t(std::max(c.cap, 1)) * 2 * d_.F;
}

void GenericPath::forward(const GContext &c) {
  const GDims &d = d_;
  const hipStream_t s = c.s;
  const int N = c.N, cap = c.cap, F = d.F, E = d.E, NH = d.NH, NI = d.NI, R = d.R, FH = d.FH;
  const std::size_t n = std::size_t(N), P = std::size_t(std::max(cap, 1));
  const unsigned g4 = blocks_for(n, 4), g4x = (g4 + 7) / 8 * 8;  // g4x: g_xcd_block's grids
  const unsigned gP = blocks_for(P, 256);
  double *xs = b_[XS], *evs = b_[EVS];
  G_CHECK(hipMemcpyAsync(xs, c.x0, n * F * sizeof(double), hipMemcpyDeviceToDevice, s));
  if (!c.resid->empty())
    hipLaunchKernelGGL(g_axpby, dim3(blocks_for(n * F, 256)), dim3(256), 0, s, n * F, (*c.resid)[0], xs,
                       (*c.x0l)[0], c.x0);
  hipLaunchKernelGGL(g_fill, dim3(blocks_for(n * E, 256)), dim3(256), 0, s, evs, n * E);
  // the basis rows, read by the full filter chains only: not when every
  // block runs on its radial tables
  if (!(c.rint_order && cls_on(c) && c.rad_tab))
    hipLaunchKernelGGL(g_rbf, dim3(gP), dim3(256), 0, s, R, c.nact, cap, c.pr, c.gamma, hw_.rbf_b, hw_.rbf_k,
                       hw_.rbf_kr, b_[RBF]);
  for (int b = 0; b < layers_; ++b) {
    const GBlock &B = bw_[b];
    double *xb = xs + b * n * F, *evb = evs + b * n * E;
    double *qb = b_[QKV] + b * n * 5 * F, *aevb = b_[AEV] + b * n * E;
    double *n1b = b_[N1] + b * n * F, *n1hb = b_[N1HAT] + b * n * F, *n1ib = b_[N1IS] + b * n;
    double *hpb = b_[HPRE] + b * n * F, *tb = b_[TOUT] + b * n * NI;
    double *p2h = b_[PRE2HAT] + b * n * F, *p2i = b_[PRE2IS] + b * n;
    double *psb = b_[PS] + b * P * NH, *pfb = pf_rows(c, b), *pab = b_[PALPHA] + b * P * 4 * NH;
    // q k v q_ev k_ev per head: out[w][h*32 + o] = sum_k x[h*32 + k] W[w][h][k][o]
    // (kokkos_integrated_block0.cpp:257-287), batch z = w NH + h
    gemm_heads<EPI_STORE, true>(s, N, 5, NH, xb, F, 0, 32, B.wqkv, 1024, qb, 5 * F, F, 32);
    if (c.qk_norm)
      hipLaunchKernelGGL(g_qk_norm, dim3(blocks_for(n * 4 * NH, 256)), dim3(256), 0, s, N, F, NH, qb,
                         b_[QKIS] + b * n * 4 * NH);
    if (b == 0 && cls_on(c)) {
      // block 0 through the element-pair tables: their rows as MFMA
      // operands, then both filters to the logits in one fused kernel
      const std::size_t NK = std::size_t(c.cls_C) * c.cls_C;
      if (!c.rad_tab || c.rad_build)  // with the radial tables filled, nothing reads these
        hipLaunchKernelGGL(g_cls_tables, dim3(unsigned(NK * 16), 2), dim3(unsigned(F)), 0, s, F, NH, FH, c.cls_C, qb,
                           c.cls_rep, B.wcat[0], B.wcat[1], B.bcat[0], B.bcat[1], B.eb0[0], B.eb0[1], b_[CLS_M],
                           b_[CLS_M] + NK * 32 * F, b_[CLS_B]);
      if (c.rad_tab) {
        // the logits from the radial tables (filled once after set_system)
        const std::size_t keys = std::size_t(c.cls_C) * (c.cls_C + 1) / 2;
        if (c.rad_build)
          hipLaunchKernelGGL(g_radial_tables, dim3(unsigned(keys * kRadialIntervals)), dim3(256), 0, s, F, NH, c.cls_C,
                             b_[CLS_M], b_[CLS_B], rad_val_, rad_slope_, rad_dom_, c.rad_tab,
                             c.rad_tab + keys * kRadialIntervals * radial_record());
        section(c, "generic_filter_fwd_block0_radial",
                [&] { launch_radial<true>(s, NH, c, c.rad_tab, rad_dom_, pab, nullptr, nullptr); });
      } else {
        section(c, "generic_filter_fwd_block0_tables", [&] {
          launch_b0<true>(s, F, R, b0_slot_bound(c), b0_args(c, B, hw_, b_[RBF], b_[CLS_M], b_[CLS_B], F, pab));
        });
      }
    } else {
    // pair invariants and both filters (kokkos_integrated_block0.cpp:166-255)
    hipLaunchKernelGGL(g_pair_inv, dim3(blocks_for(P * NH, 256)), dim3(256), 0, s, d, c.nact, cap, c.pa, evb,
                       B.att_cg, psb);
    if (b > 0 && c.rint_order) {
      // the radial tables, in bucket order
      GRadArgs R{c.rint_slots, c.rint_order, c.pa, c.pr, psb, qb, B.rrow, rbl_dom_, {B.eb0a[0], B.eb0a[1]},
                 {B.e0p[0], B.e0p[1]}, {B.wcp[0], B.wcp[1]}, hw_.exp2_256, c.inv_avg, pfb, pab};
      const dim3 grid(blocks_for(std::size_t(std::max(c.rint_max, 1)), 64));
      section(c, "generic_filter_fwd_radial", [&] {
        if (F == 128) hipLaunchKernelGGL(g_radial_fwd_rows<8>, grid, dim3(256), 0, s, R);
        else hipLaunchKernelGGL(g_radial_fwd_rows<16>, grid, dim3(256), 0, s, R);
      });
    } else {
    // both filters' rows f = [W1 | E1] [silu(W0 rbf + b0) | silu(E0 s + e0)]
    // + b1 + e1 and the attention logits from them, fused
    section(c, "generic_filter_fwd", [&] {
      FiltArgs A = filt_args(c, B, hw_, b_[RBF], psb, qb, pfb);
      A.palpha = pab;
      launch_filt<true>(s, F, R, P, A);
    });
    }
    }
    hipLaunchKernelGGL(g_attn_msg, dim3(g4x), dim3(256), 0, s, d, N, c.inc_off, c.iact, c.iother, xb, evb, qb, c.pY,
                       c.pfc, pab, B.ln1w, B.ln1b, c.ln_eps, c.norm1, n1b, n1hb, n1ib, b_[ACT], aevb);
    // post-attention node chain (kokkos_post_attention_block0.cpp:165-300)
    gemm<EPI_SILU, false>(s, N, nullptr, F, F, b_[ACT], F, B.m1, B.m1b, b_[HID], F, nullptr, 0, nullptr, 0, hpb, F);
    gemm<EPI_ADD, false>(s, N, nullptr, F, F, b_[HID], F, B.m2, B.m2b, b_[CAT], NI, nullptr, 0, n1b, F);
    hipLaunchKernelGGL(g_cat_inv, dim3(blocks_for(n * NH, 256)), dim3(256), 0, s, d, N, aevb, B.int_cg, b_[CAT]);
    gemm<EPI_STORE, false>(s, N, nullptr, NI, NI, b_[CAT], NI, B.wi, B.bi, tb, NI);
    hipLaunchKernelGGL(g_node_post, dim3(g4), dim3(256), 0, s, d, N, b_[CAT], tb, aevb, B.ln2w, B.ln2b, c.ln_eps,
                       c.norm2, xs + (b + 1) * n * F, evs + (b + 1) * n * E, p2h, p2i);
    if (!c.resid->empty() && b + 1 < layers_)
      hipLaunchKernelGGL(g_axpby, dim3(blocks_for(n * F, 256)), dim3(256), 0, s, n * F, (*c.resid)[b + 1],
                         xs + (b + 1) * n * F, (*c.x0l)[b + 1], c.x0);
  }
  // output heads (kokkos_output_heads.cpp:137-176)
  const double *xf = xs + std::size_t(layers_) * n * F;
  gemm<EPI_SILU, false>(s, N, nullptr, F, d.HO, xf, F, hw_.w1, hw_.b1, b_[HACT], d.HO, nullptr, 0, nullptr, 0,
                        b_[HHPRE], d.HO);
  gemm<EPI_STORE, false>(s, N, nullptr, 64, 64, b_[HACT] + 2 * d.HK, d.HO, hw_.hw2, hw_.hb2, b_[HKEY], 128);
  if (d.c6)
    gemm<EPI_STORE, false>(s, N, nullptr, 64, 64, b_[HACT] + 2 * d.HK + 64, d.HO, hw_.cw2, hw_.cb2, b_[HKEY] + 64,
                           128);
  hipLaunchKernelGGL(g_heads, dim3(g4), dim3(256), 0, s, d, N, c.z, b_[HACT], b_[HKEY], hw_, c.eatom, c.qraw,
                     c.heff, c.hir, c.c6eff, c.c6r);
  G_CHECK(hipGetLastError());
}

void GenericPath::reverse(const GContext &c) {
  const GDims &d = d_;
  const hipStream_t s = c.s;
  const int N = c.N, cap = c.cap, F = d.F, E = d.E, NH = d.NH, NI = d.NI, R = d.R;
  const std::size_t n = std::size_t(N), P = std::size_t(std::max(cap, 1));
  const unsigned g4 = blocks_for(n, 4), g4x = (g4 + 7) / 8 * 8;  // g4x: g_xcd_block's grids
  // heads in reverse to dE/dx of the last block's output
  hipLaunchKernelGGL(g_heads_bwd, dim3(g4), dim3(256), 0, s, d, N, c.z, b_[HHPRE], c.qseed, c.dh, c.heff, c.dc,
                     c.c6eff, hw_, b_[GHEAD]);
  gemm<EPI_STORE, true>(s, N, nullptr, d.HO, F, b_[GHEAD], d.HO, hw_.w1, nullptr, b_[GX], F);
  hipLaunchKernelGGL(g_fill, dim3(blocks_for(n * E, 256)), dim3(256), 0, s, b_[GEV], n * E);
  double *gx = b_[GX], *gev = b_[GEV];
  for (int b = layers_ - 1; b >= 0; --b) {
    const GBlock &B = bw_[b];
    const double *evb = b_[EVS] + b * n * E;
    double *qb = b_[QKV] + b * n * 5 * F, *aevb = b_[AEV] + b * n * E;
    double *n1b = b_[N1] + b * n * F, *n1hb = b_[N1HAT] + b * n * F, *n1ib = b_[N1IS] + b * n;
    double *hpb = b_[HPRE] + b * n * F, *tb = b_[TOUT] + b * n * NI;
    double *p2h = b_[PRE2HAT] + b * n * F, *p2i = b_[PRE2IS] + b * n;
    double *psb = b_[PS] + b * P * NH, *pfb = pf_rows(c, b), *pab = b_[PALPHA] + b * P * 4 * NH;
    // post-attention chain in reverse (kokkos_post_attention_reverse.cpp:107-449)
    hipLaunchKernelGGL(g_ln2_bwd, dim3(g4), dim3(256), 0, s, d, N, gx, gev, tb, aevb, p2h, p2i, B.ln2w, c.norm2,
                       b_[GT], b_[GA]);
    gemm<EPI_STORE, true>(s, N, nullptr, NI, NI, b_[GT], NI, B.wi, nullptr, b_[GCAT], NI);
    hipLaunchKernelGGL(g_cat_bwd, dim3(blocks_for(n * (F + E), 256)), dim3(256), 0, s, d, N, b_[GT], b_[GCAT], aevb,
                       B.int_cg, b_[GP], b_[GA]);
    gemm<EPI_DSILU, true>(s, N, nullptr, F, F, b_[GP], F, B.m2, nullptr, b_[GHID], F, hpb, F);
    gemm<EPI_DSILU_ADD, true>(s, N, nullptr, F, F, b_[GHID], F, B.m1, nullptr, b_[GN1], F, n1b, F, b_[GP], F);
    hipLaunchKernelGGL(g_ln1_bwd, dim3(g4), dim3(256), 0, s, F, N, b_[GN1], B.ln1w, n1hb, n1ib, c.norm1, b_[GAINV]);
    // attention reverse per pair (kokkos_attention_scatter_reverse.cpp:280-500)
    const bool tables = b == 0 && cls_on(c);
    section(c, "generic_attn_bwd_pairs", [&] {
      hipLaunchKernelGGL(F == 256 ? g_attn_bwd_pairs<4> : g_attn_bwd_pairs<2>, dim3((blocks_for(P, 4) + 7) / 8 * 8),
                         dim3(256), 0,
                         s, d, c.nact, cap, c.pa, qb, c.pY, c.pfc, pab, b_[GAINV], b_[GA], c.inv_avg,
                         b == layers_ - 1 ? 1 : 0, b_[PSC], c.dY, b_[DFC]);
    });
    if (b > 0)
      hipLaunchKernelGGL(g_attn_bwd_node, dim3((blocks_for(n * (F / 64), 4) + 7) / 8 * 8), dim3(256), 0, s, d, N, c.inc_off, c.iact, c.iother, qb, pfb,
                         c.pfc, pab, b_[PSC], b_[GAINV], b_[GQKV]);
    // filter reverse (kokkos_block2_attention_input_reverse.cpp:198-336)
    if (tables && c.rad_tab) {
      // block 0 through the radial tables: the logits' adjoints times the
      // slopes to dE/dr
      const std::size_t keys = std::size_t(c.cls_C) * (c.cls_C + 1) / 2;
      section(c, "generic_filter_bwd_block0_radial", [&] {
        launch_radial<false>(s, NH, c, c.rad_tab + keys * kRadialIntervals * radial_record(), rad_dom_, nullptr,
                             b_[PSC], b_[DFC]);
      });
    } else if (tables) {
      // block 0 through the element-pair tables, fused: the hidden rows'
      // adjoints from the table rows, through W0 to dE/dr (the spherical
      // input s has no adjoint in block 0)
      B0Args A = b0_args(c, B, hw_, b_[RBF], b_[CLS_M], b_[CLS_B], F, pab);
      A.psc = b_[PSC];
      A.dfc = b_[DFC];
      A.dr = c.dr;
      section(c, "generic_filter_bwd_block0_tables",
              [&] { launch_b0<false>(s, F, R, b0_slot_bound(c), A); });
    } else if (b > 0 && c.rint_order) {
      // the radial tables, in bucket order: df against the slope tiles to
      // dE/dr, the spherical branch to dE/ds
      GRadArgs Rg{c.rint_slots, c.rint_order, c.pa, c.pr, psb, qb, B.rdr, rbl_dom_, {B.eb0a[0], B.eb0a[1]},
                  {B.e0p[0], B.e0p[1]}, {nullptr, nullptr}, hw_.exp2_256, c.inv_avg, nullptr, nullptr,
                  {B.e0tp[0], B.e0tp[1]}, {B.wctp[0], B.wctp[1]}, b_[PSC], b_[DFC], c.rc, b_[DS], c.dr};
      const dim3 grid(blocks_for(std::size_t(std::max(c.rint_max, 1)), 64));
      section(c, "generic_filter_bwd_radial", [&] {
        if (F == 128) hipLaunchKernelGGL(g_radial_bwd_rows<8>, grid, dim3(256), 0, s, Rg);
        else hipLaunchKernelGGL(g_radial_bwd_rows<16>, grid, dim3(256), 0, s, Rg);
      });
    } else {
      // both filters fused: d hidden = [W1 | E1]^T df (df from the logits'
      // adjoints psc), (.) silu'(pre), through W0^T and E0^T to dE/dr and
      // dE/ds
      FiltArgs A = filt_args(c, B, hw_, b_[RBF], psb, qb, nullptr);
      A.psc = b_[PSC];
      A.dfc = b_[DFC];
      A.ds = b_[DS];
      A.dr = c.dr;
      section(c, "generic_filter_bwd", [&] { launch_filt<false>(s, F, R, P, A); });
    }
    // the adjoints of the block's inputs feed the block below; block 0's
    // inputs (embedding, ev = 0) do not depend on the positions
    if (b > 0) {
      if (c.qk_norm)
        hipLaunchKernelGGL(g_qk_norm_bwd, dim3(blocks_for(n * 4 * NH, 256)), dim3(256), 0, s, N, F, NH, qb,
                           b_[QKIS] + b * n * 4 * NH, b_[GQKV]);
      // gx = gainv + sum_w gqkv[w] W[w]^T per head, batch z = h
      for (int w = 0; w < 5; ++w) {
        if (w == 0)
          gemm_heads<EPI_ADD, false>(s, N, 1, NH, b_[GQKV], 5 * F, 0, 32, B.wqkv, 1024, gx, F, 0, 32, b_[GAINV], F,
                                     0, 32);
        else
          gemm_heads<EPI_ACCUM, false>(s, N, 1, NH, b_[GQKV] + w * F, 5 * F, 0, 32, B.wqkv + std::size_t(w) * NH * 1024,
                                       1024, gx, F, 0, 32);
      }
      if (!c.resid->empty())
        hipLaunchKernelGGL(g_scale, dim3(blocks_for(n * F, 256)), dim3(256), 0, s, n * F, (*c.resid)[b], gx);
      hipLaunchKernelGGL(g_ev_bwd, dim3(g4x), dim3(256), 0, s, d, N, c.inc_off, c.iact, c.iother, evb, B.att_cg,
                         b_[DS], b_[GA], gev);
    }
  }
  G_CHECK(hipGetLastError());
}

}  // namespace so3lr_amd
