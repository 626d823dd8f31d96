// Spatial (Morton) order of the owned atoms, shared by the device reneighbor
// (neighbor.hip) and the LAMMPS-list path (topology.hip).  Node n of the
// evaluation holds owned atom perm[n]; the node-ordered copies of the
// per-atom inputs come from the gathers below, and the per-atom outputs are
// scattered back through perm, so callers keep their own atom order.
#pragma once

#include <hip/hip_runtime.h>

namespace so3lr_amd {
namespace {

// the box the positions are quantised in: lo and edge lengths
struct MortonBox {
  double lo[3], len[3];
};

// 10-bit spread for a 30-bit Morton key
__device__ __forceinline__ unsigned spread3(unsigned v) {
  v &= 1023u;
  v = (v | (v << 16)) & 0x030000FFu;
  v = (v | (v << 8)) & 0x0300F00Fu;
  v = (v | (v << 4)) & 0x030C30C3u;
  v = (v | (v << 2)) & 0x09249249u;
  return v;
}

__device__ __forceinline__ unsigned quantize(double v, double lo, double len) {
  const double t = (v - lo) / len * 1024.0;
  return t < 0.0 ? 0u : (t >= 1023.0 ? 1023u : unsigned(t));
}

__global__ void k_morton(int n, const double *x, MortonBox B, int *key, int *idx) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const unsigned qx = quantize(x[3 * i], B.lo[0], B.len[0]);
  const unsigned qy = quantize(x[3 * i + 1], B.lo[1], B.len[1]);
  const unsigned qz = quantize(x[3 * i + 2], B.lo[2], B.len[2]);
  key[i] = int((spread3(qx) << 2) | (spread3(qy) << 1) | spread3(qz));
  idx[i] = i;
}

__global__ void k_gather_int(int n, const int *perm, const int *src, int *dst) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = src[perm[i]];
}

// dst[n][c] = src[perm[n]][c] for rows of `width` doubles
__global__ void k_gather_rows(int n, int width, const int *perm, const double *src, double *dst) {
  const std::size_t k = std::size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (k >= std::size_t(n) * width) return;
  const std::size_t row = k / width, c = k % width;
  dst[k] = src[std::size_t(perm[row]) * width + c];
}

}  // namespace
}  // namespace so3lr_amd
