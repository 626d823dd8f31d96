// Piecewise polynomial fits of a filter's radial hidden layer, for block 0's
// radial tables (host side; the kernels are in evaluator.hip and generic.hip),
// and of a whole radial branch W1 h(r) + bias for the blocks after 0.
//
// The radial branch of a filter is h(r) = silu(W0 b(r) + b0), b the Bernstein
// basis of x = e^{-gamma r} (kokkos_integrated_block0.cpp:117-160, 194-255).
// On [r0, r1] (r0: where the clamp x <= 1 - 1e-6 lets go; r1: the cutoff)
// cut into equal intervals i with left edges e_i = fma(i, width, r0), every
// feature of h and of dh/dr is fitted on each interval by its Chebyshev
// interpolant of the given degree in t = (r - e_i) * scale - 1
// (scale = 2 / width), evaluated in long double at the Chebyshev nodes and
// stored as monomial coefficients in t.  Block 0's attention logits are
// linear in h, so their tables are these coefficients contracted with the
// element pairs' query/key products on the device.
#pragma once

#include <vector>

namespace so3lr_amd {

// Block 0's radial tables: intervals and polynomial degree of the fits, and
// their domain as the kernels read it (intervals of width step from r0,
// t = (r - left edge) * scale - 1)
constexpr int kRadialIntervals = 256, kRadialDegree = 13, kRadialCoefs = kRadialDegree + 1;
// The blocks after 0: coarser intervals of higher degree (32 powers: two
// MFMA K chunks), so that their pairs, bucketed by (spatial block of
// kRintAtoms nodes, interval), keep a block's endpoint rows in L2
constexpr int kBlockIntervals = 32, kBlockDegree = 31, kBlockPowers = kBlockDegree + 1, kRintAtoms = 256;
struct RadialDomain {
  double r0, step, scale;
  int intervals;
};

struct RadialFit {
  int intervals = 0, degree = 0, width = 0;
  double r0 = 0.0, r1 = 0.0, step = 0.0, scale = 0.0;  // domain, interval width, 2 / width
  // [interval][power][feature]: coefficient of t^power
  std::vector<double> value, slope;  // h and dh/dr
  // largest |fit - h| (|fit' - h'|) over every feature at check points
  // between the nodes, over the largest |h| (|h'|) seen
  double value_error = 0.0, slope_error = 0.0;
};

// w0: (width, nbasis) row-major; b0: (width); basis_b: (nbasis) log prefactors
// of the Bernstein basis, exponents c and nbasis - 1 - c.  With w1 (outputs,
// width) row-major and bias (outputs) given, the fit is of the filter's
// radial branch w1 h(r) + bias instead (RadialFit::width = outputs).  Throws
// std::invalid_argument when the far clamp of x (x >= 1e-6) falls inside
// the domain.
RadialFit fit_radial_hidden(const std::vector<double> &w0, const std::vector<double> &b0, int width, int nbasis,
                            const std::vector<double> &basis_b, double gamma, double r_cut, int intervals,
                            int degree, const std::vector<double> *w1 = nullptr,
                            const std::vector<double> *bias = nullptr, int outputs = 0);

}  // namespace so3lr_amd
