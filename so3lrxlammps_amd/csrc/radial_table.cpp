#include "radial_table.hpp"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <functional>
#include <mutex>
#include <stdexcept>
#include <thread>

namespace so3lr_amd {

namespace {

using LD = long double;
constexpr LD kPi = 3.141592653589793238462643383279502884L;

struct Net {
  const std::vector<double> &w0, &b0, &bb;
  int F, R;
  LD gamma;
  const std::vector<double> *w1, *bias;  // optional output layer (O, F), (O)
  int O;                                 // outputs: O with w1, F without
};

// h and dh/dr of every feature at r >= r0 (x below its clamp)
void hidden_at(const Net &n, LD r, LD *h, LD *dh, std::vector<LD> &bas, std::vector<LD> &dbas);

// the fitted function at r: h, or w1 h + bias with the output layer;
// hs, dhs: work rows of F
void output_at(const Net &n, LD r, LD *y, LD *dy, std::vector<LD> &bas, std::vector<LD> &dbas, LD *hs, LD *dhs) {
  if (!n.w1) {
    hidden_at(n, r, y, dy, bas, dbas);
    return;
  }
  hidden_at(n, r, hs, dhs, bas, dbas);
  for (int c = 0; c < n.O; ++c) {
    const double *w = n.w1->data() + std::size_t(c) * n.F;
    LD v = (*n.bias)[c], dv = 0.0L;
    for (int f = 0; f < n.F; ++f) {
      v += LD(w[f]) * hs[f];
      dv += LD(w[f]) * dhs[f];
    }
    y[c] = v;
    dy[c] = dv;
  }
}

void hidden_at(const Net &n, LD r, LD *h, LD *dh, std::vector<LD> &bas, std::vector<LD> &dbas) {
  const LD lx = -n.gamma * r, x = std::exp(lx), l1x = std::log1p(-x), q = x / (1.0L - x);
  for (int c = 0; c < n.R; ++c) {
    const LD kc = c, kr = n.R - 1 - c;
    bas[c] = std::exp(LD(n.bb[c]) + kc * lx + kr * l1x);
    dbas[c] = -n.gamma * bas[c] * (kc - kr * q);
  }
  for (int f = 0; f < n.F; ++f) {
    LD pre = n.b0[f], dpre = 0.0L;
    const double *w = n.w0.data() + std::size_t(f) * n.R;
    for (int c = 0; c < n.R; ++c) {
      pre += LD(w[c]) * bas[c];
      dpre += LD(w[c]) * dbas[c];
    }
    const LD s = 1.0L / (1.0L + std::exp(-pre));
    h[f] = pre * s;
    dh[f] = s * (1.0L + pre * (1.0L - s)) * dpre;
  }
}

}  // namespace

namespace {

// Fits already made in this process, by the exact bytes of their inputs
// (contexts of one model fit the same layers again): at most kCacheSize.
struct CacheEntry {
  std::vector<double> key;
  RadialFit fit;
};
constexpr std::size_t kCacheSize = 16;
std::mutex cache_mutex;
std::vector<CacheEntry> cache;

std::vector<double> cache_key(const std::vector<double> &w0, const std::vector<double> &b0, int width, int nbasis,
                              const std::vector<double> &basis_b, double gamma, double r_cut, int intervals,
                              int degree, const std::vector<double> *w1, const std::vector<double> *bias,
                              int outputs) {
  std::vector<double> k{double(width), double(nbasis), gamma, r_cut, double(intervals), double(degree),
                        double(outputs), w1 ? 1.0 : 0.0};
  for (const std::vector<double> *v : {&w0, &b0, &basis_b}) k.insert(k.end(), v->begin(), v->end());
  if (w1) {
    k.insert(k.end(), w1->begin(), w1->end());
    k.insert(k.end(), bias->begin(), bias->end());
  }
  return k;
}

bool same_bytes(const std::vector<double> &a, const std::vector<double> &b) {
  return a.size() == b.size() && std::memcmp(a.data(), b.data(), a.size() * sizeof(double)) == 0;
}

RadialFit fit_uncached(const std::vector<double> &w0, const std::vector<double> &b0, int width, int nbasis,
                       const std::vector<double> &basis_b, double gamma, double r_cut, int intervals, int degree,
                       const std::vector<double> *w1, const std::vector<double> *bias, int outputs);

}  // namespace

RadialFit fit_radial_hidden(const std::vector<double> &w0, const std::vector<double> &b0, int width, int nbasis,
                            const std::vector<double> &basis_b, double gamma, double r_cut, int intervals,
                            int degree, const std::vector<double> *w1, const std::vector<double> *bias,
                            int outputs) {
  std::vector<double> key = cache_key(w0, b0, width, nbasis, basis_b, gamma, r_cut, intervals, degree, w1, bias, outputs);
  {
    std::lock_guard<std::mutex> lock(cache_mutex);
    for (const CacheEntry &e : cache)
      if (same_bytes(e.key, key)) return e.fit;
  }
  RadialFit fit = fit_uncached(w0, b0, width, nbasis, basis_b, gamma, r_cut, intervals, degree, w1, bias, outputs);
  std::lock_guard<std::mutex> lock(cache_mutex);
  if (cache.size() >= kCacheSize) cache.erase(cache.begin());
  cache.push_back(CacheEntry{std::move(key), fit});
  return fit;
}

namespace {

RadialFit fit_uncached(const std::vector<double> &w0, const std::vector<double> &b0, int width, int nbasis,
                       const std::vector<double> &basis_b, double gamma, double r_cut, int intervals, int degree,
                       const std::vector<double> *w1, const std::vector<double> *bias, int outputs) {
  if (width < 1 || nbasis < 2 || intervals < 1 || degree < 1 || gamma <= 0.0 || r_cut <= 0.0 ||
      w0.size() != std::size_t(width) * nbasis || b0.size() != std::size_t(width) ||
      basis_b.size() != std::size_t(nbasis) || (w1 != nullptr) != (bias != nullptr) ||
      (w1 && (outputs < 1 || w1->size() != std::size_t(outputs) * width || bias->size() != std::size_t(outputs))))
    throw std::invalid_argument("SO3LR: radial fit: inconsistent arguments");
  const LD g = gamma;
  // x = e^{-gamma r} stays at or above 1e-6 up to the cutoff
  if (-g * LD(r_cut) < std::log(1e-6L))
    throw std::invalid_argument("SO3LR: radial fit: the basis clamp x >= 1e-6 lies inside the cutoff");
  RadialFit fit;
  fit.intervals = intervals;
  fit.degree = degree;
  fit.width = w1 ? outputs : width;
  fit.r0 = double(-std::log1p(-1e-6L) / g);
  fit.r1 = r_cut;
  if (!(fit.r0 < fit.r1)) throw std::invalid_argument("SO3LR: radial fit: empty domain");
  fit.step = (fit.r1 - fit.r0) / intervals;
  fit.scale = 2.0 / fit.step;
  const int n = degree + 1, F = fit.width;  // F: the fitted functions
  fit.value.assign(std::size_t(intervals) * n * F, 0.0);
  fit.slope.assign(std::size_t(intervals) * n * F, 0.0);
  const Net net{w0, b0, basis_b, width, nbasis, g, w1, bias, F};

  // Chebyshev nodes, cos(pi k (j + 1/2) / n), and the monomial coefficients of T_k
  std::vector<LD> tn(n), ck(std::size_t(n) * n), tm(std::size_t(n) * n, 0.0L);
  for (int j = 0; j < n; ++j) {
    tn[j] = std::cos(kPi * (j + 0.5L) / n);
    for (int k = 0; k < n; ++k) ck[std::size_t(k) * n + j] = std::cos(kPi * k * (j + 0.5L) / n);
  }
  tm[0] = 1.0L;
  if (n > 1) tm[std::size_t(1) * n + 1] = 1.0L;
  for (int k = 2; k < n; ++k)
    for (int m = 0; m < n; ++m)
      tm[std::size_t(k) * n + m] =
          (m > 0 ? 2.0L * tm[std::size_t(k - 1) * n + m - 1] : 0.0L) - tm[std::size_t(k - 2) * n + m];

  // intervals split over up to 8 host threads, each with its own work arrays
  // and error maxima
  struct Part {
    LD err_v = 0.0L, err_d = 0.0L, max_v = 0.0L, max_d = 0.0L;
  };
  auto run = [&](int i0, int i1, Part &pt) {
    std::vector<LD> bas(nbasis), dbas(nbasis), hv(std::size_t(n) * F), dv(std::size_t(n) * F),
        cc(std::size_t(n) * F), he(F), de(F), hs(width), dhs(width);
    constexpr int kChecks = 9;  // t = -1, -0.75, ..., 1
    for (int i = i0; i < i1; ++i) {
      const double e = std::fma(double(i), fit.step, fit.r0);
      auto r_at = [&](LD t) { return LD(e) + (t + 1.0L) / LD(fit.scale); };
      for (int j = 0; j < n; ++j)
        output_at(net, r_at(tn[j]), &hv[std::size_t(j) * F], &dv[std::size_t(j) * F], bas, dbas, hs.data(),
                  dhs.data());
      for (int which = 0; which < 2; ++which) {
        const std::vector<LD> &y = which ? dv : hv;
        std::vector<double> &out = which ? fit.slope : fit.value;
        for (int k = 0; k < n; ++k)
          for (int f = 0; f < F; ++f) {
            LD s = 0.0L;
            for (int j = 0; j < n; ++j) s += y[std::size_t(j) * F + f] * ck[std::size_t(k) * n + j];
            cc[std::size_t(k) * F + f] = s * (k ? 2.0L : 1.0L) / n;
          }
        for (int m = 0; m < n; ++m)
          for (int f = 0; f < F; ++f) {
            LD s = 0.0L;
            for (int k = m; k < n; ++k) s += cc[std::size_t(k) * F + f] * tm[std::size_t(k) * n + m];
            out[(std::size_t(i) * n + m) * F + f] = double(s);
          }
      }
      // the stored (double) coefficients by Horner in double, as on the device
      for (int c = 0; c < kChecks; ++c) {
        const LD t = -1.0L + 2.0L * c / (kChecks - 1);
        output_at(net, r_at(t), he.data(), de.data(), bas, dbas, hs.data(), dhs.data());
        const double td = double(t);
        for (int f = 0; f < F; ++f) {
          double pv = fit.value[(std::size_t(i) * n + degree) * F + f];
          double pd = fit.slope[(std::size_t(i) * n + degree) * F + f];
          for (int m = degree - 1; m >= 0; --m) {
            pv = std::fma(pv, td, fit.value[(std::size_t(i) * n + m) * F + f]);
            pd = std::fma(pd, td, fit.slope[(std::size_t(i) * n + m) * F + f]);
          }
          pt.err_v = std::max(pt.err_v, std::fabs(LD(pv) - he[f]));
          pt.err_d = std::max(pt.err_d, std::fabs(LD(pd) - de[f]));
          pt.max_v = std::max(pt.max_v, std::fabs(he[f]));
          pt.max_d = std::max(pt.max_d, std::fabs(de[f]));
        }
      }
    }
  };
  const int nt = std::max(1, std::min({8, intervals, int(std::thread::hardware_concurrency())}));
  std::vector<Part> parts(nt);
  std::vector<std::thread> pool;
  for (int t = 1; t < nt; ++t)
    pool.emplace_back(run, intervals * t / nt, intervals * (t + 1) / nt, std::ref(parts[t]));
  run(0, intervals / nt, parts[0]);
  for (auto &th : pool) th.join();
  LD err_v = 0.0L, err_d = 0.0L, max_v = 0.0L, max_d = 0.0L;
  for (const Part &pt : parts) {
    err_v = std::max(err_v, pt.err_v);
    err_d = std::max(err_d, pt.err_d);
    max_v = std::max(max_v, pt.max_v);
    max_d = std::max(max_d, pt.max_d);
  }
  fit.value_error = double(err_v / std::max(max_v, LD(1e-300)));
  fit.slope_error = double(err_d / std::max(max_d, LD(1e-300)));
  return fit;
}

}  // namespace

}  // namespace so3lr_amd
