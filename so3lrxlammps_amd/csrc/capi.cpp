// C ABI of so3lr_hip (declared in include/so3lr_hip.h).
#include "../../include/so3lr_hip.h"

#include <cstring>
#include <exception>
#include <memory>
#include <new>
#include <stdexcept>
#include <string>
#include <vector>

#include "evaluator.hpp"
#include "model.hpp"

using so3lr_amd::Evaluator;
using so3lr_amd::Model;

struct so3lr_ctx {
  std::unique_ptr<Evaluator> ev;
  std::string error;
};

namespace {
thread_local std::string g_create_error;

// Map an exception to a status code; every failure keeps its message.
int fail(so3lr_ctx *ctx, const std::exception &e, int code) {
  if (ctx) ctx->error = e.what();
  else g_create_error = e.what();
  return code;
}

template <class F>
int guarded(so3lr_ctx *ctx, F &&body) {
  if (!ctx) return SO3LR_ERR_ARGUMENT;
  try {
    body();
    ctx->error.clear();
    return SO3LR_OK;
  } catch (const so3lr_amd::DeviceError &e) {
    return fail(ctx, e, SO3LR_ERR_DEVICE);
  } catch (const so3lr_amd::TopologyError &e) {
    return fail(ctx, e, SO3LR_ERR_TOPOLOGY);
  } catch (const std::invalid_argument &e) {
    return fail(ctx, e, SO3LR_ERR_ARGUMENT);
  } catch (const std::length_error &e) {
    return fail(ctx, e, SO3LR_ERR_TOPOLOGY);
  } catch (const std::domain_error &e) {
    return fail(ctx, e, SO3LR_ERR_SYSTEM);
  } catch (const std::logic_error &e) {
    return fail(ctx, e, SO3LR_ERR_STATE);
  } catch (const std::runtime_error &e) {
    return fail(ctx, e, SO3LR_ERR_MODEL);
  } catch (const std::exception &e) {  // std::bad_alloc and the like
    return fail(ctx, e, SO3LR_ERR_DEVICE);
  }
}
}  // namespace

extern "C" {

int so3lr_create(const char *model_path, int device, so3lr_ctx **out) {
  if (!out || !model_path) return SO3LR_ERR_ARGUMENT;
  *out = nullptr;
  // the LAMMPS-visible wording of PairSO3LRNativeMPI::settings
  // (plugins/lammps/pair_so3lr_native_mpi.cpp:1097-1137): the pair style
  // passes this message to error->all as it stands
  const std::string prefix = "Cannot initialize MPI-native SO3LR model: ";
  std::shared_ptr<Model> m;
  try {
    m = Model::load(model_path);
  } catch (const std::exception &e) {
    g_create_error = prefix + e.what();
    return SO3LR_ERR_MODEL;
  }
  std::unique_ptr<so3lr_ctx> ctx(new so3lr_ctx());
  try {
    ctx->ev = std::make_unique<Evaluator>(m, device);
  } catch (const so3lr_amd::DeviceError &e) {
    g_create_error = prefix + e.what();
    return SO3LR_ERR_DEVICE;
  } catch (const std::exception &e) {  // a tensor the kernels need is missing or misshapen
    g_create_error = prefix + e.what();
    return SO3LR_ERR_MODEL;
  }
  *out = ctx.release();
  g_create_error.clear();
  return SO3LR_OK;
}

void so3lr_destroy(so3lr_ctx *ctx) { delete ctx; }

const char *so3lr_last_error(const so3lr_ctx *ctx) {
  return ctx ? ctx->error.c_str() : g_create_error.c_str();
}

double so3lr_cutoff(const so3lr_ctx *ctx, int which) {
  if (!ctx || !ctx->ev) return 0.0;
  const auto &a = ctx->ev->model().arch();
  return which == 0 ? a.sr_cutoff : a.lr_cutoff;
}

int so3lr_atomic_number(const char *token) { return so3lr_amd::atomic_number_from_token(token); }

int so3lr_check_system(int64_t n, const int32_t *z, double total_charge, double multiplicity) {
  if (n <= 0 || !z) {
    g_create_error = "SO3LR: empty system";
    return SO3LR_ERR_ARGUMENT;
  }
  std::int64_t counts[119] = {0};
  for (int64_t i = 0; i < n; ++i) {
    if (z[i] < 1 || z[i] > 99) {
      g_create_error = "SO3LR: atomic numbers must lie in 1..99";
      return SO3LR_ERR_ARGUMENT;
    }
    ++counts[z[i]];
  }
  const std::string why = so3lr_amd::charge_multiplicity_problem(counts, total_charge, multiplicity);
  if (!why.empty()) {
    g_create_error = why;
    return SO3LR_ERR_SYSTEM;
  }
  g_create_error.clear();
  return SO3LR_OK;
}

int so3lr_set_system(so3lr_ctx *ctx, int64_t n_owned, const int32_t *z, double total_charge,
                     double multiplicity) {
  return guarded(ctx, [&] {
    if (n_owned <= 0 || !z) throw std::invalid_argument("SO3LR: empty system");
    std::vector<int32_t> zz(z, z + n_owned);
    ctx->ev->set_system(zz, {0, n_owned}, {total_charge}, {multiplicity});
  });
}

int so3lr_set_images(so3lr_ctx *ctx, int64_t n_owned, const int32_t *z, int64_t n_images,
                     const int64_t *image_offsets, const double *charges, const double *mults) {
  return guarded(ctx, [&] {
    if (n_owned <= 0 || !z || n_images <= 0 || !image_offsets || !charges || !mults)
      throw std::invalid_argument("SO3LR: invalid packed-image description");
    std::vector<int32_t> zz(z, z + n_owned);
    ctx->ev->set_system(zz, std::vector<int64_t>(image_offsets, image_offsets + n_images + 1),
                        std::vector<double>(charges, charges + n_images),
                        std::vector<double>(mults, mults + n_images));
  });
}

int so3lr_set_topology(so3lr_ctx *ctx, int64_t n_rows, const int32_t *owner, int sr_kind,
                       int64_t sr_inum, const int32_t *sr_ilist, const int64_t *sr_off,
                       const int32_t *sr_neigh, int64_t lr_inum, const int32_t *lr_ilist,
                       const int64_t *lr_off, const int32_t *lr_neigh) {
  return guarded(ctx, [&] {
    if (sr_kind != SO3LR_LIST_FULL && sr_kind != SO3LR_LIST_HALF)
      throw std::invalid_argument("SO3LR: unknown short-range list kind");
    ctx->ev->set_topology(n_rows, owner, sr_kind, sr_inum, sr_ilist, sr_off, sr_neigh, lr_inum, lr_ilist,
                          lr_off, lr_neigh);
  });
}

static int check_flags(int flags) {
  if (flags & ~(SO3LR_ENERGY | SO3LR_EATOM | SO3LR_VIRIAL | SO3LR_VATOM)) return SO3LR_ERR_ARGUMENT;
  return SO3LR_OK;
}

int so3lr_compute(so3lr_ctx *ctx, const double *x_rows, int flags, double *f, double *eatom,
                  double *energy, double *virial) {
  if (ctx && check_flags(flags) != SO3LR_OK) {
    ctx->error = "SO3LR: unknown compute flags";
    return check_flags(flags);
  }
  return guarded(ctx, [&] {
    if (!x_rows || !f) throw std::invalid_argument("SO3LR: positions and forces are required");
    if ((flags & SO3LR_EATOM) && !eatom) throw std::invalid_argument("SO3LR: eatom requested without a buffer");
    if ((flags & SO3LR_ENERGY) && !energy) throw std::invalid_argument("SO3LR: energy requested without a buffer");
    if ((flags & SO3LR_VIRIAL) && !virial) throw std::invalid_argument("SO3LR: virial requested without a buffer");
    ctx->ev->compute_host(x_rows, flags, f, eatom, energy, virial);
  });
}

int so3lr_compute_device(so3lr_ctx *ctx, const double *x_rows_dev, int flags, double *f_dev,
                         double *eatom_dev, double *energy, double *virial) {
  if (ctx && check_flags(flags) != SO3LR_OK) {
    ctx->error = "SO3LR: unknown compute flags";
    return check_flags(flags);
  }
  return guarded(ctx, [&] {
    if (!x_rows_dev || !f_dev) throw std::invalid_argument("SO3LR: positions and forces are required");
    if ((flags & SO3LR_EATOM) && !eatom_dev) throw std::invalid_argument("SO3LR: eatom requested without a buffer");
    ctx->ev->compute_device(x_rows_dev, flags, f_dev, (flags & SO3LR_EATOM) ? eatom_dev : nullptr, energy,
                            virial);
  });
}

int so3lr_compute_device_noalloc(so3lr_ctx *ctx, const double *x_rows_dev, int flags, double *f_dev,
                                 double *eatom_dev, double *energy, double *virial) {
  if (ctx && check_flags(flags) != SO3LR_OK) {
    ctx->error = "SO3LR: unknown compute flags";
    return check_flags(flags);
  }
  return guarded(ctx, [&] {
    if (!x_rows_dev || !f_dev) throw std::invalid_argument("SO3LR: positions and forces are required");
    if ((flags & SO3LR_EATOM) && !eatom_dev) throw std::invalid_argument("SO3LR: eatom requested without a buffer");
    ctx->ev->compute_device_noalloc(x_rows_dev, flags, f_dev, (flags & SO3LR_EATOM) ? eatom_dev : nullptr, energy,
                                    virial);
  });
}

int so3lr_reneighbor_device(so3lr_ctx *ctx, double *x_owned_dev, const double *lo, const double *hi,
                            const int *periodic, double skin) {
  return guarded(ctx, [&] {
    if (!x_owned_dev || !lo || !hi || !periodic || !(skin >= 0.0))
      throw std::invalid_argument("SO3LR: invalid device reneighbor arguments");
    ctx->ev->build_topology_device(x_owned_dev, lo, hi, periodic, skin);
  });
}

int so3lr_set_box(so3lr_ctx *ctx, const double *lo, const double *hi) {
  return guarded(ctx, [&] {
    if (!lo || !hi) throw std::invalid_argument("SO3LR: null box");
    ctx->ev->set_box(lo, hi);
  });
}

int so3lr_set_stream(so3lr_ctx *ctx, void *stream) {
  return guarded(ctx, [&] { ctx->ev->set_stream(static_cast<hipStream_t>(stream)); });
}

int so3lr_last_terms(so3lr_ctx *ctx, double *learned, double *zbl, double *lr, double *charges,
                     double *hirshfeld, double *totals, double *image_energy) {
  return guarded(ctx, [&] { ctx->ev->last_terms(learned, zbl, lr, charges, hirshfeld, totals, image_energy); });
}

int so3lr_last_vatom(so3lr_ctx *ctx, double *vatom, int on_device) {
  return guarded(ctx, [&] {
    if (!vatom) throw std::invalid_argument("SO3LR: per-atom virial requested without a buffer");
    ctx->ev->last_vatom(vatom, on_device != 0);
  });
}

int so3lr_graph_stats(const so3lr_ctx *ctx, int64_t *sr_active, int64_t *sr_cand, int64_t *lr_cand) {
  if (!ctx || !ctx->ev) return SO3LR_ERR_ARGUMENT;
  if (sr_active) *sr_active = ctx->ev->sr_active();
  if (sr_cand) *sr_cand = ctx->ev->sr_candidates();
  if (lr_cand) *lr_cand = ctx->ev->lr_candidates();
  return SO3LR_OK;
}

int so3lr_kernel_timing(so3lr_ctx *ctx, int enable) {
  return guarded(ctx, [&] { ctx->ev->set_timing(enable != 0); });
}

int so3lr_kernel_timing_read(so3lr_ctx *ctx, const char *kernel, double *total_ms, int64_t *launches,
                             int64_t *units) {
  return guarded(ctx, [&] {
    if (!kernel || !total_ms || !launches || !units) throw std::invalid_argument("SO3LR: null timing argument");
    double ms = 0;
    int64_t l = 0, u = 0;
    if (!ctx->ev->timing_read(kernel, ms, l, u)) throw std::invalid_argument(std::string("SO3LR: no timing for ") + kernel);
    *total_ms = ms;
    *launches = l;
    *units = u;
  });
}

int64_t so3lr_device_bytes(const so3lr_ctx *ctx) { return ctx && ctx->ev ? ctx->ev->device_bytes() : 0; }

}  // extern "C"
