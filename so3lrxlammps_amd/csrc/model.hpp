// .so3lr model reader, architecture descriptor and capability check (host).
//
// Format and rejection rules: source/so3lr-lammps-native/docs/FORMAT.md:12-82
// (the reader replaces NativeModel::load, src/native_model.cpp:325-406, and
// also enforces the canonical manifest encoding that the format demands).
// The architecture fields follow src/so3lr_architecture.cpp:296-451, and the
// capability refusal follows src/so3lr_capabilities.cpp:46-289, narrowed to
// what the gfx950 kernels of this library implement.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace so3lr_amd {

// --- manifest JSON value --------------------------------------------------
// The manifest is canonical JSON (docs/FORMAT.md: sorted keys, compact
// separators, ASCII with \u escapes), so members arrive in strictly
// increasing key order and are kept that way (lookups bisect).  A number
// keeps its source text: integers are read from the digits exactly, never
// through a double.
struct Json {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool b = false;
  double num = 0.0;
  std::string str;  // String: decoded UTF-8; Number: the literal as written
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;  // sorted by key, keys unique

  // Throws std::runtime_error unless `text` is canonical JSON.
  static Json parse_canonical(const std::string &text);
  const Json &at(const std::string &key) const;
  const Json *find(const std::string &key) const;
  double number() const;
  std::uint64_t uint() const;
  const std::string &string() const;
  bool boolean() const;
};

std::string sha256_hex(const std::uint8_t *data, std::size_t size);

struct Tensor {
  std::string state_key;
  std::string dtype;
  std::vector<std::size_t> shape;
  std::size_t offset = 0, nbytes = 0;
  std::size_t count() const;
};

// The v1 widths the fused kernels of evaluator.hip are written for; models of
// other widths run on the generic kernels (generic.hip).
constexpr int kF = 128;   // invariant features
constexpr int kHeads = 4; // attention heads == degree slots
constexpr int kHW = 32;   // head width
constexpr int kE = 24;    // equivariant channels, l = 1..4
constexpr int kR = 32;    // Bernstein basis size
constexpr int kNI = 132;  // interaction width F + 4
constexpr int kFH = 32;   // spherical filter hidden width F / 4
constexpr int kHH = 64;   // Hirshfeld head width
constexpr int kMaxBlocks = 8;

// Normalisation at the two positions of the post-attention block
// (src/so3lr_architecture.cpp:376-392): affine LayerNorm, RMSNorm without
// scale, or none (the second position only).
enum class NormMode : int { Layer = 0, Rms = 1, None = 2 };

struct Architecture {
  int layers = 0;
  double sr_cutoff = 0, lr_cutoff = 0, embedding_scale = 1;
  double attention_norm = 1;  // divisor of the attention logits (message_normalization)
  double ln_eps = 1e-6;
  double gamma = 0;
  // options; the defaults are the v1 model
  NormMode norm1 = NormMode::Layer, norm2 = NormMode::Layer;
  bool qk_norm = false;           // RMS-normalised q, k, q_ev, k_ev head rows
  bool residual_scalars = false;  // block input = resid[b] x + x0[b] x_embedding
  bool nlh = false;               // NLH pair-table repulsion instead of learned ZBL
  bool c6_head = false;           // C6 ratio head feeding the dispersion C6
  // widths (so3lr_architecture.cpp:197-212, 246-293, 444-446): F features in
  // F / 32 heads of 32, one equivariant head per degree slot, R radial
  // functions, the energy/charge head width; generic = not the v1 widths
  int F = kF, R = kR, heads = kHeads, E = kE, head_hidden = kF;
  std::vector<int> degrees{1, 2, 3, 4};
  bool generic = false;
  // repulsion (ZBL screening parameters: learned ZBL only)
  double zbl_ke = 0, zbl_switch_off = 0, zbl_p = 0, zbl_d = 0, zbl_a[4] = {}, zbl_c[4] = {};
  // long range
  double lr_ke = 0, lr_sigma = 0, lr_cuton_el = 0, lr_fine = 0, lr_bohr = 0, lr_hartree = 0,
         lr_disp_scale = 0, lr_cuton_disp = 0, lr_pair_scale = 0;
  std::string summary() const;
};

class Model {
 public:
  // Reads and validates a model file; throws std::runtime_error with a
  // message naming the failed rule (integrity) or the unsupported feature
  // (capability).
  static std::shared_ptr<Model> load(const std::string &path);
  static std::shared_ptr<Model> load_bytes(std::vector<std::uint8_t> bytes,
                                           const std::string &origin);

  const Json &manifest() const { return manifest_; }
  const Architecture &arch() const { return arch_; }
  bool has(const std::string &key) const { return tensors_.count(key) != 0; }
  const Tensor &tensor(const std::string &key) const;
  // float64 tensor values, shape-checked.
  std::vector<double> f64(const std::string &key, const std::vector<std::size_t> &shape) const;
  std::vector<std::int64_t> i64(const std::string &key, const std::vector<std::size_t> &shape) const;
  std::size_t tensor_count() const { return tensors_.size(); }

 private:
  std::vector<std::uint8_t> bytes_;
  std::size_t payload_begin_ = 0;
  Json manifest_;
  std::map<std::string, Tensor> tensors_;
  Architecture arch_;
  void describe_and_negotiate(const std::string &origin);
};

// Element token -> Z, as pair_coeff reads it: a symbol (any case) or an atomic
// number, 1..99; 0 means unknown (plugins/lammps/so3lr_element_map.h:15-49).
int atomic_number_from_token(const char *token);

// Charge/spin embedding (src/so3lr_charge_spin.cpp:52-141).
struct ChargeSpin {
  int F = kF;
  std::vector<double> wq[2], wk[2], wv[2], m1[2], m3[2];  // [0] charge, [1] spin
  void load(const Model &model);
  // 118 x F table (row Z-1) added to the element embedding before the scale.
  std::vector<double> table(const std::int64_t counts[119], double total_charge,
                            double unpaired) const;
};
// Empty when (Q, M) is consistent with the electron count of `counts`.
std::string charge_multiplicity_problem(const std::int64_t counts[119], double total_charge,
                                        double multiplicity);

}  // namespace so3lr_amd
