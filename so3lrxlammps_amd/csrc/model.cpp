// .so3lr reader, descriptor, capability table, element map, charge/spin table.
#include "model.hpp"

#include <algorithm>
#include <array>
#include <cerrno>
#include <cctype>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <set>
#include <sstream>
#include <stdexcept>

namespace so3lr_amd {
namespace {

[[noreturn]] void fail(const std::string &msg) {
  throw std::runtime_error("SO3LR native model: " + msg);
}

// ---------------------------------------------------------------- SHA-256
// FIPS 180-4, processed in 64-byte blocks.
struct Sha256 {
  std::uint32_t h[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                        0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
  static std::uint32_t rotr(std::uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
  void block(const std::uint8_t *p) {
    static const std::uint32_t k[64] = {
        0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4,
        0xab1c5ed5, 0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe,
        0x9bdc06a7, 0xc19bf174, 0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f,
        0x4a7484aa, 0x5cb0a9dc, 0x76f988da, 0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7,
        0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967, 0x27b70a85, 0x2e1b2138, 0x4d2c6dfc,
        0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85, 0xa2bfe8a1, 0xa81a664b,
        0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070, 0x19a4c116,
        0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
        0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7,
        0xc67178f2};
    std::uint32_t w[64];
    for (int i = 0; i < 16; ++i)
      w[i] = (std::uint32_t(p[4 * i]) << 24) | (std::uint32_t(p[4 * i + 1]) << 16) |
             (std::uint32_t(p[4 * i + 2]) << 8) | std::uint32_t(p[4 * i + 3]);
    for (int i = 16; i < 64; ++i) {
      const std::uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
      const std::uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
      w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    std::uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
    for (int i = 0; i < 64; ++i) {
      const std::uint32_t S1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25);
      const std::uint32_t ch = (e & f) ^ (~e & g);
      const std::uint32_t t1 = hh + S1 + ch + k[i] + w[i];
      const std::uint32_t S0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22);
      const std::uint32_t mj = (a & b) ^ (a & c) ^ (b & c);
      const std::uint32_t t2 = S0 + mj;
      hh = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
    }
    h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
  }
  std::array<std::uint8_t, 32> digest(const std::uint8_t *data, std::size_t n) {
    std::size_t full = n / 64;
    for (std::size_t i = 0; i < full; ++i) block(data + 64 * i);
    std::uint8_t tail[128] = {0};
    const std::size_t rem = n - 64 * full;
    std::memcpy(tail, data + 64 * full, rem);
    tail[rem] = 0x80;
    const std::size_t tail_len = rem + 9 <= 64 ? 64 : 128;
    const std::uint64_t bits = std::uint64_t(n) * 8;
    for (int i = 0; i < 8; ++i) tail[tail_len - 1 - i] = std::uint8_t(bits >> (8 * i));
    block(tail);
    if (tail_len == 128) block(tail + 64);
    std::array<std::uint8_t, 32> out{};
    for (int i = 0; i < 8; ++i)
      for (int j = 0; j < 4; ++j) out[4 * i + j] = std::uint8_t(h[i] >> (24 - 8 * j));
    return out;
  }
};

std::array<std::uint8_t, 32> sha256(const std::uint8_t *d, std::size_t n) {
  Sha256 s;
  return s.digest(d, n);
}

// ---------------------------------------------------------------- JSON
class Parser {
 public:
  explicit Parser(const std::string &t) : t_(t) {}
  Json document() {
    Json v = value();
    ws();
    if (p_ != t_.size()) fail("trailing JSON data");
    return v;
  }

 private:
  const std::string &t_;
  std::size_t p_ = 0;
  void ws() {
    while (p_ < t_.size() && (t_[p_] == ' ' || t_[p_] == '\n' || t_[p_] == '\r' || t_[p_] == '\t')) ++p_;
  }
  char next() {
    if (p_ >= t_.size()) fail("unexpected end of JSON");
    return t_[p_++];
  }
  static void utf8(std::string &o, std::uint32_t c) {
    if (c < 0x80) o += char(c);
    else if (c < 0x800) { o += char(0xc0 | (c >> 6)); o += char(0x80 | (c & 0x3f)); }
    else if (c < 0x10000) { o += char(0xe0 | (c >> 12)); o += char(0x80 | ((c >> 6) & 0x3f)); o += char(0x80 | (c & 0x3f)); }
    else { o += char(0xf0 | (c >> 18)); o += char(0x80 | ((c >> 12) & 0x3f)); o += char(0x80 | ((c >> 6) & 0x3f)); o += char(0x80 | (c & 0x3f)); }
  }
  std::uint32_t hex4() {
    std::uint32_t v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = next();
      v <<= 4;
      if (c >= '0' && c <= '9') v |= std::uint32_t(c - '0');
      else if (c >= 'a' && c <= 'f') v |= std::uint32_t(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= std::uint32_t(c - 'A' + 10);
      else fail("invalid JSON unicode escape");
    }
    return v;
  }
  std::string str() {
    ws();
    if (next() != '"') fail("expected JSON string");
    std::string o;
    for (;;) {
      const char c = next();
      if (c == '"') return o;
      if (static_cast<unsigned char>(c) < 0x20) fail("control byte in JSON string");
      if (c != '\\') { o += c; continue; }
      const char e = next();
      switch (e) {
        case '"': o += '"'; break;
        case '\\': o += '\\'; break;
        case '/': o += '/'; break;
        case 'b': o += '\b'; break;
        case 'f': o += '\f'; break;
        case 'n': o += '\n'; break;
        case 'r': o += '\r'; break;
        case 't': o += '\t'; break;
        case 'u': {
          std::uint32_t c1 = hex4();
          if (c1 >= 0xd800 && c1 <= 0xdbff) {
            if (next() != '\\' || next() != 'u') fail("invalid surrogate pair");
            const std::uint32_t c2 = hex4();
            if (c2 < 0xdc00 || c2 > 0xdfff) fail("invalid surrogate pair");
            c1 = 0x10000 + ((c1 - 0xd800) << 10) + (c2 - 0xdc00);
          }
          utf8(o, c1);
          break;
        }
        default: fail("invalid JSON escape");
      }
    }
  }
  Json num() {
    const std::size_t b = p_;
    auto digit = [&](std::size_t i) { return i < t_.size() && t_[i] >= '0' && t_[i] <= '9'; };
    if (p_ < t_.size() && t_[p_] == '-') ++p_;
    if (!digit(p_)) fail("invalid JSON number");
    if (t_[p_] == '0') ++p_;
    else while (digit(p_)) ++p_;
    if (p_ < t_.size() && t_[p_] == '.') {
      ++p_;
      if (!digit(p_)) fail("invalid JSON fraction");
      while (digit(p_)) ++p_;
    }
    if (p_ < t_.size() && (t_[p_] == 'e' || t_[p_] == 'E')) {
      ++p_;
      if (p_ < t_.size() && (t_[p_] == '+' || t_[p_] == '-')) ++p_;
      if (!digit(p_)) fail("invalid JSON exponent");
      while (digit(p_)) ++p_;
    }
    const std::string tok = t_.substr(b, p_ - b);
    char *end = nullptr;
    const double v = std::strtod(tok.c_str(), &end);
    if (end != tok.c_str() + tok.size() || !std::isfinite(v)) fail("invalid JSON number");
    Json j;
    j.kind = Json::Number;
    j.num = v;
    return j;
  }
  void word(const char *w) {
    const std::size_t n = std::strlen(w);
    if (t_.compare(p_, n, w) != 0) fail("invalid JSON literal");
    p_ += n;
  }
  Json value() {
    ws();
    if (p_ >= t_.size()) fail("unexpected end of JSON");
    const char c = t_[p_];
    Json j;
    if (c == '"') { j.kind = Json::String; j.str = str(); return j; }
    if (c == 't') { word("true"); j.kind = Json::Bool; j.b = true; return j; }
    if (c == 'f') { word("false"); j.kind = Json::Bool; j.b = false; return j; }
    if (c == 'n') { word("null"); return j; }
    if (c == '[') {
      ++p_;
      j.kind = Json::Array;
      ws();
      if (p_ < t_.size() && t_[p_] == ']') { ++p_; return j; }
      for (;;) {
        j.arr.push_back(value());
        ws();
        const char d = next();
        if (d == ']') return j;
        if (d != ',') fail("expected comma in JSON array");
      }
    }
    if (c == '{') {
      ++p_;
      j.kind = Json::Object;
      ws();
      if (p_ < t_.size() && t_[p_] == '}') { ++p_; return j; }
      for (;;) {
        std::string key = str();
        ws();
        if (next() != ':') fail("expected colon in JSON object");
        if (!j.obj.emplace(key, value()).second) fail("duplicate JSON object key");
        ws();
        const char d = next();
        if (d == '}') return j;
        if (d != ',') fail("expected comma in JSON object");
      }
    }
    return num();
  }
};

std::uint64_t le64(const std::uint8_t *p) {
  std::uint64_t v = 0;
  for (int i = 7; i >= 0; --i) v = (v << 8) | p[i];
  return v;
}
std::uint32_t le32(const std::uint8_t *p) {
  return std::uint32_t(p[0]) | (std::uint32_t(p[1]) << 8) | (std::uint32_t(p[2]) << 16) |
         (std::uint32_t(p[3]) << 24);
}

std::size_t dtype_size(const std::string &d) {
  if (d == "float64" || d == "int64") return 8;
  if (d == "float32" || d == "int32") return 4;
  if (d == "uint8" || d == "bool") return 1;
  fail("unsupported dtype " + d);
}

}  // namespace

// ------------------------------------------------------------------ Json API
Json Json::parse(const std::string &text) { return Parser(text).document(); }
const Json *Json::find(const std::string &key) const {
  if (kind != Object) return nullptr;
  const auto it = obj.find(key);
  return it == obj.end() ? nullptr : &it->second;
}
const Json &Json::at(const std::string &key) const {
  const Json *j = find(key);
  if (!j) fail("missing JSON key " + key);
  return *j;
}
double Json::number() const {
  if (kind != Number) fail("JSON value is not a number");
  return num;
}
std::uint64_t Json::uint() const {
  const double v = number();
  if (v < 0 || std::floor(v) != v || v > 9007199254740991.0) fail("JSON value is not an exact unsigned integer");
  return std::uint64_t(v);
}
const std::string &Json::string() const {
  if (kind != String) fail("JSON value is not a string");
  return str;
}
bool Json::boolean() const {
  if (kind != Bool) fail("JSON value is not a boolean");
  return b;
}

std::string sha256_hex(const std::uint8_t *data, std::size_t size) {
  const auto d = sha256(data, size);
  static const char *hx = "0123456789abcdef";
  std::string s;
  for (auto c : d) { s += hx[c >> 4]; s += hx[c & 15]; }
  return s;
}

std::size_t Tensor::count() const {
  std::size_t n = 1;
  for (auto e : shape) n *= e;
  return n;
}

std::string Architecture::summary() const {
  std::ostringstream o;
  o << "layers=" << layers << " features=" << kF << " heads=" << kHeads << "x" << kHW
    << " degrees=[1,2,3,4] rbf=" << kR << " r_cut=" << sr_cutoff << " r_cut_lr=" << lr_cutoff;
  return o.str();
}

// --------------------------------------------------------------- loading
std::shared_ptr<Model> Model::load(const std::string &path) {
  std::ifstream in(path, std::ios::binary);
  if (!in) fail("cannot open " + path);
  std::vector<std::uint8_t> bytes((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
  return load_bytes(std::move(bytes), path);
}

std::shared_ptr<Model> Model::load_bytes(std::vector<std::uint8_t> bytes, const std::string &origin) {
  constexpr std::size_t header = 128;
  static const std::uint8_t magic[8] = {'S', 'O', '3', 'L', 'R', 'N', '1', 0};
  if (bytes.size() < header) fail("file is shorter than the fixed header");
  if (std::memcmp(bytes.data(), magic, 8) != 0) fail("wrong magic");
  if (le32(bytes.data() + 8) != 1 || le32(bytes.data() + 12) != 0) fail("unsupported version or flags");
  const std::uint64_t msize = le64(bytes.data() + 16), psize = le64(bytes.data() + 24);
  if (msize > bytes.size() - header || psize != bytes.size() - header - msize) fail("header length mismatch");
  for (std::size_t i = 96; i < 128; ++i)
    if (bytes[i] != 0) fail("nonzero reserved header bytes");
  const std::uint8_t *mdata = bytes.data() + header, *pdata = mdata + msize;
  const auto md = sha256(mdata, msize), pd = sha256(pdata, psize);
  if (std::memcmp(md.data(), bytes.data() + 32, 32) != 0) fail("manifest SHA-256 mismatch");
  if (std::memcmp(pd.data(), bytes.data() + 64, 32) != 0) fail("payload SHA-256 mismatch");

  auto m = std::make_shared<Model>();
  m->payload_begin_ = header + msize;
  m->manifest_ = Json::parse(std::string(reinterpret_cast<const char *>(mdata), msize));
  const Json &mf = m->manifest_;
  if (mf.at("format").string() != "so3lr-native" || mf.at("format_version").uint() != 1)
    fail("manifest format mismatch");
  if (mf.at("endianness").string() != "little" || mf.at("tensor_alignment").uint() != 64)
    fail("manifest endianness/alignment mismatch");
  if (mf.at("model_family").string() != "SO3LR") fail("wrong model family");

  std::set<std::string> names;
  std::size_t prev_end = 0, total = 0;
  for (const Json &rec : mf.at("tensors").arr) {
    Tensor t;
    const std::string name = rec.at("name").string();
    t.state_key = rec.at("state_key").string();
    t.dtype = rec.at("dtype").string();
    t.offset = rec.at("offset").uint();
    t.nbytes = rec.at("nbytes").uint();
    std::size_t elems = 1;
    for (const Json &e : rec.at("shape").arr) {
      const std::size_t x = e.uint();
      if (x != 0 && elems > (std::size_t(-1) / x)) fail("tensor shape overflow");
      elems *= x;
      t.shape.push_back(x);
    }
    if (!names.insert(name).second || m->tensors_.count(t.state_key)) fail("duplicate tensor name/state key");
    if (t.offset % 64 != 0 || t.nbytes != elems * dtype_size(t.dtype)) fail("tensor alignment/size mismatch");
    if (t.offset < prev_end || t.offset > psize || t.nbytes > psize - t.offset) fail("tensor overlap/range error");
    for (std::size_t q = prev_end; q < t.offset; ++q)
      if (pdata[q] != 0) fail("nonzero payload padding");
    if (sha256_hex(pdata + t.offset, t.nbytes) != rec.at("sha256").string()) fail("per-tensor SHA-256 mismatch");
    prev_end = t.offset + t.nbytes;
    total += t.nbytes;
    m->tensors_.emplace(t.state_key, t);
  }
  if (prev_end != psize) fail("unreferenced trailing payload bytes");
  if (mf.at("tensor_count").uint() != m->tensors_.size() || mf.at("tensor_bytes").uint() != total)
    fail("tensor totals mismatch");
  m->bytes_ = std::move(bytes);
  m->describe_and_negotiate(origin);
  return m;
}

const Tensor &Model::tensor(const std::string &key) const {
  const auto it = tensors_.find(key);
  if (it == tensors_.end()) fail("missing tensor " + key);
  return it->second;
}

std::vector<double> Model::f64(const std::string &key, const std::vector<std::size_t> &shape) const {
  const Tensor &t = tensor(key);
  if (t.dtype != "float64" || t.shape != shape) fail("tensor contract mismatch: " + key);
  std::vector<double> v(t.count());
  std::memcpy(v.data(), bytes_.data() + payload_begin_ + t.offset, t.nbytes);
  return v;
}

std::vector<std::int64_t> Model::i64(const std::string &key, const std::vector<std::size_t> &shape) const {
  const Tensor &t = tensor(key);
  if (t.dtype != "int64" || t.shape != shape) fail("tensor contract mismatch: " + key);
  std::vector<std::int64_t> v(t.count());
  std::memcpy(v.data(), bytes_.data() + payload_begin_ + t.offset, t.nbytes);
  return v;
}

// ------------------------------------------------ descriptor + capabilities
void Model::describe_and_negotiate(const std::string &origin) {
  const Json &a = manifest_.at("architecture");
  std::vector<std::string> misses;
  auto need = [&](bool ok, const std::string &what) {
    if (!ok) misses.push_back(what);
  };
  // Keys this build can interpret or may ignore (so3lr_capabilities.cpp:95-151).
  static const std::set<std::string> known = {
      "atomic_number_capacity", "attention_head_width", "attention_heads", "avg_num_neighbors",
      "embedding_scale", "energy_theory_level_selected", "euclidean_degree_channels",
      "interaction_blocks", "invariant_features", "layer_norm_epsilon",
      "long_range_cutoff_angstrom", "lr_bohr_angstrom", "lr_dispersion_cuton_angstrom",
      "lr_dispersion_scale", "lr_electrostatic_cuton_angstrom", "lr_electrostatic_ke",
      "lr_electrostatic_sigma", "lr_fine_structure", "lr_hartree_ev", "lr_pair_scale",
      "layer_normalization_1", "layer_normalization_2", "message_normalization",
      "module_type_registry", "native_long_range_observables", "native_long_range_terms",
      "native_short_range_physical_terms", "num_embeddings", "output_heads",
      "parameter_elements", "physical_reference_table_state_keys",
      "physical_reference_table_tensor_count", "qk_norm", "qk_nonlinearity",
      "radial_basis_features", "repulsion_type", "residual_mlp_1", "residual_mlp_2",
      "runtime_element_mapping", "short_range_cutoff_angstrom", "state_tensor_count",
      "use_residual_scalars", "use_rms_norm", "zbl_a1", "zbl_a2", "zbl_a3", "zbl_a4",
      "zbl_c1", "zbl_c2", "zbl_c3", "zbl_c4", "zbl_cutoff_function", "zbl_d", "zbl_enabled",
      "zbl_ke", "zbl_p", "zbl_switch_off_angstrom"};
  for (const auto &kv : a.obj) need(known.count(kv.first) != 0, "unknown architecture key '" + kv.first + "'");
  need(manifest_.at("schema").string() == "so3lr-native-model-v2", "schema other than so3lr-native-model-v2");
  auto num = [&](const char *k) { return a.at(k).number(); };
  auto flag = [&](const char *k, bool dflt) {
    const Json *j = a.find(k);
    return j ? j->boolean() : dflt;
  };
  arch_.layers = int(a.at("interaction_blocks").uint());
  need(arch_.layers >= 1 && arch_.layers <= kMaxBlocks, "interaction_blocks outside 1..8");
  need(a.at("invariant_features").uint() == std::uint64_t(kF), "invariant_features != 128 (gfx950 kernels are built for F=128)");
  need(a.at("attention_heads").uint() == 4 && a.at("attention_head_width").uint() == 32, "attention heads other than 4 x 32");
  need(a.at("euclidean_degree_channels").uint() == 4, "euclidean_degree_channels != 4");
  need(a.at("radial_basis_features").uint() == std::uint64_t(kR), "radial_basis_features != 32");
  need(!flag("use_rms_norm", false), "RMSNorm (use_rms_norm)");
  need(!flag("qk_norm", false), "QK normalisation (qk_norm)");
  need(!flag("use_residual_scalars", false), "residual scalars (use_residual_scalars)");
  need(flag("layer_normalization_1", true) && flag("layer_normalization_2", true), "disabled LayerNorm positions");
  need(flag("residual_mlp_1", true) && !flag("residual_mlp_2", false), "residual MLP layout other than mlp_1 only");
  if (const Json *q = a.find("qk_nonlinearity")) need(q->string() == "identity", "QK nonlinearity other than identity");
  if (const Json *r = a.find("repulsion_type")) need(r->string() == "zbl_learned", "repulsion other than learned ZBL");
  else need(a.find("zbl_enabled") && a.at("zbl_enabled").number() == 1.0, "missing ZBL repulsion");
  if (const Json *zc = a.find("zbl_cutoff_function")) need(zc->string() == "phys", "ZBL cutoff function other than phys");
  if (const Json *mn = a.find("message_normalization")) need(mn->string() == "avg_num_neighbors", "message normalisation other than avg_num_neighbors");
  const Json &heads = a.at("output_heads");
  need(heads.arr.size() == 3 && heads.arr[0].string() == "atomic_energy_output_block" &&
           heads.arr[1].string() == "partial_charges_output_block" &&
           heads.arr[2].string() == "hirshfeld_output_block",
       "output heads other than energy, partial charges and Hirshfeld ratios");
  if (misses.empty()) {
    // degree layout {3,5,7,9} in every block
    for (int b = 0; b < arch_.layers; ++b) {
      const std::string p = "model.euclidean_transformers." + std::to_string(b);
      const auto rep = i64(p + ".euclidean_attention_block.degree_repeats", {4});
      need(rep == std::vector<std::int64_t>({3, 5, 7, 9}), "degree layout other than l = 1,2,3,4");
    }
    const double eps = a.find("layer_norm_epsilon") ? num("layer_norm_epsilon") : 1e-6;
    need(std::abs(eps - 1e-6) < 1e-15, "LayerNorm epsilon other than 1e-6");
    arch_.ln_eps = eps;
  }
  if (!misses.empty()) {
    std::string msg = "model '" + origin + "' needs features this gfx950 build does not implement:";
    for (const auto &s : misses) msg += "\n  - " + s;
    throw std::runtime_error(msg);
  }
  arch_.sr_cutoff = num("short_range_cutoff_angstrom");
  arch_.lr_cutoff = num("long_range_cutoff_angstrom");
  arch_.embedding_scale = num("embedding_scale");
  arch_.attention_norm = num("avg_num_neighbors");
  if (!(arch_.sr_cutoff > 0) || !(arch_.lr_cutoff >= arch_.sr_cutoff)) fail("invalid native model cutoffs");
  if (!(arch_.embedding_scale > 0) || !std::isfinite(arch_.embedding_scale)) fail("embedding scale must be positive");
  arch_.gamma = f64("model.radial_embedding.radial_basis_fn.gamma", {})[0];
  arch_.zbl_ke = num("zbl_ke");
  arch_.zbl_switch_off = num("zbl_switch_off_angstrom");
  arch_.zbl_p = num("zbl_p");
  arch_.zbl_d = num("zbl_d");
  double csum = 0;
  for (int k = 0; k < 4; ++k) {
    arch_.zbl_a[k] = num(("zbl_a" + std::to_string(k + 1)).c_str());
    arch_.zbl_c[k] = num(("zbl_c" + std::to_string(k + 1)).c_str());
    if (!(arch_.zbl_a[k] > 0) || !(arch_.zbl_c[k] > 0)) fail("invalid ZBL parameter");
    csum += arch_.zbl_c[k];
  }
  if (std::abs(csum - 1.0) > 2e-12) fail("normalized ZBL coefficients changed");
  arch_.lr_ke = num("lr_electrostatic_ke");
  arch_.lr_sigma = num("lr_electrostatic_sigma");
  arch_.lr_cuton_el = num("lr_electrostatic_cuton_angstrom");
  arch_.lr_fine = num("lr_fine_structure");
  arch_.lr_bohr = num("lr_bohr_angstrom");
  arch_.lr_hartree = num("lr_hartree_ev");
  arch_.lr_disp_scale = num("lr_dispersion_scale");
  arch_.lr_cuton_disp = num("lr_dispersion_cuton_angstrom");
  arch_.lr_pair_scale = num("lr_pair_scale");
  if (!(arch_.lr_cutoff > arch_.lr_cuton_el) || !(arch_.lr_cutoff > arch_.lr_cuton_disp) ||
      std::abs(arch_.lr_pair_scale - 0.5) > 1e-12)
    fail("LR cutoff/half-pair contract changed");
}

// ------------------------------------------------------------ element map
int atomic_number_from_token(const char *token) {
  if (token == nullptr || token[0] == '\0') return 0;
  char *end = nullptr;
  errno = 0;
  const long v = std::strtol(token, &end, 10);
  if (errno == 0 && end != token && *end == '\0') return (v >= 1 && v <= 99) ? int(v) : 0;
  static const char *sym[100] = {
      "", "H", "He", "Li", "Be", "B", "C", "N", "O", "F", "Ne", "Na", "Mg", "Al", "Si", "P", "S",
      "Cl", "Ar", "K", "Ca", "Sc", "Ti", "V", "Cr", "Mn", "Fe", "Co", "Ni", "Cu", "Zn", "Ga", "Ge",
      "As", "Se", "Br", "Kr", "Rb", "Sr", "Y", "Zr", "Nb", "Mo", "Tc", "Ru", "Rh", "Pd", "Ag",
      "Cd", "In", "Sn", "Sb", "Te", "I", "Xe", "Cs", "Ba", "La", "Ce", "Pr", "Nd", "Pm", "Sm",
      "Eu", "Gd", "Tb", "Dy", "Ho", "Er", "Tm", "Yb", "Lu", "Hf", "Ta", "W", "Re", "Os", "Ir",
      "Pt", "Au", "Hg", "Tl", "Pb", "Bi", "Po", "At", "Rn", "Fr", "Ra", "Ac", "Th", "Pa", "U",
      "Np", "Pu", "Am", "Cm", "Bk", "Cf", "Es"};
  std::string s(token);
  for (std::size_t i = 0; i < s.size(); ++i)
    s[i] = char(i == 0 ? std::toupper(static_cast<unsigned char>(s[i])) : std::tolower(static_cast<unsigned char>(s[i])));
  for (int zz = 1; zz <= 99; ++zz)
    if (s == sym[zz]) return zz;
  return 0;
}

// ------------------------------------------------------------ charge/spin
void ChargeSpin::load(const Model &model) {
  static const char *names[2] = {"model.charge_embedding.", "model.spin_embedding."};
  for (int k = 0; k < 2; ++k) {
    const std::string b = names[k];
    wq[k] = model.f64(b + "Wq.weight", {std::size_t(kF), 118});
    wk[k] = model.f64(b + "Wk", {2, std::size_t(kF)});
    wv[k] = model.f64(b + "Wv", {2, std::size_t(kF)});
    m1[k] = model.f64(b + "mlp.1.weight", {std::size_t(kF), std::size_t(kF)});
    m3[k] = model.f64(b + "mlp.3.weight", {std::size_t(kF), std::size_t(kF)});
  }
}

std::vector<double> ChargeSpin::table(const std::int64_t counts[119], double total_charge,
                                      double unpaired) const {
  std::vector<double> out(118 * kF, 0.0);
  auto silu = [](double x) { return x / (1.0 + std::exp(-x)); };
  const double psis[2] = {total_charge, unpaired};
  for (int k = 0; k < 2; ++k) {
    const double psi = psis[k];
    if (psi == 0.0) continue;  // the module's output is exactly zero
    const int row = psi < 0.0 ? 1 : 0;
    const double *key = wk[k].data() + row * kF, *val = wv[k].data() + row * kF;
    double y[119] = {0};
    double den = 0.0;
    for (int zz = 1; zz <= 118; ++zz) {
      if (counts[zz] <= 0) continue;
      double qk = 0.0;
      for (int c = 0; c < kF; ++c) qk += wq[k][c * 118 + (zz - 1)] * key[c];
      const double x = qk / std::sqrt(double(kF));
      y[zz] = std::max(x, 0.0) + std::log1p(std::exp(-std::abs(x)));  // softplus
      den += double(counts[zz]) * y[zz];
    }
    std::vector<double> x(kF), sx(kF), h(kF), sh(kF);
    for (int zz = 1; zz <= 118; ++zz) {
      if (counts[zz] <= 0) continue;
      const double w = psi * y[zz] / den;
      for (int c = 0; c < kF; ++c) { x[c] = w * val[c]; sx[c] = silu(x[c]); }
      for (int o = 0; o < kF; ++o) {
        double s = 0.0;
        for (int i = 0; i < kF; ++i) s += m1[k][o * kF + i] * sx[i];
        h[o] = s;
        sh[o] = silu(s);
      }
      for (int o = 0; o < kF; ++o) {
        double s = 0.0;
        for (int i = 0; i < kF; ++i) s += m3[k][o * kF + i] * sh[i];
        out[(zz - 1) * kF + o] += x[o] + s;
      }
    }
  }
  return out;
}

std::string charge_multiplicity_problem(const std::int64_t counts[119], double q, double mult) {
  if (!std::isfinite(q) || std::round(q) != q) return "the total charge must be an integer";
  if (!std::isfinite(mult) || std::round(mult) != mult || mult < 1.0)
    return "the spin multiplicity must be an integer >= 1";
  std::int64_t protons = 0;
  for (int zz = 1; zz <= 118; ++zz) protons += counts[zz] * zz;
  const std::int64_t electrons = protons - std::int64_t(q);
  const std::int64_t unpaired = std::int64_t(mult) - 1;
  if (electrons < 0) return "the total charge leaves a negative number of electrons";
  if (unpaired > electrons)
    return "multiplicity " + std::to_string(std::int64_t(mult)) +
           " needs more unpaired electrons than the system's " + std::to_string(electrons) + " electrons";
  if ((electrons - unpaired) % 2 != 0)
    return std::to_string(electrons) + " electrons cannot have multiplicity " +
           std::to_string(std::int64_t(mult)) +
           " (an even electron count needs an odd multiplicity and vice versa)";
  return std::string();
}

}  // namespace so3lr_amd
