// .so3lr reader, descriptor, capability table, element map, charge/spin table.
#include "model.hpp"

#include <algorithm>
#include <array>
#include <charconv>
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

// ------------------------------------------------------- canonical JSON
// Python's repr of a finite double, the spelling the exporter's canonical
// encoder writes (json.dumps uses float.__repr__): the shortest digits that
// round-trip, positional notation when the decimal point position decpt
// (value = 0.DIGITS x 10^decpt) satisfies -4 < decpt <= 16, otherwise
// d[.ddd]e(+|-)XX with at least two exponent digits; positional values
// always carry a fractional part ("4.0").
std::string python_float_repr(double v) {
  char sci[64];
  const auto res = std::to_chars(sci, sci + sizeof sci, v, std::chars_format::scientific);
  const std::string s(sci, res.ptr);  // [-]d[.ddd]e(+|-)XX
  const std::size_t epos = s.find('e');
  const bool neg = s[0] == '-';
  std::string digits;
  for (std::size_t i = neg ? 1 : 0; i < epos; ++i)
    if (s[i] != '.') digits += s[i];
  const int exp10 = std::atoi(s.c_str() + epos + 1);
  const int decpt = exp10 + 1;
  std::string out = neg ? "-" : "";
  if (decpt > -4 && decpt <= 16) {
    if (decpt <= 0) {
      out += "0." + std::string(std::size_t(-decpt), '0') + digits;
    } else if (std::size_t(decpt) >= digits.size()) {
      out += digits + std::string(std::size_t(decpt) - digits.size(), '0') + ".0";
    } else {
      out += digits.substr(0, std::size_t(decpt)) + "." + digits.substr(std::size_t(decpt));
    }
  } else {
    out += digits.substr(0, 1);
    if (digits.size() > 1) out += "." + digits.substr(1);
    const int a = exp10 < 0 ? -exp10 : exp10;
    out += exp10 < 0 ? "e-" : "e+";
    if (a < 10) out += '0';
    out += std::to_string(a);
  }
  return out;
}

// Reads the whole manifest with an explicit stack of open containers (no
// recursion, so nesting depth costs heap, not call stack).  Canonical form
// means, byte for byte, what json.dumps(sort_keys=True, separators=(",",":"),
// ensure_ascii=True) writes (docs/FORMAT.md:12-38 and the exporter's check
// that re-encoding reproduces the bytes):
//   * printable ASCII only, no whitespace between tokens;
//   * object keys strictly increasing (sorted and unique);
//   * in strings, a raw byte 0x20..0x7e other than '"' and '\', the short
//     escapes \" \\ \b \f \n \r \t, or \u with four lowercase hex digits for
//     every other code point (astral ones as a surrogate pair);
//   * integers without leading zeros, floats spelled as Python's repr;
//   * true, false, null.
class CanonicalReader {
 public:
  explicit CanonicalReader(const std::string &text) : t_(text) {}

  Json run() {
    for (std::size_t i = 0; i < t_.size(); ++i) {
      const unsigned char c = static_cast<unsigned char>(t_[i]);
      if (c < 0x20 || c > 0x7e) reject(i, "a byte outside printable ASCII");
    }
    Json done;
    bool have_done = false;
    for (;;) {
      if (!have_done) {
        // a value starts here
        if (at_end()) reject(pos_, "input ends where a value is expected");
        const char c = t_[pos_];
        if (c == '{' || c == '[') {
          Open o;
          o.node.kind = c == '{' ? Json::Object : Json::Array;
          ++pos_;
          const char close = c == '{' ? '}' : ']';
          if (!at_end() && t_[pos_] == close) {
            ++pos_;
            done = std::move(o.node);
            have_done = true;
            continue;
          }
          stack_.push_back(std::move(o));
          if (c == '{') read_key();
          continue;
        }
        done = scalar();
        have_done = true;
        continue;
      }
      // a value is complete: attach it to the innermost open container
      if (stack_.empty()) {
        if (!at_end()) reject(pos_, "text after the top-level value");
        return done;
      }
      Open &top = stack_.back();
      if (top.node.kind == Json::Array) top.node.arr.push_back(std::move(done));
      else top.node.obj.emplace_back(std::move(top.key), std::move(done));
      have_done = false;
      if (at_end()) reject(pos_, "input ends inside a container");
      const char sep = t_[pos_++];
      if (sep == ',') {
        if (top.node.kind == Json::Object) read_key();
        continue;
      }
      if (sep != (top.node.kind == Json::Object ? '}' : ']')) reject(pos_ - 1, "expected ',' or the closing bracket");
      done = std::move(top.node);
      stack_.pop_back();
      have_done = true;
    }
  }

 private:
  struct Open {
    Json node;
    std::string key;  // member being read (objects)
  };
  const std::string &t_;
  std::size_t pos_ = 0;
  std::vector<Open> stack_;

  [[noreturn]] void reject(std::size_t at, const char *why) const {
    fail("manifest is not canonical JSON at byte " + std::to_string(at) + ": " + why);
  }
  bool at_end() const { return pos_ >= t_.size(); }

  // "key": of the next member; keys must increase strictly
  void read_key() {
    Open &top = stack_.back();
    if (at_end() || t_[pos_] != '"') reject(pos_, "expected a member name");
    const std::size_t where = pos_;
    std::string key = string_token();
    if (!top.node.obj.empty() && !(top.node.obj.back().first < key))
      reject(where, "member names not in strictly increasing order");
    if (at_end() || t_[pos_] != ':') reject(pos_, "expected ':' after a member name");
    ++pos_;
    top.key = std::move(key);
  }

  Json scalar() {
    Json j;
    const char c = t_[pos_];
    if (c == '"') {
      j.kind = Json::String;
      j.str = string_token();
      return j;
    }
    for (const char *lit : {"true", "false", "null"}) {
      const std::size_t n = std::strlen(lit);
      if (t_.compare(pos_, n, lit) == 0) {
        pos_ += n;
        if (lit[0] != 'n') {
          j.kind = Json::Bool;
          j.b = lit[0] == 't';
        }
        return j;
      }
    }
    return number_token();
  }

  int hex_digit(std::size_t i) const {
    const char c = i < t_.size() ? t_[i] : '\0';
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    reject(i, "\\u needs four lowercase hexadecimal digits");
  }
  std::uint32_t u_escape() {  // pos_ at the 'u'
    std::uint32_t v = 0;
    for (int k = 1; k <= 4; ++k) v = (v << 4) | std::uint32_t(hex_digit(pos_ + k));
    pos_ += 5;
    return v;
  }
  static void put_utf8(std::string &o, std::uint32_t cp) {
    int n = cp < 0x80 ? 1 : cp < 0x800 ? 2 : cp < 0x10000 ? 3 : 4;
    static const unsigned char lead[5] = {0, 0x00, 0xc0, 0xe0, 0xf0};
    char buf[4];
    for (int k = n - 1; k > 0; --k) {
      buf[k] = char(0x80 | (cp & 0x3f));
      cp >>= 6;
    }
    buf[0] = char(lead[n] | cp);
    o.append(buf, std::size_t(n));
  }

  std::string string_token() {  // pos_ at the opening quote
    std::string out;
    ++pos_;
    for (;;) {
      if (at_end()) reject(pos_, "unterminated string");
      const char c = t_[pos_];
      if (c == '"') {
        ++pos_;
        return out;
      }
      if (c != '\\') {
        out += c;
        ++pos_;
        continue;
      }
      ++pos_;
      if (at_end()) reject(pos_, "unterminated escape");
      const char e = t_[pos_];
      static const char shorts[] = "\"\\bfnrt", decoded[] = "\"\\\b\f\n\r\t";
      if (const char *s = std::strchr(shorts, e); s && e != '\0') {
        out += decoded[s - shorts];
        ++pos_;
        continue;
      }
      if (e != 'u') reject(pos_, "an escape the canonical encoder never writes");
      const std::size_t where = pos_;
      std::uint32_t cp = u_escape();
      if (cp >= 0xdc00 && cp <= 0xdfff) reject(where, "a lone low surrogate");
      if (cp >= 0xd800 && cp <= 0xdbff) {
        if (t_.compare(pos_, 2, "\\u") != 0) reject(pos_, "a high surrogate without its low half");
        ++pos_;
        const std::uint32_t lo = u_escape();
        if (lo < 0xdc00 || lo > 0xdfff) reject(pos_, "a high surrogate without its low half");
        cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
      }
      const bool has_short = cp == '"' || cp == '\\' || cp == '\b' || cp == '\f' || cp == '\n' || cp == '\r' ||
                             cp == '\t';
      if ((cp >= 0x20 && cp <= 0x7e) || has_short) reject(where, "\\u escape of a character written literally or in short form");
      put_utf8(out, cp);
    }
  }

  Json number_token() {
    const std::size_t b = pos_;
    auto digits = [&]() {
      const std::size_t s = pos_;
      while (!at_end() && t_[pos_] >= '0' && t_[pos_] <= '9') ++pos_;
      return pos_ - s;
    };
    if (!at_end() && t_[pos_] == '-') ++pos_;
    const std::size_t int_begin = pos_;
    if (digits() == 0) reject(b, "not a value");
    const bool lead_zero = t_[int_begin] == '0' && pos_ - int_begin > 1;
    bool is_float = false;
    if (!at_end() && t_[pos_] == '.') {
      ++pos_;
      if (digits() == 0) reject(pos_, "a decimal point without digits after it");
      is_float = true;
    }
    if (!at_end() && (t_[pos_] == 'e' || t_[pos_] == 'E')) {
      ++pos_;
      if (!at_end() && (t_[pos_] == '+' || t_[pos_] == '-')) ++pos_;
      if (digits() == 0) reject(pos_, "an exponent without digits");
      is_float = true;
    }
    Json j;
    j.kind = Json::Number;
    j.str = t_.substr(b, pos_ - b);
    j.num = std::strtod(j.str.c_str(), nullptr);
    if (!std::isfinite(j.num)) reject(b, "a number outside the double range");
    if (is_float) {
      if (python_float_repr(j.num) != j.str) reject(b, "a float not spelled as its shortest repr");
    } else if (lead_zero || j.str == "-0") {
      reject(b, "an integer with a leading zero or a negative zero");
    }
    return j;
  }
};

std::uint32_t get_u32(const std::uint8_t *p) {
  std::uint32_t v = 0;
  for (int k = 3; k >= 0; --k) v = (v << 8) | p[k];
  return v;
}
std::uint64_t get_u64(const std::uint8_t *p) { return std::uint64_t(get_u32(p)) | (std::uint64_t(get_u32(p + 4)) << 32); }

// Bytes per element of the dtypes of format version 1 (docs/FORMAT.md:50-62);
// 0 for anything else.
std::size_t element_size(const std::string &dtype) {
  static const std::pair<const char *, std::size_t> table[] = {
      {"float64", 8}, {"int64", 8}, {"float32", 4}, {"int32", 4}, {"uint8", 1}, {"bool", 1}};
  for (const auto &e : table)
    if (dtype == e.first) return e.second;
  return 0;
}

}  // namespace

// ------------------------------------------------------------------ Json API
Json Json::parse_canonical(const std::string &text) { return CanonicalReader(text).run(); }
const Json *Json::find(const std::string &key) const {
  if (kind != Object) return nullptr;
  const auto it = std::lower_bound(obj.begin(), obj.end(), key,
                                   [](const std::pair<std::string, Json> &m, const std::string &k) { return m.first < k; });
  return it != obj.end() && it->first == key ? &it->second : nullptr;
}
const Json &Json::at(const std::string &key) const {
  const Json *j = find(key);
  if (!j) fail("manifest lacks the member '" + key + "'");
  return *j;
}
double Json::number() const {
  if (kind != Number) fail("manifest value '" + str + "' should be a number");
  return num;
}
std::uint64_t Json::uint() const {
  // from the literal's digits: a float literal ("3.0", "1e3") is not a count
  if (kind != Number || str.empty() || str.size() > 19 || str.find_first_not_of("0123456789") != std::string::npos)
    fail("manifest value '" + str + "' should be a non-negative integer below 10^19");
  std::uint64_t v = 0;
  for (const char c : str) v = v * 10 + std::uint64_t(c - '0');
  return v;
}
const std::string &Json::string() const {
  if (kind != String) fail("manifest value should be a string");
  return str;
}
bool Json::boolean() const {
  if (kind != Bool) fail("manifest value should be true or false");
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
  o << "layers=" << layers << " features=" << F << " heads=" << heads << "x" << kHW << " degrees=[";
  for (std::size_t s = 0; s < degrees.size(); ++s) o << (s ? "," : "") << degrees[s];
  o << "] rbf=" << R << " head_width=" << head_hidden << " r_cut=" << sr_cutoff << " r_cut_lr=" << lr_cutoff;
  static const char *norms[3] = {"layer", "rms", "none"};
  o << " norm=" << norms[int(norm1)] << "/" << norms[int(norm2)] << " attention_norm=" << attention_norm
    << " repulsion=" << (nlh ? "nlh" : "zbl") << (qk_norm ? " qk_norm" : "")
    << (residual_scalars ? " residual_scalars" : "") << (c6_head ? " c6_head" : "");
  return o.str();
}

// --------------------------------------------------------------- loading
std::shared_ptr<Model> Model::load(const std::string &path) {
  std::ifstream in(path, std::ios::binary);
  if (!in) fail("cannot read the model file " + path);
  std::vector<std::uint8_t> bytes((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
  return load_bytes(std::move(bytes), path);
}

// The container of docs/FORMAT.md:12-82, checked in four passes: the fixed
// header and both digests; the manifest text (canonical JSON) and its
// identity fields; the tensor table, record by record; then the payload as a
// sequence of zero gaps and tensors ordered by offset, which must tile it
// exactly.  The first failed rule ends the load.
std::shared_ptr<Model> Model::load_bytes(std::vector<std::uint8_t> bytes, const std::string &origin) {
  constexpr std::size_t kHeaderBytes = 128;
  const std::size_t file_size = bytes.size();
  // -- pass 1: header
  if (file_size < kHeaderBytes)
    fail("file of " + std::to_string(file_size) + " bytes cannot hold the 128-byte header");
  const std::uint8_t *h = bytes.data();
  if (std::memcmp(h, "SO3LRN1\0", 8) != 0) fail("header magic is not SO3LRN1\\0");
  const std::uint32_t version = get_u32(h + 8), flags = get_u32(h + 12);
  if (version != 1 || flags != 0)
    fail("header declares version " + std::to_string(version) + ", flags " + std::to_string(flags) +
         "; this reader takes version 1 with flags 0");
  if (std::any_of(h + 96, h + kHeaderBytes, [](std::uint8_t c) { return c != 0; }))
    fail("header bytes 96..127 are reserved and must be zero");
  const std::uint64_t man_len = get_u64(h + 16), pay_len = get_u64(h + 24);
  const std::uint64_t body = file_size - kHeaderBytes;
  if (man_len > body || pay_len != body - man_len)
    fail("header sizes (manifest " + std::to_string(man_len) + ", payload " + std::to_string(pay_len) +
         ") do not add up to the " + std::to_string(body) + " bytes after the header");
  const std::uint8_t *man = h + kHeaderBytes, *pay = man + man_len;
  if (std::memcmp(sha256(man, man_len).data(), h + 32, 32) != 0) fail("manifest digest does not match the header");
  if (std::memcmp(sha256(pay, pay_len).data(), h + 64, 32) != 0) fail("payload digest does not match the header");

  // -- pass 2: manifest text and identity
  auto m = std::make_shared<Model>();
  m->payload_begin_ = kHeaderBytes + man_len;
  m->manifest_ = Json::parse_canonical(std::string(reinterpret_cast<const char *>(man), man_len));
  const Json &mf = m->manifest_;
  struct Expect {
    const char *key, *text;
    std::uint64_t count;  // compared when text is null
  };
  static const Expect identity[] = {{"format", "so3lr-native", 0},     {"format_version", nullptr, 1},
                                    {"endianness", "little", 0},       {"tensor_alignment", nullptr, 64},
                                    {"model_family", "SO3LR", 0}};
  for (const Expect &e : identity) {
    const Json &v = mf.at(e.key);
    const bool ok = e.text ? (v.kind == Json::String && v.str == e.text) : (v.kind == Json::Number && v.uint() == e.count);
    if (!ok)
      fail(std::string("manifest '") + e.key + "' must be " + (e.text ? e.text : std::to_string(e.count)));
  }

  // -- pass 3: tensor table (names sorted and unique, as the format requires)
  const Json &table = mf.at("tensors");
  if (table.kind != Json::Array) fail("manifest 'tensors' must be an array");
  std::vector<Tensor> recs;
  std::set<std::string> keys;
  std::string last_name;
  std::uint64_t byte_total = 0;
  for (const Json &rec : table.arr) {
    const std::string name = rec.at("name").string();
    if (!recs.empty() && !(last_name < name))
      fail("tensor table: '" + name + "' is out of order or repeated (names must increase strictly)");
    last_name = name;
    Tensor t;
    t.state_key = rec.at("state_key").string();
    if (!keys.insert(t.state_key).second) fail("tensor table: state key '" + t.state_key + "' appears twice");
    t.dtype = rec.at("dtype").string();
    const std::size_t esize = element_size(t.dtype);
    if (esize == 0) fail("tensor '" + name + "': dtype '" + t.dtype + "' is not a version-1 dtype");
    std::uint64_t elems = 1;
    for (const Json &dim : rec.at("shape").arr) {
      const std::uint64_t d = dim.uint();
      if (d != 0 && elems > (std::uint64_t(1) << 62) / d) fail("tensor '" + name + "': shape too large");
      elems *= d;
      t.shape.push_back(std::size_t(d));
    }
    t.offset = std::size_t(rec.at("offset").uint());
    t.nbytes = std::size_t(rec.at("nbytes").uint());
    if (t.nbytes != elems * esize)
      fail("tensor '" + name + "': " + std::to_string(t.nbytes) + " bytes recorded, shape and dtype need " +
           std::to_string(elems * esize));
    if (t.offset % 64 != 0) fail("tensor '" + name + "': offset " + std::to_string(t.offset) + " is not 64-byte aligned");
    if (t.offset > pay_len || t.nbytes > pay_len - t.offset) fail("tensor '" + name + "' reaches past the payload");
    if (sha256_hex(pay + t.offset, t.nbytes) != rec.at("sha256").string())
      fail("tensor '" + name + "': digest does not match its bytes");
    byte_total += t.nbytes;
    recs.push_back(std::move(t));
  }
  if (mf.at("tensor_count").uint() != recs.size() || mf.at("tensor_bytes").uint() != byte_total)
    fail("manifest tensor_count / tensor_bytes disagree with the tensor table");

  // -- pass 4: payload coverage, in offset order: zero gaps, no overlap,
  // nothing after the last tensor
  std::vector<const Tensor *> by_offset;
  for (const Tensor &t : recs) by_offset.push_back(&t);
  std::stable_sort(by_offset.begin(), by_offset.end(),
                   [](const Tensor *a, const Tensor *b) { return a->offset < b->offset; });
  std::size_t cursor = 0;
  for (const Tensor *t : by_offset) {
    if (t->offset < cursor)
      fail("payload: tensor '" + t->state_key + "' at offset " + std::to_string(t->offset) + " overlaps the one before");
    if (std::any_of(pay + cursor, pay + t->offset, [](std::uint8_t c) { return c != 0; }))
      fail("payload: alignment gap before tensor '" + t->state_key + "' is not zero-filled");
    cursor = t->offset + t->nbytes;
  }
  if (cursor != pay_len) fail("payload: " + std::to_string(pay_len - cursor) + " bytes after the last tensor belong to none");
  for (Tensor &t : recs) m->tensors_.emplace(t.state_key, std::move(t));
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
  // widths: those of the released models (so3lr_capabilities.cpp:54-69):
  // F = 128 or 256 in heads of 32, one degree slot per head, R = 32 or 64
  arch_.F = int(a.at("invariant_features").uint());
  arch_.R = int(a.at("radial_basis_features").uint());
  arch_.heads = int(a.at("attention_heads").uint());
  need(arch_.F == 128 || arch_.F == 256, "invariant_features other than 128 or 256");
  need(a.at("attention_head_width").uint() == 32 && arch_.heads * 32 == arch_.F,
       "attention heads other than invariant_features / 32 heads of width 32");
  need(a.at("euclidean_degree_channels").uint() == std::uint64_t(arch_.heads),
       "euclidean_degree_channels other than attention_heads (one equivariant head per degree slot)");
  need(arch_.R == 32 || arch_.R == 64, "radial_basis_features other than 32 or 64");
  // normalisation: one module choice for both positions, each position
  // switchable; the reference's post-attention block requires the first
  // (kokkos_post_attention_block0.cpp:386-390)
  const NormMode enabled = flag("use_rms_norm", false) ? NormMode::Rms : NormMode::Layer;
  arch_.norm1 = flag("layer_normalization_1", true) ? enabled : NormMode::None;
  arch_.norm2 = flag("layer_normalization_2", true) ? enabled : NormMode::None;
  need(arch_.norm1 != NormMode::None, "no normalisation at the first position (layer_normalization_1 = false)");
  arch_.qk_norm = flag("qk_norm", false);
  arch_.residual_scalars = flag("use_residual_scalars", false);
  need(flag("residual_mlp_1", true) && !flag("residual_mlp_2", false), "residual MLP layout other than mlp_1 only");
  if (const Json *q = a.find("qk_nonlinearity")) need(q->string() == "identity", "QK nonlinearity other than identity");
  // repulsion: explicit repulsion_type, else zbl_enabled (so3lr_architecture.cpp:356-368)
  if (const Json *r = a.find("repulsion_type")) {
    need(r->string() == "zbl_learned" || r->string() == "nlh", "repulsion other than learned ZBL or NLH tables");
    arch_.nlh = r->string() == "nlh";
  } else {
    need(a.find("zbl_enabled") && a.at("zbl_enabled").number() == 1.0, "missing ZBL repulsion");
  }
  if (const Json *zc = a.find("zbl_cutoff_function")) need(zc->string() == "phys", "ZBL cutoff function other than phys");
  // attention normalisation (so3lr_architecture.cpp:126-156, 340-355)
  std::string norm_kind = "avg_num_neighbors";
  if (const Json *mn = a.find("message_normalization")) norm_kind = mn->string();
  need(norm_kind == "identity" || norm_kind == "sqrt_num_features" || norm_kind == "avg_num_neighbors",
       "message normalisation '" + norm_kind + "'");
  need(norm_kind != "avg_num_neighbors" || a.find("avg_num_neighbors") != nullptr,
       "message normalisation avg_num_neighbors without an avg_num_neighbors value");
  // heads: energy, charges, Hirshfeld ratios, optionally the C6 ratios
  // (kokkos_output_heads.cpp:271-283)
  const Json &heads = a.at("output_heads");
  const bool three = heads.arr.size() == 3;
  const bool four = heads.arr.size() == 4 && heads.arr[3].string() == "c6_ratios_output_block";
  need((three || four) && heads.arr[0].string() == "atomic_energy_output_block" &&
           heads.arr[1].string() == "partial_charges_output_block" &&
           heads.arr[2].string() == "hirshfeld_output_block",
       "output heads other than energy, partial charges, Hirshfeld ratios and optionally C6 ratios");
  arch_.c6_head = four;
  if (misses.empty()) {
    // degree slots (so3lr_architecture.cpp:246-293): block 0's repeats, each
    // 2l + 1 with l in 1..4, sorted; every block carries the same layout
    const std::size_t S = std::size_t(arch_.heads);
    const auto rep = i64("model.euclidean_transformers.0.euclidean_attention_block.degree_repeats", {S});
    arch_.degrees.clear();
    arch_.E = 0;
    for (std::size_t s = 0; s < S; ++s) {
      const std::int64_t r = rep[s];
      if (r < 3 || r > 9 || r % 2 == 0) fail("degree_repeats entries must be 2l + 1 with l in 1..4");
      arch_.degrees.push_back(int((r - 1) / 2));
      arch_.E += int(r);
      if (s > 0 && arch_.degrees[s] < arch_.degrees[s - 1]) fail("degree slots must be sorted by degree");
    }
    for (int b = 0; b < arch_.layers; ++b) {
      const std::string p = "model.euclidean_transformers." + std::to_string(b);
      for (const char *blk : {".euclidean_attention_block.degree_repeats", ".interaction_block.degree_repeats"})
        if (i64(p + blk, {S}) != rep) fail("block " + std::to_string(b) + " has another degree layout than block 0");
    }
    // the energy and charge heads' hidden width (so3lr_architecture.cpp:444-446)
    const Tensor &ew = tensor("model.atomic_energy_output_block.layers.0.weight");
    if (ew.shape.size() != 2 || ew.shape[1] != std::size_t(arch_.F) || ew.shape[0] == 0 || ew.shape[0] > 1024)
      fail("energy head first layer must be (hidden, invariant_features)");
    arch_.head_hidden = int(ew.shape[0]);
    arch_.generic = !(arch_.F == kF && arch_.R == kR && arch_.degrees == std::vector<int>({1, 2, 3, 4}) &&
                      arch_.head_hidden == kF);
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
  if (norm_kind == "identity") arch_.attention_norm = 1.0;
  else if (norm_kind == "sqrt_num_features") arch_.attention_norm = std::sqrt(double(kHW));
  else arch_.attention_norm = num("avg_num_neighbors");
  if (!(arch_.attention_norm > 0) || !std::isfinite(arch_.attention_norm)) fail("attention normalisation must be positive");
  if (!(arch_.sr_cutoff > 0) || !(arch_.lr_cutoff >= arch_.sr_cutoff)) fail("invalid native model cutoffs");
  if (!(arch_.embedding_scale > 0) || !std::isfinite(arch_.embedding_scale)) fail("embedding scale must be positive");
  arch_.gamma = f64("model.radial_embedding.radial_basis_fn.gamma", {})[0];
  // the repulsion prefactor and switch are shared by both kinds; the
  // screening parameters are learned ZBL's (so3lr_repulsion_setup.cpp:9-34)
  arch_.zbl_ke = num("zbl_ke");
  arch_.zbl_switch_off = num("zbl_switch_off_angstrom");
  if (!(arch_.zbl_ke > 0) || !(arch_.zbl_switch_off > 0)) fail("invalid repulsion prefactor or switch");
  if (arch_.nlh) {
    const Tensor &ta = tensor("physical.nlh_a");
    const std::size_t cap = ta.shape.empty() ? 0 : ta.shape[0];
    if (cap == 0 || cap > 118 || ta.shape != std::vector<std::size_t>({cap, cap, 3}) ||
        tensor("physical.nlh_b").shape != ta.shape || ta.dtype != "float64" || tensor("physical.nlh_b").dtype != "float64")
      fail("NLH repulsion tables physical.nlh_a / physical.nlh_b must be float64 (cap, cap, 3)");
  } else {
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
  }
  {
    // the Bernstein exponents k = 0..R-1 and R-1-k (the v1 filter kernels
    // step the basis through them)
    const int R = arch_.R;
    const auto k = i64("model.radial_embedding.radial_basis_fn.k", {std::size_t(R)});
    const auto kr = i64("model.radial_embedding.radial_basis_fn.k_rev", {std::size_t(R)});
    for (int c = 0; c < R; ++c)
      if (k[c] != c || kr[c] != R - 1 - c) fail("Bernstein basis exponents other than k = 0..R-1, k_rev = R-1-k");
  }
  // The filter kernels evaluate SiLU through a table-based e^x whose argument
  // reduction is exact for |x| < 2800 (the generic node layers call exp).  The
  // radial hidden layer sees W0 rbf + b0 with every Bernstein value in [0, 1],
  // and the v1 node MLP sees W1 silu(n1) + b1 with |n1_k| <= sqrt(F) |w_k| +
  // |b_k| after either normalisation: both are bounded by the weights, checked
  // here (the spherical branch clamps its argument instead).
  if (arch_.generic) {
    const std::size_t F = std::size_t(arch_.F), R = std::size_t(arch_.R);
    double worst = 0.0;
    for (int b = 0; b < arch_.layers; ++b) {
      const std::string p = "model.euclidean_transformers." + std::to_string(b) + ".";
      for (const char *fn : {"filter_net_inv.", "filter_net_ev."}) {
        const auto w0 = f64(p + fn + "mlp_rbf.0.weight", {F, R});
        const auto b0 = f64(p + fn + "mlp_rbf.0.bias", {F});
        for (std::size_t c = 0; c < F; ++c) {
          double acc = std::abs(b0[c]);
          for (std::size_t k = 0; k < R; ++k) acc += std::abs(w0[c * R + k]);
          worst = std::max(worst, acc);
        }
      }
    }
    if (!(worst < 2000.0))
      fail("weights allow SiLU arguments up to " + std::to_string(worst) +
           " in the filters' radial hidden layers; this build's activations take |x| < 2000");
  } else {
    double worst = 0.0;
    const double sf = std::sqrt(double(kF));
    for (int b = 0; b < arch_.layers; ++b) {
      const std::string p = "model.euclidean_transformers." + std::to_string(b) + ".";
      for (const char *fn : {"filter_net_inv.", "filter_net_ev."}) {
        const auto w0 = f64(p + fn + "mlp_rbf.0.weight", {std::size_t(kF), std::size_t(kR)});
        const auto b0 = f64(p + fn + "mlp_rbf.0.bias", {std::size_t(kF)});
        for (int c = 0; c < kF; ++c) {
          double acc = std::abs(b0[c]);
          for (int k = 0; k < kR; ++k) acc += std::abs(w0[std::size_t(c) * kR + k]);
          worst = std::max(worst, acc);
        }
      }
      std::vector<double> lnw(kF, 1.0), lnb(kF, 0.0);
      if (arch_.norm1 == NormMode::Layer) {
        lnw = f64(p + "layer_norm_inv_1.weight", {std::size_t(kF)});
        lnb = f64(p + "layer_norm_inv_1.bias", {std::size_t(kF)});
      }
      const auto w1 = f64(p + "mlp_1.1.weight", {std::size_t(kF), std::size_t(kF)});
      const auto b1 = f64(p + "mlp_1.1.bias", {std::size_t(kF)});
      for (int c = 0; c < kF; ++c) {
        double acc = std::abs(b1[c]);
        for (int k = 0; k < kF; ++k)
          acc += std::abs(w1[std::size_t(c) * kF + k]) * (sf * std::abs(lnw[k]) + std::abs(lnb[k]));
        worst = std::max(worst, acc);
      }
    }
    if (!(worst < 2000.0))
      fail("weights allow SiLU arguments up to " + std::to_string(worst) +
           " in the filter or node MLP hidden layers; this build's activations take |x| < 2000");
  }
  if (arch_.c6_head) {
    // a ratio head of the Hirshfeld head's widths (kokkos_output_heads.cpp:108-132;
    // the kernels here take hidden and key width 64)
    const std::string c = "model.c6_ratios_output_block.";
    const std::size_t HH = kHH, F = std::size_t(arch_.F);
    const std::pair<const char *, std::vector<std::size_t>> parts[] = {
        {"transform_features.0.weight", {HH, F}}, {"transform_features.0.bias", {HH}},
        {"transform_features.2.weight", {HH, HH}}, {"transform_features.2.bias", {HH}},
        {"q_embedding.weight", {100, HH}},       {"v_shift_embedding.weight", {100, 1}}};
    for (const auto &pt : parts)
      if (tensor(c + pt.first).dtype != "float64" || tensor(c + pt.first).shape != pt.second)
        fail("C6 ratio head tensor " + c + pt.first + " is not float64 of the Hirshfeld head's shape");
  }
  if (arch_.residual_scalars) {
    const std::vector<std::size_t> shp{std::size_t(arch_.layers)};
    for (const char *k : {"model.resid_lambdas", "model.x0_lambdas"})
      if (tensor(k).dtype != "float64" || tensor(k).shape != shp)
        fail(std::string("residual scalars ") + k + " must be float64 of length interaction_blocks");
  }
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
  F = model.arch().F;
  for (int k = 0; k < 2; ++k) {
    const std::string b = names[k];
    wq[k] = model.f64(b + "Wq.weight", {std::size_t(F), 118});
    wk[k] = model.f64(b + "Wk", {2, std::size_t(F)});
    wv[k] = model.f64(b + "Wv", {2, std::size_t(F)});
    m1[k] = model.f64(b + "mlp.1.weight", {std::size_t(F), std::size_t(F)});
    m3[k] = model.f64(b + "mlp.3.weight", {std::size_t(F), std::size_t(F)});
  }
}

std::vector<double> ChargeSpin::table(const std::int64_t counts[119], double total_charge,
                                      double unpaired) const {
  std::vector<double> out(118 * F, 0.0);
  auto silu = [](double x) { return x / (1.0 + std::exp(-x)); };
  const double psis[2] = {total_charge, unpaired};
  for (int k = 0; k < 2; ++k) {
    const double psi = psis[k];
    if (psi == 0.0) continue;  // the module's output is exactly zero
    const int row = psi < 0.0 ? 1 : 0;
    const double *key = wk[k].data() + row * F, *val = wv[k].data() + row * F;
    double y[119] = {0};
    double den = 0.0;
    for (int zz = 1; zz <= 118; ++zz) {
      if (counts[zz] <= 0) continue;
      double qk = 0.0;
      for (int c = 0; c < F; ++c) qk += wq[k][c * 118 + (zz - 1)] * key[c];
      const double x = qk / std::sqrt(double(F));
      y[zz] = std::max(x, 0.0) + std::log1p(std::exp(-std::abs(x)));  // softplus
      den += double(counts[zz]) * y[zz];
    }
    std::vector<double> x(F), sx(F), h(F), sh(F);
    for (int zz = 1; zz <= 118; ++zz) {
      if (counts[zz] <= 0) continue;
      const double w = psi * y[zz] / den;
      for (int c = 0; c < F; ++c) { x[c] = w * val[c]; sx[c] = silu(x[c]); }
      for (int o = 0; o < F; ++o) {
        double s = 0.0;
        for (int i = 0; i < F; ++i) s += m1[k][o * F + i] * sx[i];
        h[o] = s;
        sh[o] = silu(s);
      }
      for (int o = 0; o < F; ++o) {
        double s = 0.0;
        for (int i = 0; i < F; ++i) s += m3[k][o * F + i] * sh[i];
        out[(zz - 1) * F + o] += x[o] + s;
      }
    }
  }
  return out;
}

// (Q, M) against the composition.  With Z_tot the nuclear charge, the
// system has n_e = Z_tot - Q electrons, of which M - 1 are unpaired; the rest
// pair up, so n_e - (M - 1) must be even and non-negative, i.e. n_e + M is
// odd and M - 1 <= n_e.  Q and M must be whole numbers; M >= 1.  (The rule
// of src/so3lr_charge_spin.cpp:116-141.)
std::string charge_multiplicity_problem(const std::int64_t counts[119], double q, double mult) {
  constexpr double kWhole = 9007199254740992.0;  // 2^53: beyond it a double is no longer a count
  auto whole = [&](double v) { return std::isfinite(v) && std::fabs(v) < kWhole && std::nearbyint(v) == v; };
  std::ostringstream why;
  if (!whole(q)) {
    why << "total charge " << q << " is not a whole number of elementary charges";
    return why.str();
  }
  if (!whole(mult) || mult < 1.0) {
    why << "spin multiplicity " << mult << " is not a whole number of at least 1";
    return why.str();
  }
  std::int64_t z_total = 0;
  for (int zz = 1; zz <= 118; ++zz) z_total += counts[zz] * zz;
  const std::int64_t n_e = z_total - std::int64_t(q), m = std::int64_t(mult);
  if (n_e < 0) {
    why << "charge " << std::int64_t(q) << " removes more electrons than the " << z_total << " the nuclei bring";
    return why.str();
  }
  if (m - 1 > n_e) {
    why << "multiplicity " << m << " means " << (m - 1) << " unpaired electrons, but the system has only " << n_e;
    return why.str();
  }
  if ((n_e + m) % 2 == 0) {
    why << "with " << n_e << " electrons the multiplicity must be " << (n_e % 2 ? "even" : "odd") << ", not " << m;
    return why.str();
  }
  return std::string();
}

}  // namespace so3lr_amd
