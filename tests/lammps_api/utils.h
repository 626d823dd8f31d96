// Test infrastructure: utils::numeric / utils::logmesg (src/utils.h) and the
// {}-style formatting LAMMPS takes from fmt, reduced to {} and {:g}.
#pragma once
#include <cstdlib>
#include <sstream>
#include <stdexcept>
#include <string>

namespace LAMMPS_NS {
class LAMMPS;
namespace utils {

inline void format_one(std::ostringstream &out, const std::string &spec, double v) {
  if (spec == ":g") {
    char buf[64];
    std::snprintf(buf, sizeof(buf), "%g", v);
    out << buf;
  } else {
    out << v;
  }
}
template <class T> void format_one(std::ostringstream &out, const std::string &, const T &v) { out << v; }

inline void format_rest(std::ostringstream &out, const std::string &f, std::size_t pos) { out << f.substr(pos); }
template <class T, class... Rest>
void format_rest(std::ostringstream &out, const std::string &f, std::size_t pos, const T &v, const Rest &...rest) {
  const std::size_t a = f.find('{', pos);
  if (a == std::string::npos) { out << f.substr(pos); return; }
  const std::size_t b = f.find('}', a);
  out << f.substr(pos, a - pos);
  format_one(out, f.substr(a + 1, b - a - 1), v);
  format_rest(out, f, b + 1, rest...);
}
template <class... Args> std::string format(const std::string &f, const Args &...args) {
  std::ostringstream out;
  format_rest(out, f, 0, args...);
  return out.str();
}

inline double numeric(const char *, int, const std::string &str, bool, LAMMPS *) {
  char *end = nullptr;
  const double v = std::strtod(str.c_str(), &end);
  if (str.empty() || *end != '\0') throw std::runtime_error("Expected floating point parameter instead of '" + str + "'");
  return v;
}

std::string &log_text();    // what logmesg wrote (the driver owns it)
template <class... Args> void logmesg(LAMMPS *, const std::string &f, const Args &...args) {
  log_text() += format(f, args...);
}

}    // namespace utils
}    // namespace LAMMPS_NS
