// Test infrastructure: Error (src/error.h).  all/one/universe_* throw the
// formatted message (LAMMPS would print it and end the run); warning keeps it.
#pragma once
#include "pointers.h"

#include <stdexcept>
#include <string>
#include <vector>

namespace LAMMPS_NS {
struct LammpsAbort : std::runtime_error {
  using std::runtime_error::runtime_error;
};

class Error {
 public:
  std::vector<std::string> warnings;
  [[noreturn]] void all(const std::string &, int, const std::string &str) { throw LammpsAbort(str); }
  template <class... Args>
  [[noreturn]] void all(const std::string &, int, const std::string &f, const Args &...args) {
    throw LammpsAbort(utils::format(f, args...));
  }
  [[noreturn]] void one(const std::string &, int, const std::string &str) { throw LammpsAbort(str); }
  [[noreturn]] void universe_all(const std::string &, int, const std::string &str) { throw LammpsAbort(str); }
  [[noreturn]] void universe_one(const std::string &, int, const std::string &str) { throw LammpsAbort(str); }
  template <class... Args> void warning(const std::string &, int, const std::string &f, const Args &...args) {
    warnings.push_back(utils::format(f, args...));
  }
};
}    // namespace LAMMPS_NS
