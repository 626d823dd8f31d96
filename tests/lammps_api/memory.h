// Test infrastructure: Memory::create/destroy of 2-d arrays (src/memory.h):
// one contiguous block of n1*n2 values behind n1 row pointers.
#pragma once
#include "pointers.h"

namespace LAMMPS_NS {
class Memory {
 public:
  template <class T> T **create(T **&array, int n1, int n2, const char *) {
    T *data = new T[static_cast<std::size_t>(n1) * n2]();
    array = new T *[n1];
    for (int i = 0; i < n1; ++i) array[i] = data + static_cast<std::size_t>(i) * n2;
    return array;
  }
  template <class T> void destroy(T **&array) {
    if (array) {
      delete[] array[0];
      delete[] array;
    }
    array = nullptr;
  }
};
}    // namespace LAMMPS_NS
