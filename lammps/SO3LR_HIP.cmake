# PKG_SO3LR_HIP: so3lr/native/mpi (and, with MPI, so3lr/turbo) built into
# LAMMPS over libso3lr_hip.so -- the built-in route of the reference's
# PKG_SO3LR (integration/lammps_builtin/cmake/Packages/SO3LR.cmake:1-35).
# The compute lives in the prebuilt library, so this package needs neither
# Kokkos nor a GPU toolkit when LAMMPS is compiled.
#
# Install as cmake/Modules/Packages/SO3LR_HIP.cmake of a LAMMPS tree, copy
# this directory (with turbo/) to src/SO3LR_HIP/lammps/ and the repository's
# include/ to src/SO3LR_HIP/include/, add SO3LR_HIP to the package list of
# cmake/CMakeLists.txt, and configure with
#   -D PKG_SO3LR_HIP=on -D SO3LR_HIP_LIBRARY_DIR=/path/to/repo/so3lrxlammps_amd
set(SO3LR_HIP_ROOT "${LAMMPS_SOURCE_DIR}/SO3LR_HIP")
set(SO3LR_HIP_LIBRARY_DIR "" CACHE PATH "directory holding libso3lr_hip.so")
find_library(SO3LR_HIP_LIBRARY so3lr_hip HINTS "${SO3LR_HIP_LIBRARY_DIR}" REQUIRED)
RegisterStyles("${SO3LR_HIP_ROOT}/lammps")
target_sources(lammps PRIVATE "${SO3LR_HIP_ROOT}/lammps/pair_so3lr_hip.cpp")
target_include_directories(lammps PRIVATE "${SO3LR_HIP_ROOT}/include" "${SO3LR_HIP_ROOT}/lammps")
target_link_libraries(lammps PRIVATE "${SO3LR_HIP_LIBRARY}")
# so3lr/turbo sits in its own directory, so that its style is registered
# only where it can be built: with MPI and libso3lr_turbo.so
find_library(SO3LR_TURBO_LIBRARY so3lr_turbo HINTS "${SO3LR_HIP_LIBRARY_DIR}")
if(BUILD_MPI AND SO3LR_TURBO_LIBRARY)
  RegisterStyles("${SO3LR_HIP_ROOT}/lammps/turbo")
  target_sources(lammps PRIVATE "${SO3LR_HIP_ROOT}/lammps/turbo/pair_so3lr_turbo_hip.cpp")
  target_include_directories(lammps PRIVATE "${SO3LR_HIP_ROOT}/lammps/turbo")
  target_link_libraries(lammps PRIVATE "${SO3LR_TURBO_LIBRARY}")
  message(STATUS "SO3LR_HIP pair styles enabled: so3lr/native/mpi, so3lr/turbo")
else()
  message(STATUS "SO3LR_HIP pair style enabled: so3lr/native/mpi (so3lr/turbo needs MPI and libso3lr_turbo)")
endif()
