// Test infrastructure: src/version.h.
#pragma once
#define LAMMPS_VERSION "11 Feb 2026"
