// stand-in for LAMMPS memory_kokkos.h (see lammps_stub.h)
#pragma once
#include "lammps_stub.h"
