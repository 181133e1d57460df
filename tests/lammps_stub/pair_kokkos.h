// stand-in for LAMMPS pair_kokkos.h (see lammps_stub.h)
#pragma once
#include "lammps_stub.h"
