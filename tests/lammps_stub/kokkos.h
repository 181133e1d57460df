// stand-in for LAMMPS kokkos.h (see lammps_stub.h)
#pragma once
#include "lammps_stub.h"
