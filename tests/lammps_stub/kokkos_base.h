// stand-in for LAMMPS kokkos_base.h (see lammps_stub.h)
#pragma once
#include "lammps_stub.h"
