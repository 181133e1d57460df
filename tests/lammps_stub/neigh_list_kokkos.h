// stand-in for LAMMPS neigh_list_kokkos.h (see lammps_stub.h)
#pragma once
#include "lammps_stub.h"
