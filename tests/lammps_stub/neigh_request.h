// stand-in for LAMMPS neigh_request.h (see lammps_stub.h)
#pragma once
#include "lammps_stub.h"
