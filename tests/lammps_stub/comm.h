// stand-in for LAMMPS comm.h (see lammps_stub.h)
#pragma once
#include "lammps_stub.h"
