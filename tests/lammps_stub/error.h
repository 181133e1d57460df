// stand-in for LAMMPS error.h (see lammps_stub.h)
#pragma once
#include "lammps_stub.h"
