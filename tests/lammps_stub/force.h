// stand-in for LAMMPS force.h (see lammps_stub.h)
#pragma once
#include "lammps_stub.h"
