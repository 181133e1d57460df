// stand-in for LAMMPS neighbor.h (see lammps_stub.h)
#pragma once
#include "lammps_stub.h"
