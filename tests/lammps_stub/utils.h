// stand-in for LAMMPS utils.h (see lammps_stub.h)
#pragma once
#include "lammps_stub.h"
