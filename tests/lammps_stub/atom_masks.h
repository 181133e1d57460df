// stand-in for LAMMPS atom_masks.h (see lammps_stub.h)
#pragma once
#include "lammps_stub.h"
