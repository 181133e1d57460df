"""Velocity-Verlet NVE driver on the MI355X evaluator.

Used for the capacity measurement (tiled execution at millions of atoms): a
short NVE run at a fixed time step, with the neighbour graph reused while
no atom has moved more than half the skin since the graph was built (the
calculator's rule, calculator.py:2894-2899).  Units: eV, Angstrom, amu; the
time unit is Angstrom * sqrt(amu / eV) = 10.1805 fs.
"""

from __future__ import annotations

import time

import numpy as np

AMU_MASS = {1: 1.008, 6: 12.011, 7: 14.007, 8: 15.999, 13: 26.982, 14: 28.085, 22: 47.867, 26: 55.845,
            29: 63.546, 38: 87.62}
FS = 1.0 / 10.180505671156723  # one femtosecond in Angstrom*sqrt(amu/eV)
KB = 8.617333262e-5  # eV/K


class NVE:
    """Velocity Verlet for a periodic system with an MACEKokkosFloat
    evaluator (positions on the host, forces reduced on the device)."""

    def __init__(self, evaluator, system, skin=0.5, temperature=300.0, seed=0):
        self.ev = evaluator
        self.numbers = np.asarray(system["numbers"])
        self.positions = np.array(system["positions"], dtype=np.float64)
        self.cell = np.asarray(system["cell"], dtype=np.float64)
        self.inv = np.linalg.inv(self.cell)
        self.volume = abs(float(np.linalg.det(self.cell)))
        self.skin = float(skin)
        lut = {z: i for i, z in enumerate(self.ev.atomic_numbers)}
        self.types = np.array([lut[int(z)] for z in self.numbers], dtype=np.int32)
        self.masses = np.array([AMU_MASS[int(z)] for z in self.numbers])[:, None]
        rng = np.random.default_rng(seed)
        v = rng.normal(size=self.positions.shape) * np.sqrt(KB * temperature / self.masses)
        v -= (self.masses * v).sum(axis=0) / self.masses.sum()
        self.velocities = v
        self.rebuilds = 0
        self.gen = None
        self.ref = None
        self._build()
        self.forces, self.energy = self._compute()

    def _build(self):
        g = self.ev._prepare_periodic_factorized_graph(self.types, self.positions.reshape(-1), self.cell.reshape(-1),
                                                       self.inv.reshape(-1), self.ev.r_cut + self.skin)
        self.gen = g["generation"]
        self.num_edges = g["num_edges"]
        self.ref = self.positions.copy()
        self.rebuilds += 1

    def _compute(self):
        d = self.positions - self.ref
        f = d @ self.inv
        f -= np.floor(f + 0.5)
        if np.max(np.einsum("ij,ij->i", f @ self.cell, f @ self.cell)) > (0.5 * self.skin) ** 2:
            self._build()
        self.ev._compute_prepared_factorized_positions(self.gen, self.positions.reshape(-1))
        forces = self.ev._reduce_atom_forces(len(self.types), None, None, self.gen)
        return forces, self.ev._total_energy()

    def kinetic(self):
        return 0.5 * float(np.sum(self.masses * self.velocities ** 2))

    def run(self, steps, dt_fs=1.0, progress=None):
        """Advance ``steps`` steps; returns (seconds per step, total-energy
        trace [E_pot + E_kin] including the initial state).  ``progress``
        (optional) is called with (step, total energy) after every step."""
        dt = dt_fs * FS
        trace = [self.energy + self.kinetic()]
        t0 = time.perf_counter()
        for step in range(steps):
            self.velocities += 0.5 * dt * self.forces / self.masses
            self.positions += dt * self.velocities
            self.forces, self.energy = self._compute()
            self.velocities += 0.5 * dt * self.forces / self.masses
            trace.append(self.energy + self.kinetic())
            if progress:
                progress(step + 1, trace[-1])
        return (time.perf_counter() - t0) / max(steps, 1), trace
