"""Seeded synthetic atomic systems of the benchmark configurations.

A system is a plain dict: ``numbers`` int[N], ``positions`` float64[N,3] (Å),
``cell`` float64[3,3] (rows are lattice vectors), ``pbc`` bool[3].
"""

from __future__ import annotations

import math

import numpy as np

SRTIO3_A = 3.905
# Sr (0,0,0), Ti (1/2,1/2,1/2), O (1/2,1/2,0), (1/2,0,1/2), (0,1/2,1/2)
_SRTIO3_BASIS = [(38, (0.0, 0.0, 0.0)), (22, (0.5, 0.5, 0.5)),
                 (8, (0.5, 0.5, 0.0)), (8, (0.5, 0.0, 0.5)),
                 (8, (0.0, 0.5, 0.5))]


def srtio3_supercell(n, sigma=0.05, seed=0, a=SRTIO3_A):
    """Cubic SrTiO3 n x n x n supercell (5 n^3 atoms, cell order ix, iy, iz,
    then the basis) with Gaussian displacements of standard deviation
    ``sigma`` (Å) drawn from ``numpy.random.default_rng(seed)``."""
    numbers = np.array([z for z, _ in _SRTIO3_BASIS], dtype=np.int64)
    basis = np.array([f for _, f in _SRTIO3_BASIS], dtype=np.float64)
    r = np.arange(n, dtype=np.float64)
    cells = np.stack(np.meshgrid(r, r, r, indexing="ij"), axis=-1).reshape(-1, 3)
    positions = (cells[:, None, :] + basis[None, :, :]).reshape(-1, 3) * a
    rng = np.random.default_rng(seed)
    positions = positions + sigma * rng.normal(size=positions.shape)
    return {"numbers": np.tile(numbers, n ** 3),
            "positions": positions,
            "cell": np.eye(3) * (a * n),
            "pbc": np.array([True, True, True])}


IRREGULAR_ELEMENTS = (1, 6, 7, 8, 13, 14, 22, 26, 29, 38)


def irregular_box(num_atoms=20000, density=0.08, min_distance=1.8, seed=0,
                  elements=IRREGULAR_ELEMENTS):
    """Uniform random atoms in a periodic cube, rejection-sampled to a minimum
    separation, species drawn uniformly from ``elements``."""
    L = (num_atoms / density) ** (1.0 / 3.0)
    rng = np.random.default_rng(seed)
    nb = max(1, int(L // min_distance))
    bins = {}
    pos = np.empty((num_atoms, 3))
    count = 0
    d2 = min_distance * min_distance
    while count < num_atoms:
        p = rng.uniform(0.0, L, size=3)
        b = tuple((p / L * nb).astype(int) % nb)
        ok = True
        for dx in (-1, 0, 1):
            for dy in (-1, 0, 1):
                for dz in (-1, 0, 1):
                    for j in bins.get(((b[0] + dx) % nb, (b[1] + dy) % nb,
                                       (b[2] + dz) % nb), ()):
                        d = pos[j] - p
                        d -= L * np.round(d / L)
                        if d @ d < d2:
                            ok = False
                            break
                    if not ok:
                        break
                if not ok:
                    break
            if not ok:
                break
        if ok:
            pos[count] = p
            bins.setdefault(b, []).append(count)
            count += 1
    numbers = rng.choice(np.asarray(elements), size=num_atoms)
    return {"numbers": numbers.astype(np.int64), "positions": pos,
            "cell": np.eye(3) * L, "pbc": np.array([True, True, True])}


def water_box(num_molecules=10000, density_g_cm3=1.0, seed=0):
    """Rigid H2O molecules (O-H 0.957 Å, H-O-H 104.5 deg) with random
    orientations on a jittered cubic lattice in a periodic cube."""
    mass = 18.015 / 6.02214076e23  # g per molecule
    volume = num_molecules * mass / density_g_cm3 * 1e24  # Å^3
    L = volume ** (1.0 / 3.0)
    rng = np.random.default_rng(seed)
    m = int(math.ceil(num_molecules ** (1.0 / 3.0)))
    spacing = L / m
    sites = [(i, j, k) for i in range(m) for j in range(m) for k in range(m)]
    chosen = rng.permutation(len(sites))[:num_molecules]
    theta = math.radians(104.5) / 2.0
    r_oh = 0.957
    local = np.array([[0.0, 0.0, 0.0],
                      [r_oh * math.sin(theta), 0.0, r_oh * math.cos(theta)],
                      [-r_oh * math.sin(theta), 0.0, r_oh * math.cos(theta)]])
    pos = []
    numbers = []
    from .e3 import random_rotation
    for s in chosen:
        centre = (np.asarray(sites[s]) + 0.5) * spacing
        R = random_rotation(rng)
        for z, p in zip((8, 1, 1), local @ R.T + centre):
            numbers.append(z)
            pos.append(p)
    return {"numbers": np.asarray(numbers, dtype=np.int64),
            "positions": np.asarray(pos), "cell": np.eye(3) * L,
            "pbc": np.array([True, True, True])}
