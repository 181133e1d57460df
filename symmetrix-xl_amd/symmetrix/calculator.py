"""ASE-style ``Symmetrix`` calculator on the MI355X evaluator.

Caller contract of the reference calculator (symmetrix/source/symmetrix/
calculator.py): ``calculate`` (:3934-4021) reuses the prepared neighbour graph
while no atom has moved more than half the Verlet skin since it was built and
the cell, numbers and periodicity are unchanged (:2838-3093, threshold
:2894-2899); otherwise it rebuilds the graph on the device at cutoff + skin
(:2931-2971).  Skin edges are clamped to the cutoff by the evaluator.  Results
(:3821-3894): ``energy``/``free_energy`` are the FP64 sum of the node energies,
``energies`` the node energies, ``forces`` the FP64 atom forces and ``stress``
the Voigt 6-vector of sigma = -(1/V) sum_e f_e xyz_e^T.

ASE is optional: with it installed the class is an ``ase.calculators.
calculator.Calculator``; without it ``calculate`` takes any object with
``get_atomic_numbers``, ``get_positions``, ``get_cell`` and ``pbc`` (or a dict
with ``numbers``, ``positions``, ``cell``).
"""

from __future__ import annotations

import logging

import numpy as np

from .mace_kokkos import MACEKokkosFloat

log = logging.getLogger(__name__)

try:  # pragma: no cover - ASE is not installed in every environment
    from ase.calculators.calculator import Calculator as _Base
    from ase.calculators.calculator import all_changes as _all_changes
    HAVE_ASE = True
except ImportError:  # pragma: no cover
    HAVE_ASE = False
    _all_changes = ["positions", "numbers", "cell", "pbc"]

    class _Base:  # minimal stand-in with ASE's attribute names
        implemented_properties = []

        def __init__(self, **kwargs):
            self.results = {}
            self.atoms = None

        def calculate(self, atoms=None, properties=None, system_changes=None):
            if atoms is not None:
                self.atoms = atoms


def full_3x3_to_voigt_6_stress(s):
    """ASE's Voigt order: xx, yy, zz, yz, xz, xy."""
    s = np.asarray(s)
    return np.array([s[0, 0], s[1, 1], s[2, 2], 0.5 * (s[1, 2] + s[2, 1]), 0.5 * (s[0, 2] + s[2, 0]),
                     0.5 * (s[0, 1] + s[1, 0])])


def _system_arrays(atoms):
    if isinstance(atoms, dict):
        numbers = np.asarray(atoms["numbers"])
        positions = np.asarray(atoms["positions"], dtype=float)
        cell = np.asarray(atoms["cell"], dtype=float).reshape(3, 3)
        pbc = np.asarray(atoms.get("pbc", [True, True, True]), dtype=bool)
    else:
        numbers = np.asarray(atoms.get_atomic_numbers())
        positions = np.asarray(atoms.get_positions(), dtype=float)
        cell = np.asarray(atoms.get_cell(), dtype=float).reshape(3, 3)
        pbc = np.asarray(atoms.pbc, dtype=bool)
    return numbers, positions, cell, pbc


class _NeighborCache:
    def __init__(self, generation, numbers, positions, cell, pbc, num_edges):
        self.generation = generation
        self.numbers = numbers.copy()
        self.reference_positions = positions.copy()
        self.cell = cell.copy()
        self.pbc = pbc.copy()
        self.num_edges = num_edges


class Symmetrix(_Base):
    """MACE energies, forces and stress on one MI355X (FP32, direct
    streamed edges)."""

    implemented_properties = ["energy", "free_energy", "energies", "forces", "stress"]

    def __init__(self, model_file, dtype="float32", streamed_edges="direct", neighbor_skin=0.5,
                 head=None, **kwargs):
        super().__init__(**kwargs)
        if dtype not in ("float32", np.float32):
            raise ValueError("the MI355X evaluator implements dtype='float32'")
        if streamed_edges != "direct":
            raise ValueError("the MI355X evaluator implements streamed_edges='direct'")
        if not (neighbor_skin >= 0.0):
            raise ValueError("neighbor_skin must be non-negative")
        self.evaluator = MACEKokkosFloat(model_file, head or "")
        self.cutoff = float(self.evaluator.r_cut)
        self.neighbor_skin = float(neighbor_skin)
        self._types = {z: i for i, z in enumerate(self.evaluator.atomic_numbers)}
        self._neighbor_cache = None
        self.neighbor_graph_rebuilds = 0
        self.results = {}

    # -------------------------------------------------------------- graph
    def _node_types(self, numbers):
        try:
            return np.asarray([self._types[int(z)] for z in numbers], dtype=np.int32)
        except KeyError as exc:
            raise ValueError("atomic number %s is not in the model" % exc.args[0]) from None

    def _cache_valid(self, numbers, positions, cell, pbc):
        c = self._neighbor_cache
        if c is None or len(numbers) != len(c.numbers) or not np.array_equal(numbers, c.numbers):
            return False
        if not np.array_equal(cell, c.cell) or not np.array_equal(pbc, c.pbc):
            return False
        disp = positions - c.reference_positions
        # minimum image of the displacement (positions may have been wrapped)
        inv = np.linalg.inv(cell)
        f = disp @ inv
        f -= np.floor(f + 0.5)
        disp = f @ cell
        return float(np.max(np.linalg.norm(disp, axis=1), initial=0.0)) <= 0.5 * self.neighbor_skin

    def _prepare(self, numbers, positions, cell, pbc):
        if not np.all(pbc):
            raise NotImplementedError("the MI355X device neighbour list requires a fully periodic cell")
        if abs(np.linalg.det(cell)) <= 0.0:
            raise ValueError("cell must be invertible")
        if not np.isfinite(positions).all():
            raise ValueError("positions must be finite")
        types = self._node_types(numbers)
        inv = np.linalg.inv(cell)
        g = self.evaluator._prepare_periodic_factorized_graph(
            types, positions.reshape(-1), cell.reshape(-1), inv.reshape(-1), self.cutoff + self.neighbor_skin)
        self._neighbor_cache = _NeighborCache(g["generation"], numbers, positions, cell, pbc, g["num_edges"])
        self.neighbor_graph_rebuilds += 1
        return self._neighbor_cache

    # ---------------------------------------------------------- calculate
    def calculate(self, atoms=None, properties=None, system_changes=_all_changes):
        if properties is None:
            properties = self.implemented_properties
        if HAVE_ASE:
            super().calculate(atoms, properties, system_changes)
            atoms = self.atoms
        elif atoms is not None:
            self.atoms = atoms
        else:
            atoms = self.atoms
        numbers, positions, cell, pbc = _system_arrays(atoms)
        if self._cache_valid(numbers, positions, cell, pbc):
            cache = self._neighbor_cache
        else:
            cache = self._prepare(numbers, positions, cell, pbc)
        ev = self.evaluator
        ev._compute_prepared_factorized_positions(cache.generation, positions.reshape(-1))
        node_energies = np.array(ev.node_energies, dtype=np.float64, copy=True)
        energy = float(np.sum(node_energies, dtype=np.float64))
        self.results = {"energy": energy, "free_energy": energy, "energies": node_energies}
        self.results["forces"] = np.asarray(ev._reduce_atom_forces(len(numbers), None, None, cache.generation))
        if "stress" in properties:
            volume = abs(float(np.linalg.det(cell)))
            sigma = ev._reduce_stress(volume, None, cache.generation)
            self.results["stress"] = full_3x3_to_voigt_6_stress(sigma)
        return self.results

    def get_property(self, name, atoms=None, allow_calculation=True):
        if HAVE_ASE:
            return super().get_property(name, atoms, allow_calculation)
        if atoms is not None or name not in self.results:
            self.calculate(atoms, [name])
        return self.results[name]

    def get_potential_energy(self, atoms=None):
        return self.get_property("energy", atoms)

    def get_forces(self, atoms=None):
        return self.get_property("forces", atoms)

    def get_stress(self, atoms=None):
        return self.get_property("stress", atoms)
