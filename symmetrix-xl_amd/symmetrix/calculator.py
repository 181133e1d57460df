"""ASE-style ``Symmetrix`` calculator on the MI355X evaluator.

Caller contract of the reference calculator (symmetrix/source/symmetrix/
calculator.py), kept here:

* ``calculate`` (:3934-4021) runs one prepared-graph evaluation per call and
  returns ``energy``/``free_energy`` (FP64 sum of the node energies),
  ``energies``, ``forces`` (FP64 atom forces) and ``stress`` (Voigt
  6-vector of sigma = -(1/V) sum_e f_e xyz_e^T) (:3821-3894).
* Graph cache (``_cached_neighbor_geometry``, :2838-3093): the graph is built
  at cutoff + skin and reused while it stays valid.  Fully periodic cells
  keep a fractional topology: the positions split into an affine part (the
  topology's fractional positions times the current cell) and a non-affine
  rest, and the topology stays valid while
  ``||cell^-1 topology_cell||_2 (cutoff + 2 max|non-affine|) <= cutoff +
  skin`` (:2858-2887); a changed cell then only updates the evaluator's cell
  (``_update_factorized_cell``).  Other cells reuse the graph while no atom
  has moved more than skin/2 (minimum image along the periodic axes) and
  the cell is unchanged (:2888-2899).
* Neighbour backend (:83-84, 165-173, 2931-2979): the device builder
  (``_prepare_periodic_factorized_graph``) for fully periodic systems of at
  least 512 atoms, else a host list (``symmetrix.neighbors``, the ``"ijS"``
  list the reference takes from matscipy/ASE).  ``SYMMETRIX_NEIGHBOR_BACKEND``
  = ``automatic`` | ``host`` | ``kokkos`` pins it as in the reference.
* Host graphs go through ``_prepare_factorized_graph`` and one of the
  evaluator's geometry forms (:3224-3300): integer shifts under the tiled
  (fixed-workspace) plan, fractional positions and edge vectors for fully
  periodic cells, Cartesian reference positions and edge vectors otherwise;
  then ``_compute_prepared_factorized_positions``.
* ``execution_profile`` ("capacity" default, or "speed") and
  ``allow_fixed_workspace`` are passed to the evaluator's plan request
  (:1165-1190); their checks follow :827-888.

ASE is optional: with it installed the class is an ``ase.calculators.
calculator.Calculator``; without it ``calculate`` takes any object with
``get_atomic_numbers``, ``get_positions``, ``get_cell`` and ``pbc`` (or a dict
with ``numbers``, ``positions``, ``cell`` and optionally ``pbc``).
"""

from __future__ import annotations

import logging
import os
from dataclasses import dataclass

import numpy as np

from .mace_kokkos import MACEKokkosFloat
from .mace_nonlinear import MACENonlinearKokkosFloat, is_nonlinear_model
from .neighbors import neighbor_list_ijS

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


AUTOMATIC_DEVICE_NEIGHBOR_MIN_ATOMS = 512
NEIGHBOR_BACKENDS = ("automatic", "host", "kokkos")
EXECUTION_PROFILES = ("capacity", "speed")
# the fixed-workspace (tiled) plans of two- and one-interaction models
TILED_PLANS = ("mh0-dual-layer-tiled-v1", "mh0-single-layer-tiled-v1")
DEBUG_EXECUTION_PLANS = frozenset(("mh0-direct-speed", "mh0-direct-capacity-retained") + TILED_PLANS)


def full_3x3_to_voigt_6_stress(s):
    """ASE's Voigt order: xx, yy, zz, yz, xz, xy."""
    s = np.asarray(s)
    return np.array([s[0, 0], s[1, 1], s[2, 2], 0.5 * (s[1, 2] + s[2, 1]), 0.5 * (s[0, 2] + s[2, 0]),
                     0.5 * (s[0, 1] + s[1, 0])])


def _system_arrays(atoms):
    if isinstance(atoms, dict):
        numbers = np.asarray(atoms["numbers"])
        positions = np.asarray(atoms["positions"], dtype=float)
        cell = np.asarray(atoms.get("cell", np.zeros((3, 3))), dtype=float).reshape(3, 3)
        pbc = np.asarray(atoms.get("pbc", [True, True, True]), dtype=bool).reshape(3)
    else:
        numbers = np.asarray(atoms.get_atomic_numbers())
        positions = np.asarray(atoms.get_positions(), dtype=float)
        cell = np.asarray(atoms.get_cell(), dtype=float).reshape(3, 3)
        pbc = np.asarray(atoms.pbc, dtype=bool).reshape(3)
    return numbers, positions, cell, pbc


def neighbor_backend_request():
    request = os.environ.get("SYMMETRIX_NEIGHBOR_BACKEND", "automatic").strip().lower()
    if request not in NEIGHBOR_BACKENDS:
        raise ValueError("SYMMETRIX_NEIGHBOR_BACKEND must be one of %s; got %r"
                         % (", ".join(sorted(NEIGHBOR_BACKENDS)), request))
    return request


def use_device_neighbor_graph(request, eligible, num_atoms):
    """calculator.py:165-173 on a GPU evaluator."""
    if not eligible or request == "host":
        return False
    if request == "kokkos":
        return True
    return num_atoms >= AUTOMATIC_DEVICE_NEIGHBOR_MIN_ATOMS


def minimum_image(displacements, cell, pbc, inverse_cell=None):
    """Displacements wrapped to the minimum image along the periodic axes."""
    if not np.any(pbc):
        return displacements
    if inverse_cell is None:
        f = np.linalg.solve(cell.T, displacements.T).T
    else:
        f = displacements @ inverse_cell
    if np.all(pbc):
        f -= np.rint(f)
    else:
        f[:, pbc] -= np.rint(f[:, pbc])
    return f @ cell


def _max_norm(vectors):
    """Largest row norm of an (N, 3) array (0 for none)."""
    if len(vectors) == 0:
        return 0.0
    return float(np.sqrt(np.max(np.einsum("ij,ij->i", vectors, vectors))))


@dataclass
class _NeighborCache:
    numbers: np.ndarray
    pbc: np.ndarray
    topology_cell: np.ndarray
    topology_positions: np.ndarray
    topology_fractional: np.ndarray  # [N,3] when fully periodic, else empty
    cell: np.ndarray
    generation: int                  # evaluator graph token
    device: bool
    num_edges: int
    receivers: np.ndarray
    sources: np.ndarray
    shifts: np.ndarray
    shift_cart: np.ndarray = None    # shifts @ shift_cell (MH-1 host geometry)
    shift_cell: np.ndarray = None


class Symmetrix(_Base):
    """MACE energies, forces and stress on one MI355X (FP32, direct
    streamed edges)."""

    implemented_properties = ["energy", "free_energy", "energies", "forces", "stress"]
    _nonlinear = False  # an MH-1 (MACE_Nonlinear) evaluator
    # vacuum permittivity in e / (V A) (calculator.py:729)
    _macefield_eps0 = 8.8541878128e-12 / 1.602176634e-19 / 1e10

    def __init__(self, model_file, dtype="float32", use_kokkos=True, streamed_edges="direct",
                 execution_profile="capacity", allow_fixed_workspace=False, neighbor_skin=0.5, head=None,
                 _debug_execution_plan=None, electric_field=None, **kwargs):
        super().__init__(**kwargs)
        if dtype not in ("float32", np.float32):
            raise ValueError("the MI355X evaluator implements dtype='float32'")
        if not use_kokkos:
            raise ValueError("the MI355X evaluator is the device (use_kokkos=True) path")
        if streamed_edges not in ("direct", "factorized", "direct_streamed"):
            raise ValueError("the MI355X evaluator implements streamed_edges='direct'")
        if execution_profile not in EXECUTION_PROFILES:
            raise ValueError("execution_profile must be 'capacity' or 'speed'")
        if streamed_edges in ("factorized", "direct_streamed") and execution_profile == "capacity":
            execution_profile = "speed"  # the aliases keep the throughput behaviour (python_api.md:40-45)
        if not isinstance(allow_fixed_workspace, bool):
            raise ValueError("allow_fixed_workspace must be a bool.")
        if allow_fixed_workspace and execution_profile != "capacity":
            raise ValueError("allow_fixed_workspace=True requires execution_profile='capacity'.")
        if not (neighbor_skin >= 0.0):
            raise ValueError("neighbor_skin must be non-negative")
        # the private plan pin (calculator.py:831-851): a known id, with the
        # profile it belongs to
        if _debug_execution_plan is not None:
            if _debug_execution_plan not in DEBUG_EXECUTION_PLANS:
                raise ValueError("_debug_execution_plan must be one of %s or None."
                                 % sorted(DEBUG_EXECUTION_PLANS))
            required = "speed" if _debug_execution_plan == "mh0-direct-speed" else "capacity"
            if execution_profile != required:
                raise ValueError("%s requires execution_profile=%r." % (_debug_execution_plan, required))
        # MH-1 files dispatch on model_type (calculator.py:1093-1126; test_mh1.py:2678)
        self._nonlinear = is_nonlinear_model(model_file)
        if self._nonlinear:
            if allow_fixed_workspace or _debug_execution_plan is not None:
                raise ValueError("MACE_Nonlinear models have no fixed-workspace or debug execution plans.")
            self.evaluator = MACENonlinearKokkosFloat(model_file, head or "")
            self.streamed_edges = "generic"
        else:
            self.evaluator = MACEKokkosFloat(model_file, head or "")
            self.streamed_edges = "direct"
        self.execution_profile = execution_profile
        self.allow_fixed_workspace = allow_fixed_workspace
        if not self._nonlinear:
            self.evaluator._set_allow_fixed_workspace(allow_fixed_workspace)
            self.evaluator._set_execution_plan_request("direct", execution_profile, _debug_execution_plan or "")
        self.cutoff = float(self.evaluator.r_cut)
        self.neighbor_skin = float(neighbor_skin)
        self._types = {z: i for i, z in enumerate(self.evaluator.atomic_numbers)}
        self._neighbor_cache = None
        self.neighbor_cache_build_count = 0
        self.neighbor_cache_reuse_count = 0
        self.neighbor_cache_cell_update_count = 0
        self.neighbor_graph_backend = None
        self.results = {}
        # MACEField models (calculator.py:971-976, 1247-1249): the graph's
        # electric field, and the polarization -dE/dE / V among the results
        self._electric_field = electric_field
        if getattr(self.evaluator, "has_field_coupling", False):
            self.implemented_properties = list(self.implemented_properties) + ["polarization", "becs",
                                                                               "polarizability"]

    @property
    def electric_field(self):
        return self._electric_field

    @electric_field.setter
    def electric_field(self, value):
        self._electric_field = value

    def _resolve_electric_field(self, atoms):
        """calculator.py:2782-2805: the calculator's field, else the atoms'
        info["electric_field"] / info["REF_electric_field"], else zero; one
        field for the graph, shape (3,) or (1, 3)."""
        info = atoms.get("info", {}) if isinstance(atoms, dict) else getattr(atoms, "info", {})
        if self._electric_field is not None:
            field = self._electric_field
        elif "electric_field" in info:
            field = info["electric_field"]
        elif "REF_electric_field" in info:
            field = info["REF_electric_field"]
        else:
            field = np.zeros(3)
        field = np.asarray(field, dtype=float)
        if field.shape in ((3,), (1, 3)):
            return field.reshape(3)
        if field.ndim == 2 and field.shape[1] == 3:
            raise ValueError("MACEField ASE electric_field must be a graph-level electric_field with shape (3,) or "
                             "(1, 3); per-atom fields are not supported.")
        raise ValueError("electric_field must have shape (3,) or (1, 3).")

    @property
    def neighbor_graph_rebuilds(self):
        return self.neighbor_cache_build_count

    @property
    def execution_plan(self):
        if self._nonlinear:
            return {"selected_id": "mh1-generic", "streamed_edges": "generic"}
        return self.evaluator.execution_plan_report

    # -------------------------------------------------------------- graph
    def _node_types(self, numbers):
        try:
            return np.asarray([self._types[int(z)] for z in numbers], dtype=np.int32)
        except KeyError as exc:
            raise ValueError("atomic number %s is not in the model" % exc.args[0]) from None

    def _reuse(self, numbers, positions, cell, pbc):
        """'reuse', 'cell' (topology valid under a new cell) or None."""
        c = self._neighbor_cache
        if c is None or len(numbers) != len(c.numbers) or not np.array_equal(numbers, c.numbers):
            return None
        if not np.array_equal(pbc, c.pbc):
            return None
        cell_changed = not np.array_equal(cell, c.cell)
        if np.all(pbc):
            try:
                inverse = np.linalg.inv(cell)
                non_affine = positions - c.topology_fractional @ cell
                non_affine = minimum_image(non_affine, cell, pbc, inverse)
                # the topology's own cell: no deformation
                contraction = 1.0 if np.array_equal(cell, c.topology_cell) else float(
                    np.linalg.norm(np.linalg.solve(cell, c.topology_cell), ord=2))
            except np.linalg.LinAlgError:
                return None
            max_non_affine = _max_norm(non_affine)
            if contraction * (self.cutoff + 2.0 * max_non_affine) > self.cutoff + self.neighbor_skin:
                return None
            return "cell" if cell_changed else "reuse"
        if cell_changed:
            return None
        disp = minimum_image(positions - c.topology_positions, cell, pbc)
        if _max_norm(disp) > 0.5 * self.neighbor_skin:
            return None
        return "reuse"

    def _fixed_workspace_plan_selected(self):
        return (not self._nonlinear) and self.evaluator.execution_plan_report.get("selected_id") in TILED_PLANS

    def _prepare(self, numbers, positions, cell, pbc):
        if not np.isfinite(positions).all():
            raise ValueError("positions must be finite")
        types = self._node_types(numbers)
        n = len(types)
        periodic = bool(np.all(pbc))
        if np.any(pbc) and not abs(np.linalg.det(cell)) > 0.0:
            raise ValueError("a periodic cell must be invertible")
        inv = np.linalg.inv(cell) if np.any(pbc) else np.zeros((3, 3))
        frac = positions @ inv if periodic else np.zeros((0, 3))
        request = neighbor_backend_request()
        # MH-1 takes its graph in host memory (mace_nonlinear.hpp:44-51)
        device = use_device_neighbor_graph(request, periodic, n) and not self._nonlinear
        if request == "kokkos" and not periodic:
            raise RuntimeError("SYMMETRIX_NEIGHBOR_BACKEND=kokkos requires a fully periodic cell")
        ev = self.evaluator
        reach = self.cutoff + self.neighbor_skin
        if device:
            g = ev._prepare_periodic_factorized_graph(types, positions.reshape(-1), cell.reshape(-1),
                                                      inv.reshape(-1), reach)
            gen, num_edges = g["generation"], g["num_edges"]
            receivers = sources = np.zeros(0, np.int32)
            shifts = np.zeros((0, 3), np.int32)
            self.neighbor_graph_backend = "device"
        elif self._nonlinear:
            receivers, sources, shifts = neighbor_list_ijS(positions, cell, pbc, reach)
            gen, num_edges = 0, len(sources)
            self.neighbor_graph_backend = "host"
        else:
            receivers, sources, shifts = neighbor_list_ijS(positions, cell, pbc, reach)
            num_neigh = np.bincount(receivers, minlength=n).astype(np.int32)
            gen = ev._prepare_factorized_graph(n, types, num_neigh, sources, types[sources])
            num_edges = len(sources)
            pbc_i = pbc.astype(np.int32)
            if self._fixed_workspace_plan_selected():
                ev._prepare_factorized_shift_geometry(gen, positions, shifts, cell, inv, pbc_i)
            elif periodic:
                frac_xyz = frac[sources] - frac[receivers] + shifts
                ev._prepare_factorized_fractional_geometry(gen, frac, frac_xyz, cell, inv, pbc_i)
            else:
                ref_xyz = positions[sources] - positions[receivers] + shifts @ cell
                ev._prepare_factorized_geometry(gen, positions, ref_xyz, cell, inv, pbc_i)
            self.neighbor_graph_backend = "host"
        self._neighbor_cache = _NeighborCache(numbers.copy(), pbc.copy(), cell.copy(), positions.copy(),
                                              frac.copy(), cell.copy(), gen, device, num_edges, receivers,
                                              sources, shifts)
        self.neighbor_cache_build_count += 1
        return self._neighbor_cache

    def _graph(self, numbers, positions, cell, pbc):
        state = self._reuse(numbers, positions, cell, pbc)
        if state is None:
            return self._prepare(numbers, positions, cell, pbc)
        c = self._neighbor_cache
        if state == "cell":
            if not self._nonlinear:
                self.evaluator._update_factorized_cell(c.generation, cell.reshape(-1),
                                                       np.linalg.inv(cell).reshape(-1))
            c.cell = cell.copy()
            self.neighbor_cache_cell_update_count += 1
        self.neighbor_cache_reuse_count += 1
        return c

    # ---------------------------------------------------------- calculate
    def calculate(self, atoms=None, properties=None, system_changes=_all_changes):
        if properties is None:
            # the response properties run only when asked for
            properties = [p for p in self.implemented_properties if p not in ("becs", "polarizability")]
        if HAVE_ASE:
            super().calculate(atoms, properties, system_changes)
            atoms = self.atoms
        elif atoms is not None:
            self.atoms = atoms
        else:
            atoms = self.atoms
        numbers, positions, cell, pbc = _system_arrays(atoms)
        field = self._resolve_electric_field(atoms) if getattr(self.evaluator, "has_field_coupling", False) else None
        cache = self._graph(numbers, positions, cell, pbc)
        ev = self.evaluator
        volume = None
        if "stress" in properties:
            volume = abs(float(np.linalg.det(cell)))
            if not volume > 0.0:
                raise ValueError("stress needs a cell of non-zero volume")
        if self._nonlinear:
            return self._calculate_nonlinear(numbers, positions, cell, cache, volume)
        if field is not None:
            ev._set_electric_field(field)
        # the reference's sequence (positions call, node energies, atom
        # forces, stress; calculator.py:3821-3894) in one device round trip
        node_energies, forces, sigma = ev._compute_prepared_factorized_positions_results(
            cache.generation, positions.reshape(-1), volume)
        energy = float(np.sum(node_energies, dtype=np.float64))
        self.results = {"energy": energy, "free_energy": energy, "energies": node_energies}
        self.results["forces"] = forces
        if sigma is not None:
            self.results["stress"] = full_3x3_to_voigt_6_stress(sigma)
        if field is not None:
            # calculator.py:3672-3678: P = -dE/dE / V
            volume = abs(float(np.linalg.det(cell)))
            if not volume > 0.0:
                raise ValueError("polarization needs a cell of non-zero volume")
            self.results["polarization"] = -np.asarray(ev.electric_field_adj, dtype=float) / volume
            # calculator.py:3783-3817: polarizability -d2E/dE2 / (V eps0), Born
            # charges dF_i/dE from the device bins (one response for both)
            want_becs = "becs" in properties
            if want_becs or "polarizability" in properties:
                ev._compute_prepared_factorized_field_response(cache.generation, field, want_becs,
                                                               scatter_bec_bins=want_becs)
                if "polarizability" in properties:
                    pol = -np.asarray(ev.electric_field_hessian, dtype=float).reshape(3, 3)
                    self.results["polarizability"] = np.array((pol / volume / self._macefield_eps0).reshape(9))
                if want_becs:
                    self.results["becs"] = np.array(ev.electric_field_bec_bins, dtype=float).reshape(len(numbers), 9)
        return self.results

    def _calculate_nonlinear(self, numbers, positions, cell, cache, volume):
        """MH-1: the cached skin graph's edges inside the cutoff
        (calculator.py:3087-3093), one compute_node_energies_forces call,
        forces and stress reduced in FP64 (calculator.py:3821-3894)."""
        recv, src = cache.receivers, cache.sources
        # Cartesian cell shifts of the skin graph, formed once per cell
        if cache.shift_cell is None or not np.array_equal(cache.shift_cell, cell):
            cache.shift_cart = cache.shifts.astype(np.float64) @ cell
            cache.shift_cell = cell.copy()
        xyz = np.take(positions, src, axis=0)
        xyz -= np.take(positions, recv, axis=0)
        xyz += cache.shift_cart
        r2 = np.einsum("ij,ij->i", xyz, xyz)
        active = np.flatnonzero(r2 < self.cutoff * self.cutoff)
        recv, src = recv[active], src[active]
        xyz = np.take(xyz, active, axis=0)
        r = np.sqrt(r2[active])
        n = len(numbers)
        types = self._node_types(numbers)
        num_neigh = np.bincount(recv, minlength=n).astype(np.int32)
        ev = self.evaluator
        ev.compute_node_energies_forces(n, types, num_neigh, src, types[src], xyz.reshape(-1), r)
        node_energies = ev.node_energies
        nf = ev.node_forces.reshape(-1, 3)
        forces = np.empty((n, 3))
        for c in range(3):
            forces[:, c] = (np.bincount(src, weights=nf[:, c], minlength=n)
                            - np.bincount(recv, weights=nf[:, c], minlength=n))
        energy = float(np.sum(node_energies, dtype=np.float64))
        self.results = {"energy": energy, "free_energy": energy, "energies": node_energies, "forces": forces}
        if volume is not None:
            sigma = -(nf.T @ xyz) / volume
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
