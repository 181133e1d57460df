"""``MACEKokkosFloat``: the reference's FP32 evaluator class, backed by the
MI355X library.

Method names, argument meanings and error behaviour follow the reference's
pybind class (symmetrix/source/cpp/mace_kokkos.cpp): ``_prepare_factorized_graph``
(:1561), ``_prepare_periodic_factorized_graph`` (:1580, returns
``{"generation", "num_edges"}``), ``_prepare_factorized_geometry``,
``_prepare_factorized_shift_geometry`` and
``_prepare_factorized_fractional_geometry`` (:1608-1672),
``_update_factorized_cell``, ``_compute_prepared_factorized`` (:1817),
``_compute_prepared_factorized_positions`` (:1828),
``compute_node_energies_forces`` (:2169), ``_reduce_atom_forces`` (:2103),
``_reduce_stress`` (:2134), ``prepare_active_types`` (:2076), the plan
request ``_set_execution_plan_request`` / ``_set_allow_fixed_workspace`` /
``execution_plan_report`` (:266-297, 444-447), the counters
``factorized_last_graph_prepare_ms`` / ``factorized_last_evaluation_ms``
(:1045-1053) and the ``node_energies``/``node_forces``/``r_cut``/
``atomic_numbers`` attributes.  Bad inputs and stale generations raise
ValueError, device failures RuntimeError.
"""

from __future__ import annotations

import ctypes
import json

import numpy as np

from . import _native
from ._native import check, f64, i32, lib, ptr

_HIP = None


def _hip():
    """the HIP runtime, for host copies of device rows the library hands out"""
    global _HIP
    if _HIP is None:
        _HIP = ctypes.CDLL("libamdhip64.so")
        _HIP.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    return _HIP


class MACEKokkosFloat:
    """FP32 MACE evaluator on one MI355X (``streamed_edges="direct"``)."""

    precision = "float32"

    def __init__(self, filename, head=""):
        h = ctypes.c_void_p()
        check(lib.smx_evaluator_create(str(filename).encode(), (head or "").encode(), ctypes.byref(h)))
        self._h = h
        info = _native.SmxModelInfo()
        info.struct_size = ctypes.sizeof(info)
        check(lib.smx_evaluator_info(self._h, ctypes.byref(info)))
        self.num_elements = info.num_elements
        self.num_channels = info.num_channels
        self.l_max = info.l_max
        self.L_max = info.L_max
        self.num_interactions = info.num_interactions
        self.r_cut = info.r_cut
        z = np.zeros(self.num_elements, dtype=np.int32)
        check(lib.smx_evaluator_atomic_numbers(self._h, ptr(z), len(z)))
        self._atomic_numbers = z
        self.selected_head = self._head(-1)
        self.available_heads = []
        while True:
            name = self._head(len(self.available_heads))
            if name is None:
                break
            self.available_heads.append(name)
        self._num_nodes = 0
        self._num_feature_nodes = 0
        self._num_edges = 0
        self._generation = 0

    def _head(self, index):
        name = ctypes.c_char_p()
        check(lib.smx_prediction_head(self._h, index, ctypes.byref(name)))
        return None if name.value is None else name.value.decode()

    def close(self):
        if getattr(self, "_h", None):
            lib.smx_evaluator_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    # ------------------------------------------------------------ attributes
    @property
    def atomic_numbers(self):
        return [int(v) for v in self._atomic_numbers]

    @property
    def atomic_energies(self):
        out = np.zeros(self.num_elements)
        check(lib.smx_evaluator_atomic_energies(self._h, ptr(out), out.size))
        return [float(v) for v in out]

    @property
    def active_atomic_numbers(self):
        n = ctypes.c_int32()
        check(lib.smx_active_atomic_numbers(self._h, None, 0, ctypes.byref(n)))
        out = np.zeros(n.value, dtype=np.int32)
        check(lib.smx_active_atomic_numbers(self._h, ptr(out), out.size, None))
        return [int(v) for v in out]

    @property
    def streamed_edges_mode(self):
        return "direct"

    def set_streamed_edges(self, mode):
        check(lib.smx_set_streamed_edges(self._h, str(mode).encode()))

    def set_execution_plan_request(self, profile="auto", tile_receivers=0):
        """Shorthand with the tile size: ``"speed"`` (the speed profile),
        ``"capacity"`` (the model's tiled plan pinned, at most
        ``tile_receivers`` receivers per tile) or ``"auto"`` (the capacity
        profile with fixed workspaces allowed); applies to graphs prepared
        afterwards."""
        check(lib.smx_set_execution_plan(self._h, str(profile).encode(), int(tile_receivers)))

    def _set_execution_plan_request(self, algorithm, profile, debug_plan=""):
        """The reference's plan request (mace_kokkos.cpp:266-270): algorithm
        "direct", profile "capacity" or "speed", debug_plan "" or a plan id."""
        check(lib.smx_set_execution_plan_request(self._h, str(algorithm).encode(), str(profile).encode(),
                                                 str(debug_plan or "").encode()))

    def _resolve_execution_plan(self):
        """The plan is resolved when a graph is prepared; returns the report."""
        return self.execution_plan_report

    def _set_allow_fixed_workspace(self, allow):
        check(lib.smx_set_allow_fixed_workspace(self._h, 1 if allow else 0))
        self._allow_fixed = bool(allow)

    @property
    def allow_fixed_workspace(self):
        return self.execution_plan_report["allow_fixed_workspace"]

    @property
    def execution_plan_report(self):
        n = ctypes.c_int64()
        check(lib.smx_execution_plan_report(self._h, None, 0, ctypes.byref(n)))
        buf = ctypes.create_string_buffer(int(n.value))
        check(lib.smx_execution_plan_report(self._h, ctypes.addressof(buf), n.value, None))
        return json.loads(buf.value.decode())

    def _counters(self):
        c = _native.SmxEvaluatorCounters()
        c.struct_size = ctypes.sizeof(c)
        check(lib.smx_evaluator_counters(self._h, ctypes.byref(c)))
        return c

    # the prepared graph and the plan request (pybind mace_kokkos.cpp:448-449,
    # 529-562, 897-949)
    @property
    def low_memory(self):
        """the capacity profile is requested (set_low_memory(True) selects it)"""
        return self.execution_plan_report["requested_profile"] == "capacity"

    def _set_low_memory(self, enabled):
        self._set_execution_plan_request("direct", "capacity" if enabled else "speed")

    @property
    def execution_active_receiver_count(self):
        return self._num_nodes

    @property
    def execution_active_feature_node_count(self):
        return self._num_feature_nodes

    @property
    def execution_active_edge_count(self):
        return self._num_edges

    @property
    def factorized_graph_generation(self):
        return self._generation

    @property
    def factorized_prepared_graph_count(self):
        return int(self._counters().graph_prepare_count)

    @property
    def factorized_prepared_evaluation_count(self):
        return int(self._counters().evaluation_count)

    @property
    def factorized_last_graph_prepare_ms(self):
        return self._counters().last_graph_prepare_ms

    @property
    def factorized_last_evaluation_ms(self):
        return self._counters().last_evaluation_ms

    def prepare_active_types(self, node_types, neigh_types=None):
        """Tabulate the radial tables of these model types ahead of the graph
        (mace_kokkos.cpp:223-254: node types, then unseen neighbour types)."""
        types = [int(t) for t in np.asarray(node_types).ravel()]
        if neigh_types is not None:
            types += [int(t) for t in np.asarray(neigh_types).ravel()]
        seen = []
        for t in types:
            if t not in seen:
                seen.append(t)
        arr = i32(seen)
        check(lib.smx_prepare_active_types(self._h, ptr(arr) if arr.size else None, arr.size))

    @property
    def execution_plan(self):
        buf = ctypes.create_string_buffer(256)
        check(lib.smx_execution_plan(self._h, ctypes.addressof(buf), 256))
        return buf.value.decode()

    @property
    def stream(self):
        return lib.smx_evaluator_stream(self._h)

    @property
    def node_energies(self):
        out = np.zeros(self._num_nodes)
        check(lib.smx_node_energies(self._h, ptr(out), out.size))
        return out

    @property
    def node_forces(self):
        out = np.zeros(3 * self._num_edges)
        check(lib.smx_node_forces(self._h, ptr(out), out.size))
        return out

    # ----------------------------------------------------------------- graph
    def _prepare_factorized_graph(self, num_nodes, node_types, num_neigh, neigh_indices, neigh_types):
        node_types, num_neigh = i32(node_types), i32(num_neigh)
        neigh_indices, neigh_types = i32(neigh_indices), i32(neigh_types)
        if len(node_types) != num_nodes or len(num_neigh) != num_nodes:
            raise ValueError("node arrays do not match num_nodes")
        if len(neigh_types) != len(neigh_indices):
            raise ValueError("neighbour arrays have different lengths")
        gen = ctypes.c_uint64()
        check(lib.smx_prepare_factorized_graph(self._h, int(num_nodes), ptr(node_types), ptr(num_neigh),
                                               len(neigh_indices), ptr(neigh_indices), ptr(neigh_types),
                                               ctypes.byref(gen)))
        self._num_nodes = self._num_feature_nodes = int(num_nodes)
        self._num_edges = len(neigh_indices)
        self._generation = int(gen.value)
        return self._generation

    # ------------------------------------ feature graphs and split phases
    def _prepare_factorized_feature_graph(self, num_receivers, num_feature_nodes, receiver_feature_indices,
                                          node_types, feature_types, num_neigh, neigh_indices, neigh_types):
        """prepare_factorized_graph with feature nodes (mace_kokkos.hpp:378-386):
        one domain's receivers, its receivers' and ghost atoms as feature
        nodes, and edges leaving any feature node (feature indices)."""
        rf, node_types, feature_types = i32(receiver_feature_indices), i32(node_types), i32(feature_types)
        num_neigh, neigh_indices, neigh_types = i32(num_neigh), i32(neigh_indices), i32(neigh_types)
        if rf.size != num_receivers or node_types.size != num_receivers or num_neigh.size != num_receivers:
            raise ValueError("receiver arrays do not match num_receivers")
        if feature_types.size != num_feature_nodes:
            raise ValueError("feature_types does not match num_feature_nodes")
        if neigh_types.size != neigh_indices.size:
            raise ValueError("neighbour arrays have different lengths")
        gen = ctypes.c_uint64()
        check(lib.smx_prepare_factorized_feature_graph(self._h, int(num_receivers), int(num_feature_nodes), ptr(rf),
                                                       ptr(node_types), ptr(feature_types), ptr(num_neigh),
                                                       neigh_indices.size, ptr(neigh_indices), ptr(neigh_types),
                                                       ctypes.byref(gen)))
        self._num_nodes = int(num_receivers)
        self._num_feature_nodes = int(num_feature_nodes)
        self._num_edges = neigh_indices.size
        self._generation = int(gen.value)
        return self._generation

    def _edge_vectors(self, xyz, r):
        xyz, r = f64(xyz), f64(r)
        if xyz.size != 3 * self._num_edges or r.size != self._num_edges:
            raise ValueError("xyz and r do not match the prepared graph")
        return xyz, r

    def _compute_factorized_single_layer_distributed_evaluation(self, execution_graph_generation, xyz, r):
        xyz, r = self._edge_vectors(xyz, r)
        check(lib.smx_compute_factorized_single_layer_distributed_evaluation(
            self._h, int(execution_graph_generation), self._num_nodes, self._num_feature_nodes, ptr(xyz), ptr(r), 0))

    def _begin_factorized_distributed_evaluation(self, execution_graph_generation, xyz, r):
        xyz, r = self._edge_vectors(xyz, r)
        check(lib.smx_begin_factorized_distributed_evaluation(
            self._h, int(execution_graph_generation), self._num_nodes, self._num_feature_nodes, ptr(xyz), ptr(r), 0))

    def _feature_positions(self, positions):
        positions = f64(positions)
        if positions.size != 3 * self._num_feature_nodes:
            raise ValueError("positions must hold three coordinates per feature node")
        return positions

    def _begin_factorized_distributed_positions_evaluation(self, execution_graph_generation, positions):
        p = self._feature_positions(positions)
        check(lib.smx_begin_factorized_distributed_positions_evaluation(
            self._h, int(execution_graph_generation), self._num_nodes, self._num_feature_nodes, ptr(p), 0))

    def _compute_factorized_single_layer_distributed_positions_evaluation(self, execution_graph_generation,
                                                                          positions):
        p = self._feature_positions(positions)
        check(lib.smx_compute_factorized_single_layer_distributed_positions_evaluation(
            self._h, int(execution_graph_generation), self._num_nodes, self._num_feature_nodes, ptr(p), 0))

    def _distributed_rows(self, which):
        """host copy of the rows a phase leaves for the exchange: 0, the
        receivers' H1; 1, the feature nodes' H1 adjoint"""
        dev, rows, width = ctypes.c_void_p(), ctypes.c_int64(), ctypes.c_int64()
        check(lib.smx_distributed_exchange(self._h, int(which), ctypes.byref(dev), ctypes.byref(rows),
                                           ctypes.byref(width)))
        out = np.zeros((rows.value, width.value), np.float32)
        if out.size and _hip().hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), dev, ctypes.c_size_t(out.nbytes), 2):
            raise RuntimeError("hipMemcpy of the exchange rows failed")
        return out

    def _distributed_h1(self):
        return self._distributed_rows(0)

    def _distributed_h1_adjoint(self):
        return self._distributed_rows(1)

    def _exchange_rows(self, which, rows, name):
        """rows as a float32 [num_feature_nodes, row_floats] array, the
        phase's row width checked (the library reads whole rows)"""
        width = ctypes.c_int64()
        check(lib.smx_distributed_exchange(self._h, int(which), None, None, ctypes.byref(width)))
        h = np.ascontiguousarray(rows, dtype=np.float32)
        if h.shape != (self._num_feature_nodes, width.value):
            raise ValueError("%s must have shape (%d, %d)" % (name, self._num_feature_nodes, width.value))
        return h

    def _continue_factorized_distributed_evaluation(self, communicated_h1):
        h = self._exchange_rows(0, communicated_h1, "communicated H1")
        check(lib.smx_continue_factorized_distributed_evaluation(self._h, ptr(h), h.shape[0], 0))

    def _finish_factorized_distributed_evaluation(self, h1_adjoint=None):
        if h1_adjoint is None:
            check(lib.smx_finish_factorized_distributed_evaluation(self._h, None, 0, 0))
            return
        h = self._exchange_rows(1, h1_adjoint, "the H1 adjoint")
        check(lib.smx_finish_factorized_distributed_evaluation(self._h, ptr(h), h.shape[0], 0))

    def _prepare_periodic_factorized_graph(self, node_types, positions, cell, inverse_cell, neighbor_cutoff):
        node_types = i32(node_types)
        positions = f64(positions)
        if positions.size != 3 * node_types.size:
            raise ValueError("positions must hold three coordinates per node")
        cell, inverse_cell = f64(cell), f64(inverse_cell)
        if cell.size != 9 or inverse_cell.size != 9:
            raise ValueError("cell and inverse_cell must have nine entries")
        gen = ctypes.c_uint64()
        ne = ctypes.c_int64()
        check(lib.smx_prepare_periodic_factorized_graph(self._h, node_types.size, ptr(node_types), ptr(positions),
                                                        ptr(cell), ptr(inverse_cell), float(neighbor_cutoff),
                                                        ctypes.byref(gen), ctypes.byref(ne)))
        self._num_nodes = self._num_feature_nodes = node_types.size
        self._num_edges = int(ne.value)
        self._generation = int(gen.value)
        return {"generation": self._generation, "num_edges": int(ne.value)}

    def _geometry_arrays(self, positions, edges, cell, inverse_cell, pbc, edge_dtype):
        positions, cell, inverse_cell = f64(positions), f64(cell), f64(inverse_cell)
        edges = np.ascontiguousarray(np.asarray(edges, dtype=edge_dtype).reshape(-1))
        pbc = i32(np.asarray(pbc).astype(np.int32))
        if cell.size != 9 or inverse_cell.size != 9 or pbc.size != 3:
            raise ValueError("Execution R1 prepared geometry extents are inconsistent.")
        return positions, edges, cell, inverse_cell, pbc

    def _prepare_factorized_geometry(self, execution_graph_generation, reference_positions, reference_xyz, cell,
                                     inverse_cell, pbc):
        p, e, c, ic, b = self._geometry_arrays(reference_positions, reference_xyz, cell, inverse_cell, pbc,
                                               np.float64)
        check(lib.smx_prepare_factorized_geometry(self._h, int(execution_graph_generation), ptr(p), p.size, ptr(e),
                                                  e.size, ptr(c), ptr(ic), ptr(b)))

    def _prepare_factorized_shift_geometry(self, execution_graph_generation, reference_positions, shifts, cell,
                                           inverse_cell, pbc):
        p, e, c, ic, b = self._geometry_arrays(reference_positions, shifts, cell, inverse_cell, pbc, np.int32)
        check(lib.smx_prepare_factorized_shift_geometry(self._h, int(execution_graph_generation), ptr(p), p.size,
                                                        ptr(e), e.size, ptr(c), ptr(ic), ptr(b)))

    def _prepare_factorized_fractional_geometry(self, execution_graph_generation, fractional_positions,
                                                fractional_xyz, cell, inverse_cell, pbc):
        p, e, c, ic, b = self._geometry_arrays(fractional_positions, fractional_xyz, cell, inverse_cell, pbc,
                                               np.float64)
        check(lib.smx_prepare_factorized_fractional_geometry(self._h, int(execution_graph_generation), ptr(p),
                                                             p.size, ptr(e), e.size, ptr(c), ptr(ic), ptr(b)))

    def _update_factorized_cell(self, execution_graph_generation, cell, inverse_cell):
        cell, inverse_cell = f64(cell), f64(inverse_cell)
        check(lib.smx_update_factorized_cell(self._h, int(execution_graph_generation), ptr(cell),
                                             ptr(inverse_cell)))

    # ------------------------------------------------------------- evaluate
    def _compute_prepared_factorized(self, execution_graph_generation, xyz, r):
        xyz, r = f64(xyz), f64(r)
        if xyz.size != 3 * self._num_edges or r.size != self._num_edges:
            raise ValueError("xyz and r do not match the prepared graph")
        check(lib.smx_compute_prepared_factorized(self._h, int(execution_graph_generation), ptr(xyz), ptr(r)))

    def _compute_prepared_factorized_positions(self, execution_graph_generation, positions):
        positions = f64(positions)
        if positions.size != 3 * self._num_nodes:
            raise ValueError("positions do not match the prepared graph")
        check(lib.smx_compute_prepared_factorized_positions(self._h, int(execution_graph_generation),
                                                            ptr(positions)))

    def _compute_prepared_factorized_positions_results(self, execution_graph_generation, positions, volume=None):
        """The calculator's call in one: host positions in; node energies,
        atom forces and (volume given) the 3x3 stress out, behind one wait
        for the device (the reference's calculator makes these calls in
        turn, calculator.py:3821-3894)."""
        positions = f64(positions)
        if positions.size != 3 * self._num_nodes:
            raise ValueError("positions do not match the prepared graph")
        energies = np.zeros(self._num_nodes)
        forces = np.zeros((self._num_feature_nodes, 3))
        stress = None if volume is None else np.zeros((3, 3))
        check(lib.smx_compute_prepared_factorized_positions_results(
            self._h, int(execution_graph_generation), ptr(positions), 0.0 if volume is None else float(volume),
            ptr(energies), ptr(forces), None if stress is None else ptr(stress)))
        return energies, forces, stress

    # -------------------------------------------------------- MACEField
    @property
    def has_field_coupling(self):
        out = ctypes.c_int32()
        check(lib.smx_has_field_coupling(self._h, ctypes.byref(out)))
        return bool(out.value)

    def _field(self, electric_field):
        field = f64(electric_field)
        if field.size not in (3, 3 * self._num_nodes):
            raise ValueError("MACEField electric_field must have shape (3,) or (num_nodes, 3).")
        return field

    def _compute_prepared_factorized_positions_field(self, execution_graph_generation, positions, electric_field):
        positions, field = f64(positions), self._field(electric_field)
        if positions.size != 3 * self._num_nodes:
            raise ValueError("positions do not match the prepared graph")
        check(lib.smx_compute_prepared_factorized_positions_field(
            self._h, int(execution_graph_generation), ptr(positions), ptr(field), field.size))

    def _compute_prepared_factorized_field(self, execution_graph_generation, xyz, r, electric_field):
        xyz, r, field = f64(xyz), f64(r), self._field(electric_field)
        if xyz.size != 3 * self._num_edges or r.size != self._num_edges:
            raise ValueError("xyz and r do not match the prepared graph")
        check(lib.smx_compute_prepared_factorized_field(self._h, int(execution_graph_generation), ptr(xyz), ptr(r),
                                                        ptr(field), field.size))

    def _set_electric_field(self, electric_field=None):
        field = np.zeros(0) if electric_field is None else f64(electric_field)
        check(lib.smx_set_electric_field(self._h, ptr(field), field.size))

    @property
    def electric_field_adj(self):
        n = ctypes.c_int64()
        check(lib.smx_electric_field_adj(self._h, None, 0, ctypes.byref(n)))
        out = np.zeros(n.value)
        check(lib.smx_electric_field_adj(self._h, ptr(out), out.size, None))
        return out

    # MACEField response (pybind mace_kokkos.cpp:1865-1879, 2160-2167,
    # 2226-2349; mace_kokkos_response.tpp)
    _CURRENT_RESPONSE_ERROR = ("MACEField current response requires a completed prepared Execution evaluation for "
                               "the current graph token.")

    def _compute_prepared_factorized_field_response(self, execution_graph_generation, electric_field,
                                                    include_force_derivative, scatter_bec_bins=False):
        """The field Hessian and (include_force_derivative) the directed
        forces' field derivative, or with scatter_bec_bins the Born charge
        bins, of the completed field evaluation of this graph token."""
        field = f64(electric_field)
        if field.size != 3:
            raise ValueError("MACEKokkos::compute_electric_field_hessian requires a graph-level electric field.")
        check(lib.smx_compute_prepared_factorized_field_response(
            self._h, int(execution_graph_generation), ptr(field), field.size, int(bool(include_force_derivative)),
            int(bool(scatter_bec_bins))))

    def _response_values(self, fn):
        n = ctypes.c_int64()
        check(fn(self._h, None, 0, ctypes.byref(n)))
        out = np.zeros(n.value)
        if n.value:
            check(fn(self._h, ptr(out), out.size, None))
        return out

    @property
    def electric_field_hessian(self):
        """[c*3 + s] = d(dE/dE_c)/dE_s of the last response (9 values)."""
        return self._response_values(lib.smx_electric_field_hessian).tolist()

    @property
    def electric_field_force_derivative(self):
        """[s][edge][3] flattened: each edge's directed-force derivative in
        field component s (empty when the last response took none)."""
        return self._response_values(lib.smx_electric_field_force_derivative).tolist()

    @property
    def electric_field_bec_bins(self):
        """Born charge bins [num_nodes][s][3] = dF/dE_s of the last response
        that scattered them (shape (0, 3, 3) otherwise)."""
        return self._response_values(lib.smx_electric_field_bec_bins).reshape(-1, 3, 3)

    def _host_graph_response(self, num_nodes, node_types, num_neigh, neigh_indices, neigh_types, xyz, r,
                             electric_field, forces):
        token = self._prepare_factorized_graph(num_nodes, node_types, num_neigh, neigh_indices, neigh_types)
        self._compute_prepared_factorized_field(token, xyz, r, electric_field)
        self._compute_prepared_factorized_field_response(token, electric_field, forces)

    def compute_electric_field_hessian(self, num_nodes, node_types, num_neigh, neigh_indices, neigh_types, xyz, r,
                                       electric_field):
        """Evaluate the host graph in the field, then its field Hessian
        (mace_kokkos_response.tpp:2394-2408)."""
        if not self.has_field_coupling:
            raise ValueError("MACEKokkos::compute_electric_field_hessian requires field coupling.")
        self._host_graph_response(num_nodes, node_types, num_neigh, neigh_indices, neigh_types, xyz, r,
                                  electric_field, False)

    def compute_electric_field_force_derivative(self, num_nodes, node_types, num_neigh, neigh_indices, neigh_types,
                                                xyz, r, electric_field):
        """Evaluate the host graph in the field, then the Hessian and the
        per-edge force derivative (mace_kokkos_response.tpp:2436-2450)."""
        if not self.has_field_coupling:
            raise ValueError("MACEKokkos::compute_electric_field_hessian requires field coupling.")
        self._host_graph_response(num_nodes, node_types, num_neigh, neigh_indices, neigh_types, xyz, r,
                                  electric_field, True)

    def _current_response(self, graph_generation, electric_field, forces, bins):
        if not graph_generation:
            raise RuntimeError(self._CURRENT_RESPONSE_ERROR)
        self._compute_prepared_factorized_field_response(graph_generation, electric_field, forces, bins)

    def _compute_current_electric_field_hessian(self, num_nodes, node_types, num_neigh, neigh_indices, neigh_types,
                                                xyz, r, electric_field, graph_generation):
        """The response of the completed evaluation of graph_generation (the
        graph arrays are those of the prepared graph;
        mace_kokkos_response.tpp:2410-2434)."""
        self._current_response(graph_generation, electric_field, False, False)

    def _compute_current_electric_field_force_derivative(self, num_nodes, node_types, num_neigh, neigh_indices,
                                                         neigh_types, xyz, r, electric_field, graph_generation):
        self._current_response(graph_generation, electric_field, True, False)

    def _compute_current_electric_field_bec_bins(self, num_nodes, node_types, num_neigh, neigh_indices,
                                                 neigh_types, xyz, r, electric_field, graph_generation):
        self._current_response(graph_generation, electric_field, True, True)

    def _compute_prepared_factorized_positions_device(self, execution_graph_generation, positions_device_ptr):
        check(lib.smx_compute_prepared_factorized_positions_device(self._h, int(execution_graph_generation),
                                                                   ctypes.c_void_p(positions_device_ptr)))

    def compute_node_energies_forces_field(self, num_nodes, node_types, num_neigh, neigh_indices, neigh_types, xyz,
                                           r, electric_field):
        """compute_node_energies_forces of a MACEField model in an electric
        field (3 values, or 3 per node; pybind mace_kokkos.cpp:2205-2225);
        the field stays set for later calls, dE/dE is electric_field_adj."""
        if not self.has_field_coupling:
            raise ValueError("the model has no field coupling; it takes no electric_field")
        self._set_electric_field(electric_field)
        self.compute_node_energies_forces(num_nodes, node_types, num_neigh, neigh_indices, neigh_types, xyz, r)

    def compute_node_energies_forces(self, num_nodes, node_types, num_neigh, neigh_indices, neigh_types, xyz, r,
                                     execution_graph_generation=0):
        if execution_graph_generation:
            self._compute_prepared_factorized(execution_graph_generation, xyz, r)
            return
        node_types, num_neigh = i32(node_types), i32(num_neigh)
        neigh_indices, neigh_types = i32(neigh_indices), i32(neigh_types)
        xyz, r = f64(xyz), f64(r)
        if xyz.size != 3 * neigh_indices.size or r.size != neigh_indices.size:
            raise ValueError("xyz and r do not match the neighbour list")
        check(lib.smx_compute_node_energies_forces(self._h, int(num_nodes), ptr(node_types), ptr(num_neigh),
                                                   neigh_indices.size, ptr(neigh_indices), ptr(neigh_types),
                                                   ptr(xyz), ptr(r)))
        self._num_nodes = self._num_feature_nodes = int(num_nodes)
        self._num_edges = neigh_indices.size

    # ------------------------------------------------------------ reductions
    def _reduce_atom_forces(self, num_nodes, edge_receivers, edge_sources, execution_graph_generation=0):
        if execution_graph_generation == 0:
            # unprepared path: reduce the directed forces on the host
            # (the calculator's bincount fallback, calculator.py:3860-3874)
            rcv, src = i32(edge_receivers), i32(edge_sources)
            if rcv.size != src.size:
                raise ValueError("Atom-force reduction edge extents are inconsistent.")
            f = self.node_forces.reshape(-1, 3)[: rcv.size]
            out = np.zeros((num_nodes, 3))
            for c in range(3):
                out[:, c] = (np.bincount(src, weights=f[:, c], minlength=num_nodes)
                             - np.bincount(rcv, weights=f[:, c], minlength=num_nodes))
            return out
        out = np.zeros((self._num_feature_nodes, 3))
        check(lib.smx_reduce_prepared_node_forces(self._h, int(execution_graph_generation), ptr(out)))
        return out

    def _reduce_stress(self, volume, xyz, execution_graph_generation=0):
        if execution_graph_generation == 0:
            f = self.node_forces.reshape(-1, 3)
            x = f64(xyz).reshape(-1, 3)
            return (-f[: len(x)].T @ x) / volume
        out = np.zeros((3, 3))
        check(lib.smx_reduce_prepared_stress(self._h, int(execution_graph_generation), float(volume), ptr(out)))
        return out

    def _total_energy(self):
        out = ctypes.c_double()
        check(lib.smx_total_energy_device(self._h, ctypes.byref(out)))
        return float(out.value)

    def _device_outputs(self):
        o = _native.SmxDeviceOutputs()
        o.struct_size = ctypes.sizeof(o)
        check(lib.smx_device_outputs(self._h, ctypes.byref(o)))
        return o

    def synchronize(self):
        check(lib.smx_synchronize(self._h))

    # ----------------------------------------------------------- diagnostics
    def _stage(self, name):
        n = ctypes.c_int64()
        check(lib.smx_debug_stage(self._h, name.encode(), None, 0, ctypes.byref(n)))
        out = np.zeros(n.value, dtype=np.float32)
        check(lib.smx_debug_stage(self._h, name.encode(), ptr(out), out.size, ctypes.byref(n)))
        return out

    def _lammps_compute(self, args):
        """smx_lammps_compute (the pair style's single-rank path) with an
        SmxLammpsArgsV1 (device synchronised on entry) or SmxLammpsArgsV2
        (ordered after args.stream) of device pointers; returns (energy,
        virial[6])."""
        from ._native import SmxLammpsArgsV1, SmxLammpsArgsV2
        if not isinstance(args, (SmxLammpsArgsV1, SmxLammpsArgsV2)):
            raise TypeError("args must be an SmxLammpsArgsV1 or SmxLammpsArgsV2")
        args.struct_size = ctypes.sizeof(type(args))
        energy = ctypes.c_double()
        virial = (ctypes.c_double * 6)()
        check(lib.smx_lammps_compute(self._h, ctypes.cast(ctypes.byref(args), ctypes.POINTER(SmxLammpsArgsV1)),
                                     ctypes.byref(energy), virial))
        return energy.value, np.array(virial[:])

    def set_kernel_timing(self, enabled=True):
        check(lib.smx_set_kernel_timing(self._h, 1 if enabled else 0))

    def set_kernel_timing_filter(self, names=""):
        """Time only the named stages (iterable or comma-separated string)."""
        if not isinstance(names, str):
            names = ",".join(names)
        check(lib.smx_set_kernel_timing_filter(self._h, names.encode()))

    def reset_kernel_timing(self):
        check(lib.smx_kernel_timing_reset(self._h))

    def kernel_timing(self):
        """{kernel name: (total ms, launches)} of the timed launches."""
        out = {}
        i = 0
        while True:
            name = ctypes.c_char_p()
            ms = ctypes.c_double()
            n = ctypes.c_int64()
            check(lib.smx_kernel_timing(self._h, i, ctypes.byref(name), ctypes.byref(ms), ctypes.byref(n)))
            if not name.value:
                break
            out[name.value.decode()] = (ms.value, int(n.value))
            i += 1
        return out


def neighbor_list(positions, cell, cutoff, inverse_cell=None):
    """Device periodic neighbour list (bit-exact with the reference's
    builder): dict of num_neigh, offsets, sources, shifts [E,3],
    fractional_xyz [E,3], receivers."""
    positions = f64(positions)
    n = positions.size // 3
    cell = f64(cell)
    inv = f64(np.linalg.inv(cell.reshape(3, 3)) if inverse_cell is None else inverse_cell)
    ne = ctypes.c_int64(0)
    check(lib.smx_neighbor_list(n, ptr(positions), ptr(cell), ptr(inv), float(cutoff), ctypes.byref(ne),
                                None, None, None, None, None))
    E = int(ne.value)
    out = {"num_neigh": np.zeros(n, np.int32), "offsets": np.zeros(n + 1, np.int32),
           "sources": np.zeros(max(E, 1), np.int32), "shifts": np.zeros(3 * max(E, 1), np.int32),
           "fractional_xyz": np.zeros(3 * max(E, 1))}
    ne2 = ctypes.c_int64(max(E, 1))
    check(lib.smx_neighbor_list(n, ptr(positions), ptr(cell), ptr(inv), float(cutoff), ctypes.byref(ne2),
                                ptr(out["num_neigh"]), ptr(out["offsets"]), ptr(out["sources"]),
                                ptr(out["shifts"]), ptr(out["fractional_xyz"])))
    if int(ne2.value) != E:
        raise RuntimeError("neighbour list changed size between its two passes")
    out["sources"] = out["sources"][:E]
    out["shifts"] = out["shifts"][: 3 * E].reshape(E, 3)
    out["fractional_xyz"] = out["fractional_xyz"][: 3 * E].reshape(E, 3)
    out["receivers"] = np.repeat(np.arange(n, dtype=np.int32), out["num_neigh"])
    return out
