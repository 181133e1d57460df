"""ctypes wrapper of the CPU oracle (liboracle_mace.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker of the HIP path.  The product
(symmetrix-xl_amd/) never imports this module.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle_mace.so")

_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")

_lib = None


def build():
    subprocess.run(["make", "-C", _HERE, "-s"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.oracle_last_error.restype = ctypes.c_char_p
        L.oracle_load.restype = ctypes.c_void_p
        L.oracle_load.argtypes = [ctypes.c_char_p, ctypes.c_int]
        L.oracle_load_head.restype = ctypes.c_void_p
        L.oracle_load_head.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int]
        L.oracle_free.argtypes = [ctypes.c_void_p]
        L.oracle_info.argtypes = [ctypes.c_void_p, _i32p, ctypes.POINTER(ctypes.c_double)]
        L.oracle_atomic_numbers.argtypes = [ctypes.c_void_p, _i32p]
        L.oracle_evaluate.argtypes = [ctypes.c_void_p, ctypes.c_int, _i32p, _i32p, _i32p, _i32p,
                                      _f64p, _f64p, _f64p, _f64p]
        L.oracle_set_num_threads.argtypes = [ctypes.c_int]
        L.oracle_set_field.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
        L.oracle_set_response_drop.argtypes = [ctypes.c_void_p, ctypes.c_int]
        L.oracle_field_response.argtypes = [ctypes.c_void_p, ctypes.c_int, _i32p, _i32p, _i32p, _i32p,
                                            _f64p, _f64p, _f64p, ctypes.c_void_p]
        L.oracle_stage.restype = ctypes.c_longlong
        L.oracle_stage.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p, ctypes.c_longlong]
        L.oracle_radial_tables.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                           ctypes.c_void_p, ctypes.c_void_p, _i32p]
        L.oracle_radial_features.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, _i32p]
        L.oracle_spline_derivatives.argtypes = [_f64p, ctypes.c_int, ctypes.c_double, _f64p]
        L.oracle_spline_eval_f32.argtypes = [ctypes.c_float, ctypes.c_float, ctypes.c_int, ctypes.c_int,
                                             _f32p, _f32p, _f64p, ctypes.c_int, _f32p, _f32p]
        L.oracle_harmonics.argtypes = [_f64p, ctypes.c_int, ctypes.c_int, _f32p, ctypes.c_void_p]
        L.oracle_polynomial.restype = ctypes.c_double
        L.oracle_polynomial.argtypes = [ctypes.c_int, ctypes.c_int, _f64p, _i32p, _i32p, _f64p, _f64p]
        L.oracle_neighbor_count.restype = ctypes.c_longlong
        L.oracle_neighbor_count.argtypes = [_f64p, ctypes.c_int, _f64p, _f64p, ctypes.c_double]
        L.oracle_neighbor_fill.argtypes = [_f64p, ctypes.c_int, _f64p, _f64p, ctypes.c_double,
                                           _i32p, _i32p, _i32p, _i32p, _f64p]
        L.oracle_prepared_geometry.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_longlong, _i32p, _i32p, _f64p,
                                               ctypes.c_void_p, ctypes.c_void_p, _f64p, _f64p, _i32p, _f64p,
                                               ctypes.c_double, _f64p, _f64p]
        L.oracle_wrapped_fractional.argtypes = [_f64p, ctypes.c_int, _f64p, _f64p]
        L.oracle_reduce_forces.argtypes = [ctypes.c_int, ctypes.c_longlong, _i32p, _i32p, _f64p, _f64p]
        L.oracle_reduce_stress.argtypes = [ctypes.c_longlong, _f64p, _f64p, ctypes.c_double, _f64p]
        L.oracle_zbl.argtypes = [ctypes.c_double, ctypes.c_double, _f64p, _f64p, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_int, ctypes.c_int, ctypes.c_double, _f64p]
        _lib = L
    return _lib


def zbl_pair(a_exp, a_prefactor, c, covalent_radii, p, Zu, Zv, r):
    """(value, dV/dr, envelope, d envelope/dr) of one ZBL pair at r."""
    out = np.zeros(4)
    radii = _c(covalent_radii, np.float64)
    if lib().oracle_zbl(a_exp, a_prefactor, _c(c, np.float64), radii, len(radii), p, Zu, Zv, r, out) != 0:
        raise ValueError(_err())
    return tuple(float(v) for v in out)


def _err():
    return lib().oracle_last_error().decode()


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


class OracleModel:
    """The oracle evaluator for one model file, FP32 (default) or FP64."""

    def __init__(self, path, fp64=False, head=""):
        self._h = lib().oracle_load_head(path.encode(), (head or "").encode(), 1 if fp64 else 0)
        if not self._h:
            raise ValueError(_err())
        info = np.zeros(10, dtype=np.int32)
        rc = ctypes.c_double()
        lib().oracle_info(self._h, info, ctypes.byref(rc))
        (self.num_elements, self.num_channels, self.l_max, self.L_max, self.num_lm,
         self.num_LM, self.num_paths, self.num_rows, self.num_lme, self.num_m1_terms) = [int(v) for v in info]
        self.r_cut = rc.value
        z = np.zeros(self.num_elements, dtype=np.int32)
        lib().oracle_atomic_numbers(self._h, z)
        self.atomic_numbers = z

    def __del__(self):
        if getattr(self, "_h", None):
            lib().oracle_free(self._h)
            self._h = None

    def types_of(self, numbers):
        lut = {int(z): i for i, z in enumerate(self.atomic_numbers)}
        return np.array([lut[int(z)] for z in numbers], dtype=np.int32)

    def evaluate(self, node_types, num_neigh, neigh_indices, neigh_types, xyz, r, field=None):
        """Node energies and directed forces; a MACEField model needs the
        electric field (3 values, or 3 per node); dE/dE is then
        stage("field_adj")."""
        f64 = None if field is None else _c(field, np.float64).ravel()
        lib().oracle_set_field(self._h, None if f64 is None else f64.ctypes.data, 0 if f64 is None else f64.size)
        node_types = _c(node_types, np.int32)
        n = len(node_types)
        E = len(neigh_indices)
        e = np.zeros(n)
        f = np.zeros(3 * E)
        rc = lib().oracle_evaluate(self._h, n, node_types, _c(num_neigh, np.int32),
                                   _c(neigh_indices, np.int32), _c(neigh_types, np.int32),
                                   _c(xyz, np.float64).ravel(), _c(r, np.float64), e, f)
        if rc != 0:
            raise ValueError(_err())
        return e, f.reshape(E, 3)

    def field_response(self, node_types, num_neigh, neigh_indices, neigh_types, xyz, r, field, forces=True):
        """MACEField response in a graph field (3 values): the Hessian
        d2E/dE_c dE_s as [c][s], and with forces the directed forces'
        tangent [s][edge][3] (else None).  Evaluates first."""
        f64 = _c(field, np.float64).ravel()
        lib().oracle_set_field(self._h, f64.ctypes.data, f64.size)
        node_types = _c(node_types, np.int32)
        E = len(neigh_indices)
        hess = np.zeros(9)
        fd = np.zeros(9 * E) if forces else None
        rc = lib().oracle_field_response(self._h, len(node_types), node_types, _c(num_neigh, np.int32),
                                         _c(neigh_indices, np.int32), _c(neigh_types, np.int32),
                                         _c(xyz, np.float64).ravel(), _c(r, np.float64), hess,
                                         fd.ctypes.data if forces else None)
        if rc != 0:
            raise ValueError(_err())
        return hess.reshape(3, 3), (fd.reshape(3, E, 3) if forces else None)

    def set_response_drop(self, mask):
        """Leave terms out of the response's tangent (tests of the pins only)."""
        lib().oracle_set_response_drop(self._h, int(mask))

    def stage(self, name):
        size = lib().oracle_stage(self._h, name.encode(), None, 0)
        if size < 0:
            raise KeyError(name)
        out = np.zeros(size)
        lib().oracle_stage(self._h, name.encode(), out.ctypes.data, size)
        return out

    def radial_tables(self, which, ti=0, tj=0):
        """Nodal values and derivatives [function][point] of network which
        (0 R0, 1 R1, 2 A0, 3 A1) for the pair of model types (ti, tj)."""
        shape = np.zeros(2, dtype=np.int32)
        if lib().oracle_radial_tables(self._h, which, ti, tj, None, None, shape) != 0:
            raise ValueError(_err())
        v = np.zeros(int(shape[0]) * int(shape[1]))
        d = np.zeros_like(v)
        if lib().oracle_radial_tables(self._h, which, ti, tj, v.ctypes.data, d.ctypes.data, shape) != 0:
            raise ValueError(_err())
        return v.reshape(shape), d.reshape(shape)

    def radial_features(self, ti=0, tj=0):
        shape = np.zeros(2, dtype=np.int32)
        if lib().oracle_radial_features(self._h, ti, tj, None, shape) != 0:
            raise ValueError(_err())
        out = np.zeros(int(shape[0]) * int(shape[1]))
        lib().oracle_radial_features(self._h, ti, tj, out.ctypes.data, shape)
        return out.reshape(shape)


def neighbor_graph(positions, cell, cutoff):
    """Bit-exact periodic neighbour list: dict of num_neigh, offsets, sources,
    shifts [E,3], fractional_xyz [E,3]."""
    pos = _c(positions, np.float64).ravel()
    cell = _c(cell, np.float64)
    inv = np.ascontiguousarray(np.linalg.inv(cell))
    n = len(pos) // 3
    E = lib().oracle_neighbor_count(pos, n, cell.ravel(), inv.ravel(), cutoff)
    if E < 0:
        raise ValueError(_err())
    out = {"num_neigh": np.zeros(n, np.int32), "offsets": np.zeros(n + 1, np.int32),
           "sources": np.zeros(E, np.int32), "shifts": np.zeros(3 * E, np.int32),
           "fractional_xyz": np.zeros(3 * E)}
    rc = lib().oracle_neighbor_fill(pos, n, cell.ravel(), inv.ravel(), cutoff, out["num_neigh"],
                                    out["offsets"], out["sources"], out["shifts"], out["fractional_xyz"])
    if rc != 0:
        raise ValueError(_err())
    out["shifts"] = out["shifts"].reshape(E, 3)
    out["fractional_xyz"] = out["fractional_xyz"].reshape(E, 3)
    out["receivers"] = np.repeat(np.arange(n, dtype=np.int32), out["num_neigh"])
    out["inverse_cell"] = inv
    return out


GEOMETRY_KINDS = {"cartesian": 0, "fractional": 1, "shifts": 2}


def prepared_geometry_kind(kind, receivers, sources, ref_positions, ref_edges, cell, positions, cutoff,
                           pbc=(1, 1, 1)):
    """Edge vectors and lengths of a positions call on a prepared geometry
    (lifecycle.cpp:2915-3079): kind "cartesian" (ref xyz per edge),
    "fractional" (fractional positions and xyz) or "shifts" (integer cell
    shifts per edge).  Raises ValueError on an invalid edge."""
    receivers, sources = _c(receivers, np.int32), _c(sources, np.int32)
    E = len(sources)
    n = len(np.asarray(positions)) if np.ndim(positions) == 2 else len(np.asarray(positions)) // 3
    cell = _c(cell, np.float64).reshape(3, 3)
    inv = _c(np.linalg.inv(cell) if abs(np.linalg.det(cell)) > 0 else np.zeros((3, 3)), np.float64)
    xyz = np.zeros(3 * E)
    r = np.zeros(E)
    edges = _c(ref_edges, np.int32 if kind == "shifts" else np.float64).ravel()
    bad = lib().oracle_prepared_geometry(
        GEOMETRY_KINDS[kind], n, E, receivers, sources, _c(ref_positions, np.float64).ravel(),
        edges.ctypes.data if E else None, edges.ctypes.data if (E and kind == "shifts") else None,
        cell.ravel(), inv.ravel(), _c(pbc, np.int32), _c(positions, np.float64).ravel(), cutoff, xyz, r)
    if bad:
        raise ValueError("invalid edge geometry")
    return xyz.reshape(E, 3), r


def wrapped_fractional(positions, cell):
    pos = _c(positions, np.float64).ravel()
    out = np.zeros_like(pos)
    lib().oracle_wrapped_fractional(pos, len(pos) // 3, _c(np.linalg.inv(cell), np.float64).ravel(), out)
    return out.reshape(-1, 3)


def prepared_geometry(graph, cell, reference_positions, positions, cutoff):
    """Edge geometry of the periodic graph the device builder prepares: its
    fractional reference (wrapped fractional positions of reference_positions
    and the list's fractional edge vectors)."""
    cell = np.asarray(cell, dtype=np.float64)
    return prepared_geometry_kind("fractional", graph["receivers"], graph["sources"],
                                  wrapped_fractional(reference_positions, cell), graph["fractional_xyz"], cell,
                                  positions, cutoff)


def reduce_forces(n, receivers, sources, node_forces):
    out = np.zeros(3 * n)
    lib().oracle_reduce_forces(n, len(sources), _c(receivers, np.int32), _c(sources, np.int32),
                               _c(node_forces, np.float64).ravel(), out)
    return out.reshape(n, 3)


def reduce_stress(node_forces, xyz, volume):
    out = np.zeros(9)
    lib().oracle_reduce_stress(len(xyz), _c(node_forces, np.float64).ravel(),
                               _c(xyz, np.float64).ravel(), volume, out)
    return out.reshape(3, 3)


def evaluate_system(model, system, skin=0.5, positions=None, graph=None, field=None):
    """Energy, atom forces and 3x3 stress of a system with the oracle (the
    caller contract of calculator.py:3821-3894 on a fresh graph)."""
    pos0 = np.asarray(system["positions"], dtype=np.float64)
    cell = np.asarray(system["cell"], dtype=np.float64)
    if graph is None:
        graph = neighbor_graph(pos0, cell, model.r_cut + skin)
    pos = pos0 if positions is None else positions
    xyz, r = prepared_geometry(graph, cell, pos0, pos, model.r_cut)
    types = model.types_of(system["numbers"])
    e, f = model.evaluate(types, graph["num_neigh"], graph["sources"], types[graph["sources"]], xyz, r, field)
    forces = reduce_forces(len(types), graph["receivers"], graph["sources"], f)
    stress = reduce_stress(f, xyz, abs(np.linalg.det(cell)))
    out = {"energy": float(np.sum(e)), "energies": e, "forces": forces, "stress": stress,
           "node_forces": f, "graph": graph, "xyz": xyz, "r": r}
    if field is not None:
        out["field_adj"] = model.stage("field_adj")
    return out


def field_response_system(model, system, field, skin=0.5, positions=None, graph=None, forces=True):
    """The MACEField response of a system (the calculator's contract,
    calculator.py:3783-3817): Hessian [c][s], the directed forces' tangent
    [s][edge][3], Born charges bec[i][s][xyz] = dF_i/dE_s (sources plus,
    receivers minus) and the graph."""
    pos0 = np.asarray(system["positions"], dtype=np.float64)
    cell = np.asarray(system["cell"], dtype=np.float64)
    if graph is None:
        graph = neighbor_graph(pos0, cell, model.r_cut + skin)
    pos = pos0 if positions is None else positions
    xyz, r = prepared_geometry(graph, cell, pos0, pos, model.r_cut)
    types = model.types_of(system["numbers"])
    hess, fd = model.field_response(types, graph["num_neigh"], graph["sources"], types[graph["sources"]], xyz, r,
                                    field, forces)
    out = {"hessian": hess, "graph": graph, "xyz": xyz, "r": r}
    if forces:
        n = len(types)
        out["force_derivative"] = fd
        out["bec"] = np.stack([reduce_forces(n, graph["receivers"], graph["sources"], fd[s]) for s in range(3)],
                              axis=1)
    return out
