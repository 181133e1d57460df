"""MH-1 (``MACE_Nonlinear``) evaluator on one MI355X.

``MACENonlinearKokkosFloat`` mirrors the reference's pybind class of the same
name (symmetrix/source/cpp/mace_nonlinear_kokkos.cpp:19-240, the members the
calculator and pair style use): the constructor ``(filename, head)``,
``r_cut``, ``selected_head``, ``available_heads``, ``is_mh1_family``,
``mh1_node_channels``, ``mh1_edge_channels``, ``mh1_radial_size``,
``mh1_l_max``, ``mh1_family_rejection_reason``, ``atomic_numbers``,
``atomic_energies``, ``compute_node_energies_forces(num_nodes, node_types,
num_neigh, neigh_indices, neigh_types, xyz, r)`` and ``node_energies`` /
``node_forces``.  Every call goes through the C ABI of
include/symmetrix_mh1.h into the HIP kernels (libsymmetrix_mi355x.so); there
is no CPU path.
"""

from __future__ import annotations

import ctypes
import json

import numpy as np

from . import _native
from ._native import check, f64, i32, lib, ptr


def is_nonlinear_model(filename):
    """True for a ``MACE_Nonlinear`` JSON file (the reference dispatches on
    ``model_type``, not on the file name: test_mh1.py:2678)."""
    try:
        with open(filename, "rb") as f:
            head = f.read(4096).decode("utf-8", "replace")
    except OSError:
        return False
    if '"model_type"' in head:
        return '"MACE_Nonlinear"' in head.split('"model_type"', 1)[1][:64]
    try:
        with open(filename) as f:
            return json.load(f).get("model_type") == "MACE_Nonlinear"
    except (OSError, ValueError):
        return False


class MACENonlinearKokkosFloat:
    """FP32 MH-1 evaluator on one MI355X."""

    precision = "float32"

    def __init__(self, filename, head=""):
        h = ctypes.c_void_p()
        check(lib.smx_mh1_create(str(filename).encode(), (head or "").encode(), ctypes.byref(h)))
        self._h = h
        info = _native.SmxMh1Info()
        info.struct_size = ctypes.sizeof(info)
        check(lib.smx_mh1_info(self._h, ctypes.byref(info)))
        self.r_cut = info.r_cut
        self.num_elements = info.num_elements
        self.l_max = info.l_max
        self.num_interactions = info.num_interactions
        self.is_mh1_family = bool(info.is_mh1_family)
        self.mh1_node_channels = info.node_channels
        self.mh1_edge_channels = info.edge_channels
        self.mh1_radial_size = info.radial_size
        self.mh1_l_max = info.l_max if self.is_mh1_family else 0
        self.has_zbl = bool(info.has_zbl)
        self.has_field_coupling = False
        name = ctypes.c_char_p()
        check(lib.smx_mh1_selected_head(self._h, ctypes.byref(name)))
        self.selected_head = name.value.decode() if name.value else ""
        self.available_heads = [self.selected_head] if self.selected_head else []
        check(lib.smx_mh1_family_rejection(self._h, ctypes.byref(name)))
        self.mh1_family_rejection_reason = name.value.decode() if name.value else ""
        self._num_nodes = 0
        self._num_edges = 0

    def close(self):
        if getattr(self, "_h", None):
            lib.smx_mh1_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    @property
    def atomic_numbers(self):
        out = np.zeros(self.num_elements, dtype=np.int32)
        check(min(0, lib.smx_mh1_atomic_numbers(self._h, ptr(out), out.size)))
        return [int(v) for v in out]

    @property
    def atomic_energies(self):
        out = np.zeros(self.num_elements)
        check(min(0, lib.smx_mh1_atomic_energies(self._h, ptr(out), out.size)))
        return [float(v) for v in out]

    def compute_node_energies_forces(self, num_nodes, node_types, num_neigh, neigh_indices, neigh_types, xyz, r):
        t, nn, ni, nt = i32(node_types), i32(num_neigh), i32(neigh_indices), i32(neigh_types)
        x, rr = f64(xyz), f64(r)
        if x.size != 3 * rr.size or ni.size != rr.size or nt.size != rr.size:
            raise ValueError("edge arrays have inconsistent sizes")
        if t.size != num_nodes or nn.size != num_nodes:
            raise ValueError("node arrays must hold num_nodes entries")
        check(lib.smx_mh1_compute_node_energies_forces(self._h, int(num_nodes), ptr(t), ptr(nn), ptr(ni), ptr(nt),
                                                       ptr(x), ptr(rr), rr.size))
        self._num_nodes = int(num_nodes)
        self._num_edges = int(rr.size)

    @property
    def node_energies(self):
        out = np.zeros(self._num_nodes)
        check(lib.smx_mh1_node_energies(self._h, ptr(out), out.size))
        return out

    @property
    def node_forces(self):
        out = np.zeros(3 * self._num_edges)
        check(lib.smx_mh1_node_forces(self._h, ptr(out), out.size))
        return out

    def _stage(self, name):
        n = ctypes.c_int64()
        check(lib.smx_mh1_debug_stage(self._h, name.encode(), None, 0, ctypes.byref(n)))
        out = np.zeros(n.value, dtype=np.float32)
        check(lib.smx_mh1_debug_stage(self._h, name.encode(), ptr(out), out.size, ctypes.byref(n)))
        return out

    def _set_kernel_timing(self, enabled):
        check(lib.smx_mh1_set_kernel_timing(self._h, 1 if enabled else 0))

    def _kernel_timing(self):
        name, ms, n = ctypes.c_char_p(), ctypes.c_double(), ctypes.c_int64()
        count = lib.smx_mh1_kernel_timing(self._h, -1, None, None, None)
        check(min(0, count))
        out = {}
        for k in range(count):
            check(min(0, lib.smx_mh1_kernel_timing(self._h, k, ctypes.byref(name), ctypes.byref(ms),
                                                   ctypes.byref(n))))
            out[name.value.decode()] = (ms.value, n.value)
        return out
