"""ctypes mirror of the reference's R1 HIP plugin ABI as exported by
libsymmetrix_mi355x.so (include/symmetrix_r1_plugin.h; the reference's
jit_hip_plugin_abi.h:28-269), with the configure step this library adds.

``configure(model_path, ...)`` selects the model whose R1 coupling the
launchers apply; ``descriptor()`` then returns what the reference's loader
reads from ``symmetrix_jit_hip_plugin_query_v1`` (jit_hip_plugin.cpp:273-301).
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _native
from ._native import SmxR1PluginIdentity, check, lib

_u32 = ctypes.c_uint32
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_dbl = ctypes.c_double
_vp = ctypes.c_void_p

FORWARD = 1 << 0
COORDINATE_REVERSE = 1 << 1
ABI_TAG = b"symmetrix.jit.hip-plugin/1"


class RadialSpline(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("edge_types", _u32), ("intervals", _u32), ("functions", _u32),
                ("h", _dbl), ("x0", _dbl), ("coefficients", _vp)]


class ForwardArgs(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("active_type_count", _u32), ("num_nodes", _i64), ("num_edges", _i64),
                ("node_types", _vp), ("num_neigh", _vp), ("first_neigh", _vp), ("neigh_indices", _vp),
                ("neigh_types", _vp), ("type_to_active", _vp), ("radius", _vp), ("radial", RadialSpline),
                ("harmonics_values", _vp), ("neighbor_features", _vp), ("output", _vp), ("cutoff", _dbl)]


class SourceArgs(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("active_type_count", _u32), ("num_nodes", _i64), ("num_edges", _i64),
                ("node_types", _vp), ("neigh_types", _vp), ("source_offsets", _vp), ("source_edges", _vp),
                ("edge_receivers", _vp), ("type_to_active", _vp), ("radius", _vp), ("radial", RadialSpline),
                ("harmonics_values", _vp), ("output_adjoint", _vp), ("source_adjoint", _vp), ("cutoff", _dbl)]


class EdgeArgs(ctypes.Structure):
    _fields_ = [("struct_size", _u32), ("active_type_count", _u32), ("coordinate_scalar_size", _u32),
                ("coordinates_are_unit", _u32), ("num_nodes", _i64), ("num_edges", _i64), ("node_types", _vp),
                ("neigh_indices", _vp), ("neigh_types", _vp), ("edge_receivers", _vp), ("type_to_active", _vp),
                ("xyz", _vp), ("radius", _vp), ("radial", RadialSpline), ("harmonics_values", _vp),
                ("harmonics_gradients", _vp), ("neighbor_features", _vp), ("output_adjoint", _vp),
                ("directed_forces", _vp), ("cutoff", _dbl)]


ForwardLaunch = ctypes.CFUNCTYPE(_i32, ctypes.POINTER(ForwardArgs), _vp, _i32)
ReverseLaunch = ctypes.CFUNCTYPE(_i32, ctypes.POINTER(SourceArgs), ctypes.POINTER(EdgeArgs), _vp, _i32)


class PluginV1(ctypes.Structure):
    _fields_ = [("abi_version", _u32), ("struct_size", _u32), ("pointer_size", _u32), ("byte_order", _u32),
                ("capabilities", _u32), ("scalar_kind", _u32), ("scalar_size", _u32), ("reserved", _u32),
                ("abi_tag", ctypes.c_char_p), ("artifact_id", ctypes.c_char_p),
                ("contract_fingerprint", ctypes.c_char_p), ("semantic_fingerprint", ctypes.c_char_p),
                ("structure_fingerprint", ctypes.c_char_p), ("channels", _i32), ("embedding", _i32),
                ("edge_l_max", _i32), ("source_l_max", _i32), ("target_architecture", ctypes.c_char_p),
                ("target_features", ctypes.c_char_p), ("native_subgroup_width", _i32),
                ("forward_threads_per_block", _i32), ("source_threads_per_block", _i32),
                ("edge_threads_per_block", _i32), ("persistent_blocks_per_compute_unit", _i32),
                ("r1_forward_launch", ForwardLaunch), ("r1_coordinate_reverse_launch", ReverseLaunch)]


_query = lib.symmetrix_jit_hip_plugin_query_v1
_query.restype = ctypes.POINTER(PluginV1)
_query.argtypes = []


def descriptor():
    """The exported descriptor, or None before a successful configure()."""
    p = _query()
    return p.contents if p else None


def configure(model_path, artifact_id="smx-r1", contract_fingerprint="unset", semantic_fingerprint="",
              structure_fingerprint="", embedding=8, fp64_evaluation_point=False,
              persistent_blocks_per_compute_unit=4):
    ident = SmxR1PluginIdentity(ctypes.sizeof(SmxR1PluginIdentity), artifact_id.encode(),
                                contract_fingerprint.encode(), semantic_fingerprint.encode(),
                                structure_fingerprint.encode(), b"", int(embedding),
                                1 if fp64_evaluation_point else 0, int(persistent_blocks_per_compute_unit))
    check(lib.smx_r1_plugin_configure(str(model_path).encode(), ctypes.byref(ident)))
    return descriptor()


def spline_table():
    """(table [1, intervals, 4, functions] float32, h, x0) of the configured model."""
    iv, fn = ctypes.c_int32(), ctypes.c_int32()
    h, x0 = ctypes.c_double(), ctypes.c_double()
    check(lib.smx_r1_plugin_spline_table(None, 0, ctypes.byref(iv), ctypes.byref(fn), ctypes.byref(h),
                                         ctypes.byref(x0)))
    out = np.empty((1, iv.value, 4, fn.value), np.float32)
    check(lib.smx_r1_plugin_spline_table(out.ctypes.data, out.size, None, None, None, None))
    return out, h.value, x0.value


__all__ = ["RadialSpline", "ForwardArgs", "SourceArgs", "EdgeArgs", "PluginV1", "configure", "descriptor",
           "spline_table", "FORWARD", "COORDINATE_REVERSE", "ABI_TAG", "_native"]
