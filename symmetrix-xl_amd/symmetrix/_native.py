"""ctypes binding of libsymmetrix_mi355x.so (the C ABI declared in
include/symmetrix_mi355x.h).

The library is built in-tree (``make -C symmetrix-xl_amd/csrc``); there is no
fallback: importing this module raises ImportError when the library is
missing, and every entry point's error code becomes a Python exception.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libsymmetrix_mi355x.so")

SMX_OK = 0
SMX_ERR_INVALID_ARGUMENT = -1
SMX_ERR_RUNTIME = -2
SMX_ERR_LOGIC = -3
SMX_ERR_OUT_OF_MEMORY = -4
SMX_ERR_UNSUPPORTED = -5


class SymmetrixUnsupportedError(ValueError):
    """The model's shape or features have no compiled MI355X kernel set."""


class SmxModelInfo(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("num_elements", ctypes.c_int32),
                ("num_channels", ctypes.c_int32), ("l_max", ctypes.c_int32),
                ("L_max", ctypes.c_int32), ("num_interactions", ctypes.c_int32),
                ("num_paths", ctypes.c_int32), ("num_lme", ctypes.c_int32),
                ("r_cut", ctypes.c_double)]


class SmxDeviceOutputs(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("num_nodes", ctypes.c_int32),
                ("num_edges", ctypes.c_int64), ("node_energies", ctypes.c_void_p),
                ("node_forces", ctypes.c_void_p), ("atom_forces", ctypes.c_void_p),
                ("stress", ctypes.c_void_p), ("total_energy", ctypes.c_void_p),
                ("xyz", ctypes.c_void_p), ("r", ctypes.c_void_p)]


class SmxR1PluginIdentity(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("artifact_id", ctypes.c_char_p),
                ("contract_fingerprint", ctypes.c_char_p), ("semantic_fingerprint", ctypes.c_char_p),
                ("structure_fingerprint", ctypes.c_char_p), ("target_features", ctypes.c_char_p),
                ("embedding", ctypes.c_int32), ("fp64_evaluation_point", ctypes.c_int32),
                ("persistent_blocks_per_compute_unit", ctypes.c_int32)]


class SmxLammpsArgsV1(ctypes.Structure):
    """Arguments of smx_lammps_compute (device pointers as integers)."""
    _fields_ = [("struct_size", ctypes.c_uint32), ("inum", ctypes.c_int32), ("nall", ctypes.c_int32),
                ("ntypes", ctypes.c_int32), ("ilist", ctypes.c_void_p), ("numneigh", ctypes.c_void_p),
                ("neighbors", ctypes.c_void_p), ("stride_atom", ctypes.c_int64),
                ("stride_neighbor", ctypes.c_int64), ("x", ctypes.c_void_p), ("type", ctypes.c_void_p),
                ("type_to_model", ctypes.c_void_p), ("owner", ctypes.c_void_p), ("rebuild", ctypes.c_int32),
                ("reserved", ctypes.c_int32), ("f", ctypes.c_void_p), ("eatom", ctypes.c_void_p)]


class SmxEvaluatorCounters(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("reserved", ctypes.c_uint32),
                ("last_graph_prepare_ms", ctypes.c_double), ("last_evaluation_ms", ctypes.c_double),
                ("graph_prepare_count", ctypes.c_int64), ("evaluation_count", ctypes.c_int64),
                ("geometry_prepare_count", ctypes.c_int64)]


class SmxMh1Info(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("num_elements", ctypes.c_int32), ("l_max", ctypes.c_int32),
                ("num_interactions", ctypes.c_int32), ("is_mh1_family", ctypes.c_int32),
                ("node_channels", ctypes.c_int32), ("edge_channels", ctypes.c_int32),
                ("radial_size", ctypes.c_int32), ("has_zbl", ctypes.c_int32), ("r_cut", ctypes.c_double)]


class SmxLammpsArgsV2(ctypes.Structure):
    """SmxLammpsArgsV1 followed by the caller's hipStream_t: the call waits
    for the work the caller queued there instead of synchronising the device."""
    _fields_ = SmxLammpsArgsV1._fields_ + [("stream", ctypes.c_void_p)]


# (name, restype, argtypes) of every exported entry point
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_dbl = ctypes.c_double
_vp = ctypes.c_void_p
_cp = ctypes.c_char_p
_p_i32 = ctypes.POINTER(ctypes.c_int32)
_p_i64 = ctypes.POINTER(ctypes.c_int64)
_p_u64 = ctypes.POINTER(ctypes.c_uint64)
_p_dbl = ctypes.POINTER(ctypes.c_double)

SIGNATURES = [
    ("smx_abi_version", _i32, []),
    ("smx_last_error", _cp, []),
    ("smx_evaluator_create", _i32, [_cp, _cp, ctypes.POINTER(_vp)]),
    ("smx_evaluator_destroy", None, [_vp]),
    ("smx_evaluator_info", _i32, [_vp, ctypes.POINTER(SmxModelInfo)]),
    ("smx_evaluator_atomic_numbers", _i32, [_vp, _vp, _i32]),
    ("smx_evaluator_atomic_energies", _i32, [_vp, _vp, _i32]),
    ("smx_active_atomic_numbers", _i32, [_vp, _vp, _i32, _p_i32]),
    ("smx_prediction_head", _i32, [_vp, _i32, ctypes.POINTER(ctypes.c_char_p)]),
    ("smx_set_streamed_edges", _i32, [_vp, _cp]),
    ("smx_evaluator_stream", _vp, [_vp]),
    ("smx_prepare_factorized_graph", _i32, [_vp, _i32, _vp, _vp, _i64, _vp, _vp, _p_u64]),
    ("smx_prepare_factorized_graph_device", _i32, [_vp, _i32, _vp, _vp, _i64, _vp, _vp, _p_u64]),
    ("smx_prepare_factorized_feature_graph", _i32,
     [_vp, _i32, _i32, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _p_u64]),
    ("smx_prepare_factorized_feature_graph_device", _i32,
     [_vp, _i32, _i32, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _p_u64]),
    ("smx_compute_factorized_single_layer_distributed_evaluation", _i32, [_vp, _u64, _i32, _i32, _vp, _vp, _i32]),
    ("smx_begin_factorized_distributed_evaluation", _i32, [_vp, _u64, _i32, _i32, _vp, _vp, _i32]),
    ("smx_begin_factorized_distributed_positions_evaluation", _i32, [_vp, _u64, _i32, _i32, _vp, _i32]),
    ("smx_compute_factorized_single_layer_distributed_positions_evaluation", _i32,
     [_vp, _u64, _i32, _i32, _vp, _i32]),
    ("smx_continue_factorized_distributed_evaluation", _i32, [_vp, _vp, _i64, _i32]),
    ("smx_finish_factorized_distributed_evaluation", _i32, [_vp, _vp, _i64, _i32]),
    ("smx_distributed_exchange", _i32, [_vp, _i32, ctypes.POINTER(_vp), _p_i64, _p_i64]),
    ("smx_prepare_periodic_factorized_graph", _i32,
     [_vp, _i32, _vp, _vp, _vp, _vp, _dbl, _p_u64, _p_i64]),
    ("smx_set_execution_plan", _i32, [_vp, _cp, _i32]),
    ("smx_execution_plan", _i32, [_vp, _vp, _i64]),
    ("smx_update_factorized_cell", _i32, [_vp, _u64, _vp, _vp]),
    ("smx_compute_prepared_factorized", _i32, [_vp, _u64, _vp, _vp]),
    ("smx_compute_prepared_factorized_positions", _i32, [_vp, _u64, _vp]),
    ("smx_compute_prepared_factorized_positions_field", _i32, [_vp, _u64, _vp, _vp, _i64]),
    ("smx_compute_prepared_factorized_positions_results", _i32, [_vp, _u64, _vp, _dbl, _vp, _vp, _vp]),
    ("smx_compute_prepared_factorized_field", _i32, [_vp, _u64, _vp, _vp, _vp, _i64]),
    ("smx_set_electric_field", _i32, [_vp, _vp, _i64]),
    ("smx_electric_field_adj", _i32, [_vp, _vp, _i64, _p_i64]),
    ("smx_has_field_coupling", _i32, [_vp, _p_i32]),
    ("smx_compute_prepared_factorized_field_response", _i32, [_vp, _u64, _vp, _i64, _i32, _i32]),
    ("smx_electric_field_hessian", _i32, [_vp, _vp, _i64, _p_i64]),
    ("smx_electric_field_force_derivative", _i32, [_vp, _vp, _i64, _p_i64]),
    ("smx_electric_field_bec_bins", _i32, [_vp, _vp, _i64, _p_i64]),
    ("smx_compute_prepared_factorized_positions_device", _i32, [_vp, _u64, _vp]),
    ("smx_compute_node_energies_forces", _i32, [_vp, _i32, _vp, _vp, _i64, _vp, _vp, _vp, _vp]),
    ("smx_reduce_prepared_node_forces", _i32, [_vp, _u64, _vp]),
    ("smx_reduce_prepared_stress", _i32, [_vp, _u64, _dbl, _vp]),
    ("smx_node_energies", _i32, [_vp, _vp, _i64]),
    ("smx_node_forces", _i32, [_vp, _vp, _i64]),
    ("smx_total_energy_device", _i32, [_vp, _vp]),
    ("smx_device_outputs", _i32, [_vp, ctypes.POINTER(SmxDeviceOutputs)]),
    ("smx_synchronize", _i32, [_vp]),
    ("smx_lammps_compute", _i32, [_vp, ctypes.POINTER(SmxLammpsArgsV1), ctypes.POINTER(_dbl),
                                  ctypes.POINTER(_dbl)]),
    ("smx_debug_stage", _i32, [_vp, _cp, _vp, _i64, _p_i64]),
    ("smx_set_kernel_timing", _i32, [_vp, _i32]),
    ("smx_set_kernel_timing_filter", _i32, [_vp, _cp]),
    ("smx_kernel_timing_reset", _i32, [_vp]),
    ("smx_kernel_timing", _i32, [_vp, _i32, ctypes.POINTER(_cp), _p_dbl, _p_i64]),
    ("smx_neighbor_list", _i32, [_i32, _vp, _vp, _vp, _dbl, _p_i64, _vp, _vp, _vp, _vp, _vp]),
    ("smx_model_convert", _i32, [_cp, _cp, _cp]),
    ("smx_set_execution_plan_request", _i32, [_vp, _cp, _cp, _cp]),
    ("smx_set_allow_fixed_workspace", _i32, [_vp, _i32]),
    ("smx_execution_plan_report", _i32, [_vp, _vp, _i64, _p_i64]),
    ("smx_evaluator_counters", _i32, [_vp, ctypes.POINTER(SmxEvaluatorCounters)]),
    ("smx_prepare_active_types", _i32, [_vp, _vp, _i32]),
    ("smx_prepare_factorized_geometry", _i32, [_vp, _u64, _vp, _i64, _vp, _i64, _vp, _vp, _vp]),
    ("smx_prepare_factorized_shift_geometry", _i32, [_vp, _u64, _vp, _i64, _vp, _i64, _vp, _vp, _vp]),
    ("smx_prepare_factorized_fractional_geometry", _i32, [_vp, _u64, _vp, _i64, _vp, _i64, _vp, _vp, _vp]),
    ("smx_r1_plugin_configure", _i32, [_cp, ctypes.POINTER(SmxR1PluginIdentity)]),
    ("smx_r1_plugin_spline_table", _i32, [_vp, _i64, _p_i32, _p_i32, _p_dbl, _p_dbl]),
    ("smx_r1_plugin_reserve", _i32, [_vp, _i64, _i64]),
    ("smx_r1_plugin_reverse_launch_noalloc", _i32, [_vp, _vp, _vp, _vp, _i32]),
    ("smx_model_array_f32", _i32, [_cp, _cp, _vp, _i64, _p_i64, _p_i32, _p_dbl, _p_dbl]),
    ("smx_model_array_i32", _i32, [_cp, _cp, _vp, _i64, _p_i64, _p_i32]),
    # MH-1 (MACE_Nonlinear), include/symmetrix_mh1.h
    ("smx_mh1_create", _i32, [_cp, _cp, ctypes.POINTER(_vp)]),
    ("smx_mh1_destroy", None, [_vp]),
    ("smx_mh1_info", _i32, [_vp, ctypes.POINTER(SmxMh1Info)]),
    ("smx_mh1_family_rejection", _i32, [_vp, ctypes.POINTER(_cp)]),
    ("smx_mh1_atomic_numbers", _i32, [_vp, _vp, _i32]),
    ("smx_mh1_atomic_energies", _i32, [_vp, _vp, _i32]),
    ("smx_mh1_selected_head", _i32, [_vp, ctypes.POINTER(_cp)]),
    ("smx_mh1_compute_node_energies_forces", _i32, [_vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _i64]),
    ("smx_mh1_node_energies", _i32, [_vp, _vp, _i64]),
    ("smx_mh1_node_forces", _i32, [_vp, _vp, _i64]),
    ("smx_mh1_debug_stage", _i32, [_vp, _cp, _vp, _i64, _p_i64]),
    ("smx_mh1_set_kernel_timing", _i32, [_vp, _i32]),
    ("smx_mh1_kernel_timing", _i32, [_vp, _i32, ctypes.POINTER(_cp), _p_dbl, _p_i64]),
]


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            "libsymmetrix_mi355x.so is not built (expected at %s); run "
            "`make -C symmetrix-xl_amd/csrc` or __graft_entry__.build()" % LIB_PATH)
    lib = ctypes.CDLL(LIB_PATH)
    for name, res, args in SIGNATURES:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.smx_abi_version() != 1:
        raise ImportError("libsymmetrix_mi355x.so has an unexpected ABI version")
    return lib


lib = _load()


def check(rc):
    """Raise the Python exception of an SMX_ERR_* code."""
    if rc == SMX_OK:
        return
    msg = lib.smx_last_error().decode(errors="replace")
    if rc == SMX_ERR_INVALID_ARGUMENT:
        raise ValueError(msg)
    if rc == SMX_ERR_UNSUPPORTED:
        raise SymmetrixUnsupportedError(msg)
    if rc == SMX_ERR_OUT_OF_MEMORY:
        raise MemoryError(msg)
    raise RuntimeError(msg)


def ptr(a):
    """Address of a C-contiguous numpy array (None for an empty array)."""
    if a is None:
        return None
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("array must be C-contiguous")
    return a.ctypes.data if a.size else None


def i32(a):
    return np.ascontiguousarray(a, dtype=np.int32).reshape(-1)


def f64(a):
    return np.ascontiguousarray(a, dtype=np.float64).reshape(-1)


def model_array(model_path, name):
    """A model array in an operator module's layout (smx_model_array_f32/i32):
    float32 "M0_weights", "H0", "R0_spline" (returned with the grid h, x0) or
    int32 "M0_terms", "M0_offsets"."""
    is_int = name in ("M0_terms", "M0_offsets")
    count, dims = ctypes.c_int64(), (ctypes.c_int32 * 4)()
    h, x0 = ctypes.c_double(), ctypes.c_double()
    path = str(model_path).encode()
    if is_int:
        check(lib.smx_model_array_i32(path, name.encode(), None, 0, ctypes.byref(count), dims))
    else:
        check(lib.smx_model_array_f32(path, name.encode(), None, 0, ctypes.byref(count), dims, None, None))
    shape = tuple(d for d in dims if d > 0)
    out = np.empty(count.value, dtype=np.int32 if is_int else np.float32)
    if is_int:
        check(lib.smx_model_array_i32(path, name.encode(), ptr(out), out.size, ctypes.byref(count), dims))
        return out.reshape(shape)
    check(lib.smx_model_array_f32(path, name.encode(), ptr(out), out.size, ctypes.byref(count), dims,
                                  ctypes.byref(h), ctypes.byref(x0)))
    if name == "R0_spline":
        return out.reshape(shape), h.value, x0.value
    return out.reshape(shape)
