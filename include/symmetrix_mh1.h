/*
 * symmetrix_mh1.h -- C ABI of the MI355X MH-1 (MACE_Nonlinear) evaluator
 * (libsymmetrix_mi355x.so).
 *
 * Each entry point replaces one member of the reference's nonlinear
 * evaluators `MaceNonlinear` (libsymmetrix/source/mace_nonlinear.hpp:14-50)
 * and `MACENonlinearKokkos<float>` (mace_nonlinear_kokkos.hpp) as the
 * reference's pybind module exposes them
 * (symmetrix/source/cpp/mace_nonlinear_kokkos.cpp:19-240: the constructor,
 * r_cut, selected_head, available_heads, is_mh1_family, mh1_node_channels,
 * mh1_edge_channels, mh1_radial_size, mh1_l_max, atomic_numbers,
 * atomic_energies, compute_node_energies_forces, node_energies,
 * node_forces), so a ctypes/cgo/JNI binding can stand in for the
 * `MACENonlinearKokkosFloat` class.
 *
 * Conventions are those of symmetrix_mi355x.h: plain host pointers and sizes,
 * 0 or a negative SMX_ERR_* code, no exceptions, smx_last_error() for the
 * message; one evaluator per host thread; device work on the evaluator's own
 * HIP stream.  The graph of a call is the reference's CSR neighbour list:
 * num_neigh[i] edges per receiver i in order, neigh_indices/neigh_types the
 * source atom and its type, xyz[e] = r_source - r_receiver (+ cell shift),
 * r[e] = |xyz[e]|.  node_forces[e] = -dE/dxyz[e] (FP64), the reference's
 * per-edge output (mace_nonlinear.cpp:983-996).
 */
#ifndef SYMMETRIX_MH1_H
#define SYMMETRIX_MH1_H

#include <stdint.h>

#include "symmetrix_mi355x.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct SmxMh1Evaluator SmxMh1Evaluator;

/* Model facts (pybind mace_nonlinear_kokkos.cpp:22-50). */
typedef struct SmxMh1Info {
    uint32_t struct_size;
    int32_t num_elements;     /* atomic_numbers.size() */
    int32_t l_max;
    int32_t num_interactions;
    int32_t is_mh1_family;    /* analyze_mh1_family_architecture (mace_nonlinear_schema.cpp:108-207) */
    int32_t node_channels;    /* mh1_node_channels (0 unless family) */
    int32_t edge_channels;    /* mh1_edge_channels */
    int32_t radial_size;      /* mh1_radial_size */
    int32_t has_zbl;
    double r_cut;
} SmxMh1Info;

/* MaceNonlinear(filename, head) (mace_nonlinear.cpp:260-264,302-380): loads a
 * "MACE_Nonlinear" JSON file (format 3 or 4).  head may be NULL or "". */
SMX_API int32_t smx_mh1_create(const char* model_path, const char* head, SmxMh1Evaluator** out);
SMX_API void smx_mh1_destroy(SmxMh1Evaluator* ev);
SMX_API int32_t smx_mh1_info(const SmxMh1Evaluator* ev, SmxMh1Info* info);
/* mh1_family_rejection_reason (mace_nonlinear.hpp:33): "" for family models. */
SMX_API int32_t smx_mh1_family_rejection(const SmxMh1Evaluator* ev, const char** reason);
/* atomic_numbers / atomic_energies (mace_nonlinear.hpp:19-20); returns the
 * count, writing at most capacity entries. */
SMX_API int32_t smx_mh1_atomic_numbers(const SmxMh1Evaluator* ev, int32_t* out, int32_t capacity);
SMX_API int32_t smx_mh1_atomic_energies(const SmxMh1Evaluator* ev, double* out, int32_t capacity);
/* selected_head (mace_nonlinear.hpp:21); "" when the file has none. */
SMX_API int32_t smx_mh1_selected_head(const SmxMh1Evaluator* ev, const char** name);

/* compute_node_energies_forces (mace_nonlinear.hpp:44-51,
 * mace_nonlinear.cpp:471-1010): the graph in host memory; the inputs are
 * checked as the reference checks them (sizes, types, counts, finite
 * geometry) before any device work. */
SMX_API int32_t smx_mh1_compute_node_energies_forces(SmxMh1Evaluator* ev, int32_t num_nodes,
                                                     const int32_t* node_types, const int32_t* num_neigh,
                                                     const int32_t* neigh_indices, const int32_t* neigh_types,
                                                     const double* xyz, const double* r, int64_t num_edges);
/* node_energies [num_nodes] and node_forces [num_edges][3] of the last call. */
SMX_API int32_t smx_mh1_node_energies(SmxMh1Evaluator* ev, double* out, int64_t capacity);
SMX_API int32_t smx_mh1_node_forces(SmxMh1Evaluator* ev, double* out, int64_t capacity);
/* Test hook: an intermediate FP32 stage of the last call ("up0", "msg0",
 * "density0", "features0", "w0", ... with the layer index last); *count gets
 * its size. */
SMX_API int32_t smx_mh1_debug_stage(SmxMh1Evaluator* ev, const char* name, float* out, int64_t capacity,
                                    int64_t* count);
/* Per-kernel time (ms) of the last call when timing is on (bench). */
SMX_API int32_t smx_mh1_set_kernel_timing(SmxMh1Evaluator* ev, int32_t enabled);
SMX_API int32_t smx_mh1_kernel_timing(SmxMh1Evaluator* ev, int32_t index, const char** name, double* total_ms,
                                      int64_t* launches);

#ifdef __cplusplus
}
#endif

#endif /* SYMMETRIX_MH1_H */
