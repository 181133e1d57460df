/*
 * symmetrix_operator_modules.h -- the reference's M0 / R0 operator-module
 * container, built from this project's gfx950 kernels.
 *
 * The reference loads its product-basis (M0) and first-interaction radial
 * (R0) operators as HIP code objects (OperatorModule::load,
 * libsymmetrix/source/jit_operator_module.cpp:236-373; expectations built in
 * mace_kokkos_runtime.cpp:1030-1062 and :1230-1257).  A code object is
 * accepted when it defines these device symbols with the expected values:
 *
 *   symmetrix_operator_abi_version_v1        uint32  (1)
 *   symmetrix_operator_kind_v1               uint32  (1 M0, 2 R0)
 *   symmetrix_operator_scalar_kind_v1        uint32  (1 FP32, 2 FP64)
 *   symmetrix_operator_scalar_size_v1        uint32
 *   symmetrix_operator_capabilities_v1       uint32  (bits below)
 *   symmetrix_operator_input_components_v1   int32
 *   symmetrix_operator_output_components_v1  int32
 *   symmetrix_operator_correlation_v1        int32
 *   symmetrix_operator_term_count_v1         int32
 *   symmetrix_operator_threads_v1            int32   (block size of every launch)
 *   symmetrix_operator_artifact_id_v1            char[] (NUL-terminated, < 512 B)
 *   symmetrix_operator_structure_fingerprint_v1  char[]
 *   symmetrix_operator_target_v1                 char[]
 *
 * and these kernels, each taking its argument packet by value:
 *   M0: symmetrix_m0_forward_v1(SymmetrixJitM0ArgsV1),
 *       symmetrix_m0_reverse_v1(SymmetrixJitM0ArgsV1);
 *   R0: symmetrix_r0_density_prepare_v1, symmetrix_r0_forward_v1,
 *       symmetrix_r0_reverse_prepare_v1, symmetrix_r0_coordinate_reverse_v1
 *       (SymmetrixJitR0ArgsV1).
 * The loader launches min(ceil(work / threads), persistent_blocks) blocks
 * (jit_device_plugin_common.hpp:146-156), so every kernel is written for any
 * grid size.  symmetrix/operator_modules.py renders and compiles such a code
 * object for a model's contract (hipcc --genco, gfx950); the Makefile builds
 * the compiled shapes' modules with test identities.
 *
 * The argument packets below are the reference's (jit_operator_module_abi.h:
 * 5-79), byte for byte: M0 80 B, spline 40 B, R0 256 B.  They are skipped
 * when the reference's header was included first.
 */
#ifndef SYMMETRIX_OPERATOR_MODULES_H
#define SYMMETRIX_OPERATOR_MODULES_H

#include <stdint.h>

#include "symmetrix_mi355x.h"

#ifdef __cplusplus
extern "C" {
#endif

#ifndef SYMMETRIX_JIT_OPERATOR_ABI_VERSION_V1
#define SYMMETRIX_JIT_OPERATOR_ABI_VERSION_V1 1u
#define SYMMETRIX_JIT_OPERATOR_KIND_M0_V1 1u
#define SYMMETRIX_JIT_OPERATOR_KIND_R0_V1 2u
#define SYMMETRIX_JIT_OPERATOR_SCALAR_FLOAT32_V1 1u
#define SYMMETRIX_JIT_OPERATOR_SCALAR_FLOAT64_V1 2u

#define SYMMETRIX_JIT_OPERATOR_M0_FORWARD_V1 (1u << 0)
#define SYMMETRIX_JIT_OPERATOR_M0_REVERSE_V1 (1u << 1)
#define SYMMETRIX_JIT_OPERATOR_M0_ALIAS_SAFE_V1 (1u << 2)
#define SYMMETRIX_JIT_OPERATOR_M0_SCALE_ADJOINT_V1 (1u << 3)
#define SYMMETRIX_JIT_OPERATOR_M0_RESPONSE_REVERSE_V1 (1u << 4)

#define SYMMETRIX_JIT_OPERATOR_R0_DENSITY_PREPARE_V1 (1u << 8)
#define SYMMETRIX_JIT_OPERATOR_R0_FORWARD_V1 (1u << 9)
#define SYMMETRIX_JIT_OPERATOR_R0_REVERSE_PREPARE_V1 (1u << 10)
#define SYMMETRIX_JIT_OPERATOR_R0_COORDINATE_REVERSE_V1 (1u << 11)
#define SYMMETRIX_JIT_OPERATOR_R0_COMPACT_GEOMETRY_V1 (1u << 12)
#define SYMMETRIX_JIT_OPERATOR_R0_PRECOMPUTED_SCALE_V1 (1u << 13)
#define SYMMETRIX_JIT_OPERATOR_R0_RECEIVER_BATCH_V1 (1u << 14)

/* M0: output[i][LM][k] = sum_t weights[type_i][t][k] * monomial_t(input[i][:][k]);
 * reverse: input_adjoint[i][v][k] = sum_LM output_adjoint[i][LM][k] dM0/dinput
 * (assigned), and with capture_input_scale_adjoint, input_scale_adjoint[i] +=
 * sum_{v,k} input * input_adjoint (FP64). */
typedef struct SymmetrixJitM0ArgsV1 {
    uint32_t struct_size;
    uint32_t reserved;
    int64_t num_nodes;
    int32_t channels;
    int32_t capture_input_scale_adjoint;
    const int32_t* node_types;
    const void* input;          /* [N][input_components][C] */
    const void* weights;        /* [types][term_count][C] */
    const void* output_adjoint; /* [N][output_components][C] (reverse) */
    void* output;               /* [N][output_components][C] (forward) */
    void* input_adjoint;        /* [N][input_components][C] (reverse) */
    double* input_scale_adjoint; /* [N] */
} SymmetrixJitM0ArgsV1;

/* coefficients [edge_types][intervals][4][functions] */
typedef struct SymmetrixJitR0SplineV1 {
    uint32_t struct_size;
    uint32_t edge_types;
    uint32_t intervals;
    uint32_t functions;
    double h;
    double x0;
    const void* coefficients;
} SymmetrixJitR0SplineV1;

/* R0: output[i][lm][k] = s_i sum_{e in N(i), r_e < cutoff} R_{l,k}(r_e) Y_lm(e)
 * with the ordered-pair radial table (edge type receiver*n + neighbour) and
 * s_i the density scale when apply_density_scale (density_state, prepared
 * by the density kernel); coordinate reverse: directed_forces[e] -= the
 * edge's force from output_adjoint (+ the density-scale term). */
typedef struct SymmetrixJitR0ArgsV1 {
    uint32_t struct_size;
    uint32_t receiver_base;
    int64_t num_nodes;
    int64_t num_edges;
    int32_t active_type_count;
    int32_t channels;
    int32_t l_max;
    int32_t coordinates_are_unit;
    int32_t apply_density_scale;
    int32_t use_precomputed_scale_adjoint;
    const int32_t* node_types;
    const int32_t* num_neigh;
    const int32_t* first_neigh;
    const int32_t* neigh_types;
    const int32_t* edge_receivers;
    const int32_t* type_to_active;
    const void* coordinates;        /* FP64 xyz [E][3], or FP32 unit vectors */
    const double* radius;           /* [E] */
    SymmetrixJitR0SplineV1 radial;  /* Precision */
    SymmetrixJitR0SplineV1 density; /* FP64, symmetric pair types */
    const void* harmonics;          /* [E][(l_max+1)^2] */
    const void* harmonic_gradients; /* [E][3][(l_max+1)^2], or NULL: from the coordinates */
    void* output;                   /* [N][(l_max+1)^2][C] */
    void* output_adjoint;           /* [N][(l_max+1)^2][C] */
    double* density_state;          /* [N] */
    const double* precomputed_scale_adjoint; /* [N] */
    double* directed_forces;        /* [E][3] */
    double cutoff;
} SymmetrixJitR0ArgsV1;
#endif /* SYMMETRIX_JIT_OPERATOR_ABI_VERSION_V1 */

/* No counterpart in the reference (its JIT reads the model's contract in
 * Python): arrays of a model file that an operator module's caller passes,
 * in the module layouts, as float32 / int32.  name:
 *   "M0_weights"  [types][terms][C]      (dims = types, terms, C)
 *   "M0_terms"    packed monomials (variables in bytes 0..2, degree in
 *                 byte 3), canonical order   (dims = terms)
 *   "M0_offsets"  per-output term ranges      (dims = outputs + 1)
 *   "R0_spline"   [intervals][4][(l_max+1) C] (dims = intervals, 4, functions);
 *                 grid in *h, *x0 (may be NULL)
 *   "H0"          node embedding [types][C]  (dims = types, C)
 * With out == NULL only dims and *count are filled.  Returns SMX_OK or
 * SMX_ERR_*. */
SMX_API int32_t smx_model_array_f32(const char* model_path, const char* name, float* out, int64_t capacity,
                                    int64_t* count, int32_t dims[4], double* h, double* x0);
SMX_API int32_t smx_model_array_i32(const char* model_path, const char* name, int32_t* out, int64_t capacity,
                                    int64_t* count, int32_t dims[4]);

#ifdef __cplusplus
}
#endif

#endif /* SYMMETRIX_OPERATOR_MODULES_H */
