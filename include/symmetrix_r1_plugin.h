/*
 * symmetrix_r1_plugin.h -- the reference's R1 HIP plugin ABI, exported by
 * libsymmetrix_mi355x.so.
 *
 * The reference evaluator loads its R1 operator (the second interaction's
 * forward and coordinate reverse) from a shared library through
 * `symmetrix_jit_hip_plugin_query_v1` (libsymmetrix/source/jit_hip_plugin.cpp:273-301,
 * mace_kokkos.hpp:107).  This library exports that symbol with the same
 * descriptor and argument-packet layouts (jit_hip_plugin_abi.h:28-269), so
 * the reference's loader can bind the MI355X kernels in place of a JIT-built
 * plugin.  The layouts must match the reference byte for byte; the
 * declarations below are skipped when the reference's own header was
 * included first.
 *
 * Difference from a JIT artefact: one library serves every model of a
 * compiled shape, so the model is chosen at run time with
 * smx_r1_plugin_configure (before the loader calls the query; the query
 * returns NULL until then).  The descriptor's identity strings are the ones
 * the caller passes there, because they name the caller's model contract.
 *
 * Launch semantics (as the reference's generated launchers,
 * jit_codegen.py:3346-3410):
 *   r1_forward_launch: output[i][lme][k] = Phi1 of receiver i (assigned);
 *   r1_coordinate_reverse_launch: source_adjoint[s][lm2][k] += the R1
 *     source adjoint (FP64 sums, added in FP32) and directed_forces[e][c] -=
 *     the edge's R1 force (FP64);
 *   both enqueue on the caller's stream, retain no argument pointer, return
 *   the numeric hipError_t (hipErrorInvalidValue for malformed packets) and
 *   never throw.  Edges with radius >= cutoff are skipped.  The reverse
 *   expects edge_receivers non-decreasing (receiver-major edges, as the
 *   reference's prepared graph orders them) and harmonics_gradients
 *   present.  Its per-edge workspace (receiver offsets and source terms,
 *   4*(N+1) + E*n_H*C*4 bytes) belongs to the configured model and only
 *   grows: a launch on a larger graph than any before reallocates it (after
 *   the previous launch that used it has finished), so callers that must
 *   not allocate inside a launch size it first with smx_r1_plugin_reserve.
 *   Launches of one model on different streams are ordered through an event
 *   on that workspace.
 * Each configure call binds its descriptor's launchers to that model: a
 * loader that keeps an earlier descriptor keeps launching the earlier model
 * (at most 8 models per process).
 */
#ifndef SYMMETRIX_R1_PLUGIN_H
#define SYMMETRIX_R1_PLUGIN_H

#include <stdint.h>

#include "symmetrix_mi355x.h"

#ifdef __cplusplus
extern "C" {
#endif

#ifndef SYMMETRIX_JIT_HIP_PLUGIN_ABI_VERSION_V1
#define SYMMETRIX_JIT_HIP_PLUGIN_ABI_VERSION_V1 1u
#define SYMMETRIX_JIT_HIP_PLUGIN_BYTE_ORDER 0x01020304u
#define SYMMETRIX_JIT_HIP_PLUGIN_ABI_TAG_V1 "symmetrix.jit.hip-plugin/1"
#define SYMMETRIX_JIT_HIP_PLUGIN_QUERY_SYMBOL_V1 "symmetrix_jit_hip_plugin_query_v1"

enum SymmetrixJitHipScalarKindV1 {
    SYMMETRIX_JIT_HIP_SCALAR_FLOAT32_V1 = 1u,
    SYMMETRIX_JIT_HIP_SCALAR_FLOAT64_V1 = 2u,
};

enum SymmetrixJitHipPluginCapabilityV1 {
    SYMMETRIX_JIT_HIP_R1_FORWARD_LAUNCH_V1 = 1u << 0,
    SYMMETRIX_JIT_HIP_R1_COORDINATE_REVERSE_LAUNCH_V1 = 1u << 1,
    SYMMETRIX_JIT_HIP_R1_FUSED_REVERSE_LAUNCH_V1 = 1u << 2,
};

/* spline coefficients [edge_types][intervals][4][functions] (Precision) */
typedef struct SymmetrixJitHipRadialSplineV1 {
    uint32_t struct_size;
    uint32_t edge_types;
    uint32_t intervals;
    uint32_t functions;
    double h;
    double x0;
    const void* coefficients;
} SymmetrixJitHipRadialSplineV1;

typedef struct SymmetrixJitHipR1ForwardArgsV1 {
    uint32_t struct_size;
    uint32_t active_type_count;
    int64_t num_nodes;
    int64_t num_edges;
    const int32_t* node_types;
    const int32_t* num_neigh;
    const int32_t* first_neigh;
    const int32_t* neigh_indices;
    const int32_t* neigh_types;
    const int32_t* type_to_active;
    const double* radius;
    SymmetrixJitHipRadialSplineV1 radial;
    const void* harmonics_values;  /* [E][n_Y] */
    const void* neighbor_features; /* [N][n_H][C] */
    void* output;                  /* [N][n_lme][C] */
    double cutoff;
} SymmetrixJitHipR1ForwardArgsV1;

typedef struct SymmetrixJitHipR1SourceArgsV1 {
    uint32_t struct_size;
    uint32_t active_type_count;
    int64_t num_nodes;
    int64_t num_edges;
    const int32_t* node_types;
    const int32_t* neigh_types;
    const int32_t* source_offsets;
    const int32_t* source_edges;
    const int32_t* edge_receivers;
    const int32_t* type_to_active;
    const double* radius;
    SymmetrixJitHipRadialSplineV1 radial;
    const void* harmonics_values;
    const void* output_adjoint; /* [N][n_lme][C] */
    void* source_adjoint;       /* [N][n_H][C] */
    double cutoff;
} SymmetrixJitHipR1SourceArgsV1;

typedef struct SymmetrixJitHipR1EdgeArgsV1 {
    uint32_t struct_size;
    uint32_t active_type_count;
    uint32_t coordinate_scalar_size;
    uint32_t coordinates_are_unit;
    int64_t num_nodes;
    int64_t num_edges;
    const int32_t* node_types;
    const int32_t* neigh_indices;
    const int32_t* neigh_types;
    const int32_t* edge_receivers;
    const int32_t* type_to_active;
    const void* xyz;                 /* [E][3]: FP64 vectors, or unit vectors when coordinates_are_unit */
    const double* radius;
    SymmetrixJitHipRadialSplineV1 radial;
    const void* harmonics_values;
    const void* harmonics_gradients; /* [E][3][n_Y] */
    const void* neighbor_features;
    const void* output_adjoint;
    double* directed_forces;         /* [E][3] */
    double cutoff;
} SymmetrixJitHipR1EdgeArgsV1;

typedef int32_t (*SymmetrixJitHipR1ForwardLaunchV1)(const SymmetrixJitHipR1ForwardArgsV1*, void*, int32_t);
typedef int32_t (*SymmetrixJitHipR1CoordinateReverseLaunchV1)(const SymmetrixJitHipR1SourceArgsV1*,
                                                              const SymmetrixJitHipR1EdgeArgsV1*, void*, int32_t);

typedef struct SymmetrixJitHipPluginV1 {
    uint32_t abi_version;
    uint32_t struct_size;
    uint32_t pointer_size;
    uint32_t byte_order;
    uint32_t capabilities;
    uint32_t scalar_kind;
    uint32_t scalar_size;
    uint32_t reserved;
    const char* abi_tag;
    const char* artifact_id;
    const char* contract_fingerprint;
    const char* semantic_fingerprint;
    const char* structure_fingerprint;
    int32_t channels;
    int32_t embedding;
    int32_t edge_l_max;
    int32_t source_l_max;
    const char* target_architecture;
    const char* target_features;
    int32_t native_subgroup_width;
    int32_t forward_threads_per_block;
    int32_t source_threads_per_block;
    int32_t edge_threads_per_block;
    int32_t persistent_blocks_per_compute_unit;
    SymmetrixJitHipR1ForwardLaunchV1 r1_forward_launch;
    SymmetrixJitHipR1CoordinateReverseLaunchV1 r1_coordinate_reverse_launch;
} SymmetrixJitHipPluginV1;
#endif /* SYMMETRIX_JIT_HIP_PLUGIN_ABI_VERSION_V1 */

/* symmetrix_jit_hip_plugin_query_v1 (jit_hip_plugin_abi.h:265-269): the
 * descriptor of the configured model, or NULL before smx_r1_plugin_configure
 * has succeeded. */
SMX_API const SymmetrixJitHipPluginV1* symmetrix_jit_hip_plugin_query_v1(void);

/* Identity the descriptor reports (the caller's model contract) and launch
 * options.  Strings are copied. */
typedef struct SmxR1PluginIdentity {
    uint32_t struct_size;
    const char* artifact_id;
    const char* contract_fingerprint;
    const char* semantic_fingerprint;
    const char* structure_fingerprint;
    const char* target_features;        /* NULL = "" */
    int32_t embedding;                  /* embedding width the loader expects (> 0) */
    int32_t fp64_evaluation_point;      /* 0: spline point formed in FP32 (precision matched), 1: FP64 */
    int32_t persistent_blocks_per_compute_unit; /* > 0 */
} SmxR1PluginIdentity;

/* No counterpart in the reference (a JIT artefact is built per model): load
 * the model file whose R1 coupling the plugin applies, select the compiled
 * kernels of its shape (channels, l_max, L_max) and fill the descriptor.
 * Uses the current HIP device.  Returns SMX_OK or SMX_ERR_*. */
SMX_API int32_t smx_r1_plugin_configure(const char* model_path, const SmxR1PluginIdentity* identity);

/* No counterpart in the reference (its generated launchers keep no
 * workspace): size the reverse workspace of `plugin`'s model for graphs of
 * up to num_nodes receivers and num_edges edges, so that later reverse
 * launches of that size allocate nothing (e.g. before a caller captures them
 * into a HIP graph).  A reverse launch on a larger graph grows the workspace
 * itself.  Returns SMX_OK or SMX_ERR_*. */
SMX_API int32_t smx_r1_plugin_reserve(const SymmetrixJitHipPluginV1* plugin, int64_t num_nodes, int64_t num_edges);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): the coordinate reverse of `plugin`'s model, with the
 * same arguments, kernels and results as its r1_coordinate_reverse_launch,
 * but with the workspace (receiver offsets and per-edge source terms,
 * 4*(N+1) rounded up to 256 B, plus E*n_H*C*4 bytes) in a fixed 256 MiB
 * device array of the library instead of allocated memory: up to about
 * 512k edges at 32 channels and L_max 1, 131k edges at 128 channels.  Larger
 * graphs are refused with hipErrorInvalidValue and a message in
 * smx_last_error().  It calls no allocating routine.  The array is the
 * current device's (each GPU holds its own copy for the life of the
 * process); every call on a GPU shares it, so calls that overlap on one GPU
 * (several streams, or host threads) race and must be serialised by the
 * caller.  Returns the numeric hipError_t. */
SMX_API int32_t smx_r1_plugin_reverse_launch_noalloc(const SymmetrixJitHipPluginV1* plugin,
                                                     const SymmetrixJitHipR1SourceArgsV1* source_args,
                                                     const SymmetrixJitHipR1EdgeArgsV1* edge_args, void* stream,
                                                     int32_t persistent_blocks);

/* No counterpart in the reference: the configured model's R1 spline table in
 * the plugin layout [1][intervals][4][functions] (FP32; one edge type, the
 * radial networks' tabulation being the same for every type pair), with its
 * grid.  With out == NULL only the sizes are returned. */
SMX_API int32_t smx_r1_plugin_spline_table(float* out, int64_t capacity, int32_t* intervals, int32_t* functions,
                                           double* h, double* x0);

#ifdef __cplusplus
}
#endif

#endif /* SYMMETRIX_R1_PLUGIN_H */
