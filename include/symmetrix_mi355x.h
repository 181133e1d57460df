/*
 * symmetrix_mi355x.h -- C ABI of the MI355X MACE evaluator
 * (libsymmetrix_mi355x.so).
 *
 * Each entry point replaces one member of the reference's C++ evaluator
 * `MACEKokkos<float>` (libsymmetrix/source/mace_kokkos.hpp:85-1838) as the
 * reference's pybind module exposes it (symmetrix/source/cpp/mace_kokkos.cpp),
 * so a ctypes/cgo/JNI binding can stand in for the `MACEKokkosFloat` class.
 * Conventions:
 *   - plain pointers and sizes; host pointers unless the name ends in _device;
 *   - every function returns 0 on success or a negative SMX_ERR_* code, and
 *     never throws; smx_last_error() holds the message of the calling thread's
 *     last failure (the reference raises std::invalid_argument /
 *     std::runtime_error / std::logic_error, which pybind maps to ValueError /
 *     RuntimeError);
 *   - one evaluator is driven from one host thread; all device work is
 *     ordered on the evaluator's own HIP stream (smx_evaluator_stream), and
 *     calls that return host data synchronise that stream first.
 * Units: positions and cell in Angstrom, energies in eV, forces eV/Angstrom,
 * stress eV/Angstrom^3 (3x3, row-major).
 */
#ifndef SYMMETRIX_MI355X_H
#define SYMMETRIX_MI355X_H

#include <stdint.h>

#if defined(__GNUC__)
#define SMX_API __attribute__((visibility("default")))
#else
#define SMX_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define SMX_ABI_VERSION 1

enum {
    SMX_OK = 0,
    SMX_ERR_INVALID_ARGUMENT = -1, /* bad input, stale graph generation (ValueError) */
    SMX_ERR_RUNTIME = -2,          /* HIP failure, invalid geometry (RuntimeError) */
    SMX_ERR_LOGIC = -3,            /* call out of order, e.g. no graph prepared */
    SMX_ERR_OUT_OF_MEMORY = -4,    /* device or host allocation failed */
    SMX_ERR_UNSUPPORTED = -5       /* model shape/features without a kernel set */
};

typedef struct SmxEvaluator SmxEvaluator;

/* Model facts: the fields the reference exposes as read-only attributes
 * (mace_kokkos.hpp:485-497; pybind mace_kokkos.cpp:2080-2083). */
typedef struct SmxModelInfo {
    uint32_t struct_size;
    int32_t num_elements;
    int32_t num_channels;
    int32_t l_max;
    int32_t L_max;
    int32_t num_interactions;
    int32_t num_paths;
    int32_t num_lme;
    double r_cut;
} SmxModelInfo;

/* Device addresses of the evaluator's result buffers (valid until the next
 * prepare call; FP64). */
typedef struct SmxDeviceOutputs {
    uint32_t struct_size;
    int32_t num_nodes;
    int64_t num_edges;
    const double* node_energies; /* [N] */
    const double* node_forces;   /* [E][3]: -dE/dxyz_e (NULL under the tiled plan) */
    const double* atom_forces;   /* [N][3] after smx_reduce_prepared_node_forces */
    const double* stress;        /* [3][3] after smx_reduce_prepared_stress */
    const double* total_energy;  /* [1] after smx_total_energy_device */
    const double* xyz;           /* [E][3] edge vectors of the last call */
    const double* r;             /* [E] edge lengths of the last call */
} SmxDeviceOutputs;

SMX_API int32_t smx_abi_version(void);
SMX_API const char* smx_last_error(void);

/* MACEKokkos(std::string filename, std::string head) -- mace_kokkos.hpp:91;
 * pybind MACEKokkosFloat(filename, head) (mace_kokkos.cpp:2762). */
SMX_API int32_t smx_evaluator_create(const char* model_path, const char* head, SmxEvaluator** out);
SMX_API void smx_evaluator_destroy(SmxEvaluator* ev);
SMX_API int32_t smx_evaluator_info(const SmxEvaluator* ev, SmxModelInfo* info);
/* atomic_numbers property (pybind mace_kokkos.cpp:1896) */
SMX_API int32_t smx_evaluator_atomic_numbers(const SmxEvaluator* ev, int32_t* out, int32_t capacity);
/* atomic_energies property (pybind mace_kokkos.cpp:1900-1903): E0 per
 * element, model order */
SMX_API int32_t smx_evaluator_atomic_energies(const SmxEvaluator* ev, double* out, int32_t capacity);
/* active_atomic_numbers property (pybind mace_kokkos.cpp:1906-1909;
 * lifecycle.cpp:4096-4101, mace.cpp:2738): the elements whose per-pair
 * radial tables are on the device (models with a distance transform; in
 * model type order), else every element of the model.  out NULL: count only. */
SMX_API int32_t smx_active_atomic_numbers(const SmxEvaluator* ev, int32_t* out, int32_t capacity, int32_t* count);
/* selected_head / available_heads (mace_kokkos.cpp:1904-1905): index -1 gives
 * the head in use ("" when the file names none), index 0.. the heads the
 * file stores (NULL past the end).  The strings live as long as ev. */
SMX_API int32_t smx_prediction_head(const SmxEvaluator* ev, int32_t index, const char** name);
/* set_streamed_edges (mace_kokkos.hpp:93); only "direct" is implemented. */
SMX_API int32_t smx_set_streamed_edges(SmxEvaluator* ev, const char* mode);
/* hipStream_t the evaluator enqueues on */
SMX_API void* smx_evaluator_stream(SmxEvaluator* ev);

/* prepare_factorized_graph (mace_kokkos.hpp:365-370; pybind
 * _prepare_factorized_graph, mace_kokkos.cpp:1561): receiver-major CSR on
 * the host.  Returns the graph generation token. */
SMX_API int32_t smx_prepare_factorized_graph(SmxEvaluator* ev, int32_t num_nodes, const int32_t* node_types,
                                             const int32_t* num_neigh, int64_t num_edges,
                                             const int32_t* neigh_indices, const int32_t* neigh_types,
                                             uint64_t* generation);
/* prepare_factorized_graph_device (mace_kokkos.hpp:387-392): same CSR,
 * device pointers (the LAMMPS pair style's entry, pair_symmetrix_mace_kokkos.cpp:1160). */
SMX_API int32_t smx_prepare_factorized_graph_device(SmxEvaluator* ev, int32_t num_nodes,
                                                    const int32_t* node_types_device,
                                                    const int32_t* num_neigh_device, int64_t num_edges,
                                                    const int32_t* neigh_indices_device,
                                                    const int32_t* neigh_types_device, uint64_t* generation);
/* prepare_periodic_factorized_graph (mace_kokkos.hpp:393-398; pybind
 * _prepare_periodic_factorized_graph, mace_kokkos.cpp:1580): device
 * neighbour list at neighbor_cutoff; the builder's wrapped fractional
 * positions and edge images are kept as the (fractional) geometry
 * reference, so the cell may change with smx_update_factorized_cell.
 * cell rows are lattice vectors; inverse_cell = inv(cell).  A graph of more
 * than 2^31 - 4096 edges (the reference's limit) is accepted up to
 * 2^32 - 2^20 edges and runs in the tiled plan, which indexes edges with
 * 64 bits; a request pinning a direct plan, or a MACEField model, is then
 * refused. */
SMX_API int32_t smx_prepare_periodic_factorized_graph(SmxEvaluator* ev, int32_t num_nodes, const int32_t* node_types,
                                                      const double* positions, const double* cell,
                                                      const double* inverse_cell, double neighbor_cutoff,
                                                      uint64_t* generation, int64_t* num_edges);
/* Plan shorthand with the tile size (no single counterpart; the receiver
 * tile limit is mace_kokkos.hpp:542's 32768): "speed" = the speed profile,
 * "capacity" = the model's tiled plan pinned (the reference's dual-layer
 * tiled plan, mace_kokkos_evaluate.cpp:755-1148, three sweeps; for a
 * one-interaction model its single-layer tiled plan, :614-752, one sweep) with at most tile_receivers
 * receivers per tile, "auto" = the capacity profile with fixed workspaces
 * allowed.  tile_receivers 0 keeps the current limit.  Applies to graphs
 * prepared afterwards. */
SMX_API int32_t smx_set_execution_plan(SmxEvaluator* ev, const char* profile, int32_t tile_receivers);
/* execution_plan description of the prepared graph (plan, polynomial kernels,
 * tiles) as one line of text */
SMX_API int32_t smx_execution_plan(SmxEvaluator* ev, char* out, int64_t capacity);
/* _set_execution_plan_request(algorithm, profile, debug_plan) (pybind
 * mace_kokkos.cpp:266-270; mace_kokkos.hpp:95-96): algorithm "direct"
 * ("factorized" and "direct_streamed" are its aliases), profile "capacity"
 * (the reference's default) or "speed", debug_plan "" (planner) or one of
 * "mh0-direct-speed", "mh0-direct-capacity-retained",
 * "mh0-dual-layer-tiled-v1" (two-interaction models) or
 * "mh0-single-layer-tiled-v1" (one-interaction models; a tiled plan pinned
 * for the other model kind is refused when the graph is prepared,
 * mace_kokkos_runtime.cpp:2996-3030) to pin a plan.  Under "capacity" the planner
 * selects the tiled plan only when fixed workspaces are allowed and the
 * retained workspace would exceed 70% of the available device memory.
 * Applies to graphs prepared afterwards. */
SMX_API int32_t smx_set_execution_plan_request(SmxEvaluator* ev, const char* algorithm, const char* profile,
                                               const char* debug_plan);
/* _set_allow_fixed_workspace (pybind mace_kokkos.cpp:444-445; the
 * calculator's allow_fixed_workspace): permit the planner to select the
 * tiled plan. */
SMX_API int32_t smx_set_allow_fixed_workspace(SmxEvaluator* ev, int32_t allow);
/* execution_plan_report (pybind mace_kokkos.cpp:271-297) as a JSON object:
 * requested_algorithm, requested_profile, selection_source, state,
 * selected_id, selection_reason, available_bytes, reserve_bytes,
 * candidates [{id, qualified, estimated_bytes, reason}].  *size receives the
 * bytes needed (with the terminating NUL); out may be NULL. */
SMX_API int32_t smx_execution_plan_report(SmxEvaluator* ev, char* out, int64_t capacity, int64_t* size);
/* Diagnostics counters (factorized_last_graph_prepare_ms and
 * factorized_last_evaluation_ms, pybind mace_kokkos.cpp:1045-1053): host
 * wall time of the last graph preparation and of the last evaluation call
 * (a device-positions call returns before its model kernels finish). */
typedef struct SmxEvaluatorCounters {
    uint32_t struct_size;
    uint32_t reserved;
    double last_graph_prepare_ms;
    double last_evaluation_ms;
    int64_t graph_prepare_count;
    int64_t evaluation_count;
    int64_t geometry_prepare_count;
} SmxEvaluatorCounters;
SMX_API int32_t smx_evaluator_counters(const SmxEvaluator* ev, SmxEvaluatorCounters* out);
/* prepare_active_types (pybind mace_kokkos.cpp:2076; lifecycle.cpp:3949):
 * tabulate the per-type-pair radial tables of these model types now (models
 * with a distance transform) and keep them for later graphs whose types they
 * cover. */
SMX_API int32_t smx_prepare_active_types(SmxEvaluator* ev, const int32_t* types, int32_t count);
/* update_factorized_cell (mace_kokkos.hpp:436; pybind _update_factorized_cell):
 * finite entries and a non-zero determinant are required, as in
 * mace_kokkos_factorized_lifecycle.cpp:2735-2766. */
SMX_API int32_t smx_update_factorized_cell(SmxEvaluator* ev, uint64_t generation, const double* cell,
                                           const double* inverse_cell);

/* Geometry of a prepared graph for positions calls (the reference's three
 * forms, mace_kokkos.hpp:415-435; pybind _prepare_factorized_geometry,
 * _prepare_factorized_shift_geometry, _prepare_factorized_fractional_geometry,
 * mace_kokkos.cpp:1608-1672; lifecycle.cpp:2455-2733).  Each positions call
 * then forms, per atom, delta = position - reference position (the latter
 * times the cell when fractional), wrapped to the minimum image along the
 * axes with pbc[k] != 0, and per edge xyz = reference edge vector +
 * delta[src] - delta[rcv], with r >= r_cut clamped.  Counts are numbers of
 * values: positions_count = 3 N, xyz/shifts_count = 3 E of the graph.
 *   - Cartesian: reference positions and reference xyz per edge, any pbc;
 *   - fractional: fractional positions and fractional xyz per edge (edge
 *     vector = frac . cell), fully periodic and invertible cell; the cell may
 *     then change with smx_update_factorized_cell (affine strain);
 *   - shift: reference positions and integer cell shifts per edge (edge
 *     vector = pos[src] - pos[rcv] + shift . cell); only under the tiled
 *     plan, as the reference requires.
 * Non-finite values or mismatched extents: SMX_ERR_INVALID_ARGUMENT. */
SMX_API int32_t smx_prepare_factorized_geometry(SmxEvaluator* ev, uint64_t generation,
                                                const double* reference_positions, int64_t positions_count,
                                                const double* reference_xyz, int64_t xyz_count, const double* cell,
                                                const double* inverse_cell, const int32_t* pbc);
SMX_API int32_t smx_prepare_factorized_shift_geometry(SmxEvaluator* ev, uint64_t generation,
                                                      const double* reference_positions, int64_t positions_count,
                                                      const int32_t* shifts, int64_t shifts_count,
                                                      const double* cell, const double* inverse_cell,
                                                      const int32_t* pbc);
SMX_API int32_t smx_prepare_factorized_fractional_geometry(SmxEvaluator* ev, uint64_t generation,
                                                           const double* fractional_positions,
                                                           int64_t positions_count, const double* fractional_xyz,
                                                           int64_t xyz_count, const double* cell,
                                                           const double* inverse_cell, const int32_t* pbc);

/* compute_prepared_factorized(token, xyz, r) (mace_kokkos.hpp:440-443):
 * energies and directed forces from host edge vectors xyz[E][3], r[E]. */
SMX_API int32_t smx_compute_prepared_factorized(SmxEvaluator* ev, uint64_t generation, const double* xyz,
                                                const double* r);
/* compute_prepared_factorized_positions(token, positions) (mace_kokkos.hpp:444-446;
 * pybind _compute_prepared_factorized_positions, mace_kokkos.cpp:1828) */
SMX_API int32_t smx_compute_prepared_factorized_positions(SmxEvaluator* ev, uint64_t generation,
                                                          const double* positions);
/* same with positions[N][3] already in device memory.  Returns once the
 * edge geometry has been checked (an invalid edge raises, as the reference's
 * streamed-positions path does, mace_kokkos_factorized_lifecycle.cpp:790-794);
 * the model kernels stay queued on the evaluator stream, so device outputs
 * are ready for work ordered on that stream or after smx_synchronize. */
SMX_API int32_t smx_compute_prepared_factorized_positions_device(SmxEvaluator* ev, uint64_t generation,
                                                                 const double* positions_device);
/* The calculator's call in one.  No counterpart in the reference, whose
 * calculator makes these calls in turn (calculator.py:3821-3894:
 * _compute_prepared_factorized_positions, node_energies,
 * _reduce_atom_forces, _reduce_stress): host positions (3 * num_nodes) in,
 * node energies (num_nodes), atom forces (3 * num_feature_nodes) and, with
 * stress != NULL, the 3x3 stress of a cell of that volume out, through
 * pinned staging and one wait for the device.  The refusals are those of
 * smx_compute_prepared_factorized_positions and smx_reduce_prepared_stress. */
SMX_API int32_t smx_compute_prepared_factorized_positions_results(SmxEvaluator* ev, uint64_t generation,
                                                                  const double* positions, double volume,
                                                                  double* node_energies, double* forces,
                                                                  double* stress);
/* Graphs with ghost feature nodes: one GPU's share of a domain-decomposed
 * system (the LAMMPS multi-rank path, pair_symmetrix_mace_kokkos.cpp:
 * 1285-1704).  prepare_factorized_graph with feature nodes
 * (mace_kokkos.hpp:378-386, 399-413; mace_kokkos_factorized_lifecycle.cpp:
 * 949-1104, 2346-2380): num_receivers receivers, each the feature node
 * receiver_feature_indices[ii] (unique, same type), num_feature_nodes >=
 * num_receivers feature nodes of types feature_types, and edges that leave
 * any feature node (neigh_indices are feature indices; each neighbour type
 * must equal its feature node's).  Such a graph takes explicit edge vectors
 * (no prepared positions geometry), runs the retained direct plan, and is
 * evaluated by the split-phase calls below (a one-interaction model also by
 * the plain xyz call).  The node forces reduced by
 * smx_reduce_prepared_node_forces are the feature nodes' (3 *
 * num_feature_nodes doubles, caller order; ghosts' forces are the caller's
 * to return to their owners).  A field-coupled model exchanges H1 before
 * its field (H1p = M0 P + b) and the adjoint of that; the field paths and
 * linear_up run over every feature node, a per-node field
 * (smx_set_electric_field) has 3 values per feature node in the caller's
 * order, and smx_electric_field_adj returns this rank's part of dE/dE (the
 * ranks' parts sum to the whole). */
SMX_API int32_t smx_prepare_factorized_feature_graph(SmxEvaluator* ev, int32_t num_receivers,
                                                     int32_t num_feature_nodes,
                                                     const int32_t* receiver_feature_indices,
                                                     const int32_t* node_types, const int32_t* feature_types,
                                                     const int32_t* num_neigh, int64_t num_edges,
                                                     const int32_t* neigh_indices, const int32_t* neigh_types,
                                                     uint64_t* generation);
/* same arrays in device memory (checked on host copies) */
SMX_API int32_t smx_prepare_factorized_feature_graph_device(SmxEvaluator* ev, int32_t num_receivers,
                                                            int32_t num_feature_nodes,
                                                            const int32_t* receiver_feature_indices,
                                                            const int32_t* node_types, const int32_t* feature_types,
                                                            const int32_t* num_neigh, int64_t num_edges,
                                                            const int32_t* neigh_indices,
                                                            const int32_t* neigh_types, uint64_t* generation);
/* compute_factorized_single_layer_distributed_evaluation (mace_kokkos.hpp:
 * 683-688; mace_kokkos_evaluate.cpp:1495-1552): a one-interaction model over
 * a feature graph in one call (no features are exchanged); xyz[E][3] and
 * r[E] on the host or (on_device != 0) in device memory. */
SMX_API int32_t smx_compute_factorized_single_layer_distributed_evaluation(SmxEvaluator* ev, uint64_t generation,
                                                                           int32_t num_receivers,
                                                                           int32_t num_feature_nodes,
                                                                           const double* xyz, const double* r,
                                                                           int32_t on_device);
/* The positions forms (mace_kokkos.hpp:678-682, 689-693;
 * mace_kokkos_evaluate.cpp:1554-1656): instead of edge vectors, the
 * positions of the feature nodes (3 per node, caller feature order, host or
 * device); each edge vector is x[source] - x[receiver], scaled to r_cut when
 * longer, as the pair style forms them, in whichever plan the graph runs.
 * Only for graphs prepared with feature nodes (the ghosts are explicit
 * atoms there, so no cell shift is needed). */
SMX_API int32_t smx_begin_factorized_distributed_positions_evaluation(SmxEvaluator* ev, uint64_t generation,
                                                                      int32_t num_receivers,
                                                                      int32_t num_feature_nodes,
                                                                      const double* feature_positions,
                                                                      int32_t on_device);
SMX_API int32_t smx_compute_factorized_single_layer_distributed_positions_evaluation(
    SmxEvaluator* ev, uint64_t generation, int32_t num_receivers, int32_t num_feature_nodes,
    const double* feature_positions, int32_t on_device);
/* The split-phase evaluation of a two-interaction model
 * (mace_kokkos.hpp:672-697; mace_kokkos_evaluate.cpp:1658-1990):
 *  1. begin: layer 1 up to H1 of the receivers (smx_distributed_exchange
 *     which=0: num_receivers rows, receiver order);
 *  2. the caller fills H1 of every feature node (its receivers' rows placed
 *     at their feature indices, the ghosts' from their owners) and calls
 *     continue with those num_feature_nodes rows (caller feature order): layer
 *     2, energies, and the H1 adjoint of every feature node
 *     (smx_distributed_exchange which=1: num_feature_nodes rows, caller
 *     feature order, in device memory the caller may add into);
 *  3. the caller adds each ghost row's adjoint into its owner's row and calls
 *     finish, with those rows or (h1_adjoint NULL) the exchange buffer as
 *     changed in place: the layer-1 reverse and the edge forces.
 * A row is row_floats FP32 values (num_LM x the evaluator's channel count;
 * H1p rows for a field-coupled model);
 * callers copy rows whole.  Each phase returns with its outputs complete.
 * Every other call on the evaluator is refused while a phase is pending;
 * an error resets the phases. */
SMX_API int32_t smx_begin_factorized_distributed_evaluation(SmxEvaluator* ev, uint64_t generation,
                                                            int32_t num_receivers, int32_t num_feature_nodes,
                                                            const double* xyz, const double* r, int32_t on_device);
SMX_API int32_t smx_continue_factorized_distributed_evaluation(SmxEvaluator* ev, const float* communicated_h1,
                                                               int64_t rows, int32_t on_device);
SMX_API int32_t smx_finish_factorized_distributed_evaluation(SmxEvaluator* ev, const float* h1_adjoint,
                                                             int64_t rows, int32_t on_device);
/* the rows a phase leaves for the exchange (which 0: receivers' H1 after
 * begin; 1: feature nodes' H1 adjoint after continue): device pointer, row
 * count and FP32 values per row; the pair style's H1 / H1_adj views
 * (pair_symmetrix_mace_kokkos.cpp:1582-1600, 1690-1704).  With device_rows
 * and rows both NULL it reports row_floats alone, in any phase.  The
 * pointer is into the evaluator's workspace: valid until the next phase
 * call, graph or evaluation on this evaluator. */
SMX_API int32_t smx_distributed_exchange(SmxEvaluator* ev, int32_t which, float** device_rows, int64_t* rows,
                                         int64_t* row_floats);
/* MACEField models (field_coupling.hpp; mace.cpp:322-395, 1147-1240).
 * _compute_prepared_factorized_positions_field(token, positions,
 * electric_field) and _compute_prepared_factorized_field(token, xyz, r,
 * electric_field) (pybind mace_kokkos.cpp:1837-1864): the positions and xyz
 * evaluations of a field-coupled model in an electric field of 3 values (one
 * field for the graph) or 3 per node (field_count 3 or 3*num_nodes).  The
 * field stays set for later evaluations (the plain entry points and the
 * LAMMPS entry).  A model without field coupling refuses a field; a
 * field-coupled model refuses an evaluation without one, and the tiled plans
 * (mace_kokkos_runtime.cpp:3005, 3042). */
SMX_API int32_t smx_compute_prepared_factorized_positions_field(SmxEvaluator* ev, uint64_t generation,
                                                                const double* positions, const double* field,
                                                                int64_t field_count);
SMX_API int32_t smx_compute_prepared_factorized_field(SmxEvaluator* ev, uint64_t generation, const double* xyz,
                                                      const double* r, const double* field, int64_t field_count);
/* the field of later evaluations (the pair style's electric_field Ex Ey Ez
 * keyword, pair_symmetrix_mace_kokkos.cpp:207-224); field_count 0 clears it */
SMX_API int32_t smx_set_electric_field(SmxEvaluator* ev, const double* field, int64_t field_count);
/* electric_field_adj (pybind mace_kokkos.cpp:2156): dE/dE of the last field
 * evaluation, shaped like its field (3, or 3 per node); FP64 sums.  *count
 * gets the length; copies when out != NULL and capacity is large enough. */
SMX_API int32_t smx_electric_field_adj(SmxEvaluator* ev, double* out, int64_t capacity, int64_t* count);
/* has_field_coupling (the model file's flag, mace.cpp:2832) */
SMX_API int32_t smx_has_field_coupling(const SmxEvaluator* ev, int32_t* out);
/* MACEField response: _compute_prepared_factorized_field_response(token,
 * electric_field, include_force_derivative, scatter_bec_bins) (pybind
 * mace_kokkos.cpp:1865-1879; mace_kokkos_response.tpp:2504-2543, the tangents
 * :136-2343).  Runs after a completed field evaluation of the current graph
 * token, in the same graph-level field (field_count 3; a field that differs
 * from that evaluation's is refused, as is a per-node field, a feature
 * graph with ghosts, a one-interaction model and a stale token): the field
 * Hessian d2E/dE_c dE_s (smx_electric_field_hessian) and, with
 * include_force_derivative, the directed forces' field derivative per edge
 * (smx_electric_field_force_derivative) or, with scatter_bec_bins too, its
 * reduction to the atoms (smx_electric_field_bec_bins, the Born effective
 * charges dF_i/dE_s).  Leaves the evaluation's results as they were. */
SMX_API int32_t smx_compute_prepared_factorized_field_response(SmxEvaluator* ev, uint64_t generation,
                                                               const double* field, int64_t field_count,
                                                               int32_t include_force_derivative,
                                                               int32_t scatter_bec_bins);
/* electric_field_hessian (pybind mace_kokkos.cpp:2160-2163): 9 values,
 * [c*3 + s] = d(dE/dE_c)/dE_s, of the last response (FP64 sums). */
SMX_API int32_t smx_electric_field_hessian(SmxEvaluator* ev, double* out, int64_t capacity, int64_t* count);
/* electric_field_force_derivative (pybind mace_kokkos.cpp:2164-2167):
 * [3][num_edges][3], the field component's derivative of each edge's
 * directed force in the caller's edge order (9 * num_edges values), or none
 * when the last response took no force derivative or scattered it into
 * bins.  *count gets the length; copies when out != NULL. */
SMX_API int32_t smx_electric_field_force_derivative(SmxEvaluator* ev, double* out, int64_t capacity,
                                                    int64_t* count);
/* electric_field_bec_bins (pybind mace_kokkos.cpp:2335-2349): [num_nodes][3][3],
 * bins[i][s][x] = dF_ix/dE_s (edges leaving i plus, arriving minus), or none
 * when the last response scattered no bins. */
SMX_API int32_t smx_electric_field_bec_bins(SmxEvaluator* ev, double* out, int64_t capacity, int64_t* count);
/* compute_node_energies_forces with execution_graph_generation == 0
 * (mace_kokkos.hpp:654-662; pybind mace_kokkos.cpp:2169): prepares the
 * graph from the host CSR, then evaluates. */
SMX_API int32_t smx_compute_node_energies_forces(SmxEvaluator* ev, int32_t num_nodes, const int32_t* node_types,
                                                 const int32_t* num_neigh, int64_t num_edges,
                                                 const int32_t* neigh_indices, const int32_t* neigh_types,
                                                 const double* xyz, const double* r);

/* reduce_prepared_node_forces (mace_kokkos.hpp:702; pybind _reduce_atom_forces,
 * mace_kokkos.cpp:2103): F[src] += f_e, F[rcv] -= f_e in FP64.  atom_forces
 * (host, [N][3]) may be NULL to keep the result on the device. */
SMX_API int32_t smx_reduce_prepared_node_forces(SmxEvaluator* ev, uint64_t generation, double* atom_forces);
/* reduce_prepared_stress (mace_kokkos.hpp:705; pybind _reduce_stress,
 * mace_kokkos.cpp:2134): sigma = -(1/V) sum_e f_e xyz_e^T.  stress (host [9])
 * may be NULL. */
SMX_API int32_t smx_reduce_prepared_stress(SmxEvaluator* ev, uint64_t generation, double volume, double* stress);
/* node_energies / node_forces properties (mace_kokkos.hpp:501) */
SMX_API int32_t smx_node_energies(SmxEvaluator* ev, double* out, int64_t capacity);
SMX_API int32_t smx_node_forces(SmxEvaluator* ev, double* out, int64_t capacity);
/* FP64 sum of the node energies on the device (the calculator's sum,
 * calculator.py:3831-3836); total may be NULL to keep it on the device. */
SMX_API int32_t smx_total_energy_device(SmxEvaluator* ev, double* total);
SMX_API int32_t smx_device_outputs(SmxEvaluator* ev, SmxDeviceOutputs* out);
SMX_API int32_t smx_synchronize(SmxEvaluator* ev);

/* LAMMPS pair-style entry: the single-rank path of pair_style
 * symmetrix/mace/kk without domain decomposition
 * (pair_symmetrix_mace_kokkos.cpp:1010-1282), over the device arrays the
 * Kokkos pair style holds.  Local atoms ilist[ii] are the graph's nodes; every
 * neighbour j (local or ghost) of a full neighbour list becomes an edge to the
 * local atom owner[j] (the pair style's atom->map(tag[j])), with
 * xyz = x[j] - x[i] clamped to the model cutoff (r_cut/r scaling, the
 * prepared-execution rule).  The topology is rebuilt when `rebuild` is set
 * (neighbor->ago == 0), when inum or nall change, or after another graph was
 * prepared on the evaluator; otherwise only the edge vectors are refreshed.
 * Forces are added to f (ghost rows included; the caller's reverse
 * communication folds them into their owners), per-atom energies to eatom
 * (when non-NULL), and the total energy and the six virial components
 * (xx, yy, zz, xy, xz, yz: sum over edges of xyz (x) f, symmetrised) are
 * returned on the host.  Both execution plans: the direct plan reduces its
 * retained edge forces after the call, the tiled plan adds each tile's edge
 * forces to f as the tile finishes (the same rows, another summation order).
 * Ordering: the evaluator runs on its own stream.  With SmxLammpsArgsV2 the
 * call first makes that stream wait for the work the caller queued on
 * args->stream (positions update, force clearing); with SmxLammpsArgsV1 it
 * synchronises the device on entry.  The call returns after its writes to
 * f and eatom are complete.  Positions that give an invalid edge (zero
 * length or non-finite) raise SMX_ERR_INVALID_ARGUMENT with f and eatom left
 * unchanged. */
typedef struct SmxLammpsArgsV1 {
    uint32_t struct_size;
    int32_t inum;                  /* local atoms in ilist */
    int32_t nall;                  /* local + ghost atoms (rows of x, type, owner, f) */
    int32_t ntypes;                /* LAMMPS atom types */
    const int32_t* ilist;          /* [inum] local atom indices */
    const int32_t* numneigh;       /* [atom] neighbour count of each ilist atom */
    const int32_t* neighbors;      /* neighbour j of atom i at i*stride_atom + jj*stride_neighbor;
                                      bits above NEIGHMASK (0x1FFFFFFF) are masked off */
    int64_t stride_atom;
    int64_t stride_neighbor;
    const double* x;               /* [nall][3] positions (Angstrom) */
    const int32_t* type;           /* [nall] LAMMPS types, 1-based */
    const int32_t* type_to_model;  /* [ntypes] model type index of LAMMPS type t+1 (-1: not mapped) */
    const int32_t* owner;          /* [nall] local atom index each atom is an image of */
    int32_t rebuild;               /* the neighbour list was rebuilt since the last call */
    int32_t reserved;
    double* f;                     /* [nall][3] forces, added to */
    double* eatom;                 /* [nall] per-atom energies, added to; may be NULL */
} SmxLammpsArgsV1;
/* V1 followed by the caller's stream (struct_size = sizeof(SmxLammpsArgsV2));
 * pass it through the SmxLammpsArgsV1 pointer. */
typedef struct SmxLammpsArgsV2 {
    uint32_t struct_size;
    int32_t inum;
    int32_t nall;
    int32_t ntypes;
    const int32_t* ilist;
    const int32_t* numneigh;
    const int32_t* neighbors;
    int64_t stride_atom;
    int64_t stride_neighbor;
    const double* x;
    const int32_t* type;
    const int32_t* type_to_model;
    const int32_t* owner;
    int32_t rebuild;
    int32_t reserved;
    double* f;
    double* eatom;
    void* stream;                  /* hipStream_t of the caller's device work (NULL: the null stream) */
} SmxLammpsArgsV2;
SMX_API int32_t smx_lammps_compute(SmxEvaluator* ev, const SmxLammpsArgsV1* args, double* energy, double* virial);

/* Stage buffers of the last evaluation (FP32, row-major node-major) for
 * stage-level parity checks: "A0", "M0", "H1", "Phi1", "A1", "A1_adj",
 * "dPhi1", "H1_adj", "M0_adj", "A0_adj", "edge_records".  Returns the
 * element count through *count; copies when out != NULL and capacity is
 * large enough. */
SMX_API int32_t smx_debug_stage(SmxEvaluator* ev, const char* name, float* out, int64_t capacity, int64_t* count);

/* Launch timing with HIP events on the evaluator stream (off by default). */
SMX_API int32_t smx_set_kernel_timing(SmxEvaluator* ev, int32_t enabled);
/* restrict timing to the comma-separated stage names (NULL or "" = all) */
SMX_API int32_t smx_set_kernel_timing_filter(SmxEvaluator* ev, const char* names);
SMX_API int32_t smx_kernel_timing_reset(SmxEvaluator* ev);
/* index-th timed kernel name (NULL past the end), total ms and launch count */
SMX_API int32_t smx_kernel_timing(SmxEvaluator* ev, int32_t index, const char** name, double* total_ms,
                                  int64_t* launches);

/* Model-file conversion (no reference counterpart: the reference reads JSON
 * only, mace_kokkos_model.cpp via nlohmann::json).  Rewrites `source` (JSON v4
 * text or the SMXB binary form, told apart by the magic) as `format`
 * ("binary" or "json") at `destination`; the document is unchanged, so either
 * file loads through smx_evaluator_create to the same model.  SMXB stores
 * every number array as raw doubles (layout in csrc/model_binary.hpp): a
 * medium model loads without number parsing. */
SMX_API int32_t smx_model_convert(const char* source, const char* destination, const char* format);

/* Standalone periodic neighbour list (neighbor_graph_kokkos.cpp:38-405),
 * bit-exact with the reference's device builder.  Two calls: with
 * sources == NULL it returns the edge count in *num_edges; then with
 * buffers num_neigh[N], offsets[N+1], sources[E], shifts[E][3],
 * fractional_xyz[E][3] (host) it fills them. */
SMX_API int32_t smx_neighbor_list(int32_t num_nodes, const double* positions, const double* cell,
                                  const double* inverse_cell, double cutoff, int64_t* num_edges,
                                  int32_t* num_neigh, int32_t* offsets, int32_t* sources, int32_t* shifts,
                                  double* fractional_xyz);

#ifdef __cplusplus
}
#endif

#endif /* SYMMETRIX_MI355X_H */
