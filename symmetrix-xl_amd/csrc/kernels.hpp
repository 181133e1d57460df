// Device buffers and kernel-set interface shared by the evaluator and the
// HIP translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

namespace smx {

// One angular entry of a MACEField path: H1f[lm_out] += coef E_comp Z[zrow]
// (Z = H1p[lm_in] W_path) forward; H1p_adj[lm_in] += coef E_comp Y[yrow]
// (Y = H1p_adj[lm_out] W_path^T) in reverse.
struct FieldEntryDev {
    int lm_in, comp, lm_out, zrow, yrow;
    float coef;
};

// Model tables resident in HBM (owned by the evaluator).
struct DeviceModel {
    int C = 0, l_max = 0, L_max = 0, num_lm = 0, num_LM = 0, num_elements = 0;
    int num_paths = 0, num_rows = 0, num_lme = 0;
    double r_cut = 0.0;
    int intervals = 0;
    float x0 = 0.0f, h = 0.0f;
    const float4* R0c = nullptr;  // [interval][(l_max+1)*C]
    const float4* R1c = nullptr;  // [interval][P*C]
    const float* H0 = nullptr;
    const float* A0_w = nullptr;
    const float* A0_wt = nullptr;
    const std::int32_t* m0_terms = nullptr;
    const int* m0_toff = nullptr;     // [num_LM+1] term offsets per output
    std::vector<int> m0_term_offset;  // host copy
    int T0 = 0;
    const float* m0_coef = nullptr;
    const float* H1_w = nullptr;
    const float* H1_wt = nullptr;
    // pre_linear_up basis: x = M0[:,0,:] P0 and M0_adj[:,0,:] += P0 d (GEMM
    // weights P0 and P0^T, swizzled); residual: per-type H1 and x offsets
    bool pre_linear_up = false, residual = false;
    // one interaction: M1 of H1, no R1 / A1 (single_layer_readout)
    bool single_layer = false;
    // MACEField: H1p = M0 P (+ b), H1f = H1p + field terms, x = H1f[:,0,:],
    // H1 = H1f U (GEMM weights swizzled: P, U per l; W per path)
    bool field = false;
    const float* P_w = nullptr;
    const float* P_wt = nullptr;
    const float* U_w = nullptr;
    const float* U_wt = nullptr;
    const float* field_W = nullptr;
    const float* field_Wt = nullptr;
    const float* res_pre = nullptr;  // [type][NH][C]
    const FieldEntryDev* field_entries = nullptr;
    int num_field_entries = 0;
    int field_zr = 0, field_yr = 0;  // rows of Z and Y per node
    const float* P0_w = nullptr;
    const float* P0_wt = nullptr;
    const float* res_H1 = nullptr;  // [type][NH][C]
    const float* res_x = nullptr;   // [type][C]
    const float* cg = nullptr;
    const float* A1_w = nullptr;
    const float* A1_wt = nullptr;
    std::vector<std::int64_t> A1_offset;  // host copy
    std::vector<int> num_e, lme_base;     // host copy
    const std::int32_t* m1_terms = nullptr;
    int T1 = 0;
    const float* m1_coef = nullptr;
    const float* H2_T = nullptr;
    const float* H2_Tt = nullptr;
    const float* H2_M1 = nullptr;
    const float* H2_M1t = nullptr;
    const double* q = nullptr;
    const double* W1r = nullptr;
    const double* W2r = nullptr;
    int hidden = 0;
    double readout_scale = 1.0;
    const double* E0 = nullptr;
    // density scaling (A0_scaled / A1_scaled): FP64 Hermite coefficients
    // [intervals][4] of the one-output density networks on the radial grid
    bool A0_scaled = false, A1_scaled = false;
    const double* dens0 = nullptr;
    const double* dens1 = nullptr;
    double x0_f64 = 0.0, h_f64 = 0.0;
    // ZBL pair repulsion: per (type, type) 1/a, 14.3996 Z_u Z_v, r_max
    bool has_zbl = false;
    const double* zbl_pair = nullptr;
    double zbl_c[4] = {0.0, 0.0, 0.0, 0.0};
    int zbl_p = 0;
};

// One prepared graph on the device (receiver-major CSR + source transpose).
struct DeviceGraph {
    int N = 0;                        // receivers
    int F = 0;                        // feature nodes (sources may be any of them; F >= N)
    std::int64_t E = 0;
    const int* node_types = nullptr;
    const int* offsets = nullptr;     // [N+1]
    const int* neigh = nullptr;       // sources [E]
    const int* neigh_types = nullptr;
    const int* receivers = nullptr;   // [E]
    const int* soff = nullptr;        // [F+1]
    const int* sedges = nullptr;      // [E] edges ordered by source, ascending edge id
    // [E] radial-table pair of each edge (symmetric index over the active
    // types) when tables differ per pair (Agnesi transform), else null
    const int* edge_pair = nullptr;
    // The tiled plan's source transpose, with 64-bit positions and edge ids
    // (soff/sedges are then null).  Its tiles see the graph through views
    // whose per-edge arrays and 32-bit offsets start at the tile's first
    // edge, graph edge edge_base (0 in a whole-graph view).
    const long long* soff64 = nullptr;    // [F+1]
    const long long* sedges64 = nullptr;  // [E]
    long long edge_base = 0;
};

// Node linears: out[row, n] = sum_k in[row, k] W[k, n] over the rows of one
// weight group.  A row is (tile-local node, m) packed as node << 4 | m; its
// input starts at node*in_stride + in_base + m*in_mstride (likewise the
// output).  W is stored in the MFMA operand order of swizzle_gemm_weights.
struct GemmGroup {
    std::int64_t w_off;  // element offset of the group's swizzled [K][N] block
    int K, N;
    int in_stride, in_base, in_mstride;
    int out_stride, out_base, out_mstride;
};
// rows per wave tile (a multiple of 16): 16 rows x up to 128 columns per
// wave.  At the medium shape this reads each input row once per 128 output
// columns and still gives about five waves per SIMD; it measured faster than
// 32 x 64 and 64 x 64 tiles.
constexpr int kGemmRows = 16;
struct GemmTile {
    int row_start, count, group;  // rows [row_start, row_start+count), count <= kGemmRows
};
// Up to kGemmShareWaves consecutive tiles of one group: the workgroup of the
// shared-operand GEMM kernel (tile indices relative to GemmPlan::tiles).
constexpr int kGemmShareWaves = 8;
struct GemmTileSet {
    int first, count;
};
struct GemmPlan {
    const GemmTile* tiles = nullptr;
    const GemmGroup* groups = nullptr;
    const int* rows = nullptr;        // packed (node << 4 | m)
    int num_tiles = 0;
    int max_n = 0;
    int n_sub = 1;  // 16-column tiles per wave (8, 4, 2 or 1): divides every group's N/16
    const GemmTileSet* sets = nullptr;  // tiles grouped for the shared-operand kernel
    int num_sets = 0;
    bool narrow = false;  // prefer 64-column waves to 128-column ones (long K)
};

// Readout batches: up to kReadoutBatch receivers of one type, as a range of
// the tile's type-sorted node list.
constexpr int kReadoutBatch = 16;  // the readout kernel's MFMA tile rows
constexpr int kMaxReadoutHidden = 64;  // readout MLP width the readout kernel holds in LDS
struct NodeBatch {
    int start, count;
};

// A receiver tile: receivers [r0, r0+nr), their edges [e0, e0+ne) (edges
// are receiver-major, so a receiver range owns one contiguous edge range).
struct TileView {
    int r0 = 0, nr = 0;
    std::int64_t e0 = 0, ne = 0;
    GemmPlan a0, h1, a1f, a1r;
    GemmPlan cap, cap_r;  // pre_linear_up: x = M0[:,0,:] P0 and its reverse P0 d (rows (node, 0))
    GemmPlan fz, fy;      // MACEField: Z = H1p[l_in rows] W_path, Y = H1p_adj[l_out rows] W_path^T
    const int* node_list = nullptr;    // tile-local receivers sorted by type
    const NodeBatch* batches = nullptr;
    int num_batches = 0;
    const int* touched = nullptr;  // sources with an edge in the tile (ascending)
    int touched_count = 0;
    // this call's FP64 edge lengths and vectors of the tile (indexed by
    // edge - e0); set before each evaluation
    const double* r = nullptr;
    const double* xyz = nullptr;
};

// Workspace.  Tile-local arrays are indexed by receiver - r0 (or edge - e0);
// graph-wide arrays by the global index.
struct Workspace {
    // tile-local
    float* erec = nullptr;      // [ne][REC_F] forward parts of the per-edge records
    float* erec_b = nullptr;    // [ne][REC_B] reverse parts
    float* Phi0 = nullptr;      // [nr][NY][C]
    float* A0 = nullptr;        // [nr][NY][C]
    float* M0 = nullptr;        // [nr][NH][C]
    float* Phi1 = nullptr;      // [nr][NLME][C]
    float* A1 = nullptr;        // [nr][NY][C]
    float* A1_adj = nullptr;    // [nr][NY][C]
    float* M1 = nullptr;        // [nr][C]
    float* dPhi1 = nullptr;     // [nr][NLME][C]
    float* Wsrc = nullptr;      // [ne][NH][C] per-edge source-adjoint contributions
    float* M0_adj = nullptr;    // [nr][NH][C]
    float* A0_adj = nullptr;    // [nr][NY][C]
    float* Phi0_adj = nullptr;  // [nr][NY][C]
    double* node_forces = nullptr;  // [ne][3]
    // density scaling: factors s = 1 + sum_j f(r_ij) and adjoint dot
    // products of A0 and A1, [nr] each
    double* dens_s0 = nullptr;
    double* dens_s1 = nullptr;
    double* dens_dot0 = nullptr;
    double* dens_dot1 = nullptr;
    // graph-wide
    float* H1 = nullptr;        // [N][NH][C]
    float* H1_adj = nullptr;    // [N][NH][C]
    float* xaff = nullptr;      // [N][C] scalar capture M0[i,0,:]
    float* direct = nullptr;    // [N][C] direct adjoint of the scalar capture
    float* direct_m0 = nullptr; // [N][C] pre_linear_up: that adjoint carried to M0[:,0,:] (P0 d)
    double* node_energies = nullptr;  // [N]
    // MACEField (direct plan, graph-wide): the field of this evaluation
    // (FP64, 3 values or 3 per node), H1p, H1f, H1p's adjoint, the Z / Y
    // rows of the field paths, per-node dE/dE partials and dE/dE
    const double* efield = nullptr;
    int efield_per_node = 0;
    float* H1p = nullptr;       // [N][NH][C]
    float* H1f = nullptr;       // [N][NH][C]
    float* H1p_adj = nullptr;   // [N][NH][C]
    float* fzy = nullptr;       // [N][max(zr, yr)][C]
    double* field_part = nullptr;  // [N][3]
    double* field_adj = nullptr;   // [3] or [N][3]
    // split-phase evaluation (feature graphs): layer 1 stops at H1p; the
    // layer-1 reverse starts from H1p's adjoint (field paths already run)
    bool field_product_only = false;
    bool field_reverse_done = false;
};

// MACEField response buffers (direct plan, graph-wide, N nodes and E edges):
// the tangents of one field component's pass, reused for each component.
struct ResponseWorkspace {
    // seed-independent: Z = H1p W, H1f_adj = H1_adj U^T (+ direct), Y = H1f_adj W^T
    float* Z = nullptr;          // [N][zr][C]
    float* H1f_adj = nullptr;    // [N][NH][C]
    float* Y = nullptr;          // [N][yr][C]
    float* H1f_dot = nullptr;    // [N][NH][C]
    float* x_dot = nullptr;      // [N][C]
    float* H1_dot = nullptr;     // [N][NH][C]
    float* Phi1_dot = nullptr;   // [N][NLME][C]
    float* A1_dot = nullptr;     // [N][NY][C]
    float* M1_dot = nullptr;     // [N][C]
    float* g = nullptr;          // [N][NY][C] dM1/dA1
    float* gd = nullptr;         // [N][NY][C] its tangent
    float* A1_adj_dot = nullptr; // [N][NY][C]
    float* A1s_adj = nullptr;    // [N][NY][C] (A1 density scaling)
    float* direct_dot = nullptr; // [N][C]
    float* dPhi1_dot = nullptr;  // [N][NLME][C]
    float* H1_adj_dot = nullptr; // [N][NH][C]
    float* H1p_adj_dot = nullptr;  // [N][NH][C]
    float* Y_dot = nullptr;      // [N][yr][C]
    float* M0_adj_dot = nullptr; // [N][NH][C]
    float* A0_adj_dot = nullptr; // [N][NY][C]
    float* Phi0_adj_dot = nullptr;  // [N][NY][C]
    double* dot_a = nullptr;     // [N] density adjoint dot products
    double* dot_b = nullptr;     // [N]
    double* part = nullptr;      // [N][3]
    double* part_scratch = nullptr;  // [N][3]
    const double* unit = nullptr;    // [3][3] the unit field of each component
    double* hessian_t = nullptr;     // [3][3]: [s][c] = d(dE/dE_c)/dE_s
    double* forces = nullptr;        // [3][E][3] directed forces' tangent per component
};

// Timing hook: the evaluator brackets launches with events when enabled.
struct LaunchTimer {
    virtual ~LaunchTimer() = default;
    virtual void begin(const char* name, hipStream_t s) = 0;
    virtual void end(const char* name, hipStream_t s) = 0;
};

// Kernels specialised for one (C, l_max, L_max) shape.  The stages are the
// reference's direct plan split at the two places where graph-wide state is
// exchanged (H1 after layer 1, H1 adjoint after the layer-2 reverse).
struct KernelSet {
    virtual ~KernelSet() = default;
    virtual int record_floats() const = 0;          // both parts of a record
    virtual int record_forward_floats() const = 0;  // its forward part
    // "unrolled" when the product-basis kernels use compiled term tables
    virtual const char* polynomial_mode() const = 0;
    // per-edge records of tile t from its FP64 xyz and r (tile-local, in the
    // caller's edge order), written in execution order: each receiver's
    // edges by spline-table row (exec: the tile's [ne] slot -> edge map,
    // filled here).  edge_pair, indexed like xyz, selects each edge's table
    // (null: one table).
    virtual void edge_geometry(const DeviceModel& m, const DeviceGraph& g, const TileView& t, const double* xyz,
                               const double* r, const int* edge_pair, int* exec, float* erec, float* erec_b,
                               hipStream_t s) const = 0;
    // R0 forward + A0 linear; with through_h1 also M0, the scalar capture and
    // H1 rows r0.. of the graph-wide H1
    virtual void layer1_forward(const DeviceModel& m, const DeviceGraph& g, const TileView& t, const Workspace& w,
                                bool through_h1, hipStream_t s, LaunchTimer* tm) const = 0;
    // R1 forward, A1, readouts and their reverse, R1 reverse: energies,
    // direct adjoint, per-edge source terms, directed forces (assigned)
    virtual void layer2(const DeviceModel& m, const DeviceGraph& g, const TileView& t, const Workspace& w,
                        hipStream_t s, LaunchTimer* tm) const = 0;
    // One-interaction models: M1 of the tile's H1 rows, readouts and their
    // reverse: energies, the direct adjoint and the tile's H1_adj rows
    // (assigned); the tile's directed forces are zeroed (then ZBL)
    virtual void single_readout(const DeviceModel& m, const DeviceGraph& g, const TileView& t, const Workspace& w,
                                hipStream_t s, LaunchTimer* tm) const = 0;
    // H1_adj = source sums of W over the whole graph (one tile); r: edge
    // lengths indexed like W (edges with r >= r_cut have no W row)
    virtual void source_adjoint_all(const DeviceGraph& g, const Workspace& w, const double* r, double r_cut,
                                    hipStream_t s, LaunchTimer* tm) const = 0;
    // H1_adj[s] += source sums of W over one tile's edges (r of the tile)
    virtual void source_adjoint_tile(const DeviceGraph& g, const TileView& t, const Workspace& w, const double* r,
                                     double r_cut, hipStream_t s, LaunchTimer* tm) const = 0;
    // H1 reverse, M0 reverse, A0 reverse, R0 reverse (directed forces added
    // to, or assigned to, the tile's buffer)
    virtual void layer1_reverse(const DeviceModel& m, const DeviceGraph& g, const TileView& t, const Workspace& w,
                                bool accumulate_forces, hipStream_t s, LaunchTimer* tm) const = 0;
    // MACEField, rows t.r0.. of t: H1 from H1p through the field paths and
    // linear_up; and its reverse to H1p_adj, the direct adjoint entering the
    // first direct_rows rows, dE/dE summed over the t.nr rows for one field
    virtual void field_features(const DeviceModel& m, const TileView& t, const Workspace& w, hipStream_t s,
                                LaunchTimer* tm) const = 0;
    virtual void field_features_reverse(const DeviceModel& m, const TileView& t, const Workspace& w, int direct_rows,
                                        hipStream_t s, LaunchTimer* tm) const = 0;
    // MACEField response of the last direct-plan evaluation (t: its one
    // tile, every receiver; w: its retained state, w.Wsrc taken as scratch):
    // the seed-independent products, then one field component's tangent
    // pass: the Hessian column rw.hessian_t[seed] and, with forces, the
    // directed forces' tangent rw.forces[seed]
    virtual void field_response_prepare(const DeviceModel& m, const TileView& t, const Workspace& w,
                                        const ResponseWorkspace& rw, hipStream_t s, LaunchTimer* tm) const = 0;
    virtual void field_response_seed(const DeviceModel& m, const DeviceGraph& g, const TileView& t,
                                     const Workspace& w, const ResponseWorkspace& rw, int seed, bool forces,
                                     hipStream_t s, LaunchTimer* tm) const = 0;
};

// Message returned by smx_last_error() on the calling thread.
void set_last_error(const std::string& message);

// Kernels for (C, l_max, L_max).  The polynomial kernels run with every
// product-basis term unrolled when the model's canonical M0 and M1 monomial
// lists equal a compiled table (ProductTable), else from the lists in HBM.
std::unique_ptr<KernelSet> make_kernel_set(int C, int l_max, int L_max, const std::vector<std::int32_t>& m0_terms,
                                           const std::vector<std::int32_t>& m0_offsets,
                                           const std::vector<std::int32_t>& m1_terms);
// [K][N] row-major block -> MFMA B-operand order [K/16][N/16][4][16][4]
// (k chunk, column block, lane/16, lane%16, k within the lane's four)
void swizzle_gemm_weights(const float* w, int K, int N, float* out);
// paths of the compiled kernel set for (l_max, L_max), false if none
bool kernel_paths(int l_max, int L_max, std::vector<int>& le, std::vector<int>& ls, std::vector<int>& lo);

// Execution order of the edges of receivers [r0, r0+nr) (edges [e0, ...)
// of the receiver-major CSR offsets; r, edge_pair and exec tile-local):
// within each receiver the active edges by spline-table row, ties by their
// position, then the inactive ones (r >= r_cut); exec[slot] = edge.
void launch_execution_order(int r0, int nr, std::int64_t e0, const int* offsets, const double* r, double r_cut,
                            float x0, float h, int intervals, const int* edge_pair, int* exec, hipStream_t s);
// Per-edge records (spline point, Y, dY, direction) from FP64 xyz and r,
// slot s built from edge exec[s] (all tile-local; exec null: the identity).
// Forward part: [x, table row (pair * intervals + interval), source type + 1
// (0 for an inactive edge), source node, Y]; reverse part: [dY, unit
// direction, ..., the edge's row].
void geometry_records(int l_max, std::int64_t E, const double* xyz, const double* r, double r_cut, float x0, float h,
                      int intervals, const int* edge_pair, const int* exec, const int* neigh, const int* neigh_types,
                      float* erec, float* erec_b, hipStream_t s);
// edge_pair[e] = symmetric pair of the active types of receiver and source
void launch_edge_pairs(std::int64_t E, const int* receivers, const int* node_types, const int* neigh_types,
                       const int* type_to_active, int active_types, int* edge_pair, int* bad, hipStream_t s);

void launch_node_gemm(const GemmPlan& plan, const float* W, const float* in, float* out, hipStream_t s);
// rows[li][0..row_len) += bias[types[r0 + li]][0..row_len) for li < nr
void launch_type_bias(int r0, int nr, const int* types, int row_len, const float* bias, float* rows, hipStream_t s);

// Density scaling (density.hip).  Factors s0/s1 (either may be null) of the
// tile's receivers from t.r; rows [nr][row_len] scaled (divide: A /= s in
// FP64, else A *= float(1/s)); the adjoint dot products dot = sum A_adj*A
// and the scaled adjoint; the directed-force terms added to node_forces.
void launch_density_factors(const DeviceModel& m, const DeviceGraph& g, const TileView& t, double* s0, double* s1,
                            hipStream_t s);
void launch_density_scale(int nr, int row_len, const double* s, bool divide, float* A, hipStream_t st);
void launch_density_adjoint(int nr, int row_len, const float* A, const double* s, bool divide, float* adj,
                            double* dot, hipStream_t st);
void launch_density_forces(const DeviceModel& m, const DeviceGraph& g, const TileView& t, const double* s0,
                           const double* dot0, const double* s1, const double* dot1, double* node_forces,
                           hipStream_t s);
// ZBL (zbl.hip): node_energies (graph-wide) += pair energies of the tile's
// receivers, node_forces (tile-local) -= their edge gradients
void launch_zbl(const DeviceModel& m, const DeviceGraph& g, const TileView& t, double* node_energies,
                double* node_forces, hipStream_t s);

// Reductions (FP64, deterministic order)
// forces of the F feature nodes: edges leaving a node minus (receivers,
// a < N) its own edges; row a goes to atom_forces[feature_of[a]] (or a)
void launch_atom_forces(int N, int F, const int* offsets, const int* soff, const int* sedges, const int* feature_of,
                        const double* node_forces, double* atom_forces, hipStream_t s);
// rows of row_floats floats: dst[k] = src[index[k]] (gather) or
// dst[index[k]] = src[k] (scatter), k < count
void launch_gather_rows(int count, int row_floats, const int* index, const float* src, float* dst, hipStream_t s);
void launch_scatter_rows(int count, int row_floats, const int* index, const float* src, float* dst, hipStream_t s);
void launch_scatter_rows(int count, int row_values, const int* index, const double* src, double* dst,
                         hipStream_t s);
// edges with a non-finite or non-positive length or a non-finite vector
void launch_count_invalid_edges(std::int64_t E, const double* xyz, const double* r, int* invalid, hipStream_t s);
void launch_stress(std::int64_t E, const double* node_forces, const double* xyz, double volume, double* partial,
                   int partial_blocks, double* stress, hipStream_t s);
// virial[9] += sum_e f_e xyz_e^T over E edges
void launch_virial_accumulate(std::int64_t E, const double* node_forces, const double* xyz, double* partial,
                              int partial_blocks, double* virial, hipStream_t s);
void launch_scale9(const double* in, double scale, double* out, hipStream_t s);
// F[src] += f_e, F[rcv] -= f_e for one tile's edges (tile-local forces).
// t.e0/t.ne: the tile's range in the edge ids of sedges; touched/
// touched_count: the sources the tile's edges leave, listed in the index
// space of soff/sedges; offsets[r0..r0+nr] the receivers' edge ranges, whose
// first tile edge is offsets_e0 (the tile's own relative offsets: 0);
// receiver_row maps a graph node to its F row (nullptr: the node index).
void launch_tile_forces(const TileView& t, const int* touched, int touched_count, const int* offsets,
                        long long offsets_e0, const int* soff, const int* sedges, const int* receiver_row,
                        const double* node_forces, double* F, hipStream_t s);
void launch_tile_forces(const TileView& t, const int* touched, int touched_count, const int* offsets,
                        long long offsets_e0, const long long* soff, const long long* sedges,
                        const int* receiver_row, const double* node_forces, double* F, hipStream_t s);
void launch_fill_zero(float* p, std::size_t n, hipStream_t s);
void launch_fill_zero(double* p, std::size_t n, hipStream_t s);
void launch_energy_sum(int N, const double* node_energies, double* total, hipStream_t s);

// Geometry (FP64, no contraction): per-atom displacement from the reference
// positions (Cartesian, or fractional when ref_fractional; wrapped to the
// minimum image along the periodic axes), then xyz/r of the edges
// [e0, e0+ne) from each edge's reference vector.
constexpr int kGeometryDeviceFractional = 0;  // neighbour list's wfrac + packed images
constexpr int kGeometryCartesian = 1;         // reference xyz per edge
constexpr int kGeometryFractional = 2;        // reference fractional xyz per edge
constexpr int kGeometryShifts = 3;            // reference positions + integer cell shifts per edge
struct EdgeReference {
    int kind = kGeometryDeviceFractional;
    const double* wfrac = nullptr;            // [N][3] (device_fractional)
    const std::uint32_t* images = nullptr;    // [E] (device_fractional)
    const double* positions = nullptr;        // [N][3] Cartesian (shifts)
    const double* edges = nullptr;            // [E][3] (cartesian, fractional)
    const int* shifts = nullptr;              // [E][3] (shifts)
};
// (also sets *invalid, the edge pass's invalid-edge count, to zero)
void launch_displacements(int N, const double* cell, const double* inv_cell, const int pbc[3], bool ref_fractional,
                          const double* reference_positions, const double* positions, double* disp, int* invalid,
                          hipStream_t s);
void launch_edge_xyz(std::int64_t e0, std::int64_t ne, const EdgeReference& ref, const double* cell,
                     const int* receivers, const int* sources, const double* disp, double cutoff, double* xyz,
                     double* r, int* invalid, hipStream_t s);

// Neighbour list (bit-exact with the reference's device builder).
struct NeighborResult {
    std::int64_t num_edges = 0;
    int* num_neigh = nullptr;        // [N]
    int* offsets = nullptr;          // [N+1]
    int* sources = nullptr;          // [E]
    std::uint32_t* images = nullptr; // [E] packed int8 x3 bin images
    double* wfrac = nullptr;         // [N][3] wrapped fractional positions
    int* shifts = nullptr;           // [E][3] (only when requested)
    double* fractional_xyz = nullptr;  // [E][3] (only when requested)
    long long* offsets64 = nullptr;    // [N+1] (only when wide)
};
// Builds into buffers allocated with hipMalloc (freed by the caller with
// hipFree); positions/cell/inverse on the host.  with_shifts also fills
// shifts and fractional_xyz.  wide admits up to kMaxWideEdges edges and
// hands out the 64-bit offsets too; the 32-bit offsets are then filled only
// when the edge count is at most kMaxEdges.
void build_neighbor_list(int N, const double* positions_host, const double* cell_host, const double* inv_host,
                         double cutoff, bool with_shifts, NeighborResult& out, hipStream_t s, bool wide = false);

// Edge receivers and source transpose from a receiver CSR (all on device).
void launch_graph_schedule(int N, int F, std::int64_t E, const int* offsets, const int* sources, int* receivers,
                           int* soff, int* sedges, int* scratch_counts, hipStream_t s);
// receivers[e] = i for the edges of receiver i
void launch_receivers(int N, const int* offsets, int* receivers, hipStream_t s);
void launch_receivers(int N, const long long* offsets, int* receivers, hipStream_t s);
// LAMMPS pair-style entry (lammps.hip): a full neighbour list as the Kokkos
// pair style holds it, on the device.
struct LammpsList {
    const int* ilist;
    const int* numneigh;
    const int* neighbors;
    long long stride_atom, stride_neighbor;
    const int* type;
    const int* type_to_model;
    int ntypes;
    const int* owner;
};
// node_types/num_neigh of the ilist atoms and node_of_atom[atom] (-1 when
// not in ilist); bad counts unmapped types and negative counts
void lammps_nodes(int inum, int nall, const LammpsList& L, int* node_types, int* num_neigh, int* node_of_atom,
                  int* bad, hipStream_t s);
// edges of each node (offsets from num_neigh): node of the owner, its model
// type and the LAMMPS index of the neighbour
void lammps_edges(int inum, int nall, const LammpsList& L, const int* offsets, const int* node_of_atom, int* neigh,
                  int* neigh_types, int* lmp_j, int* bad, hipStream_t s);
// edge vectors of edges [e0, e0+ne), written tile-local (row e - e0)
void lammps_geometry(std::int64_t e0, std::int64_t ne, const int* receivers, const int* ilist, const int* lmp_j,
                     const double* x, double r_cut, double* xyz, double* r, int* invalid, hipStream_t s);
void lammps_forces(int nall, const int* joff, const int* jedges, const int* node_of_atom, const int* offsets,
                   const double* node_forces, double* f, hipStream_t s);
void lammps_eatom(int inum, const int* ilist, const double* node_energies, double* eatom, hipStream_t s);

// Transpose of an edge -> key map (keys in [0, K)): koff[K+1] and kedges[E]
// listing each key's edges in ascending edge order.  scratch_counts: K ints.
void launch_transpose(int K, std::int64_t E, const int* keys, int* koff, int* kedges, int* scratch_counts,
                      hipStream_t s);
// the same with 64-bit positions and edge ids (the tiled plan's source transpose)
void launch_transpose(int K, std::int64_t E, const int* keys, long long* koff, long long* kedges, int* scratch_counts,
                      hipStream_t s);
// neigh_types[e] = node_types[sources[e]]
void launch_gather_types(std::int64_t E, const int* sources, const int* node_types, int* neigh_types,
                         hipStream_t s);
// Sources with at least one edge in [e0, e0+ne), ascending, into out
// (capacity >= N); returns the count.  bitmap: N/32+1 words of scratch,
// word_counts: N/32+1 ints of scratch.
int build_touched_sources(int N, std::int64_t e0, std::int64_t ne, const int* sources, std::uint32_t* bitmap,
                          int* word_counts, int* out, hipStream_t s);
// exclusive scan of int32 counts into int64 (device), returns total on host
std::int64_t device_exclusive_scan(const int* in, long long* out, int n, hipStream_t s);

}  // namespace smx
