// Device buffers and kernel-set interface shared by the evaluator and the
// HIP translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <memory>
#include <vector>

namespace smx {

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
};

// One prepared graph on the device (receiver-major CSR + source transpose).
struct DeviceGraph {
    int N = 0;
    std::int64_t E = 0;
    const int* node_types = nullptr;
    const int* offsets = nullptr;     // [N+1]
    const int* neigh = nullptr;       // sources [E]
    const int* neigh_types = nullptr;
    const int* receivers = nullptr;   // [E]
    const int* soff = nullptr;        // [N+1]
    const int* sedges = nullptr;      // [E] edges ordered by source, ascending edge id
    const float* erec = nullptr;      // [E][REC] per-edge record
};

// Node-linear tiles: TM=16 rows of one (weight group, m) over a node list.
struct GemmGroup {
    std::int64_t w_off;  // element offset of the [K][N] row-major weight block
    int K, N;
    int in_stride, in_base, in_mstride;
    int out_stride, out_base, out_mstride;
};
struct GemmTile {
    int list_start, count, group, m;
};
struct GemmPlan {
    const GemmTile* tiles = nullptr;
    const GemmGroup* groups = nullptr;
    const int* node_list = nullptr;
    int num_tiles = 0;
    int max_n = 0;
};

// Per-call workspace (node-sized and edge-sized arrays).
struct Workspace {
    float* Phi0 = nullptr;      // [N][NY][C]
    float* A0 = nullptr;        // [N][NY][C]
    float* M0 = nullptr;        // [N][NH][C]
    float* H1 = nullptr;        // [N][NH][C]
    float* Phi1 = nullptr;      // [N][NLME][C]
    float* A1 = nullptr;        // [N][NY][C]
    float* A1_adj = nullptr;    // [N][NY][C]
    float* direct = nullptr;    // [N][C]
    float* dPhi1 = nullptr;     // [N][NLME][C]
    float* Wsrc = nullptr;      // [E][NH][C] per-edge source-adjoint contributions
    float* H1_adj = nullptr;    // [N][NH][C]
    float* M0_adj = nullptr;    // [N][NH][C]
    float* A0_adj = nullptr;    // [N][NY][C]
    float* Phi0_adj = nullptr;  // [N][NY][C]
    double* node_energies = nullptr;  // [N]
    double* node_forces = nullptr;    // [E][3]
};

// Timing hook: the evaluator brackets launches with events when enabled.
struct LaunchTimer {
    virtual ~LaunchTimer() = default;
    virtual void begin(const char* name, hipStream_t s) = 0;
    virtual void end(const char* name, hipStream_t s) = 0;
};

// Kernels specialised for one (C, l_max, L_max) shape.
struct KernelSet {
    virtual ~KernelSet() = default;
    virtual int record_floats() const = 0;
    virtual void edge_geometry(const DeviceModel& m, std::int64_t E, const double* xyz, const double* r,
                               float* erec, hipStream_t s) const = 0;
    virtual void forward(const DeviceModel& m, const DeviceGraph& g, const Workspace& w, const GemmPlan& a0,
                         const GemmPlan& h1, const GemmPlan& a1, hipStream_t s, LaunchTimer* t) const = 0;
    virtual void reverse(const DeviceModel& m, const DeviceGraph& g, const Workspace& w, const GemmPlan& a0r,
                         const GemmPlan& h1r, const GemmPlan& a1r, hipStream_t s, LaunchTimer* t) const = 0;
};

std::unique_ptr<KernelSet> make_kernel_set(int C, int l_max, int L_max);
// true if (C, l_max, L_max) has a compiled kernel set, and the paths match
bool kernel_paths(int l_max, int L_max, std::vector<int>& le, std::vector<int>& ls, std::vector<int>& lo);

// Per-edge records (spline point, Y, dY, direction) from FP64 xyz and r.
void geometry_records(int l_max, std::int64_t E, const double* xyz, const double* r, double r_cut, float x0, float h,
                      int intervals, float* erec, hipStream_t s);

void launch_node_gemm(const GemmPlan& plan, const float* W, const float* in, float* out, hipStream_t s);

// Reductions (FP64, deterministic order)
void launch_atom_forces(int N, const int* offsets, const int* soff, const int* sedges, const double* node_forces,
                        double* atom_forces, hipStream_t s);
void launch_stress(std::int64_t E, const double* node_forces, const double* xyz, double volume, double* partial,
                   int partial_blocks, double* stress, hipStream_t s);
void launch_energy_sum(int N, const double* node_energies, double* total, hipStream_t s);

// Geometry (FP64, no contraction): per-atom minimum-image displacement from
// the reference positions, then per-edge xyz/r from fractional edge vectors.
void launch_prepared_geometry(int N, std::int64_t E, const int* receivers, const int* sources,
                              const double* fractional_xyz, const double* cell, const double* inv_cell,
                              const double* reference_positions, const double* positions, double cutoff,
                              double* disp, double* xyz, double* r, int* invalid, hipStream_t s);

// Neighbour list (bit-exact with the reference's device builder).
struct NeighborBuffers;  // defined in geometry.hip
struct NeighborResult {
    std::int64_t num_edges = 0;
    int* num_neigh = nullptr;       // [N]
    int* offsets = nullptr;         // [N+1]
    int* sources = nullptr;         // [E]
    int* shifts = nullptr;          // [E][3]
    double* fractional_xyz = nullptr;  // [E][3]
};
// Builds into buffers allocated with hipMalloc (freed by the caller with
// hipFree); positions/cell/inverse on the host.
void build_neighbor_list(int N, const double* positions_host, const double* cell_host, const double* inv_host,
                         double cutoff, NeighborResult& out, hipStream_t s);

// Edge receivers and source transpose from a receiver CSR (all on device).
void launch_graph_schedule(int N, std::int64_t E, const int* offsets, const int* sources, int* receivers,
                           int* soff, int* sedges, int* scratch_counts, hipStream_t s);
// neigh_types[e] = node_types[sources[e]]
void launch_gather_types(std::int64_t E, const int* sources, const int* node_types, int* neigh_types,
                         hipStream_t s);
// exclusive scan of int32 counts into int64 (device), returns total on host
std::int64_t device_exclusive_scan(const int* in, long long* out, int n, hipStream_t s);

}  // namespace smx
