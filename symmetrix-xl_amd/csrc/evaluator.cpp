// MACE evaluator on one MI355X: host orchestration behind the C ABI of
// include/symmetrix_mi355x.h.
//
// The call sequence mirrors the reference's direct streamed-edge plan
// (libsymmetrix/source/mace_kokkos_evaluate.cpp:314-611 and the prepared-graph
// lifecycle mace_kokkos_factorized_lifecycle.cpp:905-949, 1934, 2915-3089):
//   prepare graph (receiver CSR, source transpose, generation token)
//   -> per call: edge geometry from positions, Y/dY records, layer-1 and
//      layer-2 forward, readouts, reverse through both layers (directed
//      FP64 forces per edge), then FP64 reductions on request.
// Workspaces grow to a high-water mark and are reused across calls, as the
// reference's capacity reuse does (docs/streamed_edge_execution.md:154-165).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <climits>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <new>
#include <numeric>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/symmetrix_mi355x.h"
#include "../../include/symmetrix_operator_modules.h"
#include "device_common.hpp"
#include "kernels.hpp"
#include "model.hpp"

namespace smx {
namespace {

thread_local std::string g_last_error;

// Device allocation that grows to a high-water mark.
class DevBuf {
public:
    DevBuf() = default;
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    ~DevBuf() { release(); }
    void* ensure(std::size_t bytes) {
        if (bytes > cap_) {
            release();
            if (bytes > 0) {
                const hipError_t e = hipMalloc(&ptr_, bytes);
                if (e != hipSuccess) {
                    ptr_ = nullptr;
                    cap_ = 0;
                    throw std::bad_alloc();
                }
            }
            cap_ = bytes;
        }
        return ptr_;
    }
    template <class T>
    T* as() const {
        return static_cast<T*>(ptr_);
    }
    std::size_t capacity() const { return cap_; }
    // take ownership of a hipMalloc'd block
    void adopt(void* p, std::size_t bytes) {
        release();
        ptr_ = p;
        cap_ = p ? bytes : 0;
    }
    void release() {
        if (ptr_) (void)hipFree(ptr_);
        ptr_ = nullptr;
        cap_ = 0;
    }

private:
    void* ptr_ = nullptr;
    std::size_t cap_ = 0;
};

// Synchronous upload (graph and model preparation, not the per-call path):
// the host vector may be a temporary.
template <class T>
T* upload(DevBuf& b, const std::vector<T>& v, hipStream_t s) {
    T* p = static_cast<T*>(b.ensure(std::max<std::size_t>(1, v.size()) * sizeof(T)));
    if (!v.empty()) {
        SMX_HIP(hipMemcpyAsync(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice, s));
        SMX_HIP(hipStreamSynchronize(s));
    }
    return p;
}

class EventTimer final : public LaunchTimer {
public:
    struct Entry {
        double total_ms = 0.0;
        std::int64_t launches = 0;
    };
    ~EventTimer() override {
        clear_pending();
        for (hipEvent_t e : pool_) (void)hipEventDestroy(e);
    }
    // Only launches whose name is in `filter` (comma-separated; empty = all)
    // are bracketed with events.
    void set_filter(const std::string& filter) {
        names_.clear();
        std::size_t p = 0;
        while (p <= filter.size()) {
            const std::size_t q = std::min(filter.find(',', p), filter.size());
            if (q > p) names_.push_back(filter.substr(p, q - p));
            p = q + 1;
        }
    }
    bool wanted(const char* name) const {
        return names_.empty() || std::find(names_.begin(), names_.end(), name) != names_.end();
    }
    void begin(const char* name, hipStream_t s) override {
        if (!wanted(name)) return;
        hipEvent_t a = take();
        SMX_HIP(hipEventRecord(a, s));
        open_[name] = a;
    }
    void end(const char* name, hipStream_t s) override {
        if (!wanted(name)) return;
        hipEvent_t b = take();
        SMX_HIP(hipEventRecord(b, s));
        pending_.push_back({name, open_[name], b});
        open_.erase(name);
    }
    // After the stream has been synchronised: fold the pending pairs in.
    void collect() {
        for (auto& p : pending_) {
            float ms = 0.0f;
            SMX_HIP(hipEventElapsedTime(&ms, p.a, p.b));
            Entry& e = entries_[p.name];
            if (e.launches == 0) order_.push_back(p.name);
            e.total_ms += ms;
            e.launches += 1;
        }
        clear_pending();
    }
    void reset() {
        clear_pending();
        entries_.clear();
        order_.clear();
    }
    bool get(int index, const char** name, double* ms, std::int64_t* n) const {
        if (index < 0 || index >= static_cast<int>(order_.size())) return false;
        const auto it = entries_.find(order_[index]);
        *name = it->first.c_str();
        *ms = it->second.total_ms;
        *n = it->second.launches;
        return true;
    }

private:
    struct Pending {
        std::string name;
        hipEvent_t a, b;
    };
    hipEvent_t take() {
        if (pool_.empty()) {
            hipEvent_t e;
            SMX_HIP(hipEventCreate(&e));
            return e;
        }
        hipEvent_t e = pool_.back();
        pool_.pop_back();
        return e;
    }
    void clear_pending() {
        for (auto& p : pending_) {
            pool_.push_back(p.a);
            pool_.push_back(p.b);
        }
        pending_.clear();
        for (auto& o : open_) pool_.push_back(o.second);
        open_.clear();
    }
    std::vector<hipEvent_t> pool_;
    std::vector<std::string> names_;
    std::map<std::string, hipEvent_t> open_;
    std::vector<Pending> pending_;
    std::map<std::string, Entry> entries_;
    std::vector<std::string> order_;
};

// Concatenated node-linear tiles of every receiver tile of the graph.
struct PlanSet {
    std::vector<GemmTile> tiles;
    std::vector<std::size_t> tile_begin;  // per receiver tile: first GemmTile
    std::vector<int> rows;                // packed (local node << 4 | m)
    std::vector<GemmTileSet> sets;        // per receiver tile, tiles relative to its first
    std::vector<std::size_t> set_begin;
    DevBuf d_tiles, d_rows, d_sets;
};

}  // namespace

void set_last_error(const std::string& message) { g_last_error = message; }

struct Evaluator {
    HostModel hm;
    DeviceModel dm;
    std::unique_ptr<KernelSet> ks;
    hipStream_t stream = nullptr;
    std::string streamed_edges = "direct";

    // model tables and node-linear groups (defined for every type and l)
    std::vector<std::unique_ptr<DevBuf>> model_bufs;
    std::vector<GemmGroup> groups_a0, groups_h1, groups_a1f, groups_a1r, groups_cap, groups_cap_r;
    DevBuf d_groups_a0, d_groups_h1, d_groups_a1f, d_groups_a1r, d_groups_cap, d_groups_cap_r;
    int max_n_a0 = 0, max_n_h1 = 0, max_n_a1f = 0, max_n_a1r = 0;
    int sub_a0 = 1, sub_h1 = 1, sub_a1f = 1, sub_a1r = 1, sub_cap = 1;
    // MACEField path products: Z rows per path (l_in m's), Y rows (l_out m's)
    std::vector<GemmGroup> groups_fz, groups_fy;
    DevBuf d_groups_fz, d_groups_fy;
    int sub_f = 1;
    // the electric field of the next evaluations (FP64 on the device): 3
    // values, or 3 per node; dE/dE of the last one
    std::vector<double> h_efield;
    DevBuf d_efield, d_field_part, d_field_adj;
    bool field_evaluated = false;
    std::int64_t field_adj_count = 0;  // values of the last evaluation's dE/dE
    std::vector<double> evaluated_field;  // the field the last evaluation ran in
    // MACEField response (compute_prepared_factorized_field_response,
    // mace_kokkos_response.tpp:2504-2543): tangent buffers, the Hessian
    // [c*3 + s] on the host, the force derivative [3][E][3] or the Born
    // charge bins [3][N][3] on the device
    ResponseWorkspace rws;
    DevBuf r_f32, r_f64;
    double response_hessian[9] = {0};
    bool response_done = false, response_has_forces = false, response_has_bins = false;
    int response_N = 0;
    std::int64_t response_E = 0;

    // execution plan request (set_execution_plan_request, set_allow_fixed_workspace,
    // mace_kokkos.hpp:95-96; the calculator's execution_profile and
    // allow_fixed_workspace): profile "capacity" (default) or "speed"; a
    // debug plan id pins a plan; the tiled plan is chosen by the planner only
    // when fixed workspaces are allowed
    std::string request_profile = "capacity";
    std::string debug_plan;
    bool allow_fixed = false;
    int tile_limit = 32768;         // receivers per tile in the tiled plan
    bool tiled = false;
    // report of the last planning (execution_plan_report)
    std::string plan_source = "none", plan_reason = "no graph prepared";
    std::size_t plan_available = 0, plan_untiled = 0, plan_tiled = 0;
    // pinned active types (prepare_active_types): pair tables kept for them
    std::vector<int> pinned_active;
    // counters (factorized_last_graph_prepare_ms, factorized_last_evaluation_ms)
    double last_prepare_ms = 0.0, last_evaluation_ms = 0.0;
    std::int64_t prepare_count = 0, evaluation_count = 0, geometry_prepare_count = 0;

    // graph
    std::uint64_t generation = 0, next_generation = 1;
    int N = 0;
    std::int64_t E = 0;
    // Feature graphs (prepare_factorized_graph with feature nodes,
    // lifecycle.cpp:949-1104; the domain-decomposed LAMMPS path,
    // pair_symmetrix_mace_kokkos.cpp:1285-1704): F >= N feature nodes, the
    // receivers' own and ghost atoms, any of which an edge may leave. The
    // evaluator numbers them receivers first (receiver ii is node ii), then
    // the other feature nodes in the caller's order; h_feature_of[k] is node
    // k's caller feature index (empty when the caller's order is this one).
    int F = 0;
    std::vector<int> h_feature_types, h_feature_of;
    DevBuf d_feature_of, d_h1_exchange, d_forces_caller;
    // the positions form of a feature graph: each edge's source and each
    // receiver as caller feature indices, and the feature nodes' positions
    // (edge vectors x[source] - x[receiver], as the pair style forms them)
    DevBuf d_edge_src_feature, d_recv_feature, d_fpos;
    bool fpos_mode = false;
    bool feature_prepared = false;  // the graph came through the feature-node prepare
    // split-phase (distributed) evaluation: layer 1 -> H1 of the receivers;
    // H1 of every feature node in -> layer 2 and the H1 adjoint of every
    // feature node out; the receivers' summed H1 adjoint in -> layer-1 reverse
    // (mace_kokkos_evaluate.cpp:1658-1990)
    enum class Phase { idle, prefix_complete, middle_complete };
    Phase phase = Phase::idle;
    // MACEField over a feature graph: the field paths and linear_up run over
    // every feature node (one tile of F rows, plans over all of them)
    PlanSet ps_feat_h1, ps_feat_fz, ps_feat_fy;
    TileView feature_tile;
    bool feature_graph() const { return F != N || !h_feature_of.empty(); }
    std::vector<int> h_node_types;
    std::vector<std::int64_t> h_offsets;
    DevBuf d_node_types, d_offsets, d_neigh, d_neigh_types, d_receivers, d_soff, d_sedges, d_counts;
    // The tiled plan indexes edges with 64 bits: its source transpose
    // (d_soff64/d_sedges64 in place of d_soff/d_sedges) and the device
    // neighbour list's offsets (d_offsets64, until the schedule is built;
    // d_offsets is then absent beyond kMaxEdges edges).  Each tile's kernels
    // read 32-bit offsets relative to its first edge: d_tile_off holds them,
    // tile after tile (tile ti's nr+1 values start at r0 + ti).
    DevBuf d_offsets64, d_soff64, d_sedges64, d_tile_off;
    // receiver tiles
    std::vector<TileView> tiles;
    PlanSet ps_a0, ps_h1, ps_a1f, ps_a1r, ps_cap, ps_fz, ps_fy;
    std::vector<int> h_node_list;
    std::vector<std::size_t> node_list_begin;
    std::vector<NodeBatch> h_batches;
    std::vector<std::size_t> batch_begin;
    DevBuf d_node_list, d_batches, d_touched;
    std::vector<std::size_t> touched_begin;
    int max_tile_nr = 0;
    std::int64_t max_tile_ne = 0;
    // geometry reference of the prepared graph (the reference's prepared
    // geometry kinds, lifecycle.cpp:2455-2735): the device neighbour list's
    // wrapped fractional positions + packed edge images, or host-given
    // Cartesian / fractional reference vectors, or integer cell shifts
    enum class Geometry { none, device_fractional, cartesian, fractional, shifts };
    Geometry geom = Geometry::none;
    int pbc[3] = {1, 1, 1};
    double cell[9] = {0}, inv_cell[9] = {0};
    DevBuf d_wfrac, d_images, d_ref_positions, d_ref_edges, d_disp, d_positions;
    // per call
    DevBuf d_xyz, d_r, d_invalid;
    DevBuf w_erec, w_Phi0, w_A0, w_M0, w_Phi1, w_A1, w_A1_adj, w_M1, w_dPhi1, w_Wsrc, w_M0_adj, w_A0_adj, w_Phi0_adj,
        w_node_forces, w_density, w_exec;
    DevBuf g_H1p, g_H1f, g_H1p_adj, g_fzy;
    DevBuf g_H1, g_H1_adj, g_xaff, g_direct, g_direct_m0, d_node_energies, d_atom_forces, d_virial, d_stress, d_stress_partial,
        d_total;
    Workspace ws;
    bool evaluated = false;
    bool xyz_host = false;  // this call's edge vectors came from the caller
    // The invalid-edge count of a positions call is copied to pinned host
    // memory right after the edge geometry, so the call can raise without
    // waiting for the model kernels queued behind it.
    // per-pair radial tables (Agnesi transform): the active types whose
    // tables are on the device, and each edge's table pair
    std::vector<int> pair_active;
    DevBuf d_pair_R0, d_pair_R1, d_pair_D0, d_pair_D1, d_type_to_active, d_edge_pair;
    int* h_invalid = nullptr;
    hipEvent_t geometry_done = nullptr;
    hipEvent_t geometry_ready = nullptr;   // edge geometry done on the main stream
    hipStream_t flag_stream = nullptr;     // carries the invalid-edge count to the host
    hipEvent_t caller_ready = nullptr;  // LAMMPS V2: the caller's stream, waited on
    bool geometry_flag_pending = false;
    int stress_blocks = 256;

    std::unique_ptr<EventTimer> timer;

    Evaluator(const std::string& path, const std::string& head) {
        hm.load(path, head);
        // channel counts that are neither a whole number of 64-lane waves nor
        // at most one 32-lane half are run on the next multiple of 64 with
        // zero extra channels (every cross-lane sum then spans whole waves)
        if (hm.C > 32 && hm.C % 64 != 0 && hm.C % 16 == 0) hm.pad_channels((hm.C + 63) / 64 * 64);
        std::vector<int> le, ls, lo;
        // a one-interaction model has no R1 paths; the kernel set of its
        // (l_max, L_max) serves its layer 1 and readout
        if (!kernel_paths(hm.l_max, hm.L_max, le, ls, lo) ||
            (!hm.single_layer && (le != hm.path_le || ls != hm.path_ls || lo != hm.path_lo)))
            throw std::domain_error("the model's R1 paths have no compiled kernel set (l_max " +
                                    std::to_string(hm.l_max) + ", L_max " + std::to_string(hm.L_max) + ")");
        if (hm.readout_hidden > kMaxReadoutHidden)
            throw std::domain_error("readout MLP wider than " + std::to_string(kMaxReadoutHidden) +
                                    " hidden units has no compiled kernel");
        if (hm.C % 16 != 0) throw std::domain_error("channel counts must be multiples of 16");
        ks = make_kernel_set(hm.C, hm.l_max, hm.L_max, hm.m0_terms, hm.m0_term_offset, hm.m1_terms);
        if (!ks)
            throw std::domain_error("no kernel set is compiled for " + std::to_string(hm.C) + " channels, l_max " +
                                    std::to_string(hm.l_max) + ", L_max " + std::to_string(hm.L_max));
        SMX_HIP(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
        SMX_HIP(hipHostMalloc(reinterpret_cast<void**>(&h_invalid), sizeof(int), hipHostMallocDefault));
        SMX_HIP(hipEventCreateWithFlags(&geometry_done, hipEventDisableTiming));
        SMX_HIP(hipEventCreateWithFlags(&geometry_ready, hipEventDisableTiming));
        SMX_HIP(hipStreamCreateWithFlags(&flag_stream, hipStreamNonBlocking));
        SMX_HIP(hipEventCreateWithFlags(&caller_ready, hipEventDisableTiming));
        upload_model();
        define_groups();
        SMX_HIP(hipStreamSynchronize(stream));
    }

    ~Evaluator() {
        if (stream) {
            (void)hipStreamSynchronize(stream);
            timer.reset();
            (void)hipStreamDestroy(stream);
        }
        if (flag_stream) {
            (void)hipStreamSynchronize(flag_stream);
            (void)hipStreamDestroy(flag_stream);
        }
        if (geometry_done) (void)hipEventDestroy(geometry_done);
        if (geometry_ready) (void)hipEventDestroy(geometry_ready);
        if (caller_ready) (void)hipEventDestroy(caller_ready);
        if (h_invalid) (void)hipHostFree(h_invalid);
        if (h_stage) (void)hipHostFree(h_stage);
    }

    // pinned host staging of the one-call results path: positions in,
    // energies, forces and stress out (grown on demand, freed at the end)
    double* h_stage = nullptr;
    std::size_t h_stage_count = 0;
    double* host_stage(std::size_t count) {
        if (count > h_stage_count) {
            if (h_stage) SMX_HIP(hipHostFree(h_stage));
            h_stage = nullptr;
            h_stage_count = 0;
            SMX_HIP(hipHostMalloc(reinterpret_cast<void**>(&h_stage), count * sizeof(double), hipHostMallocDefault));
            h_stage_count = count;
        }
        return h_stage;
    }

    template <class T>
    const T* put(const std::vector<T>& v) {
        model_bufs.push_back(std::make_unique<DevBuf>());
        return upload(*model_bufs.back(), v, stream);
    }

    void upload_model() {
        dm.C = hm.C;
        dm.l_max = hm.l_max;
        dm.L_max = hm.L_max;
        dm.num_lm = hm.num_lm;
        dm.num_LM = hm.num_LM;
        dm.num_elements = hm.num_elements;
        dm.num_paths = hm.num_paths;
        dm.num_rows = hm.num_rows;
        dm.num_lme = hm.num_lme;
        dm.r_cut = hm.r_cut;
        dm.intervals = hm.spline_points - 1;
        dm.x0 = hm.grid_min_f;
        dm.h = hm.h_f;
        dm.x0_f64 = hm.grid_min;
        dm.h_f64 = hm.h;
        dm.A0_scaled = hm.A0_scaled;
        dm.A1_scaled = hm.A1_scaled;
        if (hm.A0_scaled) dm.dens0 = put(hm.A0_density);
        if (hm.A1_scaled) dm.dens1 = put(hm.A1_density);
        dm.has_zbl = hm.has_zbl;
        if (hm.has_zbl) {
            dm.zbl_pair = put(hm.zbl_pair);
            for (int k = 0; k < 4; ++k) dm.zbl_c[k] = hm.zbl_c[k];
            dm.zbl_p = hm.zbl_p;
        }
        dm.R0c = reinterpret_cast<const float4*>(put(hm.R0_coef));
        dm.R1c = reinterpret_cast<const float4*>(put(hm.R1_coef));
        dm.H0 = put(hm.H0);
        const std::size_t a0_blocks = static_cast<std::size_t>(hm.num_elements) * (hm.l_max + 1);
        dm.A0_w = put(swizzled(hm.A0_w, a0_blocks, hm.C, hm.C));
        dm.A0_wt = put(swizzled(hm.A0_wt, a0_blocks, hm.C, hm.C));
        dm.m0_terms = put(hm.m0_terms);
        dm.m0_toff = put(hm.m0_term_offset);
        dm.m0_term_offset = hm.m0_term_offset;
        dm.T0 = static_cast<int>(hm.m0_terms.size());
        dm.m0_coef = put(hm.m0_coef);
        dm.H1_w = put(swizzled(hm.H1_w, hm.L_max + 1, hm.C, hm.C));
        dm.H1_wt = put(swizzled(hm.H1_wt, hm.L_max + 1, hm.C, hm.C));
        dm.pre_linear_up = hm.pre_linear_up;
        dm.residual = hm.residual;
        dm.single_layer = hm.single_layer;
        if (hm.pre_linear_up) {
            dm.P0_w = put(swizzled(hm.P0, 1, hm.C, hm.C));
            dm.P0_wt = put(swizzled(hm.P0t, 1, hm.C, hm.C));
        }
        if (hm.residual) {
            dm.res_H1 = put(hm.res_H1);
            dm.res_x = put(hm.res_x);
        }
        dm.field = hm.field;
        if (hm.field) {
            const int nl = hm.L_max + 1, np = static_cast<int>(hm.field_paths.size());
            dm.P_w = put(swizzled(hm.P_all, nl, hm.C, hm.C));
            dm.P_wt = put(swizzled(hm.P_allt, nl, hm.C, hm.C));
            dm.U_w = put(swizzled(hm.U_all, nl, hm.C, hm.C));
            dm.U_wt = put(swizzled(hm.U_allt, nl, hm.C, hm.C));
            dm.field_W = put(swizzled(hm.field_W, np, hm.C, hm.C));
            dm.field_Wt = put(swizzled(hm.field_Wt, np, hm.C, hm.C));
            if (hm.residual) dm.res_pre = put(hm.res_pre);
            // Z rows: each path's l_in m's in turn; Y rows: its l_out m's
            std::vector<int> zoff(np + 1, 0), yoff(np + 1, 0);
            for (int p = 0; p < np; ++p) {
                zoff[p + 1] = zoff[p] + 2 * hm.field_paths[p].l_in + 1;
                yoff[p + 1] = yoff[p] + 2 * hm.field_paths[p].l_out + 1;
            }
            std::vector<FieldEntryDev> ent;
            for (const auto& e : hm.field_entries) {
                const auto& fp = hm.field_paths[e.path];
                ent.push_back(FieldEntryDev{e.lm_in, e.comp, e.lm_out, zoff[e.path] + e.lm_in - fp.l_in * fp.l_in,
                                            yoff[e.path] + e.lm_out - fp.l_out * fp.l_out, e.coef});
            }
            dm.field_entries = put(ent);
            dm.num_field_entries = static_cast<int>(ent.size());
            dm.field_zr = zoff[np];
            dm.field_yr = yoff[np];
        }
        dm.cg = put(hm.cg_dense);
        {
            std::vector<float> w(hm.A1_w.size()), wt(hm.A1_wt.size());
            for (int l = 0; l <= hm.l_max; ++l) {
                const int K = hm.num_e[l] * hm.C;
                if (K == 0) continue;
                swizzle_gemm_weights(hm.A1_w.data() + hm.A1_offset[l], K, hm.C, w.data() + hm.A1_offset[l]);
                swizzle_gemm_weights(hm.A1_wt.data() + hm.A1_offset[l], hm.C, K, wt.data() + hm.A1_offset[l]);
            }
            dm.A1_w = put(w);
            dm.A1_wt = put(wt);
        }
        dm.A1_offset = hm.A1_offset;
        dm.num_e = hm.num_e;
        dm.lme_base = hm.lme_base;
        dm.m1_terms = put(hm.m1_terms);
        dm.T1 = static_cast<int>(hm.m1_terms.size());
        dm.m1_coef = put(hm.m1_coef);
        dm.H2_T = put(hm.H2_T);
        dm.H2_Tt = put(hm.H2_Tt);
        dm.H2_M1 = put(hm.H2_M1);
        dm.H2_M1t = put(hm.H2_M1t);
        dm.q = put(hm.readout_q);
        dm.W1r = put(hm.readout_W1);
        dm.W2r = put(hm.readout_W2);
        dm.hidden = hm.readout_hidden;
        dm.readout_scale = hm.readout_scale;
        dm.E0 = put(hm.atomic_energies);
    }

    // blocks [count][K][N] of a weight array in the MFMA operand order
    static std::vector<float> swizzled(const std::vector<float>& w, std::size_t count, int K, int N) {
        std::vector<float> out(w.size());
        const std::size_t blk = static_cast<std::size_t>(K) * N;
        for (std::size_t b = 0; b < count; ++b) swizzle_gemm_weights(w.data() + b * blk, K, N, out.data() + b * blk);
        return out;
    }

    // Weight groups of the node linears: A0 per (type, l), H1 per l, A1 per
    // l (forward K = num_e(l)*C -> C; reverse C -> num_e(l)*C).
    void define_groups() {
        const int C = hm.C, NY = hm.num_lm, NH = hm.num_LM, NLME = hm.num_lme;
        for (int t = 0; t < hm.num_elements; ++t)
            for (int l = 0; l <= hm.l_max; ++l)
                groups_a0.push_back(GemmGroup{(static_cast<std::int64_t>(t) * (hm.l_max + 1) + l) * C * C, C, C,
                                              NY * C, l * l * C, C, NY * C, l * l * C, C});
        for (int l = 0; l <= hm.L_max; ++l)
            groups_h1.push_back(GemmGroup{static_cast<std::int64_t>(l) * C * C, C, C, NH * C, l * l * C, C, NH * C,
                                          l * l * C, C});
        for (int l = 0; l <= hm.l_max; ++l) {
            const int ne = hm.num_e[l];
            groups_a1f.push_back(GemmGroup{hm.A1_offset[l], std::max(ne, 1) * C, C, NLME * C, hm.lme_base[l] * C,
                                           ne * C, NY * C, l * l * C, C});
            groups_a1r.push_back(GemmGroup{hm.A1_offset[l], C, std::max(ne, 1) * C, NY * C, l * l * C, C, NLME * C,
                                           hm.lme_base[l] * C, ne * C});
        }
        auto mx = [](const std::vector<GemmGroup>& g) {
            int m = 0;
            for (const auto& x : g) m = std::max(m, x.N);
            return m;
        };
        auto sub = [](const std::vector<GemmGroup>& g) {
            int n = 8;
            for (const auto& x : g)
                while ((x.N / 16) % n != 0) n /= 2;
            return n;
        };
        max_n_a0 = mx(groups_a0);
        max_n_h1 = mx(groups_h1);
        max_n_a1f = mx(groups_a1f);
        max_n_a1r = mx(groups_a1r);
        sub_a0 = sub(groups_a0);
        sub_h1 = sub(groups_h1);
        sub_a1f = sub(groups_a1f);  // (the A1 forward plan prefers 64 columns: K runs to 3C)
        sub_a1r = sub(groups_a1r);
        upload(d_groups_a0, groups_a0, stream);
        upload(d_groups_h1, groups_h1, stream);
        upload(d_groups_a1f, groups_a1f, stream);
        upload(d_groups_a1r, groups_a1r, stream);
        if (hm.pre_linear_up) {
            // x = M0[:,0,:] P0: rows (node, 0) of M0 into x [N][C]; and
            // P0 d: rows of d [N][C] into direct_m0 [N][C]
            groups_cap.push_back(GemmGroup{0, C, C, NH * C, 0, C, C, 0, 0});
            groups_cap_r.push_back(GemmGroup{0, C, C, C, 0, 0, C, 0, 0});
            sub_cap = sub(groups_cap);
            upload(d_groups_cap, groups_cap, stream);
            upload(d_groups_cap_r, groups_cap_r, stream);
        }
        if (hm.field) {
            // per path: Z = H1p[l_in rows] W into its Z rows, Y = H1p_adj[l_out
            // rows] W^T into its Y rows
            int zo = 0, yo = 0;
            for (std::size_t p = 0; p < hm.field_paths.size(); ++p) {
                const auto& fp = hm.field_paths[p];
                const std::int64_t w = static_cast<std::int64_t>(p) * C * C;
                groups_fz.push_back(GemmGroup{w, C, C, NH * C, fp.l_in * fp.l_in * C, C, dm.field_zr * C, zo * C, C});
                groups_fy.push_back(GemmGroup{w, C, C, NH * C, fp.l_out * fp.l_out * C, C, dm.field_yr * C, yo * C, C});
                zo += 2 * fp.l_in + 1;
                yo += 2 * fp.l_out + 1;
            }
            sub_f = sub(groups_fz);
            upload(d_groups_fz, groups_fz, stream);
            upload(d_groups_fy, groups_fy, stream);
        }
    }

    // ------------------------------------------------------------- planning
    // Bytes of the untiled plan for a graph (workspace high-water).
    std::size_t untiled_bytes(std::int64_t n, std::int64_t e) const {
        const std::size_t C = hm.C, NY = hm.num_lm, NH = hm.num_LM, NLME = hm.num_lme;
        const std::size_t node = ((two_layer() ? 6 : 4) * NY + 4 * NH + 2 * NLME + 3) * C * 4 + 200;
        const std::size_t edge = (ks->record_floats() + (two_layer() ? NH * C : 0)) * 4 + 24 + 32 + 24;
        return node * n + edge * e;
    }

    bool two_layer() const { return !hm.single_layer; }

    static constexpr const char* kPlanSpeed = "mh0-direct-speed";
    static constexpr const char* kPlanRetained = "mh0-direct-capacity-retained";
    static constexpr const char* kPlanTiled = "mh0-dual-layer-tiled-v1";
    static constexpr const char* kPlanSingleTiled = "mh0-single-layer-tiled-v1";
    // the tiled plan of this model: three sweeps (two interactions) or one
    // (one interaction, mace_kokkos_evaluate.cpp:614-752)
    const char* tiled_plan() const { return two_layer() ? kPlanTiled : kPlanSingleTiled; }

    // Bytes of the tiled plan: graph-wide node state plus one tile's workspace.
    std::size_t tiled_bytes(std::int64_t n, std::int64_t e) const {
        const std::size_t C = hm.C, NY = hm.num_lm, NH = hm.num_LM, NLME = hm.num_lme;
        const std::size_t nt = std::min<std::int64_t>(n, tile_limit);
        const std::size_t et = n > 0 ? static_cast<std::size_t>(static_cast<double>(e) * nt / n) + 1 : 0;
        const std::size_t graph = (2 * NH + 2) * C * 4 * n + 64 * n + 24 * e;
        const std::size_t tile = ((two_layer() ? 6 : 4) * NY + 4 * NH + 2 * NLME + 3) * C * 4 * nt +
                                 ((ks->record_floats() + (two_layer() ? NH * C : 0)) * 4 + 24 + 32 + 24) * et;
        return graph + tile;
    }

    void choose_plan() {
        std::size_t free_b = 0, total_b = 0;
        SMX_HIP(hipMemGetInfo(&free_b, &total_b));
        plan_available = free_b + workspace_bytes();
        plan_untiled = untiled_bytes(N, E);
        plan_tiled = tiled_bytes(N, E);
        // mace_kokkos_runtime.cpp:2996-3030: each tiled plan admits its own
        // model kind, and neither admits field coupling
        if (hm.field && (debug_plan == kPlanTiled || debug_plan == kPlanSingleTiled))
            throw std::invalid_argument(debug_plan + " does not support field coupling");
        if (debug_plan == kPlanTiled && !two_layer())
            throw std::invalid_argument("mh0-dual-layer-tiled-v1 requires an ordinary two-layer MACE model");
        if (debug_plan == kPlanSingleTiled && two_layer())
            throw std::invalid_argument("mh0-single-layer-tiled-v1 requires single_layer_readout=true");
        if (debug_plan == kPlanTiled || debug_plan == kPlanSingleTiled) {
            tiled = true;
            plan_source = "debug_plan";
            plan_reason = "pinned by the debug plan request";
        } else if (debug_plan == kPlanSpeed || debug_plan == kPlanRetained) {
            tiled = false;
            plan_source = "debug_plan";
            plan_reason = "pinned by the debug plan request";
        } else if (request_profile == "speed") {
            tiled = false;
            plan_source = "profile";
            plan_reason = "the speed profile retains every edge's workspace";
        } else if (!allow_fixed) {
            tiled = false;
            plan_source = "planner";
            plan_reason = "fixed workspaces are not allowed; the retained direct plan is the capacity plan";
        } else {
            tiled = plan_untiled > plan_available / 10 * 7;
            plan_source = "planner";
            plan_reason = tiled ? "the retained workspace exceeds 70% of the available device memory"
                                : "the retained workspace fits 70% of the available device memory";
        }
        if (hm.field && tiled) {
            tiled = false;
            plan_reason = "field coupling runs in the retained direct plan";
        }

        if (N <= tile_limit && debug_plan != tiled_plan() && tiled) {
            tiled = false;
            plan_reason = "the graph fits one receiver tile";
        }
        // the direct plan's edge ids are 32-bit; the tiled plan's are 64-bit
        if (E > kMaxEdges && !tiled) {
            if (hm.field)
                throw std::invalid_argument("a MACEField model runs in the retained direct plan, whose edge count is "
                                            "limited to 2^31 - 4096");
            if (debug_plan == kPlanSpeed || debug_plan == kPlanRetained)
                throw std::invalid_argument(debug_plan + " limits the edge count to 2^31 - 4096; this graph needs " +
                                            tiled_plan());
            tiled = true;
            plan_reason = "the edge count exceeds the direct plan's 32-bit edge ids";
        }
    }

    const char* selected_plan() const {
        if (tiled) return tiled_plan();
        return request_profile == "speed" || debug_plan == kPlanSpeed ? kPlanSpeed : kPlanRetained;
    }

    static std::string json_string(const std::string& v) {
        std::string o = "\"";
        for (char c : v) {
            if (c == '"' || c == '\\') o += '\\';
            o += c;
        }
        return o + "\"";
    }

    // execution_plan_report (pybind mace_kokkos.cpp:271-297) as JSON
    std::string plan_report() const {
        const bool resolved = generation != 0;
        std::string o = "{";
        o += "\"requested_algorithm\":\"direct\",";
        o += "\"requested_profile\":" + json_string(request_profile) + ",";
        o += "\"allow_fixed_workspace\":" + std::string(allow_fixed ? "true" : "false") + ",";
        o += "\"debug_plan\":" + json_string(debug_plan) + ",";
        o += "\"selection_source\":" + json_string(plan_source) + ",";
        o += "\"state\":" + json_string(resolved ? "resolved" : "pending") + ",";
        o += "\"selected_id\":" + json_string(resolved ? selected_plan() : "") + ",";
        o += "\"selection_reason\":" + json_string(plan_reason) + ",";
        o += "\"available_bytes\":" + std::to_string(plan_available) + ",";
        o += "\"reserve_bytes\":" + std::to_string(plan_available - plan_available / 10 * 7) + ",";
        o += "\"boundary_attempt\":false,";
        o += "\"tiles\":" + std::to_string(tiles.size()) + ",";
        o += "\"max_tile_receivers\":" + std::to_string(max_tile_nr) + ",";
        o += "\"candidates\":[";
        o += "{\"id\":\"" + std::string(request_profile == "speed" ? kPlanSpeed : kPlanRetained) +
             "\",\"qualified\":true,\"estimated_bytes\":" + std::to_string(plan_untiled) +
             ",\"reason\":\"every edge's workspace retained\"},";
        o += "{\"id\":\"" + std::string(tiled_plan()) + "\",\"qualified\":" +
             std::string(allow_fixed || debug_plan == tiled_plan() ? "true" : "false") +
             ",\"estimated_bytes\":" + std::to_string(plan_tiled) + ",\"reason\":\"" +
             std::string(two_layer() ? "three sweeps" : "one sweep") + " over receiver tiles of at most " +
             std::to_string(tile_limit) + " receivers\"}]}";
        return o;
    }

    std::size_t workspace_bytes() const {
        std::size_t b = 0;
        for (const DevBuf* x : {&w_erec, &w_Phi0, &w_A0, &w_M0, &w_Phi1, &w_A1, &w_A1_adj, &w_M1, &w_dPhi1, &w_Wsrc,
                                &w_M0_adj, &w_A0_adj, &w_Phi0_adj, &w_node_forces, &w_exec, &d_xyz, &d_r})
            b += x->capacity();
        return b;
    }

    void build_tiles() {
        tiles.clear();
        const int limit = tiled ? std::max(1, tile_limit) : std::max(N, 1);
        for (int r0 = 0; r0 < N || (N == 0 && r0 == 0); r0 += limit) {
            TileView t;
            t.r0 = r0;
            t.nr = std::min(limit, N - r0);
            t.e0 = h_offsets[r0];
            t.ne = h_offsets[r0 + t.nr] - t.e0;
            if (t.ne > kMaxEdges) throw std::length_error("a receiver tile holds more than 2^31 - 4096 edges");
            tiles.push_back(t);
            if (N == 0) break;
        }
        if (tiled) {
            std::vector<int> rel;
            rel.reserve(static_cast<std::size_t>(N) + tiles.size());
            for (const auto& t : tiles)
                for (int i = 0; i <= t.nr; ++i) rel.push_back(static_cast<int>(h_offsets[t.r0 + i] - t.e0));
            upload(d_tile_off, rel, stream);
        } else {
            d_tile_off.release();
        }
        max_tile_nr = 0;
        max_tile_ne = 0;
        for (const auto& t : tiles) {
            max_tile_nr = std::max(max_tile_nr, t.nr);
            max_tile_ne = std::max(max_tile_ne, t.ne);
        }
        // node lists (local rows sorted by type), readout batches and
        // node-linear tiles depend only on the tiles' receiver ranges and the
        // node types: a graph rebuilt over the same atoms (a LAMMPS neighbour
        // list rebuild) keeps them
        std::vector<int> key{N, tiled ? 1 : 0, tiled ? tile_limit : 0};
        key.insert(key.end(), h_node_types.begin(), h_node_types.end());
        if (key != plan_key) {
            plan_key.swap(key);
            build_node_plans();
        }
        assign_tile_plans();
    }

    std::vector<int> plan_key;  // (N, tiling, node types) of the node plans on the device

    // one tile over all F feature nodes: the h1 (U, U^T), fz and fy plans
    void build_feature_tile() {
        for (PlanSet* p : {&ps_feat_h1, &ps_feat_fz, &ps_feat_fy}) {
            p->tiles.clear();
            p->rows.clear();
            p->sets.clear();
            p->tile_begin.assign(1, 0);
            p->set_begin.assign(1, 0);
        }
        auto add = [&](PlanSet& P, int group, int l) {
            const int start = static_cast<int>(P.rows.size());
            for (int m = 0; m < 2 * l + 1; ++m)
                for (int q = 0; q < F; ++q) P.rows.push_back(q << 4 | m);
            const int end = static_cast<int>(P.rows.size());
            const int t0 = static_cast<int>(P.tiles.size());
            for (int s0 = start; s0 < end; s0 += kGemmRows)
                P.tiles.push_back(GemmTile{s0, std::min(kGemmRows, end - s0), group});
            const int t1 = static_cast<int>(P.tiles.size());
            for (int t = t0; t < t1; t += kGemmShareWaves)
                P.sets.push_back(GemmTileSet{t, std::min(kGemmShareWaves, t1 - t)});
        };
        for (int l = 0; l <= hm.L_max; ++l) add(ps_feat_h1, l, l);
        for (std::size_t p = 0; p < hm.field_paths.size(); ++p) {
            add(ps_feat_fz, static_cast<int>(p), hm.field_paths[p].l_in);
            add(ps_feat_fy, static_cast<int>(p), hm.field_paths[p].l_out);
        }
        auto view = [&](PlanSet& P, const DevBuf& groups, int max_n, int n_sub) {
            P.tile_begin.push_back(P.tiles.size());
            P.set_begin.push_back(P.sets.size());
            upload(P.d_tiles, P.tiles, stream);
            upload(P.d_rows, P.rows, stream);
            upload(P.d_sets, P.sets, stream);
            GemmPlan g;
            g.n_sub = n_sub;
            g.tiles = P.d_tiles.as<GemmTile>();
            g.num_tiles = static_cast<int>(P.tiles.size());
            g.groups = groups.as<GemmGroup>();
            g.rows = P.d_rows.as<int>();
            g.max_n = max_n;
            g.sets = P.d_sets.as<GemmTileSet>();
            g.num_sets = static_cast<int>(P.sets.size());
            return g;
        };
        feature_tile = TileView{};
        feature_tile.r0 = 0;
        feature_tile.nr = F;
        feature_tile.e0 = 0;
        feature_tile.ne = E;
        feature_tile.h1 = view(ps_feat_h1, d_groups_h1, max_n_h1, sub_h1);
        feature_tile.fz = view(ps_feat_fz, d_groups_fz, hm.C, sub_f);
        feature_tile.fy = view(ps_feat_fy, d_groups_fy, hm.C, sub_f);
    }

    void build_node_plans() {
        h_node_list.clear();
        node_list_begin.clear();
        h_batches.clear();
        batch_begin.clear();
        for (PlanSet* p : {&ps_a0, &ps_h1, &ps_a1f, &ps_a1r, &ps_cap, &ps_fz, &ps_fy}) {
            p->tiles.clear();
            p->tile_begin.clear();
            p->rows.clear();
            p->sets.clear();
            p->set_begin.clear();
        }
        for (const auto& t : tiles) {
            const std::size_t base = h_node_list.size();
            node_list_begin.push_back(base);
            batch_begin.push_back(h_batches.size());
            std::vector<int> order(t.nr);
            std::iota(order.begin(), order.end(), 0);
            std::stable_sort(order.begin(), order.end(), [&](int a, int b) {
                return h_node_types[t.r0 + a] < h_node_types[t.r0 + b];
            });
            h_node_list.insert(h_node_list.end(), order.begin(), order.end());
            for (PlanSet* p : {&ps_a0, &ps_h1, &ps_a1f, &ps_a1r, &ps_cap, &ps_fz, &ps_fy}) {
                p->tile_begin.push_back(p->tiles.size());
                p->set_begin.push_back(p->sets.size());
            }
            // rows (node order[a..b), m in [0, 2l+1)) of one group, cut into
            // wave tiles, and the tiles into sets of up to kGemmShareWaves
            auto add = [&](PlanSet& P, int group, int l, int a, int b) {
                const int start = static_cast<int>(P.rows.size());
                for (int m = 0; m < 2 * l + 1; ++m)
                    for (int q = a; q < b; ++q) P.rows.push_back(order[q] << 4 | m);
                const int end = static_cast<int>(P.rows.size());
                const int t0 = static_cast<int>(P.tiles.size() - P.tile_begin.back());
                for (int s0 = start; s0 < end; s0 += kGemmRows)
                    P.tiles.push_back(GemmTile{s0, std::min(kGemmRows, end - s0), group});
                const int t1 = static_cast<int>(P.tiles.size() - P.tile_begin.back());
                for (int t = t0; t < t1; t += kGemmShareWaves)
                    P.sets.push_back(GemmTileSet{t, std::min(kGemmShareWaves, t1 - t)});
            };
            for (int p = 0; p < t.nr;) {
                int q = p;
                const int type = h_node_types[t.r0 + order[p]];
                while (q < t.nr && h_node_types[t.r0 + order[q]] == type) ++q;
                for (int l = 0; l <= hm.l_max; ++l) add(ps_a0, type * (hm.l_max + 1) + l, l, p, q);
                for (int s0 = p; s0 < q; s0 += kReadoutBatch)
                    h_batches.push_back(NodeBatch{static_cast<int>(s0), std::min(kReadoutBatch, q - s0)});
                p = q;
            }
            for (int l = 0; l <= hm.L_max; ++l) add(ps_h1, l, l, 0, t.nr);
            if (hm.pre_linear_up) add(ps_cap, 0, 0, 0, t.nr);
            for (std::size_t p = 0; p < hm.field_paths.size(); ++p) {
                add(ps_fz, static_cast<int>(p), hm.field_paths[p].l_in, 0, t.nr);
                add(ps_fy, static_cast<int>(p), hm.field_paths[p].l_out, 0, t.nr);
            }
            for (int l = 0; l <= hm.l_max; ++l) {
                if (hm.num_e[l] == 0) continue;
                add(ps_a1f, l, l, 0, t.nr);
                add(ps_a1r, l, l, 0, t.nr);
            }
        }
        batch_begin.push_back(h_batches.size());
        for (PlanSet* p : {&ps_a0, &ps_h1, &ps_a1f, &ps_a1r, &ps_cap, &ps_fz, &ps_fy}) {
            p->tile_begin.push_back(p->tiles.size());
            p->set_begin.push_back(p->sets.size());
            upload(p->d_tiles, p->tiles, stream);
            upload(p->d_rows, p->rows, stream);
            upload(p->d_sets, p->sets, stream);
        }
        upload(d_node_list, h_node_list, stream);
        upload(d_batches, h_batches, stream);
    }

    // the tiles' views of the node plans, and the touched sources of each
    // tile (these depend on the edges)
    void assign_tile_plans() {
        auto view = [&](const PlanSet& P, std::size_t ti, const DevBuf& groups, int max_n, int n_sub) {
            GemmPlan g;
            g.n_sub = n_sub;
            g.tiles = P.d_tiles.as<GemmTile>() + P.tile_begin[ti];
            g.num_tiles = static_cast<int>(P.tile_begin[ti + 1] - P.tile_begin[ti]);
            g.groups = groups.as<GemmGroup>();
            g.rows = P.d_rows.as<int>();
            g.max_n = max_n;
            g.sets = P.d_sets.as<GemmTileSet>() + P.set_begin[ti];
            g.num_sets = static_cast<int>(P.set_begin[ti + 1] - P.set_begin[ti]);
            return g;
        };
        for (std::size_t ti = 0; ti < tiles.size(); ++ti) {
            tiles[ti].a0 = view(ps_a0, ti, d_groups_a0, max_n_a0, sub_a0);
            tiles[ti].h1 = view(ps_h1, ti, d_groups_h1, max_n_h1, sub_h1);
            tiles[ti].a1f = view(ps_a1f, ti, d_groups_a1f, max_n_a1f, sub_a1f);
            tiles[ti].a1f.narrow = true;
            tiles[ti].a1r = view(ps_a1r, ti, d_groups_a1r, max_n_a1r, sub_a1r);
            if (hm.pre_linear_up) {
                tiles[ti].cap = view(ps_cap, ti, d_groups_cap, hm.C, sub_cap);
                tiles[ti].cap_r = view(ps_cap, ti, d_groups_cap_r, hm.C, sub_cap);
            }
            if (hm.field) {
                tiles[ti].fz = view(ps_fz, ti, d_groups_fz, hm.C, sub_f);
                tiles[ti].fy = view(ps_fy, ti, d_groups_fy, hm.C, sub_f);
            }
            tiles[ti].node_list = d_node_list.as<int>() + node_list_begin[ti];
            tiles[ti].batches = d_batches.as<NodeBatch>() + batch_begin[ti];
            tiles[ti].num_batches = static_cast<int>(batch_begin[ti + 1] - batch_begin[ti]);
        }
        // touched sources of every tile (tiled plan only)
        touched_begin.assign(1, 0);
        if (tiled && N > 0) {
            DevBuf bitmap, counts, one;
            const int words = F / 32 + 1;
            bitmap.ensure(sizeof(std::uint32_t) * words);
            counts.ensure(sizeof(int) * words);
            one.ensure(sizeof(int) * F);
            std::vector<int> all;
            std::vector<int> host(F);
            for (auto& t : tiles) {
                const int cnt = build_touched_sources(F, t.e0, t.ne, d_neigh.as<int>(), bitmap.as<std::uint32_t>(),
                                                      counts.as<int>(), one.as<int>(), stream);
                if (cnt > 0)
                    SMX_HIP(hipMemcpy(host.data(), one.as<int>(), sizeof(int) * cnt, hipMemcpyDeviceToHost));
                all.insert(all.end(), host.begin(), host.begin() + cnt);
                touched_begin.push_back(all.size());
            }
            upload(d_touched, all, stream);
            for (std::size_t ti = 0; ti < tiles.size(); ++ti) {
                tiles[ti].touched = d_touched.as<int>() + touched_begin[ti];
                tiles[ti].touched_count = static_cast<int>(touched_begin[ti + 1] - touched_begin[ti]);
            }
        }
    }

    void ensure_workspace() {
        const std::size_t C = hm.C, NY = hm.num_lm, NH = hm.num_LM, NLME = hm.num_lme;
        const std::size_t n = std::max(N, 1), tn = std::max(max_tile_nr, 1);
        const std::size_t te = std::max<std::int64_t>(max_tile_ne, 1);
        auto f = [&](DevBuf& b, std::size_t count) { return static_cast<float*>(b.ensure(count * sizeof(float))); };
        ws.erec = f(w_erec, te * ks->record_floats());
        ws.erec_b = ws.erec + te * ks->record_forward_floats();  // reverse parts after the forward parts
        ws.Phi0 = f(w_Phi0, tn * NY * C);
        ws.A0 = f(w_A0, tn * NY * C);
        ws.M0 = f(w_M0, tn * NH * C);
        // (no Phi1, A1 or per-edge source terms with one interaction)
        const std::size_t two = two_layer() ? 1 : 0;
        ws.Phi1 = f(w_Phi1, two * tn * NLME * C);
        ws.A1 = f(w_A1, two * tn * NY * C);
        ws.A1_adj = f(w_A1_adj, two * tn * NY * C);
        ws.M1 = f(w_M1, tn * C);
        ws.dPhi1 = f(w_dPhi1, two * tn * NLME * C);
        ws.Wsrc = f(w_Wsrc, two * te * NH * C);
        ws.M0_adj = f(w_M0_adj, tn * NH * C);
        ws.A0_adj = f(w_A0_adj, tn * NY * C);
        ws.Phi0_adj = f(w_Phi0_adj, tn * NY * C);
        ws.node_forces = static_cast<double*>(w_node_forces.ensure(te * 3 * sizeof(double)));
        if (hm.A0_scaled || hm.A1_scaled) {
            double* d = static_cast<double*>(w_density.ensure(4 * tn * sizeof(double)));
            ws.dens_s0 = d;
            ws.dens_s1 = d + tn;
            ws.dens_dot0 = d + 2 * tn;
            ws.dens_dot1 = d + 3 * tn;
        }
        const std::size_t nf = std::max(F, 1);
        ws.H1 = f(g_H1, nf * NH * C);
        ws.H1_adj = f(g_H1_adj, nf * NH * C);
        ws.xaff = f(g_xaff, (hm.field ? nf : n) * C);
        ws.direct = f(g_direct, n * C);
        if (hm.pre_linear_up) ws.direct_m0 = f(g_direct_m0, n * C);
        if (hm.field) {
            ws.H1p = f(g_H1p, nf * NH * C);
            ws.H1f = f(g_H1f, nf * NH * C);
            ws.H1p_adj = f(g_H1p_adj, nf * NH * C);
            ws.fzy = f(g_fzy, nf * static_cast<std::size_t>(std::max(dm.field_zr, dm.field_yr)) * C);
            ws.field_part = static_cast<double*>(d_field_part.ensure(nf * 3 * sizeof(double)));
            d_field_adj.ensure(3 * sizeof(double));
        }
        ws.node_energies = static_cast<double*>(d_node_energies.ensure(n * sizeof(double)));
        d_atom_forces.ensure(nf * 3 * sizeof(double));
        if (feature_graph()) d_h1_exchange.ensure(nf * NH * C * sizeof(float));
        d_virial.ensure(9 * sizeof(double));
        d_stress.ensure(9 * sizeof(double));
        d_stress_partial.ensure(static_cast<std::size_t>(stress_blocks) * 9 * sizeof(double));
        d_total.ensure(sizeof(double));
        // xyz/r of one tile (host edge vectors of the whole graph grow them
        // when they are given)
        d_xyz.ensure(te * 3 * sizeof(double));
        d_r.ensure(te * sizeof(double));
        d_invalid.ensure(sizeof(int));
        d_positions.ensure(n * 3 * sizeof(double));
        d_disp.ensure(n * 3 * sizeof(double));
    }

    void validate_types(int n, const int* types) const {
        for (int i = 0; i < n; ++i)
            if (types[i] < 0 || types[i] >= hm.num_elements)
                throw std::invalid_argument("node type index is out of range");
    }

    // receiver CSR on the device -> schedule, tiles, plans, workspace, token
    // wide_offsets: the CSR's offsets are the 64-bit d_offsets64 (the device
    // neighbour list's; d_offsets is absent beyond kMaxEdges edges), else the
    // 32-bit d_offsets.  d_offsets64 serves the schedule and the host copy
    // only and is released on the way out, also when a step throws.
    std::uint64_t finish_graph(bool wide_offsets = false) {
        struct Release {
            DevBuf& b;
            ~Release() { b.release(); }
        } release_offsets64{d_offsets64};
        if (!wide_offsets) d_offsets64.release();
        // the plan first: it sets the width of the source transpose
        choose_plan();
        d_receivers.ensure(std::max<std::int64_t>(E, 1) * sizeof(int));
        d_counts.ensure(std::max(F, 1) * sizeof(int));
        if (wide_offsets)
            launch_receivers(N, d_offsets64.as<long long>(), d_receivers.as<int>(), stream);
        else
            launch_receivers(N, d_offsets.as<int>(), d_receivers.as<int>(), stream);
        if (tiled) {
            for (DevBuf* b : {&d_soff, &d_sedges}) b->release();
            d_soff64.ensure((static_cast<std::size_t>(F) + 1) * sizeof(long long));
            d_sedges64.ensure(std::max<std::int64_t>(E, 1) * sizeof(long long));
            launch_transpose(F, E, d_neigh.as<int>(), d_soff64.as<long long>(), d_sedges64.as<long long>(),
                             d_counts.as<int>(), stream);
        } else {
            for (DevBuf* b : {&d_soff64, &d_sedges64}) b->release();
            d_soff.ensure((static_cast<std::size_t>(F) + 1) * sizeof(int));
            d_sedges.ensure(std::max<std::int64_t>(E, 1) * sizeof(int));
            launch_transpose(F, E, d_neigh.as<int>(), d_soff.as<int>(), d_sedges.as<int>(), d_counts.as<int>(),
                             stream);
        }
        if (static_cast<std::int64_t>(h_offsets.size()) != static_cast<std::int64_t>(N) + 1) {
            h_offsets.resize(static_cast<std::size_t>(N) + 1);
            if (wide_offsets) {
                SMX_HIP(hipMemcpy(h_offsets.data(), d_offsets64.as<long long>(), sizeof(long long) * (N + 1),
                                  hipMemcpyDeviceToHost));
            } else {
                std::vector<int> off(static_cast<std::size_t>(N) + 1);
                SMX_HIP(hipMemcpy(off.data(), d_offsets.as<int>(), sizeof(int) * (N + 1), hipMemcpyDeviceToHost));
                h_offsets.assign(off.begin(), off.end());
            }
        }
        prepare_pair_tables();
        build_tiles();
        if (hm.field && feature_graph()) build_feature_tile();
        ensure_workspace();
        SMX_HIP(hipStreamSynchronize(stream));
        evaluated = false;
        generation = next_generation++;
        return generation;
    }

    // mace.cpp:119-214 / compact_radial.cpp:368-387: with the Agnesi
    // transform every pair of active types (a <= b) has its own tables,
    // tabulated when the active types change; edges select theirs by pair.
    void prepare_pair_tables() {
        if (!hm.agnesi) return;
        std::vector<int> act(h_node_types.begin(), h_node_types.end());
        act.insert(act.end(), h_feature_types.begin(), h_feature_types.end());
        std::sort(act.begin(), act.end());
        act.erase(std::unique(act.begin(), act.end()), act.end());
        if (act.empty()) act.push_back(0);
        // the pinned active types serve every graph whose types they cover
        if (!pinned_active.empty() && std::includes(pinned_active.begin(), pinned_active.end(), act.begin(), act.end()))
            act = pinned_active;
        tabulate_pairs(act);
        const int na = static_cast<int>(act.size());
        int* ep = static_cast<int*>(d_edge_pair.ensure(std::max<std::int64_t>(E, 1) * sizeof(int)));
        int* bad = static_cast<int*>(d_counts.ensure(std::max(N, 1) * sizeof(int)));
        launch_fill_zero(reinterpret_cast<float*>(bad), 1, stream);
        launch_edge_pairs(E, d_receivers.as<int>(), d_node_types.as<int>(), d_neigh_types.as<int>(),
                          d_type_to_active.as<int>(), na, ep, bad, stream);
        int nbad = 0;
        SMX_HIP(hipMemcpyAsync(&nbad, bad, sizeof(int), hipMemcpyDeviceToHost, stream));
        SMX_HIP(hipStreamSynchronize(stream));
        if (nbad > 0) throw std::invalid_argument("a neighbour type is not among the graph's node types");
    }

    // prepare_active_types (lifecycle.cpp:3949; pybind mace_kokkos.cpp:2076):
    // tabulate the per-pair radial tables of these model types now, and keep
    // them for every later graph whose types they cover.
    void prepare_active_types(std::vector<int> types) {
        require_idle();  // the radial tables of a pending phase stay as they are
        for (int t : types)
            if (t < 0 || t >= hm.num_elements) throw std::invalid_argument("active type index is out of range");
        std::sort(types.begin(), types.end());
        types.erase(std::unique(types.begin(), types.end()), types.end());
        pinned_active = types;
        if (hm.agnesi && !types.empty()) tabulate_pairs(types);
    }

    // per-pair tables of the active types act (a <= b pairs), when they change
    void tabulate_pairs(const std::vector<int>& act) {
        const int na = static_cast<int>(act.size());
        if (act != pair_active) {
            std::vector<float> R0, R1, t0, t1;
            std::vector<double> D0, D1, u0, u1;
            for (int a = 0; a < na; ++a)
                for (int b = a; b < na; ++b) {
                    hm.pair_tables(act[a], act[b], t0, t1, u0, u1);
                    R0.insert(R0.end(), t0.begin(), t0.end());
                    R1.insert(R1.end(), t1.begin(), t1.end());
                    D0.insert(D0.end(), u0.begin(), u0.end());
                    D1.insert(D1.end(), u1.begin(), u1.end());
                }
            dm.R0c = reinterpret_cast<const float4*>(upload(d_pair_R0, R0, stream));
            dm.R1c = reinterpret_cast<const float4*>(upload(d_pair_R1, R1, stream));
            if (hm.A0_scaled) dm.dens0 = upload(d_pair_D0, D0, stream);
            if (hm.A1_scaled) dm.dens1 = upload(d_pair_D1, D1, stream);
            std::vector<int> t2a(hm.num_elements, -1);
            for (int a = 0; a < na; ++a) t2a[act[a]] = a;
            upload(d_type_to_active, t2a, stream);
            pair_active = act;
        }
    }

    void require_idle() const {
        if (phase != Phase::idle)
            throw std::logic_error("A prepared factorized graph cannot change during a distributed evaluation.");
    }

    // num_features > n: a feature graph whose node order (receivers first)
    // and h_feature_of / h_feature_types the caller has set
    std::uint64_t prepare_graph_host(int n, const int* node_types, const int* num_neigh, std::int64_t num_edges,
                                     const int* neigh, const int* neigh_types, int num_features = -1) {
        require_idle();
        const bool plain = num_features < 0;
        if (plain) num_features = n;
        if (n < 0) throw std::invalid_argument("num_nodes must be non-negative");
        if (num_edges < 0 || num_edges > kMaxEdges)
            throw std::invalid_argument("edge count exceeds the 32-bit graph limit");
        validate_types(n, node_types);
        std::vector<int> off(n + 1, 0);
        std::int64_t total = 0;
        for (int i = 0; i < n; ++i) {
            if (num_neigh[i] < 0) throw std::invalid_argument("num_neigh must be non-negative");
            total += num_neigh[i];
            if (total > kMaxEdges) throw std::invalid_argument("edge count exceeds the 32-bit graph limit");
            off[i + 1] = static_cast<int>(total);
        }
        if (total != num_edges) throw std::invalid_argument("num_neigh does not sum to the number of edges");
        for (std::int64_t e = 0; e < num_edges; ++e) {
            if (neigh[e] < 0 || neigh[e] >= num_features)
                throw std::invalid_argument("neighbour index is out of range");
            if (neigh_types[e] < 0 || neigh_types[e] >= hm.num_elements)
                throw std::invalid_argument("neighbour type index is out of range");
        }
        invalidate_graph();
        if (plain) {
            h_feature_of.clear();
            h_feature_types.clear();
            feature_prepared = false;
        }
        N = n;
        F = num_features;
        E = num_edges;
        h_node_types.assign(node_types, node_types + n);
        h_offsets.assign(off.begin(), off.end());
        if (!h_feature_of.empty()) upload(d_feature_of, h_feature_of, stream);
        upload(d_node_types, h_node_types, stream);
        upload(d_offsets, off, stream);
        upload(d_neigh, std::vector<int>(neigh, neigh + E), stream);
        upload(d_neigh_types, std::vector<int>(neigh_types, neigh_types + E), stream);
        geom = Geometry::none;
        return finish_graph();
    }

    std::uint64_t prepare_graph_device(int n, const int* node_types, const int* num_neigh, std::int64_t num_edges,
                                       const int* neigh, const int* neigh_types) {
        // The CSR is validated on a host copy, like the host path.
        std::vector<int> t(n), nn(n), nb(num_edges), nt(num_edges);
        if (n > 0) {
            SMX_HIP(hipMemcpy(t.data(), node_types, sizeof(int) * n, hipMemcpyDeviceToHost));
            SMX_HIP(hipMemcpy(nn.data(), num_neigh, sizeof(int) * n, hipMemcpyDeviceToHost));
        }
        if (num_edges > 0) {
            SMX_HIP(hipMemcpy(nb.data(), neigh, sizeof(int) * num_edges, hipMemcpyDeviceToHost));
            SMX_HIP(hipMemcpy(nt.data(), neigh_types, sizeof(int) * num_edges, hipMemcpyDeviceToHost));
        }
        return prepare_graph_host(n, t.data(), nn.data(), num_edges, nb.data(), nt.data());
    }

    // prepare_factorized_graph with feature nodes (lifecycle.cpp:949-1104): the
    // caller's checks, then the feature nodes renumbered receivers first
    std::uint64_t prepare_feature_graph_host(int nr, int nf, const int* receiver_features, const int* node_types,
                                             const int* feature_types, const int* num_neigh, std::int64_t num_edges,
                                             const int* neigh, const int* neigh_types) {
        require_idle();
        if (nr < 0 || nf < nr) throw std::invalid_argument("Prepared Execution R1 graph extents are inconsistent.");
        if (num_edges < 0 || num_edges > kMaxEdges)
            throw std::invalid_argument("edge count exceeds the 32-bit graph limit");
        validate_types(nr, node_types);
        validate_types(nf, feature_types);
        std::vector<int> node_of(nf, -1);
        for (int ii = 0; ii < nr; ++ii) {
            const int f = receiver_features[ii];
            if (f < 0 || f >= nf) throw std::out_of_range("Prepared Execution R1 receiver feature index is out of range.");
            if (node_types[ii] != feature_types[f])
                throw std::invalid_argument("Prepared Execution R1 receiver and feature types disagree.");
            if (node_of[f] >= 0)
                throw std::invalid_argument("Prepared Execution R1 receiver feature indices must be unique.");
            node_of[f] = ii;
        }
        std::vector<int> feature_of(nf);
        for (int ii = 0; ii < nr; ++ii) feature_of[ii] = receiver_features[ii];
        int k = nr;
        for (int f = 0; f < nf; ++f)
            if (node_of[f] < 0) {
                node_of[f] = k;
                feature_of[k++] = f;
            }
        std::vector<int> src(num_edges);
        for (std::int64_t e = 0; e < num_edges; ++e) {
            const int f = neigh[e];
            if (f < 0 || f >= nf) throw std::out_of_range("Prepared Execution R1 source index is out of range.");
            if (neigh_types[e] != feature_types[f])
                throw std::invalid_argument("a neighbour type differs from its feature node's type");
            src[e] = node_of[f];
        }
        invalidate_graph();
        bool identity = true;
        for (int q = 0; q < nf && identity; ++q) identity = feature_of[q] == q;
        h_feature_types.resize(nf);
        for (int q = 0; q < nf; ++q) h_feature_types[q] = feature_types[feature_of[q]];
        if (identity)
            h_feature_of.clear();
        else
            h_feature_of.swap(feature_of);
        upload(d_edge_src_feature, std::vector<int>(neigh, neigh + num_edges), stream);
        upload(d_recv_feature, std::vector<int>(receiver_features, receiver_features + nr), stream);
        feature_prepared = true;
        if (nf == nr && identity) h_feature_types.clear();
        return prepare_graph_host(nr, node_types, num_neigh, num_edges, src.data(), neigh_types, nf);
    }

    // ------------------------------------------------- split-phase evaluation
    // edge vectors of the whole graph from the caller (host: checked here;
    // device: counted by a kernel and read back)
    void take_xyz(const double* xyz, const double* r, bool on_device) {
        fpos_mode = false;
        if (E > 0 && (!xyz || !r)) throw std::invalid_argument("xyz and r are required");
        d_xyz.ensure(std::max<std::int64_t>(E, 1) * 3 * sizeof(double));
        d_r.ensure(std::max<std::int64_t>(E, 1) * sizeof(double));
        xyz_host = true;
        if (!on_device) {
            for (std::int64_t e = 0; e < E; ++e)
                if (!std::isfinite(r[e]) || !(r[e] > 0.0) || !std::isfinite(xyz[3 * e]) ||
                    !std::isfinite(xyz[3 * e + 1]) || !std::isfinite(xyz[3 * e + 2]))
                    throw std::invalid_argument("MACE graph has an invalid distance or displacement vector");
            if (E > 0) {
                SMX_HIP(hipMemcpyAsync(d_xyz.as<double>(), xyz, E * 3 * sizeof(double), hipMemcpyHostToDevice, stream));
                SMX_HIP(hipMemcpyAsync(d_r.as<double>(), r, E * sizeof(double), hipMemcpyHostToDevice, stream));
            }
            return;
        }
        if (E > 0) {
            SMX_HIP(hipMemcpyAsync(d_xyz.as<double>(), xyz, E * 3 * sizeof(double), hipMemcpyDeviceToDevice, stream));
            SMX_HIP(hipMemcpyAsync(d_r.as<double>(), r, E * sizeof(double), hipMemcpyDeviceToDevice, stream));
        }
        launch_fill_zero(reinterpret_cast<float*>(d_invalid.as<int>()), 1, stream);
        launch_count_invalid_edges(E, d_xyz.as<double>(), d_r.as<double>(), d_invalid.as<int>(), stream);
        if (read_flag(d_invalid) > 0)
            throw std::invalid_argument("MACE graph has an invalid distance or displacement vector");
    }

    // the positions form (begin_factorized_distributed_positions_evaluation,
    // mace_kokkos_evaluate.cpp:1615-1656): 3 per feature node, host or device
    void take_feature_positions(const double* pos, bool on_device) {
        if (!feature_prepared)
            throw std::invalid_argument("the positions form takes a graph prepared with feature nodes");
        if (F > 0 && !pos) throw std::invalid_argument("feature positions are required");
        if (!on_device)
            for (std::int64_t q = 0; q < 3 * static_cast<std::int64_t>(F); ++q)
                if (!std::isfinite(pos[q])) throw std::invalid_argument("positions must be finite");
        double* dst = static_cast<double*>(d_fpos.ensure(std::max(F, 1) * 3 * sizeof(double)));
        if (F > 0)
            SMX_HIP(hipMemcpyAsync(dst, pos, static_cast<std::size_t>(F) * 3 * sizeof(double),
                                   on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, stream));
        // edge vectors of the whole graph (direct plan) or of one tile at a
        // time (tiled plan), formed where the plan forms them
        d_xyz.ensure(std::max<std::int64_t>(tiled ? max_tile_ne : E, 1) * 3 * sizeof(double));
        d_r.ensure(std::max<std::int64_t>(tiled ? max_tile_ne : E, 1) * sizeof(double));
        xyz_host = false;
        fpos_mode = true;
        launch_fill_zero(reinterpret_cast<float*>(d_invalid.as<int>()), 1, stream);
    }

    void raise_if_invalid_feature_geometry() {
        if (read_flag(d_invalid) > 0) {
            evaluated = false;
            throw std::invalid_argument("feature positions produced an invalid edge geometry (zero-length or "
                                        "non-finite edges)");
        }
    }

    void check_phase_graph(std::uint64_t token, int nr, int nf) const {
        if (phase != Phase::idle) throw std::logic_error("A factorized distributed evaluation is already active.");
        check_generation(token);
        if (nr != N || nf != F)
            throw std::invalid_argument("Distributed factorized graph or geometry extents are inconsistent.");
    }

    // a one-interaction model needs no exchanged features: one call over the
    // feature graph (mace_kokkos_evaluate.cpp:1495-1552)
    void single_layer_distributed(std::uint64_t token, int nr, int nf, const double* xyz, const double* r,
                                  const double* feature_positions, bool on_device) {
        check_phase_graph(token, nr, nf);
        if (two_layer())
            throw std::invalid_argument("Complete distributed evaluation requires a standard single-layer model.");
        if (feature_positions)
            take_feature_positions(feature_positions, on_device);
        else
            take_xyz(xyz, r, on_device);
        evaluate(nullptr);
        finish_call(true);
    }

    // begin_factorized_distributed_evaluation: layer 1 up to H1 of the receivers
    void begin_distributed(std::uint64_t token, int nr, int nf, const double* xyz, const double* r,
                           const double* feature_positions, bool on_device) {
        check_phase_graph(token, nr, nf);
        if (!two_layer())
            throw std::invalid_argument(
                "a one-interaction model is evaluated in one call (compute_factorized_single_layer_distributed_evaluation)");
        evaluated = false;
        if (feature_positions)
            take_feature_positions(feature_positions, on_device);
        else
            take_xyz(xyz, r, on_device);
        bind_field();
        for (auto& t : tiles) {
            t.r = tile_r(t);
            t.xyz = tile_xyz(t);
        }
        zero_a1_if_needed();
        if (tiled) {
            tiled_sweep_h1(nullptr);
            sync();
            if (fpos_mode) raise_if_invalid_feature_geometry();
            phase = Phase::prefix_complete;
            return;
        }
        TileView& t = tiles[0];
        tile_geometry(t, nullptr);
        // a field-coupled model exchanges H1 before the field (H1p = M0 P + b):
        // the field and linear_up then run over every feature node
        ws.field_product_only = hm.field;
        ks->layer1_forward(dm, view(), t, ws, true, stream, timer.get());
        ws.field_product_only = false;
        sync();
        if (fpos_mode) raise_if_invalid_feature_geometry();
        phase = Phase::prefix_complete;
    }

    // the H1 rows of every feature node in (caller order), layer 2, and the
    // H1 adjoint of every feature node out (caller order, in d_h1_exchange or,
    // for the caller's own order, the workspace)
    void continue_distributed(const float* h1, std::int64_t rows, bool on_device) {
        if (phase != Phase::prefix_complete)
            throw std::logic_error("Distributed factorized middle phase requires a completed prefix.");
        if (!h1 || rows < F) throw std::invalid_argument("Communicated H1 does not match the distributed graph.");
        const std::size_t row = static_cast<std::size_t>(hm.num_LM) * hm.C;
        const bool permuted = !h_feature_of.empty();
        float* rows_in = hm.field ? ws.H1p : ws.H1;  // the exchanged H1 rows
        float* dst = permuted ? d_h1_exchange.as<float>() : rows_in;
        try {
            if (F > 0)
                SMX_HIP(hipMemcpyAsync(dst, h1, F * row * sizeof(float),
                                       on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, stream));
            if (permuted)
                launch_gather_rows(F, static_cast<int>(row), d_feature_of.as<int>(), dst, rows_in, stream);
            const DeviceGraph g = view();
            const TileView& t = tiles[0];
            if (hm.field) ks->field_features(dm, feature_tile, ws, stream, timer.get());
            if (tiled) {
                tiled_sweep_layer2(nullptr);
            } else {
                ks->layer2(dm, g, t, ws, stream, timer.get());
                ks->source_adjoint_all(g, ws, tile_r(t), hm.r_cut, stream, timer.get());
            }
            // a field-coupled model's exchanged adjoint is H1p's (the
            // readout's direct adjoint enters the receivers' rows here)
            if (hm.field) ks->field_features_reverse(dm, feature_tile, ws, N, stream, timer.get());
            if (permuted)
                launch_scatter_rows(F, static_cast<int>(row), d_feature_of.as<int>(), hm.field ? ws.H1p_adj : ws.H1_adj,
                                    d_h1_exchange.as<float>(), stream);
            sync();
        } catch (...) {
            phase = Phase::idle;
            throw;
        }
        phase = Phase::middle_complete;
    }

    // the H1 adjoint the caller exchanges (caller order, F rows)
    float* h1_adjoint_exchange() {
        if (!h_feature_of.empty()) return d_h1_exchange.as<float>();
        return hm.field ? ws.H1p_adj : ws.H1_adj;
    }

    // finish_factorized_distributed_evaluation: the receivers' H1 adjoint (the
    // exchange buffer, summed over the owners' ghost images by the caller, or
    // rows given here) -> layer-1 reverse, energies and edge forces
    void finish_distributed(const float* h1_adj, std::int64_t rows, bool on_device) {
        if (phase != Phase::middle_complete)
            throw std::logic_error("Distributed factorized suffix requires a completed middle phase.");
        const std::size_t row = static_cast<std::size_t>(hm.num_LM) * hm.C;
        try {
            if (h1_adj) {
                if (rows < F) throw std::invalid_argument("the H1 adjoint does not match the distributed graph");
                if (F > 0)
                    SMX_HIP(hipMemcpyAsync(h1_adjoint_exchange(), h1_adj, F * row * sizeof(float),
                                           on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, stream));
            }
            if (!h_feature_of.empty())
                launch_gather_rows(N, static_cast<int>(row), d_feature_of.as<int>(), d_h1_exchange.as<float>(),
                                   hm.field ? ws.H1p_adj : ws.H1_adj, stream);
            if (tiled) {
                tiled_sweep_reverse(nullptr);
            } else {
                ws.field_reverse_done = hm.field;
                ks->layer1_reverse(dm, view(), tiles[0], ws, true, stream, timer.get());
                ws.field_reverse_done = false;
            }
            sync();
        } catch (...) {
            phase = Phase::idle;
            throw;
        }
        phase = Phase::idle;
        evaluated = true;
    }

    // A receiver CSR that this library's own kernels built and checked on the
    // device (the LAMMPS topology): offsets come from the host, the edge
    // arrays are copied device to device, only the node types come back.
    std::uint64_t prepare_graph_checked(int n, const int* node_types, const std::vector<int>& offsets,
                                        std::int64_t num_edges, const int* neigh, const int* neigh_types) {
        require_idle();
        invalidate_graph();
        N = F = n;
        h_feature_of.clear();
        h_feature_types.clear();
        feature_prepared = false;
        E = num_edges;
        h_node_types.resize(n);
        if (n > 0) SMX_HIP(hipMemcpy(h_node_types.data(), node_types, sizeof(int) * n, hipMemcpyDeviceToHost));
        validate_types(n, h_node_types.data());
        h_offsets.assign(offsets.begin(), offsets.end());
        upload(d_offsets, offsets, stream);
        int* nt = static_cast<int*>(d_node_types.ensure(std::max(n, 1) * sizeof(int)));
        int* nb = static_cast<int*>(d_neigh.ensure(std::max<std::int64_t>(E, 1) * sizeof(int)));
        int* nbt = static_cast<int*>(d_neigh_types.ensure(std::max<std::int64_t>(E, 1) * sizeof(int)));
        if (n > 0) SMX_HIP(hipMemcpyAsync(nt, node_types, sizeof(int) * n, hipMemcpyDeviceToDevice, stream));
        if (E > 0) {
            SMX_HIP(hipMemcpyAsync(nb, neigh, sizeof(int) * E, hipMemcpyDeviceToDevice, stream));
            SMX_HIP(hipMemcpyAsync(nbt, neigh_types, sizeof(int) * E, hipMemcpyDeviceToDevice, stream));
        }
        geom = Geometry::none;
        return finish_graph();
    }

    std::pair<std::uint64_t, std::int64_t> prepare_periodic(int n, const int* node_types, const double* positions,
                                                            const double* cell_, const double* inv_,
                                                            double cutoff) {
        require_idle();
        if (n < 0) throw std::invalid_argument("num_nodes must be non-negative");
        validate_types(n, node_types);
        invalidate_graph();
        // release the previous graph's edge arrays first (capacity runs)
        for (DevBuf* b : {&d_neigh, &d_neigh_types, &d_receivers, &d_sedges, &d_sedges64, &d_images, &d_ref_edges,
                          &d_edge_pair})
            b->release();
        NeighborResult nr;
        struct Guard {
            NeighborResult& r;
            ~Guard() {
                for (void* p : {static_cast<void*>(r.num_neigh), static_cast<void*>(r.offsets),
                                static_cast<void*>(r.sources), static_cast<void*>(r.images),
                                static_cast<void*>(r.wfrac), static_cast<void*>(r.shifts),
                                static_cast<void*>(r.fractional_xyz), static_cast<void*>(r.offsets64)})
                    if (p) (void)hipFree(p);
            }
        } guard{nr};
        // 64-bit offsets: graphs beyond kMaxEdges edges run in the tiled plan
        build_neighbor_list(n, positions, cell_, inv_, cutoff, false, nr, stream, true);
        N = F = n;
        h_feature_of.clear();
        h_feature_types.clear();
        feature_prepared = false;
        E = nr.num_edges;
        h_node_types.assign(node_types, node_types + n);
        upload(d_node_types, h_node_types, stream);
        d_offsets.adopt(nr.offsets, (N + 1) * sizeof(int));  // null beyond kMaxEdges edges
        nr.offsets = nullptr;
        d_offsets64.adopt(nr.offsets64, (N + 1) * sizeof(long long));
        nr.offsets64 = nullptr;
        d_neigh.adopt(nr.sources, std::max<std::int64_t>(E, 1) * sizeof(int));
        nr.sources = nullptr;
        d_images.adopt(nr.images, std::max<std::int64_t>(E, 1) * sizeof(std::uint32_t));
        nr.images = nullptr;
        d_wfrac.adopt(nr.wfrac, std::max(N, 1) * 3 * sizeof(double));
        nr.wfrac = nullptr;
        int* nt = static_cast<int*>(d_neigh_types.ensure(std::max<std::int64_t>(E, 1) * sizeof(int)));
        launch_gather_types(E, d_neigh.as<int>(), d_node_types.as<int>(), nt, stream);
        SMX_HIP(hipStreamSynchronize(stream));
        std::memcpy(cell, cell_, sizeof(cell));
        std::memcpy(inv_cell, inv_, sizeof(inv_cell));
        // fractional reference (prepare_periodic_factorized_graph keeps the
        // builder's wrapped fractional positions, lifecycle.cpp:2231-2244)
        geom = Geometry::device_fractional;
        pbc[0] = pbc[1] = pbc[2] = 1;
        h_offsets.clear();
        const std::uint64_t token = finish_graph(true);
        return {token, E};
    }

    // A prepare that has started to replace the graph voids the previous
    // token first: if it then fails, no call runs on a half-built graph.
    void invalidate_graph() {
        generation = 0;
        evaluated = false;
    }

    void check_generation(std::uint64_t token) const {
        if (token == 0 || token != generation)
            throw std::invalid_argument("execution graph generation is stale or was never prepared");
    }

    // ----------------------------------------------------------------- calls
    const double* tile_xyz(const TileView& t) const {
        return xyz_host ? d_xyz.as<double>() + 3 * t.e0 : d_xyz.as<double>();
    }
    const double* tile_r(const TileView& t) const { return xyz_host ? d_r.as<double>() + t.e0 : d_r.as<double>(); }

    // xyz, r and (with records) per-edge records of one tile
    void tile_geometry(const TileView& t, const double* positions, bool records = true) {
        LaunchTimer* tm = timer.get();
        if (lmp) {
            if (tm) tm->begin("edge_geometry", stream);
            lammps_geometry(t.e0, t.ne, d_receivers.as<int>(), lmp->ilist, l_lmp_j.as<int>(), lmp->x, hm.r_cut,
                            d_xyz.as<double>(), d_r.as<double>(), d_invalid.as<int>(), stream);
            if (tm) tm->end("edge_geometry", stream);
        } else if (fpos_mode) {
            if (tm) tm->begin("edge_geometry", stream);
            lammps_geometry(t.e0, t.ne, d_receivers.as<int>(), d_recv_feature.as<int>(), d_edge_src_feature.as<int>(),
                            d_fpos.as<double>(), hm.r_cut, d_xyz.as<double>(), d_r.as<double>(), d_invalid.as<int>(),
                            stream);
            if (tm) tm->end("edge_geometry", stream);
        } else if (!xyz_host) {
            if (tm) tm->begin("edge_geometry", stream);
            launch_edge_xyz(t.e0, t.ne, edge_reference(), cell, d_receivers.as<int>(), d_neigh.as<int>(),
                            d_disp.as<double>(), hm.r_cut, d_xyz.as<double>(), d_r.as<double>(), d_invalid.as<int>(),
                            stream);
            if (tm) tm->end("edge_geometry", stream);
        }
        if (!records) return;
        if (tm) tm->begin("edge_records", stream);
        const auto [g, lt] = tile_view(t);
        ks->edge_geometry(dm, g, lt, tile_xyz(t), tile_r(t), g.edge_pair ? g.edge_pair + lt.e0 : nullptr,
                          static_cast<int*>(w_exec.ensure(std::max<std::int64_t>(max_tile_ne, 1) * sizeof(int))),
                          ws.erec, ws.erec_b, stream);
        if (tm) tm->end("edge_records", stream);
        (void)positions;
    }

    EdgeReference edge_reference() const {
        EdgeReference ref;
        switch (geom) {
            case Geometry::device_fractional:
                ref.kind = kGeometryDeviceFractional;
                ref.wfrac = d_wfrac.as<double>();
                ref.images = d_images.as<std::uint32_t>();
                break;
            case Geometry::cartesian:
                ref.kind = kGeometryCartesian;
                ref.edges = d_ref_edges.as<double>();
                break;
            case Geometry::fractional:
                ref.kind = kGeometryFractional;
                ref.edges = d_ref_edges.as<double>();
                break;
            case Geometry::shifts:
                ref.kind = kGeometryShifts;
                ref.positions = d_ref_positions.as<double>();
                ref.shifts = d_ref_edges.as<int>();
                break;
            case Geometry::none:
                throw std::logic_error("the prepared graph has no geometry reference");
        }
        return ref;
    }

    // prepare_factorized_geometry / _fractional_geometry / _shift_geometry
    // (lifecycle.cpp:2455-2733): the reference positions and per-edge
    // reference vectors (Cartesian xyz, fractional xyz or integer shifts)
    // that positions calls displace.
    void prepare_geometry(std::uint64_t token, Geometry kind, const double* ref_positions,
                          std::int64_t positions_count, const void* ref_edges, std::int64_t edges_count,
                          const double* cell_, const double* inv_, const int* pbc_) {
        check_generation(token);
        require_idle();
        if (feature_graph())
            throw std::invalid_argument("a graph with ghost feature nodes takes explicit edge vectors (xyz and r)");
        if (kind == Geometry::shifts && !tiled)
            throw std::invalid_argument("Shift geometry requires a fixed-workspace tiled plan.");
        if (!cell_ || !inv_ || !pbc_ || (N > 0 && !ref_positions) || (E > 0 && !ref_edges))
            throw std::invalid_argument("prepared geometry arrays are required");
        if (positions_count != 3 * static_cast<std::int64_t>(N) || edges_count != 3 * E)
            throw std::invalid_argument("prepared geometry extents are inconsistent with the graph");
        if (kind == Geometry::fractional) {
            if (!pbc_[0] || !pbc_[1] || !pbc_[2])
                throw std::invalid_argument("Fractional geometry requires a fully periodic cell.");
            const double det = cell_[0] * (cell_[4] * cell_[8] - cell_[5] * cell_[7]) -
                               cell_[1] * (cell_[3] * cell_[8] - cell_[5] * cell_[6]) +
                               cell_[2] * (cell_[3] * cell_[7] - cell_[4] * cell_[6]);
            if (!std::isfinite(det) || det == 0.0)
                throw std::invalid_argument("Fractional geometry cell matrix must be invertible.");
        }
        auto finite = [](const double* p, std::int64_t n) {
            for (std::int64_t i = 0; i < n; ++i)
                if (!std::isfinite(p[i])) return false;
            return true;
        };
        if (!finite(ref_positions, positions_count) || !finite(cell_, 9) || !finite(inv_, 9) ||
            (kind != Geometry::shifts && !finite(static_cast<const double*>(ref_edges), edges_count)))
            throw std::invalid_argument("prepared geometry contains a non-finite value");
        double* rp = static_cast<double*>(d_ref_positions.ensure(std::max(N, 1) * 3 * sizeof(double)));
        if (N > 0)
            SMX_HIP(hipMemcpyAsync(rp, ref_positions, N * 3 * sizeof(double), hipMemcpyHostToDevice, stream));
        const std::size_t elem = kind == Geometry::shifts ? sizeof(int) : sizeof(double);
        void* re = d_ref_edges.ensure(std::max<std::int64_t>(E, 1) * 3 * elem);
        if (E > 0) SMX_HIP(hipMemcpyAsync(re, ref_edges, E * 3 * elem, hipMemcpyHostToDevice, stream));
        SMX_HIP(hipStreamSynchronize(stream));
        std::memcpy(cell, cell_, sizeof(cell));
        std::memcpy(inv_cell, inv_, sizeof(inv_cell));
        for (int k = 0; k < 3; ++k) pbc[k] = pbc_[k] != 0;
        geom = kind;
        ++geometry_prepare_count;
    }

    // queue the D2H copy of the invalid-edge count (positions and LAMMPS
    // calls).  The direct plan copies on a side stream, so the model kernels
    // follow the edge geometry on the main stream without the copy between
    // them; the tiled plan's later sweeps count again into the same flag, so
    // it copies in order on the main stream.
    void post_geometry_flag() {
        if (xyz_host) return;
        hipStream_t s = stream;
        if (!tiled) {
            SMX_HIP(hipEventRecord(geometry_ready, stream));
            SMX_HIP(hipStreamWaitEvent(flag_stream, geometry_ready, 0));
            s = flag_stream;
        }
        SMX_HIP(hipMemcpyAsync(h_invalid, d_invalid.as<int>(), sizeof(int), hipMemcpyDeviceToHost, s));
        SMX_HIP(hipEventRecord(geometry_done, s));
        geometry_flag_pending = true;
    }

    void zero_a1_if_needed() {
        if (two_layer() && std::find(hm.num_e.begin(), hm.num_e.end(), 0) != hm.num_e.end())
            launch_fill_zero(ws.A1, static_cast<std::size_t>(std::max(max_tile_nr, 1)) * hm.num_lm * hm.C, stream);
    }

    // the electric field of the next evaluations (mace.cpp:1147-1160): 3
    // values (one field for the graph) or 3 per node; an empty field clears it
    void set_field(const double* field, std::int64_t count) {
        if (count < 0 || (count > 0 && !field)) throw std::invalid_argument("electric_field is required");
        if (count > 0 && !hm.field)
            throw std::invalid_argument("the model has no field coupling; it takes no electric_field");
        for (std::int64_t i = 0; i < count; ++i)
            if (!std::isfinite(field[i])) throw std::invalid_argument("electric_field must be finite");
        if (count > 0 && count != 3 && count % 3 != 0)
            throw std::invalid_argument("MACEField electric_field must have shape (3,) or (num_nodes, 3).");
        h_efield.assign(field, field + count);
    }

    // the field's device pointers for this evaluation (mace.cpp:1151-1154)
    void bind_field() {
        field_evaluated = false;
        if (!hm.field) return;
        // one field per graph, or one per feature node (every node of a
        // graph without ghosts), in the caller's node order
        if (h_efield.size() != 3 && h_efield.size() != 3 * static_cast<std::size_t>(F))
            throw std::invalid_argument(h_efield.empty()
                                            ? "a MACEField model is evaluated with an electric field (shape (3,) or "
                                              "(num_nodes, 3))"
                                            : "MACEField electric_field must have shape (3,) or (num_nodes, 3).");
        ws.efield_per_node = h_efield.size() != 3;
        if (ws.efield_per_node && !h_feature_of.empty()) {
            // per-node values in the evaluator's node order
            std::vector<double> mine(h_efield.size());
            for (int k = 0; k < F; ++k)
                for (int c = 0; c < 3; ++c) mine[3 * k + c] = h_efield[3 * static_cast<std::size_t>(h_feature_of[k]) + c];
            upload(d_efield, mine, stream);
        } else if (!h_efield.empty()) {
            upload(d_efield, h_efield, stream);
        }
        ws.efield = d_efield.as<double>();
        ws.field_adj = ws.efield_per_node ? ws.field_part : d_field_adj.as<double>();
        if (N == 0) launch_fill_zero(ws.field_adj, 3, stream);
        // ghosts' rows of a one-call evaluation take no field term
        if (ws.efield_per_node && F > N) launch_fill_zero(ws.field_part, static_cast<std::size_t>(F) * 3, stream);
        field_adj_count = static_cast<std::int64_t>(h_efield.size());
        evaluated_field = h_efield;
        field_evaluated = true;
    }

    void ensure_response() {
        const std::size_t C = hm.C, NY = hm.num_lm, NH = hm.num_LM, NLME = hm.num_lme;
        const std::size_t n = std::max(N, 1), e = std::max<std::int64_t>(E, 1);
        const std::size_t zr = std::max(dm.field_zr, 1), yr = std::max(dm.field_yr, 1);
        // each array starts on a 256-byte boundary
        auto round = [](std::size_t v) { return (v + 63) / 64 * 64; };
        const std::size_t sizes[] = {n * zr * C,   n * NH * C, n * yr * C,   n * NH * C,   n * C,      n * NH * C,
                                     n * NLME * C, n * NY * C, n * C,        n * NY * C,   n * NY * C, n * NY * C,
                                     n * NY * C,   n * C,      n * NLME * C, n * NH * C,   n * NH * C, n * yr * C,
                                     n * NH * C,   n * NY * C, n * NY * C};
        float** slots[] = {&rws.Z,          &rws.H1f_adj,    &rws.Y,         &rws.H1f_dot,   &rws.x_dot,
                           &rws.H1_dot,     &rws.Phi1_dot,   &rws.A1_dot,    &rws.M1_dot,    &rws.g,
                           &rws.gd,         &rws.A1_adj_dot, &rws.A1s_adj,   &rws.direct_dot, &rws.dPhi1_dot,
                           &rws.H1_adj_dot, &rws.H1p_adj_dot, &rws.Y_dot,     &rws.M0_adj_dot, &rws.A0_adj_dot,
                           &rws.Phi0_adj_dot};
        static_assert(sizeof(sizes) / sizeof(sizes[0]) == sizeof(slots) / sizeof(slots[0]), "one size per array");
        std::size_t total = 0;
        for (std::size_t v : sizes) total += round(v);
        float* base = static_cast<float*>(r_f32.ensure(total * sizeof(float)));
        for (std::size_t a = 0; a < sizeof(sizes) / sizeof(sizes[0]); ++a) {
            *slots[a] = base;
            base += round(sizes[a]);
        }
        const std::size_t dsizes[] = {n, n, 3 * n, 3 * n, 9, 9, 9 * e, 9 * n};
        std::size_t dtotal = 0;
        for (std::size_t v : dsizes) dtotal += (v + 31) / 32 * 32;
        double* d = static_cast<double*>(r_f64.ensure(dtotal * sizeof(double)));
        double* at[8];
        for (int a = 0; a < 8; ++a) {
            at[a] = d;
            d += (dsizes[a] + 31) / 32 * 32;
        }
        rws.dot_a = at[0];
        rws.dot_b = at[1];
        rws.part = at[2];
        rws.part_scratch = at[3];
        rws.unit = at[4];
        rws.hessian_t = at[5];
        rws.forces = at[6];
        response_bins_dev = at[7];
        const double unit[9] = {1, 0, 0, 0, 1, 0, 0, 0, 1};
        SMX_HIP(hipMemcpyAsync(at[4], unit, sizeof(unit), hipMemcpyHostToDevice, stream));
    }
    double* response_bins_dev = nullptr;

    // the tangents of the last evaluation in each field component
    // (mace_kokkos_response.tpp:136-2343): the field Hessian, and with
    // forces the directed forces' field derivative (per edge, or reduced to
    // the atoms as Born charge bins)
    void field_response(std::uint64_t token, const double* field, std::int64_t count, bool forces, bool bins) {
        check_generation(token);
        if (!hm.field) throw std::invalid_argument("the MACEField response requires field coupling");
        if (count != 3 || !field)
            throw std::invalid_argument("the MACEField response requires a graph-level electric field (3 values)");
        if (!two_layer()) throw std::invalid_argument("the MACEField response runs two-interaction models");
        if (phase != Phase::idle || feature_graph())
            throw std::invalid_argument("the MACEField response runs on a graph without ghost feature nodes");
        if (!evaluated || !field_evaluated || tiled)
            throw std::logic_error(
                "the MACEField response requires a completed field evaluation of the current graph token");
        if (evaluated_field.size() != 3)
            throw std::invalid_argument("the MACEField response requires an evaluation in a graph-level field");
        for (int c = 0; c < 3; ++c)
            if (field[c] != evaluated_field[c])
                throw std::invalid_argument(
                    "the response's electric field differs from the field of the completed evaluation");
        ensure_response();
        const DeviceGraph g = view();
        const TileView& t = tiles[0];
        LaunchTimer* tm = timer.get();
        launch_fill_zero(rws.hessian_t, 9, stream);
        // A1 rows of an l without paths are not written by its GEMM
        if (std::find(hm.num_e.begin(), hm.num_e.end(), 0) != hm.num_e.end())
            launch_fill_zero(rws.A1_dot, static_cast<std::size_t>(N) * hm.num_lm * hm.C, stream);
        ks->field_response_prepare(dm, t, ws, rws, stream, tm);
        for (int seed = 0; seed < 3; ++seed) ks->field_response_seed(dm, g, t, ws, rws, seed, forces, stream, tm);
        if (forces && bins)
            for (int seed = 0; seed < 3; ++seed)
                launch_atom_forces(N, F, d_offsets.as<int>(), d_soff.as<int>(), d_sedges.as<int>(), nullptr,
                                   rws.forces + static_cast<std::size_t>(seed) * 3 * E,
                                   response_bins_dev + static_cast<std::size_t>(seed) * 3 * N, stream);
        double ht[9];
        SMX_HIP(hipMemcpyAsync(ht, rws.hessian_t, sizeof(ht), hipMemcpyDeviceToHost, stream));
        sync();
        for (int c = 0; c < 3; ++c)
            for (int s = 0; s < 3; ++s) response_hessian[c * 3 + s] = ht[s * 3 + c];
        response_done = true;
        response_has_forces = forces && !bins;
        response_has_bins = forces && bins;
        response_N = N;
        response_E = E;
    }

    void evaluate(const double* positions) {
        const DeviceGraph g = view();
        ws.field_product_only = ws.field_reverse_done = false;
        bind_field();
        for (auto& t : tiles) {
            t.r = tile_r(t);
            t.xyz = tile_xyz(t);
        }
        LaunchTimer* tm = timer.get();
        zero_a1_if_needed();
        if (!tiled) {
            const TileView& t = tiles[0];
            tile_geometry(t, positions);
            post_geometry_flag();
            ks->layer1_forward(dm, g, t, ws, true, stream, tm);
            if (two_layer()) {
                ks->layer2(dm, g, t, ws, stream, tm);
                ks->source_adjoint_all(g, ws, tile_r(t), hm.r_cut, stream, tm);
            } else {
                ks->single_readout(dm, g, t, ws, stream, tm);
            }
            ks->layer1_reverse(dm, g, t, ws, true, stream, tm);
            evaluated = true;
            return;
        }
        if (!two_layer()) {
            // one sweep: each tile's receivers need only their own H1 rows
            // (mace_kokkos_evaluate.cpp:614-752)
            launch_fill_zero(d_atom_forces.as<double>(), static_cast<std::size_t>(F) * 3, stream);
            launch_fill_zero(d_virial.as<double>(), 9, stream);
            // the invalid-edge count of every tile's edges first
            for (const auto& t : tiles) tile_geometry(t, positions, false);
            post_geometry_flag();
            // LAMMPS rows receive tile forces from the first tile on: raise first
            if (lmp) raise_if_invalid_geometry("LAMMPS positions");
            for (const auto& t : tiles) {
                tile_geometry(t, positions);
                const auto [gt, lt] = tile_view(t);
                ks->layer1_forward(dm, gt, lt, ws, true, stream, tm);
                ks->single_readout(dm, gt, lt, ws, stream, tm);
                ks->layer1_reverse(dm, gt, lt, ws, true, stream, tm);
                accumulate_tile_outputs(t);
            }
            forces_to_caller_order();
            evaluated = true;
            return;
        }
        // three sweeps over receiver tiles (graph-wide H1, H1 adjoint between them)
        tiled_sweep_h1(positions);
        post_geometry_flag();
        // LAMMPS rows receive tile forces from the next sweep on: raise first
        if (lmp) raise_if_invalid_geometry("LAMMPS positions");
        tiled_sweep_layer2(positions);
        tiled_sweep_reverse(positions);
        evaluated = true;
    }

    // the tiled plan's sweeps: layer 1 to H1; layer 2 with the source
    // adjoint accumulated over the tiles; the layer-1 reverse (forces and
    // virial accumulated as each tile finishes)
    void tiled_sweep_h1(const double* positions) {
        for (const auto& t : tiles) {
            tile_geometry(t, positions);
            const auto [g, lt] = tile_view(t);
            ks->layer1_forward(dm, g, lt, ws, true, stream, timer.get());
        }
    }

    void tiled_sweep_layer2(const double* positions) {
        launch_fill_zero(ws.H1_adj, static_cast<std::size_t>(F) * hm.num_LM * hm.C, stream);
        launch_fill_zero(d_atom_forces.as<double>(), static_cast<std::size_t>(F) * 3, stream);
        launch_fill_zero(d_virial.as<double>(), 9, stream);
        for (const auto& t : tiles) {
            tile_geometry(t, positions);
            const auto [g, lt] = tile_view(t);
            ks->layer2(dm, g, lt, ws, stream, timer.get());
            ks->source_adjoint_tile(g, lt, ws, tile_r(t), hm.r_cut, stream, timer.get());
            accumulate_tile_outputs(t);
        }
    }

    void tiled_sweep_reverse(const double* positions) {
        for (const auto& t : tiles) {
            tile_geometry(t, positions);
            const auto [g, lt] = tile_view(t);
            ks->layer1_forward(dm, g, lt, ws, false, stream, timer.get());
            ks->layer1_reverse(dm, g, lt, ws, false, stream, timer.get());
            accumulate_tile_outputs(t);
        }
        forces_to_caller_order();
    }

    // tiles accumulate the feature nodes' forces in the evaluator's order;
    // a feature graph's caller reads them in its own
    void forces_to_caller_order() {
        if (h_feature_of.empty() || F == 0) return;
        double* tmp = static_cast<double*>(d_forces_caller.ensure(static_cast<std::size_t>(F) * 3 * sizeof(double)));
        launch_scatter_rows(F, 3, d_feature_of.as<int>(), d_atom_forces.as<double>(), tmp, stream);
        SMX_HIP(hipMemcpyAsync(d_atom_forces.as<double>(), tmp, static_cast<std::size_t>(F) * 3 * sizeof(double),
                               hipMemcpyDeviceToDevice, stream));
    }

    void accumulate_tile_outputs(const TileView& t) {
        LaunchTimer* tm = timer.get();
        if (tm) tm->begin("tile_reductions", stream);
        if (lmp) {
            // LAMMPS rows: sources by LAMMPS index (ghosts included), receivers through ilist
            const std::size_t ti = static_cast<std::size_t>(&t - tiles.data());
            launch_tile_forces(t, l_touched.as<int>() + l_touched_begin[ti],
                               static_cast<int>(l_touched_begin[ti + 1] - l_touched_begin[ti]), d_offsets.as<int>(),
                               t.e0, l_joff.as<int>(), l_jedges.as<int>(), lmp->ilist, ws.node_forces, lmp->f, stream);
        } else {
            const auto [g, lt] = tile_view(t);
            launch_tile_forces(t, t.touched, t.touched_count, g.offsets, lt.e0, d_soff64.as<long long>(),
                               d_sedges64.as<long long>(), nullptr, ws.node_forces, d_atom_forces.as<double>(),
                               stream);
        }
        launch_virial_accumulate(t.ne, ws.node_forces, tile_xyz(t), d_stress_partial.as<double>(), stress_blocks,
                                 d_virial.as<double>(), stream);
        if (tm) tm->end("tile_reductions", stream);
    }

    // wait for the invalid-edge count queued after the first geometry pass
    // (the model kernels behind it keep running) and raise if it is not zero
    void raise_if_invalid_geometry(const char* what) {
        if (!geometry_flag_pending) return;
        geometry_flag_pending = false;
        SMX_HIP(hipEventSynchronize(geometry_done));
        const int invalid = *h_invalid;
        if (invalid > 0) {
            evaluated = false;
            throw std::invalid_argument(std::string(what) + " produced an invalid edge geometry (" +
                                        std::to_string(invalid) + " zero-length or non-finite edges)");
        }
    }

    // drain the stream; launch timings recorded so far become readable
    void sync() {
        SMX_HIP(hipStreamSynchronize(stream));
        if (timer) timer->collect();
    }

    // wait: synchronise the stream before returning (host inputs); else the
    // call returns once the geometry check is readable and the model kernels
    // stay queued on the evaluator stream (device outputs are stream-ordered)
    void finish_call(bool wait) {
        int invalid = 0;
        if (geometry_flag_pending) {
            geometry_flag_pending = false;
            SMX_HIP(hipEventSynchronize(geometry_done));
            invalid = *h_invalid;
        }
        if (wait) sync();
        if (invalid > 0) {
            evaluated = false;
            throw std::invalid_argument("positions produced an invalid edge geometry (" + std::to_string(invalid) +
                                        " zero-length or non-finite edges)");
        }
    }

    // a plain call over a graph with ghost feature nodes: one interaction only
    // (two need the ghosts' H1 from their owners, the split-phase calls)
    void require_plain_call() const {
        if (phase != Phase::idle)
            throw std::logic_error("a factorized distributed evaluation is active: finish it first");
        if (two_layer() && feature_graph())
            throw std::invalid_argument(
                "a two-interaction model on a graph with ghost feature nodes is evaluated in the split phases "
                "(begin, continue and finish_factorized_distributed_evaluation)");
    }

    void compute_positions(std::uint64_t token, const double* positions, bool on_device) {
        check_generation(token);
        require_plain_call();
        fpos_mode = false;
        if (geom == Geometry::none)
            throw std::invalid_argument("Execution R1 positions require current graph and geometry tokens: "
                                        "prepare a geometry (prepare_factorized_geometry or its fractional or "
                                        "shift form) or use compute_prepared_factorized with xyz and r");
        const double* pos = positions;
        if (!on_device) {
            for (int i = 0; i < 3 * N; ++i)
                if (!std::isfinite(positions[i])) throw std::invalid_argument("positions must be finite");
            double* dp = d_positions.as<double>();
            if (N > 0) SMX_HIP(hipMemcpyAsync(dp, positions, N * 3 * sizeof(double), hipMemcpyHostToDevice, stream));
            pos = dp;
        }
        xyz_host = false;
        if (timer) timer->begin("displacements", stream);
        const bool frac_ref = geom == Geometry::device_fractional || geom == Geometry::fractional;
        // (also clears the invalid-edge count)
        launch_displacements(N, cell, inv_cell, pbc, frac_ref,
                             geom == Geometry::device_fractional ? d_wfrac.as<double>() : d_ref_positions.as<double>(),
                             pos, d_disp.as<double>(), d_invalid.as<int>(), stream);
        if (timer) timer->end("displacements", stream);
        evaluate(pos);
        finish_call(!on_device);
    }

    // The calculator's call in one (calculator.py:3821-3894 makes these in
    // turn): host positions through pinned memory, the evaluation, the atom
    // forces and (stress non-null) the stress, and every result copied back
    // through pinned memory behind one wait for the device
    void compute_results(std::uint64_t token, const double* positions, double volume, double* energies,
                         double* forces, double* stress) {
        check_generation(token);
        require_plain_call();
        if (geom == Geometry::none)
            throw std::invalid_argument("Execution R1 positions require current graph and geometry tokens: "
                                        "prepare a geometry (prepare_factorized_geometry or its fractional or "
                                        "shift form) or use compute_prepared_factorized with xyz and r");
        if (N > 0 && (!positions || !energies || !forces)) throw std::invalid_argument("a result buffer is NULL");
        if (stress && (!(volume > 0.0) || !std::isfinite(volume))) throw std::invalid_argument("volume must be positive");
        for (int i = 0; i < 3 * N; ++i)
            if (!std::isfinite(positions[i])) throw std::invalid_argument("positions must be finite");
        const std::size_t n = N, f = F;
        double* st = host_stage(3 * n + n + 3 * f + 9);
        double* d_pos = d_positions.as<double>();
        if (N > 0) {
            std::memcpy(st, positions, 3 * n * sizeof(double));
            SMX_HIP(hipMemcpyAsync(d_pos, st, 3 * n * sizeof(double), hipMemcpyHostToDevice, stream));
        }
        fpos_mode = false;
        xyz_host = false;
        if (timer) timer->begin("displacements", stream);
        const bool frac_ref = geom == Geometry::device_fractional || geom == Geometry::fractional;
        launch_displacements(N, cell, inv_cell, pbc, frac_ref,
                             geom == Geometry::device_fractional ? d_wfrac.as<double>() : d_ref_positions.as<double>(),
                             d_pos, d_disp.as<double>(), d_invalid.as<int>(), stream);
        if (timer) timer->end("displacements", stream);
        evaluate(d_pos);
        if (!tiled)
            launch_atom_forces(N, F, d_offsets.as<int>(), d_soff.as<int>(), d_sedges.as<int>(),
                               h_feature_of.empty() ? nullptr : d_feature_of.as<int>(), ws.node_forces,
                               d_atom_forces.as<double>(), stream);
        if (stress) {
            if (!tiled)
                launch_stress(E, ws.node_forces, d_xyz.as<double>(), volume, d_stress_partial.as<double>(),
                              stress_blocks, d_stress.as<double>(), stream);
            else
                launch_scale9(d_virial.as<double>(), -1.0 / volume, d_stress.as<double>(), stream);
        }
        double* se = st + 3 * n;
        double* sf = se + n;
        double* ss = sf + 3 * f;
        if (N > 0) SMX_HIP(hipMemcpyAsync(se, ws.node_energies, n * sizeof(double), hipMemcpyDeviceToHost, stream));
        if (F > 0)
            SMX_HIP(hipMemcpyAsync(sf, d_atom_forces.as<double>(), 3 * f * sizeof(double), hipMemcpyDeviceToHost, stream));
        if (stress) SMX_HIP(hipMemcpyAsync(ss, d_stress.as<double>(), 9 * sizeof(double), hipMemcpyDeviceToHost, stream));
        finish_call(true);
        std::memcpy(energies, se, n * sizeof(double));
        std::memcpy(forces, sf, 3 * f * sizeof(double));
        if (stress) std::memcpy(stress, ss, 9 * sizeof(double));
    }

    void compute_xyz(std::uint64_t token, const double* xyz, const double* r) {
        check_generation(token);
        require_plain_call();
        fpos_mode = false;
        for (std::int64_t e = 0; e < E; ++e) {
            if (!std::isfinite(r[e]) || !(r[e] > 0.0) || !std::isfinite(xyz[3 * e]) || !std::isfinite(xyz[3 * e + 1]) ||
                !std::isfinite(xyz[3 * e + 2]))
                throw std::invalid_argument("MACE graph has an invalid distance or displacement vector");
        }
        // explicit edge vectors of the whole graph
        d_xyz.ensure(std::max<std::int64_t>(E, 1) * 3 * sizeof(double));
        d_r.ensure(std::max<std::int64_t>(E, 1) * sizeof(double));
        xyz_host = true;
        if (E > 0) {
            SMX_HIP(hipMemcpyAsync(d_xyz.as<double>(), xyz, E * 3 * sizeof(double), hipMemcpyHostToDevice, stream));
            SMX_HIP(hipMemcpyAsync(d_r.as<double>(), r, E * sizeof(double), hipMemcpyHostToDevice, stream));
        }
        evaluate(nullptr);
        finish_call(true);
    }

    void update_cell(std::uint64_t token, const double* cell_, const double* inv_) {
        check_generation(token);
        if (geom != Geometry::device_fractional && geom != Geometry::fractional && geom != Geometry::shifts)
            throw std::invalid_argument("Prepared Execution R1 cell update requires current graph and fractional or "
                                        "shift geometry tokens.");
        for (int k = 0; k < 9; ++k)
            if (!std::isfinite(cell_[k]) || !std::isfinite(inv_[k]))
                throw std::invalid_argument("cell matrices contain a non-finite value");
        const double det = cell_[0] * (cell_[4] * cell_[8] - cell_[5] * cell_[7]) -
                           cell_[1] * (cell_[3] * cell_[8] - cell_[5] * cell_[6]) +
                           cell_[2] * (cell_[3] * cell_[7] - cell_[4] * cell_[6]);
        if (!std::isfinite(det) || det == 0.0) throw std::invalid_argument("the cell matrix must be invertible");
        std::memcpy(cell, cell_, sizeof(cell));
        std::memcpy(inv_cell, inv_, sizeof(inv_cell));
    }

    DeviceGraph view() const {
        DeviceGraph g;
        g.N = N;
        g.F = F;
        g.E = E;
        g.node_types = d_node_types.as<int>();
        g.offsets = d_offsets.as<int>();
        g.neigh = d_neigh.as<int>();
        g.neigh_types = d_neigh_types.as<int>();
        g.receivers = d_receivers.as<int>();
        g.soff = d_soff.as<int>();
        g.sedges = d_sedges.as<int>();
        g.soff64 = d_soff64.as<long long>();
        g.sedges64 = d_sedges64.as<long long>();
        g.edge_pair = hm.agnesi ? d_edge_pair.as<int>() : nullptr;
        return g;
    }

    // The kernels' view of one tile.  Direct plan: the graph and the tile as
    // they are.  Tiled plan: the per-edge arrays start at the tile's first
    // edge, the offsets are the tile's relative ones and the tile's e0 is 0,
    // so the kernels' edge indices stay 32-bit at any graph size.
    std::pair<DeviceGraph, TileView> tile_view(const TileView& t) const {
        DeviceGraph g = view();
        TileView lt = t;
        if (!tiled) return {g, lt};
        const std::ptrdiff_t ti = &t - tiles.data();
        if (ti < 0 || ti >= static_cast<std::ptrdiff_t>(tiles.size()))
            throw std::logic_error("tile_view takes one of the graph's own tiles");
        g.offsets = d_tile_off.as<int>() + ti;
        g.neigh += t.e0;
        g.neigh_types += t.e0;
        g.receivers += t.e0;
        if (g.edge_pair) g.edge_pair += t.e0;
        g.E = t.ne;
        g.edge_base = t.e0;
        lt.e0 = 0;
        return {g, lt};
    }

    void require_evaluated(std::uint64_t token) const {
        check_generation(token);
        if (!evaluated) throw std::logic_error("no evaluation has run on the prepared graph");
    }

    void reduce_forces(std::uint64_t token, double* out) {
        require_evaluated(token);
        if (!tiled)
            launch_atom_forces(N, F, d_offsets.as<int>(), d_soff.as<int>(), d_sedges.as<int>(),
                               h_feature_of.empty() ? nullptr : d_feature_of.as<int>(), ws.node_forces,
                               d_atom_forces.as<double>(), stream);
        if (out) {
            if (F > 0)
                SMX_HIP(hipMemcpyAsync(out, d_atom_forces.as<double>(), F * 3 * sizeof(double), hipMemcpyDeviceToHost,
                                       stream));
            SMX_HIP(hipStreamSynchronize(stream));
        }
    }

    void reduce_stress(std::uint64_t token, double volume, double* out) {
        require_evaluated(token);
        if (!(volume > 0.0) || !std::isfinite(volume)) throw std::invalid_argument("volume must be positive");
        if (!tiled)
            launch_stress(E, ws.node_forces, d_xyz.as<double>(), volume, d_stress_partial.as<double>(), stress_blocks,
                          d_stress.as<double>(), stream);
        else
            launch_scale9(d_virial.as<double>(), -1.0 / volume, d_stress.as<double>(), stream);
        if (out) {
            SMX_HIP(hipMemcpyAsync(out, d_stress.as<double>(), 9 * sizeof(double), hipMemcpyDeviceToHost, stream));
            SMX_HIP(hipStreamSynchronize(stream));
        }
    }

    void total_energy(double* out) {
        if (!evaluated) throw std::logic_error("no evaluation has run");
        launch_energy_sum(N, ws.node_energies, d_total.as<double>(), stream);
        if (out) {
            SMX_HIP(hipMemcpyAsync(out, d_total.as<double>(), sizeof(double), hipMemcpyDeviceToHost, stream));
            SMX_HIP(hipStreamSynchronize(stream));
        }
    }

    // ---------------------------------------------------------- LAMMPS entry
    // pair_symmetrix_mace_kokkos.cpp:1010-1282: topology on a rebuild,
    // edge vectors every call, reductions into LAMMPS's per-atom arrays
    DevBuf l_node_types, l_num_neigh, l_node_of_atom, l_neigh, l_neigh_types, l_lmp_j, l_joff, l_jedges, l_counts, l_offsets,
        l_flag, l_touched;
    std::vector<std::size_t> l_touched_begin;  // tiled plan: LAMMPS atoms each tile's edges leave
    const SmxLammpsArgsV1* lmp = nullptr;      // set while a LAMMPS call evaluates
    int l_inum = -1, l_nall = -1;
    std::uint64_t l_generation = 0;
    std::vector<int> l_ilist_host;

    int read_flag(DevBuf& b) {
        int v = 0;
        SMX_HIP(hipMemcpyAsync(&v, b.as<int>(), sizeof(int), hipMemcpyDeviceToHost, stream));
        SMX_HIP(hipStreamSynchronize(stream));
        return v;
    }

    void lammps_topology(const SmxLammpsArgsV1& a, const LammpsList& L) {
        // the LAMMPS arrays below are rewritten first: a failure on the way
        // leaves no topology that a later call could take as current
        l_generation = 0;
        const int inum = a.inum, nall = a.nall;
        int* nt = static_cast<int*>(l_node_types.ensure(std::max(inum, 1) * sizeof(int)));
        int* nn = static_cast<int*>(l_num_neigh.ensure(std::max(inum, 1) * sizeof(int)));
        int* noa = static_cast<int*>(l_node_of_atom.ensure(std::max(nall, 1) * sizeof(int)));
        int* flag = static_cast<int*>(l_flag.ensure(sizeof(int)));
        launch_fill_zero(reinterpret_cast<float*>(flag), 1, stream);
        lammps_nodes(inum, nall, L, nt, nn, noa, flag, stream);
        if (read_flag(l_flag) != 0)
            throw std::invalid_argument("LAMMPS ilist holds an atom outside [0, nall), a negative neighbour count "
                                        "or a type without a model type");
        std::vector<int> h_nn(inum), off(inum + 1, 0);
        if (inum > 0) SMX_HIP(hipMemcpy(h_nn.data(), nn, sizeof(int) * inum, hipMemcpyDeviceToHost));
        std::int64_t total = 0;
        for (int ii = 0; ii < inum; ++ii) {
            total += h_nn[ii];
            if (total > kMaxEdges) throw std::invalid_argument("edge count exceeds the 32-bit graph limit");
            off[ii + 1] = static_cast<int>(total);
        }
        int* d_off = upload(l_offsets, off, stream);
        const std::size_t e = static_cast<std::size_t>(std::max<std::int64_t>(total, 1));
        int* nb = static_cast<int*>(l_neigh.ensure(e * sizeof(int)));
        int* nbt = static_cast<int*>(l_neigh_types.ensure(e * sizeof(int)));
        int* lj = static_cast<int*>(l_lmp_j.ensure(e * sizeof(int)));
        launch_fill_zero(reinterpret_cast<float*>(flag), 1, stream);
        lammps_edges(inum, nall, L, d_off, noa, nb, nbt, lj, flag, stream);
        if (read_flag(l_flag) != 0)
            throw std::invalid_argument("LAMMPS neighbour outside [0, nall), with an owner that is not a local "
                                        "ilist atom, or with an unmapped type");
        // the kernels above checked every index and type of the CSR
        prepare_graph_checked(inum, nt, off, total, nb, nbt);
        int* joff = static_cast<int*>(l_joff.ensure((static_cast<std::size_t>(nall) + 1) * sizeof(int)));
        int* jed = static_cast<int*>(l_jedges.ensure(e * sizeof(int)));
        int* cnt = static_cast<int*>(l_counts.ensure(std::max(nall, 1) * sizeof(int)));
        launch_transpose(nall, total, lj, joff, jed, cnt, stream);
        l_touched_begin.assign(1, 0);
        if (tiled && nall > 0) {
            DevBuf bitmap, counts, one;
            const int words = nall / 32 + 1;
            bitmap.ensure(sizeof(std::uint32_t) * words);
            counts.ensure(sizeof(int) * words);
            one.ensure(sizeof(int) * nall);
            std::vector<int> all, host(nall);
            for (const auto& t : tiles) {
                const int c = build_touched_sources(nall, t.e0, t.ne, lj, bitmap.as<std::uint32_t>(), counts.as<int>(),
                                                    one.as<int>(), stream);
                if (c > 0) SMX_HIP(hipMemcpy(host.data(), one.as<int>(), sizeof(int) * c, hipMemcpyDeviceToHost));
                all.insert(all.end(), host.begin(), host.begin() + c);
                l_touched_begin.push_back(all.size());
            }
            upload(l_touched, all, stream);
        }
        l_inum = inum;
        l_nall = nall;
        l_generation = generation;
    }

    void lammps_compute(const SmxLammpsArgsV1& a, double* energy, double* virial6) {
        require_idle();
        fpos_mode = false;
        if (a.struct_size < sizeof(SmxLammpsArgsV1)) throw std::invalid_argument("SmxLammpsArgsV1.struct_size is too small");
        if (a.inum < 0 || a.nall < a.inum || a.ntypes < 1)
            throw std::invalid_argument("LAMMPS counts are invalid (0 <= inum <= nall, ntypes >= 1)");
        if (a.inum > 0 && (!a.ilist || !a.numneigh || !a.neighbors))
            throw std::invalid_argument("LAMMPS neighbour list arrays are required");
        if (a.nall > 0 && (!a.x || !a.type || !a.owner || !a.f))
            throw std::invalid_argument("LAMMPS per-atom arrays (x, type, owner, f) are required");
        if (!a.type_to_model) throw std::invalid_argument("the LAMMPS type map is required");
        if (a.stride_atom < 0 || a.stride_neighbor < 0) throw std::invalid_argument("neighbour strides must be >= 0");
        const LammpsList L{a.ilist, a.numneigh, a.neighbors, a.stride_atom, a.stride_neighbor, a.type,
                           a.type_to_model, a.ntypes, a.owner};
        // order after the caller's device work on x and f
        if (a.struct_size >= sizeof(SmxLammpsArgsV2)) {
            const auto* v2 = reinterpret_cast<const SmxLammpsArgsV2*>(&a);
            SMX_HIP(hipEventRecord(caller_ready, static_cast<hipStream_t>(v2->stream)));
            SMX_HIP(hipStreamWaitEvent(stream, caller_ready, 0));
        } else {
            SMX_HIP(hipDeviceSynchronize());
        }
        if (a.rebuild || l_generation == 0 || l_generation != generation || a.inum != l_inum || a.nall != l_nall)
            lammps_topology(a, L);
        // edge vectors are made per tile from a.x (tile_geometry); forces of
        // the tiled plan go into a.f tile by tile, the direct plan's after
        // the call from its retained per-edge forces
        launch_fill_zero(reinterpret_cast<float*>(d_invalid.as<int>()), 1, stream);
        xyz_host = false;
        struct Reset {
            const SmxLammpsArgsV1*& p;
            ~Reset() { p = nullptr; }
        } reset{lmp};
        lmp = &a;
        evaluate(nullptr);
        lmp = nullptr;
        // an invalid geometry raises before anything is added to f or eatom
        raise_if_invalid_geometry("LAMMPS positions");
        if (!tiled) {
            lammps_forces(a.nall, l_joff.as<int>(), l_jedges.as<int>(), l_node_of_atom.as<int>(), d_offsets.as<int>(),
                          ws.node_forces, a.f, stream);
            launch_fill_zero(d_virial.as<double>(), 9, stream);
            launch_virial_accumulate(E, ws.node_forces, d_xyz.as<double>(), d_stress_partial.as<double>(),
                                     stress_blocks, d_virial.as<double>(), stream);
        }
        if (a.eatom) lammps_eatom(a.inum, a.ilist, ws.node_energies, a.eatom, stream);
        launch_energy_sum(N, ws.node_energies, d_total.as<double>(), stream);
        double total = 0.0, w[9];
        SMX_HIP(hipMemcpyAsync(&total, d_total.as<double>(), sizeof(double), hipMemcpyDeviceToHost, stream));
        SMX_HIP(hipMemcpyAsync(w, d_virial.as<double>(), sizeof(w), hipMemcpyDeviceToHost, stream));
        sync();
        // w[a*3+b] = sum_e f_a xyz_b; LAMMPS order xx, yy, zz, xy, xz, yz
        if (energy) *energy = total;
        if (virial6) {
            virial6[0] = w[0];
            virial6[1] = w[4];
            virial6[2] = w[8];
            virial6[3] = 0.5 * (w[1] + w[3]);
            virial6[4] = 0.5 * (w[2] + w[6]);
            virial6[5] = 0.5 * (w[5] + w[7]);
        }
    }

    const double* node_forces_device() const {
        if (tiled) throw std::logic_error("directed edge forces are not retained by the tiled execution plan");
        return ws.node_forces;
    }

    std::string plan_description() const {
        std::string s = tiled ? "direct-tiled" : "direct";
        s += std::string(" polynomials=") + ks->polynomial_mode();
        s += " tiles=" + std::to_string(tiles.size()) + " max_tile_receivers=" + std::to_string(max_tile_nr) +
             " max_tile_edges=" + std::to_string(max_tile_ne);
        return s;
    }

    std::int64_t stage(const std::string& name, float* out, std::int64_t capacity) {
        const std::int64_t n = tiled ? max_tile_nr : N, C = hm.C, NY = hm.num_lm, NH = hm.num_LM,
                           NLME = hm.num_lme;
        const float* src = nullptr;
        std::int64_t count = 0;
        if (name == "A0") src = ws.A0, count = n * NY * C;
        else if (name == "Phi0") src = ws.Phi0, count = n * NY * C;
        else if (name == "M0") src = ws.M0, count = n * NH * C;
        else if (name == "H1") src = ws.H1, count = static_cast<std::int64_t>(N) * NH * C;
        else if (name == "Phi1") src = ws.Phi1, count = n * NLME * C;
        else if (name == "A1") src = ws.A1, count = n * NY * C;
        else if (name == "A1_adj") src = ws.A1_adj, count = n * NY * C;
        else if (name == "dPhi1") src = ws.dPhi1, count = n * NLME * C;
        else if (name == "H1_adj") src = ws.H1_adj, count = static_cast<std::int64_t>(N) * NH * C;
        else if (name == "M0_adj") src = ws.M0_adj, count = n * NH * C;
        else if (name == "A0_adj") src = ws.A0_adj, count = n * NY * C;
        else if (name == "direct") src = ws.direct, count = static_cast<std::int64_t>(N) * C;
        else if (name == "edge_records")  // the forward parts [edge][x, interval, active, 0, Y...]
            src = ws.erec, count = (tiled ? max_tile_ne : E) * ks->record_forward_floats();
        else throw std::invalid_argument("unknown stage '" + name + "'");
        if (count > 0 && !src) throw std::invalid_argument("stage '" + name + "' is not held for this model");
        if (out && capacity >= count && count > 0) {
            SMX_HIP(hipMemcpyAsync(out, src, count * sizeof(float), hipMemcpyDeviceToHost, stream));
            SMX_HIP(hipStreamSynchronize(stream));
        }
        return count;
    }
};

}  // namespace smx

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
struct SmxEvaluator {
    smx::Evaluator impl;
    SmxEvaluator(const std::string& p, const std::string& h) : impl(p, h) {}
};

namespace {

template <class F>
int32_t guarded(F&& f) {
    try {
        f();
        return SMX_OK;
    } catch (const std::bad_alloc&) {
        smx::g_last_error = "out of memory (device or host allocation failed)";
        return SMX_ERR_OUT_OF_MEMORY;
    } catch (const std::domain_error& e) {
        smx::g_last_error = e.what();
        return SMX_ERR_UNSUPPORTED;
    } catch (const std::invalid_argument& e) {
        smx::g_last_error = e.what();
        return SMX_ERR_INVALID_ARGUMENT;
    } catch (const std::length_error& e) {
        smx::g_last_error = e.what();
        return SMX_ERR_INVALID_ARGUMENT;
    } catch (const std::out_of_range& e) {
        smx::g_last_error = e.what();
        return SMX_ERR_INVALID_ARGUMENT;
    } catch (const std::logic_error& e) {
        smx::g_last_error = e.what();
        return SMX_ERR_LOGIC;
    } catch (const std::exception& e) {
        smx::g_last_error = e.what();
        return SMX_ERR_RUNTIME;
    } catch (...) {
        smx::g_last_error = "unknown error";
        return SMX_ERR_RUNTIME;
    }
}

smx::Evaluator& E(SmxEvaluator* ev) {
    if (!ev) throw std::invalid_argument("evaluator handle is NULL");
    return ev->impl;
}

// Host model of the last file the array exports read (a model is parsed once
// for the several arrays a caller asks for).
std::mutex g_export_mutex;
std::string g_export_path;
std::shared_ptr<smx::HostModel> g_export_model;

std::shared_ptr<smx::HostModel> export_model(const char* path) {
    if (!path) throw std::invalid_argument("model path is NULL");
    if (!g_export_model || g_export_path != path) {
        auto m = std::make_shared<smx::HostModel>();
        m->load(path, "");
        g_export_model = std::move(m);
        g_export_path = path;
    }
    return g_export_model;
}

template <class T>
void export_array(const std::vector<T>& v, T* out, int64_t capacity, int64_t* count) {
    if (count) *count = static_cast<int64_t>(v.size());
    if (!out) return;
    if (capacity < static_cast<int64_t>(v.size())) throw std::invalid_argument("output capacity is too small");
    std::copy(v.begin(), v.end(), out);
}
// host wall time of a prepare or evaluation call, kept as the evaluator's
// last_graph_prepare_ms / last_evaluation_ms counters
template <class F>
void timed(double& ms, std::int64_t& count, F&& f) {
    const auto t0 = std::chrono::steady_clock::now();
    f();
    ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    ++count;
}

const smx::Evaluator& E(const SmxEvaluator* ev) {
    if (!ev) throw std::invalid_argument("evaluator handle is NULL");
    return ev->impl;
}

}  // namespace

extern "C" {

int32_t smx_abi_version(void) { return SMX_ABI_VERSION; }

const char* smx_last_error(void) { return smx::g_last_error.c_str(); }

int32_t smx_evaluator_create(const char* model_path, const char* head, SmxEvaluator** out) {
    return guarded([&] {
        if (!model_path || !out) throw std::invalid_argument("model path and output handle are required");
        *out = nullptr;
        *out = new SmxEvaluator(model_path, head ? head : "");
    });
}

void smx_evaluator_destroy(SmxEvaluator* ev) { delete ev; }

int32_t smx_model_convert(const char* source, const char* destination, const char* format) {
    return guarded([&] {
        if (!source || !destination || !format)
            throw std::invalid_argument("source, destination and format are required");
        smx::convert_model_file(source, destination, format);
    });
}

int32_t smx_evaluator_info(const SmxEvaluator* ev, SmxModelInfo* info) {
    return guarded([&] {
        const auto& m = E(ev).hm;
        if (!info || info->struct_size < sizeof(SmxModelInfo))
            throw std::invalid_argument("SmxModelInfo.struct_size is too small");
        info->num_elements = m.num_elements;
        info->num_channels = m.C_file;
        info->l_max = m.l_max;
        info->L_max = m.L_max;
        info->num_interactions = m.num_interactions;
        info->num_paths = m.num_paths;
        info->num_lme = m.num_lme;
        info->r_cut = m.r_cut;
    });
}

int32_t smx_evaluator_atomic_numbers(const SmxEvaluator* ev, int32_t* out, int32_t capacity) {
    return guarded([&] {
        const auto& z = E(ev).hm.atomic_numbers;
        if (!out || capacity < static_cast<int32_t>(z.size())) throw std::invalid_argument("buffer too small");
        std::copy(z.begin(), z.end(), out);
    });
}

int32_t smx_evaluator_atomic_energies(const SmxEvaluator* ev, double* out, int32_t capacity) {
    return guarded([&] {
        const auto& e0 = E(ev).hm.atomic_energies;
        if (!out || capacity < static_cast<int32_t>(e0.size())) throw std::invalid_argument("buffer too small");
        std::copy(e0.begin(), e0.end(), out);
    });
}

int32_t smx_active_atomic_numbers(const SmxEvaluator* ev, int32_t* out, int32_t capacity, int32_t* count) {
    return guarded([&] {
        const auto& e = E(ev);
        // models with per-pair radial tables keep tables for the active
        // types only; the others serve every type
        std::vector<int32_t> z;
        if (e.hm.agnesi)
            for (int t : e.pair_active) z.push_back(e.hm.atomic_numbers[t]);
        else
            z.assign(e.hm.atomic_numbers.begin(), e.hm.atomic_numbers.end());
        if (count) *count = static_cast<int32_t>(z.size());
        if (!out) return;
        if (capacity < static_cast<int32_t>(z.size())) throw std::invalid_argument("buffer too small");
        std::copy(z.begin(), z.end(), out);
    });
}

int32_t smx_prediction_head(const SmxEvaluator* ev, int32_t index, const char** name) {
    return guarded([&] {
        if (!name) throw std::invalid_argument("name output is required");
        const auto& hm = E(ev).hm;
        if (index < 0)
            *name = hm.selected_head.c_str();
        else
            *name = index < static_cast<int32_t>(hm.available_heads.size()) ? hm.available_heads[index].c_str()
                                                                             : nullptr;
    });
}

int32_t smx_set_streamed_edges(SmxEvaluator* ev, const char* mode) {
    return guarded([&] {
        auto& e = E(ev);
        const std::string m = mode ? mode : "";
        if (m != "direct")
            throw std::invalid_argument("streamed_edges mode '" + m + "' is not implemented; only 'direct' is");
        e.streamed_edges = m;
    });
}

void* smx_evaluator_stream(SmxEvaluator* ev) { return ev ? static_cast<void*>(ev->impl.stream) : nullptr; }

int32_t smx_prepare_factorized_graph(SmxEvaluator* ev, int32_t num_nodes, const int32_t* node_types,
                                     const int32_t* num_neigh, int64_t num_edges, const int32_t* neigh_indices,
                                     const int32_t* neigh_types, uint64_t* generation) {
    return guarded([&] {
        if (!generation) throw std::invalid_argument("generation output is required");
        if (num_nodes > 0 && (!node_types || !num_neigh)) throw std::invalid_argument("node arrays are required");
        if (num_edges > 0 && (!neigh_indices || !neigh_types)) throw std::invalid_argument("edge arrays are required");
        auto& e = E(ev);
        timed(e.last_prepare_ms, e.prepare_count, [&] {
            *generation = e.prepare_graph_host(num_nodes, node_types, num_neigh, num_edges, neigh_indices, neigh_types);
        });
    });
}

int32_t smx_prepare_factorized_graph_device(SmxEvaluator* ev, int32_t num_nodes, const int32_t* node_types_device,
                                            const int32_t* num_neigh_device, int64_t num_edges,
                                            const int32_t* neigh_indices_device, const int32_t* neigh_types_device,
                                            uint64_t* generation) {
    return guarded([&] {
        if (!generation) throw std::invalid_argument("generation output is required");
        if (num_edges < 0 || num_edges > INT_MAX) throw std::invalid_argument("edge count exceeds the 32-bit graph limit");
        auto& e = E(ev);
        timed(e.last_prepare_ms, e.prepare_count, [&] {
            *generation = e.prepare_graph_device(num_nodes, node_types_device, num_neigh_device, num_edges,
                                                 neigh_indices_device, neigh_types_device);
        });
    });
}

int32_t smx_prepare_periodic_factorized_graph(SmxEvaluator* ev, int32_t num_nodes, const int32_t* node_types,
                                              const double* positions, const double* cell, const double* inverse_cell,
                                              double neighbor_cutoff, uint64_t* generation, int64_t* num_edges) {
    return guarded([&] {
        if (!generation || !num_edges || !cell || !inverse_cell) throw std::invalid_argument("missing argument");
        if (num_nodes > 0 && (!node_types || !positions)) throw std::invalid_argument("node arrays are required");
        auto& e = E(ev);
        timed(e.last_prepare_ms, e.prepare_count, [&] {
            const auto r = e.prepare_periodic(num_nodes, node_types, positions, cell, inverse_cell, neighbor_cutoff);
            *generation = r.first;
            *num_edges = r.second;
        });
    });
}

int32_t smx_set_execution_plan(SmxEvaluator* ev, const char* profile, int32_t tile_receivers) {
    return guarded([&] {
        auto& e = E(ev);
        const std::string p = profile ? profile : "auto";
        if (p != "auto" && p != "speed" && p != "capacity")
            throw std::invalid_argument("execution profile must be 'auto', 'speed' or 'capacity'");
        if (tile_receivers < 0) throw std::invalid_argument("tile_receivers must be non-negative");
        // auto: capacity profile with fixed workspaces allowed; capacity: the
        // tiled plan pinned; speed: the speed profile
        e.request_profile = p == "speed" ? "speed" : "capacity";
        e.allow_fixed = p != "speed";
        e.debug_plan = p == "capacity" ? e.tiled_plan() : "";
        if (tile_receivers > 0) e.tile_limit = tile_receivers;
    });
}

int32_t smx_set_execution_plan_request(SmxEvaluator* ev, const char* algorithm, const char* profile,
                                       const char* debug_plan) {
    return guarded([&] {
        auto& e = E(ev);
        const std::string a = algorithm ? algorithm : "direct", p = profile ? profile : "capacity";
        const std::string d = debug_plan ? debug_plan : "";
        if (a != "direct" && a != "factorized" && a != "direct_streamed")
            throw std::invalid_argument("the MI355X evaluator implements the 'direct' execution algorithm");
        if (p != "capacity" && p != "speed")
            throw std::invalid_argument("execution profile must be 'capacity' or 'speed'");
        if (!d.empty() && d != smx::Evaluator::kPlanSpeed && d != smx::Evaluator::kPlanRetained &&
            d != smx::Evaluator::kPlanTiled && d != smx::Evaluator::kPlanSingleTiled)
            throw std::invalid_argument("unknown debug execution plan '" + d + "'");
        e.request_profile = p;
        e.debug_plan = d;
    });
}

int32_t smx_set_allow_fixed_workspace(SmxEvaluator* ev, int32_t allow) {
    return guarded([&] { E(ev).allow_fixed = allow != 0; });
}

int32_t smx_execution_plan_report(SmxEvaluator* ev, char* out, int64_t capacity, int64_t* size) {
    return guarded([&] {
        const std::string r = E(ev).plan_report();
        if (size) *size = static_cast<int64_t>(r.size()) + 1;
        if (out) {
            if (capacity < static_cast<int64_t>(r.size()) + 1) throw std::invalid_argument("buffer too small");
            std::memcpy(out, r.c_str(), r.size() + 1);
        }
    });
}

int32_t smx_execution_plan(SmxEvaluator* ev, char* out, int64_t capacity) {
    return guarded([&] {
        const std::string d = E(ev).plan_description();
        if (!out || capacity < static_cast<int64_t>(d.size()) + 1) throw std::invalid_argument("buffer too small");
        std::memcpy(out, d.c_str(), d.size() + 1);
    });
}

int32_t smx_evaluator_counters(const SmxEvaluator* ev, SmxEvaluatorCounters* out) {
    return guarded([&] {
        if (!out || out->struct_size < sizeof(SmxEvaluatorCounters))
            throw std::invalid_argument("SmxEvaluatorCounters.struct_size is too small");
        const auto& e = E(ev);
        out->last_graph_prepare_ms = e.last_prepare_ms;
        out->last_evaluation_ms = e.last_evaluation_ms;
        out->graph_prepare_count = e.prepare_count;
        out->evaluation_count = e.evaluation_count;
        out->geometry_prepare_count = e.geometry_prepare_count;
    });
}

int32_t smx_prepare_active_types(SmxEvaluator* ev, const int32_t* types, int32_t count) {
    return guarded([&] {
        if (count < 0 || (count > 0 && !types)) throw std::invalid_argument("active types are required");
        E(ev).prepare_active_types(std::vector<int>(types, types + count));
    });
}

int32_t smx_update_factorized_cell(SmxEvaluator* ev, uint64_t generation, const double* cell,
                                   const double* inverse_cell) {
    return guarded([&] {
        if (!cell || !inverse_cell) throw std::invalid_argument("cell and inverse cell are required");
        E(ev).update_cell(generation, cell, inverse_cell);
    });
}

int32_t smx_prepare_factorized_geometry(SmxEvaluator* ev, uint64_t generation, const double* reference_positions,
                                        int64_t positions_count, const double* reference_xyz, int64_t xyz_count,
                                        const double* cell, const double* inverse_cell, const int32_t* pbc) {
    return guarded([&] {
        E(ev).prepare_geometry(generation, smx::Evaluator::Geometry::cartesian, reference_positions, positions_count,
                               reference_xyz, xyz_count, cell, inverse_cell, pbc);
    });
}

int32_t smx_prepare_factorized_shift_geometry(SmxEvaluator* ev, uint64_t generation,
                                              const double* reference_positions, int64_t positions_count,
                                              const int32_t* shifts, int64_t shifts_count, const double* cell,
                                              const double* inverse_cell, const int32_t* pbc) {
    return guarded([&] {
        E(ev).prepare_geometry(generation, smx::Evaluator::Geometry::shifts, reference_positions, positions_count,
                               shifts, shifts_count, cell, inverse_cell, pbc);
    });
}

int32_t smx_prepare_factorized_fractional_geometry(SmxEvaluator* ev, uint64_t generation,
                                                   const double* fractional_positions, int64_t positions_count,
                                                   const double* fractional_xyz, int64_t xyz_count,
                                                   const double* cell, const double* inverse_cell,
                                                   const int32_t* pbc) {
    return guarded([&] {
        E(ev).prepare_geometry(generation, smx::Evaluator::Geometry::fractional, fractional_positions,
                               positions_count, fractional_xyz, xyz_count, cell, inverse_cell, pbc);
    });
}

int32_t smx_prepare_factorized_feature_graph(SmxEvaluator* ev, int32_t num_receivers, int32_t num_feature_nodes,
                                             const int32_t* receiver_feature_indices, const int32_t* node_types,
                                             const int32_t* feature_types, const int32_t* num_neigh, int64_t num_edges,
                                             const int32_t* neigh_indices, const int32_t* neigh_types,
                                             uint64_t* generation) {
    return guarded([&] {
        if (!generation) throw std::invalid_argument("generation output is required");
        if (num_receivers < 0 || num_feature_nodes < num_receivers)
            throw std::invalid_argument("Prepared Execution R1 graph extents are inconsistent.");
        if ((num_receivers > 0 && (!receiver_feature_indices || !node_types || !num_neigh)) ||
            (num_feature_nodes > 0 && !feature_types) || (num_edges > 0 && (!neigh_indices || !neigh_types)))
            throw std::invalid_argument("graph arrays are required");
        auto& e = E(ev);
        timed(e.last_prepare_ms, e.prepare_count, [&] {
            *generation = e.prepare_feature_graph_host(num_receivers, num_feature_nodes, receiver_feature_indices,
                                                       node_types, feature_types, num_neigh, num_edges, neigh_indices,
                                                       neigh_types);
        });
    });
}
int32_t smx_prepare_factorized_feature_graph_device(SmxEvaluator* ev, int32_t num_receivers, int32_t num_feature_nodes,
                                                    const int32_t* receiver_feature_indices, const int32_t* node_types,
                                                    const int32_t* feature_types, const int32_t* num_neigh,
                                                    int64_t num_edges, const int32_t* neigh_indices,
                                                    const int32_t* neigh_types, uint64_t* generation) {
    return guarded([&] {
        if (num_receivers < 0 || num_feature_nodes < num_receivers || num_edges < 0 || num_edges > INT_MAX)
            throw std::invalid_argument("Prepared Execution R1 graph extents are inconsistent.");
        // checked on host copies, like the reference's device entry (lifecycle.cpp:2346-2380)
        auto copy = [](const int32_t* p, std::int64_t n) {
            std::vector<int> v(static_cast<std::size_t>(n));
            if (n > 0) {
                if (!p) throw std::invalid_argument("graph arrays are required");
                SMX_HIP(hipMemcpy(v.data(), p, sizeof(int) * n, hipMemcpyDeviceToHost));
            }
            return v;
        };
        const auto rf = copy(receiver_feature_indices, num_receivers), nt = copy(node_types, num_receivers);
        const auto ft = copy(feature_types, num_feature_nodes), nn = copy(num_neigh, num_receivers);
        const auto nb = copy(neigh_indices, num_edges), nbt = copy(neigh_types, num_edges);
        if (!generation) throw std::invalid_argument("generation output is required");
        auto& e = E(ev);
        timed(e.last_prepare_ms, e.prepare_count, [&] {
            *generation = e.prepare_feature_graph_host(num_receivers, num_feature_nodes, rf.data(), nt.data(),
                                                       ft.data(), nn.data(), num_edges, nb.data(), nbt.data());
        });
    });
}
int32_t smx_compute_factorized_single_layer_distributed_evaluation(SmxEvaluator* ev, uint64_t generation,
                                                                   int32_t num_receivers, int32_t num_feature_nodes,
                                                                   const double* xyz, const double* r,
                                                                   int32_t on_device) {
    return guarded([&] {
        auto& e = E(ev);
        timed(e.last_evaluation_ms, e.evaluation_count, [&] {
            e.single_layer_distributed(generation, num_receivers, num_feature_nodes, xyz, r, nullptr, on_device != 0);
        });
    });
}
int32_t smx_begin_factorized_distributed_evaluation(SmxEvaluator* ev, uint64_t generation, int32_t num_receivers,
                                                    int32_t num_feature_nodes, const double* xyz, const double* r,
                                                    int32_t on_device) {
    return guarded([&] {
        auto& e = E(ev);
        e.begin_distributed(generation, num_receivers, num_feature_nodes, xyz, r, nullptr, on_device != 0);
    });
}
int32_t smx_begin_factorized_distributed_positions_evaluation(SmxEvaluator* ev, uint64_t generation,
                                                              int32_t num_receivers, int32_t num_feature_nodes,
                                                              const double* feature_positions, int32_t on_device) {
    return guarded([&] {
        E(ev).begin_distributed(generation, num_receivers, num_feature_nodes, nullptr, nullptr, feature_positions,
                                on_device != 0);
    });
}
int32_t smx_compute_factorized_single_layer_distributed_positions_evaluation(SmxEvaluator* ev, uint64_t generation,
                                                                             int32_t num_receivers,
                                                                             int32_t num_feature_nodes,
                                                                             const double* feature_positions,
                                                                             int32_t on_device) {
    return guarded([&] {
        auto& e = E(ev);
        timed(e.last_evaluation_ms, e.evaluation_count, [&] {
            e.single_layer_distributed(generation, num_receivers, num_feature_nodes, nullptr, nullptr,
                                       feature_positions, on_device != 0);
        });
    });
}
int32_t smx_continue_factorized_distributed_evaluation(SmxEvaluator* ev, const float* communicated_h1, int64_t rows,
                                                       int32_t on_device) {
    return guarded([&] { E(ev).continue_distributed(communicated_h1, rows, on_device != 0); });
}
int32_t smx_finish_factorized_distributed_evaluation(SmxEvaluator* ev, const float* h1_adjoint, int64_t rows,
                                                     int32_t on_device) {
    return guarded([&] {
        auto& e = E(ev);
        timed(e.last_evaluation_ms, e.evaluation_count,
              [&] { e.finish_distributed(h1_adjoint, rows, on_device != 0); });
    });
}
int32_t smx_distributed_exchange(SmxEvaluator* ev, int32_t which, float** device_rows, int64_t* rows,
                                 int64_t* row_floats) {
    return guarded([&] {
        auto& e = E(ev);
        if (row_floats) *row_floats = static_cast<int64_t>(e.hm.num_LM) * e.hm.C;
        if (!device_rows && !rows) return;  // the row width alone, at any time
        if (which == 0) {
            if (e.phase != smx::Evaluator::Phase::prefix_complete)
                throw std::logic_error("the receivers' H1 is available after the prefix phase");
            if (device_rows) *device_rows = e.hm.field ? e.ws.H1p : e.ws.H1;
            if (rows) *rows = e.N;
        } else if (which == 1) {
            if (e.phase != smx::Evaluator::Phase::middle_complete)
                throw std::logic_error("the H1 adjoint is available after the middle phase");
            if (device_rows) *device_rows = e.h1_adjoint_exchange();
            if (rows) *rows = e.F;
        } else {
            throw std::invalid_argument("which must be 0 (receivers' H1) or 1 (feature nodes' H1 adjoint)");
        }
    });
}
int32_t smx_compute_prepared_factorized(SmxEvaluator* ev, uint64_t generation, const double* xyz, const double* r) {
    return guarded([&] {
        auto& e = E(ev);
        if (e.E > 0 && (!xyz || !r)) throw std::invalid_argument("xyz and r are required");
        timed(e.last_evaluation_ms, e.evaluation_count, [&] { e.compute_xyz(generation, xyz, r); });
    });
}

int32_t smx_compute_prepared_factorized_positions(SmxEvaluator* ev, uint64_t generation, const double* positions) {
    return guarded([&] {
        auto& e = E(ev);
        if (e.N > 0 && !positions) throw std::invalid_argument("positions are required");
        timed(e.last_evaluation_ms, e.evaluation_count, [&] { e.compute_positions(generation, positions, false); });
    });
}

int32_t smx_compute_prepared_factorized_positions_results(SmxEvaluator* ev, uint64_t generation,
                                                          const double* positions, double volume,
                                                          double* node_energies, double* forces, double* stress) {
    return guarded([&] {
        auto& e = E(ev);
        timed(e.last_evaluation_ms, e.evaluation_count,
              [&] { e.compute_results(generation, positions, volume, node_energies, forces, stress); });
    });
}

int32_t smx_compute_prepared_factorized_positions_device(SmxEvaluator* ev, uint64_t generation,
                                                         const double* positions_device) {
    return guarded([&] {
        auto& e = E(ev);
        if (e.N > 0 && !positions_device) throw std::invalid_argument("positions are required");
        timed(e.last_evaluation_ms, e.evaluation_count,
              [&] { e.compute_positions(generation, positions_device, true); });
    });
}

int32_t smx_set_electric_field(SmxEvaluator* ev, const double* field, int64_t count) {
    return guarded([&] { E(ev).set_field(field, count); });
}

int32_t smx_has_field_coupling(const SmxEvaluator* ev, int32_t* out) {
    return guarded([&] {
        if (!out) throw std::invalid_argument("out is NULL");
        *out = E(ev).hm.field ? 1 : 0;
    });
}

int32_t smx_compute_prepared_factorized_positions_field(SmxEvaluator* ev, uint64_t generation,
                                                        const double* positions, const double* field,
                                                        int64_t field_count) {
    return guarded([&] {
        auto& e = E(ev);
        if (e.N > 0 && !positions) throw std::invalid_argument("positions are required");
        if (!e.hm.field) throw std::invalid_argument("the model has no field coupling; it takes no electric_field");
        e.set_field(field, field_count);
        timed(e.last_evaluation_ms, e.evaluation_count, [&] { e.compute_positions(generation, positions, false); });
    });
}

int32_t smx_compute_prepared_factorized_field(SmxEvaluator* ev, uint64_t generation, const double* xyz,
                                              const double* r, const double* field, int64_t field_count) {
    return guarded([&] {
        auto& e = E(ev);
        if (e.E > 0 && (!xyz || !r)) throw std::invalid_argument("xyz and r are required");
        if (!e.hm.field) throw std::invalid_argument("the model has no field coupling; it takes no electric_field");
        e.set_field(field, field_count);
        timed(e.last_evaluation_ms, e.evaluation_count, [&] { e.compute_xyz(generation, xyz, r); });
    });
}

int32_t smx_electric_field_adj(SmxEvaluator* ev, double* out, int64_t capacity, int64_t* count) {
    return guarded([&] {
        auto& e = E(ev);
        if (!e.field_evaluated || !e.evaluated) throw std::logic_error("no field evaluation has run");
        // the shape of the field that evaluation ran in (a field set since
        // applies to the next one)
        const std::int64_t n = e.field_adj_count;
        if (count) *count = n;
        if (!out) return;
        if (capacity < n) throw std::invalid_argument("buffer too small");
        SMX_HIP(hipMemcpyAsync(out, e.ws.field_adj, n * sizeof(double), hipMemcpyDeviceToHost, e.stream));
        SMX_HIP(hipStreamSynchronize(e.stream));
        if (n != 3 && !e.h_feature_of.empty()) {
            // per-node rows back in the caller's feature order
            const std::vector<double> mine(out, out + n);
            for (int k = 0; k < e.F; ++k)
                for (int c = 0; c < 3; ++c) out[3 * static_cast<std::size_t>(e.h_feature_of[k]) + c] = mine[3 * k + c];
        }
    });
}

int32_t smx_compute_prepared_factorized_field_response(SmxEvaluator* ev, uint64_t generation, const double* field,
                                                       int64_t field_count, int32_t include_force_derivative,
                                                       int32_t scatter_bec_bins) {
    return guarded([&] {
        E(ev).field_response(generation, field, field_count, include_force_derivative != 0,
                             include_force_derivative != 0 && scatter_bec_bins != 0);
    });
}

int32_t smx_electric_field_hessian(SmxEvaluator* ev, double* out, int64_t capacity, int64_t* count) {
    return guarded([&] {
        auto& e = E(ev);
        if (!e.response_done) throw std::logic_error("no MACEField response has run");
        if (count) *count = 9;
        if (!out) return;
        if (capacity < 9) throw std::invalid_argument("buffer too small");
        std::copy(e.response_hessian, e.response_hessian + 9, out);
    });
}

int32_t smx_electric_field_force_derivative(SmxEvaluator* ev, double* out, int64_t capacity, int64_t* count) {
    return guarded([&] {
        auto& e = E(ev);
        if (!e.response_done) throw std::logic_error("no MACEField response has run");
        const std::int64_t n = e.response_has_forces ? 9 * e.response_E : 0;
        if (count) *count = n;
        if (!out || n == 0) return;
        if (capacity < n) throw std::invalid_argument("buffer too small");
        SMX_HIP(hipMemcpyAsync(out, e.rws.forces, n * sizeof(double), hipMemcpyDeviceToHost, e.stream));
        SMX_HIP(hipStreamSynchronize(e.stream));
    });
}

int32_t smx_electric_field_bec_bins(SmxEvaluator* ev, double* out, int64_t capacity, int64_t* count) {
    return guarded([&] {
        auto& e = E(ev);
        if (!e.response_done) throw std::logic_error("no MACEField response has run");
        const std::int64_t n = e.response_has_bins ? 9 * static_cast<std::int64_t>(e.response_N) : 0;
        if (count) *count = n;
        if (!out || n == 0) return;
        if (capacity < n) throw std::invalid_argument("buffer too small");
        // device [s][i][x] -> [i][s][x]
        std::vector<double> t(n);
        SMX_HIP(hipMemcpyAsync(t.data(), e.response_bins_dev, n * sizeof(double), hipMemcpyDeviceToHost, e.stream));
        SMX_HIP(hipStreamSynchronize(e.stream));
        const int N = e.response_N;
        for (int s = 0; s < 3; ++s)
            for (int i = 0; i < N; ++i)
                for (int x = 0; x < 3; ++x)
                    out[(static_cast<std::size_t>(i) * 3 + s) * 3 + x] = t[(static_cast<std::size_t>(s) * N + i) * 3 + x];
    });
}

int32_t smx_compute_node_energies_forces(SmxEvaluator* ev, int32_t num_nodes, const int32_t* node_types,
                                         const int32_t* num_neigh, int64_t num_edges, const int32_t* neigh_indices,
                                         const int32_t* neigh_types, const double* xyz, const double* r) {
    return guarded([&] {
        auto& e = E(ev);
        std::uint64_t token = 0;
        timed(e.last_prepare_ms, e.prepare_count, [&] {
            token = e.prepare_graph_host(num_nodes, node_types, num_neigh, num_edges, neigh_indices, neigh_types);
        });
        timed(e.last_evaluation_ms, e.evaluation_count, [&] { e.compute_xyz(token, xyz, r); });
    });
}

int32_t smx_reduce_prepared_node_forces(SmxEvaluator* ev, uint64_t generation, double* atom_forces) {
    return guarded([&] { E(ev).reduce_forces(generation, atom_forces); });
}

int32_t smx_reduce_prepared_stress(SmxEvaluator* ev, uint64_t generation, double volume, double* stress) {
    return guarded([&] { E(ev).reduce_stress(generation, volume, stress); });
}

int32_t smx_node_energies(SmxEvaluator* ev, double* out, int64_t capacity) {
    return guarded([&] {
        auto& e = E(ev);
        if ((!out && e.N > 0) || capacity < e.N) throw std::invalid_argument("buffer too small");
        if (!e.evaluated) throw std::logic_error("no evaluation has run");
        if (e.N > 0)
            SMX_HIP(hipMemcpyAsync(out, e.ws.node_energies, e.N * sizeof(double), hipMemcpyDeviceToHost, e.stream));
        SMX_HIP(hipStreamSynchronize(e.stream));
    });
}

int32_t smx_node_forces(SmxEvaluator* ev, double* out, int64_t capacity) {
    return guarded([&] {
        auto& e = E(ev);
        if ((!out && e.E > 0) || capacity < 3 * e.E) throw std::invalid_argument("buffer too small");
        if (!e.evaluated) throw std::logic_error("no evaluation has run");
        const double* nf = e.node_forces_device();
        if (e.E > 0) SMX_HIP(hipMemcpyAsync(out, nf, 3 * e.E * sizeof(double), hipMemcpyDeviceToHost, e.stream));
        SMX_HIP(hipStreamSynchronize(e.stream));
    });
}

int32_t smx_total_energy_device(SmxEvaluator* ev, double* total) {
    return guarded([&] { E(ev).total_energy(total); });
}

int32_t smx_device_outputs(SmxEvaluator* ev, SmxDeviceOutputs* out) {
    return guarded([&] {
        auto& e = E(ev);
        if (!out || out->struct_size < sizeof(SmxDeviceOutputs))
            throw std::invalid_argument("SmxDeviceOutputs.struct_size is too small");
        out->num_nodes = e.N;
        out->num_edges = e.E;
        out->node_energies = e.ws.node_energies;
        out->node_forces = e.tiled ? nullptr : e.ws.node_forces;
        out->atom_forces = e.d_atom_forces.as<double>();
        out->stress = e.d_stress.as<double>();
        out->total_energy = e.d_total.as<double>();
        out->xyz = e.d_xyz.as<double>();
        out->r = e.d_r.as<double>();
    });
}

int32_t smx_lammps_compute(SmxEvaluator* ev, const SmxLammpsArgsV1* args, double* energy, double* virial) {
    return guarded([&] {
        if (!args) throw std::invalid_argument("LAMMPS arguments are required");
        E(ev).lammps_compute(*args, energy, virial);
    });
}

int32_t smx_synchronize(SmxEvaluator* ev) {
    return guarded([&] { E(ev).sync(); });
}

int32_t smx_debug_stage(SmxEvaluator* ev, const char* name, float* out, int64_t capacity, int64_t* count) {
    return guarded([&] {
        if (!name || !count) throw std::invalid_argument("stage name and count output are required");
        *count = E(ev).stage(name, out, capacity);
    });
}

int32_t smx_set_kernel_timing(SmxEvaluator* ev, int32_t enabled) {
    return guarded([&] {
        auto& e = E(ev);
        SMX_HIP(hipStreamSynchronize(e.stream));
        if (enabled && !e.timer) e.timer = std::make_unique<smx::EventTimer>();
        if (!enabled) e.timer.reset();
    });
}

int32_t smx_set_kernel_timing_filter(SmxEvaluator* ev, const char* names) {
    return guarded([&] {
        auto& e = E(ev);
        if (!e.timer) throw std::logic_error("kernel timing is not enabled");
        e.timer->set_filter(names ? names : "");
    });
}

int32_t smx_kernel_timing_reset(SmxEvaluator* ev) {
    return guarded([&] {
        auto& e = E(ev);
        if (e.timer) {
            e.sync();
            e.timer->reset();
        }
    });
}

int32_t smx_kernel_timing(SmxEvaluator* ev, int32_t index, const char** name, double* total_ms, int64_t* launches) {
    return guarded([&] {
        auto& e = E(ev);
        if (!name || !total_ms || !launches) throw std::invalid_argument("outputs are required");
        *name = nullptr;
        *total_ms = 0.0;
        *launches = 0;
        if (e.timer) {
            e.sync();
            std::int64_t n = 0;
            if (e.timer->get(index, name, total_ms, &n)) *launches = n;
        }
    });
}

int32_t smx_neighbor_list(int32_t num_nodes, const double* positions, const double* cell, const double* inverse_cell,
                          double cutoff, int64_t* num_edges, int32_t* num_neigh, int32_t* offsets, int32_t* sources,
                          int32_t* shifts, double* fractional_xyz) {
    return guarded([&] {
        if (!num_edges || !cell || !inverse_cell) throw std::invalid_argument("missing argument");
        if (num_nodes > 0 && !positions) throw std::invalid_argument("positions are required");
        hipStream_t s;
        SMX_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
        smx::NeighborResult nr;
        auto cleanup = [&]() {
            for (void* p : {static_cast<void*>(nr.num_neigh), static_cast<void*>(nr.offsets),
                            static_cast<void*>(nr.sources), static_cast<void*>(nr.images),
                            static_cast<void*>(nr.wfrac), static_cast<void*>(nr.shifts),
                            static_cast<void*>(nr.fractional_xyz)})
                if (p) (void)hipFree(p);
            (void)hipStreamDestroy(s);
        };
        try {
            smx::build_neighbor_list(num_nodes, positions, cell, inverse_cell, cutoff, true, nr, s);
            const std::int64_t Ec = nr.num_edges;
            if (sources) {
                if (Ec > *num_edges) throw std::invalid_argument("edge buffers are smaller than the edge count");
                if (!num_neigh || !offsets || !shifts || !fractional_xyz)
                    throw std::invalid_argument("all output buffers are required");
                SMX_HIP(hipMemcpy(num_neigh, nr.num_neigh, sizeof(int) * num_nodes, hipMemcpyDeviceToHost));
                SMX_HIP(hipMemcpy(offsets, nr.offsets, sizeof(int) * (num_nodes + 1), hipMemcpyDeviceToHost));
                if (Ec > 0) {
                    SMX_HIP(hipMemcpy(sources, nr.sources, sizeof(int) * Ec, hipMemcpyDeviceToHost));
                    SMX_HIP(hipMemcpy(shifts, nr.shifts, sizeof(int) * 3 * Ec, hipMemcpyDeviceToHost));
                    SMX_HIP(hipMemcpy(fractional_xyz, nr.fractional_xyz, sizeof(double) * 3 * Ec,
                                      hipMemcpyDeviceToHost));
                }
            }
            *num_edges = Ec;
        } catch (...) {
            cleanup();
            throw;
        }
        cleanup();
    });
}

int32_t smx_model_array_f32(const char* model_path, const char* name, float* out, int64_t capacity, int64_t* count,
                            int32_t dims[4], double* h, double* x0) {
    return guarded([&] {
        if (!name) throw std::invalid_argument("array name is NULL");
        std::lock_guard<std::mutex> lock(g_export_mutex);
        const auto m = export_model(model_path);
        const std::string n(name);
        int32_t d[4] = {0, 0, 0, 0};
        if (n == "M0_weights") {
            d[0] = m->num_elements;
            d[1] = static_cast<int32_t>(m->m0_terms.size());
            d[2] = m->C;
            export_array(m->m0_coef, out, capacity, count);
        } else if (n == "H0") {
            d[0] = m->num_elements;
            d[1] = m->C;
            export_array(m->H0, out, capacity, count);
        } else if (n == "R0_spline") {
            // stored [interval][function][4]; exported [interval][4][function]
            const int F = m->R0_functions, I = m->spline_points - 1;
            d[0] = I;
            d[1] = 4;
            d[2] = F;
            std::vector<float> t(static_cast<std::size_t>(I) * 4 * F);
            for (int i = 0; i < I; ++i)
                for (int f = 0; f < F; ++f)
                    for (int c = 0; c < 4; ++c)
                        t[(static_cast<std::size_t>(i) * 4 + c) * F + f] =
                            m->R0_coef[(static_cast<std::size_t>(i) * F + f) * 4 + c];
            export_array(t, out, capacity, count);
            if (h) *h = m->h;
            if (x0) *x0 = m->grid_min;
        } else {
            throw std::invalid_argument("unknown model array " + n);
        }
        if (dims) std::copy(d, d + 4, dims);
    });
}

int32_t smx_model_array_i32(const char* model_path, const char* name, int32_t* out, int64_t capacity, int64_t* count,
                            int32_t dims[4]) {
    return guarded([&] {
        if (!name) throw std::invalid_argument("array name is NULL");
        std::lock_guard<std::mutex> lock(g_export_mutex);
        const auto m = export_model(model_path);
        const std::string n(name);
        int32_t d[4] = {0, 0, 0, 0};
        if (n == "M0_terms") {
            d[0] = static_cast<int32_t>(m->m0_terms.size());
            export_array(m->m0_terms, out, capacity, count);
        } else if (n == "M0_offsets") {
            d[0] = static_cast<int32_t>(m->m0_term_offset.size());
            export_array(m->m0_term_offset, out, capacity, count);
        } else {
            throw std::invalid_argument("unknown model array " + n);
        }
        if (dims) std::copy(d, d + 4, dims);
    });
}

}  // extern "C"
