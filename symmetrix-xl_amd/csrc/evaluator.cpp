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
#include <climits>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <new>
#include <numeric>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/symmetrix_mi355x.h"
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

struct HostGemmPlan {
    std::vector<GemmTile> tiles;
    std::vector<GemmGroup> groups;
    int max_n = 0;
    DevBuf d_tiles, d_groups;
    GemmPlan view;
};

}  // namespace

struct Evaluator {
    HostModel hm;
    DeviceModel dm;
    std::unique_ptr<KernelSet> ks;
    hipStream_t stream = nullptr;
    std::string streamed_edges = "direct";

    // model tables
    std::vector<std::unique_ptr<DevBuf>> model_bufs;

    // graph
    std::uint64_t generation = 0, next_generation = 1;
    int N = 0;
    std::int64_t E = 0;
    std::vector<int> h_node_types;
    DevBuf d_node_types, d_offsets, d_neigh, d_neigh_types, d_receivers, d_soff, d_sedges, d_counts, d_node_list;
    // periodic geometry reference
    bool has_fractional = false;
    double cell[9] = {0}, inv_cell[9] = {0};
    DevBuf d_fxyz, d_ref_positions, d_disp, d_positions;
    // per call
    DevBuf d_xyz, d_r, d_erec, d_invalid;
    DevBuf w_Phi0, w_A0, w_M0, w_H1, w_Phi1, w_A1, w_A1_adj, w_direct, w_dPhi1, w_Wsrc, w_H1_adj, w_M0_adj, w_A0_adj,
        w_Phi0_adj, d_node_energies, d_node_forces, d_atom_forces, d_stress, d_stress_partial, d_total;
    Workspace ws;
    HostGemmPlan plan_a0, plan_h1, plan_a1f, plan_a1r;
    bool evaluated = false;
    int stress_blocks = 1024;

    std::unique_ptr<EventTimer> timer;

    Evaluator(const std::string& path, const std::string& head) {
        hm.load(path, head);
        std::vector<int> le, ls, lo;
        if (!kernel_paths(hm.l_max, hm.L_max, le, ls, lo) || le != hm.path_le || ls != hm.path_ls ||
            lo != hm.path_lo)
            throw std::domain_error("the model's R1 paths have no compiled kernel set (l_max " +
                                    std::to_string(hm.l_max) + ", L_max " + std::to_string(hm.L_max) + ")");
        ks = make_kernel_set(hm.C, hm.l_max, hm.L_max);
        if (!ks)
            throw std::domain_error("no kernel set is compiled for " + std::to_string(hm.C) + " channels, l_max " +
                                    std::to_string(hm.l_max) + ", L_max " + std::to_string(hm.L_max));
        SMX_HIP(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
        upload_model();
        SMX_HIP(hipStreamSynchronize(stream));
    }

    ~Evaluator() {
        if (stream) {
            (void)hipStreamSynchronize(stream);
            timer.reset();
            (void)hipStreamDestroy(stream);
        }
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
        dm.R0c = reinterpret_cast<const float4*>(put(hm.R0_coef));
        dm.R1c = reinterpret_cast<const float4*>(put(hm.R1_coef));
        dm.H0 = put(hm.H0);
        dm.A0_w = put(hm.A0_w);
        dm.A0_wt = put(hm.A0_wt);
        dm.m0_terms = put(hm.m0_terms);
        dm.m0_toff = put(hm.m0_term_offset);
        dm.m0_term_offset = hm.m0_term_offset;
        dm.T0 = static_cast<int>(hm.m0_terms.size());
        dm.m0_coef = put(hm.m0_coef);
        dm.H1_w = put(hm.H1_w);
        dm.H1_wt = put(hm.H1_wt);
        dm.cg = put(hm.cg_dense);
        dm.A1_w = put(hm.A1_w);
        dm.A1_wt = put(hm.A1_wt);
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

    // ---------------------------------------------------------------- graph
    void build_plans() {
        const int C = hm.C, NY = hm.num_lm, NH = hm.num_LM, NLME = hm.num_lme;
        // node list sorted by type (stable) -> contiguous per-type ranges
        std::vector<int> order(N);
        std::iota(order.begin(), order.end(), 0);
        std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return h_node_types[a] < h_node_types[b]; });
        upload(d_node_list, order, stream);
        std::vector<std::pair<int, std::pair<int, int>>> ranges;  // type -> [begin, end)
        for (int p = 0; p < N;) {
            int q = p;
            while (q < N && h_node_types[order[q]] == h_node_types[order[p]]) ++q;
            ranges.push_back({h_node_types[order[p]], {p, q}});
            p = q;
        }
        auto add_tiles = [](HostGemmPlan& P, int group, int m, int begin, int end) {
            for (int s = begin; s < end; s += 16) P.tiles.push_back(GemmTile{s, std::min(16, end - s), group, m});
        };
        auto finish = [&](HostGemmPlan& P) {
            for (const auto& g : P.groups) P.max_n = std::max(P.max_n, g.N);
            P.view.tiles = upload(P.d_tiles, P.tiles, stream);
            P.view.groups = upload(P.d_groups, P.groups, stream);
            P.view.node_list = d_node_list.as<int>();
            P.view.num_tiles = static_cast<int>(P.tiles.size());
            P.view.max_n = P.max_n;
        };
        for (HostGemmPlan* P : {&plan_a0, &plan_h1, &plan_a1f, &plan_a1r}) {
            P->tiles.clear();
            P->groups.clear();
            P->max_n = 0;
        }
        // A0: per (type, l), C x C
        for (const auto& tr : ranges) {
            const int t = tr.first;
            for (int l = 0; l <= hm.l_max; ++l) {
                const int g = static_cast<int>(plan_a0.groups.size());
                plan_a0.groups.push_back(GemmGroup{(static_cast<std::int64_t>(t) * (hm.l_max + 1) + l) * C * C, C, C,
                                                   NY * C, l * l * C, C, NY * C, l * l * C, C});
                for (int m = 0; m < 2 * l + 1; ++m) add_tiles(plan_a0, g, m, tr.second.first, tr.second.second);
            }
        }
        // H1: per l <= L_max
        for (int l = 0; l <= hm.L_max; ++l) {
            const int g = static_cast<int>(plan_h1.groups.size());
            plan_h1.groups.push_back(GemmGroup{static_cast<std::int64_t>(l) * C * C, C, C, NH * C, l * l * C, C,
                                               NH * C, l * l * C, C});
            for (int m = 0; m < 2 * l + 1; ++m) add_tiles(plan_h1, g, m, 0, N);
        }
        // A1 forward / reverse: per l with paths
        for (int l = 0; l <= hm.l_max; ++l) {
            const int ne = hm.num_e[l];
            if (ne == 0) continue;
            const int gf = static_cast<int>(plan_a1f.groups.size());
            plan_a1f.groups.push_back(GemmGroup{hm.A1_offset[l], ne * C, C, NLME * C, hm.lme_base[l] * C, ne * C,
                                                NY * C, l * l * C, C});
            const int gr = static_cast<int>(plan_a1r.groups.size());
            plan_a1r.groups.push_back(GemmGroup{hm.A1_offset[l], C, ne * C, NY * C, l * l * C, C, NLME * C,
                                                hm.lme_base[l] * C, ne * C});
            for (int m = 0; m < 2 * l + 1; ++m) {
                add_tiles(plan_a1f, gf, m, 0, N);
                add_tiles(plan_a1r, gr, m, 0, N);
            }
        }
        for (HostGemmPlan* P : {&plan_a0, &plan_h1, &plan_a1f, &plan_a1r}) finish(*P);
    }

    void ensure_workspace() {
        const std::size_t C = hm.C, NY = hm.num_lm, NH = hm.num_LM, NLME = hm.num_lme;
        const std::size_t n = std::max(N, 1), e = std::max<std::int64_t>(E, 1);
        auto f = [&](DevBuf& b, std::size_t count) { return static_cast<float*>(b.ensure(count * sizeof(float))); };
        ws.Phi0 = f(w_Phi0, n * NY * C);
        ws.A0 = f(w_A0, n * NY * C);
        ws.M0 = f(w_M0, n * NH * C);
        ws.H1 = f(w_H1, n * NH * C);
        ws.Phi1 = f(w_Phi1, n * NLME * C);
        ws.A1 = f(w_A1, n * NY * C);
        ws.A1_adj = f(w_A1_adj, n * NY * C);
        ws.direct = f(w_direct, n * C);
        ws.dPhi1 = f(w_dPhi1, n * NLME * C);
        ws.Wsrc = f(w_Wsrc, e * NH * C);
        ws.H1_adj = f(w_H1_adj, n * NH * C);
        ws.M0_adj = f(w_M0_adj, n * NH * C);
        ws.A0_adj = f(w_A0_adj, n * NY * C);
        ws.Phi0_adj = f(w_Phi0_adj, n * NY * C);
        ws.node_energies = static_cast<double*>(d_node_energies.ensure(n * sizeof(double)));
        ws.node_forces = static_cast<double*>(d_node_forces.ensure(e * 3 * sizeof(double)));
        d_atom_forces.ensure(n * 3 * sizeof(double));
        d_stress.ensure(9 * sizeof(double));
        d_stress_partial.ensure(static_cast<std::size_t>(stress_blocks) * 9 * sizeof(double));
        d_total.ensure(sizeof(double));
        d_xyz.ensure(e * 3 * sizeof(double));
        d_r.ensure(e * sizeof(double));
        d_erec.ensure(e * ks->record_floats() * sizeof(float));
        d_invalid.ensure(sizeof(int));
        d_positions.ensure(n * 3 * sizeof(double));
        d_disp.ensure(n * 3 * sizeof(double));
    }

    void validate_types(int n, const int* types) const {
        for (int i = 0; i < n; ++i)
            if (types[i] < 0 || types[i] >= hm.num_elements)
                throw std::invalid_argument("node type index is out of range");
    }

    // receiver CSR on the device -> schedule, plans, workspace, token
    std::uint64_t finish_graph() {
        d_receivers.ensure(std::max<std::int64_t>(E, 1) * sizeof(int));
        d_soff.ensure((N + 1) * sizeof(int));
        d_sedges.ensure(std::max<std::int64_t>(E, 1) * sizeof(int));
        d_counts.ensure(std::max(N, 1) * sizeof(int));
        launch_graph_schedule(N, E, d_offsets.as<int>(), d_neigh.as<int>(), d_receivers.as<int>(), d_soff.as<int>(),
                              d_sedges.as<int>(), d_counts.as<int>(), stream);
        build_plans();
        ensure_workspace();
        SMX_HIP(hipStreamSynchronize(stream));
        evaluated = false;
        generation = next_generation++;
        return generation;
    }

    std::uint64_t prepare_graph_host(int n, const int* node_types, const int* num_neigh, std::int64_t num_edges,
                                     const int* neigh, const int* neigh_types) {
        if (n < 0) throw std::invalid_argument("num_nodes must be non-negative");
        if (num_edges < 0 || num_edges > INT_MAX)
            throw std::invalid_argument("edge count exceeds the 32-bit graph limit");
        validate_types(n, node_types);
        std::vector<int> off(n + 1, 0);
        std::int64_t total = 0;
        for (int i = 0; i < n; ++i) {
            if (num_neigh[i] < 0) throw std::invalid_argument("num_neigh must be non-negative");
            total += num_neigh[i];
            if (total > INT_MAX) throw std::invalid_argument("edge count exceeds the 32-bit graph limit");
            off[i + 1] = static_cast<int>(total);
        }
        if (total != num_edges) throw std::invalid_argument("num_neigh does not sum to the number of edges");
        for (std::int64_t e = 0; e < num_edges; ++e) {
            if (neigh[e] < 0 || neigh[e] >= n) throw std::invalid_argument("neighbour index is out of range");
            if (neigh_types[e] < 0 || neigh_types[e] >= hm.num_elements)
                throw std::invalid_argument("neighbour type index is out of range");
        }
        N = n;
        E = num_edges;
        h_node_types.assign(node_types, node_types + n);
        upload(d_node_types, h_node_types, stream);
        upload(d_offsets, off, stream);
        upload(d_neigh, std::vector<int>(neigh, neigh + E), stream);
        upload(d_neigh_types, std::vector<int>(neigh_types, neigh_types + E), stream);
        has_fractional = false;
        return finish_graph();
    }

    std::uint64_t prepare_graph_device(int n, const int* node_types, const int* num_neigh, std::int64_t num_edges,
                                       const int* neigh, const int* neigh_types) {
        // The CSR is validated on the host copy: the reference's device path
        // trusts its LAMMPS caller, this one checks like the host path.
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

    std::pair<std::uint64_t, std::int64_t> prepare_periodic(int n, const int* node_types, const double* positions,
                                                            const double* cell_, const double* inv_,
                                                            double cutoff) {
        if (n < 0) throw std::invalid_argument("num_nodes must be non-negative");
        validate_types(n, node_types);
        NeighborResult nr;
        build_neighbor_list(n, positions, cell_, inv_, cutoff, nr, stream);
        struct Guard {
            NeighborResult& r;
            ~Guard() {
                for (void* p : {static_cast<void*>(r.num_neigh), static_cast<void*>(r.offsets),
                                static_cast<void*>(r.sources), static_cast<void*>(r.shifts),
                                static_cast<void*>(r.fractional_xyz)})
                    if (p) (void)hipFree(p);
            }
        } guard{nr};
        N = n;
        E = nr.num_edges;
        h_node_types.assign(node_types, node_types + n);
        upload(d_node_types, h_node_types, stream);
        int* off = static_cast<int*>(d_offsets.ensure((N + 1) * sizeof(int)));
        SMX_HIP(hipMemcpyAsync(off, nr.offsets, (N + 1) * sizeof(int), hipMemcpyDeviceToDevice, stream));
        int* nb = static_cast<int*>(d_neigh.ensure(std::max<std::int64_t>(E, 1) * sizeof(int)));
        if (E > 0) SMX_HIP(hipMemcpyAsync(nb, nr.sources, E * sizeof(int), hipMemcpyDeviceToDevice, stream));
        int* nt = static_cast<int*>(d_neigh_types.ensure(std::max<std::int64_t>(E, 1) * sizeof(int)));
        launch_gather_types(E, nb, d_node_types.as<int>(), nt, stream);
        double* fx = static_cast<double*>(d_fxyz.ensure(std::max<std::int64_t>(E, 1) * 3 * sizeof(double)));
        if (E > 0)
            SMX_HIP(hipMemcpyAsync(fx, nr.fractional_xyz, E * 3 * sizeof(double), hipMemcpyDeviceToDevice, stream));
        double* rp = static_cast<double*>(d_ref_positions.ensure(std::max(N, 1) * 3 * sizeof(double)));
        if (N > 0) SMX_HIP(hipMemcpyAsync(rp, positions, N * 3 * sizeof(double), hipMemcpyHostToDevice, stream));
        std::memcpy(cell, cell_, sizeof(cell));
        std::memcpy(inv_cell, inv_, sizeof(inv_cell));
        has_fractional = true;
        const std::uint64_t token = finish_graph();
        return {token, E};
    }

    void check_generation(std::uint64_t token) const {
        if (token == 0 || token != generation)
            throw std::invalid_argument("execution graph generation is stale or was never prepared");
    }

    // ----------------------------------------------------------------- calls
    void evaluate_edges() {
        const DeviceGraph g = view();
        ks->edge_geometry(dm, E, d_xyz.as<double>(), d_r.as<double>(), d_erec.as<float>(), stream);
        if (hm.num_e.end() != std::find(hm.num_e.begin(), hm.num_e.end(), 0))
            SMX_HIP(hipMemsetAsync(ws.A1, 0, sizeof(float) * std::max(N, 1) * hm.num_lm * hm.C, stream));
        LaunchTimer* t = timer.get();
        ks->forward(dm, g, ws, plan_a0.view, plan_h1.view, plan_a1f.view, stream, t);
        ks->reverse(dm, g, ws, plan_a0.view, plan_h1.view, plan_a1r.view, stream, t);
        evaluated = true;
    }

    void finish_call(bool check_invalid) {
        int invalid = 0;
        if (check_invalid)
            SMX_HIP(hipMemcpyAsync(&invalid, d_invalid.as<int>(), sizeof(int), hipMemcpyDeviceToHost, stream));
        SMX_HIP(hipStreamSynchronize(stream));
        if (timer) timer->collect();
        if (invalid > 0)
            throw std::runtime_error("prepared geometry produced " + std::to_string(invalid) +
                                     " invalid (zero-length or non-finite) edges");
    }

    void compute_positions(std::uint64_t token, const double* positions, bool on_device) {
        check_generation(token);
        if (!has_fractional)
            throw std::logic_error("the prepared graph has no periodic geometry reference; "
                                   "use compute_prepared_factorized with xyz and r");
        const double* pos = positions;
        if (!on_device) {
            for (int i = 0; i < 3 * N; ++i)
                if (!std::isfinite(positions[i])) throw std::invalid_argument("positions must be finite");
            double* dp = static_cast<double*>(d_positions.ensure(std::max(N, 1) * 3 * sizeof(double)));
            if (N > 0) SMX_HIP(hipMemcpyAsync(dp, positions, N * 3 * sizeof(double), hipMemcpyHostToDevice, stream));
            pos = dp;
        }
        SMX_HIP(hipMemsetAsync(d_invalid.as<int>(), 0, sizeof(int), stream));
        {
            if (timer) timer->begin("edge_geometry", stream);
            launch_prepared_geometry(N, E, d_receivers.as<int>(), d_neigh.as<int>(), d_fxyz.as<double>(), cell,
                                     inv_cell, d_ref_positions.as<double>(), pos, hm.r_cut, d_disp.as<double>(),
                                     d_xyz.as<double>(), d_r.as<double>(), d_invalid.as<int>(), stream);
            if (timer) timer->end("edge_geometry", stream);
        }
        evaluate_edges();
        finish_call(true);
    }

    void compute_xyz(std::uint64_t token, const double* xyz, const double* r) {
        check_generation(token);
        for (std::int64_t e = 0; e < E; ++e) {
            if (!std::isfinite(r[e]) || !(r[e] > 0.0) || !std::isfinite(xyz[3 * e]) || !std::isfinite(xyz[3 * e + 1]) ||
                !std::isfinite(xyz[3 * e + 2]))
                throw std::invalid_argument("MACE graph has an invalid distance or displacement vector");
        }
        if (E > 0) {
            SMX_HIP(hipMemcpyAsync(d_xyz.as<double>(), xyz, E * 3 * sizeof(double), hipMemcpyHostToDevice, stream));
            SMX_HIP(hipMemcpyAsync(d_r.as<double>(), r, E * sizeof(double), hipMemcpyHostToDevice, stream));
        }
        evaluate_edges();
        finish_call(false);
    }

    void update_cell(std::uint64_t token, const double* cell_, const double* inv_) {
        check_generation(token);
        if (!has_fractional) throw std::logic_error("the prepared graph has no periodic geometry reference");
        std::memcpy(cell, cell_, sizeof(cell));
        std::memcpy(inv_cell, inv_, sizeof(inv_cell));
    }

    DeviceGraph view() const {
        DeviceGraph g;
        g.N = N;
        g.E = E;
        g.node_types = d_node_types.as<int>();
        g.offsets = d_offsets.as<int>();
        g.neigh = d_neigh.as<int>();
        g.neigh_types = d_neigh_types.as<int>();
        g.receivers = d_receivers.as<int>();
        g.soff = d_soff.as<int>();
        g.sedges = d_sedges.as<int>();
        g.erec = d_erec.as<float>();
        return g;
    }

    void require_evaluated(std::uint64_t token) const {
        check_generation(token);
        if (!evaluated) throw std::logic_error("no evaluation has run on the prepared graph");
    }

    void reduce_forces(std::uint64_t token, double* out) {
        require_evaluated(token);
        launch_atom_forces(N, d_offsets.as<int>(), d_soff.as<int>(), d_sedges.as<int>(), ws.node_forces,
                           d_atom_forces.as<double>(), stream);
        if (out) {
            if (N > 0)
                SMX_HIP(hipMemcpyAsync(out, d_atom_forces.as<double>(), N * 3 * sizeof(double), hipMemcpyDeviceToHost,
                                       stream));
            SMX_HIP(hipStreamSynchronize(stream));
        }
    }

    void reduce_stress(std::uint64_t token, double volume, double* out) {
        require_evaluated(token);
        if (!(volume > 0.0) || !std::isfinite(volume)) throw std::invalid_argument("volume must be positive");
        launch_stress(E, ws.node_forces, d_xyz.as<double>(), volume, d_stress_partial.as<double>(), stress_blocks,
                      d_stress.as<double>(), stream);
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

    std::int64_t stage(const std::string& name, float* out, std::int64_t capacity) {
        const std::int64_t n = N, C = hm.C, NY = hm.num_lm, NH = hm.num_LM, NLME = hm.num_lme;
        const float* src = nullptr;
        std::int64_t count = 0;
        if (name == "A0") src = ws.A0, count = n * NY * C;
        else if (name == "Phi0") src = ws.Phi0, count = n * NY * C;
        else if (name == "M0") src = ws.M0, count = n * NH * C;
        else if (name == "H1") src = ws.H1, count = n * NH * C;
        else if (name == "Phi1") src = ws.Phi1, count = n * NLME * C;
        else if (name == "A1") src = ws.A1, count = n * NY * C;
        else if (name == "A1_adj") src = ws.A1_adj, count = n * NY * C;
        else if (name == "dPhi1") src = ws.dPhi1, count = n * NLME * C;
        else if (name == "H1_adj") src = ws.H1_adj, count = n * NH * C;
        else if (name == "M0_adj") src = ws.M0_adj, count = n * NH * C;
        else if (name == "A0_adj") src = ws.A0_adj, count = n * NY * C;
        else if (name == "direct") src = ws.direct, count = n * C;
        else if (name == "edge_records") src = d_erec.as<float>(), count = E * ks->record_floats();
        else throw std::invalid_argument("unknown stage '" + name + "'");
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

int32_t smx_evaluator_info(const SmxEvaluator* ev, SmxModelInfo* info) {
    return guarded([&] {
        const auto& m = E(ev).hm;
        if (!info || info->struct_size < sizeof(SmxModelInfo))
            throw std::invalid_argument("SmxModelInfo.struct_size is too small");
        info->num_elements = m.num_elements;
        info->num_channels = m.C;
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
        *generation = E(ev).prepare_graph_host(num_nodes, node_types, num_neigh, num_edges, neigh_indices, neigh_types);
    });
}

int32_t smx_prepare_factorized_graph_device(SmxEvaluator* ev, int32_t num_nodes, const int32_t* node_types_device,
                                            const int32_t* num_neigh_device, int64_t num_edges,
                                            const int32_t* neigh_indices_device, const int32_t* neigh_types_device,
                                            uint64_t* generation) {
    return guarded([&] {
        if (!generation) throw std::invalid_argument("generation output is required");
        if (num_edges < 0 || num_edges > INT_MAX) throw std::invalid_argument("edge count exceeds the 32-bit graph limit");
        *generation = E(ev).prepare_graph_device(num_nodes, node_types_device, num_neigh_device, num_edges,
                                                 neigh_indices_device, neigh_types_device);
    });
}

int32_t smx_prepare_periodic_factorized_graph(SmxEvaluator* ev, int32_t num_nodes, const int32_t* node_types,
                                              const double* positions, const double* cell, const double* inverse_cell,
                                              double neighbor_cutoff, uint64_t* generation, int64_t* num_edges) {
    return guarded([&] {
        if (!generation || !num_edges || !cell || !inverse_cell) throw std::invalid_argument("missing argument");
        if (num_nodes > 0 && (!node_types || !positions)) throw std::invalid_argument("node arrays are required");
        const auto r = E(ev).prepare_periodic(num_nodes, node_types, positions, cell, inverse_cell, neighbor_cutoff);
        *generation = r.first;
        *num_edges = r.second;
    });
}

int32_t smx_update_factorized_cell(SmxEvaluator* ev, uint64_t generation, const double* cell,
                                   const double* inverse_cell) {
    return guarded([&] {
        if (!cell || !inverse_cell) throw std::invalid_argument("cell and inverse cell are required");
        E(ev).update_cell(generation, cell, inverse_cell);
    });
}

int32_t smx_compute_prepared_factorized(SmxEvaluator* ev, uint64_t generation, const double* xyz, const double* r) {
    return guarded([&] {
        auto& e = E(ev);
        if (e.E > 0 && (!xyz || !r)) throw std::invalid_argument("xyz and r are required");
        e.compute_xyz(generation, xyz, r);
    });
}

int32_t smx_compute_prepared_factorized_positions(SmxEvaluator* ev, uint64_t generation, const double* positions) {
    return guarded([&] {
        auto& e = E(ev);
        if (e.N > 0 && !positions) throw std::invalid_argument("positions are required");
        e.compute_positions(generation, positions, false);
    });
}

int32_t smx_compute_prepared_factorized_positions_device(SmxEvaluator* ev, uint64_t generation,
                                                         const double* positions_device) {
    return guarded([&] {
        auto& e = E(ev);
        if (e.N > 0 && !positions_device) throw std::invalid_argument("positions are required");
        e.compute_positions(generation, positions_device, true);
    });
}

int32_t smx_compute_node_energies_forces(SmxEvaluator* ev, int32_t num_nodes, const int32_t* node_types,
                                         const int32_t* num_neigh, int64_t num_edges, const int32_t* neigh_indices,
                                         const int32_t* neigh_types, const double* xyz, const double* r) {
    return guarded([&] {
        auto& e = E(ev);
        const auto token = e.prepare_graph_host(num_nodes, node_types, num_neigh, num_edges, neigh_indices, neigh_types);
        e.compute_xyz(token, xyz, r);
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
        if (!out || capacity < e.N) throw std::invalid_argument("buffer too small");
        if (!e.evaluated) throw std::logic_error("no evaluation has run");
        if (e.N > 0)
            SMX_HIP(hipMemcpyAsync(out, e.ws.node_energies, e.N * sizeof(double), hipMemcpyDeviceToHost, e.stream));
        SMX_HIP(hipStreamSynchronize(e.stream));
    });
}

int32_t smx_node_forces(SmxEvaluator* ev, double* out, int64_t capacity) {
    return guarded([&] {
        auto& e = E(ev);
        if (!out || capacity < 3 * e.E) throw std::invalid_argument("buffer too small");
        if (!e.evaluated) throw std::logic_error("no evaluation has run");
        if (e.E > 0)
            SMX_HIP(hipMemcpyAsync(out, e.ws.node_forces, 3 * e.E * sizeof(double), hipMemcpyDeviceToHost, e.stream));
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
        out->node_forces = e.ws.node_forces;
        out->atom_forces = e.d_atom_forces.as<double>();
        out->stress = e.d_stress.as<double>();
        out->total_energy = e.d_total.as<double>();
        out->xyz = e.d_xyz.as<double>();
        out->r = e.d_r.as<double>();
    });
}

int32_t smx_synchronize(SmxEvaluator* ev) {
    return guarded([&] { SMX_HIP(hipStreamSynchronize(E(ev).stream)); });
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
        if (e.timer) e.timer->reset();
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
                            static_cast<void*>(nr.sources), static_cast<void*>(nr.shifts),
                            static_cast<void*>(nr.fractional_xyz)})
                if (p) (void)hipFree(p);
            (void)hipStreamDestroy(s);
        };
        try {
            smx::build_neighbor_list(num_nodes, positions, cell, inverse_cell, cutoff, nr, s);
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

}  // extern "C"
