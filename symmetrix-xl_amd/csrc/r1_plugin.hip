// The reference's R1 HIP plugin ABI (jit_hip_plugin_abi.h) on the MI355X
// edge kernels: symmetrix_jit_hip_plugin_query_v1 and its two launchers.
//
// The launchers validate their packets as the reference's generated ones do
// (jit_codegen.py:3346-3410) and enqueue on the caller's stream:
//   forward  -> k_r1_forward over the caller's receiver CSR (first_neigh,
//               num_neigh), output assigned;
//   reverse  -> receiver offsets from edge_receivers (binary search),
//               k_r1_reverse (directed forces subtracted, per-edge source
//               terms W into a stream-ordered workspace), then
//               k_source_gather adding the FP64 source sums to
//               source_adjoint over the caller's source transpose.
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <cstring>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/symmetrix_r1_plugin.h"
#include "device_common.hpp"
#include "edge_kernels.hpp"
#include "kernels.hpp"
#include "model.hpp"

namespace smx {
namespace {

using namespace edge;

// offsets[i] = first edge of receiver i in the receiver-major edge list
// (lower bound of i in edge_receivers), offsets[N] = E
__global__ __launch_bounds__(256) void k_offsets_from_receivers(int N, int E, const int* __restrict__ receivers,
                                                               int* __restrict__ offsets) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i > N) return;
    int lo = 0, hi = E;
    while (lo < hi) {
        const int mid = lo + ((hi - lo) >> 1);
        if (receivers[mid] < i)
            lo = mid + 1;
        else
            hi = mid;
    }
    offsets[i] = lo;
}

struct PluginState {
    SymmetrixJitHipPluginV1 descriptor{};
    std::string artifact_id, contract, semantic, structure, features, arch = "gfx950";
    int C = 0, l_max = 0, L_max = 0, NY = 0, NH = 0, NLME = 0, functions = 0;
    int fp64_point = 0;
    float* cg = nullptr;  // dense per-path coupling blocks (device)
    std::vector<float> spline;  // [intervals][4][functions]
    int intervals = 0;
    double h = 0.0, x0 = 0.0;
    bool configured = false;
    ~PluginState() {
        if (cg) (void)hipFree(cg);
    }
};

std::mutex g_mutex;
// configured states; earlier ones stay alive because a loader may still
// hold their descriptor
std::vector<std::unique_ptr<PluginState>> g_states;
PluginState* g_active = nullptr;  // read by the launchers and the query

template <int NY>
PluginEdges<NY> plugin_edges(const PluginState& st, const SymmetrixJitHipRadialSplineV1& radial,
                             const double* radius, const void* harm, const void* grad, const void* xyz, bool unit,
                             const int* node_types, const int* neigh_types, const int* type_to_active,
                             unsigned active_types, double cutoff) {
    PluginEdges<NY> p;
    p.radius = radius;
    p.harm = static_cast<const float*>(harm);
    p.grad = static_cast<const float*>(grad);
    p.xyz64 = unit ? nullptr : static_cast<const double*>(xyz);
    p.unit32 = unit ? static_cast<const float*>(xyz) : nullptr;
    p.coef = static_cast<const float*>(radial.coefficients);
    p.node_types = node_types;
    p.neigh_types = neigh_types;
    p.type_to_active = type_to_active;
    p.x0 = radial.x0;
    p.h = radial.h;
    p.cutoff = cutoff;
    p.intervals = static_cast<int>(radial.intervals);
    p.functions = static_cast<int>(radial.functions);
    p.active_types = static_cast<int>(active_types);
    p.fp64_point = st.fp64_point;
    return p;
}

bool radial_ok(const PluginState& st, const SymmetrixJitHipRadialSplineV1& r, unsigned active_types) {
    const unsigned pairs = active_types * (active_types + 1) / 2;
    return r.struct_size >= sizeof(SymmetrixJitHipRadialSplineV1) && r.coefficients != nullptr &&
           r.intervals > 0 && r.functions == static_cast<unsigned>(st.functions) && r.edge_types >= pairs &&
           std::isfinite(r.h) && r.h > 0.0 && std::isfinite(r.x0);
}

template <int C, int LMAX, int LMAXH>
int32_t forward_launch(const SymmetrixJitHipR1ForwardArgsV1* a, void* stream, int32_t persistent_blocks) {
    PluginState* st = g_active;
    if (!st || !a || a->struct_size < sizeof(SymmetrixJitHipR1ForwardArgsV1) || a->num_nodes < 0 ||
        a->num_nodes > INT32_MAX || a->num_edges < 0 || a->num_edges > INT32_MAX || !std::isfinite(a->cutoff) ||
        a->cutoff <= 0.0 || a->active_type_count == 0 || persistent_blocks <= 0 ||
        !radial_ok(*st, a->radial, a->active_type_count))
        return static_cast<int32_t>(hipErrorInvalidValue);
    if (a->num_nodes == 0) return static_cast<int32_t>(hipSuccess);
    if (!a->node_types || !a->num_neigh || !a->first_neigh || !a->type_to_active || !a->neighbor_features ||
        !a->output || (a->num_edges > 0 && (!a->neigh_indices || !a->neigh_types || !a->radius ||
                                            !a->harmonics_values)))
        return static_cast<int32_t>(hipErrorInvalidValue);
    using S = Shape<LMAX, LMAXH>;
    const auto edges = plugin_edges<S::NY>(*st, a->radial, a->radius, a->harmonics_values, nullptr, nullptr, false,
                                           a->node_types, a->neigh_types, a->type_to_active, a->active_type_count,
                                           a->cutoff);
    static_assert(SourceGroups<LMAX, LMAXH>::masks.size() == 1, "the plugin runs single-pass shapes");
    constexpr unsigned kAll = SourceGroups<LMAX, LMAXH>::masks[0];
    k_r1_forward<C, LMAX, LMAXH, kAll, false, PluginEdges<S::NY>><<<static_cast<unsigned>(a->num_nodes), C, 0,
                                                      static_cast<hipStream_t>(stream)>>>(
        0, a->first_neigh, a->num_neigh, a->neigh_indices, edges, static_cast<const float*>(a->neighbor_features),
        st->cg, static_cast<float*>(a->output));
    return static_cast<int32_t>(hipPeekAtLastError());
}

template <int C, int LMAX, int LMAXH>
int32_t reverse_launch(const SymmetrixJitHipR1SourceArgsV1* s, const SymmetrixJitHipR1EdgeArgsV1* e, void* stream,
                       int32_t persistent_blocks) {
    PluginState* st = g_active;
    if (!st || !s || !e || s->struct_size < sizeof(SymmetrixJitHipR1SourceArgsV1) ||
        e->struct_size < sizeof(SymmetrixJitHipR1EdgeArgsV1) || s->num_nodes < 0 || s->num_nodes > INT32_MAX ||
        s->num_edges < 0 || s->num_edges > INT32_MAX || s->num_edges != e->num_edges ||
        s->num_nodes != e->num_nodes || s->active_type_count != e->active_type_count || s->cutoff != e->cutoff ||
        !std::isfinite(s->cutoff) || s->cutoff <= 0.0 || s->active_type_count == 0 || persistent_blocks <= 0 ||
        !radial_ok(*st, s->radial, s->active_type_count) || !radial_ok(*st, e->radial, e->active_type_count))
        return static_cast<int32_t>(hipErrorInvalidValue);
    if (s->num_nodes == 0 || s->num_edges == 0) return static_cast<int32_t>(hipSuccess);
    const bool unit = e->coordinates_are_unit != 0;
    if (!e->node_types || !e->neigh_indices || !e->neigh_types || !e->edge_receivers || !e->type_to_active ||
        !e->xyz || !e->radius || !e->harmonics_values || !e->harmonics_gradients || !e->neighbor_features ||
        !e->output_adjoint || !e->directed_forces || !s->source_offsets || !s->source_edges ||
        !s->source_adjoint || e->coordinate_scalar_size != (unit ? sizeof(float) : sizeof(double)))
        return static_cast<int32_t>(hipErrorInvalidValue);
    using S = Shape<LMAX, LMAXH>;
    const int N = static_cast<int>(s->num_nodes);
    const std::int64_t E = s->num_edges;
    const auto hs = static_cast<hipStream_t>(stream);
    // stream-ordered workspace: receiver offsets [N+1] (padded) and W [E][NH][C]
    const std::size_t off_bytes = ((static_cast<std::size_t>(N) + 1) * sizeof(int) + 255) / 256 * 256;
    const std::size_t w_bytes = static_cast<std::size_t>(E) * S::NH * C * sizeof(float);
    void* ws = nullptr;
    hipError_t err = hipMallocAsync(&ws, off_bytes + w_bytes, hs);
    if (err != hipSuccess) return static_cast<int32_t>(err);
    int* offsets = static_cast<int*>(ws);
    float* W = reinterpret_cast<float*>(static_cast<char*>(ws) + off_bytes);
    k_offsets_from_receivers<<<blocks_for(static_cast<std::int64_t>(N) + 1, 256), 256, 0, hs>>>(
        N, static_cast<int>(E), e->edge_receivers, offsets);
    const auto edges = plugin_edges<S::NY>(*st, e->radial, e->radius, e->harmonics_values, e->harmonics_gradients,
                                           e->xyz, unit, e->node_types, e->neigh_types, e->type_to_active,
                                           e->active_type_count, e->cutoff);
    constexpr unsigned kAll = SourceGroups<LMAX, LMAXH>::masks[0];
    k_r1_reverse<C, LMAX, LMAXH, kAll, true, PluginEdges<S::NY>><<<static_cast<unsigned>(N), C, 0, hs>>>(
        0, 0, offsets, e->neigh_indices, edges, static_cast<const float*>(e->neighbor_features), st->cg,
        static_cast<const float*>(e->output_adjoint), W, e->directed_forces);
    k_source_gather<C, S::NH, true><<<static_cast<unsigned>(N), C, 0, hs>>>(
        s->source_offsets, s->source_edges, W, e->radius, e->cutoff, static_cast<float*>(s->source_adjoint));
    err = hipPeekAtLastError();
    const hipError_t ferr = hipFreeAsync(ws, hs);
    return static_cast<int32_t>(err != hipSuccess ? err : ferr);
}

}  // namespace
}  // namespace smx

extern "C" {

const SymmetrixJitHipPluginV1* symmetrix_jit_hip_plugin_query_v1(void) {
    std::lock_guard<std::mutex> lock(smx::g_mutex);
    return smx::g_active ? &smx::g_active->descriptor : nullptr;
}

int32_t smx_r1_plugin_configure(const char* model_path, const SmxR1PluginIdentity* id) {
    try {
        if (!model_path || !id || id->struct_size < sizeof(SmxR1PluginIdentity))
            throw std::invalid_argument("model path and identity are required");
        if (!id->artifact_id || !id->contract_fingerprint || !*id->artifact_id || !*id->contract_fingerprint)
            throw std::invalid_argument("artifact id and contract fingerprint are required");
        if (id->embedding <= 0 || id->persistent_blocks_per_compute_unit <= 0)
            throw std::invalid_argument("embedding and persistent blocks per compute unit must be positive");
        smx::HostModel hm;
        hm.load(model_path, "");
        auto st = std::make_unique<smx::PluginState>();
        st->C = hm.C;
        st->l_max = hm.l_max;
        st->L_max = hm.L_max;
        st->NY = hm.num_lm;
        st->NH = hm.num_LM;
        st->NLME = hm.num_lme;
        st->functions = hm.num_paths * hm.C;
        st->fp64_point = id->fp64_evaluation_point ? 1 : 0;
        SymmetrixJitHipR1ForwardLaunchV1 fwd = nullptr;
        SymmetrixJitHipR1CoordinateReverseLaunchV1 rev = nullptr;
        std::vector<int> le, ls, lo;
        if (!smx::kernel_paths(hm.l_max, hm.L_max, le, ls, lo) || le != hm.path_le ||
            ls != hm.path_ls || lo != hm.path_lo)
            throw std::domain_error("the model's R1 paths have no compiled kernels");
        if (hm.C == 32 && hm.l_max == 2 && hm.L_max == 1) {
            fwd = &smx::forward_launch<32, 2, 1>;
            rev = &smx::reverse_launch<32, 2, 1>;
        } else if (hm.C == 128 && hm.l_max == 3 && hm.L_max == 1) {
            fwd = &smx::forward_launch<128, 3, 1>;
            rev = &smx::reverse_launch<128, 3, 1>;
        } else {
            throw std::domain_error("no R1 kernels are compiled for " + std::to_string(hm.C) + " channels, l_max " +
                                    std::to_string(hm.l_max) + ", L_max " + std::to_string(hm.L_max));
        }
        const std::vector<float>& cg = hm.cg_dense;
        SMX_HIP(hipMalloc(&st->cg, std::max<std::size_t>(1, cg.size()) * sizeof(float)));
        SMX_HIP(hipMemcpy(st->cg, cg.data(), cg.size() * sizeof(float), hipMemcpyHostToDevice));
        // spline table in the plugin layout [interval][4][function]
        st->intervals = hm.spline_points - 1;
        st->h = hm.h;
        st->x0 = hm.grid_min;
        st->spline.assign(static_cast<std::size_t>(st->intervals) * 4 * st->functions, 0.0f);
        for (int iv = 0; iv < st->intervals; ++iv)
            for (int f = 0; f < st->functions; ++f)
                for (int c = 0; c < 4; ++c)
                    st->spline[(static_cast<std::size_t>(iv) * 4 + c) * st->functions + f] =
                        hm.R1_coef[(static_cast<std::size_t>(iv) * st->functions + f) * 4 + c];
        st->artifact_id = id->artifact_id;
        st->contract = id->contract_fingerprint;
        st->semantic = id->semantic_fingerprint ? id->semantic_fingerprint : "";
        st->structure = id->structure_fingerprint ? id->structure_fingerprint : "";
        st->features = id->target_features ? id->target_features : "";
        SymmetrixJitHipPluginV1& d = st->descriptor;
        std::memset(&d, 0, sizeof(d));
        d.abi_version = SYMMETRIX_JIT_HIP_PLUGIN_ABI_VERSION_V1;
        d.struct_size = sizeof(SymmetrixJitHipPluginV1);
        d.pointer_size = sizeof(void*);
        d.byte_order = SYMMETRIX_JIT_HIP_PLUGIN_BYTE_ORDER;
        d.capabilities = SYMMETRIX_JIT_HIP_R1_FORWARD_LAUNCH_V1 | SYMMETRIX_JIT_HIP_R1_COORDINATE_REVERSE_LAUNCH_V1;
        d.scalar_kind = SYMMETRIX_JIT_HIP_SCALAR_FLOAT32_V1;
        d.scalar_size = sizeof(float);
        d.abi_tag = SYMMETRIX_JIT_HIP_PLUGIN_ABI_TAG_V1;
        d.artifact_id = st->artifact_id.c_str();
        d.contract_fingerprint = st->contract.c_str();
        d.semantic_fingerprint = st->semantic.c_str();
        d.structure_fingerprint = st->structure.c_str();
        d.channels = hm.C;
        d.embedding = id->embedding;
        d.edge_l_max = hm.l_max;
        d.source_l_max = hm.L_max;
        d.target_architecture = st->arch.c_str();
        d.target_features = st->features.c_str();
        d.native_subgroup_width = smx::kWave;
        d.forward_threads_per_block = hm.C;
        d.source_threads_per_block = hm.C;
        d.edge_threads_per_block = hm.C;
        d.persistent_blocks_per_compute_unit = id->persistent_blocks_per_compute_unit;
        d.r1_forward_launch = fwd;
        d.r1_coordinate_reverse_launch = rev;
        st->configured = true;
        std::lock_guard<std::mutex> lock(smx::g_mutex);
        smx::g_states.push_back(std::move(st));
        smx::g_active = smx::g_states.back().get();
        return SMX_OK;
    } catch (const std::bad_alloc&) {
        smx::set_last_error("out of memory (device or host allocation failed)");
        return SMX_ERR_OUT_OF_MEMORY;
    } catch (const std::domain_error& e) {
        smx::set_last_error(e.what());
        return SMX_ERR_UNSUPPORTED;
    } catch (const std::invalid_argument& e) {
        smx::set_last_error(e.what());
        return SMX_ERR_INVALID_ARGUMENT;
    } catch (const std::exception& e) {
        smx::set_last_error(e.what());
        return SMX_ERR_RUNTIME;
    } catch (...) {
        smx::set_last_error("unknown error");
        return SMX_ERR_RUNTIME;
    }
}

int32_t smx_r1_plugin_spline_table(float* out, int64_t capacity, int32_t* intervals, int32_t* functions, double* h,
                                   double* x0) {
    std::lock_guard<std::mutex> lock(smx::g_mutex);
    const smx::PluginState* st = smx::g_active;
    if (!st) {
        smx::set_last_error("the R1 plugin has not been configured");
        return SMX_ERR_LOGIC;
    }
    if (intervals) *intervals = st->intervals;
    if (functions) *functions = st->functions;
    if (h) *h = st->h;
    if (x0) *x0 = st->x0;
    if (out) {
        if (capacity < static_cast<int64_t>(st->spline.size())) return SMX_ERR_INVALID_ARGUMENT;
        std::memcpy(out, st->spline.data(), st->spline.size() * sizeof(float));
    }
    return SMX_OK;
}

}  // extern "C"
