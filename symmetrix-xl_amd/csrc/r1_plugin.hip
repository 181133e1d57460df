// The reference's R1 HIP plugin ABI (jit_hip_plugin_abi.h) on the MI355X
// edge kernels: symmetrix_jit_hip_plugin_query_v1 and its two launchers.
//
// The launchers validate their packets as the reference's generated ones do
// (jit_codegen.py:3346-3410) and enqueue on the caller's stream:
//   forward  -> k_r1_forward over the caller's receiver CSR (first_neigh,
//               num_neigh), output assigned;
//   reverse  -> receiver offsets from edge_receivers (binary search),
//               k_r1_reverse (directed forces subtracted, per-edge source
//               terms W into the state's workspace), then k_source_gather
//               adding the FP64 source sums to source_adjoint over the
//               caller's source transpose.
//
// Each configured model owns one launcher slot: the descriptor of a
// configure call holds function pointers instantiated for that slot, so a
// loader that keeps an earlier descriptor keeps launching that model.  The
// reverse workspace belongs to the state and only grows (at a launch that
// needs more, or at smx_r1_plugin_reserve); an event orders its reuse
// across streams.
#include <hip/hip_runtime.h>

#include <atomic>
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
    // reverse workspace: receiver offsets and per-edge source terms W
    std::mutex ws_mutex;
    void* ws = nullptr;
    std::size_t ws_bytes = 0;
    hipEvent_t ws_done = nullptr;  // recorded after the last launch that used ws
    hipStream_t ws_stream = nullptr;
    bool ws_used = false;
    ~PluginState() {
        if (ws_done) (void)hipEventSynchronize(ws_done);
        if (ws) (void)hipFree(ws);
        if (ws_done) (void)hipEventDestroy(ws_done);
        if (cg) (void)hipFree(cg);
    }
};

// Bytes of the reverse workspace for a graph: receiver offsets [N+1] padded
// to 256 B, then W [E][NH][C] floats.
std::size_t reverse_offsets_bytes(std::int64_t N) {
    return ((static_cast<std::size_t>(N) + 1) * sizeof(int) + 255) / 256 * 256;
}
std::size_t reverse_workspace_bytes(const PluginState& st, std::int64_t N, std::int64_t E) {
    return reverse_offsets_bytes(N) + static_cast<std::size_t>(E) * st.NH * st.C * sizeof(float);
}

// Grow the state's workspace to at least `bytes` (caller holds ws_mutex):
// the previous buffer is freed once its last launch has finished.
hipError_t grow_workspace(PluginState& st, std::size_t bytes) {
    if (bytes <= st.ws_bytes) return hipSuccess;
    if (!st.ws_done) {
        const hipError_t e = hipEventCreateWithFlags(&st.ws_done, hipEventDisableTiming);
        if (e != hipSuccess) return e;
    }
    if (st.ws) {
        if (st.ws_used) {
            const hipError_t e = hipEventSynchronize(st.ws_done);
            if (e != hipSuccess) return e;
        }
        (void)hipFree(st.ws);
        st.ws = nullptr;
        st.ws_bytes = 0;
    }
    const hipError_t e = hipMalloc(&st.ws, bytes);
    if (e != hipSuccess) {
        st.ws = nullptr;
        return e;
    }
    st.ws_bytes = bytes;
    st.ws_used = false;
    return hipSuccess;
}

std::mutex g_mutex;
// configured states, each bound to one launcher slot; they stay alive because
// a loader may still hold their descriptor
constexpr int kSlots = 8;
std::vector<std::unique_ptr<PluginState>> g_states;
std::atomic<PluginState*> g_slot[kSlots];
PluginState* g_active = nullptr;  // the query's answer (guarded by g_mutex)

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

template <int C, int LMAX, int LMAXH, int SLOT>
int32_t forward_launch(const SymmetrixJitHipR1ForwardArgsV1* a, void* stream, int32_t persistent_blocks) {
    PluginState* st = g_slot[SLOT].load(std::memory_order_acquire);
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
        0, a->num_nodes, a->first_neigh, a->num_neigh, a->neigh_indices, edges,
        static_cast<const float*>(a->neighbor_features),
        st->cg, static_cast<float*>(a->output));
    return static_cast<int32_t>(hipPeekAtLastError());
}

// Checks of the reverse packets (jit_codegen.py:3346-3410); hipSuccess when
// the launch may proceed.
hipError_t check_reverse(const PluginState* st, const SymmetrixJitHipR1SourceArgsV1* s,
                         const SymmetrixJitHipR1EdgeArgsV1* e, int32_t persistent_blocks) {
    if (!st || !s || !e || s->struct_size < sizeof(SymmetrixJitHipR1SourceArgsV1) ||
        e->struct_size < sizeof(SymmetrixJitHipR1EdgeArgsV1) || s->num_nodes < 0 || s->num_nodes > INT32_MAX ||
        s->num_edges < 0 || s->num_edges > INT32_MAX || s->num_edges != e->num_edges ||
        s->num_nodes != e->num_nodes || s->active_type_count != e->active_type_count || s->cutoff != e->cutoff ||
        !std::isfinite(s->cutoff) || s->cutoff <= 0.0 || s->active_type_count == 0 || persistent_blocks <= 0 ||
        !radial_ok(*st, s->radial, s->active_type_count) || !radial_ok(*st, e->radial, e->active_type_count))
        return hipErrorInvalidValue;
    if (s->num_nodes == 0 || s->num_edges == 0) return hipSuccess;
    const bool unit = e->coordinates_are_unit != 0;
    if (!e->node_types || !e->neigh_indices || !e->neigh_types || !e->edge_receivers || !e->type_to_active ||
        !e->xyz || !e->radius || !e->harmonics_values || !e->harmonics_gradients || !e->neighbor_features ||
        !e->output_adjoint || !e->directed_forces || !s->source_offsets || !s->source_edges ||
        !s->source_adjoint || e->coordinate_scalar_size != (unit ? sizeof(float) : sizeof(double)))
        return hipErrorInvalidValue;
    return hipSuccess;
}

// The reverse kernels over a workspace of reverse_workspace_bytes(N, E):
// receiver offsets, then W.
template <int C, int LMAX, int LMAXH>
hipError_t reverse_kernels(const PluginState& st, const SymmetrixJitHipR1SourceArgsV1* s,
                           const SymmetrixJitHipR1EdgeArgsV1* e, hipStream_t hs, void* ws) {
    using S = Shape<LMAX, LMAXH>;
    const int N = static_cast<int>(s->num_nodes);
    const std::int64_t E = s->num_edges;
    const bool unit = e->coordinates_are_unit != 0;
    int* offsets = static_cast<int*>(ws);
    float* W = reinterpret_cast<float*>(static_cast<char*>(ws) + reverse_offsets_bytes(N));
    k_offsets_from_receivers<<<blocks_for(static_cast<std::int64_t>(N) + 1, 256), 256, 0, hs>>>(
        N, static_cast<int>(E), e->edge_receivers, offsets);
    const auto edges = plugin_edges<S::NY>(st, e->radial, e->radius, e->harmonics_values, e->harmonics_gradients,
                                           e->xyz, unit, e->node_types, e->neigh_types, e->type_to_active,
                                           e->active_type_count, e->cutoff);
    constexpr unsigned kAll = SourceGroups<LMAX, LMAXH>::masks[0];
    k_r1_reverse<C, LMAX, LMAXH, kAll, true, PluginEdges<S::NY>><<<static_cast<unsigned>(N), C, 0, hs>>>(
        0, 0, offsets, e->neigh_indices, edges, static_cast<const float*>(e->neighbor_features), st.cg,
        static_cast<const float*>(e->output_adjoint), W, e->directed_forces);
    k_source_gather<C, S::NH, true><<<static_cast<unsigned>(N), C, 0, hs>>>(
        s->source_offsets, s->source_edges, W, e->radius, e->cutoff, static_cast<float*>(s->source_adjoint));
    return hipPeekAtLastError();
}

template <int C, int LMAX, int LMAXH, int SLOT>
int32_t reverse_launch(const SymmetrixJitHipR1SourceArgsV1* s, const SymmetrixJitHipR1EdgeArgsV1* e, void* stream,
                       int32_t persistent_blocks) {
    PluginState* st = g_slot[SLOT].load(std::memory_order_acquire);
    hipError_t err = check_reverse(st, s, e, persistent_blocks);
    if (err != hipSuccess || s->num_nodes == 0 || s->num_edges == 0) return static_cast<int32_t>(err);
    const auto hs = static_cast<hipStream_t>(stream);
    std::lock_guard<std::mutex> lock(st->ws_mutex);
    err = grow_workspace(*st, reverse_workspace_bytes(*st, s->num_nodes, s->num_edges));
    if (err != hipSuccess) return static_cast<int32_t>(err);
    // a launch on another stream than the workspace's last one waits for it
    if (st->ws_used && st->ws_stream != hs) {
        err = hipStreamWaitEvent(hs, st->ws_done, 0);
        if (err != hipSuccess) return static_cast<int32_t>(err);
    }
    err = reverse_kernels<C, LMAX, LMAXH>(*st, s, e, hs, st->ws);
    const hipError_t rec = hipEventRecord(st->ws_done, hs);
    st->ws_stream = hs;
    st->ws_used = true;
    return static_cast<int32_t>(err != hipSuccess ? err : rec);
}

// Launcher pointers of one shape for slot `slot`.
template <int C, int LMAX, int LMAXH, int SLOT = 0>
bool slot_launchers(int slot, SymmetrixJitHipR1ForwardLaunchV1& fwd, SymmetrixJitHipR1CoordinateReverseLaunchV1& rev) {
    if constexpr (SLOT < kSlots) {
        if (slot == SLOT) {
            fwd = &forward_launch<C, LMAX, LMAXH, SLOT>;
            rev = &reverse_launch<C, LMAX, LMAXH, SLOT>;
            return true;
        }
        return slot_launchers<C, LMAX, LMAXH, SLOT + 1>(slot, fwd, rev);
    } else {
        return false;
    }
}

// ---------------------------------------------------------------------------
// Allocation-free reverse launch: the workspace (receiver offsets and W) lives
// in a fixed device array, one per GPU, held until the process ends.  Host
// code uses the address hipGetSymbolAddress reports for the current device,
// never the array's name.
// ---------------------------------------------------------------------------
constexpr std::size_t kScratchBytes = std::size_t(256) << 20;  // 256 MiB
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// The scratch address on the current device (looked up once per device).
hipError_t scratch_address(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return hipSuccess;
}

PluginState* state_of(const SymmetrixJitHipPluginV1* plugin) {
    std::lock_guard<std::mutex> lock(g_mutex);
    for (const auto& p : g_states)
        if (&p->descriptor == plugin) return p.get();
    return nullptr;
}

}  // namespace
}  // namespace smx

extern "C" {

int32_t smx_r1_plugin_reverse_launch_noalloc(const SymmetrixJitHipPluginV1* plugin,
                                             const SymmetrixJitHipR1SourceArgsV1* s,
                                             const SymmetrixJitHipR1EdgeArgsV1* e, void* stream,
                                             int32_t persistent_blocks) {
    smx::PluginState* st = smx::state_of(plugin);
    if (!st) {
        smx::set_last_error("the descriptor was not returned by this library's R1 plugin query");
        return static_cast<int32_t>(hipErrorInvalidValue);
    }
    hipError_t err = smx::check_reverse(st, s, e, persistent_blocks);
    if (err != hipSuccess) {
        smx::set_last_error("malformed R1 reverse packets");
        return static_cast<int32_t>(err);
    }
    if (s->num_nodes == 0 || s->num_edges == 0) return static_cast<int32_t>(hipSuccess);
    const std::size_t need = smx::reverse_workspace_bytes(*st, s->num_nodes, s->num_edges);
    if (need > smx::kScratchBytes) {
        smx::set_last_error("the allocation-free R1 reverse launch needs " + std::to_string(need) +
                            " bytes of workspace for " + std::to_string(s->num_nodes) + " nodes and " +
                            std::to_string(s->num_edges) + " edges; its fixed scratch holds " +
                            std::to_string(smx::kScratchBytes) + " bytes (" +
                            std::to_string(st->NH * st->C * sizeof(float)) + " bytes per edge at this shape)");
        return static_cast<int32_t>(hipErrorInvalidValue);
    }
    void* ws = nullptr;
    err = smx::scratch_address(&ws);
    if (err != hipSuccess) {
        smx::set_last_error(std::string("scratch address: ") + hipGetErrorString(err));
        return static_cast<int32_t>(err);
    }
    const auto hs = static_cast<hipStream_t>(stream);
    if (st->C == 32 && st->l_max == 2 && st->L_max == 1)
        err = smx::reverse_kernels<32, 2, 1>(*st, s, e, hs, ws);
    else if (st->C == 128 && st->l_max == 3 && st->L_max == 1)
        err = smx::reverse_kernels<128, 3, 1>(*st, s, e, hs, ws);
    else
        err = hipErrorInvalidValue;
    return static_cast<int32_t>(err);
}


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
        std::lock_guard<std::mutex> lock(smx::g_mutex);
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
        const int slot = static_cast<int>(smx::g_states.size());
        if (slot >= smx::kSlots)
            throw std::logic_error("at most " + std::to_string(smx::kSlots) +
                                   " R1 plugin models can be configured in one process");
        if (hm.C == 32 && hm.l_max == 2 && hm.L_max == 1) {
            smx::slot_launchers<32, 2, 1>(slot, fwd, rev);
        } else if (hm.C == 128 && hm.l_max == 3 && hm.L_max == 1) {
            smx::slot_launchers<128, 3, 1>(slot, fwd, rev);
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
        smx::g_states.push_back(std::move(st));
        smx::g_active = smx::g_states.back().get();
        smx::g_slot[slot].store(smx::g_active, std::memory_order_release);
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
    } catch (const std::logic_error& e) {
        smx::set_last_error(e.what());
        return SMX_ERR_LOGIC;
    } catch (const std::exception& e) {
        smx::set_last_error(e.what());
        return SMX_ERR_RUNTIME;
    } catch (...) {
        smx::set_last_error("unknown error");
        return SMX_ERR_RUNTIME;
    }
}

int32_t smx_r1_plugin_reserve(const SymmetrixJitHipPluginV1* plugin, int64_t num_nodes, int64_t num_edges) {
    smx::PluginState* st = smx::state_of(plugin);
    if (!st) {
        smx::set_last_error("the descriptor was not returned by this library's R1 plugin query");
        return SMX_ERR_INVALID_ARGUMENT;
    }
    if (num_nodes < 0 || num_nodes > INT32_MAX || num_edges < 0 || num_edges > INT32_MAX) {
        smx::set_last_error("node and edge counts must lie in [0, 2^31)");
        return SMX_ERR_INVALID_ARGUMENT;
    }
    std::lock_guard<std::mutex> lock(st->ws_mutex);
    const hipError_t e = smx::grow_workspace(*st, smx::reverse_workspace_bytes(*st, num_nodes, num_edges));
    if (e != hipSuccess) {
        smx::set_last_error(std::string("R1 plugin workspace: ") + hipGetErrorString(e));
        return e == hipErrorOutOfMemory ? SMX_ERR_OUT_OF_MEMORY : SMX_ERR_RUNTIME;
    }
    return SMX_OK;
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
