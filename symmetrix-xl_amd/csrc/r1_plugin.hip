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
// Shapes: every (channels, l_max, L_max) the evaluator compiles, with the
// caller's channel count where the kernels pad it (96 on 128 lanes, 224 on
// 256).  A shape whose coupling rows exceed one pass's registers (L_max 2)
// runs one forward and one reverse pass per group of source components, as
// the evaluator does: the forward's first pass assigns Phi1 and the others
// add to it; every reverse pass subtracts its force part and writes its own
// source components of W.
//
// Each configured model owns one launcher slot: the descriptor of a
// configure call holds function pointers instantiated for that slot, so a
// loader that keeps an earlier descriptor keeps launching that model.  A
// configure call with the same model file (same bytes) and the same
// identity returns the existing descriptor instead of taking a new slot.
// Configure is host-only; the coupling table goes to the device at the first
// launch or smx_r1_plugin_reserve.  The reverse workspace belongs to the
// state and only grows (at a launch that needs more, or at
// smx_r1_plugin_reserve); an event orders its reuse across streams.
#include <hip/hip_runtime.h>

#include <atomic>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <tuple>
#include <utility>
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

// A compiled plugin shape: kernel lanes C, l_max, L_max and the caller's
// channel count CF (<= C).
template <int C_, int LMAX_, int LMAXH_, int CF_>
struct PluginShape {
    static constexpr int C = C_, LMAX = LMAX_, LMAXH = LMAXH_, CF = CF_;
    using S = Shape<LMAX, LMAXH>;
    using Groups = SourceGroups<LMAX, LMAXH>;
    using Edges = PluginEdges<S::NY, C, CF>;
    static constexpr int kGroups = static_cast<int>(Groups::masks.size());
};
using PluginShapes = std::tuple<PluginShape<32, 2, 1, 32>, PluginShape<128, 3, 1, 128>, PluginShape<128, 3, 0, 128>,
                                PluginShape<128, 3, 0, 96>, PluginShape<128, 3, 2, 128>, PluginShape<256, 3, 2, 256>,
                                PluginShape<256, 3, 2, 224>>;

// f(PluginShape{}) for the shape (C, l_max, L_max, CF); false if none
template <std::size_t I = 0, class F>
bool with_shape(int C, int l_max, int L_max, int CF, F&& f) {
    if constexpr (I < std::tuple_size_v<PluginShapes>) {
        using PS = std::tuple_element_t<I, PluginShapes>;
        if (PS::C == C && PS::LMAX == l_max && PS::LMAXH == L_max && PS::CF == CF) {
            f(PS{});
            return true;
        }
        return with_shape<I + 1>(C, l_max, L_max, CF, std::forward<F>(f));
    } else {
        return false;
    }
}

struct PluginState {
    SymmetrixJitHipPluginV1 descriptor{};
    // identity: the model file (path and a digest of its bytes) and the
    // caller's identity fields
    std::string path, artifact_id, contract, semantic, structure, features, arch = "gfx950";
    std::uint64_t file_digest = 0;
    int embedding = 0, persistent = 0;
    int C = 0, CF = 0, l_max = 0, L_max = 0, NY = 0, NH = 0, NLME = 0, functions = 0;
    int fp64_point = 0;
    std::vector<float> cg_host;   // dense per-path coupling blocks
    float* cg = nullptr;          // their device copy (first launch or reserve)
    std::mutex dev_mutex;
    std::vector<float> spline;  // [intervals][4][functions], functions = paths * CF
    int intervals = 0;
    double h = 0.0, x0 = 0.0;
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
    bool same_identity(const PluginState& o) const {
        return path == o.path && file_digest == o.file_digest && artifact_id == o.artifact_id &&
               contract == o.contract && semantic == o.semantic && structure == o.structure &&
               features == o.features && embedding == o.embedding && persistent == o.persistent &&
               fp64_point == o.fp64_point;
    }
};

// The coupling table on the device (uploaded once, on the current device).
hipError_t ensure_device_tables(PluginState& st) {
    std::lock_guard<std::mutex> lock(st.dev_mutex);
    if (st.cg) return hipSuccess;
    float* p = nullptr;
    hipError_t e = hipMalloc(&p, std::max<std::size_t>(1, st.cg_host.size()) * sizeof(float));
    if (e != hipSuccess) return e;
    e = hipMemcpy(p, st.cg_host.data(), st.cg_host.size() * sizeof(float), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(p);
        return e;
    }
    st.cg = p;
    return hipSuccess;
}

// FNV-1a digest of a file's bytes
std::uint64_t file_digest(const std::string& path) {
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) throw std::invalid_argument("cannot open model file '" + path + "'");
    std::uint64_t h = 1469598103934665603ull;
    unsigned char buf[1 << 16];
    std::size_t n;
    while ((n = std::fread(buf, 1, sizeof(buf), f)) > 0)
        for (std::size_t i = 0; i < n; ++i) h = (h ^ buf[i]) * 1099511628211ull;
    std::fclose(f);
    return h;
}

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
constexpr int kSlots = 16;
std::vector<std::unique_ptr<PluginState>> g_states;
std::atomic<PluginState*> g_slot[kSlots];
PluginState* g_active = nullptr;  // the query's answer (guarded by g_mutex)

template <class PS>
typename PS::Edges plugin_edges(const PluginState& st, const SymmetrixJitHipRadialSplineV1& radial,
                                const double* radius, const void* harm, const void* grad, const void* xyz, bool unit,
                                const int* node_types, const int* neigh_types, const int* type_to_active,
                                unsigned active_types, double cutoff) {
    typename PS::Edges p;
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

template <class PS, int SLOT>
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
    hipError_t err = ensure_device_tables(*st);
    if (err != hipSuccess) return static_cast<int32_t>(err);
    const auto edges = plugin_edges<PS>(*st, a->radial, a->radius, a->harmonics_values, nullptr, nullptr, false,
                                        a->node_types, a->neigh_types, a->type_to_active, a->active_type_count,
                                        a->cutoff);
    const auto hs = static_cast<hipStream_t>(stream);
    static_for<0, PS::kGroups>([&](auto gc) {
        constexpr int gi = gc;
        if (err != hipSuccess) return;
        k_r1_forward<PS::C, PS::LMAX, PS::LMAXH, PS::Groups::masks[gi], (gi > 0), typename PS::Edges, PS::CF>
            <<<static_cast<unsigned>(a->num_nodes), PS::C, 0, hs>>>(
                0, static_cast<int>(a->num_nodes), a->first_neigh, a->num_neigh, a->neigh_indices, edges,
                static_cast<const float*>(a->neighbor_features), st->cg, static_cast<float*>(a->output));
        err = hipPeekAtLastError();
    });
    return static_cast<int32_t>(err);
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
template <class PS>
hipError_t reverse_kernels(const PluginState& st, const SymmetrixJitHipR1SourceArgsV1* s,
                           const SymmetrixJitHipR1EdgeArgsV1* e, hipStream_t hs, void* ws) {
    const int N = static_cast<int>(s->num_nodes);
    const std::int64_t E = s->num_edges;
    const bool unit = e->coordinates_are_unit != 0;
    int* offsets = static_cast<int*>(ws);
    float* W = reinterpret_cast<float*>(static_cast<char*>(ws) + reverse_offsets_bytes(N));
    k_offsets_from_receivers<<<blocks_for(static_cast<std::int64_t>(N) + 1, 256), 256, 0, hs>>>(
        N, static_cast<int>(E), e->edge_receivers, offsets);
    hipError_t err = hipPeekAtLastError();
    const auto edges = plugin_edges<PS>(st, e->radial, e->radius, e->harmonics_values, e->harmonics_gradients,
                                        e->xyz, unit, e->node_types, e->neigh_types, e->type_to_active,
                                        e->active_type_count, e->cutoff);
    static_for<0, PS::kGroups>([&](auto gc) {
        constexpr int gi = gc;
        if (err != hipSuccess) return;
        k_r1_reverse<PS::C, PS::LMAX, PS::LMAXH, PS::Groups::masks[gi], true, typename PS::Edges, PS::CF>
            <<<static_cast<unsigned>(N), PS::C, 0, hs>>>(0, 0, offsets, e->neigh_indices, edges,
                                                         static_cast<const float*>(e->neighbor_features), st.cg,
                                                         static_cast<const float*>(e->output_adjoint), W,
                                                         e->directed_forces);
        err = hipPeekAtLastError();
    });
    if (err != hipSuccess) return err;
    k_source_gather<PS::C, PS::S::NH, true, PS::CF><<<static_cast<unsigned>(N), PS::C, 0, hs>>>(
        s->source_offsets, s->source_edges, W, e->radius, e->cutoff, static_cast<float*>(s->source_adjoint));
    return hipPeekAtLastError();
}

template <class PS, int SLOT>
int32_t reverse_launch(const SymmetrixJitHipR1SourceArgsV1* s, const SymmetrixJitHipR1EdgeArgsV1* e, void* stream,
                       int32_t persistent_blocks) {
    PluginState* st = g_slot[SLOT].load(std::memory_order_acquire);
    hipError_t err = check_reverse(st, s, e, persistent_blocks);
    if (err != hipSuccess || s->num_nodes == 0 || s->num_edges == 0) return static_cast<int32_t>(err);
    err = ensure_device_tables(*st);
    if (err != hipSuccess) return static_cast<int32_t>(err);
    const auto hs = static_cast<hipStream_t>(stream);
    std::lock_guard<std::mutex> lock(st->ws_mutex);
    err = grow_workspace(*st, reverse_workspace_bytes(*st, s->num_nodes, s->num_edges));
    if (err != hipSuccess) return static_cast<int32_t>(err);
    // a launch on another stream than the workspace's last one waits for it
    if (st->ws_used && st->ws_stream != hs) {
        err = hipStreamWaitEvent(hs, st->ws_done, 0);
        if (err != hipSuccess) return static_cast<int32_t>(err);
    }
    err = reverse_kernels<PS>(*st, s, e, hs, st->ws);
    const hipError_t rec = hipEventRecord(st->ws_done, hs);
    st->ws_stream = hs;
    st->ws_used = true;
    return static_cast<int32_t>(err != hipSuccess ? err : rec);
}

// Launcher pointers of one shape for slot `slot`.
template <class PS, int SLOT = 0>
void slot_launchers(int slot, SymmetrixJitHipR1ForwardLaunchV1& fwd, SymmetrixJitHipR1CoordinateReverseLaunchV1& rev) {
    if constexpr (SLOT < kSlots) {
        if (slot == SLOT) {
            fwd = &forward_launch<PS, SLOT>;
            rev = &reverse_launch<PS, SLOT>;
            return;
        }
        slot_launchers<PS, SLOT + 1>(slot, fwd, rev);
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
    {
        std::lock_guard<std::mutex> lock(st->dev_mutex);
        if (!st->cg) {
            smx::set_last_error("the allocation-free R1 reverse launch needs the model's tables on the device: "
                                "call smx_r1_plugin_reserve (or one launch) with this descriptor first");
            return static_cast<int32_t>(hipErrorNotInitialized);
        }
    }
    void* ws = nullptr;
    err = smx::scratch_address(&ws);
    if (err != hipSuccess) {
        smx::set_last_error(std::string("scratch address: ") + hipGetErrorString(err));
        return static_cast<int32_t>(err);
    }
    const auto hs = static_cast<hipStream_t>(stream);
    err = hipErrorInvalidValue;
    smx::with_shape(st->C, st->l_max, st->L_max, st->CF,
                    [&](auto ps) { err = smx::reverse_kernels<decltype(ps)>(*st, s, e, hs, ws); });
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
        auto st = std::make_unique<smx::PluginState>();
        st->path = model_path;
        st->file_digest = smx::file_digest(st->path);
        st->artifact_id = id->artifact_id;
        st->contract = id->contract_fingerprint;
        st->semantic = id->semantic_fingerprint ? id->semantic_fingerprint : "";
        st->structure = id->structure_fingerprint ? id->structure_fingerprint : "";
        st->features = id->target_features ? id->target_features : "";
        st->embedding = id->embedding;
        st->persistent = id->persistent_blocks_per_compute_unit;
        st->fp64_point = id->fp64_evaluation_point ? 1 : 0;
        std::lock_guard<std::mutex> lock(smx::g_mutex);
        // the same model file and identity: the existing descriptor
        for (const auto& p : smx::g_states)
            if (p->same_identity(*st)) {
                smx::g_active = p.get();
                return SMX_OK;
            }
        const int slot = static_cast<int>(smx::g_states.size());
        if (slot >= smx::kSlots)
            throw std::logic_error("at most " + std::to_string(smx::kSlots) +
                                   " distinct R1 plugin models can be configured in one process");
        smx::HostModel hm;
        hm.load(model_path, "");
        // the evaluator's lane rule: 96 and 224 channels run on 128 and 256
        // lanes (the file's channel count stays the caller's array stride)
        if (hm.C > 32 && hm.C % 64 != 0 && hm.C % 16 == 0) hm.pad_channels((hm.C + 63) / 64 * 64);
        if (hm.single_layer || hm.num_paths == 0)
            throw std::domain_error("a one-interaction model has no R1 operator");
        st->C = hm.C;
        st->CF = hm.C_file;
        st->l_max = hm.l_max;
        st->L_max = hm.L_max;
        st->NY = hm.num_lm;
        st->NH = hm.num_LM;
        st->NLME = hm.num_lme;
        st->functions = hm.num_paths * hm.C_file;
        std::vector<int> le, ls, lo;
        if (!smx::kernel_paths(hm.l_max, hm.L_max, le, ls, lo) || le != hm.path_le ||
            ls != hm.path_ls || lo != hm.path_lo)
            throw std::domain_error("the model's R1 paths have no compiled kernels");
        SymmetrixJitHipR1ForwardLaunchV1 fwd = nullptr;
        SymmetrixJitHipR1CoordinateReverseLaunchV1 rev = nullptr;
        if (!smx::with_shape(hm.C, hm.l_max, hm.L_max, hm.C_file,
                             [&](auto ps) { smx::slot_launchers<decltype(ps)>(slot, fwd, rev); }))
            throw std::domain_error("no R1 kernels are compiled for " + std::to_string(hm.C_file) +
                                    " channels, l_max " + std::to_string(hm.l_max) + ", L_max " +
                                    std::to_string(hm.L_max));
        st->cg_host = hm.cg_dense;
        // spline table in the plugin layout [interval][4][function] over the
        // file's channels (the model's table is padded to C lanes)
        st->intervals = hm.spline_points - 1;
        st->h = hm.h;
        st->x0 = hm.grid_min;
        st->spline.assign(static_cast<std::size_t>(st->intervals) * 4 * st->functions, 0.0f);
        const int padded_functions = hm.num_paths * hm.C;
        for (int iv = 0; iv < st->intervals; ++iv)
            for (int p = 0; p < hm.num_paths; ++p)
                for (int k = 0; k < hm.C_file; ++k)
                    for (int c = 0; c < 4; ++c)
                        st->spline[(static_cast<std::size_t>(iv) * 4 + c) * st->functions + p * hm.C_file + k] =
                            hm.R1_coef[(static_cast<std::size_t>(iv) * padded_functions + p * hm.C + k) * 4 + c];
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
        d.channels = hm.C_file;
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
    hipError_t e = smx::ensure_device_tables(*st);
    if (e == hipSuccess) {
        std::lock_guard<std::mutex> lock(st->ws_mutex);
        e = smx::grow_workspace(*st, smx::reverse_workspace_bytes(*st, num_nodes, num_edges));
    }
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
