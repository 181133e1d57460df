// Streamed-edge R1 kernels (gfx950, wave64), shared by the evaluator and the
// reference-compatible R1 plugin entry points.
//
// Mapping: one workgroup owns one receiver; lanes are channels, so per-channel
// data (spline coefficients, H1 rows, coupling adjoints) is read coalesced and
// the per-edge quantities (evaluation point, Y, dY, direction) are
// wave-uniform.  Receivers are owned, never shared: every receiver quantity is
// a deterministic segment sum without atomics.
//
// The kernels read their per-edge inputs through a policy:
//  * RecordEdges: this build's packed per-edge records and float4 spline table
//    (the evaluator's own layout);
//  * PluginEdges: the separate arrays of the reference's plugin argument
//    packets (radius, harmonics, harmonic gradients, coordinates, spline
//    coefficients [edge type][interval][4][function], type maps;
//    jit_hip_plugin_abi.h:37-222), with the reference's evaluation point and
//    radial formulas (jit_codegen.py:2380-2496).
//
// Reference math: R1 forward mace.cpp:2023-2084 (h1_phi1.cpp:1385-1845),
// R1 reverse mace.cpp:2199-2303 (factorized_execution.cpp:471-1460).
#pragma once

#include <hip/hip_runtime.h>

#include <array>
#include <cstdint>

#include "device_common.hpp"
#include "coupling_rows.hpp"
#include "shapes.hpp"

namespace smx {
namespace edge {
namespace {

__device__ __forceinline__ float spline_value(float4 c, float x, float xx, float xxx) {
    return c.x + c.y * x + c.z * xx + c.w * xxx;
}
// slope c1 + 2 c2 x + 3 c3 x^2 with the edge's factors x2 = 2x (exact) and
// xx3 = 3x^2 formed once per edge
__device__ __forceinline__ float spline_slope(float4 c, float x2, float xx3) { return c.y + c.z * x2 + c.w * xx3; }
__device__ __forceinline__ bool edge_active(const float* rec) { return __float_as_int(rec[2]) != 0; }

template <int C>
struct Lanes {
    static constexpr int NW = (C + kWave - 1) / kWave;
    static constexpr int WIDTH = C < kWave ? C : kWave;
};

// ---------------------------------------------------------------------------
// Receiver records staged through LDS.  A receiver's edge records are
// contiguous; they are copied in chunks of kRecordChunk edges with coalesced
// float4 loads into one of two LDS buffers, the next chunk's loads in flight
// while the current chunk is processed, so the wave-uniform record fields
// come from LDS (broadcast reads) rather than from scalar loads that miss.
//   for (c = 0; c < chunks(); ++c) { const float* r = begin(c); ... end(c); }
// begin/end synchronise the workgroup; every thread must run the loop.
// ---------------------------------------------------------------------------
constexpr int kRecordChunk = 16;

// native 4-float vector: copies are plain vector loads and stores (float4,
// a struct, copies through memcpy and keeps the staging array in scratch)
typedef float stage4 __attribute__((ext_vector_type(4)));

constexpr int stage_per(int C, int REC) { return (kRecordChunk * (REC / 4) + C - 1) / C; }

template <int C, int REC>
struct RecordStage {
    static constexpr int R4 = REC / 4;               // float4 per record
    static constexpr int SLOTS = kRecordChunk * R4;  // float4 per buffer
    static constexpr int PER = (SLOTS + C - 1) / C;  // float4 per thread
};

// Loads of chunk c into held (unconditional: past the chunk they repeat its
// last float4, so there is no branch and they stay in flight while the
// current chunk runs).
template <int C, int REC>
__device__ __forceinline__ void stage_fetch(stage4 (&held)[stage_per(C, REC)], const stage4* __restrict__ src,
                                            int c, int edges) {
    using RS = RecordStage<C, REC>;
    const int limit = min(kRecordChunk, edges - c * kRecordChunk) * RS::R4;
#pragma unroll
    for (int p = 0; p < RS::PER; ++p) {
        const int idx = min(static_cast<int>(threadIdx.x) + p * C, limit - 1);
        held[p] = src[static_cast<std::size_t>(c) * RS::SLOTS + idx];
    }
}

template <int C, int REC>
__device__ __forceinline__ void stage_commit(const stage4 (&held)[stage_per(C, REC)], stage4* buf, int c,
                                             int edges) {
    using RS = RecordStage<C, REC>;
    const int limit = min(kRecordChunk, edges - c * kRecordChunk) * RS::R4;
#pragma unroll
    for (int p = 0; p < RS::PER; ++p) {
        const int idx = static_cast<int>(threadIdx.x) + p * C;
        if (idx < limit) buf[(c & 1) * RS::SLOTS + idx] = held[p];
    }
}

// Two-part records: the forward part (RF floats per edge at srcF) and the
// reverse part (RB floats per edge at srcB) of chunk c, laid out in LDS as
// records of RF + RB floats.
template <int C, int RF, int RB>
__device__ __forceinline__ void stage_fetch2(stage4 (&held)[stage_per(C, RF + RB)], const stage4* __restrict__ srcF,
                                             const stage4* __restrict__ srcB, int c, int edges) {
    using RS = RecordStage<C, RF + RB>;
    constexpr int F4 = RF / 4, B4 = RB / 4;
    const int limit = min(kRecordChunk, edges - c * kRecordChunk) * RS::R4;
#pragma unroll
    for (int p = 0; p < RS::PER; ++p) {
        const int idx = min(static_cast<int>(threadIdx.x) + p * C, limit - 1);
        const int j = c * kRecordChunk + idx / RS::R4, q = idx % RS::R4;
        held[p] = q < F4 ? srcF[static_cast<std::size_t>(j) * F4 + q] : srcB[static_cast<std::size_t>(j) * B4 + q - F4];
    }
}

template <int C, int RF, int RB, class BODY>
__device__ __forceinline__ void staged_records2(stage4* buf, const stage4* __restrict__ srcF,
                                                const stage4* __restrict__ srcB, int edges, BODY&& body) {
    constexpr int REC = RF + RB;
    using RS = RecordStage<C, REC>;
    const int chunks = (edges + kRecordChunk - 1) / kRecordChunk;
    stage4 held[RS::PER];
    if (chunks > 0) {
        stage_fetch2<C, RF, RB>(held, srcF, srcB, 0, edges);
        stage_commit<C, REC>(held, buf, 0, edges);
    }
    __syncthreads();
    for (int c = 0; c < chunks; ++c) {
        if (c + 1 < chunks) stage_fetch2<C, RF, RB>(held, srcF, srcB, c + 1, edges);
        body(reinterpret_cast<const float*>(buf + (c & 1) * RS::SLOTS), c * kRecordChunk,
             min(kRecordChunk, edges - c * kRecordChunk));
        if (c + 1 < chunks) stage_commit<C, REC>(held, buf, c + 1, edges);
        __syncthreads();
    }
}

// Runs body(chunk_records, first_edge_offset, count) over the chunks of
// `edges` records at src (records contiguous), staged through two LDS
// buffers of SLOTS float4 each at buf.
template <int C, int REC, class BODY>
__device__ __forceinline__ void staged_records(stage4* buf, const stage4* __restrict__ src, int edges, BODY&& body) {
    using RS = RecordStage<C, REC>;
    const int chunks = (edges + kRecordChunk - 1) / kRecordChunk;
    stage4 held[RS::PER];
    if (chunks > 0) {
        stage_fetch<C, REC>(held, src, 0, edges);
        stage_commit<C, REC>(held, buf, 0, edges);
    }
    __syncthreads();
    for (int c = 0; c < chunks; ++c) {
        if (c + 1 < chunks) stage_fetch<C, REC>(held, src, c + 1, edges);
        body(reinterpret_cast<const float*>(buf + (c & 1) * RS::SLOTS), c * kRecordChunk,
             min(kRecordChunk, edges - c * kRecordChunk));
        if (c + 1 < chunks) stage_commit<C, REC>(held, buf, c + 1, edges);
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Edge-input policies
// ---------------------------------------------------------------------------
// Packed records in two parts per execution slot (tile-local slot e - e0):
// forward [x, table row, source type + 1 (0: inactive), source node, Y[NY]]
// (RF floats) and reverse [dY/dX[NY], dY/dY[NY], dY/dZ[NY], u[3], edge row]
// (RB floats); the Hermite table [row][function] as float4 (c0..c3).  The
// slots of a receiver hold its edges in execution order (by table row), so
// consecutive edges often share a row and the kernels keep its coefficients
// in registers (kReuse); per-edge outputs (directed forces, source terms W)
// go to the edge's own row in the caller's order (the reverse part's last
// field, tile-local).  With STAGED a receiver's records (both parts) are
// staged through LDS in chunks (staged_records2; the fields then sit in
// VGPRs), else the wave reads the forward part with scalar loads (SGPRs) --
// the forward kernels need nothing else.
template <int C, int NY, int RF, int RB, bool STAGED>
struct RecordEdges {
    const float* __restrict__ erec;    // forward parts [ne][RF]
    const float* __restrict__ erec_b;  // reverse parts [ne][RB]
    long long e0;
    const float4* __restrict__ coef;
    int functions;

    static constexpr int REC = STAGED ? RF + RB : RF;  // record stride where the kernel reads it
    static constexpr int kStageSlots = STAGED ? RecordStage<C, RF + RB>::SLOTS : 1;
    static constexpr int kEdgeRow = RF + RB - 1;       // caller row field (staged records)
    static constexpr bool kReuse = true;               // table rows shared by consecutive slots
    // The unstaged records can be read one edge ahead (hold): the fields a
    // forward pass needs, wave-uniform, so they sit in SGPRs.
    static constexpr bool kHold = !STAGED;
    struct Held {
        float x;
        int iv, active, src;
        float y[NY];
    };
    __device__ __forceinline__ void hold(int e, Held& h) const {
        const float* r = erec + static_cast<std::size_t>(e - e0) * RF;
        h.x = r[0];
        h.iv = __float_as_int(r[1]);
        h.active = __float_as_int(r[2]);
        h.src = __float_as_int(r[3]);
#pragma unroll
        for (int lm = 0; lm < NY; ++lm) h.y[lm] = r[4 + lm];
    }
    struct Point {
        const float* rec;
        const float4* cf;
        float x, xx, xxx, x2, xx3;
    };
    __device__ __forceinline__ int row(const Point& p) const { return __float_as_int(p.rec[1]); }
    __device__ __forceinline__ float4 coef_at(const Point& p, int f) const { return p.cf[f]; }
    __device__ __forceinline__ int source(const Point& p, int /*e*/, const int* /*neigh*/) const {
        return __float_as_int(p.rec[3]);
    }
    // tile-local row of the per-edge outputs of slot j of a staged chunk
    __device__ __forceinline__ long long out_row(const float* chunk, int j, long long /*slot*/) const {
        static_assert(STAGED, "the caller row is read from staged records");
        return __float_as_int(chunk[j * REC + kEdgeRow]);
    }
    // body(first edge, count, staged records of the chunk) over [ea, eb)
    template <class BODY>
    __device__ __forceinline__ void chunks(int ea, int eb, stage4* lds, BODY&& body) const {
        if constexpr (STAGED) {
            const std::size_t first = static_cast<std::size_t>(ea - e0);
            const stage4* srcF = reinterpret_cast<const stage4*>(erec) + first * (RF / 4);
            const stage4* srcB = reinterpret_cast<const stage4*>(erec_b) + first * (RB / 4);
            staged_records2<C, RF, RB>(lds, srcF, srcB, eb - ea, [&](const float* chunk, int f, int n)
                                                                     __attribute__((always_inline)) {
                body(ea + f, n, chunk);
            });
        } else {
            for (int c0 = ea; c0 < eb; c0 += kRecordChunk) body(c0, min(kRecordChunk, eb - c0), nullptr);
        }
    }
    __device__ __forceinline__ bool open_at(int e, int /*receiver*/, const float* chunk, int j, Point& p) const {
        p.rec = STAGED ? chunk + j * REC : erec + static_cast<std::size_t>(e - e0) * RF;
        if (!edge_active(p.rec)) return false;
        p.x = p.rec[0];
        p.xx = p.x * p.x;
        p.xxx = p.xx * p.x;
        p.x2 = 2.0f * p.x;
        p.xx3 = 3.0f * p.xx;
        p.cf = coef + static_cast<std::size_t>(__float_as_int(p.rec[1])) * functions;
        return true;
    }
    __device__ __forceinline__ float Y(const Point& p, int lm) const { return p.rec[4 + lm]; }
    // reverse fields: staged records only
    __device__ __forceinline__ float dY(const Point& p, int c, int lm) const {
        static_assert(STAGED, "the reverse fields are read from staged records");
        return p.rec[RF + c * NY + lm];
    }
    __device__ __forceinline__ float u(const Point& p, int c) const {
        static_assert(STAGED, "the reverse fields are read from staged records");
        return p.rec[RF + 3 * NY + c];
    }
    __device__ __forceinline__ float value(const Point& p, int f) const {
        return spline_value(p.cf[f], p.x, p.xx, p.xxx);
    }
    __device__ __forceinline__ void value_slope(const Point& p, int f, float& R, float& dR) const {
        const float4 c = p.cf[f];
        R = spline_value(c, p.x, p.xx, p.xxx);
        dR = spline_slope(c, p.x2, p.xx3);
    }
};

// Symmetric pair index over active types (jit_codegen.py:2490-2496).
__device__ __forceinline__ int pair_type(int a, int b, int n) {
    return a <= b ? a * (2 * n - a - 1) / 2 + b : b * (2 * n - b - 1) / 2 + a;
}

// The reference plugin's per-edge arrays.  Activity is radius < cutoff; the
// evaluation point is formed in FP32 from the rounded radius (fp64_point 0,
// the precision-matched form) or in FP64 and rounded (fp64_point 1); the
// slope uses the factors (2x) and (3xx) formed before the multiply
// (jit_codegen.py:2387-2485).  C is the kernel's lane count and CF the
// caller's channel count (CF < C for a model whose channels the kernels pad:
// functions are then p * CF + k and lanes k >= CF read zero coefficients).
template <int NY, int C, int CF = C>
struct PluginEdges {
    const double* __restrict__ radius;
    const float* __restrict__ harm;    // [E][NY]
    const float* __restrict__ grad;    // [E][3][NY]
    const double* __restrict__ xyz64;  // [E][3] (coordinates_are_unit == 0)
    const float* __restrict__ unit32;  // [E][3] (coordinates_are_unit != 0)
    const float* __restrict__ coef;    // [edge type][interval][4][function]
    const int* __restrict__ node_types;
    const int* __restrict__ neigh_types;
    const int* __restrict__ type_to_active;
    double x0, h, cutoff;
    int intervals, functions, active_types, fp64_point;

    static constexpr int kStageSlots = 1;
    static constexpr bool kHold = false;
    static constexpr bool kReuse = false;
    struct Point {
        int e;
        const float* c0;  // coefficient c0 of function 0 of this edge's interval
        float x, xx, xxx, x2, xx3;
    };
    __device__ __forceinline__ int row(const Point&) const { return 0; }
    __device__ __forceinline__ float4 coef_at(const Point&, int) const { return float4{}; }
    __device__ __forceinline__ int source(const Point&, int e, const int* neigh) const { return neigh[e]; }
    // the caller's arrays are in edge order: slot e writes row e
    __device__ __forceinline__ long long out_row(const float*, int, long long slot) const { return slot; }
    template <class BODY>
    __device__ __forceinline__ void chunks(int ea, int eb, stage4*, BODY&& body) const {
        for (int c0 = ea; c0 < eb; c0 += kRecordChunk) body(c0, min(kRecordChunk, eb - c0), nullptr);
    }
    __device__ __forceinline__ bool open_at(int e, int receiver, const float*, int, Point& p) const {
        return open(e, receiver, p);
    }
    __device__ __forceinline__ bool open(int e, int receiver, Point& p) const {
        const double r = radius[e];
        if (!(r < cutoff)) return false;
        int iv;
        if (fp64_point) {
            iv = static_cast<int>(floor((r - x0) / h));
            double x = r - x0 - h * iv;
            if (iv < 0) {
                iv = 0;
                x = 0.0;
            } else if (iv >= intervals) {
                iv = intervals - 1;
                x = h;
            }
            const double xx = x * x;
            p.x = static_cast<float>(x);
            p.xx = static_cast<float>(xx);
            p.xxx = static_cast<float>(xx * x);
            p.x2 = static_cast<float>(2.0 * x);
            p.xx3 = static_cast<float>(3.0 * xx);
        } else {
            const float rf = static_cast<float>(r), x0f = static_cast<float>(x0), hf = static_cast<float>(h);
            iv = static_cast<int>(floorf((rf - x0f) / hf));
            float x = rf - x0f - hf * static_cast<float>(iv);
            if (iv < 0) {
                iv = 0;
                x = 0.0f;
            } else if (iv >= intervals) {
                iv = intervals - 1;
                x = hf;
            }
            p.x = x;
            p.xx = x * x;
            p.xxx = p.xx * x;
            p.x2 = static_cast<float>(2.0 * static_cast<double>(x));
            p.xx3 = static_cast<float>(3.0 * static_cast<double>(p.xx));
        }
        const int t = pair_type(type_to_active[node_types[receiver]], type_to_active[neigh_types[e]], active_types);
        p.c0 = coef + (static_cast<std::size_t>(t) * intervals + iv) * 4 * functions;
        p.e = e;
        return true;
    }
    __device__ __forceinline__ float Y(const Point& p, int lm) const {
        return harm[static_cast<std::size_t>(p.e) * NY + lm];
    }
    __device__ __forceinline__ float dY(const Point& p, int c, int lm) const {
        return grad[(static_cast<std::size_t>(p.e) * 3 + c) * NY + lm];
    }
    __device__ __forceinline__ float u(const Point& p, int c) const {
        return unit32 ? unit32[3 * static_cast<std::size_t>(p.e) + c]
                      : static_cast<float>(xyz64[3 * static_cast<std::size_t>(p.e) + c] / radius[p.e]);
    }
    // the caller's function index of kernel function f = p * C + k, or -1
    // for a padding lane
    __device__ __forceinline__ static int caller_function(int f) {
        if constexpr (CF == C) {
            return f;
        } else {
            const int p = f / C, k = f - p * C;
            return k < CF ? p * CF + k : -1;
        }
    }
    __device__ __forceinline__ float value(const Point& p, int f) const {
        f = caller_function(f);
        if (CF != C && f < 0) return 0.0f;
        const float c0 = p.c0[f], c1 = p.c0[functions + f], c2 = p.c0[2 * functions + f],
                    c3 = p.c0[3 * functions + f];
        return c0 + c1 * p.x + c2 * p.xx + c3 * p.xxx;
    }
    __device__ __forceinline__ void value_slope(const Point& p, int f, float& R, float& dR) const {
        f = caller_function(f);
        if (CF != C && f < 0) {
            R = dR = 0.0f;
            return;
        }
        const float c0 = p.c0[f], c1 = p.c0[functions + f], c2 = p.c0[2 * functions + f],
                    c3 = p.c0[3 * functions + f];
        R = c0 + c1 * p.x + c2 * p.xx + c3 * p.xxx;
        dR = c1 + c2 * p.x2 + c3 * p.xx3;
    }
};

// ---------------------------------------------------------------------------
// Per-edge directed forces: per-lane partials (fx,fy,fz) are summed over the
// channels of the workgroup.  Each row of 16 lanes is reduced with DPP and
// its sum parked in LDS; chunks of edges are finalised together, summing the
// row partials of every wave.
// ---------------------------------------------------------------------------
template <int C, int CHUNK>
struct EdgeForceSink {
    static constexpr int ROWS = (C + 15) / 16;  // 16-lane rows of the workgroup
    float (*part)[CHUNK][3];                    // [ROWS][CHUNK][3]
    __device__ __forceinline__ void put(int slot, float fx, float fy, float fz) {
        fx = row_total(fx);
        fy = row_total(fy);
        fz = row_total(fz);
        if (threadIdx.x % 16 == 0) {
            const int r = threadIdx.x / 16;
            part[r][slot][0] = fx;
            part[r][slot][1] = fy;
            part[r][slot][2] = fz;
        }
    }
    __device__ __forceinline__ void zero(int slot) {
        if (threadIdx.x % 16 == 0) {
            const int r = threadIdx.x / 16;
            part[r][slot][0] = part[r][slot][1] = part[r][slot][2] = 0.0f;
        }
    }
    // node_forces[row(el)] = -f (assign) or node_forces[row(el)] -= f
    // (accumulate) for the chunk's slots el < count
    template <bool ACCUMULATE, class ROW>
    __device__ __forceinline__ void flush(int count, double* __restrict__ node_forces, ROW&& row) {
        __syncthreads();
        for (int t = threadIdx.x; t < count * 3; t += C) {
            const int el = t / 3, comp = t % 3;
            float s = 0.0f;
#pragma unroll
            for (int r = 0; r < ROWS; ++r) s += part[r][el][comp];
            double* dst = node_forces + static_cast<std::size_t>(row(el)) * 3 + comp;
            if (ACCUMULATE)
                *dst = *dst - static_cast<double>(s);
            else
                *dst = 0.0 - static_cast<double>(s);
        }
        __syncthreads();
    }
};

// ---------------------------------------------------------------------------
// Row groups.  A coupling row (p, m1, m2) reads source component
// lm2 = ls_p^2 + m2.  A group is a set of source components (bit mask); the
// R1 kernels process the rows of one group, so a shape whose rows do not fit
// the registers of one pass runs one pass per group.  Groups of one shape
// are disjoint, so each source-adjoint component W[lm2] comes from exactly one
// pass; Phi1 and the forces are sums over the passes.
// ---------------------------------------------------------------------------
// Only live rows are kept: rows whose real-basis 3j coefficients vanish for
// every output m (coupling_rows.hpp; the loader refuses a model with a term
// in such a row) contribute nothing to Phi1, G or W, and are neither held in
// registers nor accumulated.
template <int LMAX, int LMAXH, unsigned MASK>
struct RowGroup {
    using S = Shape<LMAX, LMAXH>;
    static constexpr bool in(int p, int m2) {
        return ((MASK >> (S::paths[p].ls * S::paths[p].ls + m2)) & 1u) != 0;
    }
    // row (p, m1, m2) is in the group and carries coupling coefficients
    static constexpr bool live(int p, int m1, int m2) {
        return in(p, m2) && coupling_live(S::paths[p].le, S::paths[p].ls, S::paths[p].lo, m1, m2);
    }
    static constexpr int live_count(int p) {
        int n = 0;
        for (int m1 = 0; m1 < 2 * S::paths[p].le + 1; ++m1)
            for (int m2 = 0; m2 < 2 * S::paths[p].ls + 1; ++m2) n += live(p, m1, m2) ? 1 : 0;
        return n;
    }
    static constexpr bool used(int p) { return live_count(p) > 0; }
    static constexpr bool m1_live(int p, int m1) {
        for (int m2 = 0; m2 < 2 * S::paths[p].ls + 1; ++m2)
            if (live(p, m1, m2)) return true;
        return false;
    }
    static constexpr bool m2_live(int p, int m2) {
        for (int m1 = 0; m1 < 2 * S::paths[p].le + 1; ++m1)
            if (live(p, m1, m2)) return true;
        return false;
    }
    static constexpr std::array<int, S::P + 1> make_base() {
        std::array<int, S::P + 1> b{};
        for (int p = 0; p < S::P; ++p) b[p + 1] = b[p] + live_count(p);
        return b;
    }
    static constexpr std::array<int, S::P + 1> base = make_base();
    static constexpr int NR = base[S::P] > 0 ? base[S::P] : 1;
    // register index of a live row: its rank among path p's live rows
    static constexpr int row(int p, int m1, int m2) {
        int n = 0;
        for (int a = 0; a < 2 * S::paths[p].le + 1; ++a)
            for (int b = 0; b < 2 * S::paths[p].ls + 1; ++b) {
                if (a == m1 && b == m2) return base[p] + n;
                n += live(p, a, b) ? 1 : 0;
            }
        return -1;
    }
    static constexpr bool component(int lm2) { return ((MASK >> lm2) & 1u) != 0; }
};

// Row groups of a shape, as source-component masks: one pass for L_max 1
// (88 rows at l_max 3); for L_max 2 (243 rows) the 0e+1o components (88
// rows), then 2e components m2 0-2 (93 rows) and 3-4 (62 rows).
template <int LMAX, int LMAXH>
struct SourceGroups;
template <int LMAX>
struct SourceGroups<LMAX, 0> {
    static constexpr std::array<unsigned, 1> masks{0x1u};
};
template <int LMAX>
struct SourceGroups<LMAX, 1> {
    static constexpr std::array<unsigned, 1> masks{0xfu};
};
// L_max 2: the l <= 1 components, then the five l = 2 ones.  A pass
// re-reads the records and recomputes the spline and harmonic terms, so
// fewer passes pay less of that work: the l = 2 pass runs at three waves per
// SIMD in the forward (158 VGPRs) and two in the reverse (256 VGPRs, a few
// spilled); against three passes (l <= 1, lm 4-6, lm 7-8) the wide config
// measured 6% faster with the reverse in two passes and 3% more with the
// forward too.
template <int LMAX>
struct SourceGroups<LMAX, 2> {
    static constexpr std::array<unsigned, 2> masks{0x00fu, 0x1f0u};
};

// Channel slices of the R1 forward over unstaged records: with C >= 128 each
// 64-lane wave is a workgroup of its own holding one slice of a receiver's
// channels, and the slices go to alternate XCDs (slice = XCD mod slices), so
// an XCD reads only its slice of the spline table and of the H1 rows and its
// 4 MB L2 holds that working set; the receivers are cut into contiguous
// ranges, one per group of XCDs (ranges of nearby atoms share sources).
template <int C, class EDGES>
constexpr int r1_forward_slices() {
    return (EDGES::kHold && C >= 128 && kXcds % (C >= 128 ? C / 64 : 1) == 0) ? C / 64 : 1;
}
// grid of the forward over nr receivers (padded to whole rounds of XCDs)
template <int C, class EDGES>
inline unsigned r1_forward_blocks(int nr) {
    constexpr int SL = r1_forward_slices<C, EDGES>();
    if constexpr (SL == 1) return static_cast<unsigned>(nr);
    const int per_xcd = (nr * SL + kXcds - 1) / kXcds;  // receivers per range
    return static_cast<unsigned>(per_xcd * kXcds);
}

// ---------------------------------------------------------------------------
// R1 forward: rows[i,(p,m1,m2),k] = sum_j R1_{p,k}(r) Y_{lm1} H1[j,lm2,k];
// Phi1[i,lme,k] = sum CG rows (dense per-path coupling blocks).  Each output
// lme comes from one path (lme = lme_base[lo] + mo*num_e[lo] + e_p), so it is
// written once per pass: assigned (zero for paths outside the group) or,
// with ACCUMULATE, added.  Receiver i = r0 + li owns edges [first[i],
// first[i]+count[i]) (or [first[i], first[i+1]) when count is null); Phi1
// rows are indexed by li.  H1 and Phi1 rows hold CF channels (CF <= C: the
// lanes k >= CF of a caller's unpadded arrays neither read nor write).
// ---------------------------------------------------------------------------
// At least four waves per SIMD: the single-pass shapes need 145 VGPRs for
// three, and at four (128 VGPRs, two spilled) the medium call is 0.7% faster.
// A pass over more than four source components (the l = 2 pass) keeps three
// (158 VGPRs; capped at 128 it spills 48).
constexpr int r1_forward_waves(unsigned mask) { return __builtin_popcount(mask) > 4 ? 3 : 4; }
template <int C, int LMAX, int LMAXH, unsigned MASK, bool ACCUMULATE, class EDGES, int CF = C>
__global__ __launch_bounds__(C) __attribute__((amdgpu_waves_per_eu(r1_forward_waves(MASK)))) void k_r1_forward(int r0, int nr, const int* __restrict__ first,
                                                  const int* __restrict__ count, const int* __restrict__ neigh,
                                                  EDGES edges, const float* __restrict__ H1,
                                                  const float* __restrict__ cg, float* __restrict__ Phi1) {
    using S = Shape<LMAX, LMAXH>;
    using RG = RowGroup<LMAX, LMAXH, MASK>;
    constexpr int NH = S::NH;
    constexpr int SL = r1_forward_slices<C, EDGES>();
    int li, k = threadIdx.x;
    if constexpr (SL == 1) {
        li = xcd_remap(blockIdx.x, gridDim.x);
    } else {
        // block b runs on XCD b mod 8: slice (b mod 8) mod SL of receiver
        // (b mod 8) / SL * per_xcd + b / 8 (no barrier below: the padding
        // blocks leave at once)
        const int x = static_cast<int>(blockIdx.x) % kXcds, j = static_cast<int>(blockIdx.x) / kXcds;
        li = (x / SL) * static_cast<int>(gridDim.x / kXcds) + j;
        if (li >= nr) return;
        k += (x % SL) * (C / SL);
    }
    const int i = r0 + li;
    const bool lane_on = CF == C || k < CF;
    float rows[RG::NR];
#pragma unroll
    for (int r = 0; r < RG::NR; ++r) rows[r] = 0.0f;
    const int ea = first[i], eb = count ? ea + count[i] : first[i + 1];
    // rows += R_p(r) Y_lm1 h_lm2 for one edge, given its radial values
    // (radial(p)), harmonics (Y(lm)) and source row hj
    auto add_edge = [&](auto&& radial, auto&& Y, const float* hj) __attribute__((always_inline)) {
        float h[NH];
#pragma unroll
        for (int q = 0; q < NH; ++q) h[q] = (RG::component(q) && lane_on) ? hj[q * CF] : 0.0f;
        static_for<0, S::P>([&](auto pc) {
            constexpr int p = pc;
            if constexpr (RG::used(p)) {
                constexpr int le = S::paths[p].le, ls = S::paths[p].ls;
                const float rad = radial(p);
                if constexpr (ls == 0) {
                    // one source component: scale R by it once
                    const float rh = rad * h[0];
                    static_for<0, 2 * le + 1>([&](auto m1c) {
                        constexpr int m1 = m1c;
                        if constexpr (RG::live(p, m1, 0)) {
                            constexpr int r = RG::row(p, m1, 0);
                            rows[r] += rh * Y(le * le + m1);
                        }
                    });
                } else {
                    static_for<0, 2 * le + 1>([&](auto m1c) {
                        constexpr int m1 = m1c;
                        if constexpr (RG::m1_live(p, m1)) {
                            const float ry = rad * Y(le * le + m1);
                            static_for<0, 2 * ls + 1>([&](auto m2c) {
                                constexpr int m2 = m2c;
                                if constexpr (RG::live(p, m1, m2)) {
                                    constexpr int r = RG::row(p, m1, m2);
                                    rows[r] += ry * h[ls * ls + m2];
                                }
                            });
                        }
                    });
                }
            }
        });
    };
    if constexpr (EDGES::kHold) {
        // The wave-uniform record fields (source node included) of slot e+1
        // are loaded while slot e runs, so a slot starts with its spline and
        // H1 loads instead of a chain of dependent scalar loads.  The table
        // row's coefficients of the group's paths stay in registers while
        // consecutive slots share the row.
        static_assert(CF == C, "held records are the evaluator's own, unpadded-stride layout");
        typename EDGES::Held cur, nxt;
        float4 cc[S::P];
        int cached = -1;
        if (ea < eb) edges.hold(ea, cur);
        for (int e = ea; e < eb; ++e) {
            const int en = min(e + 1, eb - 1);
            edges.hold(en, nxt);
            if (cur.active) {
                const float x = cur.x, xx = x * x, xxx = xx * x;
                if (cur.iv != cached) {
                    cached = cur.iv;
                    const float4* cf = edges.coef + static_cast<std::size_t>(cur.iv) * edges.functions;
                    static_for<0, S::P>([&](auto pc) {
                        if constexpr (RG::used(pc)) cc[pc] = cf[pc * C + k];
                    });
                }
                add_edge([&](int p) { return spline_value(cc[p], x, xx, xxx); }, [&](int lm) { return cur.y[lm]; },
                         H1 + static_cast<std::size_t>(cur.src) * NH * C + k);
            }
            cur = nxt;
        }
    } else {
        __shared__ stage4 stage_buf[2 * EDGES::kStageSlots];
        edges.chunks(ea, eb, stage_buf, [&](int e_first, int n, const float* chunk) __attribute__((always_inline)) {
            for (int j = 0; j < n; ++j) {
                const int e = e_first + j;
                typename EDGES::Point pt;
                if (!edges.open_at(e, i, chunk, j, pt)) continue;
                add_edge([&](int p) { return edges.value(pt, p * C + k); }, [&](int lm) { return edges.Y(pt, lm); },
                         H1 + static_cast<std::size_t>(edges.source(pt, e, neigh)) * NH * CF + k);
            }
        });
    }
    float* out = Phi1 + static_cast<std::size_t>(li) * S::NLME * CF + k;
    if (!lane_on) return;
    static_for<0, S::P>([&](auto pc) {
        constexpr int p = pc;
        constexpr int le = S::paths[p].le, ls = S::paths[p].ls, lo = S::paths[p].lo, co = S::cg_offset[p];
        static_for<0, 2 * lo + 1>([&](auto mc) {
            constexpr int mo = mc;
            constexpr int q = S::lme(p, mo);
            if constexpr (RG::used(p)) {
                float o = 0.0f;
                static_for<0, 2 * le + 1>([&](auto m1c) {
                    constexpr int m1 = m1c;
                    static_for<0, 2 * ls + 1>([&](auto m2c) {
                        constexpr int m2 = m2c;
                        if constexpr (RG::live(p, m1, m2)) {
                            constexpr int r = RG::row(p, m1, m2);
                            o += cg[co + (m1 * (2 * ls + 1) + m2) * (2 * lo + 1) + mo] * rows[r];
                        }
                    });
                });
                out[q * CF] = ACCUMULATE ? out[q * CF] + o : o;
            } else if constexpr (!ACCUMULATE) {
                out[q * CF] = 0.0f;
            }
        });
    });
}

// ---------------------------------------------------------------------------
// Fused R1 reverse, receiver-owned, over the rows of one group: per edge the
// directed force
//   f_e = -sum_k sum_rows G[row] H1[j,lm2] (u dR Y_lm1 + R dY_lm1)
// and the per-edge source-adjoint components in the group
//   W_e[lm2,k] = sum_{p,m1} R Y_lm1 G[row]   (zero for inactive edges)
// that k_source_gather sums over each source's edges.  G = CG^T dPhi1[li].
// W and node_forces are indexed by e - e0; forces are assigned (-f) or, with
// FORCE_ACCUMULATE, subtracted from what the buffer holds.  H1 and dPhi1
// rows hold CF channels (lanes k >= CF read zero, so their G, W and force
// parts are zero); W rows always hold C.
// ---------------------------------------------------------------------------
// STORE_W false: the forces alone (the source terms are not written).  At
// least two waves per SIMD: the l = 2 pass of L_max-2 models would otherwise
// take 264 registers and run one wave per SIMD.
template <int C, int LMAX, int LMAXH, unsigned MASK, bool FORCE_ACCUMULATE, class EDGES, int CF = C,
          bool STORE_W = true>
__global__ __launch_bounds__(C) __attribute__((amdgpu_waves_per_eu(2))) void k_r1_reverse(int r0, long long e0, const int* __restrict__ offsets,
                                                  const int* __restrict__ neigh, EDGES edges,
                                                  const float* __restrict__ H1, const float* __restrict__ cg,
                                                  const float* __restrict__ dPhi1, float* __restrict__ Wsrc,
                                                  double* __restrict__ node_forces) {
    using S = Shape<LMAX, LMAXH>;
    using RG = RowGroup<LMAX, LMAXH, MASK>;
    constexpr int NY = S::NY, NH = S::NH;
    __shared__ float part[EdgeForceSink<C, kRecordChunk>::ROWS][kRecordChunk][3];
    EdgeForceSink<C, kRecordChunk> sink{part};
    __shared__ stage4 stage_buf[2 * EDGES::kStageSlots];
    const int li = xcd_remap(blockIdx.x, gridDim.x);
    const int i = r0 + li;
    const int k = threadIdx.x;
    const bool lane_on = CF == C || k < CF;
    float G[RG::NR];
#pragma unroll
    for (int r = 0; r < RG::NR; ++r) G[r] = 0.0f;
    {
        const float* d = dPhi1 + static_cast<std::size_t>(li) * S::NLME * CF + k;
        static_for<0, S::P>([&](auto pc) {
            constexpr int p = pc;
            if constexpr (RG::used(p)) {
                constexpr int le = S::paths[p].le, ls = S::paths[p].ls, lo = S::paths[p].lo, co = S::cg_offset[p];
                static_for<0, 2 * lo + 1>([&](auto mc) {
                    constexpr int mo = mc;
                    const float dq = lane_on ? d[S::lme(p, mo) * CF] : 0.0f;
                    static_for<0, 2 * le + 1>([&](auto m1c) {
                        constexpr int m1 = m1c;
                        static_for<0, 2 * ls + 1>([&](auto m2c) {
                            constexpr int m2 = m2c;
                            if constexpr (RG::live(p, m1, m2)) {
                                constexpr int r = RG::row(p, m1, m2);
                                G[r] += cg[co + (m1 * (2 * ls + 1) + m2) * (2 * lo + 1) + mo] * dq;
                            }
                        });
                    });
                });
            }
        });
    }
    const int ea = offsets[i], eb = offsets[i + 1];
    [[maybe_unused]] float4 cc[S::P];
    [[maybe_unused]] int cached = -1;
    edges.chunks(ea, eb, stage_buf, [&](int c0, int n, const float* chunk) __attribute__((always_inline)) {
        for (int j = 0; j < n; ++j) {
            const int e = c0 + j;
            typename EDGES::Point pt;
            if (!edges.open_at(e, i, chunk, j, pt)) {
                // inactive edges (r >= cutoff) contribute nothing: their W is
                // not written and the source gathers skip them
                sink.zero(j);
                continue;
            }
            [[maybe_unused]] float* wdst =
                STORE_W ? Wsrc + static_cast<std::size_t>(edges.out_row(chunk, j, e - e0)) * NH * C + k : nullptr;
            if constexpr (EDGES::kReuse) {
                // the row's coefficients stay in registers while consecutive
                // slots share it (the row is wave-uniform)
                const int row = edges.row(pt);
                if (row != cached) {
                    cached = row;
                    static_for<0, S::P>([&](auto pc) {
                        if constexpr (RG::used(pc)) cc[pc] = edges.coef_at(pt, pc * C + k);
                    });
                }
            }
            const float* hj = H1 + static_cast<std::size_t>(edges.source(pt, e, neigh)) * NH * CF + k;
            float h[NH], W[NH];
#pragma unroll
            for (int q = 0; q < NH; ++q) {
                h[q] = (RG::component(q) && lane_on) ? hj[q * CF] : 0.0f;
                W[q] = 0.0f;
            }
            // Per path p, with T[m2] = sum_m1 Y_m1 G[p,m1,m2] and
            // s[m1] = sum_m2 G[p,m1,m2] h_m2:
            //   W[m2] += R T[m2],  A += dR sum_m2 h_m2 T[m2],  SB[lm1] += R s[m1];
            // then f = u A + sum_lm1 dY_lm1 SB[lm1].
            float A = 0.0f, SB[NY];
#pragma unroll
            for (int v = 0; v < NY; ++v) SB[v] = 0.0f;
            static_for<0, S::P>([&](auto pc) {
                constexpr int p = pc;
                if constexpr (RG::used(p)) {
                    constexpr int le = S::paths[p].le, ls = S::paths[p].ls;
                    float R, dR;
                    if constexpr (EDGES::kReuse) {
                        R = spline_value(cc[p], pt.x, pt.xx, pt.xxx);
                        dR = spline_slope(cc[p], pt.x2, pt.xx3);
                    } else {
                        edges.value_slope(pt, p * C + k, R, dR);
                    }
                    float T[2 * ls + 1];
                    static_for<0, 2 * ls + 1>([&](auto m2c) { T[m2c] = 0.0f; });
                    if constexpr (ls == 0) {
                        // one source component: SB += (R h0) G
                        const float rh = R * h[0];
                        static_for<0, 2 * le + 1>([&](auto m1c) {
                            constexpr int m1 = m1c;
                            if constexpr (RG::live(p, m1, 0)) {
                                constexpr int r = RG::row(p, m1, 0);
                                const float g = G[r];
                                T[0] += edges.Y(pt, le * le + m1) * g;
                                SB[le * le + m1] += rh * g;
                            }
                        });
                    } else {
                        static_for<0, 2 * le + 1>([&](auto m1c) {
                            constexpr int m1 = m1c;
                            if constexpr (RG::m1_live(p, m1)) {
                                const float y = edges.Y(pt, le * le + m1);
                                float sr = 0.0f;
                                static_for<0, 2 * ls + 1>([&](auto m2c) {
                                    constexpr int m2 = m2c;
                                    if constexpr (RG::live(p, m1, m2)) {
                                        constexpr int r = RG::row(p, m1, m2);
                                        const float g = G[r];
                                        T[m2] += y * g;
                                        sr += g * h[ls * ls + m2];
                                    }
                                });
                                SB[le * le + m1] += R * sr;
                            }
                        });
                    }
                    float hT = 0.0f;
                    static_for<0, 2 * ls + 1>([&](auto m2c) {
                        constexpr int m2 = m2c;
                        if constexpr (RG::m2_live(p, m2)) {
                            W[ls * ls + m2] += R * T[m2];
                            hT += h[ls * ls + m2] * T[m2];
                        }
                    });
                    A += dR * hT;
                }
            });
            float b0 = 0.0f, b1 = 0.0f, b2 = 0.0f;
#pragma unroll
            for (int v = 0; v < NY; ++v) {
                b0 += SB[v] * edges.dY(pt, 0, v);
                b1 += SB[v] * edges.dY(pt, 1, v);
                b2 += SB[v] * edges.dY(pt, 2, v);
            }
            // W is streamed (read once, by the source gather): keep it out of
            // the cache lines that H1 and the spline table reuse
            if constexpr (STORE_W) {
#pragma unroll
                for (int q = 0; q < NH; ++q)
                    if (RG::component(q)) __builtin_nontemporal_store(W[q], wdst + q * C);
            }
            sink.put(j, edges.u(pt, 0) * A + b0, edges.u(pt, 1) * A + b1, edges.u(pt, 2) * A + b2);
        }
        sink.template flush<FORCE_ACCUMULATE>(n, node_forces,
                                              [&](int el) { return edges.out_row(chunk, el, c0 + el - e0); });
    });
}

// ---------------------------------------------------------------------------
// Source adjoint: sum over the edges leaving s (source-transpose order) of
// W_e, accumulated in FP64 like the reference's source-adjoint accumulator.
// Only active edges (r < r_cut; r indexed like W) have a W row; the others
// contribute zero and are skipped, which saves reading a quarter of W at a
// 0.5 A skin.  Each wave reads one edge id and length per lane for the next
// 64 transpose slots, takes the ballot of the active ones and walks its set
// bits in order, eight rows in flight at a time; the sum keeps the
// source-transpose order (a padded slot adds +0.0, which leaves the FP64
// accumulator unchanged: it starts at +0.0 and so is never -0.0).  T is the
// transpose's position and edge-id type (int, or long long in the tiled
// plan); e_base is the first edge of the rows of Wsrc and r.
// ---------------------------------------------------------------------------
template <int C, int NH, class T = int>
__device__ __forceinline__ void gather_source_rows(const T* __restrict__ sedges, T t0, T t1, long long e_base,
                                                   const float* __restrict__ Wsrc, const double* __restrict__ r,
                                                   double r_cut, int k, double* acc) {
    constexpr int L = C < kWave ? C : kWave;
    constexpr int G = 8;
    const int lane = threadIdx.x % kWave;
    for (T base = t0; base < t1; base += L) {
        int e = 0;
        bool on = false;
        if (base + lane < t1) {
            e = static_cast<int>(sedges[base + lane] - e_base);
            on = r[e] < r_cut;
        }
        unsigned long long live = __ballot(on);
        while (live) {
            float w[G][NH];
#pragma unroll
            for (int u = 0; u < G; ++u) {
                if (live) {
                    const int l = __builtin_ctzll(live);
                    live &= live - 1;
                    const int eu = __builtin_amdgcn_readlane(e, l);
                    const float* row = Wsrc + static_cast<std::size_t>(eu) * NH * C + k;
#pragma unroll
                    for (int q = 0; q < NH; ++q) w[u][q] = __builtin_nontemporal_load(row + q * C);
                } else {
#pragma unroll
                    for (int q = 0; q < NH; ++q) w[u][q] = 0.0f;
                }
            }
#pragma unroll
            for (int u = 0; u < G; ++u)
#pragma unroll
                for (int q = 0; q < NH; ++q) acc[q] += static_cast<double>(w[u][q]);
        }
    }
}

// H1_adj[s] = (or, with ACCUMULATE, +=) the FP64 sum of W over s's edges;
// H1_adj rows hold CF <= C channels
template <int C, int NH, bool ACCUMULATE, int CF = C>
__global__ __launch_bounds__(C) void k_source_gather(const int* __restrict__ soff, const int* __restrict__ sedges,
                                                     const float* __restrict__ Wsrc, const double* __restrict__ r,
                                                     double r_cut, float* __restrict__ H1_adj) {
    const int s = xcd_remap(blockIdx.x, gridDim.x);
    const int k = threadIdx.x;
    double acc[NH];
#pragma unroll
    for (int q = 0; q < NH; ++q) acc[q] = 0.0;
    gather_source_rows<C, NH>(sedges, soff[s], soff[s + 1], 0, Wsrc, r, r_cut, k, acc);
    if (CF != C && k >= CF) return;
    float* dst = H1_adj + static_cast<std::size_t>(s) * NH * CF + k;
#pragma unroll
    for (int q = 0; q < NH; ++q) dst[q * CF] = ACCUMULATE ? dst[q * CF] + static_cast<float>(acc[q])
                                                         : static_cast<float>(acc[q]);
}

}  // namespace
}  // namespace edge
}  // namespace smx
