// Kernels of the M0 / R0 operator modules (gfx950, wave64): the
// reference's operator-module launch semantics (jit_operator_codegen.py:
// 130-277 M0, 653-898 R0; launch grids jit_operator_module.cpp:453-637) on
// this project's device code.  Every kernel runs correctly for any grid
// (the loader launches min(ceil(work / threads), persistent_blocks) blocks):
// work is taken in grid-stride steps whose trip count is uniform across a
// block, so the cross-lane reductions see every lane.
//
// Mapping:
//  * M0: lane = (node, channel) owner, channel fastest (coalesced rows), the
//    monomial list unrolled on register-resident inputs (polynomial.hpp);
//  * R0 forward: a team of C lanes owns a receiver (lanes = channels), the
//    spline point and harmonics of an edge are wave-uniform;
//  * R0 coordinate reverse: a wave owns an edge; its lanes stride over the
//    channels and the force is a wave reduction in FP64;
//  * density prepare / reverse prepare: a wave owns a node.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/symmetrix_operator_modules.h"
#include "harmonics.hpp"
#include "polynomial.hpp"

namespace smx {
namespace opmod {

constexpr int kThreads = 256;  // block size of every module kernel
constexpr int kWaveLanes = 64;

template <class T, int WIDTH>
__device__ __forceinline__ T lanes_sum(T v) {
#pragma unroll
    for (int off = WIDTH / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, WIDTH);
    return v;
}

// ---------------------------------------------------------------------------
// M0: output[i][LM][k] = sum_t w[type_i][t][k] mono_t(input[i][:][k]);
// reverse: input_adjoint = sum_LM output_adjoint[LM] dM0_LM/dinput (assigned;
// all inputs of an owner are read before its adjoint is written, so input
// and input_adjoint may alias), and with capture_input_scale_adjoint
// input_scale_adjoint[i] += sum_{v,k} input input_adjoint in FP64.
// ---------------------------------------------------------------------------
template <int C, int NIN, class TAB>
__device__ __forceinline__ void m0_forward(const SymmetrixJitM0ArgsV1& a) {
    const float* input = static_cast<const float*>(a.input);
    const float* weights = static_cast<const float*>(a.weights);
    float* output = static_cast<float*>(a.output);
    const long long owners = a.num_nodes * C;
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    for (long long owner = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; owner < owners;
         owner += stride) {
        const long long node = owner / C;
        const int k = static_cast<int>(owner % C);
        float x[NIN];
#pragma unroll
        for (int v = 0; v < NIN; ++v) x[v] = input[(node * NIN + v) * C + k];
        const float* cf = weights + static_cast<long long>(a.node_types[node]) * TAB::NT * C + k;
        static_range<0, TAB::NOUT>([&](auto oc) {
            constexpr int o = oc;
            output[(node * TAB::NOUT + o) * C + k] = poly_ct<TAB, TAB::offset[o], TAB::offset[o + 1], C>(x, cf);
        });
    }
}

template <int C, int NIN, class TAB>
__device__ __forceinline__ void m0_reverse(const SymmetrixJitM0ArgsV1& a) {
    constexpr int SEG = C < kWaveLanes ? C : kWaveLanes;  // lanes of one node within a wave
    static_assert(kWaveLanes % SEG == 0, "channels must divide the wave or be a multiple of it");
    const float* input = static_cast<const float*>(a.input);
    const float* weights = static_cast<const float*>(a.weights);
    const float* adjoint = static_cast<const float*>(a.output_adjoint);
    float* input_adjoint = static_cast<float*>(a.input_adjoint);
    const long long owners = a.num_nodes * C;
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    for (long long base = static_cast<long long>(blockIdx.x) * blockDim.x; base < owners; base += stride) {
        const long long owner = base + threadIdx.x;
        const bool valid = owner < owners;
        const long long node = valid ? owner / C : 0;
        const int k = static_cast<int>(owner % C);
        double scale = 0.0;
        if (valid) {
            float x[NIN], grad[NIN];
#pragma unroll
            for (int v = 0; v < NIN; ++v) {
                x[v] = input[(node * NIN + v) * C + k];
                grad[v] = 0.0f;
            }
            const float* cf = weights + static_cast<long long>(a.node_types[node]) * TAB::NT * C + k;
            static_range<0, TAB::NOUT>([&](auto oc) {
                constexpr int o = oc;
                const float adj = adjoint[(node * TAB::NOUT + o) * C + k];
                float g[NIN];
#pragma unroll
                for (int v = 0; v < NIN; ++v) g[v] = 0.0f;
                poly_grad_ct<TAB, TAB::offset[o], TAB::offset[o + 1], C>(x, cf, g);
#pragma unroll
                for (int v = 0; v < NIN; ++v) grad[v] += g[v] * adj;
            });
#pragma unroll
            for (int v = 0; v < NIN; ++v) {
                input_adjoint[(node * NIN + v) * C + k] = grad[v];
                scale += static_cast<double>(x[v]) * static_cast<double>(grad[v]);
            }
        }
        if (a.capture_input_scale_adjoint) {
            // one FP64 add per node segment of the wave (fixed lane order)
            scale = lanes_sum<double, SEG>(scale);
            if (valid && threadIdx.x % SEG == 0) atomicAdd(a.input_scale_adjoint + node, scale);
        }
    }
}

// ---------------------------------------------------------------------------
// R0
// ---------------------------------------------------------------------------
// Spline evaluation point of the reference module (FP64 interval search,
// point rounded to FP32; clamped to the table).
struct SplinePoint {
    int interval;
    float x;
};
__device__ __forceinline__ SplinePoint spline_point(const SymmetrixJitR0SplineV1& s, double radius) {
    int iv = static_cast<int>(floor((radius - s.x0) / s.h));
    float x = static_cast<float>(radius - s.x0 - s.h * iv);
    if (iv < 0) {
        iv = 0;
        x = 0.0f;
    } else if (iv >= static_cast<int>(s.intervals)) {
        iv = static_cast<int>(s.intervals) - 1;
        x = static_cast<float>(s.h);
    }
    return {iv, x};
}

// value and slope of function f at the point (Precision = FP32 table)
__device__ __forceinline__ float radial_at(const SymmetrixJitR0SplineV1& s, int type, int f, SplinePoint p,
                                           float* slope) {
    const float* c = static_cast<const float*>(s.coefficients) +
                     (static_cast<std::size_t>(type) * s.intervals + p.interval) * 4 * s.functions + f;
    const float c0 = c[0], c1 = c[s.functions], c2 = c[2 * s.functions], c3 = c[3 * s.functions];
    const float x = p.x;
    if (slope) *slope = c1 + 2.0f * c2 * x + 3.0f * c3 * x * x;
    return c0 + c1 * x + c2 * x * x + c3 * x * x * x;
}

// density spline (FP64 table, symmetric pair types)
__device__ __forceinline__ double density_at(const SymmetrixJitR0SplineV1& s, int type, double radius,
                                             double* slope) {
    int iv = static_cast<int>(floor((radius - s.x0) / s.h));
    double x = radius - s.x0 - s.h * iv;
    if (iv < 0) {
        iv = 0;
        x = 0.0;
    } else if (iv >= static_cast<int>(s.intervals)) {
        iv = static_cast<int>(s.intervals) - 1;
        x = s.h;
    }
    const double* c = static_cast<const double*>(s.coefficients) +
                      (static_cast<std::size_t>(type) * s.intervals + iv) * 4 * s.functions;
    const double c0 = c[0], c1 = c[s.functions], c2 = c[2 * s.functions], c3 = c[3 * s.functions];
    *slope = c1 + 2.0 * c2 * x + 3.0 * c3 * x * x;
    return c0 + c1 * x + c2 * x * x + c3 * x * x * x;
}

__device__ __forceinline__ int symmetric_pair(int a, int b, int n) {
    const int lo = a <= b ? a : b, hi = a <= b ? b : a;
    return lo * (2 * n - lo - 1) / 2 + hi;
}

// unit direction of edge e (FP32 unit vectors, or FP64 xyz / r)
__device__ __forceinline__ void edge_direction(const SymmetrixJitR0ArgsV1& a, long long e, double (&u)[3]) {
    if (a.coordinates_are_unit) {
        const float* c = static_cast<const float*>(a.coordinates);
        for (int q = 0; q < 3; ++q) u[q] = static_cast<double>(c[3 * e + q]);
    } else {
        const double* c = static_cast<const double*>(a.coordinates);
        for (int q = 0; q < 3; ++q) u[q] = c[3 * e + q] / a.radius[e];
    }
}

// density_state[i] = 1 / (1 + sum_{active e} density(r_e)); a wave per node
__device__ __forceinline__ void r0_density_prepare(const SymmetrixJitR0ArgsV1& a) {
    const int lane = threadIdx.x % kWaveLanes;
    const long long waves = static_cast<long long>(gridDim.x) * (kThreads / kWaveLanes);
    for (long long node = static_cast<long long>(blockIdx.x) * (kThreads / kWaveLanes) + threadIdx.x / kWaveLanes;
         node < a.num_nodes; node += waves) {
        const int rt = a.type_to_active[a.node_types[node]];
        const int begin = a.first_neigh[node];
        double density = 0.0;
        for (int j = lane; j < a.num_neigh[node]; j += kWaveLanes) {
            const int e = begin + j;
            const double r = a.radius[e];
            if (!(r < a.cutoff)) continue;
            double unused;
            density += density_at(a.density, symmetric_pair(rt, a.type_to_active[a.neigh_types[e]],
                                                             a.active_type_count), r, &unused);
        }
        density = lanes_sum<double, kWaveLanes>(density);
        if (lane == 0) a.density_state[node] = 1.0 / (1.0 + density);
    }
}

// output[i][lm][k] = s_i sum_e R_{l,k}(r_e) Y_lm(e); a team of C lanes per
// receiver (C <= kThreads and dividing it)
template <int C, int LMAX>
__device__ __forceinline__ void r0_forward(const SymmetrixJitR0ArgsV1& a) {
    constexpr int NY = (LMAX + 1) * (LMAX + 1);
    constexpr int TEAMS = kThreads / C;
    static_assert(kThreads % C == 0, "channels must divide the block");
    const float* harm = static_cast<const float*>(a.harmonics);
    float* output = static_cast<float*>(a.output);
    const int k = threadIdx.x % C;
    const long long teams = static_cast<long long>(gridDim.x) * TEAMS;
    for (long long node = static_cast<long long>(blockIdx.x) * TEAMS + threadIdx.x / C; node < a.num_nodes;
         node += teams) {
        const int rt = a.type_to_active[a.node_types[node]];
        const int begin = a.first_neigh[node], count = a.num_neigh[node];
        float acc[NY];
#pragma unroll
        for (int v = 0; v < NY; ++v) acc[v] = 0.0f;
        for (int j = 0; j < count; ++j) {
            const int e = begin + j;
            const double r = a.radius[e];
            if (!(r < a.cutoff)) continue;
            const int type = rt * a.active_type_count + a.type_to_active[a.neigh_types[e]];
            const SplinePoint p = spline_point(a.radial, r);
            const float* y = harm + static_cast<std::size_t>(e) * NY;
#pragma unroll
            for (int l = 0; l <= LMAX; ++l) {
                const float R = radial_at(a.radial, type, l * C + k, p, nullptr);
#pragma unroll
                for (int m = 0; m < 2 * l + 1; ++m) acc[l * l + m] += R * y[l * l + m];
            }
        }
        const float scale = a.apply_density_scale ? static_cast<float>(a.density_state[node]) : 1.0f;
#pragma unroll
        for (int v = 0; v < NY; ++v)
            output[(static_cast<std::size_t>(node) * NY + v) * C + k] = a.apply_density_scale ? acc[v] * scale : acc[v];
    }
}

// dot_i = precomputed[i] or sum output * output_adjoint (FP64);
// output_adjoint[i] *= density_state[i]; density_state[i] = dot_i density_state[i]
template <int C, int LMAX>
__device__ __forceinline__ void r0_reverse_prepare(const SymmetrixJitR0ArgsV1& a) {
    constexpr int NY = (LMAX + 1) * (LMAX + 1);
    constexpr int VALUES = NY * C;
    const float* output = static_cast<const float*>(a.output);
    float* adjoint = static_cast<float*>(a.output_adjoint);
    const int lane = threadIdx.x % kWaveLanes;
    const long long waves = static_cast<long long>(gridDim.x) * (kThreads / kWaveLanes);
    for (long long node = static_cast<long long>(blockIdx.x) * (kThreads / kWaveLanes) + threadIdx.x / kWaveLanes;
         node < a.num_nodes; node += waves) {
        const std::size_t base = static_cast<std::size_t>(node) * VALUES;
        double dot = 0.0;
        if (!a.use_precomputed_scale_adjoint)
            for (int v = lane; v < VALUES; v += kWaveLanes)
                dot += static_cast<double>(output[base + v]) * static_cast<double>(adjoint[base + v]);
        dot = lanes_sum<double, kWaveLanes>(dot);
        if (a.use_precomputed_scale_adjoint) dot = a.precomputed_scale_adjoint[node];
        const double inverse = a.density_state[node];
        const float inv = static_cast<float>(inverse);
        for (int v = lane; v < VALUES; v += kWaveLanes) adjoint[base + v] *= inv;
        if (lane == 0) a.density_state[node] = dot * inverse;
    }
}

// directed_forces[e] -= sum_{l,k,m} adj[i,lm,k] (dR_{l,k} Y_lm u + R_{l,k} dY_lm)
// (+ density_state[i] density'(r) u with the density scale); a wave per
// edge, lanes over channels, the force summed in FP64
template <int C, int LMAX>
__device__ __forceinline__ void r0_coordinate_reverse(const SymmetrixJitR0ArgsV1& a) {
    constexpr int NY = (LMAX + 1) * (LMAX + 1);
    const float* harm = static_cast<const float*>(a.harmonics);
    const float* grads = static_cast<const float*>(a.harmonic_gradients);
    const float* adjoint = static_cast<const float*>(a.output_adjoint);
    const int lane = threadIdx.x % kWaveLanes;
    const long long waves = static_cast<long long>(gridDim.x) * (kThreads / kWaveLanes);
    for (long long e = static_cast<long long>(blockIdx.x) * (kThreads / kWaveLanes) + threadIdx.x / kWaveLanes;
         e < a.num_edges; e += waves) {
        const double r = a.radius[e];
        if (!(r < a.cutoff)) continue;
        const long long node = static_cast<long long>(a.edge_receivers[e]) - a.receiver_base;
        const int rt = a.type_to_active[a.node_types[node]];
        const int nt = a.type_to_active[a.neigh_types[e]];
        const int type = rt * a.active_type_count + nt;
        double u[3];
        edge_direction(a, e, u);
        float dY[3 * NY];
        if (grads) {
#pragma unroll
            for (int q = 0; q < 3 * NY; ++q) dY[q] = grads[static_cast<std::size_t>(e) * 3 * NY + q];
        } else {
            const float d[3] = {static_cast<float>(u[0]), static_cast<float>(u[1]), static_cast<float>(u[2])};
            edge_harmonics<LMAX>(d, static_cast<float>(r), nullptr, dY);
        }
        const float* y = harm + static_cast<std::size_t>(e) * NY;
        const SplinePoint p = spline_point(a.radial, r);
        double f0 = 0.0, f1 = 0.0, f2 = 0.0;
        for (int k = lane; k < C; k += kWaveLanes) {
#pragma unroll
            for (int l = 0; l <= LMAX; ++l) {
                float dR;
                const float R = radial_at(a.radial, type, l * C + k, p, &dR);
#pragma unroll
                for (int m = 0; m < 2 * l + 1; ++m) {
                    const int lm = l * l + m;
                    const float adj = adjoint[(static_cast<std::size_t>(node) * NY + lm) * C + k];
                    const double rs = static_cast<double>(adj * dR * y[lm]);
                    const double as = static_cast<double>(adj * R);
                    f0 += rs * u[0] + as * static_cast<double>(dY[lm]);
                    f1 += rs * u[1] + as * static_cast<double>(dY[NY + lm]);
                    f2 += rs * u[2] + as * static_cast<double>(dY[2 * NY + lm]);
                }
            }
        }
        f0 = lanes_sum<double, kWaveLanes>(f0);
        f1 = lanes_sum<double, kWaveLanes>(f1);
        f2 = lanes_sum<double, kWaveLanes>(f2);
        if (lane == 0) {
            double* out = a.directed_forces + 3 * e;
            out[0] -= f0;
            out[1] -= f1;
            out[2] -= f2;
            if (a.apply_density_scale) {
                double slope;
                (void)density_at(a.density, symmetric_pair(rt, nt, a.active_type_count), r, &slope);
                const double c = a.density_state[node] * slope;
                out[0] += c * u[0];
                out[1] += c * u[1];
                out[2] += c * u[2];
            }
        }
    }
}

}  // namespace opmod
}  // namespace smx
