// Density scaling of A0 and A1 (models with A0_scaled / A1_scaled): each
// receiver's A rows are divided by s_i = 1 + sum_j f(r_ij), where f is a
// one-output radial network with tanh(v^2) postprocessing, tabulated as an
// FP64 Hermite spline.
//
// Reference semantics (Kokkos evaluator):
//   * s_i: FP64 sum over every CSR edge of i (skin edges included, their r
//     clamped to the cutoff), then + 1.0 (mace_kokkos_first_interaction.cpp:
//     1389-1406; mace_kokkos_second_interaction.cpp:1455-1473);
//   * A0 /= s in FP64 (first_interaction.cpp:1409-1415); A1 *= float(1/s)
//     (second_interaction.cpp:1474-1487);
//   * reverse: dot = sum_lmk A_adj*A (FP32 products, FP64 sum); directed
//     edge forces += (dot/s) f'(r) r^ (first_interaction.cpp:1508-1528,
//     second_interaction.cpp:1673-1710); A0_adj /= s, A1_adj *= float(1/s).
//   * FP64 spline evaluation radial_function_set_kokkos.hpp:48-62,104-146.
//
// All of this is per receiver or per edge and small next to the edge
// kernels: one wave per receiver for the factors, one workgroup per receiver
// for the adjoint dot product, one thread per edge for the forces.
#include <hip/hip_runtime.h>

#include "device_common.hpp"
#include "kernels.hpp"

namespace smx {
namespace {

struct DensitySpline {
    const double* c;  // [pair][interval][4]
    int intervals;
    double x0, h;
};

// f(r), f'(r) of the density spline of table pair `pair` ([pair][interval][4])
__device__ __forceinline__ void density_eval(const DensitySpline& sp, int pair, double r, double& f, double& d) {
    int iv = static_cast<int>(floor((r - sp.x0) / sp.h));
    double x = r - sp.x0 - sp.h * iv;
    if (iv < 0) {
        iv = 0;
        x = 0.0;
    } else if (iv >= sp.intervals) {
        iv = sp.intervals - 1;
        x = sp.h;
    }
    const double xx = x * x;
    const double* c = sp.c + 4 * (static_cast<std::size_t>(pair) * sp.intervals + iv);
    f = c[0] + c[1] * x + c[2] * xx + c[3] * (xx * x);
    d = c[1] + c[2] * (2.0 * x) + c[3] * (3.0 * xx);
}

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// s[i] = 1 + sum_e f(r_e) over receiver r0+i's edges; one wave per receiver
// (four per workgroup).  r is indexed by edge - e0.
__global__ __launch_bounds__(256) void k_density_factors(int nr, int r0, long long e0, const int* __restrict__ offsets,
                                                         const double* __restrict__ r,
                                                         const int* __restrict__ edge_pair, DensitySpline sp0,
                                                         DensitySpline sp1, double* __restrict__ s0,
                                                         double* __restrict__ s1) {
    const int i = blockIdx.x * 4 + threadIdx.x / kWave;
    if (i >= nr) return;
    const int lane = threadIdx.x % kWave;
    const long long ea = offsets[r0 + i] - e0, eb = offsets[r0 + i + 1] - e0;
    double a0 = 0.0, a1 = 0.0;
    for (long long e = ea + lane; e < eb; e += kWave) {
        double f, d;
        const int pair = edge_pair ? edge_pair[e0 + e] : 0;
        if (s0) {
            density_eval(sp0, pair, r[e], f, d);
            a0 += f;
        }
        if (s1) {
            density_eval(sp1, pair, r[e], f, d);
            a1 += f;
        }
    }
    if (s0) {
        a0 = wave_sum_f64(a0);
        if (lane == 0) s0[i] = a0 + 1.0;
    }
    if (s1) {
        a1 = wave_sum_f64(a1);
        if (lane == 0) s1[i] = a1 + 1.0;
    }
}

// Rows [nr][row_len]: A /= s (FP64 division) or A *= float(1/s).
__global__ __launch_bounds__(256) void k_density_scale(int row_len, const double* __restrict__ s, bool divide,
                                                       float* __restrict__ A) {
    const int i = blockIdx.x;
    const double si = s[i];
    const float inv = static_cast<float>(1.0 / si);
    float* row = A + static_cast<std::size_t>(i) * row_len;
    for (int j = threadIdx.x; j < row_len; j += blockDim.x)
        row[j] = divide ? static_cast<float>(static_cast<double>(row[j]) / si) : row[j] * inv;
}

// dot[i] = sum_j (float)(adj*a) in FP64 over row i, then adj scaled like A.
// Fixed per-thread strides and a fixed LDS tree: deterministic.
__global__ __launch_bounds__(256) void k_density_adjoint(int row_len, const float* __restrict__ A,
                                                         const double* __restrict__ s, bool divide,
                                                         float* __restrict__ adj, double* __restrict__ dot) {
    __shared__ double part[256 / kWave];
    const int i = blockIdx.x;
    const float* a = A + static_cast<std::size_t>(i) * row_len;
    float* g = adj + static_cast<std::size_t>(i) * row_len;
    double acc = 0.0;
    for (int j = threadIdx.x; j < row_len; j += blockDim.x) acc += static_cast<double>(g[j] * a[j]);
    acc = wave_sum_f64(acc);
    if (threadIdx.x % kWave == 0) part[threadIdx.x / kWave] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        for (int w = 0; w < static_cast<int>(blockDim.x) / kWave; ++w) t += part[w];
        dot[i] = t;
    }
    const double si = s[i];
    const float inv = static_cast<float>(1.0 / si);
    for (int j = threadIdx.x; j < row_len; j += blockDim.x)
        g[j] = divide ? static_cast<float>(static_cast<double>(g[j]) / si) : g[j] * inv;
}

// Directed forces of the tile's edges: += (dot1/s1 f1'(r)) (xyz/r), then
// += dot0/s0 f0'(r) xyz/r (the two reference expressions), per component.
__global__ __launch_bounds__(256) void k_density_forces(long long ne, long long e0, int r0,
                                                        const int* __restrict__ receivers,
                                                        const double* __restrict__ xyz,
                                                        const double* __restrict__ r, DensitySpline sp0,
                                                        const double* __restrict__ s0, const double* __restrict__ dot0,
                                                        DensitySpline sp1, const double* __restrict__ s1,
                                                        const double* __restrict__ dot1,
                                                        const int* __restrict__ edge_pair, double* __restrict__ nf) {
    const long long le = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (le >= ne) return;
    const int i = receivers[e0 + le] - r0;
    const double re = r[le];
    const int pair = edge_pair ? edge_pair[e0 + le] : 0;
    double f[3] = {nf[3 * le], nf[3 * le + 1], nf[3 * le + 2]};
    if (dot1) {
        double v, d;
        density_eval(sp1, pair, re, v, d);
        const double scale = dot1[i] / s1[i] * d;
        for (int c = 0; c < 3; ++c) f[c] += scale * (xyz[3 * le + c] / re);
    }
    if (dot0) {
        double v, d;
        density_eval(sp0, pair, re, v, d);
        for (int c = 0; c < 3; ++c) f[c] += dot0[i] / s0[i] * d * xyz[3 * le + c] / re;
    }
    for (int c = 0; c < 3; ++c) nf[3 * le + c] = f[c];
}

DensitySpline spline_of(const DeviceModel& m, const double* c) { return {c, m.intervals, m.x0_f64, m.h_f64}; }

}  // namespace

void launch_density_factors(const DeviceModel& m, const DeviceGraph& g, const TileView& t, double* s0, double* s1,
                            hipStream_t s) {
    if (t.nr == 0 || (!s0 && !s1)) return;
    if (!t.r) throw std::logic_error("density scaling needs the tile's edge lengths");
    k_density_factors<<<(t.nr + 3) / 4, 256, 0, s>>>(t.nr, t.r0, t.e0, g.offsets, t.r, g.edge_pair,
                                                     spline_of(m, m.dens0), spline_of(m, m.dens1), s0, s1);
    SMX_LAUNCH_CHECK("density_factors");
}

void launch_density_scale(int nr, int row_len, const double* s, bool divide, float* A, hipStream_t st) {
    if (nr == 0) return;
    k_density_scale<<<nr, 256, 0, st>>>(row_len, s, divide, A);
    SMX_LAUNCH_CHECK("density_scale");
}

void launch_density_adjoint(int nr, int row_len, const float* A, const double* s, bool divide, float* adj,
                            double* dot, hipStream_t st) {
    if (nr == 0) return;
    k_density_adjoint<<<nr, 256, 0, st>>>(row_len, A, s, divide, adj, dot);
    SMX_LAUNCH_CHECK("density_adjoint");
}

void launch_density_forces(const DeviceModel& m, const DeviceGraph& g, const TileView& t, const double* s0,
                           const double* dot0, const double* s1, const double* dot1, double* node_forces,
                           hipStream_t s) {
    if (t.ne == 0 || (!dot0 && !dot1)) return;
    if (!t.r || !t.xyz) throw std::logic_error("density scaling needs the tile's edge geometry");
    k_density_forces<<<static_cast<unsigned>((t.ne + 255) / 256), 256, 0, s>>>(
        t.ne, t.e0, t.r0, g.receivers, t.xyz, t.r, spline_of(m, m.dens0), s0, dot0, spline_of(m, m.dens1), s1, dot1,
        g.edge_pair, node_forces);
    SMX_LAUNCH_CHECK("density_forces");
}

}  // namespace smx
