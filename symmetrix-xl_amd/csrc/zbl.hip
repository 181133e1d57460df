// ZBL pair repulsion (models with has_zbl), FP64: for every CSR edge of a
// receiver, V(r) = 0.5 * 14.3996 Z_u Z_v / r * phi(r/a) * envelope(r/r_max)
// with phi the four-exponential screening function; the receiver's energy
// gains sum_j V and the edge's directed force loses (xyz/r) dV/dr.
//
// Reference: zbl_kokkos.cpp:11-56 (pair constants 1/a, 14.3996 Z_u Z_v and
// r_max = covalent radius sum, formed on the host per pair), :92-139 (value
// and gradient), :163-199 (per-receiver energy sum and edge forces);
// applied to every edge of the prepared graph (mace_kokkos_evaluate.cpp:
// 418-434).  One wave per receiver, lanes over its edges.
#include <hip/hip_runtime.h>

#include "device_common.hpp"
#include "kernels.hpp"

namespace smx {
namespace {

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

struct ZblArgs {
    const double* pair;  // [type][type][3]: 1/a, bare prefactor, r_max
    int num_types;
    double c[4];
    int p;
};

__device__ __forceinline__ void zbl_value_gradient(const ZblArgs& z, int tu, int tv, double r, double& value,
                                                   double& gradient) {
    const double* pc = z.pair + 3 * (static_cast<std::size_t>(tu) * z.num_types + tv);
    const double inverse_a = pc[0], bare_prefactor = pc[1], r_max = pc[2];
    if (r >= r_max) {
        value = gradient = 0.0;
        return;
    }
    const double ra = r * inverse_a;
    const double e0 = z.c[0] * exp(-3.2 * ra), e1 = z.c[1] * exp(-0.9423 * ra), e2 = z.c[2] * exp(-0.4028 * ra),
                 e3 = z.c[3] * exp(-0.2016 * ra);
    const double phi = e0 + e1 + e2 + e3;
    const double dphi = inverse_a * (-3.2 * e0 + -0.9423 * e1 + -0.4028 * e2 + -0.2016 * e3);
    const double inv_r = 1.0 / r;
    const double bare = bare_prefactor * inv_r * phi;
    const double bare_g = bare_prefactor * inv_r * inv_r * (r * dphi - phi);
    const double p = z.p;
    const double c0 = (p + 1.0) * (p + 2.0) / 2.0, c1 = p * (p + 2.0), c2 = p * (p + 1.0) / 2.0;
    const double x = r / r_max;
    const double xm1 = pow(x, p - 1.0), xp = xm1 * x, xp1 = xp * x, xp2 = xp1 * x;
    const double env = 1.0 - c0 * xp + c1 * xp1 - c2 * xp2;
    const double env_g = (-c0 * p * xm1 + c1 * (p + 1.0) * xp - c2 * (p + 2.0) * xp1) / r_max;
    value = 0.5 * bare * env;
    gradient = 0.5 * (bare * env_g + bare_g * env);
}

// receivers r0..r0+nr: node_energies (graph-wide) += sum_j V; nf (tile-local,
// [ne][3]) -= (xyz/r) dV/dr; xyz and r tile-local
__global__ __launch_bounds__(256) void k_zbl(int nr, int r0, long long e0, const int* __restrict__ offsets,
                                             const int* __restrict__ node_types,
                                             const int* __restrict__ neigh_types, ZblArgs z,
                                             const double* __restrict__ xyz, const double* __restrict__ r,
                                             double* __restrict__ node_energies, double* __restrict__ nf) {
    const int i = blockIdx.x * 4 + threadIdx.x / kWave;
    if (i >= nr) return;
    const int lane = threadIdx.x % kWave;
    const int tu = node_types[r0 + i];
    const long long ea = offsets[r0 + i] - e0, eb = offsets[r0 + i + 1] - e0;
    double energy = 0.0;
    for (long long e = ea + lane; e < eb; e += kWave) {
        double v, g;
        const double re = r[e];
        zbl_value_gradient(z, tu, neigh_types[e0 + e], re, v, g);
        energy += v;
        for (int c = 0; c < 3; ++c) nf[3 * e + c] -= xyz[3 * e + c] / re * g;
    }
    energy = wave_sum_f64(energy);
    if (lane == 0) node_energies[r0 + i] += energy;
}

}  // namespace

void launch_zbl(const DeviceModel& m, const DeviceGraph& g, const TileView& t, double* node_energies,
                double* node_forces, hipStream_t s) {
    if (!m.has_zbl || t.nr == 0) return;
    if (!t.r || !t.xyz) throw std::logic_error("ZBL needs the tile's edge geometry");
    ZblArgs z{m.zbl_pair, m.num_elements, {m.zbl_c[0], m.zbl_c[1], m.zbl_c[2], m.zbl_c[3]}, m.zbl_p};
    k_zbl<<<(t.nr + 3) / 4, 256, 0, s>>>(t.nr, t.r0, t.e0, g.offsets, g.node_types, g.neigh_types, z, t.xyz, t.r,
                                         node_energies, node_forces);
    SMX_LAUNCH_CHECK("zbl");
}

}  // namespace smx
