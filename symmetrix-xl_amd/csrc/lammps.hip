// Device side of the LAMMPS pair-style entry (smx_lammps_compute): graph
// topology from a full LAMMPS neighbour list, per-call edge vectors from the
// local and ghost positions, and the reductions into LAMMPS's per-atom arrays.
//
// Reference: pair_symmetrix_mace_kokkos.cpp:1010-1282 (compute_no_domain_
// decomposition): node types through the LAMMPS->model type map, edges to
// atom->map(tag[j]), xyz = x[j] - x[i] scaled to the cutoff when longer
// (prepared execution keeps every listed neighbour), f[j] += f_e and
// f[i] -= sum_e f_e, per-atom energies, and the six virial components.
// Here the force reduction is a deterministic gather: each atom sums the
// edges that point at it (a transpose by LAMMPS index) and, for a local atom,
// subtracts its own edges, instead of atomic adds.
#include <hip/hip_runtime.h>

#include "device_common.hpp"
#include "kernels.hpp"

namespace smx {
namespace {

constexpr int kNeighMask = 0x1FFFFFFF;  // LAMMPS NEIGHMASK (neighbor.h)

__device__ __forceinline__ int model_type(int t, const int* type_to_model, int ntypes) {
    return (t >= 1 && t <= ntypes) ? type_to_model[t - 1] : -1;
}

__global__ void k_lmp_nodes(int inum, int nall, LammpsList L, int* __restrict__ node_types,
                            int* __restrict__ num_neigh, int* __restrict__ node_of_atom, int* __restrict__ bad) {
    const int ii = blockIdx.x * blockDim.x + threadIdx.x;
    if (ii >= inum) return;
    const int i = L.ilist[ii];
    int t = -1, n = 0;
    if (i >= 0 && i < nall) {
        t = model_type(L.type[i], L.type_to_model, L.ntypes);
        n = L.numneigh[i];
        node_of_atom[i] = ii;
    }
    if (t < 0 || n < 0) {
        atomicAdd(bad, 1);
        t = 0;
        n = 0;
    }
    node_types[ii] = t;
    num_neigh[ii] = n;
}

// Each workgroup takes 64 consecutive ilist entries (one per lane, so the
// lanes of a wave read one neighbour slot of 64 atoms: coalesced for the
// column-major Kokkos list) and kEdgePhases waves, wave w taking the slots
// jj = w, w + kEdgePhases, ...
constexpr int kEdgePhases = 16;
__global__ __launch_bounds__(64 * kEdgePhases) void k_lmp_edges(int inum, int nall, LammpsList L,
                                                                const int* __restrict__ offsets,
                                                                const int* __restrict__ node_of_atom,
                                                                int* __restrict__ neigh, int* __restrict__ neigh_types,
                                                                int* __restrict__ lmp_j, int* __restrict__ bad) {
    const int ii = blockIdx.x * 64 + static_cast<int>(threadIdx.x % 64);
    const int phase = static_cast<int>(threadIdx.x / 64);
    if (ii >= inum) return;
    const int i = L.ilist[ii];
    const int e0 = offsets[ii], n = offsets[ii + 1] - e0;
    for (int jj = phase; jj < n; jj += kEdgePhases) {
        const int j = L.neighbors[static_cast<long long>(i) * L.stride_atom + static_cast<long long>(jj) * L.stride_neighbor] &
                      kNeighMask;
        int node = -1, t = -1;
        if (j < nall) {
            const int o = L.owner[j];
            if (o >= 0 && o < nall) node = node_of_atom[o];
            t = model_type(L.type[j], L.type_to_model, L.ntypes);
        }
        if (node < 0 || t < 0) {
            atomicAdd(bad, 1);
            neigh[e0 + jj] = ii;
            neigh_types[e0 + jj] = 0;
            lmp_j[e0 + jj] = i;
            continue;
        }
        neigh[e0 + jj] = node;
        neigh_types[e0 + jj] = t;
        lmp_j[e0 + jj] = j;
    }
}

// xyz = x[j] - x[i], scaled to the cutoff when longer; a non-finite or zero
// length is counted and parked at the cutoff (no force)
__global__ void k_lmp_geometry(long long e0, long long ne, const int* __restrict__ receivers,
                               const int* __restrict__ ilist, const int* __restrict__ lmp_j,
                               const double* __restrict__ x, double r_cut, double* __restrict__ xyz,
                               double* __restrict__ r, int* __restrict__ invalid) {
    const long long le = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (le >= ne) return;
    const long long e = e0 + le;
    const int i = ilist[receivers[e]], j = lmp_j[e];
    const double dx = x[3 * static_cast<long long>(j)] - x[3 * static_cast<long long>(i)];
    const double dy = x[3 * static_cast<long long>(j) + 1] - x[3 * static_cast<long long>(i) + 1];
    const double dz = x[3 * static_cast<long long>(j) + 2] - x[3 * static_cast<long long>(i) + 2];
    const double r2 = dx * dx + dy * dy + dz * dz;
    if (!isfinite(r2) || !(r2 > 0.0)) {
        atomicAdd(invalid, 1);
        xyz[3 * le] = r_cut;
        xyz[3 * le + 1] = 0.0;
        xyz[3 * le + 2] = 0.0;
        r[le] = r_cut;
        return;
    }
    const double d = sqrt(r2);
    const double scale = d >= r_cut ? r_cut / d : 1.0;
    xyz[3 * le] = scale * dx;
    xyz[3 * le + 1] = scale * dy;
    xyz[3 * le + 2] = scale * dz;
    r[le] = scale * d;
}

// f[a] += sum of the edges pointing at atom a - (a local) sum of a's edges
__global__ void k_lmp_forces(int nall, const int* __restrict__ joff, const int* __restrict__ jedges,
                             const int* __restrict__ node_of_atom, const int* __restrict__ offsets,
                             const double* __restrict__ nf, double* __restrict__ f) {
    const int a = blockIdx.x * blockDim.x + threadIdx.x;
    if (a >= nall) return;
    double fx = 0.0, fy = 0.0, fz = 0.0;
    for (int q = joff[a]; q < joff[a + 1]; ++q) {
        const long long e = jedges[q];
        fx += nf[3 * e];
        fy += nf[3 * e + 1];
        fz += nf[3 * e + 2];
    }
    const int ii = node_of_atom[a];
    if (ii >= 0)
        for (long long e = offsets[ii]; e < offsets[ii + 1]; ++e) {
            fx -= nf[3 * e];
            fy -= nf[3 * e + 1];
            fz -= nf[3 * e + 2];
        }
    f[3 * static_cast<long long>(a)] += fx;
    f[3 * static_cast<long long>(a) + 1] += fy;
    f[3 * static_cast<long long>(a) + 2] += fz;
}

__global__ void k_lmp_eatom(int inum, const int* __restrict__ ilist, const double* __restrict__ node_energies,
                            double* __restrict__ eatom) {
    const int ii = blockIdx.x * blockDim.x + threadIdx.x;
    if (ii < inum) eatom[ilist[ii]] += node_energies[ii];
}

__global__ void k_fill_int(int n, int value, int* __restrict__ p) {
    const int q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q < n) p[q] = value;
}

}  // namespace

void lammps_nodes(int inum, int nall, const LammpsList& L, int* node_types, int* num_neigh, int* node_of_atom,
                  int* bad, hipStream_t s) {
    if (nall > 0) {
        k_fill_int<<<blocks_for(nall, 256), 256, 0, s>>>(nall, -1, node_of_atom);
        SMX_LAUNCH_CHECK("lammps_node_map");
    }
    if (inum == 0) return;
    k_lmp_nodes<<<blocks_for(inum, 256), 256, 0, s>>>(inum, nall, L, node_types, num_neigh, node_of_atom, bad);
    SMX_LAUNCH_CHECK("lammps_nodes");
}

void lammps_edges(int inum, int nall, const LammpsList& L, const int* offsets, const int* node_of_atom, int* neigh,
                  int* neigh_types, int* lmp_j, int* bad, hipStream_t s) {
    if (inum == 0) return;
    k_lmp_edges<<<blocks_for(inum, 64), 64 * kEdgePhases, 0, s>>>(inum, nall, L, offsets, node_of_atom, neigh,
                                                                   neigh_types, lmp_j, bad);
    SMX_LAUNCH_CHECK("lammps_edges");
}

void lammps_geometry(std::int64_t e0, std::int64_t ne, const int* receivers, const int* ilist, const int* lmp_j,
                     const double* x, double r_cut, double* xyz, double* r, int* invalid, hipStream_t s) {
    if (ne == 0) return;
    k_lmp_geometry<<<blocks_for(ne, 256), 256, 0, s>>>(e0, ne, receivers, ilist, lmp_j, x, r_cut, xyz, r, invalid);
    SMX_LAUNCH_CHECK("lammps_geometry");
}

void lammps_forces(int nall, const int* joff, const int* jedges, const int* node_of_atom, const int* offsets,
                   const double* node_forces, double* f, hipStream_t s) {
    if (nall == 0) return;
    k_lmp_forces<<<blocks_for(nall, 256), 256, 0, s>>>(nall, joff, jedges, node_of_atom, offsets, node_forces, f);
    SMX_LAUNCH_CHECK("lammps_forces");
}

void lammps_eatom(int inum, const int* ilist, const double* node_energies, double* eatom, hipStream_t s) {
    if (inum == 0) return;
    k_lmp_eatom<<<blocks_for(inum, 256), 256, 0, s>>>(inum, ilist, node_energies, eatom);
    SMX_LAUNCH_CHECK("lammps_eatom");
}

}  // namespace smx
