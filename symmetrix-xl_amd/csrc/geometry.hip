// Graph and geometry kernels: periodic neighbour list, edge schedules,
// prepared edge geometry and per-edge spherical harmonics.
//
// This translation unit is compiled with -ffp-contract=off: the neighbour
// list must be bit-exact with the reference's device builder
// (libsymmetrix/source/neighbor_graph_kokkos.cpp:38-405), which evaluates
// every FP64 expression without fused multiply-adds, and the edge geometry
// (mace_kokkos_factorized_lifecycle.cpp:2915-3079) and harmonics
// (spherical_harmonic_device.hpp:150-199) follow the same rounding.
#include <algorithm>
#include <climits>
#include <cmath>
#include <stdexcept>
#include <vector>

#include "device_common.hpp"
#include "harmonics.hpp"
#include "kernels.hpp"
#include "shapes.hpp"

namespace smx {
namespace {

struct Mat3 {
    double v[9];
};

// ---------------------------------------------------------------------------
// Exclusive scan of int32 counts into int64 offsets (three passes).
// ---------------------------------------------------------------------------
constexpr int kScanThreads = 256;
constexpr int kScanItems = 8;
constexpr int kScanTile = kScanThreads * kScanItems;

__global__ __launch_bounds__(kScanThreads) void k_scan_tiles(const int* __restrict__ in, long long* __restrict__ out,
                                                             int n, long long* __restrict__ tile_sums) {
    __shared__ long long warp_tot[kScanThreads / kWave];
    const int base = blockIdx.x * kScanTile + threadIdx.x * kScanItems;
    long long v[kScanItems];
    long long run = 0;
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        const int idx = base + j;
        const long long x = idx < n ? static_cast<long long>(in[idx]) : 0;
        v[j] = run;
        run += x;
    }
    // exclusive scan of the per-thread totals across the workgroup
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    long long incl = run;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const long long y = __shfl_up(incl, off, kWave);
        if (lane >= off) incl += y;
    }
    if (lane == kWave - 1) warp_tot[wave] = incl;
    __syncthreads();
    long long wave_base = 0;
    for (int w = 0; w < wave; ++w) wave_base += warp_tot[w];
    const long long excl = wave_base + incl - run;
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        const int idx = base + j;
        if (idx < n) out[idx] = excl + v[j];
    }
    if (threadIdx.x == kScanThreads - 1) tile_sums[blockIdx.x] = excl + run;
}

__global__ __launch_bounds__(1024) void k_scan_tile_sums(long long* __restrict__ sums, int tiles) {
    // single workgroup, sequential over chunks of 1024 with a running carry
    __shared__ long long warp_tot[1024 / kWave];
    __shared__ long long carry;
    if (threadIdx.x == 0) carry = 0;
    __syncthreads();
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    for (int c0 = 0; c0 < tiles; c0 += 1024) {
        const int idx = c0 + threadIdx.x;
        const long long x = idx < tiles ? sums[idx] : 0;
        long long incl = x;
        for (int off = 1; off < kWave; off <<= 1) {
            const long long y = __shfl_up(incl, off, kWave);
            if (lane >= off) incl += y;
        }
        if (lane == kWave - 1) warp_tot[wave] = incl;
        __syncthreads();
        long long wb = 0;
        for (int w = 0; w < wave; ++w) wb += warp_tot[w];
        const long long base = carry;
        __syncthreads();
        if (idx < tiles) sums[idx] = base + wb + incl - x;
        if (threadIdx.x == 1023) carry = base + wb + incl;
        __syncthreads();
    }
    if (threadIdx.x == 0) sums[tiles] = carry;
}

__global__ __launch_bounds__(kScanThreads) void k_scan_add(long long* __restrict__ out, int n,
                                                           const long long* __restrict__ tile_sums, int tiles) {
    const int idx = blockIdx.x * kScanThreads + threadIdx.x;
    if (idx < n) out[idx] += tile_sums[idx / kScanTile];
    if (idx == 0) out[n] = tile_sums[tiles];
}

__global__ void k_i64_to_i32(const long long* __restrict__ in, int* __restrict__ out, int n) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx < n) out[idx] = static_cast<int>(in[idx]);
}

// ---------------------------------------------------------------------------
// Neighbour list (neighbor_graph_kokkos.cpp:117-402)
// ---------------------------------------------------------------------------
struct BinGrid {
    int bins[3];
    int reach[3];
};

__device__ __forceinline__ int floor_div(int a, int b) {
    const int q = a / b, r = a % b;
    return q - ((r != 0 && r < 0) ? 1 : 0);
}

__global__ void k_wrap(int N, const double* __restrict__ pos, Mat3 cell, Mat3 inv, BinGrid g,
                       double* __restrict__ wfrac, double* __restrict__ wpos, int* __restrict__ wrap,
                       int* __restrict__ abin, int* __restrict__ bsize) {
    const int a = blockIdx.x * blockDim.x + threadIdx.x;
    if (a >= N) return;
    double f[3];
    for (int ax = 0; ax < 3; ++ax) {
        double v = 0.0;
        for (int c = 0; c < 3; ++c) v += pos[3 * a + c] * inv.v[3 * c + ax];
        const int w = static_cast<int>(floor(v));
        v -= w;
        f[ax] = v;
        wfrac[3 * a + ax] = v;
        wrap[3 * a + ax] = w;
    }
    for (int c = 0; c < 3; ++c) {
        double v = 0.0;
        for (int ax = 0; ax < 3; ++ax) v += f[ax] * cell.v[3 * ax + c];
        wpos[3 * a + c] = v;
    }
    const int x = min(g.bins[0] - 1, static_cast<int>(f[0] * g.bins[0]));
    const int y = min(g.bins[1] - 1, static_cast<int>(f[1] * g.bins[1]));
    const int z = min(g.bins[2] - 1, static_cast<int>(f[2] * g.bins[2]));
    const int b = (z * g.bins[1] + y) * g.bins[0] + x;
    abin[a] = b;
    atomicAdd(&bsize[b], 1);
}

__global__ void k_bin_fill(int N, const int* __restrict__ abin, int* __restrict__ cursor, int* __restrict__ batoms) {
    const int a = blockIdx.x * blockDim.x + threadIdx.x;
    if (a >= N) return;
    const int slot = atomicAdd(&cursor[abin[a]], 1);
    batoms[slot] = a;
}

// Ascending order within each segment (the bins' atom lists,
// neighbor_graph_kokkos.cpp:233-249, and each source's edge list).  One
// wave per segment: the segment is copied to LDS, each item's place is the
// number of smaller items (the items of a segment are distinct), and the
// items are written back in place.  Segments longer than the LDS copy fall
// back to one lane's insertion sort.
constexpr int kSortLds = 2048;

template <class T>
__global__ __launch_bounds__(kWave) void k_sort_segments(int nseg, const long long* __restrict__ off,
                                                         T* __restrict__ items) {
    __shared__ T buf[kSortLds];
    const int seg = blockIdx.x;
    if (seg >= nseg) return;
    const long long lo = off[seg], hi = off[seg + 1];
    const long long n = hi - lo;
    if (n <= 1) return;
    const int lane = threadIdx.x;
    if (n <= kSortLds) {
        const int m = static_cast<int>(n);
        for (int t = lane; t < m; t += kWave) buf[t] = items[lo + t];
        __syncthreads();
        for (int t = lane; t < m; t += kWave) {
            const T v = buf[t];
            int rank = 0;
            for (int u = 0; u < m; ++u) rank += buf[u] < v ? 1 : 0;
            items[lo + rank] = v;
        }
        return;
    }
    if (lane != 0) return;
    for (long long p = lo + 1; p < hi; ++p) {
        const T v = items[p];
        long long q = p - 1;
        while (q >= lo && items[q] > v) {
            items[q + 1] = items[q];
            --q;
        }
        items[q + 1] = v;
    }
}

// inclusive prefix sum over the wave's lanes
__device__ __forceinline__ int wave_inclusive_sum(int x) {
    const int lane = threadIdx.x % kWave;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const int t = __shfl_up(x, d, kWave);
        if (lane >= d) x += t;
    }
    return x;
}

// One wave per receiver, lanes over the stencil bins in the reference's
// dz -> dy -> dx order (neighbor_graph_kokkos.cpp:258-332): each lane scans
// its bin's ascending atom list (d^2 <= rc^2 accepted, the receiver itself at
// zero image excluded); a prefix sum of the lanes' counts gives each lane's
// first output slot, so the edges come out in exactly the sequential order.
// FILL = false counts, FILL = true writes.
constexpr int kVisitWaves = 4;

template <bool FILL>
__global__ __launch_bounds__(kVisitWaves* kWave) void k_neighbor_visit(
    int N, Mat3 cell, BinGrid g, double cut2, const double* __restrict__ wfrac, const double* __restrict__ wpos,
    const int* __restrict__ wrap, const int* __restrict__ abin, const long long* __restrict__ boff,
    const int* __restrict__ batoms, int* __restrict__ counts, const long long* __restrict__ eoff,
    int* __restrict__ sources, std::uint32_t* __restrict__ images, int* __restrict__ shifts,
    double* __restrict__ fxyz) {
    const int rcv = blockIdx.x * kVisitWaves + static_cast<int>(threadIdx.x) / kWave;
    const int lane = threadIdx.x % kWave;
    if (rcv >= N) return;  // the whole wave
    const int rb = abin[rcv];
    const int rx = rb % g.bins[0], ry = (rb / g.bins[0]) % g.bins[1], rz = rb / (g.bins[0] * g.bins[1]);
    const int nx = 2 * g.reach[0] + 1, ny = 2 * g.reach[1] + 1, nz = 2 * g.reach[2] + 1;
    const int nst = nx * ny * nz;
    const double p0 = wpos[3 * rcv], p1 = wpos[3 * rcv + 1], p2 = wpos[3 * rcv + 2];
    long long done = FILL ? eoff[rcv] : 0;
    for (int s0 = 0; s0 < nst; s0 += kWave) {
        const int st = s0 + lane;
        int image[3] = {0, 0, 0};
        long long b0 = 0, b1 = 0;
        if (st < nst) {
            const int ix = st % nx, iy = (st / nx) % ny, iz = st / (nx * ny);
            const int raw_z = rz + iz - g.reach[2], sz = floor_div(raw_z, g.bins[2]), bz = raw_z - sz * g.bins[2];
            const int raw_y = ry + iy - g.reach[1], sy = floor_div(raw_y, g.bins[1]), by = raw_y - sy * g.bins[1];
            const int raw_x = rx + ix - g.reach[0], sx = floor_div(raw_x, g.bins[0]), bx = raw_x - sx * g.bins[0];
            const int sb = (bz * g.bins[1] + by) * g.bins[0] + bx;
            image[0] = sx;
            image[1] = sy;
            image[2] = sz;
            b0 = boff[sb];
            b1 = boff[sb + 1];
        }
        const bool zero_image = image[0] == 0 && image[1] == 0 && image[2] == 0;
        // image displacement of the bin (the same sums the sequential scan forms per pair)
        auto accept = [&](int src) __attribute__((always_inline)) {
            if (src == rcv && zero_image) return false;
            double d2 = 0.0;
            const double rp[3] = {p0, p1, p2};
            for (int c = 0; c < 3; ++c) {
                double d = wpos[3 * src + c] - rp[c];
                for (int ax = 0; ax < 3; ++ax) d += image[ax] * cell.v[3 * ax + c];
                d2 += d * d;
            }
            return !(d2 > cut2);
        };
        int cnt = 0;
        for (long long idx = b0; idx < b1; ++idx) cnt += accept(batoms[idx]) ? 1 : 0;
        const int incl = wave_inclusive_sum(cnt);
        const int wave_total = __shfl(incl, kWave - 1, kWave);
        if (FILL && cnt > 0) {
            long long e = done + (incl - cnt);
            for (long long idx = b0; idx < b1; ++idx) {
                const int src = batoms[idx];
                if (!accept(src)) continue;
                sources[e] = src;
                images[e] = (static_cast<std::uint32_t>(image[0]) & 0xffu) |
                            ((static_cast<std::uint32_t>(image[1]) & 0xffu) << 8) |
                            ((static_cast<std::uint32_t>(image[2]) & 0xffu) << 16);
                if (shifts) {
                    for (int ax = 0; ax < 3; ++ax) {
                        shifts[3 * e + ax] = image[ax] - wrap[3 * src + ax] + wrap[3 * rcv + ax];
                        fxyz[3 * e + ax] = wfrac[3 * src + ax] - wfrac[3 * rcv + ax] + image[ax];
                    }
                }
                ++e;
            }
        }
        done += wave_total;
    }
    if (!FILL && lane == 0) counts[rcv] = static_cast<int>(done);
}

// ---------------------------------------------------------------------------
// Edge schedules: receiver of each edge, source transpose (edges ordered by
// source, ascending edge id) -- lifecycle.cpp:3605-3823.
// ---------------------------------------------------------------------------
template <class Off>
__global__ void k_receivers(int N, const Off* __restrict__ off, int* __restrict__ receivers) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N) return;
    for (long long e = off[i]; e < off[i + 1]; ++e) receivers[e] = i;
}

__global__ void k_count_sources(long long E, const int* __restrict__ sources, int* __restrict__ counts) {
    const long long e = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= E) return;
    atomicAdd(&counts[sources[e]], 1);
}

__global__ void k_fill_sources(long long E, const int* __restrict__ sources, int* __restrict__ cursor,
                               int* __restrict__ sedges) {
    const long long e = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const int slot = atomicAdd(&cursor[sources[e]], 1);
    sedges[slot] = static_cast<int>(e);
}

// the same with 64-bit slots and edge ids (graphs beyond 2^31 edges)
__global__ void k_fill_sources_wide(long long E, const int* __restrict__ sources,
                                    unsigned long long* __restrict__ cursor, long long* __restrict__ sedges) {
    const long long e = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const unsigned long long slot = atomicAdd(&cursor[sources[e]], 1ull);
    sedges[slot] = e;
}

__global__ void k_gather_int(long long n, const int* __restrict__ idx, const int* __restrict__ table,
                             int* __restrict__ out) {
    const long long e = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e < n) out[e] = table[idx[e]];
}

__global__ void k_copy_i64_i32_plus(const long long* __restrict__ in, int* __restrict__ out, int n) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx <= n) out[idx] = static_cast<int>(in[idx]);
}

// ---------------------------------------------------------------------------
// Prepared geometry (lifecycle.cpp:2915-3079)
// ---------------------------------------------------------------------------
// Per-atom displacement from the geometry reference
// (mace_kokkos_factorized_lifecycle.cpp:2975-3006): the reference position is
// ref (Cartesian) or ref . cell (fractional reference); delta = pos - reference;
// without periodicity the displacement is delta, otherwise delta in lattice
// coordinates with the periodic components wrapped to [-1/2, 1/2), back in
// Cartesian coordinates.
__global__ void k_displacements(int N, Mat3 cell, Mat3 inv, int pbc_mask, int ref_fractional,
                                const double* __restrict__ ref, const double* __restrict__ pos,
                                double* __restrict__ disp, int* __restrict__ invalid) {
    const int a = blockIdx.x * blockDim.x + threadIdx.x;
    if (a == 0) *invalid = 0;  // the edge pass that follows counts into it
    if (a >= N) return;
    double delta[3], f[3];
    for (int c = 0; c < 3; ++c) {
        double reference = ref[3 * a + c];
        if (ref_fractional) {
            reference = 0.0;
            for (int lat = 0; lat < 3; ++lat) reference += ref[3 * a + lat] * cell.v[3 * lat + c];
        }
        delta[c] = pos[3 * a + c] - reference;
    }
    if (pbc_mask == 0) {
        for (int c = 0; c < 3; ++c) disp[3 * a + c] = delta[c];
        return;
    }
    for (int lat = 0; lat < 3; ++lat) {
        f[lat] = 0.0;
        for (int c = 0; c < 3; ++c) f[lat] += delta[c] * inv.v[3 * c + lat];
        if (pbc_mask & (1 << lat)) f[lat] -= floor(f[lat] + 0.5);
    }
    for (int c = 0; c < 3; ++c) {
        double v = 0.0;
        for (int lat = 0; lat < 3; ++lat) v += f[lat] * cell.v[3 * lat + c];
        disp[3 * a + c] = v;
    }
}

__device__ __forceinline__ int image_component(std::uint32_t packed, int ax) {
    return static_cast<int>(static_cast<std::int8_t>((packed >> (8 * ax)) & 0xffu));
}

// Edges [e0, e0+ne): the edge's reference vector, then
// xyz = reference + disp[src] - disp[rcv], r = |xyz| clamped to the cutoff
// with xyz scaled to it (lifecycle.cpp:3009-3048, 1860-1880).  References:
//   device_fractional: (wfrac[src] - wfrac[rcv] + image) . cell, the
//                      fractional edge vector the neighbour list formed;
//   cartesian:         ref_edges[e];
//   fractional:        ref_edges[e] . cell;
//   shifts:            ref_pos[src] - ref_pos[rcv] + shift_e . cell.
__global__ void k_edge_xyz(long long e0, long long ne, int kind, Mat3 cell, const int* __restrict__ receivers,
                           const int* __restrict__ sources, const double* __restrict__ wfrac,
                           const std::uint32_t* __restrict__ images, const double* __restrict__ ref_pos,
                           const double* __restrict__ ref_edges, const int* __restrict__ shifts,
                           const double* __restrict__ disp, double cutoff, double* __restrict__ xyz,
                           double* __restrict__ r, int* __restrict__ invalid) {
    const long long le = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (le >= ne) return;
    const long long e = e0 + le;
    const int rc = receivers[e], sc = sources[e];
    double vec[3], d2 = 0.0;
    if (kind == kGeometryDeviceFractional) {
        const std::uint32_t img = images[e];
        double fr[3];
        for (int ax = 0; ax < 3; ++ax) fr[ax] = wfrac[3 * sc + ax] - wfrac[3 * rc + ax] + image_component(img, ax);
        for (int c = 0; c < 3; ++c) {
            double ref = 0.0;
            for (int lat = 0; lat < 3; ++lat) ref += fr[lat] * cell.v[3 * lat + c];
            vec[c] = ref + disp[3 * sc + c] - disp[3 * rc + c];
            d2 += vec[c] * vec[c];
        }
    } else {
        for (int c = 0; c < 3; ++c) {
            double ref;
            if (kind == kGeometryShifts) {
                ref = ref_pos[3 * sc + c] - ref_pos[3 * rc + c];
                for (int lat = 0; lat < 3; ++lat)
                    ref += static_cast<double>(shifts[3 * e + lat]) * cell.v[3 * lat + c];
            } else if (kind == kGeometryFractional) {
                ref = 0.0;
                for (int lat = 0; lat < 3; ++lat) ref += ref_edges[3 * e + lat] * cell.v[3 * lat + c];
            } else {
                ref = ref_edges[3 * e + c];
            }
            vec[c] = ref + disp[3 * sc + c] - disp[3 * rc + c];
            d2 += vec[c] * vec[c];
        }
    }
    if (!isfinite(d2) || !(d2 > 0.0)) {
        atomicAdd(invalid, 1);
        xyz[3 * le] = cutoff;
        xyz[3 * le + 1] = 0.0;
        xyz[3 * le + 2] = 0.0;
        r[le] = cutoff;
        return;
    }
    const double dist = sqrt(d2);
    const double scale = dist >= cutoff ? cutoff / dist : 1.0;
    for (int c = 0; c < 3; ++c) xyz[3 * le + c] = scale * vec[c];
    r[le] = dist >= cutoff ? cutoff : dist;
}

// Touched-source sets of a tile: mark, count per 32-bit word, compact.
__global__ void k_mark_sources(long long e0, long long ne, const int* __restrict__ sources,
                               std::uint32_t* __restrict__ bitmap) {
    const long long le = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (le >= ne) return;
    const int src = sources[e0 + le];
    atomicOr(&bitmap[src >> 5], 1u << (src & 31));
}

__global__ void k_word_counts(int words, const std::uint32_t* __restrict__ bitmap, int* __restrict__ counts) {
    const int w = blockIdx.x * blockDim.x + threadIdx.x;
    if (w < words) counts[w] = __popc(bitmap[w]);
}

__global__ void k_compact_bits(int words, const std::uint32_t* __restrict__ bitmap,
                               const long long* __restrict__ word_off, int* __restrict__ out) {
    const int w = blockIdx.x * blockDim.x + threadIdx.x;
    if (w >= words) return;
    std::uint32_t b = bitmap[w];
    long long o = word_off[w];
    while (b) {
        const int bit = __ffs(b) - 1;
        out[o++] = (w << 5) + bit;
        b &= b - 1u;
    }
}

// ---------------------------------------------------------------------------
// Per-edge records: spline point, Y, dY/dxyz, unit direction
// ---------------------------------------------------------------------------
// One thread per edge builds its record in LDS; the workgroup then writes
// its contiguous block of records with coalesced float4 stores (a record per
// lane written directly strides 288 B between lanes).
constexpr int kRecordThreads = 128;

// Spline evaluation point of an edge of length rf (cubic_spline_set.cpp:
// 33-46): the interval, clamped to the table, and the offset in it.
__device__ __forceinline__ int spline_point(float rf, float x0, float h, int intervals, float& xloc) {
    int interval = static_cast<int>(floorf((rf - x0) / h));
    xloc = rf - x0 - h * static_cast<float>(interval);
    if (interval < 0) {
        interval = 0;
        xloc = 0.0f;
    } else if (interval >= intervals) {
        interval = intervals - 1;
        xloc = h;
    }
    return interval;
}

// table row of edge e (the pair's block of intervals, one block without
// per-pair tables), or INT_MAX for an inactive edge
__device__ __forceinline__ int edge_row(const double* __restrict__ r, const int* __restrict__ edge_pair,
                                        long long e, double r_cut, float x0, float h, int intervals) {
    const double re = r[e];
    if (!(re < r_cut)) return INT_MAX;
    float xloc;
    const int interval = spline_point(static_cast<float>(re), x0, h, intervals, xloc);
    return (edge_pair ? edge_pair[e] * intervals : 0) + interval;
}

// One wave (workgroup) per receiver: each lane ranks its edges (lane, lane
// + 64, ...) against all of the receiver's edges.  Order: (row, position); a
// rank is a slot of the receiver's segment.  The rows of up to kOrderStage
// edges are staged in LDS (padded to whole int4s with inactive rows, which
// rank after every edge) and read back four at a time; a longer segment
// reads them from the edge lengths.
constexpr int kOrderStage = 512;
__global__ __launch_bounds__(64) void k_execution_order(int r0, long long e0, const int* __restrict__ offsets,
                                                        const double* __restrict__ r, double r_cut, float x0,
                                                        float h, int intervals, const int* __restrict__ edge_pair,
                                                        int* __restrict__ exec) {
    __shared__ int4 rows4[kOrderStage / 4];
    int* rows = reinterpret_cast<int*>(rows4);
    const int li = blockIdx.x;
    const int lane = threadIdx.x;
    const long long ea = offsets[r0 + li] - e0;
    const int n = offsets[r0 + li + 1] - offsets[r0 + li];
    if (n <= kOrderStage) {
        const int n4 = (n + 3) & ~3;
        for (int j = lane; j < n4; j += 64)
            rows[j] = j < n ? edge_row(r, edge_pair, ea + j, r_cut, x0, h, intervals) : INT_MAX;
        __syncthreads();
        for (int j0 = 0; j0 < n; j0 += 64) {
            const int j = j0 + lane;
            const int kj = j < n ? rows[j] : INT_MAX;
            int rank = 0;
            for (int m = 0; m < n4; m += 4) {
                const int4 q = rows4[m >> 2];
                rank += (q.x < kj || (q.x == kj && m < j)) ? 1 : 0;
                rank += (q.y < kj || (q.y == kj && m + 1 < j)) ? 1 : 0;
                rank += (q.z < kj || (q.z == kj && m + 2 < j)) ? 1 : 0;
                rank += (q.w < kj || (q.w == kj && m + 3 < j)) ? 1 : 0;
            }
            if (j < n) exec[ea + rank] = static_cast<int>(ea + j);
        }
        return;
    }
    for (int j0 = 0; j0 < n; j0 += 64) {
        const int j = j0 + lane;
        const int kj = j < n ? edge_row(r, edge_pair, ea + j, r_cut, x0, h, intervals) : INT_MAX;
        int rank = 0;
        for (int m = 0; m < n; ++m) {
            const int km = edge_row(r, edge_pair, ea + m, r_cut, x0, h, intervals);
            rank += (km < kj || (km == kj && m < j)) ? 1 : 0;
        }
        if (j < n) exec[ea + rank] = static_cast<int>(ea + j);
    }
}

template <int LMAX>
__global__ __launch_bounds__(kRecordThreads) void k_edge_records(long long E, const double* __restrict__ xyz,
                                                                 const double* __restrict__ r, double r_cut,
                                                                 float x0, float h, int intervals,
                                                                 const int* __restrict__ edge_pair,
                                                                 const int* __restrict__ exec,
                                                                 const int* __restrict__ neigh,
                                                                 const int* __restrict__ neigh_types,
                                                                 float* __restrict__ erec,
                                                                 float* __restrict__ erec_b) {
    using S = Shape<LMAX, 0>;
    static_assert(S::REC_F % 4 == 0 && S::REC_B % 4 == 0, "record parts are whole float4s");
    static_assert(S::REC_U + 3 < S::REC, "the reverse part has a free field for the edge's row");
    __shared__ float4 stage[kRecordThreads * S::REC / 4];
    const long long base = static_cast<long long>(blockIdx.x) * kRecordThreads;
    const long long slot = base + threadIdx.x;
    float* rec = reinterpret_cast<float*>(stage) + threadIdx.x * S::REC;
    if (slot < E) {
        const long long e = exec ? exec[slot] : slot;
        const double re = r[e];
        if (!(re < r_cut)) {
            for (int q = 0; q < S::REC; ++q) rec[q] = 0.0f;
        } else {
            float d[3];
            for (int c = 0; c < 3; ++c) d[c] = static_cast<float>(xyz[3 * e + c] / re);
            const float rf = static_cast<float>(re);
            float xloc;
            const int interval = spline_point(rf, x0, h, intervals, xloc);
            rec[0] = xloc;
            rec[1] = __int_as_float((edge_pair ? edge_pair[e] * intervals : 0) + interval);
            rec[2] = __int_as_float(neigh_types[e] + 1);
            rec[3] = __int_as_float(neigh[e]);
            edge_harmonics<LMAX>(d, rf, rec + S::REC_Y, rec + S::REC_DY);
            rec[S::REC_U] = d[0];
            rec[S::REC_U + 1] = d[1];
            rec[S::REC_U + 2] = d[2];
            for (int q = S::REC_U + 3; q < S::REC; ++q) rec[q] = 0.0f;
        }
        rec[S::REC - 1] = __int_as_float(static_cast<int>(e));
    }
    __syncthreads();
    // the two parts to their arrays, coalesced float4 rows
    constexpr int R4 = S::REC / 4, F4 = S::REC_F / 4, B4 = S::REC_B / 4;
    const long long count = E - base < kRecordThreads ? E - base : kRecordThreads;
    float4* dst = reinterpret_cast<float4*>(erec + base * S::REC_F);
    for (int q = threadIdx.x; q < count * F4; q += kRecordThreads) dst[q] = stage[(q / F4) * R4 + q % F4];
    float4* dstb = reinterpret_cast<float4*>(erec_b + base * S::REC_B);
    for (int q = threadIdx.x; q < count * B4; q += kRecordThreads) dstb[q] = stage[(q / B4) * R4 + F4 + q % B4];
}

// Symmetric pair index over the active types (a <= b: a(2n-a-1)/2 + b,
// mace.cpp:216-229); an edge whose types are not active is counted in bad.
__global__ void k_edge_pairs(long long E, const int* __restrict__ receivers, const int* __restrict__ node_types,
                             const int* __restrict__ neigh_types, const int* __restrict__ type_to_active, int n,
                             int* __restrict__ edge_pair, int* __restrict__ bad) {
    const long long e = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const int a = type_to_active[node_types[receivers[e]]], b = type_to_active[neigh_types[e]];
    if (a < 0 || b < 0) {
        atomicAdd(bad, 1);
        edge_pair[e] = 0;
        return;
    }
    edge_pair[e] = a <= b ? a * (2 * n - a - 1) / 2 + b : b * (2 * n - b - 1) / 2 + a;
}

Mat3 mat3(const double* p) {
    Mat3 m;
    for (int i = 0; i < 9; ++i) m.v[i] = p[i];
    return m;
}

template <class T>
T* dev_alloc(std::size_t n) {
    void* p = nullptr;
    SMX_HIP(hipMalloc(&p, std::max<std::size_t>(1, n) * sizeof(T)));
    return static_cast<T*>(p);
}

}  // namespace

std::int64_t device_exclusive_scan(const int* in, long long* out, int n, hipStream_t s) {
    const int tiles = std::max(1, (n + kScanTile - 1) / kScanTile);
    long long* sums = dev_alloc<long long>(tiles + 1);
    k_scan_tiles<<<tiles, kScanThreads, 0, s>>>(in, out, n, sums);
    SMX_LAUNCH_CHECK("scan_tiles");
    k_scan_tile_sums<<<1, 1024, 0, s>>>(sums, tiles);
    SMX_LAUNCH_CHECK("scan_tile_sums");
    k_scan_add<<<blocks_for(std::max(n, 1), kScanThreads), kScanThreads, 0, s>>>(out, n, sums, tiles);
    SMX_LAUNCH_CHECK("scan_add");
    long long total = 0;
    SMX_HIP(hipMemcpyAsync(&total, out + n, sizeof(long long), hipMemcpyDeviceToHost, s));
    SMX_HIP(hipStreamSynchronize(s));
    SMX_HIP(hipFree(sums));
    return total;
}

void build_neighbor_list(int N, const double* positions_host, const double* cell_host, const double* inv_host,
                         double cutoff, bool with_shifts, NeighborResult& out, hipStream_t s, bool wide) {
    if (!std::isfinite(cutoff) || !(cutoff > 0.0)) throw std::invalid_argument("neighbor cutoff must be positive");
    if (N < 0) throw std::invalid_argument("negative atom count");
    for (int i = 0; i < 3 * N; ++i)
        if (!std::isfinite(positions_host[i])) throw std::invalid_argument("positions must be finite");
    for (int row = 0; row < 3; ++row)
        for (int col = 0; col < 3; ++col) {
            double prod = 0.0;
            for (int k = 0; k < 3; ++k) prod += cell_host[3 * row + k] * inv_host[3 * k + col];
            if (std::abs(prod - (row == col ? 1.0 : 0.0)) > 1e-9)
                throw std::invalid_argument("cell and inverse cell are inconsistent");
        }
    BinGrid g;
    for (int ax = 0; ax < 3; ++ax) {
        double ins = 0.0;
        for (int c = 0; c < 3; ++c) ins += inv_host[3 * c + ax] * inv_host[3 * c + ax];
        if (!(ins > 0.0)) throw std::invalid_argument("cell must be invertible");
        const double face = 1.0 / std::sqrt(ins);
        g.bins[ax] = std::max(1, static_cast<int>(std::floor(face / cutoff)));
        const double rch = std::ceil(cutoff * std::sqrt(ins) * g.bins[ax]) + 1.0;
        g.reach[ax] = std::max(1, static_cast<int>(rch));
    }
    const long long nb_ll = static_cast<long long>(g.bins[0]) * g.bins[1] * g.bins[2];
    if (nb_ll > INT_MAX / 2) throw std::invalid_argument("neighbor bin grid is too large");
    // images are stored as signed bytes: |image| <= reach + 1
    for (int ax = 0; ax < 3; ++ax)
        if (g.reach[ax] + 1 > 127) throw std::invalid_argument("cell is too small for the cutoff (image range)");
    const int nb = static_cast<int>(nb_ll);
    const Mat3 cell = mat3(cell_host), inv = mat3(inv_host);
    const double cut2 = cutoff * cutoff;

    double* d_pos = dev_alloc<double>(3 * static_cast<std::size_t>(N));
    double* wfrac = dev_alloc<double>(3 * static_cast<std::size_t>(N));
    out.wfrac = wfrac;  // kept: the geometry reference of the graph
    double* wpos = dev_alloc<double>(3 * static_cast<std::size_t>(N));
    int* wrap = dev_alloc<int>(3 * static_cast<std::size_t>(N));
    int* abin = dev_alloc<int>(N);
    int* bsize = dev_alloc<int>(nb);
    long long* boff = dev_alloc<long long>(nb + 1);
    int* cursor = dev_alloc<int>(nb);
    int* batoms = dev_alloc<int>(N);
    int* counts = dev_alloc<int>(N);
    long long* eoff = dev_alloc<long long>(N + 1);
    auto release = [&]() {
        for (void* p : {static_cast<void*>(d_pos), static_cast<void*>(wpos),
                        static_cast<void*>(wrap), static_cast<void*>(abin), static_cast<void*>(bsize),
                        static_cast<void*>(boff), static_cast<void*>(cursor), static_cast<void*>(batoms),
                        static_cast<void*>(counts), static_cast<void*>(eoff)})
            (void)hipFree(p);
        eoff = nullptr;
    };
    try {
        SMX_HIP(hipMemcpyAsync(d_pos, positions_host, 3 * sizeof(double) * N, hipMemcpyHostToDevice, s));
        SMX_HIP(hipMemsetAsync(bsize, 0, sizeof(int) * nb, s));
        const unsigned ab = blocks_for(std::max(N, 1), 256);
        if (N > 0) {
            k_wrap<<<ab, 256, 0, s>>>(N, d_pos, cell, inv, g, wfrac, wpos, wrap, abin, bsize);
            SMX_LAUNCH_CHECK("neighbor_wrap");
        }
        device_exclusive_scan(bsize, boff, nb, s);
        k_i64_to_i32<<<blocks_for(nb, 256), 256, 0, s>>>(boff, cursor, nb);
        SMX_LAUNCH_CHECK("neighbor_cursor");
        if (N > 0) {
            k_bin_fill<<<ab, 256, 0, s>>>(N, abin, cursor, batoms);
            SMX_LAUNCH_CHECK("neighbor_bin_fill");
        }
        k_sort_segments<<<nb, kWave, 0, s>>>(nb, boff, batoms);
        SMX_LAUNCH_CHECK("neighbor_sort_bins");
        const unsigned vb = blocks_for(std::max(N, 1), kVisitWaves);
        if (N > 0) {
            k_neighbor_visit<false><<<vb, kVisitWaves * kWave, 0, s>>>(N, cell, g, cut2, wfrac, wpos, wrap, abin, boff,
                                                                       batoms, counts, nullptr, nullptr, nullptr,
                                                                       nullptr, nullptr);
            SMX_LAUNCH_CHECK("neighbor_count");
        }
        const long long E = device_exclusive_scan(counts, eoff, N, s);
        if (E > (wide ? kMaxWideEdges : kMaxEdges))
            throw std::length_error(wide ? "neighbor edge count exceeds the tiled plan's edge limit"
                                         : "neighbor edge count exceeds the 32-bit graph limit");
        out.num_edges = E;
        out.num_neigh = dev_alloc<int>(N);
        out.sources = dev_alloc<int>(E);
        out.images = dev_alloc<std::uint32_t>(E);
        if (with_shifts) {
            out.shifts = dev_alloc<int>(3 * static_cast<std::size_t>(E));
            out.fractional_xyz = dev_alloc<double>(3 * static_cast<std::size_t>(E));
        }
        SMX_HIP(hipMemcpyAsync(out.num_neigh, counts, sizeof(int) * N, hipMemcpyDeviceToDevice, s));
        if (E <= kMaxEdges) {
            out.offsets = dev_alloc<int>(N + 1);
            k_copy_i64_i32_plus<<<blocks_for(N + 1, 256), 256, 0, s>>>(eoff, out.offsets, N);
            SMX_LAUNCH_CHECK("neighbor_offsets");
        }
        if (N > 0 && E > 0) {
            k_neighbor_visit<true><<<vb, kVisitWaves * kWave, 0, s>>>(N, cell, g, cut2, wfrac, wpos, wrap, abin, boff,
                                                                      batoms, nullptr, eoff, out.sources, out.images,
                                                                      out.shifts, out.fractional_xyz);
            SMX_LAUNCH_CHECK("neighbor_fill");
        }
        SMX_HIP(hipStreamSynchronize(s));
        if (wide) {
            out.offsets64 = eoff;  // the caller's now
            eoff = nullptr;
        }
    } catch (...) {
        release();
        throw;
    }
    release();
}

void launch_transpose(int K, std::int64_t E, const int* keys, int* koff, int* kedges, int* scratch_counts,
                      hipStream_t s) {
    if (K == 0) return;
    SMX_HIP(hipMemsetAsync(scratch_counts, 0, sizeof(int) * K, s));
    if (E > 0) {
        k_count_sources<<<blocks_for(E, 256), 256, 0, s>>>(E, keys, scratch_counts);
        SMX_LAUNCH_CHECK("transpose_count");
    }
    long long* off64 = dev_alloc<long long>(K + 1);
    try {
        device_exclusive_scan(scratch_counts, off64, K, s);
        k_copy_i64_i32_plus<<<blocks_for(K + 1, 256), 256, 0, s>>>(off64, koff, K);
        SMX_LAUNCH_CHECK("transpose_offsets");
        k_i64_to_i32<<<blocks_for(K, 256), 256, 0, s>>>(off64, scratch_counts, K);
        SMX_LAUNCH_CHECK("transpose_cursor");
        if (E > 0) {
            k_fill_sources<<<blocks_for(E, 256), 256, 0, s>>>(E, keys, scratch_counts, kedges);
            SMX_LAUNCH_CHECK("transpose_fill");
        }
        k_sort_segments<<<K, kWave, 0, s>>>(K, off64, kedges);
        SMX_LAUNCH_CHECK("transpose_sort");
        SMX_HIP(hipStreamSynchronize(s));
    } catch (...) {
        (void)hipFree(off64);
        throw;
    }
    SMX_HIP(hipFree(off64));
}

void launch_transpose(int K, std::int64_t E, const int* keys, long long* koff, long long* kedges, int* scratch_counts,
                      hipStream_t s) {
    if (K == 0) return;
    SMX_HIP(hipMemsetAsync(scratch_counts, 0, sizeof(int) * K, s));
    if (E > 0) {
        k_count_sources<<<blocks_for(E, 256), 256, 0, s>>>(E, keys, scratch_counts);
        SMX_LAUNCH_CHECK("transpose_count");
    }
    device_exclusive_scan(scratch_counts, koff, K, s);
    if (E > 0) {
        // each key's write cursor starts at its segment
        unsigned long long* cursor = dev_alloc<unsigned long long>(K);
        try {
            SMX_HIP(hipMemcpyAsync(cursor, koff, sizeof(long long) * K, hipMemcpyDeviceToDevice, s));
            k_fill_sources_wide<<<blocks_for(E, 256), 256, 0, s>>>(E, keys, cursor, kedges);
            SMX_LAUNCH_CHECK("transpose_fill");
            SMX_HIP(hipStreamSynchronize(s));
        } catch (...) {
            (void)hipFree(cursor);
            throw;
        }
        SMX_HIP(hipFree(cursor));
    }
    k_sort_segments<<<K, kWave, 0, s>>>(K, koff, kedges);
    SMX_LAUNCH_CHECK("transpose_sort");
    SMX_HIP(hipStreamSynchronize(s));
}

void launch_receivers(int N, const int* offsets, int* receivers, hipStream_t s) {
    if (N == 0) return;
    k_receivers<<<blocks_for(N, 256), 256, 0, s>>>(N, offsets, receivers);
    SMX_LAUNCH_CHECK("graph_receivers");
}

void launch_receivers(int N, const long long* offsets, int* receivers, hipStream_t s) {
    if (N == 0) return;
    k_receivers<<<blocks_for(N, 256), 256, 0, s>>>(N, offsets, receivers);
    SMX_LAUNCH_CHECK("graph_receivers");
}

void launch_graph_schedule(int N, int F, std::int64_t E, const int* offsets, const int* sources, int* receivers,
                           int* soff, int* sedges, int* scratch_counts, hipStream_t s) {
    launch_receivers(N, offsets, receivers, s);
    launch_transpose(F, E, sources, soff, sedges, scratch_counts, s);
}

__global__ void k_count_invalid_edges(std::int64_t E, const double* __restrict__ xyz, const double* __restrict__ r,
                                      int* __restrict__ invalid) {
    const std::int64_t e = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const double d = r[e];
    if (!isfinite(d) || !(d > 0.0) || !isfinite(xyz[3 * e]) || !isfinite(xyz[3 * e + 1]) || !isfinite(xyz[3 * e + 2]))
        atomicAdd(invalid, 1);
}

void launch_count_invalid_edges(std::int64_t E, const double* xyz, const double* r, int* invalid, hipStream_t s) {
    if (E == 0) return;
    k_count_invalid_edges<<<blocks_for(E, 256), 256, 0, s>>>(E, xyz, r, invalid);
    SMX_LAUNCH_CHECK("count_invalid_edges");
}

void launch_edge_pairs(std::int64_t E, const int* receivers, const int* node_types, const int* neigh_types,
                       const int* type_to_active, int active_types, int* edge_pair, int* bad, hipStream_t s) {
    if (E == 0) return;
    k_edge_pairs<<<blocks_for(E, 256), 256, 0, s>>>(E, receivers, node_types, neigh_types, type_to_active,
                                                    active_types, edge_pair, bad);
    SMX_LAUNCH_CHECK("edge_pairs");
}

void launch_gather_types(std::int64_t E, const int* sources, const int* node_types, int* neigh_types,
                         hipStream_t s) {
    if (E == 0) return;
    k_gather_int<<<blocks_for(E, 256), 256, 0, s>>>(E, sources, node_types, neigh_types);
    SMX_LAUNCH_CHECK("gather_types");
}

void launch_displacements(int N, const double* cell, const double* inv_cell, const int pbc[3], bool ref_fractional,
                          const double* reference_positions, const double* positions, double* disp, int* invalid,
                          hipStream_t s) {
    const int mask = (pbc[0] ? 1 : 0) | (pbc[1] ? 2 : 0) | (pbc[2] ? 4 : 0);
    k_displacements<<<blocks_for(std::max(N, 1), 256), 256, 0, s>>>(
        N, mat3(cell), mat3(inv_cell), mask, ref_fractional ? 1 : 0, reference_positions, positions, disp, invalid);
    SMX_LAUNCH_CHECK("geometry_displacements");
}

void launch_edge_xyz(std::int64_t e0, std::int64_t ne, const EdgeReference& ref, const double* cell,
                     const int* receivers, const int* sources, const double* disp, double cutoff, double* xyz,
                     double* r, int* invalid, hipStream_t s) {
    if (ne == 0) return;
    k_edge_xyz<<<blocks_for(ne, 256), 256, 0, s>>>(e0, ne, ref.kind, mat3(cell), receivers, sources, ref.wfrac,
                                                   ref.images, ref.positions, ref.edges, ref.shifts, disp, cutoff,
                                                   xyz, r, invalid);
    SMX_LAUNCH_CHECK("geometry_edges");
}

int build_touched_sources(int N, std::int64_t e0, std::int64_t ne, const int* sources, std::uint32_t* bitmap,
                          int* word_counts, int* out, hipStream_t s) {
    const int words = N / 32 + 1;
    SMX_HIP(hipMemsetAsync(bitmap, 0, sizeof(std::uint32_t) * words, s));
    if (ne > 0) {
        k_mark_sources<<<blocks_for(ne, 256), 256, 0, s>>>(e0, ne, sources, bitmap);
        SMX_LAUNCH_CHECK("touched_mark");
    }
    k_word_counts<<<blocks_for(words, 256), 256, 0, s>>>(words, bitmap, word_counts);
    SMX_LAUNCH_CHECK("touched_count");
    long long* off = dev_alloc<long long>(words + 1);
    long long total = 0;
    try {
        total = device_exclusive_scan(word_counts, off, words, s);
        k_compact_bits<<<blocks_for(words, 256), 256, 0, s>>>(words, bitmap, off, out);
        SMX_LAUNCH_CHECK("touched_compact");
        SMX_HIP(hipStreamSynchronize(s));
    } catch (...) {
        (void)hipFree(off);
        throw;
    }
    SMX_HIP(hipFree(off));
    return static_cast<int>(total);
}

void launch_execution_order(int r0, int nr, std::int64_t e0, const int* offsets, const double* r, double r_cut,
                            float x0, float h, int intervals, const int* edge_pair, int* exec, hipStream_t s) {
    if (nr == 0) return;
    k_execution_order<<<nr, 64, 0, s>>>(r0, e0, offsets, r, r_cut, x0, h, intervals, edge_pair, exec);
    SMX_LAUNCH_CHECK("execution_order");
}

void geometry_records(int l_max, std::int64_t E, const double* xyz, const double* r, double r_cut, float x0, float h,
                      int intervals, const int* edge_pair, const int* exec, const int* neigh, const int* neigh_types,
                      float* erec, float* erec_b, hipStream_t s) {
    if (E == 0) return;
    if (l_max == 3)
        k_edge_records<3><<<blocks_for(E, kRecordThreads), kRecordThreads, 0, s>>>(
            E, xyz, r, r_cut, x0, h, intervals, edge_pair, exec, neigh, neigh_types, erec, erec_b);
    else if (l_max == 2)
        k_edge_records<2><<<blocks_for(E, kRecordThreads), kRecordThreads, 0, s>>>(
            E, xyz, r, r_cut, x0, h, intervals, edge_pair, exec, neigh, neigh_types, erec, erec_b);
    else
        throw std::invalid_argument("edge records are compiled for l_max 2 and 3");
    SMX_LAUNCH_CHECK("edge_records");
}

}  // namespace smx
