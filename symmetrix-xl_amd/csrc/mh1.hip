// MH-1 (MACE_Nonlinear) evaluator on MI355X: HIP kernels, the evaluation
// schedule and the C ABI of include/symmetrix_mh1.h.
//
// Reference: libsymmetrix/source/mace_nonlinear.cpp:471-1010 (one
// compute_node_energies_forces call: harmonics, radial features, per layer
// the up/residual/skip linears, the conditioned edge MLPs, the "uvu"
// convolution summed into receivers, the density normalisation, gate,
// linear_2, product basis; readouts and energies; then the reverse pass to
// per-edge forces) and its Kokkos form mace_nonlinear_kokkos_impl.tpp.
//
// MI355X layout (FP32 arithmetic, FP64 energies and forces):
// * node rows [N][dim] in the irreps layout of each linear; one thread per
//   (node, output element) for the linears, which walk the instruction
//   table of their output block (adjacent threads read adjacent weights and
//   the same input row);
// * edge MLPs over tiles of edges in LDS (radial features formed in the
//   tile, the first layer's embedding columns read as per-type rows); the
//   reverse re-runs the tile forward and keeps each layer's input in LDS;
// * the convolution: one thread per (receiver, channel), the receiver's
//   edges streamed in CSR order, each thread's output components accumulated
//   in its own LDS column (no atomics: the sum over a receiver's edges is a
//   sequential loop, so results are run-to-run identical); the reverse
//   writes per-edge weight adjoints and first-input adjoints, reduces the
//   harmonic adjoints over the channel lanes with butterflies, and a gather
//   over the source transpose sums the first-input adjoints per source;
// * the product basis: one thread per (node, channel) walking the compiled
//   monomial terms, the channel's angular components in LDS.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <numeric>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "../../include/symmetrix_mh1.h"
#include "device_common.hpp"
#include "harmonics.hpp"
#include "mh1_model.hpp"
#include "mh1_paths.hpp"

namespace smx {
void set_last_error(const std::string& message);  // evaluator.cpp

namespace mh1 {
namespace {

constexpr int kTpThreads = 128;
constexpr std::size_t kMaxLds = 60 * 1024;

// ------------------------------------------------------------- device views

constexpr int kLinearMaxBlocks = 32;

struct DLinear {
    int in_dim, out_dim;
    const int* instr;
    const int* block_first;
    const int* elem;
    const float* W;
    const float* bias;
    const float* out_mask;
    const float* in_mask;
    // output blocks (offset, multiplicity, width) for the MFMA form; nblk 0 when there are more than
    // kLinearMaxBlocks (the per-element kernel runs)
    int nblk;
    int blk_off[kLinearMaxBlocks], blk_mul[kLinearMaxBlocks], blk_d[kLinearMaxBlocks];
};

constexpr int kRegStages = MlpTables::kRegStages;
// 16-edge tiles per wave in the register-form edge MLPs (forward, reverse, first half of a split reverse)
constexpr int kRegTilesFwd = 2, kRegTilesRev = 1, kRegTilesOut = 2;

// A stage of the register form: widths and parameter offsets (see MlpTables::reg_stage).
struct DMlpStage {
    int in, out, w, b, wt, ln;
    float eps;
};

struct DMlp {
    int num_layers, radial, first_width, num_types, width, tape_width;
    const int* layers;
    const float* eps;
    const float* params;
    const float* type_rows;
    const int* wt_offset;    // per layer: transposed weights [in][out] (linear layers)
    const int* tape_offset;  // per layer: output offset in the edge's tape row (-1: last layer)
    int reg_hw, reg_stages;  // register form (reg_hw 0: the LDS-tile kernels run)
    DMlpStage st[kRegStages + 1];  // hidden stages from 0, the final linear at kRegStages
};

// the reverse of a register-form MLP with a wide final linear runs in two kernels
inline bool mlp_split(const DMlp& m) { return m.reg_hw && m.st[kRegStages].out >= 64; }

struct DRadial {
    int nb, p, apply_cutoff, agnesi, num_types;
    double prefactor, r_cut, a, q, pp;
    double bessel[32];
    const double* r0;  // [type][type] Agnesi length
};

struct DTp {
    int channels, in1_dim, out_dim, numel, slots, nin1, num_paths;
    const int* paths;
    const int* in1_slot;
    const int* out_slot;
    const int* entries;
    const float* values;
    int compiled;        // family structure index (mh1_paths.hpp) or -1
    const float* cval;   // its Wigner values x path weight, structure order
};

struct DGate {
    int in_dim, out_dim;
    const int* out_src;
    const int* out_gate;
    const float* out_const;
    const int* in_kind;
    const int* in_out;
    const int* in_aux;
    const int* in_count;
    const float* in_const;
};

struct DProduct {
    int channels, angular, in_dim, out_dim, out_slots, num_terms;
    const int* ang_src;
    const int* out_slot;
    const int* terms;
    const float* coef;
};

struct DZbl {
    int num_types;
    const double* pair;  // [type][type][3]: 1/a, bare prefactor, r_max
    double c[4];
    int p;
};

typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }

// Ends an MFMA chain whose results VALU or memory instructions read next.  A
// read of an MFMA result needs ten wait states after a v_mfma_f32_16x16x4_f32
// (8 passes) on every path.  Where a chain sat in a runtime-conditional block,
// the compiler padded only the fall-through path into the join: the assembly
// showed a read of the last accumulator register right after its MFMA on the
// taken branch (a stale value, no error).  Sixteen wait states after the
// chain, with the scheduler fenced on both sides, cover every path;
// check_mfma_waits.py verifies the generated assembly.
__device__ __forceinline__ void mfma_settle() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 7\n\ts_nop 7");
    __builtin_amdgcn_sched_barrier(0);
}

// ---------------------------------------------------------------- radial

// Bessel features of the (Agnesi-transformed) distance, the polynomial
// envelope applied when apply_cutoff; value and d/dr (mace_nonlinear.cpp:
// 383-449), FP64.
__device__ __forceinline__ void envelope(const DRadial& rd, double r, double& env, double& denv) {
    const double x = r / rd.r_cut;
    const double p = rd.p;
    if (r < rd.r_cut) {
        const double xp = pow(x, p);
        env = 1.0 - 0.5 * (p + 1.0) * (p + 2.0) * xp + p * (p + 2.0) * xp * x - 0.5 * p * (p + 1.0) * xp * x * x;
        const double xm1 = pow(x, p - 1.0);
        denv = (-0.5 * p * (p + 1.0) * (p + 2.0) * xm1 + p * (p + 1.0) * (p + 2.0) * xp -
                0.5 * p * (p + 1.0) * (p + 2.0) * xp * x) / rd.r_cut;
    } else {
        env = 0.0;
        denv = 0.0;
    }
}

__device__ void radial_eval(const DRadial& rd, double r, int ts, int tt, double* f, double* df, double& env,
                            double& denv) {
    envelope(rd, r, env, denv);
    double t = r, dt = 1.0;
    if (rd.agnesi) {
        const double r0 = rd.r0[ts * rd.num_types + tt];
        const double u = r / r0;
        const double us = pow(u, rd.q - rd.pp);
        const double den = 1.0 + us;
        const double g = rd.a * pow(u, rd.q) / den;
        const double dg = rd.a * (rd.q * pow(u, rd.q - 1.0) * den - (rd.q - rd.pp) * pow(u, 2.0 * rd.q - rd.pp - 1.0)) /
                          (den * den);
        t = 1.0 / (1.0 + g);
        dt = -dg / (r0 * (1.0 + g) * (1.0 + g));
    }
    for (int k = 0; k < rd.nb; ++k) {
        const double w = rd.bessel[k];
        double s, c;
        sincos(w * t, &s, &c);
        const double base = rd.prefactor * s / t;
        if (f) f[k] = rd.apply_cutoff ? base * env : base;
        if (df) {
            const double db = rd.prefactor * (w * c * t - s) / (t * t) * dt;
            df[k] = rd.apply_cutoff ? db * env + base * denv : db;
        }
    }
}

// ---------------------------------------------------------------- kernels

// radial features of one edge straight into out[0..nb) (FP64 arithmetic)
__device__ __forceinline__ void radial_features_to(const DRadial& rd, double r, int ts, int tt, float* out) {
    double env, denv;
    envelope(rd, r, env, denv);
    double t = r;
    if (rd.agnesi) {
        const double r0 = rd.r0[ts * rd.num_types + tt];
        const double u = r / r0;
        t = 1.0 / (1.0 + rd.a * pow(u, rd.q) / (1.0 + pow(u, rd.q - rd.pp)));
    }
    for (int k = 0; k < rd.nb; ++k) {
        const double base = rd.prefactor * sin(rd.bessel[k] * t) / t;
        out[k] = static_cast<float>(rd.apply_cutoff ? base * env : base);
    }
}

// Per edge: harmonics, cutoff and the radial features the edge MLPs share.
template <int LMAX>
__global__ __launch_bounds__(256) void k_geometry(long long E, const double* __restrict__ xyz,
                                                  const double* __restrict__ r, const DRadial rd,
                                                  const int* __restrict__ ets, const int* __restrict__ ett,
                                                  float* __restrict__ Y, float* __restrict__ cut,
                                                  float* __restrict__ rad) {
    constexpr int NY = (LMAX + 1) * (LMAX + 1);
    const long long e = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
    if (e >= E) return;
    const float d[3] = {static_cast<float>(xyz[3 * e]), static_cast<float>(xyz[3 * e + 1]),
                        static_cast<float>(xyz[3 * e + 2])};
    float y[NY], g[3 * NY];
    edge_harmonics<LMAX>(d, static_cast<float>(r[e]), y, g);
    for (int q = 0; q < NY; ++q) Y[e * NY + q] = y[q];
    double env = 0.0, denv = 0.0;
    envelope(rd, r[e], env, denv);
    cut[e] = static_cast<float>(env);
    radial_features_to(rd, r[e], ets[e], ett[e], rad + e * rd.nb);
}

// node features of the embedding: one row per type
__global__ __launch_bounds__(256) void k_embed(int N, int dim, const int* __restrict__ types,
                                               const float* __restrict__ table, float* __restrict__ out) {
    const long long t = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
    if (t >= static_cast<long long>(N) * dim) return;
    const int n = static_cast<int>(t / dim), j = static_cast<int>(t % dim);
    out[t] = table[static_cast<std::size_t>(types[n]) * dim + j];
}

// y = (op(x) + bias) * mask (+ addend) (accumulate: y += ...); one thread per
// (node, output element).  The instructions of the element's output block are
// walked in file order (e3nn.cpp:146-166).
__global__ __launch_bounds__(256) void k_linear(const DLinear op, int N, const float* __restrict__ x,
                                                float* __restrict__ y, const float* __restrict__ addend,
                                                int accumulate) {
    const long long t = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
    if (t >= static_cast<long long>(N) * op.out_dim) return;
    const int n = static_cast<int>(t / op.out_dim), j = static_cast<int>(t % op.out_dim);
    const int b = op.elem[3 * j], w = op.elem[3 * j + 1], m = op.elem[3 * j + 2];
    const float* xr = x + static_cast<std::size_t>(n) * op.in_dim;
    float acc = 0.0f;
    for (int q = op.block_first[b]; q < op.block_first[b + 1]; ++q) {
        const int* I = op.instr + 6 * q;
        const int in_off = I[0] + m, mul_in = I[1], d = I[2], mul_out = I[5];
        const float* Wp = op.W + I[3] + w;
        if (op.in_mask) {
            for (int u = 0; u < mul_in; ++u) acc += Wp[u * mul_out] * xr[in_off + u * d] * op.in_mask[in_off + u * d];
        } else {
            for (int u = 0; u < mul_in; ++u) acc += Wp[u * mul_out] * xr[in_off + u * d];
        }
    }
    if (op.bias) acc += op.bias[j];
    if (op.out_mask) acc *= op.out_mask[j];
    if (addend) acc += addend[t];
    if (accumulate)
        y[t] += acc;
    else
        y[t] = acc;
}

// The same linear on MFMA (v_mfma_f32_16x16x4_f32): one workgroup of four
// waves per tile of 16 rows (node, component) x 64 output channels of one
// output block; K runs over the input channels of every instruction into that
// block, every fourth 4-channel step to each wave (the node-count launches are
// a few hundred tiles: split K gives four times the waves and a quarter of the
// serial load-MFMA chain).  The partial tiles meet in LDS and wave w finishes
// columns 16w..16w+15.  Tiles are numbered block by block (rows, then column
// blocks).
__global__ __launch_bounds__(256) void k_linear_mfma(const DLinear op, int N, const float* __restrict__ x,
                                                     float* __restrict__ y, const float* __restrict__ addend,
                                                     int accumulate) {
    __shared__ v4f part[4][4][64];  // [wave][column chunk][lane]
    long long t = blockIdx.x;
    int b = 0;
    for (; b < op.nblk; ++b) {
        const long long cnt = ((static_cast<long long>(N) * op.blk_d[b] + 15) / 16) * ((op.blk_mul[b] + 63) / 64);
        if (t < cnt) break;
        t -= cnt;
    }
    if (b == op.nblk) return;
    const int d = op.blk_d[b], mul = op.blk_mul[b], boff = op.blk_off[b];
    const int ctiles = (mul + 63) / 64;
    const long long R = static_cast<long long>(N) * d;
    const long long row0 = (t / ctiles) * 16;
    const int col0 = static_cast<int>(t % ctiles) * 64;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 15, kg = lane >> 4;
    const long long row = row0 + r;
    const bool rok = row < R;
    const int n = rok ? static_cast<int>(row / d) : 0, m = rok ? static_cast<int>(row % d) : 0;
    v4f acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    for (int q = op.block_first[b]; q < op.block_first[b + 1]; ++q) {
        const int* I = op.instr + 6 * q;
        const int in_off = I[0] + m, mul_in = I[1], w_off = I[3];
        const float* xr = x + static_cast<std::size_t>(n) * op.in_dim + in_off;
        for (int k0 = 4 * wave; k0 < mul_in; k0 += 16) {
            const int u = k0 + kg;
            float a = 0.0f;
            if (rok && u < mul_in) {
                a = xr[u * d];
                if (op.in_mask) a *= op.in_mask[in_off + u * d];
            }
            const float* wr = op.W + w_off + static_cast<std::size_t>(u) * mul;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int c = col0 + 16 * j + r;
                const float bv = (u < mul_in && c < mul) ? wr[c] : 0.0f;
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, bv, acc[j], 0, 0, 0);
            }
        }
    }
    mfma_settle();
#pragma unroll
    for (int j = 0; j < 4; ++j) part[wave][j][lane] = acc[j];
    __syncthreads();
    const int j = wave;
    const int c = col0 + 16 * j + r;
    if (c >= mul) return;
    const v4f sum = (part[0][j][lane] + part[1][j][lane]) + (part[2][j][lane] + part[3][j][lane]);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const long long rr = row0 + 4 * kg + v;
        if (rr >= R) continue;
        const int nn = static_cast<int>(rr / d), mm = static_cast<int>(rr % d);
        const int jo = boff + c * d + mm;
        const std::size_t idx = static_cast<std::size_t>(nn) * op.out_dim + jo;
        float val = sum[v];
        if (op.bias) val += op.bias[jo];
        if (op.out_mask) val *= op.out_mask[jo];
        if (addend) val += addend[idx];
        y[idx] = accumulate ? y[idx] + val : val;
    }
}

// Edge-tile GEMM on MFMA (v_mfma_f32_16x16x4_f32): wave w of the workgroup
// owns rows 16w..16w+15 of the tile; D[row][c] = sum_k A[row][k] B(k, c) with
// A in LDS (row stride lda) or global memory, B(k, c) = B[k * ldb + c] in
// global memory (weights, L1/L2 resident).  Lane l supplies A[l%16][k0+l/16]
// and B(k0+l/16, c0+l%16) and holds D[4(l/16)+v][l%16].  K and the columns are
// padded to the fragment size with zeros, rows from a_rows on read zeros;
// `epi(row, col, value)` stores.
template <class Epi>
__device__ __forceinline__ void tile_gemm(const float* A, int lda, int a_rows, int K, const float* __restrict__ B,
                                          int ldb, int N, Epi epi) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = lane & 15, kg = lane >> 4;
    if ((K & 3) == 0 && (N & 63) == 0 && a_rows >= static_cast<int>(blockDim.x / 4)) {
        // every row valid, K and the columns whole fragments: no predicates, pointer steps only
        const float* arow = A + static_cast<std::size_t>(16 * wave + r) * lda + kg;
        for (int c0 = 0; c0 < N; c0 += 64) {
            v4f acc[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            const float* ap = arow;
            const float* bp = B + static_cast<std::size_t>(kg) * ldb + c0 + r;

            for (int k0 = 0; k0 < K; k0 += 4) {
                const float a = *ap;
                const float b0 = bp[0], b1 = bp[16], b2 = bp[32], b3 = bp[48];
                acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b0, acc[0], 0, 0, 0);
                acc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b1, acc[1], 0, 0, 0);
                acc[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b2, acc[2], 0, 0, 0);
                acc[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b3, acc[3], 0, 0, 0);
                ap += 4;
                bp += 4 * static_cast<std::size_t>(ldb);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int v = 0; v < 4; ++v) epi(16 * wave + 4 * kg + v, c0 + 16 * j + r, acc[j][v]);
        }
        return;
    }
    const bool row_ok = 16 * wave + r < a_rows;
    const float* arow = A + static_cast<std::size_t>(row_ok ? 16 * wave + r : 0) * lda;
    for (int c0 = 0; c0 < N; c0 += 64) {
        v4f acc[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

        for (int k0 = 0; k0 < K; k0 += 4) {
            const int k = k0 + kg;
            const float a = (row_ok && k < K) ? arow[k] : 0.0f;
            const float* brow = B + static_cast<std::size_t>(k) * ldb;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int c = c0 + 16 * j + r;
                const float b = (k < K && c < N) ? brow[c] : 0.0f;
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[j], 0, 0, 0);
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = c0 + 16 * j + r;
            if (c < N) {
#pragma unroll
                for (int v = 0; v < 4; ++v) epi(16 * wave + 4 * kg + v, c, acc[j][v]);
            }
        }
    }
}

// Sum over the four lanes that share a tile row (rows = blockDim / 4).
__device__ __forceinline__ float row4_sum(float v) {
    v += __shfl_xor(v, 1, kWave);
    v += __shfl_xor(v, 2, kWave);
    return v;
}

// Mean and 1/std of each tile row of x (LDS, row stride ld), four lanes per
// row: every lane of the row gets them in mean/rs, lane 0 also stores them.
__device__ __forceinline__ void ln_stats(const float* x, int ld, int w, int ne, float eps, float* stats, float& mean_out,
                                         float& rs_out) {
    const int row = threadIdx.x >> 2, j = threadIdx.x & 3;
    const float* xr = x + row * ld;
    float s = 0.0f;
    if (row < ne)
        for (int k = j; k < w; k += 4) s += xr[k];
    const float mean = row4_sum(s) / w;
    float v = 0.0f;
    if (row < ne)
        for (int k = j; k < w; k += 4) v += (xr[k] - mean) * (xr[k] - mean);
    v = row4_sum(v) / w;
    mean_out = mean;
    rs_out = 1.0f / sqrtf(v + eps);
    if (j == 0) {
        stats[2 * row] = mean;
        stats[2 * row + 1] = rs_out;
    }
}

// Forward of an affine MLP over tiles of 16*waves edges: linear layers on
// MFMA, LayerNorm and SiLU as passes over the tile in LDS (two buffers of row
// stride ld).  A layer's output that feeds a LayerNorm or SiLU also goes to
// the tape ([E][width] blocks, layer-major) for the reverse; the last layer
// writes out [E][out_dim].
__global__ __launch_bounds__(256) void k_mlp_forward(const DMlp m, const DRadial rd, long long E, int ld,
                                                     const float* __restrict__ rad, const int* __restrict__ ets,
                                                     const int* __restrict__ ett, float* __restrict__ out,
                                                     float* __restrict__ tape) {
    extern __shared__ float lds[];
    const int rows = blockDim.x / 4;  // 16 per wave
    float* a = lds;
    float* b = lds + rows * ld;
    float* stats = lds + 2 * rows * ld;
    const long long e0 = static_cast<long long>(blockIdx.x) * rows;
    const int ne = static_cast<int>(min(static_cast<long long>(rows), E - e0));
    const int* ts = ets + e0;
    const int* tt = ett + e0;
    for (int idx = threadIdx.x; idx < rows * ld; idx += blockDim.x) a[idx] = 0.0f;
    __syncthreads();
    for (int idx = threadIdx.x; idx < ne * rd.nb; idx += blockDim.x)
        a[(idx / rd.nb) * ld + idx % rd.nb] = rad[e0 * rd.nb + idx];
    __syncthreads();
    for (int L = 0; L < m.num_layers; ++L) {
        const int type = m.layers[4 * L], in = m.layers[4 * L + 1], w = m.layers[4 * L + 2], off = m.layers[4 * L + 3];
        const bool last = L == m.num_layers - 1;
        float* tl = m.tape_offset[L] >= 0 ? tape + static_cast<std::size_t>(m.tape_offset[L]) * E + e0 * w : nullptr;
        if (type == 0) {
            const float* WT = m.params + m.wt_offset[L];
            const float* bias = m.params + off + static_cast<std::size_t>(w) * in;
            tile_gemm(a, ld, rows, in, WT, w, w, [&](int row, int c, float v) {
                if (row >= ne) {
                    if (!last) b[row * ld + c] = 0.0f;
                    return;
                }
                v += L == 0 ? m.type_rows[static_cast<std::size_t>(ts[row]) * m.first_width + c] +
                                  m.type_rows[static_cast<std::size_t>(m.num_types + tt[row]) * m.first_width + c]
                            : bias[c];
                if (last) {
                    out[(e0 + row) * w + c] = v;
                } else {
                    b[row * ld + c] = v;
                    if (tl) tl[row * w + c] = v;
                }
            });
            float* t = a;
            a = b;
            b = t;
        } else if (type == 1) {
            const float* g = m.params + off;
            const float* bb = g + w;
            float mean_r, rs_r;
            ln_stats(a, ld, w, ne, m.eps[L], stats, mean_r, rs_r);
            __syncthreads();
            for (int idx = threadIdx.x; idx < ne * w; idx += blockDim.x) {
                const int e = idx / w, j = idx % w;
                const float v = (a[e * ld + j] - stats[2 * e]) * stats[2 * e + 1] * g[j] + bb[j];
                b[e * ld + j] = v;
                if (tl) tl[idx] = v;
            }
            float* t = a;
            a = b;
            b = t;
        } else {
            for (int idx = threadIdx.x; idx < ne * w; idx += blockDim.x) {
                float* p = a + (idx / w) * ld + idx % w;
                *p = *p * sigmoidf_(*p);
                if (tl) tl[idx] = *p;
            }
        }
        __syncthreads();
    }
}

// Reverse of an affine MLP: gout [E][out_dim] pulled back through the layers
// (linear layers on MFMA with the row-major weights as B; LayerNorm and SiLU
// from their inputs on the tape, staged in LDS) to the radial features:
// rad_adj [E][nb] +=.
__global__ __launch_bounds__(256) void k_mlp_reverse(const DMlp m, const DRadial rd, long long E, int ld,
                                                     const float* __restrict__ tape, const float* __restrict__ gout,
                                                     float* __restrict__ rad_adj) {
    extern __shared__ float lds[];
    const int rows = blockDim.x / 4;
    float* g = lds;
    float* h = lds + rows * ld;
    float* x = lds + 2 * rows * ld;
    float* stats = lds + 3 * rows * ld;
    const long long e0 = static_cast<long long>(blockIdx.x) * rows;
    const int ne = static_cast<int>(min(static_cast<long long>(rows), E - e0));
    bool from_gout = true;
    for (int L = m.num_layers - 1; L >= 0; --L) {
        const int type = m.layers[4 * L], in = m.layers[4 * L + 1], w = m.layers[4 * L + 2], off = m.layers[4 * L + 3];
        if (type == 0) {
            const float* W = m.params + off;  // [w][in]: B(k = output, c = input)
            // the last layer reads its adjoint rows straight from gout (rows past the edges read zeros)
            const float* A = from_gout ? gout + e0 * w : g;
            tile_gemm(A, from_gout ? w : ld, from_gout ? ne : rows, w, W, in, in, [&](int row, int c, float v) {
                if (L == 0) {
                    if (row < ne) rad_adj[(e0 + row) * rd.nb + c] += v;
                } else {
                    h[row * ld + c] = row < ne ? v : 0.0f;
                }
            });
            from_gout = false;
        } else {
            // this layer's input is layer L-1's output, kept on the tape
            const float* tin = tape + static_cast<std::size_t>(m.tape_offset[L - 1]) * E + e0 * w;
            for (int idx = threadIdx.x; idx < ne * w; idx += blockDim.x) x[(idx / w) * ld + idx % w] = tin[idx];
            __syncthreads();
            if (type == 1) {
                const float* gam = m.params + off;
                float mean, rs;
                ln_stats(x, ld, w, ne, m.eps[L], stats, mean, rs);
                // row means of g*gamma and g*gamma*xhat (four lanes per row)
                const int row = threadIdx.x >> 2, j = threadIdx.x & 3;
                float mg = 0.0f, mgx = 0.0f;
                if (row < ne) {
                    for (int k = j; k < w; k += 4) {
                        const float gh = g[row * ld + k] * gam[k];
                        mg += gh;
                        mgx += gh * (x[row * ld + k] - mean) * rs;
                    }
                }
                mg = row4_sum(mg) / w;
                mgx = row4_sum(mgx) / w;
                __syncthreads();
                if (j == 0) {
                    stats[4 * rows + 2 * row] = mg;
                    stats[4 * rows + 2 * row + 1] = mgx;
                }
                __syncthreads();
                for (int idx = threadIdx.x; idx < rows * w; idx += blockDim.x) {
                    const int e = idx / w, k = idx % w;
                    float v = 0.0f;
                    if (e < ne) {
                        const float rs = stats[2 * e + 1];
                        const float xh = (x[e * ld + k] - stats[2 * e]) * rs;
                        v = rs * (g[e * ld + k] * gam[k] - stats[4 * rows + 2 * e] - xh * stats[4 * rows + 2 * e + 1]);
                    }
                    h[e * ld + k] = v;
                }
            } else {
                for (int idx = threadIdx.x; idx < rows * w; idx += blockDim.x) {
                    const int e = idx / w, k = idx % w;
                    float v = 0.0f;
                    if (e < ne) {
                        const float xv = x[e * ld + k];
                        const float sg = sigmoidf_(xv);
                        v = g[e * ld + k] * (sg + xv * sg * (1.0f - sg));
                    }
                    h[e * ld + k] = v;
                }
            }
        }
        __syncthreads();
        float* t = g;
        g = h;
        h = t;
    }
}

// ---- edge MLPs in registers
//
// The units of a layer are the rows and the edges the columns of
// v_mfma_f32_16x16x4_f32: lane (r, kg) of a wave (r = lane % 16, kg =
// lane / 16) holds, for edge e0 + 16t + r of its t-th tile of 16 edges,
// units 16i + 4kg + v (v < 4) of a layer in x[t][i][v] (the D layout).  With
// the k index of step (J, v) of lane group kg taken as 16J + 4kg + v, the same
// registers are the B operand of the next layer, and the A operand (weight row
// 16i + r) is one 16-byte load per J: a tile's activations never leave
// registers and no LDS is used.  Every hidden stage has the width 16 MT, so
// the MFMA chains are straight-line code.  Lanes r, r+16, r+32, r+48 hold one edge, so
// a LayerNorm's row sums are the lane's 16 units plus two cross-group shuffles.
// The reverse recomputes the hidden stages from the radial features instead
// of reading a tape, as the reference's streamed reverse re-runs the
// conditioned MLPs per edge block (mace_nonlinear.cpp:916-929).

__device__ __forceinline__ v4f ld4(const float* p) { return *reinterpret_cast<const v4f*>(p); }


// entries k..k+3 of a row of n floats, zeros from n on (one 16-byte load when n % 4 == 0)
__device__ __forceinline__ v4f ld4_row(const float* row, int k, int n) {
    if ((n & 3) == 0) {
        v4f x{0.0f, 0.0f, 0.0f, 0.0f};
        if (k < n) x = ld4(row + k);
        return x;
    }
    v4f x;
#pragma unroll
    for (int v = 0; v < 4; ++v) x[v] = k + v < n ? row[k + v] : 0.0f;
    return x;
}

__device__ __forceinline__ void st4_row(float* row, int k, int n, v4f v) {
    if ((n & 3) == 0) {
        if (k < n) *reinterpret_cast<v4f*>(row + k) = v;
        return;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q)
        if (k + q < n) row[k + q] = v[q];
}

// logistic function with the hardware reciprocal (1 ulp) in place of an IEEE division
__device__ __forceinline__ float sigmoid_rcp(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

// sum over the four lane groups that hold one edge
__device__ __forceinline__ float group4_sum(float v) {
    v += __shfl_xor(v, 16, kWave);
    v += __shfl_xor(v, 32, kWave);
    return v;
}

// acc[t][i] = sum_k W[16i + r][k] x[t][k] (W row-major with row stride K; K = M = 16 MT)
template <int MT, int NT>
__device__ __forceinline__ void reg_linear(const float* __restrict__ W, int K, int M, const float (&x)[NT][MT][4],
                                           v4f (&acc)[NT][MT]) {
    const int lane = threadIdx.x & 63, r = lane & 15, kg = lane >> 4;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < MT; ++i) acc[t][i] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int J = 0; J < MT; ++J) {
        v4f a[MT];
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            a[i] = ld4(W + static_cast<std::size_t>(16 * i + r) * K + 16 * J + 4 * kg);
        }
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
            for (int i = 0; i < MT; ++i) {
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    acc[t][i] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][v], x[t][J][v], acc[t][i], 0, 0, 0);
            }
    }
    mfma_settle();
}

// A stage's LayerNorm (when it has one) and SiLU of its linear output acc, into x.  With SAVE the
// normalized values (the SiLU input, without a LayerNorm) and 1/std per edge are kept for the reverse.
template <int MT, int NT, bool SAVE>
__device__ __forceinline__ void reg_norm_silu(const float* __restrict__ params, const DMlpStage& S,
                                              const v4f (&acc)[NT][MT], float (&x)[NT][MT][4],
                                              float (&xs)[NT][MT][4], float (&rs)[NT]) {
    const int kg = (threadIdx.x & 63) >> 4;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        float mean = 0.0f, rstd = 1.0f;
        if (S.ln >= 0) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < MT; ++i) {
    #pragma unroll
                for (int v = 0; v < 4; ++v) s += acc[t][i][v];
            }
            mean = group4_sum(s) / S.out;
            float q = 0.0f;
#pragma unroll
            for (int i = 0; i < MT; ++i) {
    #pragma unroll
                for (int v = 0; v < 4; ++v) q += (acc[t][i][v] - mean) * (acc[t][i][v] - mean);
            }
            rstd = 1.0f / sqrtf(group4_sum(q) / S.out + S.eps);
        }
        if (SAVE) rs[t] = rstd;
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            v4f g{1.0f, 1.0f, 1.0f, 1.0f}, b{0.0f, 0.0f, 0.0f, 0.0f};
            if (S.ln >= 0) {
                g = ld4(params + S.ln + 16 * i + 4 * kg);
                b = ld4(params + S.ln + S.out + 16 * i + 4 * kg);
            }
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float h = (acc[t][i][v] - mean) * rstd;
                if (SAVE) xs[t][i][v] = h;
                const float z = h * g[v] + b[v];
                x[t][i][v] = z * sigmoid_rcp(z);
            }
        }
    }
}

// Reverse of reg_norm_silu: g (adjoint of the stage's output) to gx (adjoint of its linear output),
// SiLU from z = xs * gamma + beta recomputed, then LayerNorm
// dx = rstd (gamma g - mean(gamma g) - xhat mean(gamma g xhat)).
template <int MT, int NT>
__device__ __forceinline__ void reg_silu_norm_reverse(const float* __restrict__ params, const DMlpStage& S,
                                                      const v4f (&g)[NT][MT], const float (&xs)[NT][MT][4],
                                                      const float (&rs)[NT], float (&gx)[NT][MT][4]) {
    const int kg = (threadIdx.x & 63) >> 4;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        float m1 = 0.0f, m2 = 0.0f;
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            v4f ga{1.0f, 1.0f, 1.0f, 1.0f}, be{0.0f, 0.0f, 0.0f, 0.0f};
            if (S.ln >= 0) {
                ga = ld4(params + S.ln + 16 * i + 4 * kg);
                be = ld4(params + S.ln + S.out + 16 * i + 4 * kg);
            }
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float h = xs[t][i][v];
                const float z = h * ga[v] + be[v];
                const float sg = sigmoid_rcp(z);
                const float gh = g[t][i][v] * (sg + z * sg * (1.0f - sg)) * ga[v];
                gx[t][i][v] = gh;
                m1 += gh;
                m2 += gh * h;
            }
        }
        if (S.ln >= 0) {
            m1 = group4_sum(m1) / S.out;
            m2 = group4_sum(m2) / S.out;
#pragma unroll
            for (int i = 0; i < MT; ++i) {
    #pragma unroll
                for (int v = 0; v < 4; ++v) gx[t][i][v] = rs[t] * (gx[t][i][v] - m1 - xs[t][i][v] * m2);
            }
        }
    }
}

// The hidden stages of a tile of NT x 16 edges from e0: the conditioned first linear over the radial
// features plus the per-type rows, then each later stage's linear and bias; every stage ends in
// reg_norm_silu.  x receives the last stage's output.
template <int HW, int NT, bool SAVE>
__device__ __forceinline__ void reg_hidden(const DMlp& m, long long E, long long e0, const float* __restrict__ rad,
                                           const int* __restrict__ ets, const int* __restrict__ ett,
                                           float (&x)[NT][HW / 16][4], float (&xs)[kRegStages][NT][HW / 16][4],
                                           float (&rs)[kRegStages][NT]) {
    constexpr int MT = HW / 16;
    const int lane = threadIdx.x & 63, r = lane & 15, kg = lane >> 4;
    const int nb = m.radial;
    long long ec[NT];  // the tile's edges (past E: the last edge, whose columns are never stored)
#pragma unroll
    for (int t = 0; t < NT; ++t) ec[t] = min(e0 + 16 * t + r, E - 1);
    v4f acc[NT][MT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < MT; ++i) acc[t][i] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    const DMlpStage& S0 = m.st[0];
    const float* W0 = m.params + S0.w;  // [S0.out][nb]
    for (int k0 = 0; k0 < nb; k0 += 4) {
        const int k = k0 + kg;
        float b[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            b[t] = 0.0f;
            if (k < nb) b[t] = rad[ec[t] * nb + k];
        }
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            float a = 0.0f;
            if (k < nb) a = W0[(16 * i + r) * nb + k];
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[t][i] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b[t], acc[t][i], 0, 0, 0);
        }
    }
    mfma_settle();
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const float* ps = m.type_rows + static_cast<std::size_t>(ets[ec[t]]) * S0.out + 4 * kg;
        const float* pt = m.type_rows + static_cast<std::size_t>(m.num_types + ett[ec[t]]) * S0.out + 4 * kg;
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            acc[t][i] += ld4(ps + 16 * i) + ld4(pt + 16 * i);
        }
    }
    reg_norm_silu<MT, NT, SAVE>(m.params, S0, acc, x, xs[0], rs[0]);
#pragma unroll
    for (int h = 1; h < kRegStages; ++h) {
        if (h >= m.reg_stages) break;
        const DMlpStage& S = m.st[h];
        reg_linear<MT, NT>(m.params + S.w, S.in, S.out, x, acc);
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                    acc[t][i] += ld4(m.params + S.b + 16 * i + 4 * kg);
            }
        reg_norm_silu<MT, NT, SAVE>(m.params, S, acc, x, xs[h], rs[h]);
    }
}

// Forward of an edge MLP in registers: one wave per NT x 16 edges, out [E][out_dim].
template <int HW, int NT>
__global__ __launch_bounds__(256) void k_mlp_forward_r(const DMlp m, long long E, const float* __restrict__ rad,
                                                       const int* __restrict__ ets, const int* __restrict__ ett,
                                                       float* __restrict__ out) {
    constexpr int MT = HW / 16;
    const int lane = threadIdx.x & 63, r = lane & 15, kg = lane >> 4;
    const long long e0 = (static_cast<long long>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6)) * (16 * NT);
    if (e0 >= E) return;
    float x[NT][MT][4], xs[kRegStages][NT][MT][4], rs[kRegStages][NT];
    reg_hidden<HW, NT, false>(m, E, e0, rad, ets, ett, x, xs, rs);
    const DMlpStage& F = m.st[kRegStages];
    const float* W = m.params + F.w;
    const float* bias = m.params + F.b;
    const int K = F.in, M = F.out;
    // two 16-row tiles of the output per pass (independent MFMA chains); rows past M read row M-1
    // and are not stored
    for (int i0 = 0; i0 < M; i0 += 32) {
        const int ra = min(i0 + r, M - 1), rb = min(i0 + 16 + r, M - 1);
        v4f acc[NT][2];
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t][0] = acc[t][1] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int J = 0; J < MT; ++J) {
                const v4f a0 = ld4(W + static_cast<std::size_t>(ra) * K + 16 * J + 4 * kg);
            const v4f a1 = ld4(W + static_cast<std::size_t>(rb) * K + 16 * J + 4 * kg);
#pragma unroll
            for (int v = 0; v < 4; ++v)
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    acc[t][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0[v], x[t][J][v], acc[t][0], 0, 0, 0);
                    acc[t][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1[v], x[t][J][v], acc[t][1], 0, 0, 0);
                }
        }
        mfma_settle();
        const v4f b0 = ld4_row(bias, i0 + 4 * kg, M), b1 = ld4_row(bias, i0 + 16 + 4 * kg, M);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const long long e = e0 + 16 * t + r;
            if (e >= E) continue;
            float* orow = out + e * M;
            st4_row(orow, i0 + 4 * kg, M, acc[t][0] + b0);
            st4_row(orow, i0 + 16 + 4 * kg, M, acc[t][1] + b1);
        }
    }
}

// Adjoint of the last hidden stage's output from the final linear's output adjoint:
// g[t][i] = sum_k W_F[k][16i + r] gout[e][k] (W_F^T rows as the A operand, gout rows as B).
template <int MT, int NT>
__device__ __forceinline__ void reg_out_reverse(const DMlp& m, const long long (&ec)[NT], const float* __restrict__ gout,
                                                v4f (&g)[NT][MT]) {
    const int lane = threadIdx.x & 63, r = lane & 15, kg = lane >> 4;
    const DMlpStage& F = m.st[kRegStages];
    const float* WT = m.params + F.wt;  // [F.in][F.out]
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < MT; ++i) g[t][i] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    for (int k0 = 0; k0 < F.out; k0 += 16) {
        v4f gb[NT], a[MT];
#pragma unroll
        for (int t = 0; t < NT; ++t) gb[t] = ld4_row(gout + ec[t] * F.out, k0 + 4 * kg, F.out);
#pragma unroll
        for (int i = 0; i < MT; ++i)
            a[i] = ld4_row(WT + static_cast<std::size_t>(16 * i + r) * F.out, k0 + 4 * kg, F.out);
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    g[t][i] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][v], gb[t][v], g[t][i], 0, 0, 0);
    }
    mfma_settle();
}

// First half of a split reverse (wide outputs): reg_out_reverse over tiles of NT x 16 edges, g
// written [E][HW] (edge row, unit) for the second half.  Few registers, so enough waves stream
// gout from HBM while others run MFMAs.
template <int HW, int NT>
__global__ __launch_bounds__(256) void k_mlp_out_reverse_r(const DMlp m, long long E, const float* __restrict__ gout,
                                                           float* __restrict__ gbuf) {
    constexpr int MT = HW / 16;
    const int lane = threadIdx.x & 63, r = lane & 15, kg = lane >> 4;
    const long long e0 = (static_cast<long long>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6)) * (16 * NT);
    if (e0 >= E) return;
    long long ec[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) ec[t] = min(e0 + 16 * t + r, E - 1);
    v4f g[NT][MT];
    reg_out_reverse<MT, NT>(m, ec, gout, g);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const long long e = e0 + 16 * t + r;
        if (e >= E) continue;
#pragma unroll
        for (int i = 0; i < MT; ++i) *reinterpret_cast<v4f*>(gbuf + e * HW + 16 * i + 4 * kg) = g[t][i];
    }
}

// Reverse of an edge MLP in registers: the hidden stages recomputed (normalized values kept), gout
// [E][out_dim] pulled back through the final linear (or, with SPLIT, its result read from gbuf
// [E][HW]) and every stage to the radial features: rad_adj [E][nb] +=.
template <int HW, int NT, bool SPLIT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void k_mlp_reverse_r(const DMlp m, long long E, const float* __restrict__ rad,
                                                       const int* __restrict__ ets, const int* __restrict__ ett,
                                                       const float* __restrict__ gout, const float* __restrict__ gbuf,
                                                       float* __restrict__ rad_adj) {
    constexpr int MT = HW / 16;
    const int lane = threadIdx.x & 63, r = lane & 15, kg = lane >> 4;
    const long long e0 = (static_cast<long long>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6)) * (16 * NT);
    if (e0 >= E) return;
    long long ec[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) ec[t] = min(e0 + 16 * t + r, E - 1);
    v4f g[NT][MT];
    if constexpr (SPLIT) {
        // issued before the recompute, which hides their latency
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int i = 0; i < MT; ++i) g[t][i] = ld4(gbuf + ec[t] * HW + 16 * i + 4 * kg);
    }
    float x[NT][MT][4], xs[kRegStages][NT][MT][4], rs[kRegStages][NT];
    reg_hidden<HW, NT, true>(m, E, e0, rad, ets, ett, x, xs, rs);
    if constexpr (!SPLIT) reg_out_reverse<MT, NT>(m, ec, gout, g);
    float gx[NT][MT][4];
#pragma unroll
    for (int h = kRegStages - 1; h >= 0; --h) {
        if (h >= m.reg_stages) continue;
        const DMlpStage& S = m.st[h];
        reg_silu_norm_reverse<MT, NT>(m.params, S, g, xs[h], rs[h], gx);
        if (h > 0) {
            // adjoint of the previous stage's output: W_h^T gx, W_h^T = [S.in][S.out] row-major
            reg_linear<MT, NT>(m.params + S.wt, S.out, S.in, gx, g);
            continue;
        }
        // radial adjoint: rad_adj[e][k] += sum_u W0[u][k] gx[e][u], W0^T = [nb][S.out]
        const int nb = m.radial;
        const float* WT0 = m.params + S.wt;
        for (int k0 = 0; k0 < nb; k0 += 16) {
            const int kr = min(k0 + r, nb - 1);
            const bool kv = k0 + r < nb;
            v4f acc[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int J = 0; J < MT; ++J) {
                v4f a = ld4(WT0 + static_cast<std::size_t>(kr) * S.out + 16 * J + 4 * kg);
                if (!kv) a = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int v = 0; v < 4; ++v)
#pragma unroll
                    for (int t = 0; t < NT; ++t)
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[v], gx[t][J][v], acc[t], 0, 0, 0);
            }
            mfma_settle();
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const long long e = e0 + 16 * t + r;
                if (e >= E) continue;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int k = k0 + 4 * kg + v;
                    if (k < nb) rad_adj[e * nb + k] += acc[t][v];
                }
            }
        }
    }
}

// Convolution into receivers: msg[i][(block, u, k)] = sum over the receiver's
// edges of pw * w[e][path][u] * sum_ab W3j[a][b][k] up[src][(block1, u, a)]
// Y[e][l2^2 + b] (e3nn.cpp:343-357), plus the density sum (tanh of the
// squared density output, mace_nonlinear.cpp:702-708).  Thread per (receiver,
// channel); the channel's output and first-input components in LDS columns.
__global__ __launch_bounds__(kTpThreads) void k_tp_forward(const DTp t, int N, const int* __restrict__ offsets,
                                                            const int* __restrict__ src,
                                                            const float* __restrict__ up,
                                                            const float* __restrict__ Y, int NY,
                                                            const float* __restrict__ wraw,
                                                            const float* __restrict__ cut,
                                                            const float* __restrict__ draw,
                                                            float* __restrict__ msg, float* __restrict__ density) {
    extern __shared__ float lds[];
    float* acc = lds;                          // [slots][kTpThreads]
    float* x1 = lds + t.slots * kTpThreads;    // [nin1][kTpThreads]
    const int tid = threadIdx.x;
    const long long gt = blockIdx.x * static_cast<long long>(kTpThreads) + tid;
    const int i = static_cast<int>(gt / t.channels), u = static_cast<int>(gt % t.channels);
    if (i >= N) return;
    for (int s = 0; s < t.slots; ++s) acc[s * kTpThreads + tid] = 0.0f;
    float dens = 0.0f;
    for (int e = offsets[i]; e < offsets[i + 1]; ++e) {
        const float* urow = up + static_cast<std::size_t>(src[e]) * t.in1_dim;
        for (int q = 0; q < t.nin1; ++q)
            x1[q * kTpThreads + tid] = urow[t.in1_slot[3 * q] + u * t.in1_slot[3 * q + 1] + t.in1_slot[3 * q + 2]];
        const float cf = cut ? cut[e] : 1.0f;
        const float* ye = Y + static_cast<std::size_t>(e) * NY;
        const float* we = wraw + static_cast<std::size_t>(e) * t.numel;
        for (int p = 0; p < t.num_paths; ++p) {
            const int* P = t.paths + 8 * p;
            const float w = we[P[5] + u] * cf;
            for (int q = P[6]; q < P[6] + P[7]; ++q) {
                const int ent = t.entries[q];
                const int a = ent & 255, b = (ent >> 8) & 255, k = ent >> 16;
                acc[(P[3] + k) * kTpThreads + tid] += w * t.values[q] * x1[(P[0] + a) * kTpThreads + tid] * ye[P[2] + b];
            }
        }
        const float dr = draw[e];
        dens += tanhf(dr * dr) * cf;
    }
    float* mrow = msg + static_cast<std::size_t>(i) * t.out_dim;
    for (int s = 0; s < t.slots; ++s)
        mrow[t.out_slot[3 * s] + u * t.out_slot[3 * s + 1] + t.out_slot[3 * s + 2]] = acc[s * kTpThreads + tid];
    if (u == 0) density[i] = dens;
}

// Reverse of the convolution for the receiver's edges (e3nn.cpp:361-407 and
// mace_nonlinear.cpp:851-900): per edge the weight adjoints (times the cutoff
// when the cutoff is on the weights), the first-input adjoint rows (gathered
// per source afterwards), the harmonic adjoints and the cutoff and density
// adjoints (summed over the channel lanes).
__global__ __launch_bounds__(kTpThreads) void k_tp_reverse(
    const DTp t, int N, const int* __restrict__ offsets, const int* __restrict__ src, const float* __restrict__ up,
    const float* __restrict__ Y, int NY, const float* __restrict__ wraw, const float* __restrict__ cut,
    const float* __restrict__ draw, const float* __restrict__ amsg, const float* __restrict__ adens,
    float* __restrict__ wadj, float* __restrict__ a1, float* __restrict__ Yadj, float* __restrict__ cut_adj,
    float* __restrict__ adraw) {
    extern __shared__ float lds[];
    float* g = lds;                               // [slots]
    float* x1 = g + t.slots * kTpThreads;         // [nin1]
    float* xa = x1 + t.nin1 * kTpThreads;         // [nin1]
    float* ya = xa + t.nin1 * kTpThreads;         // [NY]
    const int tid = threadIdx.x;
    const long long gt = blockIdx.x * static_cast<long long>(kTpThreads) + tid;
    const int i = static_cast<int>(gt / t.channels), u = static_cast<int>(gt % t.channels);
    if (i >= N) return;
    const float* grow = amsg + static_cast<std::size_t>(i) * t.out_dim;
    for (int s = 0; s < t.slots; ++s)
        g[s * kTpThreads + tid] = grow[t.out_slot[3 * s] + u * t.out_slot[3 * s + 1] + t.out_slot[3 * s + 2]];
    const float ad = adens[i];
    for (int e = offsets[i]; e < offsets[i + 1]; ++e) {
        const float* urow = up + static_cast<std::size_t>(src[e]) * t.in1_dim;
        for (int q = 0; q < t.nin1; ++q) {
            x1[q * kTpThreads + tid] = urow[t.in1_slot[3 * q] + u * t.in1_slot[3 * q + 1] + t.in1_slot[3 * q + 2]];
            xa[q * kTpThreads + tid] = 0.0f;
        }
        for (int b = 0; b < NY; ++b) ya[b * kTpThreads + tid] = 0.0f;
        const float cf = cut ? cut[e] : 1.0f;
        const float* ye = Y + static_cast<std::size_t>(e) * NY;
        const float* we = wraw + static_cast<std::size_t>(e) * t.numel;
        float* wa = wadj + static_cast<std::size_t>(e) * t.numel;
        float cpart = 0.0f;
        for (int p = 0; p < t.num_paths; ++p) {
            const int* P = t.paths + 8 * p;
            const float wr = we[P[5] + u];
            const float w = wr * cf;
            float gw = 0.0f;
            for (int q = P[6]; q < P[6] + P[7]; ++q) {
                const int ent = t.entries[q];
                const int a = ent & 255, b = (ent >> 8) & 255, k = ent >> 16;
                const float vg = t.values[q] * g[(P[3] + k) * kTpThreads + tid];
                const float xv = x1[(P[0] + a) * kTpThreads + tid];
                const float yv = ye[P[2] + b];
                gw += vg * xv * yv;
                xa[(P[0] + a) * kTpThreads + tid] += vg * w * yv;
                ya[(P[2] + b) * kTpThreads + tid] += vg * w * xv;
            }
            wa[P[5] + u] = gw * cf;
            cpart += gw * wr;
        }
        float* arow = a1 + static_cast<std::size_t>(e) * t.in1_dim;
        for (int q = 0; q < t.nin1; ++q)
            arow[t.in1_slot[3 * q] + u * t.in1_slot[3 * q + 1] + t.in1_slot[3 * q + 2]] = xa[q * kTpThreads + tid];
        // sums over the receiver's channel lanes (aligned groups of t.channels lanes)
        for (int b = 0; b < NY; ++b) {
            float v = ya[b * kTpThreads + tid];
            for (int off = t.channels / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
            if (u == 0) Yadj[static_cast<std::size_t>(e) * NY + b] += v;
        }
        for (int off = t.channels / 2; off > 0; off >>= 1) cpart += __shfl_xor(cpart, off, kWave);
        if (u == 0) {
            const float dr = draw[e];
            const float base = tanhf(dr * dr);
            adraw[e] = ad * (1.0f - base * base) * 2.0f * dr * cf;
            if (cut_adj) cut_adj[e] += cpart + ad * base;
        }
    }
}

// ---- convolution kernels of the compiled family structures (mh1_paths.hpp):
// the same sums as k_tp_forward / k_tp_reverse with every path, Wigner
// position and slot a compile-time constant, so accumulators, the channel's
// first-input components, the edge's harmonics and adjoints stay in registers
// (the Wigner values are uniform loads from the model tables).

template <class S, int P, int Q>
__device__ __forceinline__ void tpc_fwd_entry(float (&acc)[S::kSlots], const float (&x1)[S::kIn1], const float* y,
                                              float w, const float* __restrict__ cv) {
    constexpr TpPathC p = S::paths[P];
    constexpr TpEntryC en = S::entries[p.first + Q];
    acc[p.out_base + en.k] += w * cv[p.first + Q] * x1[p.in_base + en.a] * y[p.l2 * p.l2 + en.b];
}

template <class S, int P, int... Q>
__device__ __forceinline__ void tpc_fwd_path(float (&acc)[S::kSlots], const float (&x1)[S::kIn1], const float* y,
                                             float w, const float* __restrict__ cv, std::integer_sequence<int, Q...>) {
    (tpc_fwd_entry<S, P, Q>(acc, x1, y, w, cv), ...);
}

template <class S, int... P>
__device__ __forceinline__ void tpc_fwd(float (&acc)[S::kSlots], const float (&x1)[S::kIn1], const float* y,
                                        const float (&w)[S::kPaths], const float* __restrict__ cv,
                                        std::integer_sequence<int, P...>) {
    (tpc_fwd_path<S, P>(acc, x1, y, w[P], cv, std::make_integer_sequence<int, S::paths[P].count>{}), ...);
}

template <class S, int P, int Q>
__device__ __forceinline__ void tpc_rev_entry(const float (&g)[S::kSlots], const float (&x1)[S::kIn1],
                                              const float* y, float w, const float* __restrict__ cv, float& gw,
                                              float (&xa)[S::kIn1], float* ya) {
    constexpr TpPathC p = S::paths[P];
    constexpr TpEntryC en = S::entries[p.first + Q];
    const float vg = cv[p.first + Q] * g[p.out_base + en.k];
    const float xv = x1[p.in_base + en.a], yv = y[p.l2 * p.l2 + en.b];
    gw += vg * xv * yv;
    xa[p.in_base + en.a] += vg * w * yv;
    ya[p.l2 * p.l2 + en.b] += vg * w * xv;
}

template <class S, int P, int... Q>
__device__ __forceinline__ void tpc_rev_path(const float (&g)[S::kSlots], const float (&x1)[S::kIn1], const float* y,
                                             float w, const float* __restrict__ cv, float& gw, float (&xa)[S::kIn1],
                                             float* ya, std::integer_sequence<int, Q...>) {
    (tpc_rev_entry<S, P, Q>(g, x1, y, w, cv, gw, xa, ya), ...);
}

template <class S, int... P>
__device__ __forceinline__ void tpc_rev(const float (&g)[S::kSlots], const float (&x1)[S::kIn1], const float* y,
                                        const float (&w)[S::kPaths], const float* __restrict__ cv,
                                        float (&gw)[S::kPaths], float (&xa)[S::kIn1], float* ya,
                                        std::integer_sequence<int, P...>) {
    (tpc_rev_path<S, P>(g, x1, y, w[P], cv, gw[P], xa, ya, std::make_integer_sequence<int, S::paths[P].count>{}),
     ...);
}

// first-input components of channel u: the 0e value, then the 1o triple
template <class S>
__device__ __forceinline__ void tpc_load_x1(const float* urow, int E, int u, float (&x1)[S::kIn1]) {
    x1[0] = urow[u];
    if constexpr (S::kIn1 == 4) {
#pragma unroll
        for (int a = 0; a < 3; ++a) x1[1 + a] = urow[E + 3 * u + a];
    }
}

template <int L1MAX, int LMAX>
__global__ __launch_bounds__(kTpThreads) void k_tp_forward_c(const DTp t, int N, const int* __restrict__ offsets,
                                                              const int* __restrict__ src,
                                                              const float* __restrict__ up,
                                                              const float* __restrict__ Y,
                                                              const float* __restrict__ wraw,
                                                              const float* __restrict__ cut,
                                                              const float* __restrict__ draw,
                                                              float* __restrict__ msg, float* __restrict__ density) {
    using S = TpStructure<L1MAX, LMAX>;
    constexpr int NY = (LMAX + 1) * (LMAX + 1);
    const long long gt = blockIdx.x * static_cast<long long>(kTpThreads) + threadIdx.x;
    const int E = t.channels;
    const int i = static_cast<int>(gt / E), u = static_cast<int>(gt % E);
    if (i >= N) return;
    float acc[S::kSlots];
#pragma unroll
    for (int s = 0; s < S::kSlots; ++s) acc[s] = 0.0f;
    float dens = 0.0f;
    for (int e = offsets[i]; e < offsets[i + 1]; ++e) {
        float x1[S::kIn1];
        tpc_load_x1<S>(up + static_cast<std::size_t>(src[e]) * t.in1_dim, E, u, x1);
        float y[NY];
#pragma unroll
        for (int b = 0; b < NY; ++b) y[b] = Y[static_cast<std::size_t>(e) * NY + b];
        const float cf = cut ? cut[e] : 1.0f;
        const float* we = wraw + static_cast<std::size_t>(e) * t.numel + u;
        float w[S::kPaths];
#pragma unroll
        for (int p = 0; p < S::kPaths; ++p) w[p] = we[p * E] * cf;
        tpc_fwd<S>(acc, x1, y, w, t.cval, std::make_integer_sequence<int, S::kPaths>{});
        const float dr = draw[e];
        dens += tanhf(dr * dr) * cf;
    }
    float* mrow = msg + static_cast<std::size_t>(i) * t.out_dim;
#pragma unroll
    for (int p = 0; p < S::kPaths; ++p) {
        // output block of path p: per-channel slots out_base.., E * out_base floats before it
        const int ob = S::paths[p].out_base, d3 = 2 * S::paths[p].l3 + 1;
#pragma unroll
        for (int k = 0; k < 7; ++k)
            if (k < d3) mrow[E * ob + u * d3 + k] = acc[ob + k];
    }
    if (u == 0) density[i] = dens;
}

template <int L1MAX, int LMAX>
__global__ __launch_bounds__(kTpThreads) __attribute__((amdgpu_waves_per_eu(3))) void k_tp_reverse_c(
    const DTp t, int N, const int* __restrict__ offsets, const int* __restrict__ src, const float* __restrict__ up,
    const float* __restrict__ Y, const float* __restrict__ wraw, const float* __restrict__ cut,
    const float* __restrict__ draw, const float* __restrict__ amsg, const float* __restrict__ adens,
    float* __restrict__ wadj, float* __restrict__ a1, float* __restrict__ Yadj, float* __restrict__ cut_adj,
    float* __restrict__ adraw) {
    using S = TpStructure<L1MAX, LMAX>;
    constexpr int NY = (LMAX + 1) * (LMAX + 1);
    const long long gt = blockIdx.x * static_cast<long long>(kTpThreads) + threadIdx.x;
    const int E = t.channels;
    const int i = static_cast<int>(gt / E), u = static_cast<int>(gt % E);
    if (i >= N) return;
    float g[S::kSlots];
    const float* grow = amsg + static_cast<std::size_t>(i) * t.out_dim;
#pragma unroll
    for (int p = 0; p < S::kPaths; ++p) {
        const int ob = S::paths[p].out_base, d3 = 2 * S::paths[p].l3 + 1;
#pragma unroll
        for (int k = 0; k < 7; ++k)
            if (k < d3) g[ob + k] = grow[E * ob + u * d3 + k];
    }
    const float ad = adens[i];
    for (int e = offsets[i]; e < offsets[i + 1]; ++e) {
        float x1[S::kIn1];
        tpc_load_x1<S>(up + static_cast<std::size_t>(src[e]) * t.in1_dim, E, u, x1);
        float y[NY];
#pragma unroll
        for (int b = 0; b < NY; ++b) y[b] = Y[static_cast<std::size_t>(e) * NY + b];
        const float cf = cut ? cut[e] : 1.0f;
        const float* we = wraw + static_cast<std::size_t>(e) * t.numel + u;
        float wr[S::kPaths], w[S::kPaths], gw[S::kPaths], xa[S::kIn1], ya[NY];
#pragma unroll
        for (int p = 0; p < S::kPaths; ++p) {
            wr[p] = we[p * E];
            w[p] = wr[p] * cf;
            gw[p] = 0.0f;
        }
#pragma unroll
        for (int a = 0; a < S::kIn1; ++a) xa[a] = 0.0f;
#pragma unroll
        for (int b = 0; b < NY; ++b) ya[b] = 0.0f;
        tpc_rev<S>(g, x1, y, w, t.cval, gw, xa, ya, std::make_integer_sequence<int, S::kPaths>{});
        float* wa = wadj + static_cast<std::size_t>(e) * t.numel + u;
        float cpart = 0.0f;
#pragma unroll
        for (int p = 0; p < S::kPaths; ++p) {
            wa[p * E] = gw[p] * cf;
            cpart += gw[p] * wr[p];
        }
        float* arow = a1 + static_cast<std::size_t>(e) * t.in1_dim;
        arow[u] = xa[0];
        if constexpr (S::kIn1 == 4) {
#pragma unroll
            for (int a = 0; a < 3; ++a) arow[E + 3 * u + a] = xa[1 + a];
        }
        // sums over the receiver's channel lanes (aligned groups of E lanes)
        float* yo = Yadj + static_cast<std::size_t>(e) * NY;
        if (E >= 16) {
            // reduce-scatter of the (padded) 16 harmonic adjoints: four halving
            // steps leave lane u with value u / (E/16), summed over 16 lanes;
            // plain butterflies finish the rest (15 shuffles instead of 16 log2 E)
            float v[16];
#pragma unroll
            for (int b = 0; b < 16; ++b) v[b] = b < NY ? ya[b] : 0.0f;
#pragma unroll
            for (int s = 0, half = 8; s < 4; ++s, half >>= 1) {
                const int off = E >> (s + 1);
                const bool up = (u & off) != 0;
#pragma unroll
                for (int q = 0; q < half; ++q) {
                    const float send = up ? v[q] : v[half + q];
                    const float keep = up ? v[half + q] : v[q];
                    v[q] = keep + __shfl_xor(send, off, kWave);
                }
            }
            for (int off = E >> 5; off > 0; off >>= 1) v[0] += __shfl_xor(v[0], off, kWave);
            const int group = E >> 4;
            if (u % group == 0 && u / group < NY) yo[u / group] += v[0];
        } else {
#pragma unroll
            for (int b = 0; b < NY; ++b) {
                float v = ya[b];
                for (int off = E / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
                if (u == 0) yo[b] += v;
            }
        }
        for (int off = E / 2; off > 0; off >>= 1) cpart += __shfl_xor(cpart, off, kWave);
        if (u == 0) {
            const float dr = draw[e];
            const float base = tanhf(dr * dr);
            adraw[e] = ad * (1.0f - base * base) * 2.0f * dr * cf;
            if (cut_adj) cut_adj[e] += cpart + ad * base;
        }
    }
}

// adjoint rows of the first input, summed per source over the source
// transpose (deterministic order): aup[s] += sum_e a1[e]
__global__ __launch_bounds__(256) void k_gather_sources(int N, int dim, const int* __restrict__ t_off,
                                                        const int* __restrict__ t_edges,
                                                        const float* __restrict__ a1, float* __restrict__ aup) {
    const long long t = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
    if (t >= static_cast<long long>(N) * dim) return;
    const int s = static_cast<int>(t / dim), c = static_cast<int>(t % dim);
    // eight edges per step: their indices, then their rows, in flight together
    float acc = 0.0f;
    int q = t_off[s];
    const int qe = t_off[s + 1];
    for (; q + 8 <= qe; q += 8) {
        int e[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) e[k] = t_edges[q + k];
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = a1[static_cast<std::size_t>(e[k]) * dim + c];
        acc += ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
    }
    for (; q < qe; ++q) acc += a1[static_cast<std::size_t>(t_edges[q]) * dim + c];
    aup[t] += acc;
}

// pre_gate = lin1 / (alpha + beta * density) + residual (mace_nonlinear.cpp:751-760)
__global__ __launch_bounds__(256) void k_pregate(int N, int dim, const float* __restrict__ lin1,
                                                 const float* __restrict__ res, const float* __restrict__ density,
                                                 float alpha, float beta, float* __restrict__ pre) {
    const long long t = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
    if (t >= static_cast<long long>(N) * dim) return;
    const int n = static_cast<int>(t / dim);
    pre[t] = lin1[t] / (alpha + beta * density[n]) + res[t];
}

__global__ __launch_bounds__(256) void k_gate_forward(const DGate gt, int N, const float* __restrict__ x,
                                                      float* __restrict__ y) {
    const long long t = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
    if (t >= static_cast<long long>(N) * gt.out_dim) return;
    const int n = static_cast<int>(t / gt.out_dim), j = static_cast<int>(t % gt.out_dim);
    const float* xr = x + static_cast<std::size_t>(n) * gt.in_dim;
    const float v = xr[gt.out_src[j]];
    const int gi = gt.out_gate[j];
    y[t] = gi < 0 ? gt.out_const[j] * v * sigmoidf_(v) : gt.out_const[j] * sigmoidf_(xr[gi]) * v;
}

// gate adjoint per input element (mace_nonlinear.cpp:103-142)
__global__ __launch_bounds__(256) void k_gate_reverse(const DGate gt, int N, const float* __restrict__ x,
                                                      const float* __restrict__ G, float* __restrict__ A) {
    const long long t = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
    if (t >= static_cast<long long>(N) * gt.in_dim) return;
    const int n = static_cast<int>(t / gt.in_dim), i = static_cast<int>(t % gt.in_dim);
    const float* xr = x + static_cast<std::size_t>(n) * gt.in_dim;
    const float* gr = G + static_cast<std::size_t>(n) * gt.out_dim;
    const int kind = gt.in_kind[i], o = gt.in_out[i];
    const float c = gt.in_const[i];
    float a;
    if (kind == 0) {
        const float v = xr[i], s = sigmoidf_(v);
        a = gr[o] * c * (s + v * s * (1.0f - s));
    } else if (kind == 1) {
        a = gr[o] * c * sigmoidf_(xr[gt.in_aux[i]]);
    } else {
        const float s = sigmoidf_(xr[i]);
        float dot = 0.0f;
        for (int k = 0; k < gt.in_count[i]; ++k) dot += xr[gt.in_aux[i] + k] * gr[o + k];
        a = c * s * (1.0f - s) * dot;
    }
    A[t] = a;
}

// a_lin = a_pre / norm, a_dens = -beta / norm^2 sum_j a_pre[j] lin1[j]
// (mace_nonlinear.cpp:825-834); one wave per node
__global__ __launch_bounds__(256) void k_norm_reverse(int N, int dim, const float* __restrict__ apre,
                                                      const float* __restrict__ lin1,
                                                      const float* __restrict__ density, float alpha, float beta,
                                                      float* __restrict__ alin, float* __restrict__ adens) {
    const int lane = threadIdx.x % kWave;
    const long long n = (blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x) / kWave;
    if (n >= N) return;
    const float norm = alpha + beta * density[n];
    const float* ap = apre + n * dim;
    const float* l1 = lin1 + n * dim;
    float dot = 0.0f;
    for (int j = lane; j < dim; j += kWave) {
        dot += ap[j] * l1[j];
        alin[n * dim + j] = ap[j] / norm;
    }
    dot = wave_sum<kWave>(dot);
    if (lane == 0) adens[n] = -dot * beta / (norm * norm);
}

// Product basis: one thread per (node, channel); the channel's angular
// components in LDS (the last slot holds 1 for monomials of lower degree).
__global__ __launch_bounds__(256) void k_product_forward(const DProduct P, int N, const int* __restrict__ elems,
                                                         const float* __restrict__ X, float* __restrict__ out) {
    __shared__ float x[17 * 256];
    __shared__ float o[16 * 256];
    const int tid = threadIdx.x;
    const long long t = blockIdx.x * static_cast<long long>(blockDim.x) + tid;
    if (t >= static_cast<long long>(N) * P.channels) return;
    const int n = static_cast<int>(t / P.channels), f = static_cast<int>(t % P.channels);
    const float* xr = X + static_cast<std::size_t>(n) * P.in_dim;
    for (int a = 0; a < P.angular; ++a)
        x[a * 256 + tid] = xr[P.ang_src[3 * a] + f * P.ang_src[3 * a + 1] + P.ang_src[3 * a + 2]];
    x[P.angular * 256 + tid] = 1.0f;
    for (int s = 0; s < P.out_slots; ++s) o[s * 256 + tid] = 0.0f;
    const float* cf = P.coef + (static_cast<std::size_t>(elems ? elems[n] : 0) * P.num_terms) * P.channels + f;
    for (int q = 0; q < P.num_terms; ++q) {
        const int* T = P.terms + 4 * q;
        o[T[3] * 256 + tid] += cf[static_cast<std::size_t>(q) * P.channels] * x[T[0] * 256 + tid] *
                               x[T[1] * 256 + tid] * x[T[2] * 256 + tid];
    }
    float* orow = out + static_cast<std::size_t>(n) * P.out_dim;
    for (int s = 0; s < P.out_slots; ++s)
        orow[P.out_slot[3 * s] + f * P.out_slot[3 * s + 1] + P.out_slot[3 * s + 2]] = o[s * 256 + tid];
}

__global__ __launch_bounds__(256) void k_product_reverse(const DProduct P, int N, const int* __restrict__ elems,
                                                         const float* __restrict__ X, const float* __restrict__ G,
                                                         float* __restrict__ A) {
    __shared__ float x[17 * 256];
    __shared__ float ax[17 * 256];
    __shared__ float g[16 * 256];
    const int tid = threadIdx.x;
    const long long t = blockIdx.x * static_cast<long long>(blockDim.x) + tid;
    if (t >= static_cast<long long>(N) * P.channels) return;
    const int n = static_cast<int>(t / P.channels), f = static_cast<int>(t % P.channels);
    const float* xr = X + static_cast<std::size_t>(n) * P.in_dim;
    for (int a = 0; a < P.angular; ++a) {
        x[a * 256 + tid] = xr[P.ang_src[3 * a] + f * P.ang_src[3 * a + 1] + P.ang_src[3 * a + 2]];
        ax[a * 256 + tid] = 0.0f;
    }
    x[P.angular * 256 + tid] = 1.0f;
    ax[P.angular * 256 + tid] = 0.0f;
    const float* gr = G + static_cast<std::size_t>(n) * P.out_dim;
    for (int s = 0; s < P.out_slots; ++s)
        g[s * 256 + tid] = gr[P.out_slot[3 * s] + f * P.out_slot[3 * s + 1] + P.out_slot[3 * s + 2]];
    const float* cf = P.coef + (static_cast<std::size_t>(elems ? elems[n] : 0) * P.num_terms) * P.channels + f;
    for (int q = 0; q < P.num_terms; ++q) {
        const int* T = P.terms + 4 * q;
        const float cg = cf[static_cast<std::size_t>(q) * P.channels] * g[T[3] * 256 + tid];
        const float x0 = x[T[0] * 256 + tid], x1 = x[T[1] * 256 + tid], x2 = x[T[2] * 256 + tid];
        ax[T[0] * 256 + tid] += cg * x1 * x2;
        ax[T[1] * 256 + tid] += cg * x0 * x2;
        ax[T[2] * 256 + tid] += cg * x0 * x1;
    }
    float* arow = A + static_cast<std::size_t>(n) * P.in_dim;
    for (int a = 0; a < P.angular; ++a)
        arow[P.ang_src[3 * a] + f * P.ang_src[3 * a + 1] + P.ang_src[3 * a + 2]] = ax[a * 256 + tid];
}

// readout activation: y = c * silu(x); reverse: a = g * c * silu'(x)
__global__ __launch_bounds__(256) void k_silu_scaled(long long n, float c, const float* __restrict__ x,
                                                     const float* __restrict__ g, float* __restrict__ y) {
    const long long t = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
    if (t >= n) return;
    const float v = x[t], s = sigmoidf_(v);
    y[t] = g ? g[t] * c * (s + v * s * (1.0f - s)) : c * v * s;
}

__global__ __launch_bounds__(256) void k_fill(long long n, float v, float* __restrict__ y) {
    const long long t = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
    if (t < n) y[t] = v;
}

__device__ __forceinline__ void zbl_pair(const DZbl& z, int tu, int tv, double r, double& value, double& grad) {
    const double* pc = z.pair + 3 * (static_cast<std::size_t>(tu) * z.num_types + tv);
    const double ia = pc[0], bare_pref = pc[1], rmax = pc[2];
    if (r >= rmax) {
        value = grad = 0.0;
        return;
    }
    const double ra = r * ia;
    const double e0 = z.c[0] * exp(-3.2 * ra), e1 = z.c[1] * exp(-0.9423 * ra), e2 = z.c[2] * exp(-0.4028 * ra),
                 e3 = z.c[3] * exp(-0.2016 * ra);
    const double phi = e0 + e1 + e2 + e3;
    const double dphi = ia * (-3.2 * e0 - 0.9423 * e1 - 0.4028 * e2 - 0.2016 * e3);
    const double bare = bare_pref / r * phi;
    const double bare_g = bare_pref / (r * r) * (r * dphi - phi);
    const double p = z.p, x = r / rmax;
    const double xm1 = pow(x, p - 1.0), xp = xm1 * x;
    const double env = 1.0 - (p + 1.0) * (p + 2.0) / 2.0 * xp + p * (p + 2.0) * xp * x - p * (p + 1.0) / 2.0 * xp * x * x;
    const double denv =
        (-(p + 1.0) * (p + 2.0) / 2.0 * p * xm1 + p * (p + 2.0) * (p + 1.0) * xp - p * (p + 1.0) / 2.0 * (p + 2.0) * xp * x) /
        rmax;
    value = 0.5 * bare * env;
    grad = 0.5 * (bare * denv + bare_g * env);
}

// node energies: E_i = e0[type] + scale * sum_layers readout_l(i) + shift (+ scale * ZBL)
// (mace_nonlinear.cpp:770-781, 1000-1009)
__global__ __launch_bounds__(256) void k_energies(int N, int num_readouts, const int* __restrict__ types,
                                                  const double* __restrict__ e0, double scale, double shift,
                                                  const float* __restrict__ ro, const int* __restrict__ offsets,
                                                  const int* __restrict__ ets, const double* __restrict__ r,
                                                  const DZbl z, int has_zbl, double* __restrict__ out) {
    const int n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= N) return;
    double s = 0.0;
    for (int k = 0; k < num_readouts; ++k) s += ro[static_cast<std::size_t>(k) * N + n];
    double e = e0[types[n]] + scale * s + shift;
    if (has_zbl) {
        double zs = 0.0;
        for (int q = offsets[n]; q < offsets[n + 1]; ++q) {
            double v, g;
            zbl_pair(z, types[n], ets[q], r[q], v, g);
            zs += v;
        }
        e += scale * zs;
    }
    out[n] = e;
}

// per-edge forces: -(dE/dr xyz/r + sum_lm dE/dY_lm dY_lm/dxyz) (mace_nonlinear.cpp:983-996)
template <int LMAX>
__global__ __launch_bounds__(256) void k_edge_forces(long long E, const double* __restrict__ xyz,
                                                     const double* __restrict__ r, const DRadial rd,
                                                     const int* __restrict__ ets, const int* __restrict__ ett,
                                                     const float* __restrict__ rad_adj,
                                                     const float* __restrict__ cut_adj,
                                                     const float* __restrict__ Yadj, const DZbl z, int has_zbl,
                                                     double scale, double* __restrict__ nf) {
    constexpr int NY = (LMAX + 1) * (LMAX + 1);
    const long long e = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
    if (e >= E) return;
    const double re = r[e];
    double df[32], env, denv;
    radial_eval(rd, re, ets[e], ett[e], nullptr, df, env, denv);
    double dr = 0.0;
    for (int k = 0; k < rd.nb; ++k) dr += static_cast<double>(rad_adj[e * rd.nb + k]) * df[k];
    if (cut_adj) dr += static_cast<double>(cut_adj[e]) * denv;
    const float d[3] = {static_cast<float>(xyz[3 * e]), static_cast<float>(xyz[3 * e + 1]),
                        static_cast<float>(xyz[3 * e + 2])};
    float y[NY], g[3 * NY];
    edge_harmonics<LMAX>(d, static_cast<float>(re), y, g);
    double zg = 0.0;
    if (has_zbl) {
        double v;
        zbl_pair(z, ett[e], ets[e], re, v, zg);
    }
    for (int c = 0; c < 3; ++c) {
        double v = (dr + scale * zg) * xyz[3 * e + c] / re;
        for (int q = 0; q < NY; ++q) v += static_cast<double>(Yadj[e * NY + q]) * g[c * NY + q];
        nf[3 * e + c] = -v;
    }
}

// ----------------------------------------------------------------- host side

inline unsigned blocks_for(long long n, int threads) { return static_cast<unsigned>((n + threads - 1) / threads); }

class Arena {
public:
    ~Arena() {
        if (ptr_) (void)hipFree(ptr_);
    }
    void reserve(std::size_t bytes) {
        if (bytes <= cap_) return;
        if (ptr_) SMX_HIP(hipFree(ptr_));
        ptr_ = nullptr;
        cap_ = 0;
        if (hipMalloc(&ptr_, bytes) != hipSuccess) {
            ptr_ = nullptr;
            throw std::bad_alloc();
        }
        cap_ = bytes;
    }
    char* base() const { return static_cast<char*>(ptr_); }

private:
    void* ptr_ = nullptr;
    std::size_t cap_ = 0;
};

// grow-only pinned host block (hipHostMalloc): the staging area of a call's
// host inputs and results, one DMA transfer each way
class PinnedArena {
public:
    PinnedArena() = default;
    PinnedArena(const PinnedArena&) = delete;
    PinnedArena& operator=(const PinnedArena&) = delete;
    ~PinnedArena() {
        if (ptr_) (void)hipHostFree(ptr_);
    }
    void reserve(std::size_t bytes) {
        if (bytes <= cap_) return;
        if (ptr_) SMX_HIP(hipHostFree(ptr_));
        ptr_ = nullptr;
        cap_ = 0;
        if (hipHostMalloc(&ptr_, bytes, hipHostMallocDefault) != hipSuccess) {
            ptr_ = nullptr;
            throw std::bad_alloc();
        }
        cap_ = bytes;
    }
    char* base() const { return static_cast<char*>(ptr_); }

private:
    void* ptr_ = nullptr;
    std::size_t cap_ = 0;
};

// carves aligned sub-buffers out of one block (sizes first, then addresses)
class Layout {
public:
    template <class T>
    std::size_t add(std::size_t count) {
        off_ = (off_ + 255) & ~static_cast<std::size_t>(255);
        const std::size_t at = off_;
        off_ += std::max<std::size_t>(1, count) * sizeof(T);
        return at;
    }
    std::size_t size() const { return off_ + 256; }

private:
    std::size_t off_ = 0;
};

struct Timer {
    bool enabled = false;
    struct Pending {
        std::string name;
        hipEvent_t a, b;
    };
    std::vector<Pending> pending;
    std::vector<std::string> order;
    std::map<std::string, std::pair<double, long long>> totals;
    void begin(const char* name, hipStream_t s, hipEvent_t& a) {
        if (!enabled) return;
        SMX_HIP(hipEventCreate(&a));
        SMX_HIP(hipEventRecord(a, s));
        (void)name;
    }
    void end(const char* name, hipStream_t s, hipEvent_t a) {
        if (!enabled) return;
        hipEvent_t b;
        SMX_HIP(hipEventCreate(&b));
        SMX_HIP(hipEventRecord(b, s));
        pending.push_back({name, a, b});
    }
    void collect() {
        for (auto& p : pending) {
            float ms = 0.0f;
            SMX_HIP(hipEventElapsedTime(&ms, p.a, p.b));
            auto it = totals.find(p.name);
            if (it == totals.end()) {
                order.push_back(p.name);
                totals[p.name] = {ms, 1};
            } else {
                it->second.first += ms;
                it->second.second += 1;
            }
            (void)hipEventDestroy(p.a);
            (void)hipEventDestroy(p.b);
        }
        pending.clear();
    }
};

class Evaluator {
public:
    // The file is parsed and checked here; the device tables are made on the
    // first compute call (after its inputs are checked), so a model's facts and
    // its load errors need no GPU.
    Evaluator(const std::string& path, const std::string& head) : model_(Model::load(path, head)) {}
    void ensure_device() {
        if (uploaded_) return;
        if (!stream_) SMX_HIP(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
        if (params_) {
            SMX_HIP(hipFree(params_));
            params_ = nullptr;
        }
        inter_.clear();
        prod_.clear();
        ro_.clear();
        upload_model();
        uploaded_ = true;
    }
    ~Evaluator() {
        if (params_) (void)hipFree(params_);
        if (stream_) (void)hipStreamDestroy(stream_);
    }
    const Model& model() const { return model_; }
    void compute(int N, const int* types, const int* num_neigh, const int* neigh, const int* neigh_types,
                 const double* xyz, const double* r, long long E);
    // the last call's results (pinned host memory, valid until the next call)
    struct Span {
        const double* data;
        std::size_t size;
    };
    Span node_energies() const { return {num_energies_ ? energies_ : nullptr, num_energies_}; }
    Span node_forces() const { return {num_forces_ ? forces_ : nullptr, num_forces_}; }
    std::vector<float> stage(const std::string& name);
    Timer timer;

private:
    struct LinearDev {
        DLinear fwd, rev;
    };
    struct InteractionDev {
        LinearDev up, skip, res, lin1, lin2;
        DTp tp;
        DMlp wmlp, dmlp;
        DGate gate;
        float alpha, beta;
    };
    struct ProductDev {
        DProduct P;
        LinearDev lin;
    };
    struct ReadoutDev {
        bool nonlinear;
        LinearDev l1, l2;
        float c;
    };

    void upload_model();
    void launch_linear(const DLinear& op, int N, const float* x, float* y, const float* addend, bool accumulate,
                       const char* name);
    template <class K, class... A>
    void launch(const char* name, K kernel, unsigned grid, unsigned block, std::size_t lds, A... args) {
        if (grid == 0) return;
        hipEvent_t a = nullptr;
        timer.begin(name, stream_, a);
        hipLaunchKernelGGL(kernel, dim3(grid), dim3(block), lds, stream_, args...);
        SMX_LAUNCH_CHECK(name);
        timer.end(name, stream_, a);
    }

    Model model_;
    bool uploaded_ = false;
    hipStream_t stream_ = nullptr;
    void* params_ = nullptr;
    std::vector<InteractionDev> inter_;
    std::vector<ProductDev> prod_;
    std::vector<ReadoutDev> ro_;
    DRadial rad_{};
    DZbl zbl_{};
    const float* embed_table_ = nullptr;
    const double* atomic_e_ = nullptr;
    int embed_dim_ = 0;
    Arena work_;
    PinnedArena host_in_, host_out_;
    const double* energies_ = nullptr;
    const double* forces_ = nullptr;
    std::size_t num_energies_ = 0, num_forces_ = 0;
    // last call's stage buffers (device) for the debug hook
    std::map<std::string, std::pair<const float*, std::size_t>> stages_;
};

// ---- model upload: every table into one device block

struct Packer {
    std::vector<char> bytes;
    template <class T>
    std::size_t put(const std::vector<T>& v) {
        std::size_t at = (bytes.size() + 255) & ~static_cast<std::size_t>(255);
        bytes.resize(at + std::max<std::size_t>(1, v.size()) * sizeof(T), 0);
        if (!v.empty()) std::memcpy(bytes.data() + at, v.data(), v.size() * sizeof(T));
        return at;
    }
};

void Evaluator::upload_model() {
    Packer pk;
    struct LinOff {
        std::size_t instr, bf, elem, W, bias, om, im;
        bool has_bias, has_om, has_im;
        int in_dim, out_dim;
        std::vector<int> blocks;
    };
    auto put_lin = [&](const LinearTables& T) {
        return LinOff{pk.put(T.instr), pk.put(T.block_first), pk.put(T.elem), pk.put(T.weights), pk.put(T.bias),
                      pk.put(T.out_mask), pk.put(T.in_mask), !T.bias.empty(), !T.out_mask.empty(),
                      !T.in_mask.empty(), T.in_dim, T.out_dim, T.out_blocks};
    };
    struct MlpOff {
        std::size_t layers, eps, params, rows, wt, tape;
    };
    auto put_mlp = [&](const MlpTables& T) {
        return MlpOff{pk.put(T.layers), pk.put(T.eps), pk.put(T.params), pk.put(T.type_rows), pk.put(T.wt_offset),
                      pk.put(T.tape_offset)};
    };
    const Model& M = model_;
    const int nt = static_cast<int>(M.atomic_numbers.size());
    // embedding rows per type (FP64 on the host)
    std::vector<float> table;
    embed_dim_ = M.embedding.out.dim;
    for (int t = 0; t < nt; ++t) {
        const LinearTables& T = M.embedding.fwd;
        for (int j = 0; j < T.out_dim; ++j) {
            const int b = T.elem[3 * j], ch = T.elem[3 * j + 1];
            double acc = 0.0;
            for (int q = T.block_first[b]; q < T.block_first[b + 1]; ++q) {
                const int* I = &T.instr[6 * q];
                for (int u = 0; u < I[1]; ++u)
                    if (I[0] + u * I[2] == M.model_indices[t]) acc += T.weights[I[3] + u * I[5] + ch];
            }
            if (!T.bias.empty()) acc += T.bias[j];
            if (!T.out_mask.empty()) acc *= T.out_mask[j];
            table.push_back(static_cast<float>(acc));
        }
    }
    const std::size_t o_table = pk.put(table);
    const std::size_t o_ae = pk.put(M.atomic_energies);
    std::vector<double> r0(static_cast<std::size_t>(nt) * nt, 1.0);
    if (M.agnesi)
        for (int a = 0; a < nt; ++a)
            for (int b = 0; b < nt; ++b)
                r0[a * nt + b] = 0.5 * (M.covalent_radii[M.model_atomic_numbers[M.model_indices[a]]] +
                                        M.covalent_radii[M.model_atomic_numbers[M.model_indices[b]]]);
    const std::size_t o_r0 = pk.put(r0);
    std::vector<double> zpair(static_cast<std::size_t>(nt) * nt * 3, 0.0);
    if (M.has_zbl)
        for (int a = 0; a < nt; ++a)
            for (int b = 0; b < nt; ++b) {
                const int za = M.atomic_numbers[a], zb = M.atomic_numbers[b];
                double* pc = &zpair[3 * (static_cast<std::size_t>(a) * nt + b)];
                pc[0] = (std::pow(static_cast<double>(za), M.zbl_a_exp) + std::pow(static_cast<double>(zb), M.zbl_a_exp)) /
                        (M.zbl_a_prefactor * 0.529);
                pc[1] = 14.3996 * static_cast<double>(za * zb);
                pc[2] = M.zbl_radii[za] + M.zbl_radii[zb];
            }
    const std::size_t o_zbl = pk.put(zpair);

    struct InterOff {
        LinOff up[2], skip[2], res[2], lin1[2], lin2[2];
        std::size_t tp_paths, tp_in1, tp_out, tp_ent, tp_val, tp_cval;
        MlpOff w, d;
        std::size_t g[9];
    };
    std::vector<InterOff> io;
    for (const Interaction& I : M.interactions) {
        InterOff o{};
        const Linear* lins[5] = {&I.up, &I.skip, &I.res, &I.lin1, &I.lin2};
        LinOff* outs[5] = {o.up, o.skip, o.res, o.lin1, o.lin2};
        for (int k = 0; k < 5; ++k) {
            outs[k][0] = put_lin(lins[k]->fwd);
            outs[k][1] = put_lin(lins[k]->rev);
        }
        o.tp_paths = pk.put(I.tp.paths);
        o.tp_in1 = pk.put(I.tp.in1_slot);
        o.tp_out = pk.put(I.tp.out_slot);
        o.tp_ent = pk.put(I.tp.entries);
        o.tp_val = pk.put(I.tp.values);
        o.tp_cval = pk.put(I.tp.compiled_values);
        o.w = put_mlp(I.weights_mlp);
        o.d = put_mlp(I.density_mlp);
        const GateTables& G = I.gate;
        o.g[0] = pk.put(G.out_src);
        o.g[1] = pk.put(G.out_gate);
        o.g[2] = pk.put(G.out_const);
        o.g[3] = pk.put(G.in_kind);
        o.g[4] = pk.put(G.in_out);
        o.g[5] = pk.put(G.in_aux);
        o.g[6] = pk.put(G.in_count);
        o.g[7] = pk.put(G.in_const);
        io.push_back(o);
    }
    struct ProdOff {
        std::size_t ang, slot, terms, coef;
        LinOff lin[2];
    };
    std::vector<ProdOff> po;
    for (const ProductTables& P : M.products)
        po.push_back(ProdOff{pk.put(P.ang_src), pk.put(P.out_slot), pk.put(P.terms), pk.put(P.coef),
                             {put_lin(P.linear.fwd), put_lin(P.linear.rev)}});
    std::vector<std::array<LinOff, 4>> roo;
    for (const Readout& R : M.readouts) {
        std::array<LinOff, 4> a{};
        a[0] = put_lin(R.lin1.fwd);
        a[1] = put_lin(R.lin1.rev);
        if (R.nonlinear) {
            a[2] = put_lin(R.lin2.fwd);
            a[3] = put_lin(R.lin2.rev);
        }
        roo.push_back(a);
    }
    SMX_HIP(hipMalloc(&params_, pk.bytes.size()));
    SMX_HIP(hipMemcpy(params_, pk.bytes.data(), pk.bytes.size(), hipMemcpyHostToDevice));
    char* base = static_cast<char*>(params_);
    auto F = [&](std::size_t o) { return reinterpret_cast<const float*>(base + o); };
    auto I_ = [&](std::size_t o) { return reinterpret_cast<const int*>(base + o); };
    auto lin = [&](const LinOff& o) {
        DLinear d{o.in_dim, o.out_dim, I_(o.instr), I_(o.bf), I_(o.elem), F(o.W),
                  o.has_bias ? F(o.bias) : nullptr, o.has_om ? F(o.om) : nullptr, o.has_im ? F(o.im) : nullptr,
                  0, {}, {}, {}};
        const int nb = static_cast<int>(o.blocks.size() / 3);
        if (nb <= kLinearMaxBlocks) {
            d.nblk = nb;
            for (int b = 0; b < nb; ++b) {
                d.blk_off[b] = o.blocks[3 * b];
                d.blk_mul[b] = o.blocks[3 * b + 1];
                d.blk_d[b] = o.blocks[3 * b + 2];
            }
        }
        return d;
    };
    auto mlp = [&](const MlpTables& T, const MlpOff& o) {
        DMlp d{T.num_layers, T.radial, T.first_width, nt, T.max_hidden, T.tape_width, I_(o.layers), F(o.eps),
               F(o.params), F(o.rows), I_(o.wt), I_(o.tape), T.reg_hw, T.reg_stages, {}};
        // hidden stages from slot 0, the final linear in slot kRegStages
        for (int k = 0; T.reg_hw && k <= T.reg_stages; ++k) {
            const int* S = &T.reg_stage[6 * k];
            d.st[k < T.reg_stages ? k : kRegStages] = DMlpStage{S[0], S[1], S[2], S[3], S[4], S[5], T.reg_eps[k]};
        }
        return d;
    };
    embed_table_ = F(o_table);
    atomic_e_ = reinterpret_cast<const double*>(base + o_ae);
    rad_.nb = static_cast<int>(M.bessel.size());
    rad_.p = M.cutoff_p;
    rad_.apply_cutoff = M.apply_cutoff ? 1 : 0;
    rad_.agnesi = M.agnesi ? 1 : 0;
    rad_.num_types = nt;
    rad_.prefactor = M.prefactor;
    rad_.r_cut = M.r_cut;
    rad_.a = M.agnesi_a;
    rad_.q = M.agnesi_q;
    rad_.pp = M.agnesi_p;
    for (int k = 0; k < rad_.nb; ++k) rad_.bessel[k] = M.bessel[k];
    rad_.r0 = reinterpret_cast<const double*>(base + o_r0);
    zbl_.num_types = nt;
    zbl_.pair = reinterpret_cast<const double*>(base + o_zbl);
    for (int k = 0; k < 4; ++k) zbl_.c[k] = M.zbl_c[k];
    zbl_.p = M.zbl_p;
    for (std::size_t k = 0; k < M.interactions.size(); ++k) {
        const Interaction& I = M.interactions[k];
        const InterOff& o = io[k];
        InteractionDev d{};
        d.up = {lin(o.up[0]), lin(o.up[1])};
        d.skip = {lin(o.skip[0]), lin(o.skip[1])};
        d.res = {lin(o.res[0]), lin(o.res[1])};
        d.lin1 = {lin(o.lin1[0]), lin(o.lin1[1])};
        d.lin2 = {lin(o.lin2[0]), lin(o.lin2[1])};
        d.tp = DTp{I.tp.channels, I.tp.in1_dim, I.tp.out_dim, I.tp.numel, I.tp.slots, I.tp.in1_per_channel,
                   I.tp.num_paths, I_(o.tp_paths), I_(o.tp_in1), I_(o.tp_out), I_(o.tp_ent), F(o.tp_val),
                   I.tp.compiled, F(o.tp_cval)};
        d.wmlp = mlp(I.weights_mlp, o.w);
        d.dmlp = mlp(I.density_mlp, o.d);
        d.gate = DGate{I.gate.in_dim, I.gate.out_dim, I_(o.g[0]), I_(o.g[1]), F(o.g[2]), I_(o.g[3]),
                       I_(o.g[4]), I_(o.g[5]), I_(o.g[6]), F(o.g[7])};
        d.alpha = static_cast<float>(I.alpha);
        d.beta = static_cast<float>(I.beta);
        inter_.push_back(d);
    }
    for (std::size_t k = 0; k < M.products.size(); ++k) {
        const ProductTables& P = M.products[k];
        const ProdOff& o = po[k];
        prod_.push_back(ProductDev{DProduct{P.channels, P.angular, P.in_dim, P.out_dim, P.out_slots, P.num_terms,
                                            I_(o.ang), I_(o.slot), I_(o.terms), F(o.coef)},
                                   {lin(o.lin[0]), lin(o.lin[1])}});
    }
    for (std::size_t k = 0; k < M.readouts.size(); ++k) {
        const Readout& R = M.readouts[k];
        ReadoutDev d{};
        d.nonlinear = R.nonlinear;
        d.l1 = {lin(roo[k][0]), lin(roo[k][1])};
        if (R.nonlinear) d.l2 = {lin(roo[k][2]), lin(roo[k][3])};
        d.c = static_cast<float>(R.activation_constant);
        ro_.push_back(d);
    }
}

void Evaluator::launch_linear(const DLinear& op, int N, const float* x, float* y, const float* addend,
                              bool accumulate, const char* name) {
    if (op.nblk == 0) {
        launch(name, k_linear, blocks_for(static_cast<long long>(N) * op.out_dim, 256), 256, 0, op, N, x, y, addend,
               accumulate ? 1 : 0);
        return;
    }
    long long tiles = 0;
    for (int b = 0; b < op.nblk; ++b)
        tiles += ((static_cast<long long>(N) * op.blk_d[b] + 15) / 16) * ((op.blk_mul[b] + 63) / 64);
    if (tiles > 0x7fffffffLL) throw std::invalid_argument("MH-1: linear too large for one launch");
    launch(name, k_linear_mfma, static_cast<unsigned>(tiles), 256, 0, op, N, x, y, addend, accumulate ? 1 : 0);
}

// row stride of an MLP tile buffer: the widest layer plus 4 (two-way LDS
// bank conflicts at most on the MFMA A reads)
int mlp_ld(const DMlp& m) { return ((m.width + 3) / 4) * 4 + 4; }

// forward: two tile buffers and row statistics; reverse: three buffers (the
// adjoint, the next adjoint, the staged tape input) and four statistics per row
std::size_t mlp_lds(const DMlp& m, int waves, bool reverse) {
    const int rows = 16 * waves;
    return static_cast<std::size_t>((reverse ? 3 : 2) * rows * mlp_ld(m) + 6 * rows) * sizeof(float);
}

// waves per tile workgroup: four unless the reverse's buffers exceed the LDS budget
int mlp_waves(const DMlp& m) {
    int w = 4;
    while (w > 1 && mlp_lds(m, w, true) > kMaxLds) w /= 2;
    if (mlp_lds(m, w, true) > kMaxLds)
        throw std::domain_error("MH-1 model: an edge MLP layer is too wide for the LDS tile");
    return w;
}

void Evaluator::compute(int N, const int* types, const int* num_neigh, const int* neigh, const int* neigh_types,
                        const double* xyz, const double* r, long long E) {
    const Model& M = model_;
    const int nt = static_cast<int>(M.atomic_numbers.size());
    // ---- input checks (mace_nonlinear.cpp:475-521)
    if (N < 0 || E < 0) throw std::invalid_argument("MH-1: negative node or edge count");
    if ((N > 0 && (!types || !num_neigh)) || (E > 0 && (!neigh || !neigh_types || !xyz || !r)))
        throw std::invalid_argument("MH-1: a graph array is NULL");
    if (E > kMaxEdges) throw std::invalid_argument("MH-1: more than 2^31 edges in one call");
    long long total = 0;
    for (int i = 0; i < N; ++i) {
        if (types[i] < 0 || types[i] >= nt) throw std::invalid_argument("MH-1: node type out of range");
        if (num_neigh[i] < 0) throw std::invalid_argument("MH-1: negative neighbour count");
        total += num_neigh[i];
    }
    if (total != E) throw std::invalid_argument("MH-1: neighbour counts do not sum to the edge count");
    for (long long e = 0; e < E; ++e) {
        if (neigh[e] < 0 || neigh[e] >= N || neigh_types[e] != types[neigh[e]])
            throw std::invalid_argument("MH-1: edge source out of range or of the wrong type");
        if (!(r[e] > 0.0) || !std::isfinite(r[e]) || !std::isfinite(xyz[3 * e]) || !std::isfinite(xyz[3 * e + 1]) ||
            !std::isfinite(xyz[3 * e + 2]))
            throw std::invalid_argument("MH-1: edge length or vector is not finite and positive");
    }
    // past the checks a call replaces the results (a rejected graph leaves the last ones)
    num_energies_ = num_forces_ = 0;
    ensure_device();
    // ---- host-side graph arrays
    std::vector<int> offsets(N + 1, 0), tt(E), t_off(N + 1, 0), t_edges(E);
    for (int i = 0; i < N; ++i) offsets[i + 1] = offsets[i] + num_neigh[i];
    for (int i = 0; i < N; ++i)
        for (int e = offsets[i]; e < offsets[i + 1]; ++e) tt[e] = types[i];
    for (long long e = 0; e < E; ++e) ++t_off[neigh[e] + 1];
    for (int i = 0; i < N; ++i) t_off[i + 1] += t_off[i];
    {
        std::vector<int> fill(t_off.begin(), t_off.end() - 1);
        for (long long e = 0; e < E; ++e) t_edges[fill[neigh[e]]++] = static_cast<int>(e);
    }
    const int NY = M.num_lm, R = static_cast<int>(M.bessel.size());
    const int L = static_cast<int>(M.interactions.size());
    // ---- workspace layout
    Layout lay;
    const std::size_t o_types = lay.add<int>(N), o_off = lay.add<int>(N + 1), o_src = lay.add<int>(E),
                      o_ts = lay.add<int>(E), o_tt = lay.add<int>(E), o_toff = lay.add<int>(N + 1),
                      o_tedge = lay.add<int>(E), o_xyz = lay.add<double>(3 * E), o_r = lay.add<double>(E),
                      o_Y = lay.add<float>(static_cast<std::size_t>(E) * NY), o_cut = lay.add<float>(E),
                      o_rad = lay.add<float>(static_cast<std::size_t>(E) * M.bessel.size()),
                      o_feat0 = lay.add<float>(static_cast<std::size_t>(N) * embed_dim_);
    struct LayerOff {
        std::size_t up, res, skip, msg, dens, lin1, pre, gated, iout, feat, wraw, draw, wtape, dtape;
        std::size_t a_feat, contr, a_iout, a_gated, a_pre, a_lin, a_msg, a_up, a_dens, wadj, a1, adraw;
    };
    std::vector<LayerOff> lo(L);
    for (int k = 0; k < L; ++k) {
        const Interaction& I = M.interactions[k];
        const std::size_t n = N;
        LayerOff& o = lo[k];
        o.up = lay.add<float>(n * I.up.out.dim);
        o.res = lay.add<float>(n * I.res.out.dim);
        o.skip = lay.add<float>(n * I.skip.out.dim);
        o.msg = lay.add<float>(n * I.tp.out_dim);
        o.dens = lay.add<float>(n);
        o.lin1 = lay.add<float>(n * I.lin1.out.dim);
        o.pre = lay.add<float>(n * I.gate.in_dim);
        o.gated = lay.add<float>(n * I.gate.out_dim);
        o.iout = lay.add<float>(n * I.lin2.out.dim);
        o.feat = lay.add<float>(n * M.products[k].out_dim);
        o.wraw = lay.add<float>(static_cast<std::size_t>(E) * I.tp.numel);
        // the register-form kernels recompute the hidden stages and keep no tape
        o.wtape = lay.add<float>(static_cast<std::size_t>(E) * (I.weights_mlp.reg_hw ? 0 : I.weights_mlp.tape_width));
        o.dtape = lay.add<float>(static_cast<std::size_t>(E) * (I.density_mlp.reg_hw ? 0 : I.density_mlp.tape_width));
        o.draw = lay.add<float>(E);
        o.a_feat = lay.add<float>(n * M.products[k].out_dim);
        o.contr = lay.add<float>(n * M.products[k].out_dim);
        o.a_iout = lay.add<float>(n * I.lin2.out.dim);
        o.a_gated = lay.add<float>(n * I.gate.out_dim);
        o.a_pre = lay.add<float>(n * I.gate.in_dim);
        o.a_lin = lay.add<float>(n * I.gate.in_dim);
        o.a_msg = lay.add<float>(n * I.tp.out_dim);
        o.a_up = lay.add<float>(n * I.up.out.dim);
        o.a_dens = lay.add<float>(n);
        o.wadj = lay.add<float>(static_cast<std::size_t>(E) * I.tp.numel);
        o.a1 = lay.add<float>(static_cast<std::size_t>(E) * I.tp.in1_dim);
        o.adraw = lay.add<float>(E);
    }
    int ro_width = 1;
    for (const Readout& ro : M.readouts) ro_width = std::max(ro_width, ro.nonlinear ? ro.lin1.out.dim : 1);
    int mlpg_width = 0;  // the split reverse's [E][width] buffer
    for (const InteractionDev& I : inter_)
        for (const DMlp* m : {&I.wmlp, &I.dmlp})
            if (mlp_split(*m)) mlpg_width = std::max(mlpg_width, m->reg_hw);
    const std::size_t o_elems = lay.add<int>(N);
    const std::size_t o_ro = lay.add<float>(static_cast<std::size_t>(L) * N),
                      o_h = lay.add<float>(static_cast<std::size_t>(N) * ro_width),
                      o_act = lay.add<float>(static_cast<std::size_t>(N) * ro_width),
                      o_ones = lay.add<float>(N), o_radadj = lay.add<float>(static_cast<std::size_t>(E) * R),
                      o_mlpg = lay.add<float>(static_cast<std::size_t>(E) * mlpg_width),
                      o_Yadj = lay.add<float>(static_cast<std::size_t>(E) * NY), o_cadj = lay.add<float>(E),
                      o_en = lay.add<double>(N), o_nf = lay.add<double>(3 * E);
    work_.reserve(lay.size());
    char* W = work_.base();
    auto f = [&](std::size_t o) { return reinterpret_cast<float*>(W + o); };
    auto ip = [&](std::size_t o) { return reinterpret_cast<int*>(W + o); };
    auto dp = [&](std::size_t o) { return reinterpret_cast<double*>(W + o); };
    // the host inputs lead the layout: staged at their device offsets in pinned memory, one transfer
    const std::size_t in_end = o_r + sizeof(double) * static_cast<std::size_t>(E);
    host_in_.reserve(in_end);
    char* H = host_in_.base();
    auto put = [&](std::size_t o, const void* src, std::size_t bytes) {
        if (bytes) std::memcpy(H + o, src, bytes);
    };
    put(o_types, types, sizeof(int) * N);
    put(o_off, offsets.data(), sizeof(int) * (N + 1));
    put(o_src, neigh, sizeof(int) * E);
    put(o_ts, neigh_types, sizeof(int) * E);
    put(o_tt, tt.data(), sizeof(int) * E);
    put(o_toff, t_off.data(), sizeof(int) * (N + 1));
    put(o_tedge, t_edges.data(), sizeof(int) * E);
    put(o_xyz, xyz, sizeof(double) * 3 * E);
    put(o_r, r, sizeof(double) * E);
    SMX_HIP(hipMemcpyAsync(W, H, in_end, hipMemcpyHostToDevice, stream_));
    std::vector<int> midx(N);
    for (int i = 0; i < N; ++i) midx[i] = M.model_indices[types[i]];
    if (N) SMX_HIP(hipMemcpyAsync(W + o_elems, midx.data(), sizeof(int) * N, hipMemcpyHostToDevice, stream_));
    const int* d_types = ip(o_types);
    const int* d_off = ip(o_off);
    const int* d_src = ip(o_src);
    const int* d_ts = ip(o_ts);
    const int* d_tt = ip(o_tt);
    const double* d_xyz = dp(o_xyz);
    const double* d_r = dp(o_r);
    float* Y = f(o_Y);
    float* cut = f(o_cut);
    const unsigned eg = blocks_for(E, 256);
    switch (M.l_max) {
        case 0: launch("mh1_geometry", k_geometry<0>, eg, 256, 0, E, d_xyz, d_r, rad_, d_ts, d_tt, Y, cut, f(o_rad)); break;
        case 1: launch("mh1_geometry", k_geometry<1>, eg, 256, 0, E, d_xyz, d_r, rad_, d_ts, d_tt, Y, cut, f(o_rad)); break;
        case 2: launch("mh1_geometry", k_geometry<2>, eg, 256, 0, E, d_xyz, d_r, rad_, d_ts, d_tt, Y, cut, f(o_rad)); break;
        default: launch("mh1_geometry", k_geometry<3>, eg, 256, 0, E, d_xyz, d_r, rad_, d_ts, d_tt, Y, cut, f(o_rad)); break;
    }
    const float* cut_w = M.apply_cutoff ? nullptr : cut;
    float* feats = f(o_feat0);
    launch("mh1_embed", k_embed, blocks_for(static_cast<long long>(N) * embed_dim_, 256), 256, 0, N, embed_dim_,
           d_types, embed_table_, feats);
    stages_.clear();
    const float* radf = f(o_rad);
    float* mlpg = f(o_mlpg);
    // edge MLPs: the register form when the MLP has it, else the LDS-tile kernels with a tape
    auto mlp_forward = [&](const DMlp& m, float* out, float* tape) {
        if (m.reg_hw) {
            auto k = m.reg_hw == 16 ? k_mlp_forward_r<16, kRegTilesFwd>
                   : m.reg_hw == 32 ? k_mlp_forward_r<32, kRegTilesFwd> : k_mlp_forward_r<64, kRegTilesFwd>;
            launch("mh1_mlp_forward", k, blocks_for(E, 64 * kRegTilesFwd), 256, 0, m, E, radf, d_ts, d_tt, out);
            return;
        }
        const int W = mlp_waves(m);
        launch("mh1_mlp_forward", k_mlp_forward, blocks_for(E, 16 * W), 64 * W, mlp_lds(m, W, false), m, rad_, E,
               mlp_ld(m), radf, d_ts, d_tt, out, tape);
    };
    auto mlp_reverse = [&](const DMlp& m, const float* tape, const float* gout, float* radadj) {
        if (m.reg_hw) {
            const bool split = mlp_split(m);
            if (split) {
                auto ka = m.reg_hw == 16 ? k_mlp_out_reverse_r<16, kRegTilesOut>
                        : m.reg_hw == 32 ? k_mlp_out_reverse_r<32, kRegTilesOut> : k_mlp_out_reverse_r<64, kRegTilesOut>;
                launch("mh1_mlp_out_reverse", ka, blocks_for(E, 64 * kRegTilesOut), 256, 0, m, E, gout, mlpg);
            }
            auto k = m.reg_hw == 16 ? (split ? k_mlp_reverse_r<16, kRegTilesRev, true> : k_mlp_reverse_r<16, kRegTilesRev, false>)
                   : m.reg_hw == 32 ? (split ? k_mlp_reverse_r<32, kRegTilesRev, true> : k_mlp_reverse_r<32, kRegTilesRev, false>)
                   : (split ? k_mlp_reverse_r<64, kRegTilesRev, true> : k_mlp_reverse_r<64, kRegTilesRev, false>);
            launch("mh1_mlp_reverse", k, blocks_for(E, 64 * kRegTilesRev), 256, 0, m, E, radf, d_ts, d_tt, gout,
                   static_cast<const float*>(mlpg), radadj);
            return;
        }
        const int W = mlp_waves(m);
        launch("mh1_mlp_reverse", k_mlp_reverse, blocks_for(E, 16 * W), 64 * W, mlp_lds(m, W, true), m, rad_, E,
               mlp_ld(m), tape, gout, radadj);
    };
    // ---- forward (mace_nonlinear.cpp:583-768)
    for (int k = 0; k < L; ++k) {
        const InteractionDev& I = inter_[k];
        const LayerOff& o = lo[k];
        const std::string s = std::to_string(k);
        launch_linear(I.up.fwd, N, feats, f(o.up), nullptr, false, "mh1_linear_up");
        launch_linear(I.res.fwd, N, f(o.up), f(o.res), nullptr, false, "mh1_linear_res");
        launch_linear(I.skip.fwd, N, feats, f(o.skip), nullptr, false, "mh1_linear_skip");
        mlp_forward(I.wmlp, f(o.wraw), f(o.wtape));
        mlp_forward(I.dmlp, f(o.draw), f(o.dtape));
        const unsigned tpg = blocks_for(static_cast<long long>(N) * I.tp.channels, kTpThreads);
        if (I.tp.compiled >= 0) {
            auto kf = I.tp.compiled == 0 ? k_tp_forward_c<0, 2> : I.tp.compiled == 1 ? k_tp_forward_c<0, 3>
                    : I.tp.compiled == 2 ? k_tp_forward_c<1, 2> : k_tp_forward_c<1, 3>;
            launch("mh1_tp_forward", kf, tpg, kTpThreads, 0, I.tp, N, d_off, d_src, static_cast<const float*>(f(o.up)),
                   static_cast<const float*>(Y), static_cast<const float*>(f(o.wraw)), cut_w,
                   static_cast<const float*>(f(o.draw)), f(o.msg), f(o.dens));
        } else {
            const std::size_t tp_lds = static_cast<std::size_t>(I.tp.slots + I.tp.nin1) * kTpThreads * 4;
            launch("mh1_tp_forward_table", k_tp_forward, tpg, kTpThreads, tp_lds, I.tp, N, d_off, d_src, f(o.up), Y, NY,
                   f(o.wraw), cut_w, f(o.draw), f(o.msg), f(o.dens));
        }
        launch_linear(I.lin1.fwd, N, f(o.msg), f(o.lin1), nullptr, false, "mh1_linear_1");
        launch("mh1_pregate", k_pregate, blocks_for(static_cast<long long>(N) * I.gate.in_dim, 256), 256, 0, N,
               I.gate.in_dim, f(o.lin1), f(o.res), f(o.dens), I.alpha, I.beta, f(o.pre));
        launch("mh1_gate", k_gate_forward, blocks_for(static_cast<long long>(N) * I.gate.out_dim, 256), 256, 0,
               I.gate, N, f(o.pre), f(o.gated));
        launch_linear(I.lin2.fwd, N, f(o.gated), f(o.iout), nullptr, false, "mh1_linear_2");
        const ProductDev& P = prod_[k];
        const int* elems = M.products[k].agnostic ? nullptr : ip(o_elems);
        launch("mh1_product_forward", k_product_forward, blocks_for(static_cast<long long>(N) * P.P.channels, 256), 256,
               0, P.P, N, elems, f(o.iout), f(o.contr));
        launch_linear(P.lin.fwd, N, f(o.contr), f(o.feat), M.products[k].use_sc ? f(o.skip) : nullptr, false,
                      "mh1_product_linear");
        feats = f(o.feat);
        stages_["up" + s] = {f(o.up), static_cast<std::size_t>(N) * M.interactions[k].up.out.dim};
        stages_["msg" + s] = {f(o.msg), static_cast<std::size_t>(N) * M.interactions[k].tp.out_dim};
        stages_["density" + s] = {f(o.dens), static_cast<std::size_t>(N)};
        stages_["w" + s] = {f(o.wraw), static_cast<std::size_t>(E) * M.interactions[k].tp.numel};
        stages_["pre_gate" + s] = {f(o.pre), static_cast<std::size_t>(N) * M.interactions[k].gate.in_dim};
        stages_["interaction_out" + s] = {f(o.iout), static_cast<std::size_t>(N) * M.interactions[k].lin2.out.dim};
        stages_["features" + s] = {f(o.feat), static_cast<std::size_t>(N) * M.products[k].out_dim};
    }
    // ---- readouts and energies
    float* ro = f(o_ro);
    for (int k = 0; k < L; ++k) {
        const ReadoutDev& R_ = ro_[k];
        const float* x = f(lo[k].feat);
        if (!R_.nonlinear) {
            launch_linear(R_.l1.fwd, N, x, ro + static_cast<std::size_t>(k) * N, nullptr, false, "mh1_readout");
        } else {
            const long long nh = static_cast<long long>(N) * R_.l1.fwd.out_dim;
            launch_linear(R_.l1.fwd, N, x, f(o_h), nullptr, false, "mh1_readout");
            launch("mh1_readout_act", k_silu_scaled, blocks_for(nh, 256), 256, 0, nh, R_.c, f(o_h),
                   static_cast<const float*>(nullptr), f(o_act));
            launch_linear(R_.l2.fwd, N, f(o_act), ro + static_cast<std::size_t>(k) * N, nullptr, false, "mh1_readout");
        }
    }
    launch("mh1_energies", k_energies, blocks_for(N, 256), 256, 0, N, L, d_types, atomic_e_, M.scale, M.shift, ro,
           d_off, d_ts, d_r, zbl_, M.has_zbl ? 1 : 0, dp(o_en));
    // ---- reverse (mace_nonlinear.cpp:782-1000)
    const float scale_f = static_cast<float>(M.scale);
    launch("mh1_fill", k_fill, blocks_for(N, 256), 256, 0, static_cast<long long>(N), scale_f, f(o_ones));
    for (int k = 0; k < L; ++k) {
        const ReadoutDev& R_ = ro_[k];
        float* af = f(lo[k].a_feat);
        if (!R_.nonlinear) {
            launch_linear(R_.l1.rev, N, f(o_ones), af, nullptr, false, "mh1_readout_reverse");
        } else {
            const long long nh = static_cast<long long>(N) * R_.l1.fwd.out_dim;
            launch_linear(R_.l1.fwd, N, f(lo[k].feat), f(o_h), nullptr, false, "mh1_readout_reverse");
            launch_linear(R_.l2.rev, N, f(o_ones), f(o_act), nullptr, false, "mh1_readout_reverse");
            launch("mh1_readout_act", k_silu_scaled, blocks_for(nh, 256), 256, 0, nh, R_.c, f(o_h), f(o_act), f(o_act));
            launch_linear(R_.l1.rev, N, f(o_act), af, nullptr, false, "mh1_readout_reverse");
        }
    }
    float* radadj = f(o_radadj);
    float* Yadj = f(o_Yadj);
    float* cadj = f(o_cadj);
    launch("mh1_fill", k_fill, blocks_for(static_cast<long long>(E) * R, 256), 256, 0, static_cast<long long>(E) * R,
           0.0f, radadj);
    launch("mh1_fill", k_fill, blocks_for(static_cast<long long>(E) * NY, 256), 256, 0,
           static_cast<long long>(E) * NY, 0.0f, Yadj);
    launch("mh1_fill", k_fill, eg, 256, 0, static_cast<long long>(E), 0.0f, cadj);
    for (int k = L - 1; k >= 0; --k) {
        const InteractionDev& I = inter_[k];
        const ProductDev& P = prod_[k];
        const LayerOff& o = lo[k];
        const int* elems = M.products[k].agnostic ? nullptr : ip(o_elems);
        const float* in_feats = k == 0 ? f(o_feat0) : f(lo[k - 1].feat);
        // product: a_contracted = linear^T(a_feat), then through the contraction
        float* a_contr = f(o.contr);
        launch_linear(P.lin.rev, N, f(o.a_feat), a_contr, nullptr, false, "mh1_product_linear_reverse");
        launch("mh1_product_reverse", k_product_reverse, blocks_for(static_cast<long long>(N) * P.P.channels, 256),
               256, 0, P.P, N, elems, f(o.iout), a_contr, f(o.a_iout));
        launch_linear(I.lin2.rev, N, f(o.a_iout), f(o.a_gated), nullptr, false, "mh1_linear_2_reverse");
        launch("mh1_gate_reverse", k_gate_reverse, blocks_for(static_cast<long long>(N) * I.gate.in_dim, 256), 256, 0,
               I.gate, N, f(o.pre), f(o.a_gated), f(o.a_pre));
        launch("mh1_norm_reverse", k_norm_reverse, blocks_for(static_cast<long long>(N) * kWave, 256), 256, 0, N,
               I.gate.in_dim, f(o.a_pre), f(o.lin1), f(o.dens), I.alpha, I.beta, f(o.a_lin), f(o.a_dens));
        launch_linear(I.lin1.rev, N, f(o.a_lin), f(o.a_msg), nullptr, false, "mh1_linear_1_reverse");
        launch_linear(I.res.rev, N, f(o.a_pre), f(o.a_up), nullptr, false, "mh1_linear_res_reverse");
        const unsigned tpg = blocks_for(static_cast<long long>(N) * I.tp.channels, kTpThreads);
        if (I.tp.compiled >= 0) {
            auto kr = I.tp.compiled == 0 ? k_tp_reverse_c<0, 2> : I.tp.compiled == 1 ? k_tp_reverse_c<0, 3>
                    : I.tp.compiled == 2 ? k_tp_reverse_c<1, 2> : k_tp_reverse_c<1, 3>;
            launch("mh1_tp_reverse", kr, tpg, kTpThreads, 0, I.tp, N, d_off, d_src,
                   static_cast<const float*>(f(o.up)), static_cast<const float*>(Y),
                   static_cast<const float*>(f(o.wraw)), cut_w, static_cast<const float*>(f(o.draw)),
                   static_cast<const float*>(f(o.a_msg)), static_cast<const float*>(f(o.a_dens)), f(o.wadj), f(o.a1),
                   Yadj, M.apply_cutoff ? static_cast<float*>(nullptr) : cadj, f(o.adraw));
        } else {
            const std::size_t tp_lds = static_cast<std::size_t>(I.tp.slots + 2 * I.tp.nin1 + NY) * kTpThreads * 4;
            launch("mh1_tp_reverse_table", k_tp_reverse, tpg, kTpThreads, tp_lds, I.tp, N, d_off, d_src, f(o.up), Y, NY,
                   f(o.wraw), cut_w, f(o.draw), f(o.a_msg), f(o.a_dens), f(o.wadj), f(o.a1), Yadj,
                   M.apply_cutoff ? nullptr : cadj, f(o.adraw));
        }
        launch("mh1_gather_sources", k_gather_sources,
               blocks_for(static_cast<long long>(N) * I.tp.in1_dim, 256), 256, 0, N, I.tp.in1_dim, ip(o_toff),
               ip(o_tedge), f(o.a1), f(o.a_up));
        mlp_reverse(I.wmlp, f(o.wtape), f(o.wadj), radadj);
        mlp_reverse(I.dmlp, f(o.dtape), f(o.adraw), radadj);
        stages_["w_adj" + std::to_string(k)] = {f(o.wadj), static_cast<std::size_t>(E) * M.interactions[k].tp.numel};
        stages_["density_adj" + std::to_string(k)] = {f(o.adraw), static_cast<std::size_t>(E)};
        if (k > 0) {
            // a_feat[k-1] += up^T(a_up) + skip^T(a_skip), a_skip = a_feat[k] when the product has a skip
            float* prev = f(lo[k - 1].a_feat);
            launch_linear(I.up.rev, N, f(o.a_up), prev, nullptr, true, "mh1_linear_up_reverse");
            if (M.products[k].use_sc)
                launch_linear(I.skip.rev, N, f(o.a_feat), prev, nullptr, true, "mh1_linear_skip_reverse");
        }
        (void)in_feats;
    }
    switch (M.l_max) {
        case 0: launch("mh1_edge_forces", k_edge_forces<0>, eg, 256, 0, E, d_xyz, d_r, rad_, d_ts, d_tt, radadj,
                       M.apply_cutoff ? static_cast<const float*>(nullptr) : cadj, Yadj, zbl_, M.has_zbl ? 1 : 0,
                       M.scale, dp(o_nf)); break;
        case 1: launch("mh1_edge_forces", k_edge_forces<1>, eg, 256, 0, E, d_xyz, d_r, rad_, d_ts, d_tt, radadj,
                       M.apply_cutoff ? static_cast<const float*>(nullptr) : cadj, Yadj, zbl_, M.has_zbl ? 1 : 0,
                       M.scale, dp(o_nf)); break;
        case 2: launch("mh1_edge_forces", k_edge_forces<2>, eg, 256, 0, E, d_xyz, d_r, rad_, d_ts, d_tt, radadj,
                       M.apply_cutoff ? static_cast<const float*>(nullptr) : cadj, Yadj, zbl_, M.has_zbl ? 1 : 0,
                       M.scale, dp(o_nf)); break;
        default: launch("mh1_edge_forces", k_edge_forces<3>, eg, 256, 0, E, d_xyz, d_r, rad_, d_ts, d_tt, radadj,
                        M.apply_cutoff ? static_cast<const float*>(nullptr) : cadj, Yadj, zbl_, M.has_zbl ? 1 : 0,
                        M.scale, dp(o_nf)); break;
    }
    stages_["Yadj"] = {Yadj, static_cast<std::size_t>(E) * NY};
    stages_["rad_adj"] = {radadj, static_cast<std::size_t>(E) * R};
    // energies and per-edge forces end the layout: one transfer into pinned memory
    const std::size_t out_end = o_nf + sizeof(double) * 3 * static_cast<std::size_t>(E);
    host_out_.reserve(out_end - o_en);
    SMX_HIP(hipMemcpyAsync(host_out_.base(), W + o_en, out_end - o_en, hipMemcpyDeviceToHost, stream_));
    SMX_HIP(hipStreamSynchronize(stream_));
    energies_ = reinterpret_cast<const double*>(host_out_.base());
    forces_ = reinterpret_cast<const double*>(host_out_.base() + (o_nf - o_en));
    num_energies_ = static_cast<std::size_t>(N);
    num_forces_ = 3 * static_cast<std::size_t>(E);
    timer.collect();
}

std::vector<float> Evaluator::stage(const std::string& name) {
    auto it = stages_.find(name);
    if (it == stages_.end()) throw std::invalid_argument("MH-1: no stage named '" + name + "' in the last call");
    std::vector<float> out(it->second.second);
    if (!out.empty())
        SMX_HIP(hipMemcpyAsync(out.data(), it->second.first, out.size() * sizeof(float), hipMemcpyDeviceToHost,
                               stream_));
    SMX_HIP(hipStreamSynchronize(stream_));
    return out;
}

template <class F>
int32_t guarded(F&& fn) {
    try {
        fn();
        return SMX_OK;
    } catch (const std::bad_alloc&) {
        set_last_error("out of memory (device or host allocation failed)");
        return SMX_ERR_OUT_OF_MEMORY;
    } catch (const std::domain_error& e) {
        set_last_error(e.what());
        return SMX_ERR_UNSUPPORTED;
    } catch (const std::invalid_argument& e) {
        set_last_error(e.what());
        return SMX_ERR_INVALID_ARGUMENT;
    } catch (const std::out_of_range& e) {
        set_last_error(e.what());
        return SMX_ERR_INVALID_ARGUMENT;
    } catch (const std::logic_error& e) {
        set_last_error(e.what());
        return SMX_ERR_LOGIC;
    } catch (const std::exception& e) {
        set_last_error(e.what());
        return SMX_ERR_RUNTIME;
    } catch (...) {
        set_last_error("unknown error");
        return SMX_ERR_RUNTIME;
    }
}

}  // namespace
}  // namespace mh1
}  // namespace smx

struct SmxMh1Evaluator {
    std::unique_ptr<smx::mh1::Evaluator> impl;
};

namespace {
smx::mh1::Evaluator& ev_of(SmxMh1Evaluator* ev) {
    if (!ev || !ev->impl) throw std::invalid_argument("MH-1 evaluator handle is NULL");
    return *ev->impl;
}
const smx::mh1::Evaluator& ev_of(const SmxMh1Evaluator* ev) {
    if (!ev || !ev->impl) throw std::invalid_argument("MH-1 evaluator handle is NULL");
    return *ev->impl;
}
}  // namespace

extern "C" {

int32_t smx_mh1_create(const char* model_path, const char* head, SmxMh1Evaluator** out) {
    return smx::mh1::guarded([&] {
        if (!model_path || !out) throw std::invalid_argument("model path and output handle are required");
        *out = nullptr;
        auto h = std::make_unique<SmxMh1Evaluator>();
        h->impl = std::make_unique<smx::mh1::Evaluator>(model_path, head ? head : "");
        *out = h.release();
    });
}

void smx_mh1_destroy(SmxMh1Evaluator* ev) { delete ev; }

int32_t smx_mh1_info(const SmxMh1Evaluator* ev, SmxMh1Info* info) {
    return smx::mh1::guarded([&] {
        if (!info) throw std::invalid_argument("info is NULL");
        const smx::mh1::Model& M = ev_of(ev).model();
        SmxMh1Info v{};
        v.struct_size = sizeof(SmxMh1Info);
        v.num_elements = static_cast<int32_t>(M.atomic_numbers.size());
        v.l_max = M.l_max;
        v.num_interactions = static_cast<int32_t>(M.interactions.size());
        v.is_mh1_family = M.family ? 1 : 0;
        v.node_channels = M.family_node_channels;
        v.edge_channels = M.family_edge_channels;
        v.radial_size = M.family_radial;
        v.has_zbl = M.has_zbl ? 1 : 0;
        v.r_cut = M.r_cut;
        *info = v;
    });
}

int32_t smx_mh1_family_rejection(const SmxMh1Evaluator* ev, const char** reason) {
    return smx::mh1::guarded([&] {
        if (!reason) throw std::invalid_argument("reason is NULL");
        *reason = ev_of(ev).model().family_rejection.c_str();
    });
}

int32_t smx_mh1_atomic_numbers(const SmxMh1Evaluator* ev, int32_t* out, int32_t capacity) {
    int32_t n = 0;
    const int32_t rc = smx::mh1::guarded([&] {
        const auto& z = ev_of(ev).model().atomic_numbers;
        n = static_cast<int32_t>(z.size());
        for (int32_t i = 0; out && i < std::min(n, capacity); ++i) out[i] = z[i];
    });
    return rc ? rc : n;
}

int32_t smx_mh1_atomic_energies(const SmxMh1Evaluator* ev, double* out, int32_t capacity) {
    int32_t n = 0;
    const int32_t rc = smx::mh1::guarded([&] {
        const auto& e = ev_of(ev).model().atomic_energies;
        n = static_cast<int32_t>(e.size());
        for (int32_t i = 0; out && i < std::min(n, capacity); ++i) out[i] = e[i];
    });
    return rc ? rc : n;
}

int32_t smx_mh1_selected_head(const SmxMh1Evaluator* ev, const char** name) {
    return smx::mh1::guarded([&] {
        if (!name) throw std::invalid_argument("name is NULL");
        *name = ev_of(ev).model().selected_head.c_str();
    });
}

int32_t smx_mh1_compute_node_energies_forces(SmxMh1Evaluator* ev, int32_t num_nodes, const int32_t* node_types,
                                             const int32_t* num_neigh, const int32_t* neigh_indices,
                                             const int32_t* neigh_types, const double* xyz, const double* r,
                                             int64_t num_edges) {
    return smx::mh1::guarded([&] {
        ev_of(ev).compute(num_nodes, node_types, num_neigh, neigh_indices, neigh_types, xyz, r, num_edges);
    });
}

int32_t smx_mh1_node_energies(SmxMh1Evaluator* ev, double* out, int64_t capacity) {
    return smx::mh1::guarded([&] {
        const auto v = ev_of(ev).node_energies();
        if (v.size == 0) return;
        if (!out || capacity < static_cast<int64_t>(v.size)) throw std::invalid_argument("output buffer too small");
        std::copy(v.data, v.data + v.size, out);
    });
}

int32_t smx_mh1_node_forces(SmxMh1Evaluator* ev, double* out, int64_t capacity) {
    return smx::mh1::guarded([&] {
        const auto v = ev_of(ev).node_forces();
        if (v.size == 0) return;
        if (!out || capacity < static_cast<int64_t>(v.size)) throw std::invalid_argument("output buffer too small");
        std::copy(v.data, v.data + v.size, out);
    });
}

int32_t smx_mh1_debug_stage(SmxMh1Evaluator* ev, const char* name, float* out, int64_t capacity, int64_t* count) {
    return smx::mh1::guarded([&] {
        if (!name) throw std::invalid_argument("stage name is NULL");
        const std::vector<float> v = ev_of(ev).stage(name);
        if (count) *count = static_cast<int64_t>(v.size());
        if (out) std::copy(v.begin(), v.begin() + std::min<int64_t>(capacity, static_cast<int64_t>(v.size())), out);
    });
}

int32_t smx_mh1_set_kernel_timing(SmxMh1Evaluator* ev, int32_t enabled) {
    return smx::mh1::guarded([&] {
        auto& t = ev_of(ev).timer;
        t.enabled = enabled != 0;
        t.totals.clear();
        t.order.clear();
    });
}

int32_t smx_mh1_kernel_timing(SmxMh1Evaluator* ev, int32_t index, const char** name, double* total_ms,
                              int64_t* launches) {
    int32_t n = 0;
    const int32_t rc = smx::mh1::guarded([&] {
        auto& t = ev_of(ev).timer;
        n = static_cast<int32_t>(t.order.size());
        if (index >= 0 && index < n) {
            const std::string& k = t.order[index];
            if (name) *name = k.c_str();
            if (total_ms) *total_ms = t.totals[k].first;
            if (launches) *launches = t.totals[k].second;
        }
    });
    return rc ? rc : n;
}

}  // extern "C"
