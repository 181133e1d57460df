// MACE interaction kernels for MI355X (gfx950, wave64), FP32 with the
// reference's FP64 islands (readout, node energies, directed forces, source
// adjoint accumulation).
//
// Mapping: one workgroup owns one receiver (edge kernels) or one node (node
// kernels); lanes are channels, so every per-channel table (spline
// coefficients, H0/H1 features, polynomial coefficients) is read coalesced
// while the per-edge quantities (Y, dY, spline interval, direction) are
// wave-uniform and come through the scalar cache.  Receivers are owned, never
// shared: every node quantity is a deterministic segment sum without atomics.
//
// Reference math (libsymmetrix/source):
//   R0 forward  mace.cpp:1356-1403 (first_interaction.cpp:620-883)
//   R0 reverse  mace.cpp:1486-1560 (first_interaction.cpp:992-1335)
//   M0          mace.cpp:1639-1689, multivariate_polynomial.cpp:11-131
//   R1 forward  mace.cpp:2023-2084 (h1_phi1.cpp:1385-1845)
//   R1 reverse  mace.cpp:2199-2303 (factorized_execution.cpp:471-1460)
//   M1/H2/readouts and their adjoints mace.cpp:2461-2657 with the FP64
//   policy of mace_kokkos.hpp:1805-1828
#include <algorithm>
#include <stdexcept>
#include <string>
#include <type_traits>

#include "device_common.hpp"
#include "harmonic_gradients.hpp"
#include "edge_kernels.hpp"
#include "kernels.hpp"
#include "polynomial.hpp"
#include "product_tables.hpp"
#include "shapes.hpp"

namespace smx {
namespace {

using namespace edge;

typedef float v4f __attribute__((ext_vector_type(4)));

// Sum over the workgroup (C lanes, one value each); every lane gets the total.
template <int C>
__device__ __forceinline__ double block_sum(double v, double* sbuf) {
    v = wave_sum<Lanes<C>::WIDTH>(v);
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    if (lane == 0) sbuf[wave] = v;
    __syncthreads();
    double t = 0.0;
#pragma unroll
    for (int w = 0; w < Lanes<C>::NW; ++w) t += sbuf[w];
    __syncthreads();
    return t;
}

// ---------------------------------------------------------------------------
// Layer 1: Phi0[i,lm,k] = sum_j R0_{l,k}(r_ij) Y_lm(ij) H0[type_j,k]
// The forward parts of the receiver's records (in execution order, the
// source type in the activity field) are staged through LDS; the table
// row's coefficients stay in registers while consecutive slots share it.
// ---------------------------------------------------------------------------
template <int C, int LMAX>
__global__ __launch_bounds__(C) void k_r0_forward(int r0, long long e0, const int* __restrict__ offsets,
                                                  const float* __restrict__ erec, const float4* __restrict__ R0c,
                                                  const float* __restrict__ H0, float* __restrict__ Phi0) {
    using S = Shape<LMAX, 0>;
    constexpr int NY = S::NY, NF = (LMAX + 1) * C;
    const int li = xcd_remap(blockIdx.x, gridDim.x);
    const int i = r0 + li;
    const int k = threadIdx.x;
    float acc[NY];
#pragma unroll
    for (int v = 0; v < NY; ++v) acc[v] = 0.0f;
    const int ea = offsets[i], eb = offsets[i + 1];
    __shared__ stage4 stage_buf[2 * RecordStage<C, S::REC_F>::SLOTS];
    const stage4* src = reinterpret_cast<const stage4*>(erec) + static_cast<std::size_t>(ea - e0) * (S::REC_F / 4);
    float4 cc[LMAX + 1];
    int cached = -1;
    staged_records<C, S::REC_F>(stage_buf, src, eb - ea, [&](const float* chunk, int /*first*/, int n)
                                                             __attribute__((always_inline)) {
        for (int j = 0; j < n; ++j) {
            const float* rec = chunk + j * S::REC_F;
            if (!edge_active(rec)) continue;
            const float x = rec[0];
            const int iv = __float_as_int(rec[1]);
            const float xx = x * x, xxx = xx * x;
            const float h0 = H0[(__float_as_int(rec[2]) - 1) * C + k];
            if (iv != cached) {
                cached = iv;
                const float4* cf = R0c + static_cast<std::size_t>(iv) * NF + k;
                static_for<0, LMAX + 1>([&](auto lc) { cc[lc] = cf[lc * C]; });
            }
            static_for<0, LMAX + 1>([&](auto lc) {
                constexpr int l = lc;
                const float rh = spline_value(cc[l], x, xx, xxx) * h0;
                static_for<0, 2 * l + 1>([&](auto mc) {
                    constexpr int lm = l * l + mc;
                    acc[lm] += rh * rec[S::REC_Y + lm];
                });
            });
        }
    });
#pragma unroll
    for (int v = 0; v < NY; ++v) Phi0[(static_cast<std::size_t>(li) * NY + v) * C + k] = acc[v];
}

// degree l of harmonic index q = l^2 + m
constexpr int harmonic_degree(int q) {
    int l = 0;
    while ((l + 1) * (l + 1) <= q) ++l;
    return l;
}

// Layer-1 reverse: node_forces[e] -= sum_k sum_lm Phi0_adj[i,lm,k] H0 (u dR Y + R dY)
// (records in execution order; each slot's force goes to its edge's row).
// The gradient term goes through the identity of the records' gradients
// (harmonic_gradients.hpp): dY^c_q = (sum_q' G[q][c][q'] Y_q' - l u_c Y_q) / r
// with q' of degree l - 1, so with Q[c][q'] = sum_q Phi0_adj[q] G[q][c][q']
// formed once per receiver and s_l = sum_m Phi0_adj[lm] Y_lm,
//   sum_lm Phi0_adj[lm] R_l dY^c_lm = (sum_l R_l sum_q' Y_q' Q[c][q'] - u_c sum_l l R_l s_l) / r,
// 43 products per edge and channel at l_max 3 instead of 64.  1/r is the
// trace of the l = 1 gradient block (a tangent projector: trace 2) over 2 sqrt(3).
template <int C, int LMAX, bool ACCUMULATE>
__global__ __launch_bounds__(C) void k_r0_reverse(int r0, long long e0, const int* __restrict__ offsets,
                                                  const float* __restrict__ erec, const float* __restrict__ erec_b,
                                                  const float4* __restrict__ R0c, const float* __restrict__ H0,
                                                  const float* __restrict__ Phi0_adj, double* __restrict__ node_forces) {
    using S = Shape<LMAX, 0>;
    constexpr int NY = S::NY, NF = (LMAX + 1) * C;
    __shared__ float part[EdgeForceSink<C, kRecordChunk>::ROWS][kRecordChunk][3];
    EdgeForceSink<C, kRecordChunk> sink{part};
    __shared__ stage4 stage_buf[2 * RecordStage<C, S::REC>::SLOTS];
    const int li = xcd_remap(blockIdx.x, gridDim.x);
    const int i = r0 + li;
    const int k = threadIdx.x;
    float padj[NY];
#pragma unroll
    for (int v = 0; v < NY; ++v) padj[v] = Phi0_adj[(static_cast<std::size_t>(li) * NY + v) * C + k];
    // Q[c][q'] over the harmonics q' of degree < l_max
    constexpr int NQ = LMAX * LMAX;
    float qg[3][NQ > 0 ? NQ : 1];
    static_for<0, 3>([&](auto cc_) {
        constexpr int c = cc_;
        static_for<0, NQ>([&](auto qc) {
            constexpr int qp = qc, d = harmonic_degree(qp);
            float acc = 0.0f;
            static_for<0, 2 * d + 3>([&](auto mc) {
                constexpr int q = (d + 1) * (d + 1) + mc;
                constexpr double gv = kHarmonicGrad[q][c][qp - d * d];
                if constexpr (gv != 0.0) acc += padj[q] * static_cast<float>(gv);
            });
            qg[c][qp] = acc;
        });
    });
    const int ea = offsets[i], eb = offsets[i + 1];
    const stage4* srcF = reinterpret_cast<const stage4*>(erec) + static_cast<std::size_t>(ea - e0) * (S::REC_F / 4);
    const stage4* srcB = reinterpret_cast<const stage4*>(erec_b) + static_cast<std::size_t>(ea - e0) * (S::REC_B / 4);
    float4 cc[LMAX + 1];
    int cached = -1;
    staged_records2<C, S::REC_F, S::REC_B>(stage_buf, srcF, srcB, eb - ea, [&](const float* chunk, int /*first*/,
                                                                               int n) __attribute__((always_inline)) {
        for (int j = 0; j < n; ++j) {
            const float* rec = chunk + j * S::REC;
            if (!edge_active(rec)) {
                sink.zero(j);
                continue;
            }
            const float x = rec[0];
            const int iv = __float_as_int(rec[1]);
            const float xx = x * x, xxx = xx * x, x2 = 2.0f * x, xx3 = 3.0f * xx;
            const float h0 = H0[(__float_as_int(rec[2]) - 1) * C + k];
            if (iv != cached) {
                cached = iv;
                const float4* cf = R0c + static_cast<std::size_t>(iv) * NF + k;
                static_for<0, LMAX + 1>([&](auto lc) { cc[lc] = cf[lc * C]; });
            }
            // per l: s_l = sum_m adj Y_lm and the gradient sums q_c; the
            // radial factor (dR_l - l R_l / r) of s_l and R_l of q_c, the
            // common factor H0[type_j] applied once
            [[maybe_unused]] float rinv = 0.0f;
            if constexpr (LMAX >= 1)
                rinv = (rec[S::REC_DY + 1] + rec[S::REC_DY + NY + 2] + rec[S::REC_DY + 2 * NY + 3]) *
                       static_cast<float>(0.28867513459481287);  // 1 / (2 sqrt 3)
            float a = 0.0f, b0 = 0.0f, b1 = 0.0f, b2 = 0.0f;
            static_for<0, LMAX + 1>([&](auto lc) {
                constexpr int l = lc;
                const float4 c4 = cc[l];
                const float R = spline_value(c4, x, xx, xxx);
                const float dR = spline_slope(c4, x2, xx3);
                float sa = 0.0f;
                static_for<0, 2 * l + 1>([&](auto mc) {
                    constexpr int lm = l * l + mc;
                    sa += padj[lm] * rec[S::REC_Y + lm];
                });
                if constexpr (l == 0) {
                    a += dR * sa;
                } else {
                    a += (dR - static_cast<float>(l) * R * rinv) * sa;
                    float q0 = 0.0f, q1 = 0.0f, q2 = 0.0f;
                    static_for<0, 2 * l - 1>([&](auto jc) {
                        constexpr int qp = (l - 1) * (l - 1) + jc;
                        const float y = rec[S::REC_Y + qp];
                        q0 += y * qg[0][qp];
                        q1 += y * qg[1][qp];
                        q2 += y * qg[2][qp];
                    });
                    b0 += R * q0;
                    b1 += R * q1;
                    b2 += R * q2;
                }
            });
            const float u0 = rec[S::REC_U], u1 = rec[S::REC_U + 1], u2 = rec[S::REC_U + 2];
            sink.put(j, h0 * (u0 * a + rinv * b0), h0 * (u1 * a + rinv * b1), h0 * (u2 * a + rinv * b2));
        }
        sink.template flush<ACCUMULATE>(
            n, node_forces, [&](int el) { return __float_as_int(chunk[el * S::REC + S::REC - 1]); });
    });
}

// ---------------------------------------------------------------------------
// Product basis (symmetric contraction) polynomials.  Two forms:
//  * unrolled: the monomial list is a compiled table (ProductTable), every
//    term is straight-line code on the variables held in registers;
//  * table-driven: variables live in LDS (column k per lane) so the
//    wave-uniform monomial list in HBM can index them.
// Both sum the terms of an output in list order; the gradient follows the
// product rule in the reference's order (the coefficient times the other
// factors in turn, multivariate_polynomial.cpp:60-131).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float monomial(const float* xs, int C, int k, int pk) {
    const int deg = pk >> 24;
    float prod = xs[(pk & 0xff) * C + k];
    if (deg > 1) prod *= xs[((pk >> 8) & 0xff) * C + k];
    if (deg > 2) prod *= xs[((pk >> 16) & 0xff) * C + k];
    return prod;
}

// gs[v] += d f / d x_v for one term with coefficient c
__device__ __forceinline__ void monomial_grad(const float* xs, float* gs, int C, int k, int pk, float c) {
    const int deg = pk >> 24;
    const int v0 = pk & 0xff, v1 = (pk >> 8) & 0xff, v2 = (pk >> 16) & 0xff;
    if (deg == 1) {
        gs[v0 * C + k] += c;
    } else if (deg == 2) {
        const float x0 = xs[v0 * C + k], x1 = xs[v1 * C + k];
        gs[v0 * C + k] += c * x1;
        gs[v1 * C + k] += c * x0;
    } else {
        const float x0 = xs[v0 * C + k], x1 = xs[v1 * C + k], x2 = xs[v2 * C + k];
        gs[v0 * C + k] += c * x1 * x2;
        gs[v1 * C + k] += c * x0 * x2;
        gs[v2 * C + k] += c * x0 * x1;
    }
}

// Rows li of the tile workspace belong to receiver i = r0 + li; graph-wide
// arrays (types, scalar capture x, direct adjoint, energies) use i.
template <int C, int NY, int NH, class TAB>
__global__ __launch_bounds__(C) void k_m0_forward_ct(int r0, const int* __restrict__ types,
                                                     const float* __restrict__ A0, const float* __restrict__ coef,
                                                     float* __restrict__ M0, float* __restrict__ xaff) {
    const int li = blockIdx.x;
    const int i = r0 + li;
    const int k = threadIdx.x;
    float x[NY];
#pragma unroll
    for (int v = 0; v < NY; ++v) x[v] = A0[(static_cast<std::size_t>(li) * NY + v) * C + k];
    const float* cf = coef + static_cast<std::size_t>(types[i]) * TAB::NT * C + k;
    static_range<0, NH>([&](auto LMc) {
        constexpr int LM = LMc;
        const float f = poly_ct<TAB, TAB::offset[LM], TAB::offset[LM + 1], C>(x, cf);
        M0[(static_cast<std::size_t>(li) * NH + LM) * C + k] = f;
        // v4 "m0_composite" readout basis: x = M0[i, 0, :] (h1_affine_schema.hpp)
        if constexpr (LM == 0) xaff[static_cast<std::size_t>(i) * C + k] = f;
    });
}

template <int C, int NY, int NH, class TAB>
__global__ __launch_bounds__(C) void k_m0_reverse_ct(int r0, const int* __restrict__ types,
                                                     const float* __restrict__ A0, const float* __restrict__ M0_adj,
                                                     const float* __restrict__ direct, const float* __restrict__ coef,
                                                     float* __restrict__ A0_adj) {
    const int li = blockIdx.x;
    const int i = r0 + li;
    const int k = threadIdx.x;
    float x[NY], acc[NY];
#pragma unroll
    for (int v = 0; v < NY; ++v) {
        x[v] = A0[(static_cast<std::size_t>(li) * NY + v) * C + k];
        acc[v] = 0.0f;
    }
    const float* cf = coef + static_cast<std::size_t>(types[i]) * TAB::NT * C + k;
    static_range<0, NH>([&](auto LMc) {
        constexpr int LM = LMc;
        float adj = M0_adj[(static_cast<std::size_t>(li) * NH + LM) * C + k];
        if constexpr (LM == 0) {
            if (direct) adj += direct[static_cast<std::size_t>(i) * C + k];
        }
        float g[NY];
#pragma unroll
        for (int v = 0; v < NY; ++v) g[v] = 0.0f;
        poly_grad_ct<TAB, TAB::offset[LM], TAB::offset[LM + 1], C>(x, cf, g);
#pragma unroll
        for (int v = 0; v < NY; ++v) acc[v] += g[v] * adj;
    });
#pragma unroll
    for (int v = 0; v < NY; ++v) A0_adj[(static_cast<std::size_t>(li) * NY + v) * C + k] = acc[v];
}

template <int C, int NY, int NH>
__global__ __launch_bounds__(C) void k_m0_forward(int r0, const int* __restrict__ types, const float* __restrict__ A0,
                                                  const std::int32_t* __restrict__ terms, const int* __restrict__ toff,
                                                  int T0, const float* __restrict__ coef, float* __restrict__ M0,
                                                  float* __restrict__ xaff) {
    __shared__ float xs[NY * C];
    const int li = blockIdx.x;
    const int i = r0 + li;
    const int k = threadIdx.x;
#pragma unroll
    for (int v = 0; v < NY; ++v) xs[v * C + k] = A0[(static_cast<std::size_t>(li) * NY + v) * C + k];
    const float* cf = coef + static_cast<std::size_t>(types[i]) * T0 * C + k;
#pragma unroll
    for (int LM = 0; LM < NH; ++LM) {
        const int begin = toff[LM], end = toff[LM + 1];
        float f = 0.0f;
        for (int t = begin; t < end; ++t) f += cf[static_cast<std::size_t>(t) * C] * monomial(xs, C, k, terms[t]);
        M0[(static_cast<std::size_t>(li) * NH + LM) * C + k] = f;
        if (LM == 0) xaff[static_cast<std::size_t>(i) * C + k] = f;
    }
}

template <int C, int NY, int NH>
__global__ __launch_bounds__(C) void k_m0_reverse(int r0, const int* __restrict__ types, const float* __restrict__ A0,
                                                  const float* __restrict__ M0_adj, const float* __restrict__ direct,
                                                  const std::int32_t* __restrict__ terms, const int* __restrict__ toff,
                                                  int T0, const float* __restrict__ coef,
                                                  float* __restrict__ A0_adj) {
    __shared__ float xs[NY * C];
    __shared__ float gs[NY * C];
    const int li = blockIdx.x;
    const int i = r0 + li;
    const int k = threadIdx.x;
#pragma unroll
    for (int v = 0; v < NY; ++v) xs[v * C + k] = A0[(static_cast<std::size_t>(li) * NY + v) * C + k];
    float acc[NY];
#pragma unroll
    for (int v = 0; v < NY; ++v) acc[v] = 0.0f;
    const float* cf = coef + static_cast<std::size_t>(types[i]) * T0 * C + k;
#pragma unroll
    for (int LM = 0; LM < NH; ++LM) {
        const int begin = toff[LM], end = toff[LM + 1];
        float adj = M0_adj[(static_cast<std::size_t>(li) * NH + LM) * C + k];
        if (LM == 0 && direct) adj += direct[static_cast<std::size_t>(i) * C + k];
#pragma unroll
        for (int v = 0; v < NY; ++v) gs[v * C + k] = 0.0f;
        for (int t = begin; t < end; ++t) monomial_grad(xs, gs, C, k, terms[t], cf[static_cast<std::size_t>(t) * C]);
#pragma unroll
        for (int v = 0; v < NY; ++v) acc[v] += gs[v * C + k] * adj;
    }
#pragma unroll
    for (int v = 0; v < NY; ++v) A0_adj[(static_cast<std::size_t>(li) * NY + v) * C + k] = acc[v];
}

// M1 of one node and channel, and (with G) its gradient dM1/dA1 (unscaled).
// TAB is a compiled ProductTable or void for the table-driven form (then
// xs/gs are the node's variables and gradient in LDS, column k).
template <class TAB, int C, int NY>
struct M1Poly {
    __device__ __forceinline__ static float value(const float* __restrict__ A1row, const float* __restrict__ cf,
                                                  const std::int32_t* __restrict__, int, float*, int k) {
        float x[NY];
#pragma unroll
        for (int v = 0; v < NY; ++v) x[v] = A1row[v * C + k];
        return poly_ct<TAB, 0, TAB::NT, C>(x, cf);
    }
    __device__ __forceinline__ static void grad(const float* __restrict__ A1row, const float* __restrict__ cf,
                                                const std::int32_t* __restrict__, int, float*, float*, int k,
                                                float* g) {
        float x[NY];
#pragma unroll
        for (int v = 0; v < NY; ++v) {
            x[v] = A1row[v * C + k];
            g[v] = 0.0f;
        }
        poly_grad_ct<TAB, 0, TAB::NT, C>(x, cf, g);
    }
};

template <int C, int NY>
struct M1Poly<void, C, NY> {
    __device__ __forceinline__ static float value(const float* __restrict__ A1row, const float* __restrict__ cf,
                                                  const std::int32_t* __restrict__ terms, int T1, float* xs, int k) {
#pragma unroll
        for (int v = 0; v < NY; ++v) xs[v * C + k] = A1row[v * C + k];
        float m = 0.0f;
        for (int s = 0; s < T1; ++s) m += cf[static_cast<std::size_t>(s) * C] * monomial(xs, C, k, terms[s]);
        return m;
    }
    __device__ __forceinline__ static void grad(const float* __restrict__ A1row, const float* __restrict__ cf,
                                                const std::int32_t* __restrict__ terms, int T1, float* xs, float* gs,
                                                int k, float* g) {
#pragma unroll
        for (int v = 0; v < NY; ++v) {
            xs[v * C + k] = A1row[v * C + k];
            gs[v * C + k] = 0.0f;
        }
        for (int s = 0; s < T1; ++s) monomial_grad(xs, gs, C, k, terms[s], cf[static_cast<std::size_t>(s) * C]);
#pragma unroll
        for (int v = 0; v < NY; ++v) g[v] = gs[v * C + k];
    }
};

// M1 of every receiver and its gradient dM1/dA1 (unscaled), one receiver
// per workgroup: M1[li,k] and grad[li,v,k] (the gradient is scaled by the M1
// adjoint in k_readout once the readout reverse has produced it).
template <int C, int NY, class M1TAB>
__global__ __launch_bounds__(C) void k_m1(int r0, const int* __restrict__ types, const float* __restrict__ A1,
                                          const std::int32_t* __restrict__ m1_terms, int T1,
                                          const float* __restrict__ m1_coef, float* __restrict__ M1,
                                          float* __restrict__ grad) {
    using Poly = M1Poly<M1TAB, C, NY>;
    constexpr bool kLds = std::is_same_v<M1TAB, void>;
    __shared__ float xs[kLds ? NY * C : 1], gs[kLds ? NY * C : 1];
    const int li = blockIdx.x;
    const int k = threadIdx.x;
    const float* cf = m1_coef + static_cast<std::size_t>(types[r0 + li]) * T1 * C + k;
    const float* row = A1 + static_cast<std::size_t>(li) * NY * C;
    M1[static_cast<std::size_t>(li) * C + k] = Poly::value(row, cf, m1_terms, T1, xs, k);
    float g[NY];
    Poly::grad(row, cf, m1_terms, T1, xs, gs, k, g);
#pragma unroll
    for (int v = 0; v < NY; ++v) grad[(static_cast<std::size_t>(li) * NY + v) * C + k] = g[v];
}

// H2 (FP64), readouts (FP64) and their adjoints for a tile of up to 16
// receivers of one type:
//   E_i = E0[z] + q.x + MLP(H2), H2 = T_z^T x + W^T M1 (x = M0[i,0,:])
//   direct = q + T_z H2_adj, A1_adj[v] = dM1/dA1_v * (W H2_adj)
// Readout MLP: hidden = SiLU*scale(W1 H2), E += W2 . hidden (mace.cpp:2600-2657).
// On entry A1_adj holds the unscaled M1 gradient from k_m1.
//
// The four products (H2; the MLP pre-activations W1 H2; the hidden adjoint
// times W1; T and W times H2_adj) run as FP64 MFMA tiles
// (v_mfma_f64_16x16x4_f64, exact FP64 products and sums): the tile's 16
// receivers are the 16 rows, each of the workgroup's kReadoutWaves waves
// takes every kReadoutWaves-th 16-column block, the row operands come from LDS and the weights (FP32
// values, widened) straight from L2.  Lane l supplies A[l%16][l/16] and
// B[l/16][l%16] and holds D[l/16 + 4v][l%16], v = 0..3.
// ---------------------------------------------------------------------------
typedef double v4d __attribute__((ext_vector_type(4)));
static_assert(kReadoutBatch == 16, "readout tiles are the 16 rows of an FP64 MFMA tile");

__device__ __forceinline__ v4d mfma_f64(double a, double b, v4d c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}

constexpr int kReadoutWaves = 8;

template <int C, int NY>
__global__ __launch_bounds__(64 * kReadoutWaves) void k_readout(
    int r0, const NodeBatch* __restrict__ batches, const int* __restrict__ node_list, const int* __restrict__ types,
    const float* __restrict__ M1, const float* __restrict__ xaff, const float* __restrict__ H2_T,
    const float* __restrict__ H2_Tt, const float* __restrict__ H2_M1, const float* __restrict__ H2_M1t,
    const double* __restrict__ q, const double* __restrict__ W1r, const double* __restrict__ W2r, int hidden,
    double scale, const double* __restrict__ E0, double* __restrict__ node_energies, float* __restrict__ direct,
    float* __restrict__ A1_adj) {
    static_assert(C % 16 == 0, "16-column MFMA blocks");
    constexpr int R = kReadoutBatch, NT = C / 16, WAVES = kReadoutWaves, THREADS = 64 * WAVES;
    constexpr int HMAX = kMaxReadoutHidden;
    // The energy terms sP are written after the last read of sA, so they
    // share its storage where it is large enough (C >= 64): at 256 channels
    // the workgroup then needs 74 KB of LDS and two fit a CU.
    constexpr bool kShareA = sizeof(float) * (2 * C + 1) >= sizeof(double) * (HMAX + 1);
    __shared__ __align__(16) float sA[R][2 * C + 1];  // [x | M1] rows (FP32 values)
    __shared__ double sH[R][C + 1];                   // H2, then its adjoint
    __shared__ double sZ[R][HMAX + 1];                // pre-activations, then W2 act'(z)
    __shared__ double sPown[kShareA ? 1 : R][HMAX + 1];
    // W2 act(z) terms of the energy
    double (*sP)[HMAX + 1] = kShareA ? reinterpret_cast<double (*)[HMAX + 1]>(&sA[0][0]) : sPown;
    const NodeBatch b = batches[blockIdx.x];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r = lane & 15, kk = lane >> 4;
    const int t = types[r0 + node_list[b.start]];
    for (int p = tid; p < R * C; p += THREADS) {
        const int n = p / C, k = p % C;
        const bool ok = n < b.count;
        const int li = ok ? node_list[b.start + n] : 0;
        sA[n][k] = ok ? xaff[static_cast<std::size_t>(r0 + li) * C + k] : 0.0f;
        sA[n][C + k] = ok ? M1[static_cast<std::size_t>(li) * C + k] : 0.0f;
    }
    for (int p = tid; p < R * (HMAX + 1); p += THREADS) sZ[p / (HMAX + 1)][p % (HMAX + 1)] = 0.0;
    __syncthreads();
    // q . x of each receiver, read now (sA is overwritten below)
    double qx = 0.0;
    if (tid < b.count)
        for (int k = 0; k < C; ++k) qx += q[k] * static_cast<double>(sA[tid][k]);
    // H2[n][c] = sum_in T[in][c] x[n][in] + sum_in W[in][c] M1[n][in]
    {
        const float* T = H2_T + static_cast<std::size_t>(t) * C * C;
        for (int j = w; j < NT; j += WAVES) {
            const int col = 16 * j + r;
            // the two products accumulate separately (independent MFMA chains)
            v4d ax = {0.0, 0.0, 0.0, 0.0}, am = {0.0, 0.0, 0.0, 0.0};
#pragma unroll 8
            for (int k0 = 0; k0 < C; k0 += 4) {
                ax = mfma_f64(sA[r][k0 + kk], T[(k0 + kk) * C + col], ax);
                am = mfma_f64(sA[r][C + k0 + kk], H2_M1[(k0 + kk) * C + col], am);
            }
#pragma unroll
            for (int v = 0; v < 4; ++v) sH[kk + 4 * v][col] = ax[v] + am[v];
        }
    }
    __syncthreads();
    // z[n][hd] = W1[hd] . H2[n]; columns past hidden stay zero
    const int HT = (hidden + 15) / 16;
    for (int j = w; j < HT; j += WAVES) {
        const int hd = 16 * j + r;
        const double* w1 = W1r + static_cast<std::size_t>(min(hd, hidden - 1)) * C;
        const bool ok = hd < hidden;
        v4d acc = {0.0, 0.0, 0.0, 0.0};
#pragma unroll 8
        for (int k0 = 0; k0 < C; k0 += 4) acc = mfma_f64(sH[r][k0 + kk], ok ? w1[k0 + kk] : 0.0, acc);
#pragma unroll
        for (int v = 0; v < 4; ++v) sZ[kk + 4 * v][hd] = acc[v];
    }
    __syncthreads();
    // activation: energy terms and g = W2 act'(z) (sA is no longer read:
    // the z phase's barrier follows the H2 phase's last read of it)
    for (int p = tid; p < R * hidden; p += THREADS) {
        const int n = p / hidden, hd = p % hidden;
        const double z = sZ[n][hd];
        const double sg = 1.0 / (1.0 + exp(-z));
        sP[n][hd] = W2r[hd] * (scale * z * sg);
        sZ[n][hd] = W2r[hd] * (scale * sg + scale * z * sg * (1.0 - sg));
    }
    __syncthreads();
    if (tid < b.count) {
        const int n = tid;
        double out = 0.0;
        for (int hd = 0; hd < hidden; ++hd) out += sP[n][hd];
        node_energies[r0 + node_list[b.start + n]] = E0[t] + qx + out;
    }
    // H2 adjoint h2a[n][c] = sum_hd g[n][hd] W1[hd][c] (over sH: H2 is no
    // longer read)
    for (int j = w; j < NT; j += WAVES) {
        const int col = 16 * j + r;
        v4d acc = {0.0, 0.0, 0.0, 0.0};
        for (int k0 = 0; k0 < 16 * HT; k0 += 4) {
            const int hd = k0 + kk;
            acc = mfma_f64(sZ[r][hd], hd < hidden ? W1r[static_cast<std::size_t>(hd) * C + col] : 0.0, acc);
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) sH[kk + 4 * v][col] = acc[v];
    }
    __syncthreads();
    // direct = q + T H2_adj; M1 adjoint = W H2_adj
    {
        const float* Tt = H2_Tt + static_cast<std::size_t>(t) * C * C;
        for (int j = w; j < NT; j += WAVES) {
            const int col = 16 * j + r;
            v4d ad = {0.0, 0.0, 0.0, 0.0}, as = {0.0, 0.0, 0.0, 0.0};
#pragma unroll 8
            for (int k0 = 0; k0 < C; k0 += 4) {
                const double a = sH[r][k0 + kk];
                ad = mfma_f64(a, Tt[(k0 + kk) * C + col], ad);
                as = mfma_f64(a, H2_M1t[(k0 + kk) * C + col], as);
            }
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int n = kk + 4 * v;
                if (n < b.count) {
                    const int li = node_list[b.start + n];
                    direct[static_cast<std::size_t>(r0 + li) * C + col] = static_cast<float>(q[col] + ad[v]);
                    const float m1adj = static_cast<float>(as[v]);
                    float* g = A1_adj + static_cast<std::size_t>(li) * NY * C + col;
#pragma unroll
                    for (int u = 0; u < NY; ++u) g[u * C] = g[u * C] * m1adj;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Tiled execution: per-tile contributions of edges to their sources.  The
// edges of source s inside the tile's edge range [e0, e1) are a contiguous
// run of s's source-transpose segment (edge ids ascend within a segment and
// edges are receiver-major), found by a binary search.  T is the
// transpose's position and edge-id type: long long for the tiled plan's own
// graphs (beyond 2^31 edges), int for the LAMMPS neighbour transpose.
// ---------------------------------------------------------------------------
template <class T>
__device__ __forceinline__ T lower_edge(const T* __restrict__ sedges, T lo, T hi, long long key) {
    while (lo < hi) {
        // lo + hi can exceed 2^31 when the graph has more than 2^30 edges
        const T mid = lo + ((hi - lo) >> 1);
        if (sedges[mid] < key)
            lo = mid + 1;
        else
            hi = mid;
    }
    return lo;
}

// H1_adj[s] += sum over the tile's edges leaving s of W_e (FP64 sum, one
// read-modify-write per source and tile; tiles run in order).
template <int C, int NH, class T>
__global__ __launch_bounds__(C) void k_tile_source_adjoint(const int* __restrict__ touched, long long e0, long long e1,
                                                           const T* __restrict__ soff, const T* __restrict__ sedges,
                                                           const float* __restrict__ Wsrc,
                                                           const double* __restrict__ r, double r_cut,
                                                           float* __restrict__ H1_adj) {
    const int s = touched[blockIdx.x];
    const int k = threadIdx.x;
    double acc[NH];
#pragma unroll
    for (int q = 0; q < NH; ++q) acc[q] = 0.0;
    const T hi = soff[s + 1];
    const T lo = lower_edge(sedges, soff[s], hi, e0);
    const T end = lower_edge(sedges, lo, hi, e1);
    gather_source_rows<C, NH>(sedges, lo, end, e0, Wsrc, r, r_cut, k, acc);
    float* dst = H1_adj + static_cast<std::size_t>(s) * NH * C + k;
#pragma unroll
    for (int q = 0; q < NH; ++q) dst[q * C] = dst[q * C] + static_cast<float>(acc[q]);
}

// F[s] += sum of the tile's directed forces on edges leaving s (one wave per source)
template <class T>
__global__ __launch_bounds__(256) void k_tile_forces_sources(const int* __restrict__ touched, int count, long long e0,
                                                             long long e1, const T* __restrict__ soff,
                                                             const T* __restrict__ sedges,
                                                             const double* __restrict__ nf, double* __restrict__ F) {
    const int b = blockIdx.x * (256 / kWave) + threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    if (b >= count) return;
    const int s = touched[b];
    const T hi = soff[s + 1];
    const T lo = lower_edge(sedges, soff[s], hi, e0);
    double f0 = 0.0, f1 = 0.0, f2 = 0.0;
    for (T t = lo + lane; t < hi; t += kWave) {
        const long long e = sedges[t];
        if (e >= e1) break;
        const std::size_t le = static_cast<std::size_t>(e - e0);
        f0 += nf[3 * le];
        f1 += nf[3 * le + 1];
        f2 += nf[3 * le + 2];
    }
    f0 = wave_sum<kWave>(f0);
    f1 = wave_sum<kWave>(f1);
    f2 = wave_sum<kWave>(f2);
    if (lane == 0) {
        F[3 * static_cast<std::size_t>(s)] += f0;
        F[3 * static_cast<std::size_t>(s) + 1] += f1;
        F[3 * static_cast<std::size_t>(s) + 2] += f2;
    }
}

// F[i] -= sum of the directed forces on the edges arriving at receiver i of the tile
__global__ __launch_bounds__(256) void k_tile_forces_receivers(int r0, int nr, long long e0,
                                                               const int* __restrict__ offsets,
                                                               const int* __restrict__ receiver_row,
                                                               const double* __restrict__ nf, double* __restrict__ F) {
    const int li = blockIdx.x * (256 / kWave) + threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    if (li >= nr) return;
    const int i = r0 + li;
    double f0 = 0.0, f1 = 0.0, f2 = 0.0;
    for (int e = offsets[i] + lane; e < offsets[i + 1]; e += kWave) {
        const std::size_t le = static_cast<std::size_t>(e - e0);
        f0 += nf[3 * le];
        f1 += nf[3 * le + 1];
        f2 += nf[3 * le + 2];
    }
    f0 = wave_sum<kWave>(f0);
    f1 = wave_sum<kWave>(f1);
    f2 = wave_sum<kWave>(f2);
    if (lane == 0) {
        const std::size_t row = receiver_row ? static_cast<std::size_t>(receiver_row[i]) : static_cast<std::size_t>(i);
        F[3 * row] -= f0;
        F[3 * row + 1] -= f1;
        F[3 * row + 2] -= f2;
    }
}

// rows[li][c] += bias[types[r0 + li]][c]
__global__ __launch_bounds__(256) void k_type_bias(int r0, int nr, const int* __restrict__ types, int row_len,
                                                   const float* __restrict__ bias, float* __restrict__ rows) {
    const long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= static_cast<long long>(nr) * row_len) return;
    const int li = static_cast<int>(idx / row_len), c = static_cast<int>(idx % row_len);
    rows[idx] += bias[static_cast<std::size_t>(types[r0 + li]) * row_len + c];
}

// ---------------------------------------------------------------------------
// MACEField field terms (mace_kokkos_h1_phi1.cpp:846-1150).  One workgroup per
// node, lanes over channels; the path products Z = H1p[l_in rows] W and
// Y = H1p_adj[l_out rows] W^T come from the node GEMM, so these kernels only
// mix the m components with the entries' coef E_comp.
// ---------------------------------------------------------------------------
// H1f[i,lm] = H1p[i,lm] + sum over the entries into lm of coef E_comp Z[i,zrow];
// x = H1f[i,0,:] (the scalar input of readout_1 and the skip).  One pass
// over the entries with the NH rows of the lane's channel in registers (each
// row takes its entries in list order).
template <int C, int NH>
__global__ __launch_bounds__(C) void k_field_combine(int r0, int zr, const FieldEntryDev* __restrict__ entries,
                                                     int ne, const double* __restrict__ field, int per_node,
                                                     const float* __restrict__ H1p, const float* __restrict__ Z,
                                                     float* __restrict__ H1f, float* __restrict__ xaff) {
    const int i = r0 + static_cast<int>(blockIdx.x);
    const int k = threadIdx.x;
    const double* E = field + (per_node ? 3 * static_cast<std::size_t>(i) : 0);
    const std::size_t base = static_cast<std::size_t>(i) * NH * C;
    const float* z = Z + static_cast<std::size_t>(i) * zr * C;
    float v[NH];
#pragma unroll
    for (int q = 0; q < NH; ++q) v[q] = H1p[base + static_cast<std::size_t>(q) * C + k];
    for (int e = 0; e < ne; ++e) {
        const FieldEntryDev en = entries[e];
        const float add = (en.coef * static_cast<float>(E[en.comp])) * z[static_cast<std::size_t>(en.zrow) * C + k];
        static_for<0, NH>([&](auto qc) {
            if (en.lm_out == qc) v[qc] += add;
        });
    }
#pragma unroll
    for (int q = 0; q < NH; ++q) H1f[base + static_cast<std::size_t>(q) * C + k] = v[q];
    xaff[static_cast<std::size_t>(i) * C + k] = v[0];
}

// H1p_adj[i,0,:] += direct[i,:] (x = H1f[:,0,:], mace.cpp:1798-1804)
__global__ void k_field_direct_add(int r0, int NH, int C, const float* __restrict__ direct,
                                   float* __restrict__ H1p_adj) {
    const int i = r0 + static_cast<int>(blockIdx.x);
    const int k = threadIdx.x;
    H1p_adj[static_cast<std::size_t>(i) * NH * C + k] += direct[static_cast<std::size_t>(i) * C + k];
}

// H1p_adj[i,lm] += sum over the entries from lm of E_comp (coef Y[i,yrow]) and
// the node's dE/dE_c = sum of H1p[i,lm_in,k] coef Y[i,yrow,k] (FP32 products,
// FP64 sums) into part[i][c].  One pass over the entries in list order, the
// NH rows of the lane's channel in registers.
template <int C, int NH>
__global__ __launch_bounds__(C) void k_field_reverse_combine(int r0, int yr,
                                                            const FieldEntryDev* __restrict__ entries, int ne,
                                                            const double* __restrict__ field, int per_node,
                                                            const float* __restrict__ H1p, const float* __restrict__ Y,
                                                            float* __restrict__ H1p_adj, double* __restrict__ part) {
    __shared__ double sbuf[Lanes<C>::NW];
    const int i = r0 + static_cast<int>(blockIdx.x);
    const int k = threadIdx.x;
    const double* E = field + (per_node ? 3 * static_cast<std::size_t>(i) : 0);
    const std::size_t base = static_cast<std::size_t>(i) * NH * C;
    const float* y = Y + static_cast<std::size_t>(i) * yr * C;
    float v[NH], hp[NH];
#pragma unroll
    for (int q = 0; q < NH; ++q) {
        v[q] = H1p_adj[base + static_cast<std::size_t>(q) * C + k];
        hp[q] = H1p[base + static_cast<std::size_t>(q) * C + k];
    }
    double acc[3] = {0.0, 0.0, 0.0};
    for (int e = 0; e < ne; ++e) {
        const FieldEntryDev en = entries[e];
        const float contribution = en.coef * y[static_cast<std::size_t>(en.yrow) * C + k];
        const float ec = static_cast<float>(E[en.comp]);
        static_for<0, NH>([&](auto qc) {
            if (en.lm_in == qc) {
                v[qc] += ec * contribution;
                const double d = static_cast<double>(hp[qc] * contribution);
                if (en.comp == 0) acc[0] += d;
                else if (en.comp == 1) acc[1] += d;
                else acc[2] += d;
            }
        });
    }
#pragma unroll
    for (int q = 0; q < NH; ++q) H1p_adj[base + static_cast<std::size_t>(q) * C + k] = v[q];
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        const double t = block_sum<C>(acc[c], sbuf);
        if (k == 0) part[3 * static_cast<std::size_t>(i) + c] = t;
    }
}

// dE/dE of a graph field: out[c] = sum_i part[i][c] in a fixed order
__global__ __launch_bounds__(256) void k_field_adj_sum(int N, const double* __restrict__ part, double* __restrict__ out) {
    __shared__ double sbuf[256];
    for (int c = 0; c < 3; ++c) {
        double t = 0.0;
        for (int i = threadIdx.x; i < N; i += 256) t += part[3 * static_cast<std::size_t>(i) + c];
        sbuf[threadIdx.x] = t;
        __syncthreads();
        for (int w = 128; w > 0; w >>= 1) {
            if (static_cast<int>(threadIdx.x) < w) sbuf[threadIdx.x] += sbuf[threadIdx.x + w];
            __syncthreads();
        }
        if (threadIdx.x == 0) out[c] = sbuf[0];
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// MACEField response (mace_kokkos_response.tpp:136-2343): the tangent d/dE_s
// of a completed evaluation for one field component s.  H1f is linear in the
// field, so its tangent is the entries of component s applied to Z; the
// other tangents run through the evaluation's own kernels (R1 forward and
// reverse, node GEMMs, M0 reverse, R0 reverse) on tangent buffers, plus the
// kernels below for the two nonlinear stages the reverse differentiates
// again: the M1 polynomial and the readout MLP.
// ---------------------------------------------------------------------------
// H1f_dot[i,lm] = sum over the entries of component seed into lm of coef Z[i,zrow];
// x_dot = H1f_dot[i,0,:]
template <int C, int NH>
__global__ __launch_bounds__(C) void k_field_tangent(int zr, const FieldEntryDev* __restrict__ entries, int ne,
                                                     int seed, const float* __restrict__ Z,
                                                     float* __restrict__ H1f_dot, float* __restrict__ x_dot) {
    const int i = static_cast<int>(blockIdx.x);
    const int k = threadIdx.x;
    const float* z = Z + static_cast<std::size_t>(i) * zr * C;
    float v[NH];
#pragma unroll
    for (int q = 0; q < NH; ++q) v[q] = 0.0f;
    for (int e = 0; e < ne; ++e) {
        const FieldEntryDev en = entries[e];
        if (en.comp != seed) continue;
        const float add = en.coef * z[static_cast<std::size_t>(en.zrow) * C + k];
        static_for<0, NH>([&](auto qc) {
            if (en.lm_out == qc) v[qc] += add;
        });
    }
#pragma unroll
    for (int q = 0; q < NH; ++q) H1f_dot[(static_cast<std::size_t>(i) * NH + q) * C + k] = v[q];
    x_dot[static_cast<std::size_t>(i) * C + k] = v[0];
}

// M1's tangent along A1_dot: M1_dot = sum_v g_v A1_dot_v, the gradient g and
// its derivative gd along A1_dot (each factor of a term differentiated in
// turn).  Lanes are channels.  With a compiled term table (M1TAB) the terms
// are straight-line code on register-resident variables, one workgroup of C
// lanes per node; else the monomial list is read from HBM with the
// variables in LDS, kTangentLanes channels per workgroup (blockIdx.y picks
// the channel block).
constexpr int kTangentLanes = 128;
template <int C, class M1TAB>
constexpr int m1_tangent_lanes() {
    return std::is_same_v<M1TAB, void> ? (C < kTangentLanes ? C : kTangentLanes) : C;
}

template <int C, int NY, class M1TAB>
__global__ __launch_bounds__((m1_tangent_lanes<C, M1TAB>())) void k_m1_tangent(
    const int* __restrict__ types, const float* __restrict__ A1, const float* __restrict__ A1_dot,
    const std::int32_t* __restrict__ terms, int T1, const float* __restrict__ m1_coef, float* __restrict__ M1_dot,
    float* __restrict__ g, float* __restrict__ gd) {
    constexpr int L = m1_tangent_lanes<C, M1TAB>();
    static_assert(C % L == 0, "whole channel blocks");
    const int i = static_cast<int>(blockIdx.x);
    const int j = threadIdx.x;
    const int k = static_cast<int>(blockIdx.y) * L + j;
    const std::size_t row = static_cast<std::size_t>(i) * NY * C + k;
    const float* cf = m1_coef + static_cast<std::size_t>(types[i]) * T1 * C + k;
    if constexpr (!std::is_same_v<M1TAB, void>) {
        float x[NY], dx[NY], gv[NY], gdv[NY];
#pragma unroll
        for (int v = 0; v < NY; ++v) {
            x[v] = A1[row + v * C];
            dx[v] = A1_dot[row + v * C];
            gv[v] = 0.0f;
            gdv[v] = 0.0f;
        }
        M1_dot[static_cast<std::size_t>(i) * C + k] = poly_tangent_ct<M1TAB, 0, M1TAB::NT, C>(x, dx, cf, gv, gdv);
#pragma unroll
        for (int v = 0; v < NY; ++v) {
            g[row + v * C] = gv[v];
            gd[row + v * C] = gdv[v];
        }
        return;
    } else {
        __shared__ float xs[NY * L], dxs[NY * L], gs[NY * L], gds[NY * L];
#pragma unroll
        for (int v = 0; v < NY; ++v) {
            xs[v * L + j] = A1[row + v * C];
            dxs[v * L + j] = A1_dot[row + v * C];
            gs[v * L + j] = 0.0f;
            gds[v * L + j] = 0.0f;
        }
        float fd = 0.0f;
        for (int t = 0; t < T1; ++t) {
            const int pk = terms[t];
            const float c = cf[static_cast<std::size_t>(t) * C];
            const int deg = pk >> 24;
            const int v0 = pk & 0xff, v1 = (pk >> 8) & 0xff, v2 = (pk >> 16) & 0xff;
            const float x0 = xs[v0 * L + j], d0 = dxs[v0 * L + j];
            if (deg == 1) {
                gs[v0 * L + j] += c;
                fd += c * d0;
            } else if (deg == 2) {
                const float x1 = xs[v1 * L + j], d1 = dxs[v1 * L + j];
                gs[v0 * L + j] += c * x1;
                gs[v1 * L + j] += c * x0;
                gds[v0 * L + j] += c * d1;
                gds[v1 * L + j] += c * d0;
                fd += c * (x1 * d0 + x0 * d1);
            } else {
                const float x1 = xs[v1 * L + j], d1 = dxs[v1 * L + j];
                const float x2 = xs[v2 * L + j], d2 = dxs[v2 * L + j];
                gs[v0 * L + j] += c * x1 * x2;
                gs[v1 * L + j] += c * x0 * x2;
                gs[v2 * L + j] += c * x0 * x1;
                gds[v0 * L + j] += c * (d1 * x2 + x1 * d2);
                gds[v1 * L + j] += c * (d0 * x2 + x0 * d2);
                gds[v2 * L + j] += c * (d0 * x1 + x0 * d1);
                fd += c * (x1 * x2 * d0 + x0 * x2 * d1 + x0 * x1 * d2);
            }
        }
        M1_dot[static_cast<std::size_t>(i) * C + k] = fd;
#pragma unroll
        for (int v = 0; v < NY; ++v) {
            g[row + v * C] = gs[v * L + j];
            gd[row + v * C] = gds[v * L + j];
        }
    }
}

// The readout's tangent for one node (FP64, one workgroup of C lanes): H2 and
// H2_dot = T^T x_dot + W^T M1_dot, the MLP's pre-activations and their
// tangents, H2_adj = sum_h W2 act'(z) W1 and H2_adj_dot = sum_h W2 act''(z)
// z_dot W1, then direct_dot = T H2_adj_dot and the M1 adjoint and its tangent
// W H2_adj(_dot), which scale the M1 gradient and its tangent into
//   A1_adj_dot = g float(M1_adj_dot) + gd float(M1_adj)
// and (a1s_adj non-null) the A1 adjoint itself, g float(M1_adj).
template <int C>
__global__ __launch_bounds__(C) void k_readout_tangent(
    const int* __restrict__ types, int NY, const float* __restrict__ M1, const float* __restrict__ M1_dot,
    const float* __restrict__ xaff, const float* __restrict__ x_dot, const float* __restrict__ H2_T,
    const float* __restrict__ H2_Tt, const float* __restrict__ H2_M1, const float* __restrict__ H2_M1t,
    const double* __restrict__ W1r, const double* __restrict__ W2r, int hidden, double scale,
    const float* __restrict__ g, const float* __restrict__ gd, float* __restrict__ direct_dot,
    float* __restrict__ A1_adj_dot, float* __restrict__ a1s_adj) {
    __shared__ double sx[C], sxd[C], sm[C], smd[C], sh[C], shd[C];
    __shared__ double sa[kMaxReadoutHidden], sad[kMaxReadoutHidden];
    const int i = static_cast<int>(blockIdx.x);
    const int k = threadIdx.x;
    const int t = types[i];
    sx[k] = xaff[static_cast<std::size_t>(i) * C + k];
    sxd[k] = x_dot[static_cast<std::size_t>(i) * C + k];
    sm[k] = M1[static_cast<std::size_t>(i) * C + k];
    smd[k] = M1_dot[static_cast<std::size_t>(i) * C + k];
    __syncthreads();
    {
        const float* T = H2_T + static_cast<std::size_t>(t) * C * C;
        double h = 0.0, hd = 0.0;
        for (int in = 0; in < C; ++in) {
            const double a = T[in * C + k], b = H2_M1[in * C + k];
            h += a * sx[in] + b * sm[in];
            hd += a * sxd[in] + b * smd[in];
        }
        sh[k] = h;
        shd[k] = hd;
    }
    __syncthreads();
    for (int hdn = k; hdn < hidden; hdn += C) {
        const double* w1 = W1r + static_cast<std::size_t>(hdn) * C;
        double z = 0.0, zd = 0.0;
        for (int c = 0; c < C; ++c) {
            z += w1[c] * sh[c];
            zd += w1[c] * shd[c];
        }
        const double sg = 1.0 / (1.0 + exp(-z));
        // act(z) = scale z sigmoid(z): act' and act''
        const double act1 = scale * sg + scale * z * sg * (1.0 - sg);
        const double act2 = scale * sg * (1.0 - sg) * (2.0 + z * (1.0 - 2.0 * sg));
        sa[hdn] = W2r[hdn] * act1;
        sad[hdn] = W2r[hdn] * act2 * zd;
    }
    __syncthreads();
    double ha = 0.0, had = 0.0;
    for (int hdn = 0; hdn < hidden; ++hdn) {
        const double w = W1r[static_cast<std::size_t>(hdn) * C + k];
        ha += sa[hdn] * w;
        had += sad[hdn] * w;
    }
    __syncthreads();
    sh[k] = ha;
    shd[k] = had;
    __syncthreads();
    const float* Tt = H2_Tt + static_cast<std::size_t>(t) * C * C;
    double dd = 0.0, m1a = 0.0, m1ad = 0.0;
    for (int o = 0; o < C; ++o) {
        const double wt = H2_M1t[o * C + k];
        dd += static_cast<double>(Tt[o * C + k]) * shd[o];
        m1a += wt * sh[o];
        m1ad += wt * shd[o];
    }
    direct_dot[static_cast<std::size_t>(i) * C + k] = static_cast<float>(dd);
    const float fa = static_cast<float>(m1a), fad = static_cast<float>(m1ad);
    for (int v = 0; v < NY; ++v) {
        const std::size_t q = (static_cast<std::size_t>(i) * NY + v) * C + k;
        A1_adj_dot[q] = g[q] * fad + gd[q] * fa;
        if (a1s_adj) a1s_adj[q] = g[q] * fa;
    }
}

__global__ void k_fill_f32(std::size_t n, float* __restrict__ p) {
    for (std::size_t j = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x; j < n;
         j += static_cast<std::size_t>(gridDim.x) * blockDim.x)
        p[j] = 0.0f;
}

__global__ void k_fill_f64(std::size_t n, double* __restrict__ p) {
    for (std::size_t j = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x; j < n;
         j += static_cast<std::size_t>(gridDim.x) * blockDim.x)
        p[j] = 0.0;
}

// ---------------------------------------------------------------------------
// Node linears on MFMA (v_mfma_f32_16x16x4_f32, FP32 in and out).  One wave
// computes a kGemmRows x 16*NSUB-column block as (kGemmRows/16) x NSUB tiles
// of 16x16.  In a tile, lane l supplies A[l%16][kk] and B[kk][l%16] with
// kk = l/16 and holds D[4*(l/16)+v][l%16].  The K order inside one 16-wide
// chunk is permuted so that step s uses k = k0 + 4*(l/16) + s: each lane then
// reads four consecutive inputs of its row with one 16-byte load, and the
// weights are pre-swizzled (swizzle_gemm_weights) so that the B operands of
// one chunk and 16-column block are one contiguous 1 KB float4 load per wave.
// Per chunk a wave issues RI + NSUB loads and 4*RI*NSUB MFMAs.  Two operand
// sets alternate: the loads of chunk kc+1 are in flight while chunk kc runs on
// the MFMA unit (a three-set ring measured the same at the medium shape: it
// costs two waves per SIMD of occupancy).  NSUB is a template constant so that the chunk body is
// straight-line code (no per-tile branches) and the only waits are for the
// operands of the chunk about to run.
// ---------------------------------------------------------------------------
template <int RI, int NSUB>
struct GemmOperands {
    float4 a[RI], b[NSUB];
};

template <int RI, int NSUB>
__device__ __forceinline__ void gemm_load(GemmOperands<RI, NSUB>& o, const float* const (&arow)[RI],
                                          const float4* __restrict__ B, int kc, int nblk) {
#pragma unroll
    for (int i = 0; i < RI; ++i) o.a[i] = *reinterpret_cast<const float4*>(arow[i] + 16 * kc);
#pragma unroll
    for (int j = 0; j < NSUB; ++j) o.b[j] = B[(static_cast<std::size_t>(kc) * nblk + j) * 64];
}

template <int RI, int NSUB>
__device__ __forceinline__ void gemm_chunk(v4f (&acc)[RI][NSUB], const GemmOperands<RI, NSUB>& o) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
        for (int i = 0; i < RI; ++i) {
            const float av = s == 0 ? o.a[i].x : s == 1 ? o.a[i].y : s == 2 ? o.a[i].z : o.a[i].w;
#pragma unroll
            for (int j = 0; j < NSUB; ++j) {
                const float bv = s == 0 ? o.b[j].x : s == 1 ? o.b[j].y : s == 2 ? o.b[j].z : o.b[j].w;
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[i][j], 0, 0, 0);
            }
        }
    }
}

template <int NSUB>
__global__ __launch_bounds__(64) void k_node_gemm(const GemmTile* __restrict__ tiles,
                                                  const GemmGroup* __restrict__ groups, const int* __restrict__ rows,
                                                  const float* __restrict__ W, const float* __restrict__ in,
                                                  float* __restrict__ out) {
    constexpr int RI = kGemmRows / 16;  // 16-row MFMA tiles per wave
    // blockIdx.x: row tile; blockIdx.y: 16*NSUB-column block.  (Dispatch
    // order x-fastest: concurrent waves share one column block's weights.
    // Grouping a tile's column blocks on one XCD measured slower.)
    const GemmTile tile = tiles[blockIdx.x];
    const GemmGroup g = groups[tile.group];
    const int n0 = blockIdx.y * 16 * NSUB;
    if (n0 >= g.N) return;
    const int lane = threadIdx.x;
    const int r = lane & 15, kg = lane >> 4;
    const float* arow[RI];
#pragma unroll
    for (int i = 0; i < RI; ++i) {
        // rows past the tile's count repeat its last row (their results are not stored)
        const int q = min(16 * i + r, tile.count - 1);
        const int pk = rows[tile.row_start + q];
        arow[i] = in + static_cast<std::size_t>(pk >> 4) * g.in_stride + g.in_base + (pk & 15) * g.in_mstride + 4 * kg;
    }
    const int nblk = g.N / 16;
    const float4* B = reinterpret_cast<const float4*>(W + g.w_off) + (n0 / 16) * 64 + lane;
    v4f acc[RI][NSUB];
#pragma unroll
    for (int i = 0; i < RI; ++i)
#pragma unroll
        for (int j = 0; j < NSUB; ++j) acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    const int chunks = g.K / 16;
    GemmOperands<RI, NSUB> o0, o1;
    gemm_load(o0, arow, B, 0, nblk);
    int kc = 0;
    for (; kc + 2 <= chunks; kc += 2) {
        gemm_load(o1, arow, B, kc + 1, nblk);
        gemm_chunk(acc, o0);
        gemm_load(o0, arow, B, min(kc + 2, chunks - 1), nblk);
        gemm_chunk(acc, o1);
        // issue order: each load set, then the chunk that does not need it,
        // so every load is one full chunk of MFMAs ahead of its use (left
        // alone, the scheduler sinks the loads towards their use)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            __builtin_amdgcn_sched_group_barrier(0x020, RI + NSUB, 0);     // VMEM reads
            __builtin_amdgcn_sched_group_barrier(0x008, 4 * RI * NSUB, 0);  // MFMA
        }
    }
    if (kc < chunks) gemm_chunk(acc, o0);
#pragma unroll
    for (int i = 0; i < RI; ++i) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int q = 16 * i + 4 * kg + v;
            if (q >= tile.count) continue;
            const int pk = rows[tile.row_start + q];
            float* orow = out + static_cast<std::size_t>(pk >> 4) * g.out_stride + g.out_base + (pk & 15) * g.out_mstride +
                          n0 + r;
#pragma unroll
            for (int j = 0; j < NSUB; ++j) orow[16 * j] = acc[i][j][v];
        }
    }
}

// Shared-operand form for large linears: a workgroup of kGemmShareWaves waves
// takes consecutive 16-row tiles of one group (a GemmTileSet) and one
// 128-column block.  The B operands of each 16-wide K chunk (8 KB) are loaded
// once per workgroup into LDS (double-buffered, one float4 per thread) and
// read by every wave, so the weights cross L2 once per 128 rows instead of
// once per 16.  The A rows, operand values and MFMA order per output tile are
// those of k_node_gemm.  Waves past the set's tile count load and wait with
// the others but store nothing.
__global__ __launch_bounds__(64 * kGemmShareWaves) void k_node_gemm_shared(
    const GemmTileSet* __restrict__ sets, const GemmTile* __restrict__ tiles, const GemmGroup* __restrict__ groups,
    const int* __restrict__ rows, const float* __restrict__ W, const float* __restrict__ in, float* __restrict__ out) {
    constexpr int NSUB = 8;
    const GemmTileSet set = sets[blockIdx.x];
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const GemmTile tile = tiles[set.first + min(wave, set.count - 1)];
    const GemmGroup g = groups[tile.group];
    const int n0 = blockIdx.y * 16 * NSUB;
    if (n0 >= g.N) return;  // uniform: the set's tiles share the group
    const int r = lane & 15, kg = lane >> 4;
    const float* arow;
    {
        const int q = min(r, tile.count - 1);
        const int pk = rows[tile.row_start + q];
        arow = in + static_cast<std::size_t>(pk >> 4) * g.in_stride + g.in_base + (pk & 15) * g.in_mstride + 4 * kg;
    }
    const int nblk = g.N / 16;
    // chunk kc's operands of this column block: NSUB*64 float4, contiguous
    const float4* B = reinterpret_cast<const float4*>(W + g.w_off) + (n0 / 16) * 64 + threadIdx.x;
    __shared__ float4 sb[2][NSUB * 64];
    static_assert(NSUB * 64 == 64 * kGemmShareWaves, "one B float4 per thread");
    v4f acc[NSUB];
#pragma unroll
    for (int j = 0; j < NSUB; ++j) acc[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    const int chunks = g.K / 16;
    // operands two chunks ahead: chunk kc runs from a0 and LDS buffer kc&1
    // while the global loads of chunks kc+1 (a1, b1) and kc+2 (a2, b2) are
    // in flight; b1 enters LDS at the end of chunk kc
    const std::size_t bstep = static_cast<std::size_t>(nblk) * 64;
    float4 a0 = *reinterpret_cast<const float4*>(arow);
    float4 a1 = a0, b1 = B[0];
    if (chunks > 1) {
        a1 = *reinterpret_cast<const float4*>(arow + 16);
        b1 = B[bstep];
    }
    sb[0][threadIdx.x] = B[0];
    __syncthreads();
    for (int kc = 0; kc < chunks; ++kc) {
        float4 a2 = a1, b2 = b1;
        if (kc + 2 < chunks) {
            a2 = *reinterpret_cast<const float4*>(arow + 16 * (kc + 2));
            b2 = B[static_cast<std::size_t>(kc + 2) * bstep];
        }
        float4 b[NSUB];
#pragma unroll
        for (int j = 0; j < NSUB; ++j) b[j] = sb[kc & 1][j * 64 + lane];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const float av = s == 0 ? a0.x : s == 1 ? a0.y : s == 2 ? a0.z : a0.w;
#pragma unroll
            for (int j = 0; j < NSUB; ++j) {
                const float bv = s == 0 ? b[j].x : s == 1 ? b[j].y : s == 2 ? b[j].z : b[j].w;
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[j], 0, 0, 0);
            }
        }
        if (kc + 1 < chunks) sb[(kc + 1) & 1][threadIdx.x] = b1;
        __syncthreads();
        a0 = a1;
        a1 = a2;
        b1 = b2;
    }
    if (wave >= set.count) return;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int q = 4 * kg + v;
        if (q >= tile.count) continue;
        const int pk = rows[tile.row_start + q];
        float* orow = out + static_cast<std::size_t>(pk >> 4) * g.out_stride + g.out_base + (pk & 15) * g.out_mstride +
                      n0 + r;
#pragma unroll
        for (int j = 0; j < NSUB; ++j) orow[16 * j] = acc[j][v];
    }
}

// ---------------------------------------------------------------------------
// Reductions
// ---------------------------------------------------------------------------
// One wave per atom: F[a] = sum over edges leaving a of f_e - sum over edges
// arriving at a of f_e (FP64; fixed lane partition, deterministic).
__global__ __launch_bounds__(256) void k_atom_forces(int N, int num_features, const int* __restrict__ offsets,
                                                     const int* __restrict__ soff, const int* __restrict__ sedges,
                                                     const int* __restrict__ feature_of,
                                                     const double* __restrict__ nf, double* __restrict__ F) {
    const int a = blockIdx.x * (256 / kWave) + threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    if (a >= num_features) return;
    double f0 = 0.0, f1 = 0.0, f2 = 0.0;
    for (int t = soff[a] + lane; t < soff[a + 1]; t += kWave) {
        const std::size_t e = static_cast<std::size_t>(sedges[t]);
        f0 += nf[3 * e];
        f1 += nf[3 * e + 1];
        f2 += nf[3 * e + 2];
    }
    if (a < N)
        for (int e = offsets[a] + lane; e < offsets[a + 1]; e += kWave) {
            f0 -= nf[3 * static_cast<std::size_t>(e)];
            f1 -= nf[3 * static_cast<std::size_t>(e) + 1];
            f2 -= nf[3 * static_cast<std::size_t>(e) + 2];
        }
    f0 = wave_sum<kWave>(f0);
    f1 = wave_sum<kWave>(f1);
    f2 = wave_sum<kWave>(f2);
    if (lane == 0) {
        const std::size_t o = 3 * static_cast<std::size_t>(feature_of ? feature_of[a] : a);
        F[o] = f0;
        F[o + 1] = f1;
        F[o + 2] = f2;
    }
}

constexpr int kReduceThreads = 256;

__global__ __launch_bounds__(kReduceThreads) void k_stress_partial(std::int64_t E, const double* __restrict__ nf,
                                                                   const double* __restrict__ xyz,
                                                                   double* __restrict__ partial) {
    double s[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
    const std::int64_t stride = static_cast<std::int64_t>(gridDim.x) * blockDim.x;
    for (std::int64_t e = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < E; e += stride)
        for (int a = 0; a < 3; ++a)
            for (int b = 0; b < 3; ++b) s[3 * a + b] += nf[3 * e + a] * xyz[3 * e + b];
    __shared__ double red[9][kReduceThreads / kWave];
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    for (int c = 0; c < 9; ++c) {
        const double v = wave_sum<kWave>(s[c]);
        if (lane == 0) red[c][wave] = v;
    }
    __syncthreads();
    if (threadIdx.x < 9) {
        double t = 0.0;
        for (int w = 0; w < kReduceThreads / kWave; ++w) t += red[threadIdx.x][w];
        partial[static_cast<std::size_t>(blockIdx.x) * 9 + threadIdx.x] = t;
    }
}

// out[c] = scale * sum of the partials (or out[c] += ... when accumulating)
__global__ __launch_bounds__(kReduceThreads) void k_stress_final(int blocks, const double* __restrict__ partial,
                                                                 double scale, int accumulate,
                                                                 double* __restrict__ out) {
    __shared__ double red[9][kReduceThreads / kWave];
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    for (int c = 0; c < 9; ++c) {
        double t = 0.0;
        for (int b = threadIdx.x; b < blocks; b += kReduceThreads) t += partial[static_cast<std::size_t>(b) * 9 + c];
        t = wave_sum<kWave>(t);
        if (lane == 0) red[c][wave] = t;
    }
    __syncthreads();
    if (threadIdx.x < 9) {
        double t = 0.0;
        for (int w = 0; w < kReduceThreads / kWave; ++w) t += red[threadIdx.x][w];
        out[threadIdx.x] = accumulate ? out[threadIdx.x] + scale * t : scale * t;
    }
}

__global__ void k_scale9(const double* __restrict__ in, double scale, double* __restrict__ out) {
    if (threadIdx.x < 9) out[threadIdx.x] = scale * in[threadIdx.x];
}

__global__ __launch_bounds__(1024) void k_energy_sum(int N, const double* __restrict__ e, double* __restrict__ total) {
    double s = 0.0;
    for (int i = threadIdx.x; i < N; i += blockDim.x) s += e[i];
    __shared__ double red[1024 / kWave];
    s = wave_sum<kWave>(s);
    if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        for (int w = 0; w < 1024 / kWave; ++w) t += red[w];
        total[0] = t;
    }
}

// ---------------------------------------------------------------------------
// Kernel set of one shape
// ---------------------------------------------------------------------------
struct TimerScope {
    LaunchTimer* t;
    const char* name;
    hipStream_t s;
    TimerScope(LaunchTimer* t_, const char* n, hipStream_t s_) : t(t_), name(n), s(s_) {
        if (t) t->begin(name, s);
    }
    ~TimerScope() {
        if (t) t->end(name, s);
    }
};

// M0TAB / M1TAB: compiled ProductTable of the model's M0 / M1 monomial lists,
// or void for the table-driven polynomial kernels.
template <int C, int LMAX, int LMAXH, class M0TAB, class M1TAB>
struct KernelSetImpl final : KernelSet {
    using S = Shape<LMAX, LMAXH>;
    static constexpr bool kM0Unrolled = !std::is_same_v<M0TAB, void>;
    // R1 forward reads records with scalar loads (its VGPRs hold the 88+
    // coupling rows); the R1 reverse stages them through LDS
    using Records = RecordEdges<C, S::NY, S::REC_F, S::REC_B, false>;
    using StagedRecords = RecordEdges<C, S::NY, S::REC_F, S::REC_B, true>;
    using Groups = SourceGroups<LMAX, LMAXH>;
    static constexpr int kGroups = static_cast<int>(Groups::masks.size());
    int record_floats() const override { return S::REC; }
    int record_forward_floats() const override { return S::REC_F; }
    template <class R = Records>
    static R records(const DeviceModel& m, const TileView& t, const Workspace& w) {
        return R{w.erec, w.erec_b, t.e0, m.R1c, S::P * C};
    }
    const char* polynomial_mode() const override { return kM0Unrolled ? "unrolled" : "table"; }

    void edge_geometry(const DeviceModel& m, const DeviceGraph& g, const TileView& t, const double* xyz,
                       const double* r, const int* edge_pair, int* exec, float* erec, float* erec_b,
                       hipStream_t s) const override {
        launch_execution_order(t.r0, t.nr, t.e0, g.offsets, r, m.r_cut, m.x0, m.h, m.intervals, edge_pair, exec, s);
        geometry_records(LMAX, t.ne, xyz, r, m.r_cut, m.x0, m.h, m.intervals, edge_pair, exec, g.neigh + t.e0,
                         g.neigh_types + t.e0, erec, erec_b, s);
    }

    void layer1_forward(const DeviceModel& m, const DeviceGraph& g, const TileView& t, const Workspace& w,
                        bool through_h1, hipStream_t s, LaunchTimer* tm) const override {
        if (t.nr == 0) return;
        {
            TimerScope ts(tm, "r0_forward", s);
            k_r0_forward<C, LMAX><<<t.nr, C, 0, s>>>(t.r0, t.e0, g.offsets, w.erec, m.R0c, m.H0, w.Phi0);
            SMX_LAUNCH_CHECK("r0_forward");
        }
        {
            TimerScope ts(tm, "a0_linear", s);
            launch_node_gemm(t.a0, m.A0_w, w.Phi0, w.A0, s);
        }
        if (m.A0_scaled) {
            TimerScope ts(tm, "a0_density_scale", s);
            launch_density_factors(m, g, t, w.dens_s0, nullptr, s);
            launch_density_scale(t.nr, S::NY * C, w.dens_s0, true, w.A0, s);
        }
        if (!through_h1) return;
        {
            TimerScope ts(tm, "m0_forward", s);
            if constexpr (kM0Unrolled)
                k_m0_forward_ct<C, S::NY, S::NH, M0TAB><<<t.nr, C, 0, s>>>(t.r0, g.node_types, w.A0, m.m0_coef, w.M0,
                                                                          w.xaff);
            else
                k_m0_forward<C, S::NY, S::NH><<<t.nr, C, 0, s>>>(t.r0, g.node_types, w.A0, m.m0_terms, m.m0_toff,
                                                                m.T0, m.m0_coef, w.M0, w.xaff);
            SMX_LAUNCH_CHECK("m0_forward");
        }
        if (m.field) {
            if (w.field_product_only)
                field_product(m, g, t, w, s, tm);
            else
                field_forward(m, g, t, w, s, tm);
            return;
        }
        {
            TimerScope ts(tm, "h1_linear", s);
            launch_node_gemm(t.h1, m.H1_w, w.M0, w.H1 + static_cast<std::size_t>(t.r0) * S::NH * C, s);
        }
        if (m.pre_linear_up) {
            // the readout_1 / skip input in the pre_linear_up basis:
            // x = M0[:,0,:] P0 (+ the residual's lm-0 row)
            // (mace.cpp:1759-1783, 1863-1872)
            TimerScope ts(tm, "h1_affine_scalar", s);
            float* x = w.xaff + static_cast<std::size_t>(t.r0) * C;
            launch_node_gemm(t.cap, m.P0_w, w.M0, x, s);
            if (m.residual) launch_type_bias(t.r0, t.nr, g.node_types, C, m.res_x, x, s);
        }
        if (m.residual) {
            // H1 += the residual through linear_up (mace.cpp:1843-1862)
            TimerScope ts(tm, "h1_residual", s);
            launch_type_bias(t.r0, t.nr, g.node_types, S::NH * C, m.res_H1,
                             w.H1 + static_cast<std::size_t>(t.r0) * S::NH * C, s);
        }
    }

    // MACEField H1 (mace.cpp:1845-1895, 1147-1186): H1p = M0 P (+ b),
    // Z = H1p[l_in rows] W per path, H1f = H1p + coef E Z (and x = H1f[:,0,:]),
    // H1 = H1f U
    void field_product(const DeviceModel& m, const DeviceGraph& g, const TileView& t, const Workspace& w,
                       hipStream_t s, LaunchTimer* tm) const {
        TimerScope ts(tm, "h1_product", s);
        const std::size_t row0 = static_cast<std::size_t>(t.r0) * S::NH * C;
        launch_node_gemm(t.h1, m.P_w, w.M0, w.H1p + row0, s);
        if (m.residual) launch_type_bias(t.r0, t.nr, g.node_types, S::NH * C, m.res_pre, w.H1p + row0, s);
    }

    void field_forward(const DeviceModel& m, const DeviceGraph& g, const TileView& t, const Workspace& w,
                       hipStream_t s, LaunchTimer* tm) const {
        field_product(m, g, t, w, s, tm);
        field_features(m, t, w, s, tm);
    }

    void field_features(const DeviceModel& m, const TileView& t, const Workspace& w, hipStream_t s,
                        LaunchTimer* tm) const override {
        if (t.nr == 0) return;
        TimerScope ts(tm, "h1_field", s);
        const std::size_t row0 = static_cast<std::size_t>(t.r0) * S::NH * C;
        launch_node_gemm(t.fz, m.field_W, w.H1p + row0, w.fzy + static_cast<std::size_t>(t.r0) * m.field_zr * C, s);
        k_field_combine<C, S::NH><<<t.nr, C, 0, s>>>(t.r0, m.field_zr, m.field_entries, m.num_field_entries,
                                                     w.efield, w.efield_per_node, w.H1p, w.fzy, w.H1f, w.xaff);
        SMX_LAUNCH_CHECK("field_combine");
        launch_node_gemm(t.h1, m.U_w, w.H1f + row0, w.H1 + row0, s);
    }

    // its reverse (mace.cpp:1897-1940, 1189-1240): H1p_adj = H1_adj U^T + x's
    // adjoint on lm 0, Y = H1p_adj[l_out rows] W^T, H1p_adj += coef E Y with
    // dE/dE, M0_adj = H1p_adj P^T
    void field_reverse(const DeviceModel& m, const TileView& t, const Workspace& w, hipStream_t s,
                       LaunchTimer* tm) const {
        field_features_reverse(m, t, w, t.nr, s, tm);
        TimerScope ts(tm, "h1_product_reverse", s);
        launch_node_gemm(t.h1, m.P_wt, w.H1p_adj + static_cast<std::size_t>(t.r0) * S::NH * C, w.M0_adj, s);
    }

    void field_features_reverse(const DeviceModel& m, const TileView& t, const Workspace& w, int direct_rows,
                                hipStream_t s, LaunchTimer* tm) const override {
        if (t.nr == 0) return;
        TimerScope ts(tm, "h1_field_reverse", s);
        const std::size_t row0 = static_cast<std::size_t>(t.r0) * S::NH * C;
        launch_node_gemm(t.h1, m.U_wt, w.H1_adj + row0, w.H1p_adj + row0, s);
        if (direct_rows > 0) {
            k_field_direct_add<<<direct_rows, C, 0, s>>>(t.r0, S::NH, C, w.direct, w.H1p_adj);
            SMX_LAUNCH_CHECK("field_direct_add");
        }
        launch_node_gemm(t.fy, m.field_Wt, w.H1p_adj + row0, w.fzy + static_cast<std::size_t>(t.r0) * m.field_yr * C,
                         s);
        k_field_reverse_combine<C, S::NH><<<t.nr, C, 0, s>>>(t.r0, m.field_yr, m.field_entries, m.num_field_entries,
                                                             w.efield, w.efield_per_node, w.H1p, w.fzy, w.H1p_adj,
                                                             w.field_part);
        SMX_LAUNCH_CHECK("field_reverse_combine");
        if (!w.efield_per_node) {
            k_field_adj_sum<<<1, 256, 0, s>>>(t.r0 + t.nr, w.field_part, w.field_adj);
            SMX_LAUNCH_CHECK("field_adj_sum");
        }
    }

    void layer2(const DeviceModel& m, const DeviceGraph& g, const TileView& t, const Workspace& w, hipStream_t s,
                LaunchTimer* tm) const override {
        if (t.nr == 0) return;
        {
            TimerScope ts(tm, "r1_forward", s);
            static_for<0, kGroups>([&](auto gc) {
                constexpr int gi = gc;
                constexpr int SL = r1_forward_slices<C, Records>();
                k_r1_forward<C, LMAX, LMAXH, Groups::masks[gi], (gi > 0), Records>
                    <<<r1_forward_blocks<C, Records>(t.nr), C / SL, 0, s>>>(t.r0, t.nr, g.offsets, nullptr, g.neigh,
                                                                           records(m, t, w), w.H1, m.cg, w.Phi1);
                SMX_LAUNCH_CHECK("r1_forward");
            });
        }
        {
            TimerScope ts(tm, "a1_linear", s);
            launch_node_gemm(t.a1f, m.A1_w, w.Phi1, w.A1, s);
        }
        if (m.A1_scaled) {
            TimerScope ts(tm, "a1_density_scale", s);
            launch_density_factors(m, g, t, nullptr, w.dens_s1, s);
            launch_density_scale(t.nr, S::NY * C, w.dens_s1, false, w.A1, s);
        }
        {
            TimerScope ts(tm, "readout", s);
            k_m1<C, S::NY, M1TAB><<<t.nr, C, 0, s>>>(t.r0, g.node_types, w.A1, m.m1_terms, m.T1, m.m1_coef, w.M1,
                                                    w.A1_adj);
            SMX_LAUNCH_CHECK("m1");
            k_readout<C, S::NY><<<t.num_batches, 64 * kReadoutWaves, 0, s>>>(
                t.r0, t.batches, t.node_list, g.node_types, w.M1, w.xaff, m.H2_T, m.H2_Tt, m.H2_M1, m.H2_M1t, m.q,
                m.W1r, m.W2r, m.hidden, m.readout_scale, m.E0, w.node_energies, w.direct, w.A1_adj);
            SMX_LAUNCH_CHECK("readout");
        }
        if (m.A1_scaled) {
            TimerScope ts(tm, "a1_density_reverse", s);
            launch_density_adjoint(t.nr, S::NY * C, w.A1, w.dens_s1, false, w.A1_adj, w.dens_dot1, s);
        }
        {
            TimerScope ts(tm, "a1_linear_reverse", s);
            launch_node_gemm(t.a1r, m.A1_wt, w.A1_adj, w.dPhi1, s);
        }
        {
            TimerScope ts(tm, "r1_reverse", s);
            static_for<0, kGroups>([&](auto gc) {
                constexpr int gi = gc;
                k_r1_reverse<C, LMAX, LMAXH, Groups::masks[gi], (gi > 0), StagedRecords><<<t.nr, C, 0, s>>>(
                    t.r0, t.e0, g.offsets, g.neigh, records<StagedRecords>(m, t, w), w.H1, m.cg, w.dPhi1, w.Wsrc,
                    w.node_forces);
                SMX_LAUNCH_CHECK("r1_reverse");
            });
        }
        if (m.A1_scaled) {
            TimerScope ts(tm, "a1_density_forces", s);
            launch_density_forces(m, g, t, nullptr, nullptr, w.dens_s1, w.dens_dot1, w.node_forces, s);
        }
        if (m.has_zbl) {
            TimerScope ts(tm, "zbl", s);
            launch_zbl(m, g, t, w.node_energies, w.node_forces, s);
        }
    }

    void single_readout(const DeviceModel& m, const DeviceGraph& g, const TileView& t, const Workspace& w,
                        hipStream_t s, LaunchTimer* tm) const override {
        if (t.nr == 0) return;
        // mace.cpp:265-281: M1 of H1 (its NH components, table-driven
        // polynomial), H2, readouts, reverse H2 and M1 into H1_adj
        const float* h1 = w.H1 + static_cast<std::size_t>(t.r0) * S::NH * C;
        float* h1_adj = w.H1_adj + static_cast<std::size_t>(t.r0) * S::NH * C;
        {
            TimerScope ts(tm, "readout", s);
            k_m1<C, S::NH, void><<<t.nr, C, 0, s>>>(t.r0, g.node_types, h1, m.m1_terms, m.T1, m.m1_coef, w.M1,
                                                   h1_adj);
            SMX_LAUNCH_CHECK("m1");
            k_readout<C, S::NH><<<t.num_batches, 64 * kReadoutWaves, 0, s>>>(
                t.r0, t.batches, t.node_list, g.node_types, w.M1, w.xaff, m.H2_T, m.H2_Tt, m.H2_M1, m.H2_M1t, m.q,
                m.W1r, m.W2r, m.hidden, m.readout_scale, m.E0, w.node_energies, w.direct, h1_adj);
            SMX_LAUNCH_CHECK("readout");
        }
        // the directed forces of the tile's edges start at zero: ZBL and the
        // layer-1 reverse add to them
        launch_fill_zero(w.node_forces, static_cast<std::size_t>(t.ne) * 3, s);
        if (m.has_zbl) {
            TimerScope ts(tm, "zbl", s);
            launch_zbl(m, g, t, w.node_energies, w.node_forces, s);
        }
    }

    void source_adjoint_all(const DeviceGraph& g, const Workspace& w, const double* r, double r_cut, hipStream_t s,
                            LaunchTimer* tm) const override {
        if (g.F == 0) return;
        TimerScope ts(tm, "source_gather", s);
        k_source_gather<C, S::NH, false><<<g.F, C, 0, s>>>(g.soff, g.sedges, w.Wsrc, r, r_cut, w.H1_adj);
        SMX_LAUNCH_CHECK("source_gather");
    }

    void source_adjoint_tile(const DeviceGraph& g, const TileView& t, const Workspace& w, const double* r,
                             double r_cut, hipStream_t s, LaunchTimer* tm) const override {
        if (t.touched_count == 0) return;
        TimerScope ts(tm, "source_gather", s);
        const long long e0 = g.edge_base + t.e0;
        if (g.sedges64)
            k_tile_source_adjoint<C, S::NH><<<t.touched_count, C, 0, s>>>(t.touched, e0, e0 + t.ne, g.soff64,
                                                                         g.sedges64, w.Wsrc, r, r_cut, w.H1_adj);
        else
            k_tile_source_adjoint<C, S::NH><<<t.touched_count, C, 0, s>>>(t.touched, e0, e0 + t.ne, g.soff, g.sedges,
                                                                         w.Wsrc, r, r_cut, w.H1_adj);
        SMX_LAUNCH_CHECK("tile_source_adjoint");
    }

    void layer1_reverse(const DeviceModel& m, const DeviceGraph& g, const TileView& t, const Workspace& w,
                        bool accumulate_forces, hipStream_t s, LaunchTimer* tm) const override {
        if (t.nr == 0) return;
        // the direct adjoint of the readout_1 / skip input enters M0_adj[:,0,:]
        // as is (m0_composite) or as P0 d (pre_linear_up, mace.cpp:1785-1814);
        // with field coupling it entered H1p_adj[:,0,:] already
        const float* direct = w.direct;
        if (m.field && w.field_reverse_done) {
            TimerScope ts(tm, "h1_product_reverse", s);
            launch_node_gemm(t.h1, m.P_wt, w.H1p_adj + static_cast<std::size_t>(t.r0) * S::NH * C, w.M0_adj, s);
            direct = nullptr;
        } else if (m.field) {
            field_reverse(m, t, w, s, tm);
            direct = nullptr;
        } else {
            TimerScope ts(tm, "h1_linear_reverse", s);
            launch_node_gemm(t.h1, m.H1_wt, w.H1_adj + static_cast<std::size_t>(t.r0) * S::NH * C, w.M0_adj, s);
        }
        if (m.pre_linear_up && !m.field) {
            TimerScope ts(tm, "h1_affine_scalar_reverse", s);
            launch_node_gemm(t.cap_r, m.P0_wt, w.direct + static_cast<std::size_t>(t.r0) * C,
                             w.direct_m0 + static_cast<std::size_t>(t.r0) * C, s);
            direct = w.direct_m0;
        }
        {
            TimerScope ts(tm, "m0_reverse", s);
            if constexpr (kM0Unrolled)
                k_m0_reverse_ct<C, S::NY, S::NH, M0TAB><<<t.nr, C, 0, s>>>(t.r0, g.node_types, w.A0, w.M0_adj,
                                                                          direct, m.m0_coef, w.A0_adj);
            else
                k_m0_reverse<C, S::NY, S::NH><<<t.nr, C, 0, s>>>(t.r0, g.node_types, w.A0, w.M0_adj, direct,
                                                                m.m0_terms, m.m0_toff, m.T0, m.m0_coef, w.A0_adj);
            SMX_LAUNCH_CHECK("m0_reverse");
        }
        if (m.A0_scaled) {
            TimerScope ts(tm, "a0_density_reverse", s);
            launch_density_adjoint(t.nr, S::NY * C, w.A0, w.dens_s0, true, w.A0_adj, w.dens_dot0, s);
        }
        {
            TimerScope ts(tm, "a0_linear_reverse", s);
            launch_node_gemm(t.a0, m.A0_wt, w.A0_adj, w.Phi0_adj, s);
        }
        {
            TimerScope ts(tm, "r0_reverse", s);
            if (accumulate_forces)
                k_r0_reverse<C, LMAX, true><<<t.nr, C, 0, s>>>(t.r0, t.e0, g.offsets, w.erec, w.erec_b, m.R0c, m.H0,
                                                               w.Phi0_adj, w.node_forces);
            else
                k_r0_reverse<C, LMAX, false><<<t.nr, C, 0, s>>>(t.r0, t.e0, g.offsets, w.erec, w.erec_b, m.R0c, m.H0,
                                                                w.Phi0_adj, w.node_forces);
            SMX_LAUNCH_CHECK("r0_reverse");
        }
        if (m.A0_scaled) {
            TimerScope ts(tm, "a0_density_forces", s);
            launch_density_forces(m, g, t, w.dens_s0, w.dens_dot0, nullptr, nullptr, w.node_forces, s);
        }
    }

    void field_response_prepare(const DeviceModel& m, const TileView& t, const Workspace& w,
                                const ResponseWorkspace& rw, hipStream_t s, LaunchTimer* tm) const override {
        if constexpr (LMAXH == 0) {
            throw std::invalid_argument("MACEField models have a hidden L_max of 1 or 2");
        } else {
            if (t.nr == 0) return;
            TimerScope ts(tm, "field_response_prepare", s);
            launch_node_gemm(t.fz, m.field_W, w.H1p, rw.Z, s);
            launch_node_gemm(t.h1, m.U_wt, w.H1_adj, rw.H1f_adj, s);
            k_field_direct_add<<<t.nr, C, 0, s>>>(0, S::NH, C, w.direct, rw.H1f_adj);
            SMX_LAUNCH_CHECK("field_direct_add");
            launch_node_gemm(t.fy, m.field_Wt, rw.H1f_adj, rw.Y, s);
        }
    }

    // One field component's tangent (mace_kokkos_response.tpp:396-2343) over
    // the direct plan's single tile (receivers and feature nodes are the
    // same N nodes, r0 = e0 = 0)
    void field_response_seed(const DeviceModel& m, const DeviceGraph& g, const TileView& t, const Workspace& w,
                             const ResponseWorkspace& rw, int seed, bool forces, hipStream_t s,
                             LaunchTimer* tm) const override {
        if constexpr (LMAXH == 0) {
            throw std::invalid_argument("MACEField models have a hidden L_max of 1 or 2");
        } else {
            const int N = t.nr;
            if (N == 0) return;
            double* f = rw.forces + static_cast<std::size_t>(seed) * 3 * t.ne;
            TimerScope ts(tm, "field_response", s);
            // H1f_dot (and x_dot), H1_dot = H1f_dot U
            k_field_tangent<C, S::NH><<<N, C, 0, s>>>(m.field_zr, m.field_entries, m.num_field_entries, seed, rw.Z,
                                                      rw.H1f_dot, rw.x_dot);
            SMX_LAUNCH_CHECK("field_tangent");
            launch_node_gemm(t.h1, m.U_w, rw.H1f_dot, rw.H1_dot, s);
            // Phi1_dot: the R1 forward of H1_dot; A1_dot (density-scaled like A1)
            static_for<0, kGroups>([&](auto gc) {
                constexpr int gi = gc;
                constexpr int SL = r1_forward_slices<C, Records>();
                k_r1_forward<C, LMAX, LMAXH, Groups::masks[gi], (gi > 0), Records>
                    <<<r1_forward_blocks<C, Records>(N), C / SL, 0, s>>>(0, N, g.offsets, nullptr, g.neigh,
                                                                         records(m, t, w), rw.H1_dot, m.cg,
                                                                         rw.Phi1_dot);
                SMX_LAUNCH_CHECK("r1_forward");
            });
            launch_node_gemm(t.a1f, m.A1_w, rw.Phi1_dot, rw.A1_dot, s);
            if (m.A1_scaled) launch_density_scale(N, S::NY * C, w.dens_s1, false, rw.A1_dot, s);
            // M1_dot, the M1 gradient and its tangent; the readout's tangent
            constexpr int TL = m1_tangent_lanes<C, M1TAB>();
            k_m1_tangent<C, S::NY, M1TAB><<<dim3(N, C / TL), TL, 0, s>>>(
                g.node_types, w.A1, rw.A1_dot, m.m1_terms, m.T1, m.m1_coef, rw.M1_dot, rw.g, rw.gd);
            SMX_LAUNCH_CHECK("m1_tangent");
            k_readout_tangent<C><<<N, C, 0, s>>>(g.node_types, S::NY, w.M1, rw.M1_dot, w.xaff, rw.x_dot, m.H2_T,
                                                 m.H2_Tt, m.H2_M1, m.H2_M1t, m.W1r, m.W2r, m.hidden,
                                                 m.readout_scale, rw.g, rw.gd, rw.direct_dot, rw.A1_adj_dot,
                                                 m.A1_scaled ? rw.A1s_adj : nullptr);
            SMX_LAUNCH_CHECK("readout_tangent");
            if (m.A1_scaled) {
                // the scale's adjoint dot product sum A1_adj A1 and its tangent
                // (both factors), then the adjoint's tangent scaled by 1/s
                launch_density_adjoint(N, S::NY * C, w.A1, w.dens_s1, false, rw.A1_adj_dot, rw.dot_a, s);
                launch_density_adjoint(N, S::NY * C, rw.A1_dot, w.dens_s1, false, rw.A1s_adj, rw.dot_b, s);
            }
            launch_node_gemm(t.a1r, m.A1_wt, rw.A1_adj_dot, rw.dPhi1_dot, s);
            // the R1 reverse, bilinear in (H1, dPhi1): (H1, dPhi1_dot) gives
            // the source terms of H1_adj_dot and part of the forces,
            // (H1_dot, dPhi1) the rest of the forces (its source terms are
            // not formed)
            static_for<0, kGroups>([&](auto gc) {
                constexpr int gi = gc;
                k_r1_reverse<C, LMAX, LMAXH, Groups::masks[gi], (gi > 0), StagedRecords><<<N, C, 0, s>>>(
                    0, 0, g.offsets, g.neigh, records<StagedRecords>(m, t, w), w.H1, m.cg, rw.dPhi1_dot, w.Wsrc, f);
                SMX_LAUNCH_CHECK("r1_reverse");
            });
            k_source_gather<C, S::NH, false><<<g.F, C, 0, s>>>(g.soff, g.sedges, w.Wsrc, t.r, m.r_cut,
                                                               rw.H1_adj_dot);
            SMX_LAUNCH_CHECK("source_gather");
            if (forces) {
                static_for<0, kGroups>([&](auto gc) {
                    constexpr int gi = gc;
                    k_r1_reverse<C, LMAX, LMAXH, Groups::masks[gi], true, StagedRecords, C, false><<<N, C, 0, s>>>(
                        0, 0, g.offsets, g.neigh, records<StagedRecords>(m, t, w), rw.H1_dot, m.cg, w.dPhi1, nullptr,
                        f);
                    SMX_LAUNCH_CHECK("r1_reverse");
                });
                if (m.A1_scaled) {
                    launch_density_forces(m, g, t, nullptr, nullptr, w.dens_s1, rw.dot_a, f, s);
                    launch_density_forces(m, g, t, nullptr, nullptr, w.dens_s1, rw.dot_b, f, s);
                }
            }
            // the field terms' reverse: H1f_adj_dot = H1_adj_dot U^T (+
            // direct_dot), its path products Y_dot, then H1p_adj_dot += coef
            // (E Y_dot + [c = seed] Y) with the Hessian column from Y_dot
            launch_node_gemm(t.h1, m.U_wt, rw.H1_adj_dot, rw.H1p_adj_dot, s);
            k_field_direct_add<<<N, C, 0, s>>>(0, S::NH, C, rw.direct_dot, rw.H1p_adj_dot);
            SMX_LAUNCH_CHECK("field_direct_add");
            launch_node_gemm(t.fy, m.field_Wt, rw.H1p_adj_dot, rw.Y_dot, s);
            k_field_reverse_combine<C, S::NH><<<N, C, 0, s>>>(0, m.field_yr, m.field_entries, m.num_field_entries,
                                                              w.efield, 0, w.H1p, rw.Y_dot, rw.H1p_adj_dot, rw.part);
            SMX_LAUNCH_CHECK("field_reverse_combine");
            k_field_adj_sum<<<1, 256, 0, s>>>(N, rw.part, rw.hessian_t + 3 * seed);
            SMX_LAUNCH_CHECK("field_adj_sum");
            k_field_reverse_combine<C, S::NH><<<N, C, 0, s>>>(0, m.field_yr, m.field_entries, m.num_field_entries,
                                                              rw.unit + 3 * seed, 0, w.H1p, rw.Y, rw.H1p_adj_dot,
                                                              rw.part_scratch);
            SMX_LAUNCH_CHECK("field_reverse_combine");
            if (!forces) return;
            // the layer-1 reverse of H1p_adj_dot (M0 and A0 do not depend on
            // the field): M0_adj_dot, A0_adj_dot (density scale), the R0 reverse
            launch_node_gemm(t.h1, m.P_wt, rw.H1p_adj_dot, rw.M0_adj_dot, s);
            if constexpr (kM0Unrolled)
                k_m0_reverse_ct<C, S::NY, S::NH, M0TAB><<<N, C, 0, s>>>(0, g.node_types, w.A0, rw.M0_adj_dot, nullptr,
                                                                       m.m0_coef, rw.A0_adj_dot);
            else
                k_m0_reverse<C, S::NY, S::NH><<<N, C, 0, s>>>(0, g.node_types, w.A0, rw.M0_adj_dot, nullptr,
                                                             m.m0_terms, m.m0_toff, m.T0, m.m0_coef, rw.A0_adj_dot);
            SMX_LAUNCH_CHECK("m0_reverse");
            if (m.A0_scaled) launch_density_adjoint(N, S::NY * C, w.A0, w.dens_s0, true, rw.A0_adj_dot, rw.dot_a, s);
            launch_node_gemm(t.a0, m.A0_wt, rw.A0_adj_dot, rw.Phi0_adj_dot, s);
            k_r0_reverse<C, LMAX, true><<<N, C, 0, s>>>(0, 0, g.offsets, w.erec, w.erec_b, m.R0c, m.H0,
                                                        rw.Phi0_adj_dot, f);
            SMX_LAUNCH_CHECK("r0_reverse");
            if (m.A0_scaled) launch_density_forces(m, g, t, w.dens_s0, rw.dot_a, nullptr, nullptr, f, s);
        }
    }
};

template <int LMAX, int LMAXH>
void paths_of(std::vector<int>& le, std::vector<int>& ls, std::vector<int>& lo) {
    using S = Shape<LMAX, LMAXH>;
    le.clear();
    ls.clear();
    lo.clear();
    for (int p = 0; p < S::P; ++p) {
        le.push_back(S::paths[p].le);
        ls.push_back(S::paths[p].ls);
        lo.push_back(S::paths[p].lo);
    }
}

// true when the canonical lists equal the compiled table TAB
template <class TAB>
bool table_matches(const std::vector<std::int32_t>& terms, const std::vector<std::int32_t>& offsets) {
    if constexpr (!TAB::available) {
        return false;
    } else {
        if (terms.size() != static_cast<std::size_t>(TAB::NT) || offsets.size() != TAB::offset.size()) return false;
        for (int t = 0; t < TAB::NT; ++t)
            if (terms[t] != TAB::terms[t]) return false;
        for (std::size_t o = 0; o < offsets.size(); ++o)
            if (offsets[o] != TAB::offset[o]) return false;
        return true;
    }
}

template <int C, int LMAX, int LMAXH, int CORR>
std::unique_ptr<KernelSet> pick_polynomials(const std::vector<std::int32_t>& m0_terms,
                                            const std::vector<std::int32_t>& m0_offsets,
                                            const std::vector<std::int32_t>& m1_terms) {
    using T0 = ProductTable<LMAX, LMAXH, CORR>;
    using T1 = ProductTable<LMAX, 0, CORR>;
    const std::vector<std::int32_t> m1_offsets{0, static_cast<std::int32_t>(m1_terms.size())};
    // each product basis unrolled when its list is a compiled table (a
    // one-interaction model's M1, over H1's components, never is)
    bool m0 = false, m1 = false;
    if constexpr (T0::available) m0 = table_matches<T0>(m0_terms, m0_offsets);
    if constexpr (T1::available) m1 = table_matches<T1>(m1_terms, m1_offsets);
    if constexpr (T0::available && T1::available)
        if (m0 && m1) return std::make_unique<KernelSetImpl<C, LMAX, LMAXH, T0, T1>>();
    if constexpr (T0::available)
        if (m0) return std::make_unique<KernelSetImpl<C, LMAX, LMAXH, T0, void>>();
    if constexpr (T1::available)
        if (m1) return std::make_unique<KernelSetImpl<C, LMAX, LMAXH, void, T1>>();
    return std::make_unique<KernelSetImpl<C, LMAX, LMAXH, void, void>>();
}

int max_degree(const std::vector<std::int32_t>& terms) {
    int d = 0;
    for (const std::int32_t t : terms) d = std::max(d, t >> 24);
    return d;
}

}  // namespace

std::unique_ptr<KernelSet> make_kernel_set(int C, int l_max, int L_max, const std::vector<std::int32_t>& m0_terms,
                                           const std::vector<std::int32_t>& m0_offsets,
                                           const std::vector<std::int32_t>& m1_terms) {
    const int corr = std::max(max_degree(m0_terms), max_degree(m1_terms));
    if (C == 256 && l_max == 3 && L_max == 2)
        return corr == 3 ? pick_polynomials<256, 3, 2, 3>(m0_terms, m0_offsets, m1_terms)
                         : std::make_unique<KernelSetImpl<256, 3, 2, void, void>>();
    if (C == 32 && l_max == 2 && L_max == 1)
        return corr == 2 ? pick_polynomials<32, 2, 1, 2>(m0_terms, m0_offsets, m1_terms)
                         : std::make_unique<KernelSetImpl<32, 2, 1, void, void>>();
    if (C == 128 && l_max == 3 && L_max == 1)
        return corr == 3 ? pick_polynomials<128, 3, 1, 3>(m0_terms, m0_offsets, m1_terms)
                         : std::make_unique<KernelSetImpl<128, 3, 1, void, void>>();
    // the shapes of the MACE-OMAT-0 small (128x0e, l_max 3) and MP-0b2 large
    // (128x0e+128x1o+128x2e) checkpoints
    // (symmetrix/test/data/execution_contracts/jit_r1_mace_{omat0_small,mp0b2_large}_contract.json)
    if (C == 128 && l_max == 3 && L_max == 0)
        return corr == 3 ? pick_polynomials<128, 3, 0, 3>(m0_terms, m0_offsets, m1_terms)
                         : std::make_unique<KernelSetImpl<128, 3, 0, void, void>>();
    if (C == 128 && l_max == 3 && L_max == 2)
        return corr == 3 ? pick_polynomials<128, 3, 2, 3>(m0_terms, m0_offsets, m1_terms)
                         : std::make_unique<KernelSetImpl<128, 3, 2, void, void>>();
    return nullptr;
}

bool kernel_paths(int l_max, int L_max, std::vector<int>& le, std::vector<int>& ls, std::vector<int>& lo) {
    if (l_max == 2 && L_max == 1) {
        paths_of<2, 1>(le, ls, lo);
        return true;
    }
    if (l_max == 3 && L_max == 1) {
        paths_of<3, 1>(le, ls, lo);
        return true;
    }
    if (l_max == 3 && L_max == 0) {
        paths_of<3, 0>(le, ls, lo);
        return true;
    }
    if (l_max == 3 && L_max == 2) {
        paths_of<3, 2>(le, ls, lo);
        return true;
    }
    return false;
}

void launch_node_gemm(const GemmPlan& plan, const float* W, const float* in, float* out, hipStream_t s) {
    if (plan.num_tiles == 0) return;
    // Narrower waves (64 columns) when 128-column waves would give fewer than
    // about 8 per SIMD (1024 SIMDs): more waves fill the chip better than the
    // wider tile's operand reuse pays (the 5,000-node linears run 8% faster).
    int n_sub = plan.n_sub;
    const long long waves128 = static_cast<long long>(plan.num_tiles) * ((plan.max_n + 127) / 128);
    // Large linears (at least ~32 waves per SIMD): the shared-operand kernel
    // (measured 15-20% faster from 480,000 rows on; slower at 80,000).
    if (n_sub == 8 && plan.sets && plan.num_sets > 0 && waves128 >= 32 * 1024) {
        const dim3 grid(plan.num_sets, (plan.max_n + 127) / 128);
        k_node_gemm_shared<<<grid, 64 * kGemmShareWaves, 0, s>>>(plan.sets, plan.tiles, plan.groups, plan.rows, W,
                                                                 in, out);
        SMX_LAUNCH_CHECK("node_gemm_shared");
        return;
    }
    if (n_sub == 8 && (plan.narrow || waves128 < 8 * 1024)) n_sub = 4;
    const int cols = 16 * n_sub;
    const dim3 grid(plan.num_tiles, (plan.max_n + cols - 1) / cols);
    const unsigned block = 64;
    switch (n_sub) {
        case 8:
            k_node_gemm<8><<<grid, block, 0, s>>>(plan.tiles, plan.groups, plan.rows, W, in, out);
            break;
        case 4:
            k_node_gemm<4><<<grid, block, 0, s>>>(plan.tiles, plan.groups, plan.rows, W, in, out);
            break;
        case 2:
            k_node_gemm<2><<<grid, block, 0, s>>>(plan.tiles, plan.groups, plan.rows, W, in, out);
            break;
        default:
            k_node_gemm<1><<<grid, block, 0, s>>>(plan.tiles, plan.groups, plan.rows, W, in, out);
            break;
    }
    SMX_LAUNCH_CHECK("node_gemm");
}

void swizzle_gemm_weights(const float* w, int K, int N, float* out) {
    if (K % 16 != 0 || N % 16 != 0) throw std::invalid_argument("node-linear dimensions must be multiples of 16");
    const int nblk = N / 16;
    for (int kc = 0; kc < K / 16; ++kc)
        for (int nb = 0; nb < nblk; ++nb)
            for (int kg = 0; kg < 4; ++kg)
                for (int c = 0; c < 16; ++c)
                    for (int s = 0; s < 4; ++s)
                        out[((((static_cast<std::size_t>(kc) * nblk + nb) * 4 + kg) * 16 + c) * 4) + s] =
                            w[static_cast<std::size_t>(16 * kc + 4 * kg + s) * N + 16 * nb + c];
}

void launch_atom_forces(int N, int F, const int* offsets, const int* soff, const int* sedges, const int* feature_of,
                        const double* node_forces, double* atom_forces, hipStream_t s) {
    if (F == 0) return;
    k_atom_forces<<<blocks_for(F, 256 / kWave), 256, 0, s>>>(N, F, offsets, soff, sedges, feature_of, node_forces,
                                                             atom_forces);
    SMX_LAUNCH_CHECK("atom_forces");
}

template <class T, bool kScatter>
__global__ __launch_bounds__(256) void k_move_rows(int row_floats, const int* __restrict__ index,
                                                   const T* __restrict__ src, T* __restrict__ dst) {
    const std::size_t k = blockIdx.x;
    const std::size_t from = kScatter ? k : static_cast<std::size_t>(index[k]);
    const std::size_t to = kScatter ? static_cast<std::size_t>(index[k]) : k;
    for (int q = threadIdx.x; q < row_floats; q += 256) dst[to * row_floats + q] = src[from * row_floats + q];
}

void launch_gather_rows(int count, int row_floats, const int* index, const float* src, float* dst, hipStream_t s) {
    if (count == 0) return;
    k_move_rows<float, false><<<count, 256, 0, s>>>(row_floats, index, src, dst);
    SMX_LAUNCH_CHECK("gather_rows");
}

void launch_scatter_rows(int count, int row_floats, const int* index, const float* src, float* dst, hipStream_t s) {
    if (count == 0) return;
    k_move_rows<float, true><<<count, 256, 0, s>>>(row_floats, index, src, dst);
    SMX_LAUNCH_CHECK("scatter_rows");
}

void launch_scatter_rows(int count, int row_values, const int* index, const double* src, double* dst,
                         hipStream_t s) {
    if (count == 0) return;
    k_move_rows<double, true><<<count, 256, 0, s>>>(row_values, index, src, dst);
    SMX_LAUNCH_CHECK("scatter_rows_f64");
}

void launch_stress(std::int64_t E, const double* node_forces, const double* xyz, double volume, double* partial,
                   int partial_blocks, double* stress, hipStream_t s) {
    k_stress_partial<<<partial_blocks, kReduceThreads, 0, s>>>(E, node_forces, xyz, partial);
    SMX_LAUNCH_CHECK("stress_partial");
    k_stress_final<<<1, kReduceThreads, 0, s>>>(partial_blocks, partial, -1.0 / volume, 0, stress);
    SMX_LAUNCH_CHECK("stress_final");
}

void launch_virial_accumulate(std::int64_t E, const double* node_forces, const double* xyz, double* partial,
                              int partial_blocks, double* virial, hipStream_t s) {
    if (E == 0) return;
    k_stress_partial<<<partial_blocks, kReduceThreads, 0, s>>>(E, node_forces, xyz, partial);
    SMX_LAUNCH_CHECK("virial_partial");
    k_stress_final<<<1, kReduceThreads, 0, s>>>(partial_blocks, partial, 1.0, 1, virial);
    SMX_LAUNCH_CHECK("virial_accumulate");
}

void launch_scale9(const double* in, double scale, double* out, hipStream_t s) {
    k_scale9<<<1, 64, 0, s>>>(in, scale, out);
    SMX_LAUNCH_CHECK("scale9");
}

template <class T>
void tile_forces(const TileView& t, const int* touched, int touched_count, const int* offsets, long long offsets_e0,
                 const T* soff, const T* sedges, const int* receiver_row, const double* node_forces, double* F,
                 hipStream_t s) {
    if (touched_count > 0) {
        k_tile_forces_sources<<<blocks_for(touched_count, 256 / kWave), 256, 0, s>>>(
            touched, touched_count, t.e0, t.e0 + t.ne, soff, sedges, node_forces, F);
        SMX_LAUNCH_CHECK("tile_forces_sources");
    }
    if (t.nr > 0) {
        k_tile_forces_receivers<<<blocks_for(t.nr, 256 / kWave), 256, 0, s>>>(t.r0, t.nr, offsets_e0, offsets,
                                                                              receiver_row, node_forces, F);
        SMX_LAUNCH_CHECK("tile_forces_receivers");
    }
}

void launch_tile_forces(const TileView& t, const int* touched, int touched_count, const int* offsets,
                        long long offsets_e0, const int* soff, const int* sedges, const int* receiver_row,
                        const double* node_forces, double* F, hipStream_t s) {
    tile_forces(t, touched, touched_count, offsets, offsets_e0, soff, sedges, receiver_row, node_forces, F, s);
}

void launch_tile_forces(const TileView& t, const int* touched, int touched_count, const int* offsets,
                        long long offsets_e0, const long long* soff, const long long* sedges,
                        const int* receiver_row, const double* node_forces, double* F, hipStream_t s) {
    tile_forces(t, touched, touched_count, offsets, offsets_e0, soff, sedges, receiver_row, node_forces, F, s);
}

void launch_type_bias(int r0, int nr, const int* types, int row_len, const float* bias, float* rows, hipStream_t s) {
    const long long n = static_cast<long long>(nr) * row_len;
    if (n == 0) return;
    k_type_bias<<<static_cast<unsigned>((n + 255) / 256), 256, 0, s>>>(r0, nr, types, row_len, bias, rows);
    SMX_LAUNCH_CHECK("type_bias");
}

void launch_fill_zero(float* p, std::size_t n, hipStream_t s) {
    if (n == 0) return;
    k_fill_f32<<<static_cast<unsigned>(std::min<std::size_t>((n + 255) / 256, 4096)), 256, 0, s>>>(n, p);
    SMX_LAUNCH_CHECK("fill_f32");
}

void launch_fill_zero(double* p, std::size_t n, hipStream_t s) {
    if (n == 0) return;
    k_fill_f64<<<static_cast<unsigned>(std::min<std::size_t>((n + 255) / 256, 4096)), 256, 0, s>>>(n, p);
    SMX_LAUNCH_CHECK("fill_f64");
}

void launch_energy_sum(int N, const double* node_energies, double* total, hipStream_t s) {
    k_energy_sum<<<1, 1024, 0, s>>>(N, node_energies, total);
    SMX_LAUNCH_CHECK("energy_sum");
}

}  // namespace smx
