// Product-basis polynomials with a compiled term table (device code shared
// by the evaluator's unrolled kernels and the M0 operator module).  A table
// TAB holds packed monomials (variables v0 <= v1 <= v2 in bytes 0..2, degree
// in byte 3) in TAB::terms and per-output term ranges in TAB::offset; every
// term becomes straight-line code on register-resident variables.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "shapes.hpp"

namespace smx {

template <std::int32_t PK>
__device__ __forceinline__ float monomial_ct(const float* x) {
    constexpr int deg = PK >> 24, v0 = PK & 0xff, v1 = (PK >> 8) & 0xff, v2 = (PK >> 16) & 0xff;
    if constexpr (deg == 1)
        return x[v0];
    else if constexpr (deg == 2)
        return x[v0] * x[v1];
    else
        return x[v0] * x[v1] * x[v2];
}

template <std::int32_t PK>
__device__ __forceinline__ void monomial_grad_ct(const float* x, float* g, float c) {
    constexpr int deg = PK >> 24, v0 = PK & 0xff, v1 = (PK >> 8) & 0xff, v2 = (PK >> 16) & 0xff;
    if constexpr (deg == 1) {
        g[v0] += c;
    } else if constexpr (deg == 2) {
        g[v0] += c * x[v1];
        g[v1] += c * x[v0];
    } else {
        g[v0] += c * x[v1] * x[v2];
        g[v1] += c * x[v0] * x[v2];
        g[v2] += c * x[v0] * x[v1];
    }
}

// one term's share of the tangent along dx: g += its gradient, gd += the
// gradient's derivative along dx (each factor differentiated in turn);
// returns the term's derivative along dx
template <std::int32_t PK>
__device__ __forceinline__ float monomial_tangent_ct(const float* x, const float* dx, float* g, float* gd, float c) {
    constexpr int deg = PK >> 24, v0 = PK & 0xff, v1 = (PK >> 8) & 0xff, v2 = (PK >> 16) & 0xff;
    if constexpr (deg == 1) {
        g[v0] += c;
        return c * dx[v0];
    } else if constexpr (deg == 2) {
        g[v0] += c * x[v1];
        g[v1] += c * x[v0];
        gd[v0] += c * dx[v1];
        gd[v1] += c * dx[v0];
        return c * (x[v1] * dx[v0] + x[v0] * dx[v1]);
    } else {
        g[v0] += c * x[v1] * x[v2];
        g[v1] += c * x[v0] * x[v2];
        g[v2] += c * x[v0] * x[v1];
        gd[v0] += c * (dx[v1] * x[v2] + x[v1] * dx[v2]);
        gd[v1] += c * (dx[v0] * x[v2] + x[v0] * dx[v2]);
        gd[v2] += c * (dx[v0] * x[v1] + x[v0] * dx[v1]);
        return c * (x[v1] * x[v2] * dx[v0] + x[v0] * x[v2] * dx[v1] + x[v0] * x[v1] * dx[v2]);
    }
}

// f = sum_t c_t mono_t(x) over the compiled terms [B, E); cf points at the
// lane's coefficient of term 0 (stride C between terms).
template <class TAB, int B, int E, int C>
__device__ __forceinline__ float poly_ct(const float* x, const float* __restrict__ cf) {
    float f = 0.0f;
    static_range<B, E>([&](auto tc) {
        constexpr int t = tc;
        f += cf[t * C] * monomial_ct<TAB::terms[t]>(x);
    });
    return f;
}

template <class TAB, int B, int E, int C>
__device__ __forceinline__ void poly_grad_ct(const float* x, const float* __restrict__ cf, float* g) {
    static_range<B, E>([&](auto tc) {
        constexpr int t = tc;
        monomial_grad_ct<TAB::terms[t]>(x, g, cf[t * C]);
    });
}

// the derivative of the polynomial along dx (returned), its gradient g and
// the gradient's derivative gd along dx (g, gd accumulated)
template <class TAB, int B, int E, int C>
__device__ __forceinline__ float poly_tangent_ct(const float* x, const float* dx, const float* __restrict__ cf,
                                                 float* g, float* gd) {
    float fd = 0.0f;
    static_range<B, E>([&](auto tc) {
        constexpr int t = tc;
        fd += monomial_tangent_ct<TAB::terms[t]>(x, dx, g, gd, cf[t * C]);
    });
    return fd;
}

}  // namespace smx
