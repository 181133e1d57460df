// Real spherical harmonics of an edge direction and their Cartesian
// gradients (device code shared by the evaluator's edge records and the R0
// operator module).  Conventions of the reference (spherical_harmonic_device.hpp:
// 113-199, mace.cpp:1283-1298): evaluated at the shuffled direction (z, x, y),
// scaled by sqrt(4 pi), gradient (d - u u.d)/r returned in the unshuffled
// order.
#pragma once

#include <hip/hip_runtime.h>

namespace smx {

constexpr double kSqrt4Pi = 3.5449077018110318;

// Orthonormal real harmonics l <= LMAX of a unit vector (x,y,z) (already in the
// shuffled frame (z, x, y) of the edge) and their Cartesian partials.
template <int LMAX>
__device__ __forceinline__ void real_harmonics(float x, float y, float z, float* v, float* dx, float* dy, float* dz) {
    const double pi = 3.14159265358979323846;
    v[0] = static_cast<float>(0.5 / sqrt(pi));
    dx[0] = dy[0] = dz[0] = 0.0f;
    if constexpr (LMAX >= 1) {
        const float c1 = static_cast<float>(sqrt(3.0 / (4.0 * pi)));
        v[1] = c1 * y; dx[1] = 0.0f; dy[1] = c1; dz[1] = 0.0f;
        v[2] = c1 * z; dx[2] = 0.0f; dy[2] = 0.0f; dz[2] = c1;
        v[3] = c1 * x; dx[3] = c1; dy[3] = 0.0f; dz[3] = 0.0f;
    }
    if constexpr (LMAX >= 2) {
        const float c2 = static_cast<float>(0.5 * sqrt(15.0 / pi));
        const float c20 = static_cast<float>(0.25 * sqrt(5.0 / pi));
        const float c22 = static_cast<float>(0.25 * sqrt(15.0 / pi));
        v[4] = c2 * x * y; dx[4] = c2 * y; dy[4] = c2 * x; dz[4] = 0.0f;
        v[5] = c2 * y * z; dx[5] = 0.0f; dy[5] = c2 * z; dz[5] = c2 * y;
        v[6] = c20 * (2 * z * z - x * x - y * y); dx[6] = -2 * c20 * x; dy[6] = -2 * c20 * y; dz[6] = 4 * c20 * z;
        v[7] = c2 * x * z; dx[7] = c2 * z; dy[7] = 0.0f; dz[7] = c2 * x;
        v[8] = c22 * (x * x - y * y); dx[8] = 2 * c22 * x; dy[8] = -2 * c22 * y; dz[8] = 0.0f;
    }
    if constexpr (LMAX >= 3) {
        const float c33 = static_cast<float>(0.25 * sqrt(35.0 / (2.0 * pi)));
        const float c32 = static_cast<float>(0.5 * sqrt(105.0 / pi));
        const float c31 = static_cast<float>(0.25 * sqrt(21.0 / (2.0 * pi)));
        const float c30 = static_cast<float>(0.25 * sqrt(7.0 / pi));
        const float c32b = static_cast<float>(0.25 * sqrt(105.0 / pi));
        const float r2 = x * x + y * y;
        v[9] = c33 * y * (3 * x * x - y * y);
        dx[9] = c33 * 6 * x * y; dy[9] = c33 * (3 * x * x - 3 * y * y); dz[9] = 0.0f;
        v[10] = c32 * x * y * z;
        dx[10] = c32 * y * z; dy[10] = c32 * x * z; dz[10] = c32 * x * y;
        v[11] = c31 * y * (4 * z * z - r2);
        dx[11] = c31 * (-2 * x * y); dy[11] = c31 * (4 * z * z - x * x - 3 * y * y); dz[11] = c31 * 8 * y * z;
        v[12] = c30 * z * (2 * z * z - 3 * r2);
        dx[12] = c30 * (-6 * x * z); dy[12] = c30 * (-6 * y * z); dz[12] = c30 * (6 * z * z - 3 * r2);
        v[13] = c31 * x * (4 * z * z - r2);
        dx[13] = c31 * (4 * z * z - 3 * x * x - y * y); dy[13] = c31 * (-2 * x * y); dz[13] = c31 * 8 * x * z;
        v[14] = c32b * z * (x * x - y * y);
        dx[14] = c32b * 2 * x * z; dy[14] = -c32b * 2 * y * z; dz[14] = c32b * (x * x - y * y);
        v[15] = c33 * x * (x * x - 3 * y * y);
        dx[15] = c33 * (3 * x * x - 3 * y * y); dy[15] = -c33 * 6 * x * y; dz[15] = 0.0f;
    }
}

// Y[lm] and dY/dX, dY/dY, dY/dZ ([3][NY] at grad) of the edge with unit
// direction d (unshuffled) and length r, in FP32.
template <int LMAX>
__device__ __forceinline__ void edge_harmonics(const float (&d)[3], float r, float* Y, float* grad) {
    constexpr int NY = (LMAX + 1) * (LMAX + 1);
    // (x, y, z) -> (z, x, y), renormalised in FP32
    float x = d[2], y = d[0], z = d[1];
    const float rr = x * x + y * y + z * z;
    const float inv = 1.0f / sqrtf(rr);
    x *= inv;
    y *= inv;
    z *= inv;
    float v[NY], dx[NY], dy[NY], dz[NY];
    real_harmonics<LMAX>(x, y, z, v, dx, dy, dz);
    const float scale = static_cast<float>(kSqrt4Pi) / r;
    for (int q = 0; q < NY; ++q) {
        if (Y) Y[q] = static_cast<float>(static_cast<double>(v[q]) * kSqrt4Pi);
        const float radial = dx[q] * x + dy[q] * y + dz[q] * z;
        const float gx = dx[q] - x * radial;
        const float gy = dy[q] - y * radial;
        const float gz = dz[q] - z * radial;
        // unshuffle: d/dX = d/dy', d/dY = d/dz', d/dZ = d/dx'
        grad[q] = scale * gy;
        grad[NY + q] = scale * gz;
        grad[2 * NY + q] = scale * gx;
    }
}

}  // namespace smx
