// Shared helpers of the HIP kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

namespace smx {

constexpr int kWave = 64;
// Edge ids are int32 (the reference's cardinality guard,
// mace_kokkos_runtime.cpp:199); the margin keeps strided int loops over edge
// ranges (stride <= 4096) from overflowing.
constexpr long long kMaxEdges = 2147483647LL - 4096;
constexpr int kXcds = 8;

inline void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}
#define SMX_HIP(call) ::smx::hip_check((call), #call)
#define SMX_LAUNCH_CHECK(name) ::smx::hip_check(hipGetLastError(), name)

// MI355X dispatches workgroups round-robin over its 8 XCDs, each with its own
// L2.  Remap so that XCD x processes one contiguous range of the logical
// index space: neighbouring receivers share neighbours, so their features stay
// in that XCD's L2.  The map is a bijection on [0, n).
__device__ __forceinline__ int xcd_remap(int b, int n) {
    const int q = n / kXcds, r = n % kXcds;
    const int x = b % kXcds, j = b / kXcds;
    return x * q + (x < r ? x : r) + j;
}

// Butterfly sum over the first `width` lanes of a wave (width a power of two
// <= 64); every participating lane ends with the total.
template <int WIDTH>
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = WIDTH / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, WIDTH);
    return v;
}

template <int WIDTH>
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int off = WIDTH / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, WIDTH);
    return v;
}

inline unsigned blocks_for(std::int64_t n, int per_block) {
    return static_cast<unsigned>((n + per_block - 1) / per_block);
}

}  // namespace smx
