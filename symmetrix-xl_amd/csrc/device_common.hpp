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
// The tiled plan indexes the graph's edges with 64 bits (each tile's kernels
// see 32-bit offsets relative to the tile's first edge); its bound keeps a
// one-thread-per-edge launch under the 2^32 work-items of a dispatch.
constexpr long long kMaxWideEdges = (1LL << 32) - (1LL << 20);
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

// v + v[lane permuted by the DPP control CTRL] on the rows in ROW_MASK
// (other rows add 0)
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
    const int moved = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false);
    return v + __int_as_float(moved);
}

// Sum over each row of 16 lanes with DPP (quad permutes, half-row and row
// mirrors); every lane of a row holds its row's sum.
__device__ __forceinline__ float row_total(float v) {
    v = dpp_add<0xb1, 0xf>(v);   // quad_perm [1,0,3,2]
    v = dpp_add<0x4e, 0xf>(v);   // quad_perm [2,3,0,1]
    v = dpp_add<0x141, 0xf>(v);  // row_half_mirror
    return dpp_add<0x140, 0xf>(v);  // row_mirror
}

// Sum over the first WIDTH (32 or 64) lanes of a wave with DPP row
// operations (quad permutes, half-row and row mirrors, then the row
// broadcasts 15 and 31), returned wave-uniform from the last lane.
template <int WIDTH>
__device__ __forceinline__ float wave_total(float v) {
    static_assert(WIDTH == 32 || WIDTH == 64, "DPP reduction over 32 or 64 lanes");
    v = dpp_add<0xb1, 0xf>(v);   // quad_perm [1,0,3,2]
    v = dpp_add<0x4e, 0xf>(v);   // quad_perm [2,3,0,1]
    v = dpp_add<0x141, 0xf>(v);  // row_half_mirror: sums of 8
    v = dpp_add<0x140, 0xf>(v);  // row_mirror: every lane of a row holds the row sum
    v = dpp_add<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
    if constexpr (WIDTH == 64) {
        v = dpp_add<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
        return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
    } else {
        return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
    }
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
