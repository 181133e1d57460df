// Compile-time structure of a MACE interaction for the kernels' template
// parameters: edge harmonics up to LMAX, node features up to LMAXH.
//
// The R1 ("uvu") paths are those of MACE's second-interaction tensor product
// as the reference's extractor lists them (extract_mace_data.py:1326-1400):
// source irreps outer, edge irreps next, output irreps in the target
// 0e+1o+...+LMAX with matching parity, then stably sorted by output l.  The
// rows (path, m_edge, m_source) and outputs lme = lme_base[l] + m*num_e[l] + e
// follow the same file's numbering.  The evaluator checks the model file's
// path lists against this table before it selects a kernel set.
#pragma once

#include <array>
#include <type_traits>
#include <utility>

namespace smx {

template <int B, int E, class F>
__host__ __device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(static_cast<F&&>(f));
    }
}

// f(integral_constant<B>), ..., f(integral_constant<E-1>) without recursion
// (long unrolled ranges such as product-basis term lists)
template <int B, class F, int... I>
__host__ __device__ __forceinline__ void static_range_impl(F& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, B + I>{}), ...);
}
template <int B, int E, class F>
__host__ __device__ __forceinline__ void static_range(F&& f) {
    if constexpr (B < E) static_range_impl<B>(f, std::make_integer_sequence<int, E - B>{});
}

struct R1Path {
    int le, ls, lo;
};

template <int LMAX, int LMAXH>
struct Shape {
    static constexpr int NY = (LMAX + 1) * (LMAX + 1);
    static constexpr int NH = (LMAXH + 1) * (LMAXH + 1);

    static constexpr bool allowed(int le, int ls, int lo) {
        const int a = ls > le ? ls - le : le - ls;
        return lo >= a && lo <= ls + le && lo <= LMAX && ((ls + le + lo) % 2 == 0);
    }
    static constexpr int count_paths() {
        int n = 0;
        for (int ls = 0; ls <= LMAXH; ++ls)
            for (int le = 0; le <= LMAX; ++le)
                for (int lo = 0; lo <= LMAX; ++lo)
                    if (allowed(le, ls, lo)) ++n;
        return n;
    }
    static constexpr int P = count_paths();
    static constexpr std::array<R1Path, P> make_paths() {
        std::array<R1Path, P> out{};
        int n = 0;
        for (int target = 0; target <= LMAX; ++target)
            for (int ls = 0; ls <= LMAXH; ++ls)
                for (int le = 0; le <= LMAX; ++le)
                    for (int lo = 0; lo <= LMAX; ++lo)
                        if (lo == target && allowed(le, ls, lo)) out[n++] = R1Path{le, ls, lo};
        return out;
    }
    static constexpr std::array<R1Path, P> paths = make_paths();

    static constexpr std::array<int, P + 1> make_row_base() {
        std::array<int, P + 1> b{};
        for (int p = 0; p < P; ++p) b[p + 1] = b[p] + (2 * paths[p].le + 1) * (2 * paths[p].ls + 1);
        return b;
    }
    static constexpr std::array<int, P + 1> row_base = make_row_base();
    static constexpr int NROWS = row_base[P];

    static constexpr std::array<int, P + 1> make_cg_offset() {
        std::array<int, P + 1> b{};
        for (int p = 0; p < P; ++p)
            b[p + 1] = b[p] + (2 * paths[p].le + 1) * (2 * paths[p].ls + 1) * (2 * paths[p].lo + 1);
        return b;
    }
    static constexpr std::array<int, P + 1> cg_offset = make_cg_offset();

    static constexpr std::array<int, LMAX + 1> make_num_e() {
        std::array<int, LMAX + 1> n{};
        for (int p = 0; p < P; ++p) n[paths[p].lo] += 1;
        return n;
    }
    static constexpr std::array<int, LMAX + 1> num_e = make_num_e();
    static constexpr std::array<int, LMAX + 2> make_lme_base() {
        std::array<int, LMAX + 2> b{};
        for (int l = 0; l <= LMAX; ++l) b[l + 1] = b[l] + (2 * l + 1) * num_e[l];
        return b;
    }
    static constexpr std::array<int, LMAX + 2> lme_base = make_lme_base();
    static constexpr int NLME = lme_base[LMAX + 1];
    static constexpr std::array<int, P> make_e_index() {
        std::array<int, P> e{};
        std::array<int, LMAX + 1> seen{};
        for (int p = 0; p < P; ++p) e[p] = seen[paths[p].lo]++;
        return e;
    }
    static constexpr std::array<int, P> e_index = make_e_index();

    // output index of (path p, output m)
    static constexpr int lme(int p, int mo) {
        return lme_base[paths[p].lo] + mo * num_e[paths[p].lo] + e_index[p];
    }

    // per-edge records in two arrays, each padded to whole float4s: the
    // forward part [x, interval, active, pad, Y[NY]] that the forward edge
    // kernels read, and the reverse part [dY/dx[NY], dY/dy[NY], dY/dz[NY],
    // u[3]] that only the reverse kernels add.  A reverse kernel stages a
    // record in LDS as the two parts back to back (REC floats), so the
    // offsets below index that concatenation.
    static constexpr int REC_F = (4 + NY + 3) / 4 * 4;
    static constexpr int REC_B = (3 * NY + 3 + 3) / 4 * 4;
    static constexpr int REC = REC_F + REC_B;
    static constexpr int REC_Y = 4;
    static constexpr int REC_DY = REC_F;
    static constexpr int REC_U = REC_F + 3 * NY;
};

}  // namespace smx
