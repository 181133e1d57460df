// CPU ORACLE — test infrastructure only.
//
// A C++/OpenMP restatement of the reference's MACE energy + forces + stress
// path, used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline as
// the checker of the HIP path.  It is never part of the product: the product
// library (symmetrix-xl_amd/csrc) neither links nor loads it.
//
// What it restates (file:line in the reference snapshot):
//   * periodic neighbour list, bit-exact (IEEE double, no FMA contraction):
//     libsymmetrix/source/neighbor_graph_kokkos.cpp:38-405
//   * prepared edge geometry with the cutoff clamp:
//     libsymmetrix/source/mace_kokkos_factorized_lifecycle.cpp:2915-3079
//   * compact radial tabulation: compact_radial.cpp:110-387 (features :227-267,
//     MLP :269-289 via multilayer_perceptron.cpp:30-80, spline derivatives
//     :326-366); Hermite coefficients and evaluation cubic_spline_set.cpp:8-96
//   * stage math of the streamed serial evaluator mace.cpp:232-319 and
//     :1356-2657 (A0 :1356-1403, reverse A0 :1486-1560, M0 :1639-1689,
//     H1 :1691-1757, v4 affine capture :1759-1814, Phi1 :2023-2084,
//     reverse Phi1 :2199-2303, A1 :2305-2379, M1 :2461-2514, H2 :2516-2620,
//     readouts :2622-2657; one-interaction models :255-281 with M1 over
//     the H1 components :2461-2514; MACEField field coupling :322-395,
//     1147-1240 with the path compilation of field_coupling.hpp:60-238 and
//     the Kokkos forms mace_kokkos_h1_phi1.cpp:846-1150), with the Kokkos evaluator's precision policy
//     (FP64 H2, readouts, node energies, directed forces, and the FP64
//     accumulation of the FP32 source adjoint: mace_kokkos.hpp:501,907-909,
//     1805-1828)
//   * polynomial semantics: multivariate_polynomial.cpp:11-103 (a repeated
//     monomial keeps its first coefficient)
//   * force and stress reductions: mace_kokkos_evaluate.cpp:49-128, 189-291
//   * ZBL pair repulsion (FP64): zbl_kokkos.cpp:11-160 (pair constants,
//     value and gradient with the polynomial envelope), applied per edge
//     before the model as mace_kokkos_evaluate.cpp:418-434 does
//     (node_energies += sum_j V, directed forces -= (xyz/r) dV/dr)
//   * density scaling of A0 and A1 as the Kokkos evaluator computes it (FP64
//     splines and sums): mace_kokkos_first_interaction.cpp:1335-1419
//     (A0 /= 1 + sum_j f0(r_ij)), :1421-1531 (reverse: edge forces
//     (dA0.A0)/s * f0'(r) r^, A0_adj /= s); mace_kokkos_second_interaction.cpp:
//     1310-1490 (A1 *= float(1/s)), :1493-1720 (reverse, A1_adj *= float(1/s));
//     tanh-square networks compact_radial.cpp:17-24,181-193,295-303; FP64
//     splines radial_function_set_kokkos.cpp:14-45, .hpp:48-146
//
// Y: the reference evaluates sphericart's real harmonics at the shuffled
// direction (z, x, y) and scales by sqrt(4 pi) rounding once from double
// (spherical_harmonic_device.hpp:15-199).  sphericart is not vendored, so the
// polynomials are written here from the real-harmonic closed forms; edges with
// r >= r_cut carry Y = 0 as in the direct plan (:201-223).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <map>
#include <memory>
#include <numeric>
#include <stdexcept>
#include <string>
#include <vector>

#include <omp.h>

#include "../symmetrix-xl_amd/csrc/json_lite.hpp"

namespace oracle {

using json_lite::Value;

thread_local std::string last_error;

// ---------------------------------------------------------------------------
// Compact radial model (compact_radial.cpp)
// ---------------------------------------------------------------------------

struct Network {
    std::vector<int> shape;
    std::vector<std::vector<double>> weights;  // [layer][out*in]
    double scale = 1.0;
    bool tanh_square = false;  // postprocess "tanh-square": tanh(v^2)
};

static Network parse_network(const Value& v) {
    Network n;
    n.shape = v.at("shape").as_ints();
    const Value& w = v.at("weights");
    for (std::size_t i = 0; i < w.size(); ++i) n.weights.push_back(w.at(i).as_doubles());
    n.scale = v.at("activation_scale").as_number();
    const std::string post = v.get_string("postprocess", "");
    if (!post.empty() && post != "tanh-square")
        throw std::invalid_argument("radial network has unsupported postprocessing");
    n.tanh_square = post == "tanh-square";
    if (v.at("activation").as_string() != "silu")
        throw std::invalid_argument("radial network must use SiLU");
    if (n.shape.size() < 2 || n.weights.size() != n.shape.size() - 1)
        throw std::invalid_argument("radial network has an invalid shape");
    for (std::size_t l = 0; l < n.weights.size(); ++l)
        if (n.weights[l].size() != static_cast<std::size_t>(n.shape[l]) * n.shape[l + 1])
            throw std::invalid_argument("radial network has invalid weights");
    return n;
}

// multilayer_perceptron.cpp:30-80: hidden layers scale*x*sigmoid(x), linear output.
static void mlp_forward(const Network& n, const double* in, double* out) {
    std::vector<double> cur(in, in + n.shape[0]);
    for (std::size_t l = 0; l < n.weights.size(); ++l) {
        const int ni = n.shape[l], no = n.shape[l + 1];
        std::vector<double> nxt(no, 0.0);
        for (int o = 0; o < no; ++o) {
            double s = 0.0;
            for (int i = 0; i < ni; ++i) s += n.weights[l][static_cast<std::size_t>(o) * ni + i] * cur[i];
            nxt[o] = s;
        }
        if (l + 1 < n.weights.size())
            for (int o = 0; o < no; ++o) nxt[o] = n.scale * nxt[o] / (1.0 + std::exp(-nxt[o]));
        cur.swap(nxt);
    }
    std::copy(cur.begin(), cur.end(), out);
}

struct RadialModel {
    double grid_min = 0, h = 0, r_max = 0, prefactor = 0;
    int points = 0, p = 0;
    std::vector<double> bessel;
    Network R0, R1, A0, A1;
    bool has_R1 = false, has_A0 = false, has_A1 = false;
    // Agnesi distance transform (compact_radial.cpp:144-163, 233-247)
    bool agnesi = false;
    double agnesi_a = 0, agnesi_q = 0, agnesi_p = 0;
    std::vector<double> covalent_radii;  // per model type

    void load(const Value& def, double r_cut) {
        grid_min = def.at("spline_grid_min").as_number();
        points = def.at("num_spline_points").as_int();
        if (!(grid_min > 0.0) || points < 4)
            throw std::invalid_argument("compact radial grid is invalid");
        h = (r_cut - grid_min) / (points - 1);
        const Value& basis = def.at("basis");
        if (basis.at("type").as_string() != "bessel")
            throw std::invalid_argument("only a Bessel basis is supported");
        bessel = basis.at("weights").as_doubles();
        prefactor = basis.at("prefactor").as_number();
        const Value& cut = def.at("cutoff");
        if (cut.at("type").as_string() != "polynomial")
            throw std::invalid_argument("only a polynomial cutoff is supported");
        r_max = cut.at("r_max").as_number();
        p = cut.at("p").as_int();
        if (std::abs(r_max - r_cut) > 1e-12)
            throw std::invalid_argument("compact radial cutoff does not match r_cut");
        const Value& tr = def.at("distance_transform");
        const std::string tt = tr.at("type").as_string();
        agnesi = tt == "agnesi";
        if (agnesi) {
            agnesi_a = tr.at("a").as_number();
            agnesi_q = tr.at("q").as_number();
            agnesi_p = tr.at("p").as_number();
            covalent_radii = tr.at("covalent_radii").as_doubles();
        } else if (tt != "none") {
            throw std::invalid_argument("unsupported distance transform");
        }
        const Value& nets = def.at("networks");
        R0 = parse_network(nets.at("R0"));
        if (nets.contains("R1")) { R1 = parse_network(nets.at("R1")); has_R1 = true; }
        if (R0.tanh_square || (has_R1 && R1.tanh_square))
            throw std::invalid_argument("R0/R1 networks cannot use postprocessing");
        // density networks: Bessel features in, one output, tanh-square
        auto density = [&](const char* name, Network& net, bool& has) {
            if (!nets.contains(name)) return;
            net = parse_network(nets.at(name));
            has = true;
            if (net.shape.front() != static_cast<int>(bessel.size()) || net.shape.back() != 1 || !net.tanh_square)
                throw std::invalid_argument(std::string("compact radial ") + name +
                                            " network has an invalid shape or postprocessing");
        };
        density("A0", A0, has_A0);
        density("A1", A1, has_A1);
    }

    // compact_radial.cpp:227-267: the features of the pair (ti, tj) (model
    // types); without a transform every pair has the same features
    std::vector<double> features(int ti = 0, int tj = 0) const {
        const std::size_t nb = bessel.size();
        std::vector<double> f(static_cast<std::size_t>(points) * nb);
        double r0 = 1.0;
        if (agnesi) {
            if (ti < 0 || tj < 0 || ti >= static_cast<int>(covalent_radii.size()) ||
                tj >= static_cast<int>(covalent_radii.size()))
                throw std::out_of_range("agnesi covalent radius index out of range");
            r0 = 0.5 * (covalent_radii[ti] + covalent_radii[tj]);
        }
        for (int node = 0; node < points; ++node) {
            const double r = grid_min + node * h;
            double x = r;
            if (agnesi) {
                const double s = r / r0;
                x = 1.0 / (1.0 + agnesi_a * std::pow(s, agnesi_q) / (1.0 + std::pow(s, agnesi_q - agnesi_p)));
            }
            double cutoff_value = 0.0;
            if (r < r_max) {
                const double s = r / r_max;
                cutoff_value = 1.0 - ((p + 1.0) * (p + 2.0) / 2.0) * std::pow(s, p)
                    + p * (p + 2.0) * std::pow(s, p + 1)
                    - (p * (p + 1.0) / 2.0) * std::pow(s, p + 2);
            }
            for (std::size_t b = 0; b < nb; ++b)
                f[node * nb + b] = prefactor * std::sin(bessel[b] * x) / x * cutoff_value;
        }
        return f;
    }

    // compact_radial.cpp:326-366: not-a-knot left, clamped (zero) right.
    std::vector<double> spline_derivatives(const std::vector<double>& v) const {
        const int n = points, unknowns = n - 2;
        std::vector<double> lower(unknowns, 0.0), diag(unknowns, 4.0), upper(unknowns, 0.0), rhs(unknowns, 0.0);
        const double left = 2.0 * (-v[0] + 2.0 * v[1] - v[2]) / h;
        upper[0] = 2.0;
        rhs[0] = 3.0 * (v[2] - v[0]) / h - left;
        for (int node = 2; node < n - 1; ++node) {
            const int row = node - 1;
            lower[row] = 1.0;
            if (node + 1 <= n - 2) upper[row] = 1.0;
            rhs[row] = 3.0 * (v[node + 1] - v[node - 1]) / h;
        }
        for (int row = 1; row < unknowns; ++row) {
            const double factor = lower[row] / diag[row - 1];
            diag[row] -= factor * upper[row - 1];
            rhs[row] -= factor * rhs[row - 1];
        }
        std::vector<double> sol(unknowns, 0.0);
        sol.back() = rhs.back() / diag.back();
        for (int row = unknowns - 2; row >= 0; --row)
            sol[row] = (rhs[row] - upper[row] * sol[row + 1]) / diag[row];
        std::vector<double> d(n, 0.0);
        for (int node = 1; node < n - 1; ++node) d[node] = sol[node - 1];
        d[0] = d[2] + left;
        d.back() = 0.0;
        return d;
    }

    // Nodal values and derivatives [function][node] of a network on the grid.
    void tabulate(const Network& net, std::vector<std::vector<double>>& values,
                  std::vector<std::vector<double>>& derivs, int ti = 0, int tj = 0) const {
        const auto f = features(ti, tj);
        const int nout = net.shape.back();
        values.assign(nout, std::vector<double>(points));
        std::vector<double> out(nout);
        for (int node = 0; node < points; ++node) {
            mlp_forward(net, f.data() + static_cast<std::size_t>(node) * bessel.size(), out.data());
            for (int o = 0; o < nout; ++o) values[o][node] = net.tanh_square ? std::tanh(out[o] * out[o]) : out[o];
        }
        derivs.resize(nout);
        for (int o = 0; o < nout; ++o) derivs[o] = spline_derivatives(values[o]);
    }
};

// ---------------------------------------------------------------------------
// ZBL pair repulsion (zbl_kokkos.cpp:11-160, FP64)
// ---------------------------------------------------------------------------
struct Zbl {
    static constexpr double kExp[4] = {-3.2, -0.9423, -0.4028, -0.2016};
    static constexpr double kPrefactor = 14.3996;
    double a_exp = 0, a_prefactor = 0;
    double c[4] = {0, 0, 0, 0};
    std::vector<double> radii;
    int p = 0;

    void init(double a_exp_, double a_prefactor_, const std::vector<double>& c_, const std::vector<double>& radii_,
              int p_) {
        if (c_.size() != 4) throw std::invalid_argument("ZBL requires four screening coefficients");
        if (radii_.empty()) throw std::invalid_argument("ZBL requires at least one covalent radius");
        if (!(a_prefactor_ > 0.0)) throw std::invalid_argument("ZBL screening prefactor must be positive");
        if (p_ < 1) throw std::invalid_argument("ZBL envelope power must be positive");
        a_exp = a_exp_;
        a_prefactor = a_prefactor_;
        for (int i = 0; i < 4; ++i) c[i] = c_[i];
        radii = radii_;
        p = p_;
    }
    // polynomial envelope and its derivative (zbl_kokkos.cpp:125-137)
    void envelope(double r, double r_max, double& v, double& g) const {
        if (r >= r_max) {
            v = g = 0.0;
            return;
        }
        const double c0 = (p + 1.0) * (p + 2.0) / 2.0, c1 = p * (p + 2.0), c2 = p * (p + 1.0) / 2.0;
        const double x = r / r_max;
        const double xm1 = std::pow(x, p - 1), xp = xm1 * x, xp1 = xp * x, xp2 = xp1 * x;
        v = 1.0 - c0 * xp + c1 * xp1 - c2 * xp2;
        g = (-c0 * p * xm1 + c1 * (p + 1.0) * xp - c2 * (p + 2.0) * xp1) / r_max;
    }
    // value and dV/dr of one directed edge (zbl_kokkos.cpp:92-139)
    void value_gradient(int Zu, int Zv, double r, double& value, double& gradient) const {
        if (Zu < 0 || Zv < 0 || Zu >= static_cast<int>(radii.size()) || Zv >= static_cast<int>(radii.size()))
            throw std::out_of_range("ZBL atomic number outside the covalent-radius table");
        const double inverse_a = (std::pow(static_cast<double>(Zu), a_exp) + std::pow(static_cast<double>(Zv), a_exp)) /
                                 (a_prefactor * 0.529);
        const double bare_prefactor = kPrefactor * static_cast<double>(Zu * Zv);
        const double r_max = radii[Zu] + radii[Zv];
        if (r >= r_max) {
            value = gradient = 0.0;
            return;
        }
        const double ra = r * inverse_a;
        double e[4];
        for (int i = 0; i < 4; ++i) e[i] = c[i] * std::exp(kExp[i] * ra);
        const double phi = e[0] + e[1] + e[2] + e[3];
        const double dphi = inverse_a * (kExp[0] * e[0] + kExp[1] * e[1] + kExp[2] * e[2] + kExp[3] * e[3]);
        const double inv_r = 1.0 / r;
        const double bare = bare_prefactor * inv_r * phi;
        const double bare_g = bare_prefactor * inv_r * inv_r * (r * dphi - phi);
        double env, env_g;
        envelope(r, r_max, env, env_g);
        value = 0.5 * bare * env;
        gradient = 0.5 * (bare * env_g + bare_g * env);
    }
};

// ---------------------------------------------------------------------------
// Cubic Hermite spline set (cubic_spline_set.cpp:8-96), arithmetic in P.
// ---------------------------------------------------------------------------

template <class P>
struct SplineSet {
    P h{}, x0{};
    int num_nodes = 0, num_splines = 0;
    std::vector<P> c;  // [interval][4][function]

    SplineSet(P h_, const std::vector<std::vector<P>>& v, const std::vector<std::vector<P>>& d, P x0_)
        : h(h_), x0(x0_) {
        num_nodes = static_cast<int>(v[0].size());
        num_splines = static_cast<int>(v.size());
        c.assign(static_cast<std::size_t>(4) * num_splines * (num_nodes - 1), P(0));
        for (int i = 0; i < num_nodes - 1; ++i)
            for (int j = 0; j < num_splines; ++j) {
                c[(4 * i) * num_splines + j] = v[j][i];
                c[(4 * i + 1) * num_splines + j] = d[j][i];
                c[(4 * i + 2) * num_splines + j] =
                    (-3 * v[j][i] - 2 * h * d[j][i] + 3 * v[j][i + 1] - h * d[j][i + 1]) / (h * h);
                c[(4 * i + 3) * num_splines + j] =
                    (2 * v[j][i] + h * d[j][i] - 2 * v[j][i + 1] + h * d[j][i + 1]) / (h * h * h);
            }
    }
    struct Point { int interval; P x, xx, xxx; };
    Point point(P r) const {
        int interval = static_cast<int>(std::floor((r - x0) / h));
        P x = r - x0 - h * interval;
        if (interval < 0) { interval = 0; x = 0; }
        else if (interval >= num_nodes - 1) { interval = num_nodes - 2; x = h; }
        const P xx = x * x;
        return {interval, x, xx, xx * x};
    }
    const P* coefficients(const Point& pt) const {
        return c.data() + static_cast<std::size_t>(4) * pt.interval * num_splines;
    }
};

// ---------------------------------------------------------------------------
// Real spherical harmonics l <= 3 (component normalisation), P precision.
// Values at unit vector (x,y,z) already shuffled; returns raw orthonormal values
// and the Cartesian gradients on the sphere before normalisation.
// ---------------------------------------------------------------------------

template <class P>
static void sph_raw(int l_max, P x, P y, P z, P* v, P* dx, P* dy, P* dz) {
    // constants of the orthonormal real harmonics
    const double pi = 3.14159265358979323846;
    const P c0 = P(0.5 / std::sqrt(pi));
    v[0] = c0; dx[0] = dy[0] = dz[0] = 0;
    if (l_max < 1) return;
    const P c1 = P(std::sqrt(3.0 / (4.0 * pi)));
    v[1] = c1 * y; dx[1] = 0; dy[1] = c1; dz[1] = 0;
    v[2] = c1 * z; dx[2] = 0; dy[2] = 0; dz[2] = c1;
    v[3] = c1 * x; dx[3] = c1; dy[3] = 0; dz[3] = 0;
    if (l_max < 2) return;
    const P c2 = P(0.5 * std::sqrt(15.0 / pi));
    const P c20 = P(0.25 * std::sqrt(5.0 / pi));
    const P c22 = P(0.25 * std::sqrt(15.0 / pi));
    v[4] = c2 * x * y; dx[4] = c2 * y; dy[4] = c2 * x; dz[4] = 0;
    v[5] = c2 * y * z; dx[5] = 0; dy[5] = c2 * z; dz[5] = c2 * y;
    v[6] = c20 * (2 * z * z - x * x - y * y); dx[6] = -2 * c20 * x; dy[6] = -2 * c20 * y; dz[6] = 4 * c20 * z;
    v[7] = c2 * x * z; dx[7] = c2 * z; dy[7] = 0; dz[7] = c2 * x;
    v[8] = c22 * (x * x - y * y); dx[8] = 2 * c22 * x; dy[8] = -2 * c22 * y; dz[8] = 0;
    if (l_max < 3) return;
    const P c33 = P(0.25 * std::sqrt(35.0 / (2.0 * pi)));
    const P c32 = P(0.5 * std::sqrt(105.0 / pi));
    const P c31 = P(0.25 * std::sqrt(21.0 / (2.0 * pi)));
    const P c30 = P(0.25 * std::sqrt(7.0 / pi));
    const P c32b = P(0.25 * std::sqrt(105.0 / pi));
    const P r2 = x * x + y * y;
    v[9] = c33 * y * (3 * x * x - y * y);
    dx[9] = c33 * 6 * x * y; dy[9] = c33 * (3 * x * x - 3 * y * y); dz[9] = 0;
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
    dx[15] = c33 * (3 * x * x - 3 * y * y); dy[15] = -c33 * 6 * x * y; dz[15] = 0;
}

static constexpr double kSqrt4Pi = 3.5449077018110318;

// Y and dY/dxyz of one edge from its unit direction (unshuffled) and radius,
// following spherical_harmonic_device.hpp:150-199 (value normalisation
// float(double(v)*sqrt(4 pi)); gradients (d - u (u.d))/r scaled by sqrt(4 pi)).
template <class P>
static void edge_harmonics(int l_max, const P dir[3], P radius, P* Y, P* G) {
    const int n = (l_max + 1) * (l_max + 1);
    P x = dir[2], y = dir[0], z = dir[1];
    const P rr = x * x + y * y + z * z;
    const P inv = P(1) / std::sqrt(rr);
    x *= inv; y *= inv; z *= inv;
    P v[16], dx[16], dy[16], dz[16];
    sph_raw<P>(l_max, x, y, z, v, dx, dy, dz);
    for (int i = 0; i < n; ++i) Y[i] = static_cast<P>(static_cast<double>(v[i]) * kSqrt4Pi);
    if (!G) return;
    const P scale = static_cast<P>(kSqrt4Pi) / radius;
    for (int i = 0; i < n; ++i) {
        const P radial = dx[i] * x + dy[i] * y + dz[i] * z;
        const P gx = (dx[i] - x * radial);
        const P gy = (dy[i] - y * radial);
        const P gz = (dz[i] - z * radial);
        // unshuffle: d/dX = d/dy', d/dY = d/dz', d/dZ = d/dx'
        G[i] = scale * gy;
        G[n + i] = scale * gz;
        G[2 * n + i] = scale * gx;
    }
}

// ---------------------------------------------------------------------------
// Multivariate polynomial (multivariate_polynomial.cpp:11-103): keep the first
// coefficient of a repeated monomial; f = sum c_t prod x; gradient by product
// rule.  Arithmetic in P.
// ---------------------------------------------------------------------------

struct MonomialSet {
    std::vector<std::vector<int>> monos;  // deduplicated, first occurrence
    std::vector<int> source_index;        // index into the file's coefficient list
};

static MonomialSet dedupe_monomials(const std::vector<std::vector<int>>& monos) {
    MonomialSet s;
    std::map<std::vector<int>, int> seen;
    for (std::size_t i = 0; i < monos.size(); ++i) {
        if (seen.count(monos[i])) continue;
        seen[monos[i]] = static_cast<int>(i);
        s.monos.push_back(monos[i]);
        s.source_index.push_back(static_cast<int>(i));
    }
    return s;
}

template <class P>
static P poly_eval_grad(const MonomialSet& ms, const P* coef, const P* x, P* g, int nvar) {
    P f = 0;
    if (g) for (int v = 0; v < nvar; ++v) g[v] = 0;
    for (std::size_t t = 0; t < ms.monos.size(); ++t) {
        const auto& m = ms.monos[t];
        P prod = 1;
        for (int v : m) prod *= x[v];
        f += coef[t] * prod;
        if (g) {
            for (std::size_t q = 0; q < m.size(); ++q) {
                P d = coef[t];
                for (std::size_t q2 = 0; q2 < m.size(); ++q2)
                    if (q2 != q) d *= x[m[q2]];
                g[m[q]] += d;
            }
        }
    }
    return f;
}

// The directional derivative along dx of the polynomial and of its gradient:
// returns sum_v g_v dx_v, with g the gradient and gd its derivative along dx
// (each factor of a term differentiated in turn, as poly_eval_grad does).
template <class P>
static P poly_tangent(const MonomialSet& ms, const P* coef, const P* x, const P* dx, P* g, P* gd, int nvar) {
    P fd = 0;
    for (int v = 0; v < nvar; ++v) g[v] = gd[v] = 0;
    for (std::size_t t = 0; t < ms.monos.size(); ++t) {
        const auto& m = ms.monos[t];
        for (std::size_t q = 0; q < m.size(); ++q) {
            P d = coef[t];
            for (std::size_t q2 = 0; q2 < m.size(); ++q2)
                if (q2 != q) d *= x[m[q2]];
            g[m[q]] += d;
            fd += d * dx[m[q]];
            P dd = 0;
            for (std::size_t q3 = 0; q3 < m.size(); ++q3) {
                if (q3 == q) continue;
                P e = coef[t];
                for (std::size_t q2 = 0; q2 < m.size(); ++q2)
                    if (q2 != q && q2 != q3) e *= x[m[q2]];
                dd += e * dx[m[q3]];
            }
            gd[m[q]] += dd;
        }
    }
    return fd;
}

// ---------------------------------------------------------------------------
// Model and evaluator
// ---------------------------------------------------------------------------

template <class P>
struct Mace {
    int num_elements = 0, C = 0, l_max = 0, L_max = 0, num_lm = 0, num_LM = 0;
    double r_cut = 0;
    std::vector<int> atomic_numbers;
    std::vector<double> atomic_energies;
    RadialModel radial;
    std::vector<P> H0;                      // [type][C]
    std::vector<std::vector<std::vector<P>>> A0_w;  // [type][l][C*C]
    std::vector<MonomialSet> M0_monos;      // [LM]
    std::vector<std::vector<P>> M0_coef;    // [type*num_LM + LM][k*T + t]
    std::vector<P> H1_w;                    // [l][C][C]
    // h1_affine_mode "pre_linear_up" (mace.cpp:1759-1810): the scalar input
    // of readout_1 and the H2 skip is x = M0[:,0,:] P0 (+ residual), and its
    // direct adjoint d enters M0_adj as P0 d
    bool pre_linear_up = false;
    std::vector<P> P0;                      // [C][C] [in][out], H1_product_weights l = 0
    // first_interaction_residual (mace.cpp:1843-1875, 2796-2826): H1 +=
    // fused[type] (the residual through linear_up), x += residual[type][lm 0]
    bool residual = false;
    // single_layer_readout (mace.cpp:255-281, 2461-2514, 2676-2679): one
    // interaction; M1 is taken of H1 (its num_LM components) instead of A1,
    // so there is no R1, Phi1 or A1, and the M1 adjoint is H1's adjoint
    bool single_layer = false;
    // MACEField (field_coupling.hpp:60-238; mace.cpp:322-395, 1147-1240):
    // with the split H1 weights, H1p = M0 P (+ residual b), then
    // H1f[lm_out] = H1p[lm_out] + sum over angular entries of
    // (coef E_c) H1p[lm_in] W_path, x = H1f[:,0,:], H1 = H1f U; the reverse
    // carries H1_adj U^T (+ x's adjoint on lm 0) back through the field
    // terms and accumulates dE/dE_c in FP64
    bool has_field = false;
    struct FieldEntry {
        int lm_in, comp, lm_out, path;
        P coef;
    };
    std::vector<FieldEntry> field_entries;
    std::vector<P> field_W;                  // [path][C][C] [in][out]
    std::vector<P> P_all, U_all;             // [l][C][C] H1_product / H1_linear_up weights
    std::vector<P> res_b;                    // [type][LM][C] the residual before linear_up
    std::vector<double> field_in;            // the evaluation's field: 3 (graph) or 3n (per node)
    std::vector<double> field_adj;           // dE/dE, shaped like field_in
    std::vector<P> H1_pre, H1_field;         // pre-field H1p and H1f (stages)
    std::vector<P> res_fused;               // [type][LM][C]
    std::vector<P> res_x;                   // [type][C]
    std::vector<int> Phi1_l, Phi1_l1, Phi1_l2, Phi1_lme, Phi1_row;
    std::vector<P> Phi1_cg;
    int num_rows = 0, num_lme = 0;
    std::vector<int> num_e;                 // paths per output l
    std::vector<int> lme_base;              // first lme of output l
    std::vector<std::vector<P>> A1_w;       // [l][e*C*C]
    MonomialSet M1_monos;
    std::vector<std::vector<P>> M1_coef;    // [type][k*T + t]
    std::vector<std::vector<double>> H2_T;  // [type][C*C] (float-rounded, used in FP64)
    std::vector<double> H2_M1;              // [C*C]
    std::vector<double> q;                  // readout_1 (FP64)
    int hidden = 16;
    std::vector<double> W1, W2;             // readout_2 (FP64)
    double readout_scale = 1.0;

    // active radial tables
    std::vector<int> active_types, type_to_active;
    std::vector<std::shared_ptr<SplineSet<P>>> spl0, spl1;
    // ZBL pair repulsion
    bool has_zbl = false;
    Zbl zbl;
    std::vector<double> zbl_energies, zbl_forces;  // per node, per edge [3]
    // density scaling: FP64 splines of the A0/A1 networks (one function)
    bool A0_scaled = false, A1_scaled = false;
    std::vector<std::shared_ptr<SplineSet<double>>> dens0, dens1;  // per active pair
    std::vector<double> A0_scale, A1_scale;  // per node: 1 + sum_j f(r_ij)

    // state of the last evaluation (exposed for stage-level debugging)
    std::vector<P> Y, Ygrad, A0, M0, M0_grad, H1, xaff, Phi1, A1, M1, M1_grad, A1_adj, dPhi1,
        H1_adj, M0_adj, A0_adj;
    std::vector<double> H2, H2_adj, direct;
    std::vector<double> node_energies, node_forces;
    std::vector<double> node_forces_r1;  // directed forces of the R1 reverse alone
    // layer-1 intermediates: Phi0 = sum_e R0 Y H0 before the A0 linear, its
    // adjoint (A0_adj through the transposed linear) and the directed forces
    // of the R0 reverse alone
    std::vector<P> Phi0, Phi0_adj;
    std::vector<double> node_forces_r0;
    // directed-force terms of the A0/A1 density scales
    std::vector<double> density_forces;

    static P cast(double v) {
        if (!std::isfinite(v) || std::abs(v) > static_cast<double>(std::numeric_limits<P>::max()))
            throw std::invalid_argument("model value outside the requested precision range");
        return static_cast<P>(v);
    }
    static std::vector<P> castv(const std::vector<double>& v) {
        std::vector<P> o(v.size());
        for (std::size_t i = 0; i < v.size(); ++i) o[i] = cast(v[i]);
        return o;
    }

    // prediction_heads.hpp:10-88: the selected head's payload (its atomic
    // energies, readouts and zbl_c) stands in for the top-level fields
    std::string selected_head;

    void load(const std::string& path, const std::string& head = "") {
        const Value j = json_lite::parse_file(path);
        const Value* payload = nullptr;
        if (const Value* ph = j.find("prediction_heads")) {
            selected_head = head.empty() ? ph->at("default").as_string() : head;
            payload = ph->at("parameters").find(selected_head);
            if (!payload) throw std::invalid_argument("prediction head '" + selected_head + "' is not in the model");
        } else {
            selected_head = j.get_string("head", "");
            if (!head.empty() && head != selected_head)
                throw std::invalid_argument("prediction head '" + head + "' is not in the model");
        }
        auto field = [&](const char* name) -> const Value& {
            if (payload && payload->contains(name)) return payload->at(name);
            return j.at(name);
        };
        if (j.get_int("symmetrix_format_version", 1) != 4)
            throw std::invalid_argument("only Symmetrix MACE format version 4 is supported");
        const std::string h1_mode = j.get_string("h1_affine_mode", "");
        if (h1_mode != "m0_composite" && h1_mode != "pre_linear_up")
            throw std::invalid_argument("h1_affine_mode must be 'm0_composite' or 'pre_linear_up'");
        pre_linear_up = h1_mode == "pre_linear_up";
        residual = j.get_bool("first_interaction_residual", false);
        single_layer = j.get_bool("single_layer_readout", false);
        has_field = j.get_bool("has_field_coupling", false);
        {
            const std::string mt = j.get_string("model_type", "MACE");
            if (mt != "MACE" && mt != "MACEField") throw std::invalid_argument("unsupported model_type");
        }
        // h1_affine_schema.hpp:230-236: field coupling needs the pre_linear_up basis
        if (has_field && !pre_linear_up)
            throw std::invalid_argument("a field-coupled model needs h1_affine_mode 'pre_linear_up'");
        // h1_affine_schema.hpp:227-237, mace.cpp:2676-2679
        if (j.get_int("num_interactions", 2) != (single_layer ? 1 : 2))
            throw std::invalid_argument("interaction count and single-layer readout metadata disagree");
        if (residual && !pre_linear_up && !single_layer)
            throw std::invalid_argument("a first-interaction residual needs h1_affine_mode 'pre_linear_up'");
        if (pre_linear_up && single_layer)
            throw std::invalid_argument("the pre_linear_up basis applies to two-interaction models only");
        if (j.get_string("radial_representation", "") != "compact")
            throw std::invalid_argument("only the compact radial representation is supported");
        num_elements = j.at("num_elements").as_int();
        C = j.at("num_channels").as_int();
        r_cut = j.at("r_cut").as_number();
        l_max = j.at("l_max").as_int();
        L_max = j.at("L_max").as_int();
        num_lm = (l_max + 1) * (l_max + 1);
        num_LM = (L_max + 1) * (L_max + 1);
        if (l_max > 3 || L_max > l_max) throw std::invalid_argument("l_max must be <= 3");
        atomic_numbers = j.at("atomic_numbers").as_ints();
        atomic_energies = field("atomic_energies").as_doubles();
        radial.load(j.at("compact_radial"), r_cut);
        // mace_kokkos_model.cpp:191-198
        has_zbl = j.at("has_zbl").as_bool();
        if (has_zbl)
            zbl.init(j.at("zbl_a_exp").as_number(), j.at("zbl_a_prefactor").as_number(), field("zbl_c").as_doubles(),
                     j.at("zbl_covalent_radii").as_doubles(), j.at("zbl_p").as_int());
        // mace_kokkos_model.cpp:200,215-216,1109,1122-1123
        A0_scaled = j.at("A0_scaled").as_bool();
        A1_scaled = j.get_bool("A1_scaled", false);
        if (A0_scaled != radial.has_A0) throw std::invalid_argument("compact radial A0 network does not match A0_scaled");
        if (A1_scaled != radial.has_A1) throw std::invalid_argument("compact radial A1 network does not match A1_scaled");
        if (radial.has_R1 == single_layer)
            throw std::invalid_argument("compact radial R1 network does not match the interaction count");
        if (single_layer && A1_scaled) throw std::invalid_argument("a one-interaction model has no A1 to scale");
        H0 = castv(j.at("H0_weights").as_doubles());
        const Value& a0 = j.at("A0_weights");
        A0_w.resize(num_elements);
        for (int t = 0; t < num_elements; ++t)
            for (int l = 0; l <= l_max; ++l) A0_w[t].push_back(castv(a0.at(t).at(l).as_doubles()));
        // M0
        const Value& m0m = j.at("M0_monomials");
        const Value& m0w = j.at("M0_weights");
        M0_monos.resize(num_LM);
        M0_coef.assign(static_cast<std::size_t>(num_elements) * num_LM, {});
        for (int LM = 0; LM < num_LM; ++LM) {
            const Value& ml = m0m.at(std::to_string(LM));
            std::vector<std::vector<int>> monos;
            for (std::size_t i = 0; i < ml.size(); ++i) monos.push_back(ml.at(i).as_ints());
            M0_monos[LM] = dedupe_monomials(monos);
            const int T = static_cast<int>(M0_monos[LM].monos.size());
            for (int t = 0; t < num_elements; ++t) {
                auto& dst = M0_coef[t * num_LM + LM];
                dst.resize(static_cast<std::size_t>(C) * T);
                const Value& wl = m0w.at(std::to_string(t)).at(std::to_string(LM));
                for (int k = 0; k < C; ++k) {
                    const auto cf = wl.at(std::to_string(k)).as_doubles();
                    if (cf.size() != monos.size()) throw std::invalid_argument("M0 coefficient count mismatch");
                    for (int s = 0; s < T; ++s) dst[k * T + s] = cast(cf[M0_monos[LM].source_index[s]]);
                }
            }
        }
        H1_w = castv(j.at("H1_weights").as_doubles());
        if (pre_linear_up) {
            const auto pw = castv(j.at("H1_product_weights").as_doubles());
            if (pw.size() != H1_w.size()) throw std::invalid_argument("H1_product_weights has the wrong size");
            P0.assign(pw.begin(), pw.begin() + static_cast<std::size_t>(C) * C);
        }
        if (has_field) load_field(j);
        if (residual) {
            // fused[a][lm][out] = sum_in residual[a][lm][in] U_l[in][out] in
            // Precision, in the reference's loop order (mace.cpp:2809-2822)
            const auto U = castv(j.at("H1_linear_up_weights").as_doubles());
            const auto b = castv(j.at("H1_first_residual_weights").as_doubles());
            res_b = b;
            const int LM = (L_max + 1) * (L_max + 1);
            if (U.size() != H1_w.size() || b.size() != static_cast<std::size_t>(num_elements) * LM * C)
                throw std::invalid_argument("residual weights have the wrong size");
            res_fused.assign(b.size(), P(0));
            res_x.assign(static_cast<std::size_t>(num_elements) * C, P(0));
            for (int a = 0; a < num_elements; ++a) {
                for (int l = 0; l <= L_max; ++l)
                    for (int m = 0; m < 2 * l + 1; ++m)
                        for (int out = 0; out < C; ++out)
                            for (int in = 0; in < C; ++in) {
                                const int lm = l * l + m;
                                res_fused[(static_cast<std::size_t>(a) * LM + lm) * C + out] +=
                                    b[(static_cast<std::size_t>(a) * LM + lm) * C + in] *
                                    U[(static_cast<std::size_t>(l) * C + in) * C + out];
                            }
                for (int k = 0; k < C; ++k) res_x[static_cast<std::size_t>(a) * C + k] =
                    b[static_cast<std::size_t>(a) * LM * C + k];
            }
        }
        if (!single_layer) {
            Phi1_l = j.at("Phi1_l").as_ints();
            Phi1_l1 = j.at("Phi1_l1").as_ints();
            Phi1_l2 = j.at("Phi1_l2").as_ints();
            Phi1_lme = j.at("Phi1_lme").as_ints();
            Phi1_row = j.at("Phi1_lelm1lm2").as_ints();
            Phi1_cg = castv(j.at("Phi1_clebsch_gordan").as_doubles());
        }
        num_lme = 0;
        for (int l : Phi1_l) num_lme += 2 * l + 1;
        num_rows = 0;
        for (std::size_t p = 0; p < Phi1_l.size(); ++p) num_rows += (2 * Phi1_l1[p] + 1) * (2 * Phi1_l2[p] + 1);
        num_e.assign(l_max + 1, 0);
        for (int l : Phi1_l) num_e[l] += 1;
        lme_base.assign(l_max + 2, 0);
        for (int l = 0; l <= l_max; ++l) lme_base[l + 1] = lme_base[l] + (2 * l + 1) * num_e[l];
        if (!single_layer) {
            const Value& a1 = j.at("A1_weights");
            for (int l = 0; l <= l_max; ++l) A1_w.push_back(castv(a1.at(l).as_doubles()));
        }
        // M1: variables are A1's num_lm components, or H1's num_LM ones
        const Value& m1m = j.at("M1_monomials");
        std::vector<std::vector<int>> monos1;
        const int m1_vars = single_layer ? num_LM : num_lm;
        for (std::size_t i = 0; i < m1m.size(); ++i) {
            monos1.push_back(m1m.at(i).as_ints());
            for (int v : monos1.back())
                if (v < 0 || v >= m1_vars) throw std::invalid_argument("M1 monomial variable out of range");
        }
        M1_monos = dedupe_monomials(monos1);
        const int T1 = static_cast<int>(M1_monos.monos.size());
        const Value& m1w = j.at("M1_weights");
        M1_coef.resize(num_elements);
        for (int t = 0; t < num_elements; ++t) {
            M1_coef[t].resize(static_cast<std::size_t>(C) * T1);
            for (int k = 0; k < C; ++k) {
                const auto cf = m1w.at(std::to_string(t)).at(std::to_string(k)).as_doubles();
                for (int s = 0; s < T1; ++s) M1_coef[t][k * T1 + s] = cast(cf[M1_monos.source_index[s]]);
            }
        }
        // H2 and readouts: the OpenMP backend keeps H2 weights in Precision and
        // accumulates H2 in FP64 (mace_kokkos.hpp:1805-1816).
        const Value& t2 = j.at(pre_linear_up ? "H2_weights_for_H1_pre_linear_up" : "H2_weights_for_M0");
        for (int t = 0; t < num_elements; ++t) {
            const auto w = t2.at(t).as_doubles();
            std::vector<double> r(w.size());
            for (std::size_t i = 0; i < w.size(); ++i) r[i] = static_cast<double>(cast(w[i]));
            H2_T.push_back(r);
        }
        {
            const auto w = j.at("H2_weights_for_M1").as_doubles();
            H2_M1.resize(w.size());
            for (std::size_t i = 0; i < w.size(); ++i) H2_M1[i] = static_cast<double>(cast(w[i]));
        }
        q = field(pre_linear_up ? "readout_1_weights_for_H1_pre_linear_up" : "readout_1_weights_for_M0").as_doubles();
        hidden = j.get_int("readout_2_hidden_size", 16);
        W1 = field("readout_2_weights_1").as_doubles();
        W2 = field("readout_2_weights_2").as_doubles();
        readout_scale = j.at("readout_2_scale_factor").as_number();
        if (W1.size() != static_cast<std::size_t>(hidden) * C || W2.size() != static_cast<std::size_t>(hidden))
            throw std::invalid_argument("readout weights do not match the hidden size");
        type_to_active.assign(num_elements, -1);
    }

    P field_value(int i, int c) const {
        return static_cast<P>(field_in[field_in.size() == 3 ? c : 3 * static_cast<std::size_t>(i) + c]);
    }

    // H1p = M0 P (+ b), H1f = H1p + field terms, x = H1f[:,0,:], H1 = H1f U
    // (mace.cpp:1759-1783, 1845-1895; the field terms in the Kokkos order,
    // mace_kokkos_h1_phi1.cpp:895-919: per output, the entry's coef E_c
    // times each input's product in turn)
    void field_forward(int n, const int* types) {
        const std::size_t Cs = static_cast<std::size_t>(C), LMC = static_cast<std::size_t>(num_LM) * Cs;
        if (field_in.size() != 3 && field_in.size() != 3 * static_cast<std::size_t>(n))
            throw std::invalid_argument("MACEField electric_field must have shape (3,) or (num_nodes, 3)");
        H1_pre.assign(n * LMC, P(0));
        H1_field.assign(n * LMC, P(0));
        H1.assign(n * LMC, P(0));
#pragma omp parallel for schedule(static)
        for (int i = 0; i < n; ++i) {
            P* hp = &H1_pre[i * LMC];
            P* hf = &H1_field[i * LMC];
            for (int l = 0; l <= L_max; ++l)
                for (int m = 0; m < 2 * l + 1; ++m) {
                    const P* src = &M0[i * LMC + (l * l + m) * Cs];
                    P* dst = hp + (l * l + m) * Cs;
                    const P* W = &P_all[static_cast<std::size_t>(l) * Cs * Cs];
                    for (int kp = 0; kp < C; ++kp)
                        for (int k = 0; k < C; ++k) dst[k] += src[kp] * W[kp * Cs + k];
                }
            if (residual)
                for (std::size_t v = 0; v < LMC; ++v) hp[v] += res_b[static_cast<std::size_t>(types[i]) * LMC + v];
            for (int lo = 0; lo < num_LM; ++lo)
                for (int out = 0; out < C; ++out) {
                    P value = hp[lo * Cs + out];
                    for (const auto& e : field_entries) {
                        if (e.lm_out != lo) continue;
                        const P af = e.coef * field_value(i, e.comp);
                        const P* W = &field_W[static_cast<std::size_t>(e.path) * Cs * Cs];
                        for (int in = 0; in < C; ++in) value += af * hp[e.lm_in * Cs + in] * W[in * Cs + out];
                    }
                    hf[lo * Cs + out] = value;
                }
            for (int k = 0; k < C; ++k) xaff[i * Cs + k] = hf[k];
            for (int l = 0; l <= L_max; ++l)
                for (int m = 0; m < 2 * l + 1; ++m) {
                    const P* src = hf + (l * l + m) * Cs;
                    P* dst = &H1[i * LMC + (l * l + m) * Cs];
                    const P* W = &U_all[static_cast<std::size_t>(l) * Cs * Cs];
                    for (int kp = 0; kp < C; ++kp)
                        for (int k = 0; k < C; ++k) dst[k] += src[kp] * W[kp * Cs + k];
                }
        }
    }

    // H1p_adj = H1_adj U^T (+ x's adjoint on lm 0), then back through the
    // field terms (mace_kokkos_h1_phi1.cpp:928-1150: per input, each entry's
    // coef times W applied to the output adjoint; dE/dE_c summed in FP64),
    // then M0_adj = H1p_adj P^T
    void field_reverse(int n) {
        const std::size_t Cs = static_cast<std::size_t>(C), LMC = static_cast<std::size_t>(num_LM) * Cs;
        const bool global = field_in.size() == 3;
        field_adj.assign(field_in.size(), 0.0);
        std::vector<double> part(static_cast<std::size_t>(n) * 3, 0.0);
#pragma omp parallel for schedule(static)
        for (int i = 0; i < n; ++i) {
            std::vector<P> a(LMC, P(0)), a2(LMC);
            for (int l = 0; l <= L_max; ++l)
                for (int m = 0; m < 2 * l + 1; ++m) {
                    const P* src = &H1_adj[i * LMC + (l * l + m) * Cs];
                    P* dst = &a[(l * l + m) * Cs];
                    const P* W = &U_all[static_cast<std::size_t>(l) * Cs * Cs];
                    for (int k = 0; k < C; ++k) {
                        P acc = 0;
                        for (int kp = 0; kp < C; ++kp) acc += src[kp] * W[k * Cs + kp];
                        dst[k] = acc;
                    }
                }
            for (int k = 0; k < C; ++k) a[k] += static_cast<P>(direct[i * Cs + k]);
            const P* hp = &H1_pre[i * LMC];
            for (int li = 0; li < num_LM; ++li)
                for (int in = 0; in < C; ++in) {
                    P value = a[li * Cs + in];
                    for (const auto& e : field_entries) {
                        if (e.lm_in != li) continue;
                        const P* W = &field_W[static_cast<std::size_t>(e.path) * Cs * Cs + in * Cs];
                        if (global) {
                            P tr = 0;
                            for (int out = 0; out < C; ++out) tr += W[out] * a[e.lm_out * Cs + out];
                            const P contribution = e.coef * tr;
                            value += field_value(i, e.comp) * contribution;
                            part[3 * static_cast<std::size_t>(i) + e.comp] +=
                                static_cast<double>(hp[li * Cs + in] * contribution);
                        } else {
                            const P af = e.coef * field_value(i, e.comp);
                            for (int out = 0; out < C; ++out) value += af * W[out] * a[e.lm_out * Cs + out];
                            for (int out = 0; out < C; ++out)
                                part[3 * static_cast<std::size_t>(i) + e.comp] +=
                                    static_cast<double>(e.coef * W[out] * hp[li * Cs + in] * a[e.lm_out * Cs + out]);
                        }
                    }
                    a2[li * Cs + in] = value;
                }
            for (int l = 0; l <= L_max; ++l)
                for (int m = 0; m < 2 * l + 1; ++m) {
                    const P* src = &a2[(l * l + m) * Cs];
                    P* dst = &M0_adj[i * LMC + (l * l + m) * Cs];
                    const P* W = &P_all[static_cast<std::size_t>(l) * Cs * Cs];
                    for (int k = 0; k < C; ++k) {
                        P acc = 0;
                        for (int kp = 0; kp < C; ++kp) acc += src[kp] * W[k * Cs + kp];
                        dst[k] = acc;
                    }
                }
        }
        for (int i = 0; i < n; ++i)
            for (int c = 0; c < 3; ++c) field_adj[global ? c : 3 * static_cast<std::size_t>(i) + c] += part[3 * i + c];
    }

    // ---- MACEField response (mace_kokkos_response.tpp:136-2343 with the
    // reducer of mace_kokkos_response.cpp:49-140): for each field component s,
    // the tangent d/dE_s of the last evaluation, forward and reverse.  The
    // field enters H1f linearly, so H1f_dot = sum over the entries of
    // component s of coef H1p[lm_in] W; the tangent then runs through R1, A1
    // (and its density scale), M1 (the polynomial's gradient and its
    // derivative), H2 and the readout MLP (FP64, with act''), their reverses,
    // the R1 reverse (bilinear in H1 and dPhi1: both tangents), and the field
    // terms' reverse, where the Hessian column s is collected:
    //   field_hessian[c*3 + s] = sum_i sum_entries(c) coef H1p[lm_in] W . H1f_adj_dot[lm_out]
    // With forces, the layer-1 reverse carries H1p_adj_dot to the directed
    // forces' tangent field_force_derivative[s][e][3] (M0, A0 and the R0
    // path depend on the field only through the adjoint).  Needs the state
    // of evaluate() on the same inputs and one field for the graph.
    std::vector<double> field_hessian, field_force_derivative;
    // terms of the tangent left out, for the tests that show each is needed:
    // 1 the M1 gradient's tangent, 2 act'', 4 the (dPhi1, H1_dot) half of the
    // R1 reverse, 8 its (dPhi1_dot, H1) half, 16 the seed's own field term in
    // the field reverse, 32 the density scales' tangents
    int response_drop = 0;

    void field_response(int n, const int* types, const int* num_neigh, const int* neigh, const int* neigh_types,
                        const double* xyz, const double* r, bool with_forces) {
        if (!has_field) throw std::invalid_argument("the MACEField response needs a field-coupled model");
        if (single_layer) throw std::invalid_argument("the MACEField response runs two-interaction models");
        if (field_in.size() != 3)
            throw std::invalid_argument("the MACEField response needs one electric field for the graph (3 values)");
        std::vector<long long> off(n + 1, 0);
        for (int i = 0; i < n; ++i) off[i + 1] = off[i] + num_neigh[i];
        const long long E = off[n];
        const int nY = num_lm;
        const std::size_t Cs = static_cast<std::size_t>(C), LMC = static_cast<std::size_t>(num_LM) * Cs;
        const std::size_t YC = static_cast<std::size_t>(nY) * Cs, LMEC = static_cast<std::size_t>(num_lme) * Cs;
        const int np = static_cast<int>(Phi1_l.size());
        std::vector<int> row_base(np);
        for (int p = 0; p < np; ++p) row_base[p] = row_base_of_path(p);
        std::vector<int> recv(E);
        for (int i = 0; i < n; ++i)
            for (long long e = off[i]; e < off[i + 1]; ++e) recv[e] = i;
        std::vector<char> active(E);
        std::vector<P> dirs(3 * static_cast<std::size_t>(E), P(0));
        for (long long e = 0; e < E; ++e) {
            active[e] = r[e] < r_cut;
            if (active[e])
                for (int c = 0; c < 3; ++c) dirs[3 * e + c] = static_cast<P>(xyz[3 * e + c] / r[e]);
        }
        std::vector<long long> soff(n + 1, 0);
        for (long long e = 0; e < E; ++e) soff[neigh[e] + 1] += 1;
        for (int s = 0; s < n; ++s) soff[s + 1] += soff[s];
        std::vector<long long> sedges(E), cursor(soff.begin(), soff.end() - 1);
        for (long long e = 0; e < E; ++e) sedges[cursor[neigh[e]]++] = e;
        auto lin_fwd = [&](const P* src, const P* W, P* dst) {  // dst[k] = sum_kp src[kp] W[kp][k]
            for (int k = 0; k < C; ++k) dst[k] = 0;
            for (int kp = 0; kp < C; ++kp)
                for (int k = 0; k < C; ++k) dst[k] += src[kp] * W[kp * Cs + k];
        };
        auto lin_rev = [&](const P* src, const P* W, P* dst) {  // dst[k] = sum_kp src[kp] W[k][kp]
            for (int k = 0; k < C; ++k) {
                P acc = 0;
                for (int kp = 0; kp < C; ++kp) acc += src[kp] * W[k * Cs + kp];
                dst[k] = acc;
            }
        };
        auto radial1 = [&](long long e, P* rad, P* drad) {
            const auto& sp = *spl1[pair_index(types[recv[e]], neigh_types[e])];
            const auto pt = sp.point(static_cast<P>(r[e]));
            const P* cf = sp.coefficients(pt);
            const int ns = sp.num_splines;
            for (int f = 0; f < ns; ++f) {
                rad[f] = cf[f] + cf[ns + f] * pt.x + cf[2 * ns + f] * pt.xx + cf[3 * ns + f] * pt.xxx;
                drad[f] = cf[ns + f] + P(2.0) * cf[2 * ns + f] * pt.x + P(3.0) * cf[3 * ns + f] * pt.xx;
            }
        };
        // seed-independent: the primal rows of dPhi1 (CG) and H1f_adj = H1_adj U^T (+ direct on lm 0)
        std::vector<P> rows(static_cast<std::size_t>(n) * num_rows * Cs, P(0)), H1f_adj(n * LMC, P(0));
        std::vector<double> M1_adj(n * Cs, 0.0);
#pragma omp parallel for schedule(static)
        for (int i = 0; i < n; ++i) {
            P* rw = &rows[static_cast<std::size_t>(i) * num_rows * Cs];
            for (std::size_t t = 0; t < Phi1_cg.size(); ++t)
                for (int k = 0; k < C; ++k) rw[Phi1_row[t] * Cs + k] += Phi1_cg[t] * dPhi1[i * LMEC + Phi1_lme[t] * Cs + k];
            for (int l = 0; l <= L_max; ++l)
                for (int m = 0; m < 2 * l + 1; ++m)
                    lin_rev(&H1_adj[i * LMC + (l * l + m) * Cs], &U_all[static_cast<std::size_t>(l) * Cs * Cs],
                            &H1f_adj[i * LMC + (l * l + m) * Cs]);
            for (int k = 0; k < C; ++k) H1f_adj[i * LMC + k] += static_cast<P>(direct[i * Cs + k]);
            for (int in = 0; in < C; ++in) {
                double s1 = 0.0;
                for (int o = 0; o < C; ++o) s1 += H2_M1[in * Cs + o] * H2_adj[i * Cs + o];
                M1_adj[i * Cs + in] = s1;
            }
        }
        field_hessian.assign(9, 0.0);
        field_force_derivative.assign(with_forces ? 9 * static_cast<std::size_t>(E) : 0, 0.0);
        const int T1 = static_cast<int>(M1_monos.monos.size());
        for (int seed = 0; seed < 3; ++seed) {
            // 1. H1f_dot, x_dot = H1f_dot[:,0,:], H1_dot = H1f_dot U
            std::vector<P> H1f_dot(n * LMC, P(0)), H1_dot(n * LMC, P(0));
#pragma omp parallel for schedule(static)
            for (int i = 0; i < n; ++i) {
                const P* hp = &H1_pre[i * LMC];
                P* hd = &H1f_dot[i * LMC];
                for (const auto& en : field_entries) {
                    if (en.comp != seed) continue;
                    const P* W = &field_W[static_cast<std::size_t>(en.path) * Cs * Cs];
                    for (int out = 0; out < C; ++out) {
                        P z = 0;
                        for (int in = 0; in < C; ++in) z += hp[en.lm_in * Cs + in] * W[in * Cs + out];
                        hd[en.lm_out * Cs + out] += en.coef * z;
                    }
                }
                for (int l = 0; l <= L_max; ++l)
                    for (int m = 0; m < 2 * l + 1; ++m)
                        lin_fwd(hd + (l * l + m) * Cs, &U_all[static_cast<std::size_t>(l) * Cs * Cs],
                                &H1_dot[i * LMC + (l * l + m) * Cs]);
            }
            // 2-3. Phi1_dot (the R1 forward of H1_dot), A1_dot (scaled like A1)
            std::vector<P> A1_dot(n * YC, P(0));
#pragma omp parallel for schedule(dynamic, 16)
            for (int i = 0; i < n; ++i) {
                std::vector<P> rw(static_cast<std::size_t>(num_rows) * Cs, P(0)), rad(np * Cs), drad(np * Cs);
                std::vector<P> phi(LMEC, P(0));
                for (long long e = off[i]; e < off[i + 1]; ++e) {
                    if (!active[e]) continue;
                    radial1(e, rad.data(), drad.data());
                    const P* Hj = &H1_dot[static_cast<std::size_t>(neigh[e]) * LMC];
                    for (int p = 0; p < np; ++p) {
                        const int l1 = Phi1_l1[p], l2 = Phi1_l2[p];
                        int row = row_base[p];
                        for (int lm1 = l1 * l1; lm1 <= l1 * (l1 + 2); ++lm1)
                            for (int lm2 = l2 * l2; lm2 <= l2 * (l2 + 2); ++lm2) {
                                const P y = Y[e * nY + lm1];
                                for (int k = 0; k < C; ++k) rw[row * Cs + k] += rad[p * Cs + k] * y * Hj[lm2 * Cs + k];
                                ++row;
                            }
                    }
                }
                for (std::size_t t = 0; t < Phi1_cg.size(); ++t)
                    for (int k = 0; k < C; ++k) phi[Phi1_lme[t] * Cs + k] += Phi1_cg[t] * rw[Phi1_row[t] * Cs + k];
                P* ad = &A1_dot[i * YC];
                for (int l = 0; l <= l_max; ++l) {
                    const int ne = num_e[l];
                    const P* W = A1_w[l].data();
                    for (int m = 0; m < 2 * l + 1; ++m)
                        for (int e2 = 0; e2 < ne; ++e2) {
                            const P* src = &phi[(lme_base[l] + m * ne + e2) * Cs];
                            for (int kp = 0; kp < C; ++kp)
                                for (int k = 0; k < C; ++k)
                                    ad[(l * l + m) * Cs + k] += src[kp] * W[(static_cast<std::size_t>(e2) * Cs + kp) * Cs + k];
                        }
                }
                if (A1_scaled) {
                    const P inv = static_cast<P>(1.0 / A1_scale[i]);
                    for (std::size_t v = 0; v < YC; ++v) ad[v] *= inv;
                }
            }
            // 4-7. M1 tangent, readout tangents (FP64), A1 adjoint tangent
            // (and its density scale), dPhi1_dot
            std::vector<P> dPhi1_dot(n * LMEC, P(0));
            std::vector<double> direct_dot(n * Cs, 0.0);
            std::vector<double> fdot(with_forces ? 3 * static_cast<std::size_t>(E) : 0, 0.0);
            std::vector<double> dens_dot1(n, 0.0);
#pragma omp parallel for schedule(static)
            for (int i = 0; i < n; ++i) {
                const int t = types[i];
                std::vector<P> g(YC), gd(YC), M1_dot(Cs);
                P x[16], dx[16], gv[16], gdv[16];
                for (int k = 0; k < C; ++k) {
                    for (int v = 0; v < nY; ++v) {
                        x[v] = A1[i * YC + v * Cs + k];
                        dx[v] = A1_dot[i * YC + v * Cs + k];
                    }
                    M1_dot[k] = poly_tangent<P>(M1_monos, M1_coef[t].data() + static_cast<std::size_t>(k) * T1, x, dx, gv,
                                                gdv, nY);
                    for (int v = 0; v < nY; ++v) {
                        g[v * Cs + k] = gv[v];
                        gd[v * Cs + k] = gdv[v];
                    }
                }
                const double* h2 = &H2[i * Cs];
                std::vector<double> h2d(Cs), zd(hidden), h2ad(Cs);
                for (int o = 0; o < C; ++o) {
                    double s = 0.0;
                    for (int in = 0; in < C; ++in)
                        s += H2_T[t][in * Cs + o] * static_cast<double>(H1f_dot[i * LMC + in]);
                    for (int in = 0; in < C; ++in) s += H2_M1[in * Cs + o] * static_cast<double>(M1_dot[in]);
                    h2d[o] = s;
                }
                std::vector<double> dd(hidden);
                for (int hdn = 0; hdn < hidden; ++hdn) {
                    double z = 0.0, zt = 0.0;
                    for (int k = 0; k < C; ++k) {
                        z += W1[hdn * Cs + k] * h2[k];
                        zt += W1[hdn * Cs + k] * h2d[k];
                    }
                    const double sg = 1.0 / (1.0 + std::exp(-z));
                    // d/dz of scale (sg + z sg (1 - sg))
                    const double act2 = readout_scale * sg * (1.0 - sg) * (2.0 + z * (1.0 - 2.0 * sg));
                    dd[hdn] = (response_drop & 2) ? 0.0 : W2[hdn] * act2 * zt;
                }
                for (int k = 0; k < C; ++k) {
                    double s = 0.0;
                    for (int hdn = 0; hdn < hidden; ++hdn) s += dd[hdn] * W1[hdn * Cs + k];
                    h2ad[k] = s;
                }
                std::vector<P> a1s_adj_dot(YC), a1s_adj(YC);
                for (int in = 0; in < C; ++in) {
                    double sd = 0.0, s1 = 0.0;
                    for (int o = 0; o < C; ++o) {
                        sd += H2_T[t][in * Cs + o] * h2ad[o];
                        s1 += H2_M1[in * Cs + o] * h2ad[o];
                    }
                    direct_dot[i * Cs + in] = sd;
                    const P m1adj_dot = static_cast<P>(s1), m1adj = static_cast<P>(M1_adj[i * Cs + in]);
                    for (int v = 0; v < nY; ++v) {
                        a1s_adj_dot[v * Cs + in] =
                            g[v * Cs + in] * m1adj_dot + ((response_drop & 1) ? P(0) : gd[v * Cs + in] * m1adj);
                        a1s_adj[v * Cs + in] = g[v * Cs + in] * m1adj;
                    }
                }
                if (A1_scaled && !(response_drop & 32)) {
                    // dot = sum A1_adj A1 in the scaled basis: its tangent
                    const P* a = &A1[i * YC];
                    const P* ad = &A1_dot[i * YC];
                    double dot = 0.0;
                    for (std::size_t v = 0; v < YC; ++v)
                        dot += static_cast<double>(a1s_adj_dot[v] * a[v]) + static_cast<double>(a1s_adj[v] * ad[v]);
                    dens_dot1[i] = dot;
                }
                if (A1_scaled) {
                    const P inv = static_cast<P>(1.0 / A1_scale[i]);
                    for (std::size_t v = 0; v < YC; ++v) a1s_adj_dot[v] *= inv;
                }
                for (int l = 0; l <= l_max; ++l) {
                    const int ne = num_e[l];
                    const P* W = A1_w[l].data();
                    for (int m = 0; m < 2 * l + 1; ++m)
                        for (int e2 = 0; e2 < ne; ++e2) {
                            P* dst = &dPhi1_dot[i * LMEC + (lme_base[l] + m * ne + e2) * Cs];
                            for (int k = 0; k < C; ++k) {
                                const P* wr = W + (static_cast<std::size_t>(e2) * Cs + k) * Cs;
                                P s = 0;
                                for (int kp = 0; kp < C; ++kp) s += a1s_adj_dot[(l * l + m) * Cs + kp] * wr[kp];
                                dst[k] = s;
                            }
                        }
                }
            }
            if (with_forces && A1_scaled)
                for (int i = 0; i < n; ++i)
                    for (long long e = off[i]; e < off[i + 1]; ++e) {
                        double f, d;
                        density_eval(*dens1[pair_index(types[i], neigh_types[e])], r[e], f, d);
                        const double scale = dens_dot1[i] / A1_scale[i] * d;
                        for (int c = 0; c < 3; ++c) fdot[3 * e + c] += scale * (xyz[3 * e + c] / r[e]);
                    }
            // 8. the R1 reverse's tangents: edge forces from (dPhi1_dot, H1)
            // and (dPhi1, H1_dot); H1_adj_dot from dPhi1_dot over the transpose
            std::vector<P> rows_dot(static_cast<std::size_t>(n) * num_rows * Cs, P(0));
#pragma omp parallel for schedule(static)
            for (int i = 0; i < n; ++i) {
                P* rw = &rows_dot[static_cast<std::size_t>(i) * num_rows * Cs];
                for (std::size_t t = 0; t < Phi1_cg.size(); ++t)
                    for (int k = 0; k < C; ++k)
                        rw[Phi1_row[t] * Cs + k] += Phi1_cg[t] * dPhi1_dot[i * LMEC + Phi1_lme[t] * Cs + k];
            }
            if (with_forces) {
#pragma omp parallel
                {
                std::vector<P> rad(np * Cs), drad(np * Cs);
#pragma omp for schedule(dynamic, 64)
                for (long long e = 0; e < E; ++e) {
                    if (!active[e]) continue;
                    const int i = recv[e];
                    radial1(e, rad.data(), drad.data());
                    const P* ra = &rows[static_cast<std::size_t>(i) * num_rows * Cs];
                    const P* rd = &rows_dot[static_cast<std::size_t>(i) * num_rows * Cs];
                    const P* Hj = &H1[static_cast<std::size_t>(neigh[e]) * LMC];
                    const P* Hd = &H1_dot[static_cast<std::size_t>(neigh[e]) * LMC];
                    const P* y = &Y[e * nY];
                    const P* gy = &Ygrad[e * 3 * nY];
                    double f[3] = {0, 0, 0};
                    for (int p = 0; p < np; ++p) {
                        const int l1 = Phi1_l1[p], l2 = Phi1_l2[p];
                        int row = row_base[p];
                        for (int lm1 = l1 * l1; lm1 <= l1 * (l1 + 2); ++lm1)
                            for (int lm2 = l2 * l2; lm2 <= l2 * (l2 + 2); ++lm2) {
                                P radial_sum = 0, angular_sum = 0;
                                for (int k = 0; k < C; ++k) {
                                    const P b = ((response_drop & 8) ? P(0) : rd[row * Cs + k] * Hj[lm2 * Cs + k]) +
                                                ((response_drop & 4) ? P(0) : ra[row * Cs + k] * Hd[lm2 * Cs + k]);
                                    radial_sum += b * drad[p * Cs + k];
                                    angular_sum += b * rad[p * Cs + k];
                                }
                                for (int c = 0; c < 3; ++c)
                                    f[c] -= static_cast<double>(dirs[3 * e + c] * radial_sum * y[lm1] +
                                                                angular_sum * gy[c * nY + lm1]);
                                ++row;
                            }
                    }
                    for (int c = 0; c < 3; ++c) fdot[3 * e + c] += f[c];
                }
                }
            }
            std::vector<P> H1_adj_dot(n * LMC, P(0));
#pragma omp parallel for schedule(dynamic, 16)
            for (int s = 0; s < n; ++s) {
                std::vector<double> acc(LMC, 0.0);
                std::vector<P> rad(np * Cs), drad(np * Cs);
                for (long long q2 = soff[s]; q2 < soff[s + 1]; ++q2) {
                    const long long e = sedges[q2];
                    if (!active[e]) continue;
                    radial1(e, rad.data(), drad.data());
                    const P* rd = &rows_dot[static_cast<std::size_t>(recv[e]) * num_rows * Cs];
                    const P* y = &Y[e * nY];
                    for (int p = 0; p < np; ++p) {
                        const int l1 = Phi1_l1[p], l2 = Phi1_l2[p];
                        int row = row_base[p];
                        for (int lm1 = l1 * l1; lm1 <= l1 * (l1 + 2); ++lm1)
                            for (int lm2 = l2 * l2; lm2 <= l2 * (l2 + 2); ++lm2) {
                                for (int k = 0; k < C; ++k)
                                    acc[lm2 * Cs + k] += static_cast<double>(rad[p * Cs + k] * y[lm1] * rd[row * Cs + k]);
                                ++row;
                            }
                    }
                }
                for (std::size_t v = 0; v < LMC; ++v) H1_adj_dot[s * LMC + v] = static_cast<P>(acc[v]);
            }
            // 9. the field terms' reverse tangent and the Hessian column
            std::vector<double> part(static_cast<std::size_t>(n) * 3, 0.0);
            std::vector<P> H1p_adj_dot(n * LMC, P(0));
#pragma omp parallel for schedule(static)
            for (int i = 0; i < n; ++i) {
                std::vector<P> ad(LMC);
                for (int l = 0; l <= L_max; ++l)
                    for (int m = 0; m < 2 * l + 1; ++m)
                        lin_rev(&H1_adj_dot[i * LMC + (l * l + m) * Cs], &U_all[static_cast<std::size_t>(l) * Cs * Cs],
                                &ad[(l * l + m) * Cs]);
                for (int k = 0; k < C; ++k) ad[k] += static_cast<P>(direct_dot[i * Cs + k]);
                const P* hp = &H1_pre[i * LMC];
                const P* fa = &H1f_adj[i * LMC];
                for (int li = 0; li < num_LM; ++li)
                    for (int in = 0; in < C; ++in) {
                        P value = ad[li * Cs + in];
                        for (const auto& en : field_entries) {
                            if (en.lm_in != li) continue;
                            const P* W = &field_W[static_cast<std::size_t>(en.path) * Cs * Cs + in * Cs];
                            P tr_dot = 0, tr = 0;
                            for (int out = 0; out < C; ++out) {
                                tr_dot += W[out] * ad[en.lm_out * Cs + out];
                                tr += W[out] * fa[en.lm_out * Cs + out];
                            }
                            value += field_value(i, en.comp) * (en.coef * tr_dot);
                            if (en.comp == seed && !(response_drop & 16)) value += en.coef * tr;
                            part[3 * static_cast<std::size_t>(i) + en.comp] +=
                                static_cast<double>(hp[li * Cs + in] * (en.coef * tr_dot));
                        }
                        H1p_adj_dot[i * LMC + li * Cs + in] = value;
                    }
            }
            for (int i = 0; i < n; ++i)
                for (int c = 0; c < 3; ++c) field_hessian[c * 3 + seed] += part[3 * static_cast<std::size_t>(i) + c];
            if (!with_forces) continue;
            // 10. the layer-1 reverse of H1p_adj_dot: M0, A0 (density scale),
            // the R0 reverse
            std::vector<double> dens_dot0(n, 0.0);
#pragma omp parallel for schedule(dynamic, 16)
            for (int i = 0; i < n; ++i) {
                std::vector<P> m0a(LMC), a0a(YC, P(0)), padj(YC), rad(Cs), drad(Cs);
                for (int l = 0; l <= L_max; ++l)
                    for (int m = 0; m < 2 * l + 1; ++m)
                        lin_rev(&H1p_adj_dot[i * LMC + (l * l + m) * Cs], &P_all[static_cast<std::size_t>(l) * Cs * Cs],
                                &m0a[(l * l + m) * Cs]);
                for (int v = 0; v < nY; ++v)
                    for (int LM = 0; LM < num_LM; ++LM) {
                        const P* g = &M0_grad[((static_cast<std::size_t>(i) * num_LM + LM) * nY + v) * Cs];
                        for (int k = 0; k < C; ++k) a0a[v * Cs + k] += g[k] * m0a[LM * Cs + k];
                    }
                if (A0_scaled) {
                    const P* a = &A0[i * YC];
                    double dot = 0.0;
                    for (std::size_t v = 0; v < YC; ++v) dot += static_cast<double>(a0a[v] * a[v]);
                    dens_dot0[i] = (response_drop & 32) ? 0.0 : dot;
                    for (std::size_t v = 0; v < YC; ++v)
                        a0a[v] = static_cast<P>(static_cast<double>(a0a[v]) / A0_scale[i]);
                }
                for (int l = 0; l <= l_max; ++l)
                    for (int m = 0; m < 2 * l + 1; ++m)
                        lin_rev(&a0a[(l * l + m) * Cs], A0_w[types[i]][l].data(), &padj[(l * l + m) * Cs]);
                for (long long e = off[i]; e < off[i + 1]; ++e) {
                    if (!active[e]) continue;
                    const auto& sp = *spl0[pair_index(types[i], neigh_types[e])];
                    const auto pt = sp.point(static_cast<P>(r[e]));
                    const P* cf = sp.coefficients(pt);
                    const int ns = sp.num_splines;
                    const P* h0 = &H0[static_cast<std::size_t>(neigh_types[e]) * Cs];
                    const P* y = &Y[e * nY];
                    const P* gy = &Ygrad[e * 3 * nY];
                    double f[3] = {0, 0, 0};
                    for (int l = 0; l <= l_max; ++l) {
                        for (int k = 0; k < C; ++k) {
                            const int fi = l * C + k;
                            rad[k] = cf[fi] + cf[ns + fi] * pt.x + cf[2 * ns + fi] * pt.xx + cf[3 * ns + fi] * pt.xxx;
                            drad[k] = cf[ns + fi] + P(2.0) * cf[2 * ns + fi] * pt.x + P(3.0) * cf[3 * ns + fi] * pt.xx;
                        }
                        for (int m = -l; m <= l; ++m) {
                            const int lm = l * l + l + m;
                            P radial_sum = 0, angular_sum = 0;
                            for (int k = 0; k < C; ++k) {
                                radial_sum += padj[lm * Cs + k] * drad[k] * h0[k];
                                angular_sum += padj[lm * Cs + k] * rad[k] * h0[k];
                            }
                            for (int c = 0; c < 3; ++c)
                                f[c] -= static_cast<double>(dirs[3 * e + c] * radial_sum * y[lm] + angular_sum * gy[c * nY + lm]);
                        }
                    }
                    for (int c = 0; c < 3; ++c) fdot[3 * e + c] += f[c];
                }
            }
            if (A0_scaled)
                for (int i = 0; i < n; ++i)
                    for (long long e = off[i]; e < off[i + 1]; ++e) {
                        double f, d;
                        density_eval(*dens0[pair_index(types[i], neigh_types[e])], r[e], f, d);
                        for (int c = 0; c < 3; ++c)
                            fdot[3 * e + c] += dens_dot0[i] / A0_scale[i] * d * xyz[3 * e + c] / r[e];
                    }
            std::copy(fdot.begin(), fdot.end(), field_force_derivative.begin() + 3 * static_cast<std::size_t>(E) * seed);
        }
    }

    // field_coupling.hpp:60-238 (compile_field_coupling) and mace.cpp:2832-2860
    void load_field(const Value& j) {
        if (L_max < 1 || L_max > 2) throw std::invalid_argument("MACEField supports 1 <= L_max <= 2");
        const Value& list = j.at("field_couplings");
        if (list.size() != 1) throw std::invalid_argument("MACEField JSON must contain exactly one field coupling");
        const Value& cp = list.at(0);
        const bool legacy = !cp.contains("schema_version");
        if (!legacy && cp.at("schema_version").as_int() != 1)
            throw std::invalid_argument("unsupported MACEField field-coupling schema version");
        if (legacy && L_max != 1) throw std::invalid_argument("unversioned MACEField coupling needs L_max == 1");
        std::string hidden;
        for (int l = 0; l <= L_max; ++l)
            hidden += (l ? "+" : "") + std::to_string(C) + "x" + std::to_string(l) + (l % 2 ? "o" : "e");
        if (cp.at("field_feats_irreps_in1").as_string() != hidden || cp.at("field_feats_irreps_in2").as_string() != "1x1o" ||
            cp.at("field_feats_irreps_out").as_string() != hidden ||
            cp.at("field_linear_irreps_in").as_string() != hidden ||
            cp.at("field_linear_irreps_out").as_string() != hidden)
            throw std::invalid_argument("MACEField coupling must use the canonical equal-channel hidden irreps");
        const std::size_t hs = static_cast<std::size_t>(num_LM) * C;
        for (const char* key : {"field_feats_output_mask", "field_linear_output_mask"}) {
            const auto m = cp.at(key).as_doubles();
            if (m.size() != hs) throw std::invalid_argument(std::string("MACEField ") + key + " has an invalid size");
            for (double v : m)
                if (v != 1.0) throw std::invalid_argument(std::string("MACEField ") + key + " must contain only ones");
        }
        if (cp.at("field_linear_bias").size() != 0) throw std::invalid_argument("MACEField field_linear bias must be empty");
        const auto wf = j_doubles(cp.at("field_feats_weight"));
        const auto wl = j_doubles(cp.at("field_linear_weight"));
        const Value& fi_list = cp.at("field_feats_instructions");
        const Value& li_list = cp.at("field_linear_instructions");
        const std::size_t cc = static_cast<std::size_t>(C) * C;
        if (fi_list.size() * cc != wf.size()) throw std::invalid_argument("MACEField field_feats weight size mismatch");
        if (li_list.size() * cc != wl.size()) throw std::invalid_argument("MACEField field_linear weight size mismatch");
        const auto U = j.at("H1_linear_up_weights").as_doubles();
        const auto Pw = j.at("H1_product_weights").as_doubles();
        if (U.size() != static_cast<std::size_t>(L_max + 1) * cc || Pw.size() != U.size())
            throw std::invalid_argument("MACEField JSON must contain split H1 product and linear_up weights");
        P_all = castv(Pw);
        U_all = castv(U);
        for (std::size_t li = 0; li < li_list.size(); ++li) {
            const Value& ins = li_list.at(li);
            if (ins.at("path_shape").as_ints() != std::vector<int>{C, C})
                throw std::invalid_argument("MACEField field_linear instructions must be shaped (C, C)");
            const int a = ins.at("i_in").as_int(), b = ins.at("i_out").as_int();
            if (a < 0 || a > L_max || b != a)
                throw std::invalid_argument("MACEField field_linear instructions must keep each angular block");
        }
        field_entries.clear();
        field_W.clear();
        int path = 0;
        for (std::size_t fi = 0; fi < fi_list.size(); ++fi) {
            const Value& ins = fi_list.at(fi);
            if (ins.at("connection_mode").as_string() != "uvw" ||
                ins.at("path_shape").as_ints() != std::vector<int>{C, 1, C})
                throw std::invalid_argument("MACEField field_feats instructions must be uvw paths (C, 1, C)");
            const int lin = ins.at("i_in1").as_int(), blk = ins.at("i_in2").as_int(), lmid = ins.at("i_out").as_int();
            if (blk != 0 || lin < 0 || lin > L_max || lmid < 0 || lmid > L_max || std::abs(lin - lmid) != 1)
                throw std::invalid_argument("MACEField field_feats instruction is not an adjacent-rank 1o coupling");
            const int din = 2 * lin + 1, dmid = 2 * lmid + 1;
            std::vector<double> w3(static_cast<std::size_t>(din) * 3 * dmid, 0.0);
            if (legacy) {
                // the unversioned files' fixed pattern (field_coupling.hpp:145-156)
                for (int c = 0; c < 3; ++c) w3[lin == 0 ? c * 3 + c : c * 4] = 1.0 / std::sqrt(3.0);
            } else {
                if (ins.at("wigner_3j_shape").as_ints() != std::vector<int>{din, 3, dmid})
                    throw std::invalid_argument("MACEField Wigner tensor shape does not match its path");
                w3 = ins.at("wigner_3j").as_doubles();
                if (w3.size() != static_cast<std::size_t>(din) * 3 * dmid)
                    throw std::invalid_argument("MACEField Wigner tensor has an invalid size");
            }
            bool found = false;
            for (std::size_t li = 0; li < li_list.size(); ++li) {
                const Value& lins = li_list.at(li);
                if (lins.at("i_in").as_int() != lmid) continue;
                found = true;
                const int lout = lins.at("i_out").as_int();
                const int dout = 2 * lout + 1;
                for (int mi = 0; mi < din; ++mi)
                    for (int c = 0; c < 3; ++c)
                        for (int mo = 0; mo < dout; ++mo) {
                            const double w = w3[(static_cast<std::size_t>(mi) * 3 + c) * dout + mo];
                            if (std::abs(w) > 1e-14)
                                field_entries.push_back({lin * lin + mi, c, lout * lout + mo, path, cast(w)});
                        }
                const double scale = ins.at("path_weight").as_number() * lins.at("path_weight").as_number();
                for (int in = 0; in < C; ++in)
                    for (int out = 0; out < C; ++out) {
                        double v = 0.0;
                        for (int mid = 0; mid < C; ++mid)
                            v += wf[fi * cc + static_cast<std::size_t>(in) * C + mid] *
                                 wl[li * cc + static_cast<std::size_t>(mid) * C + out];
                        field_W.push_back(cast(scale * v));
                    }
                ++path;
            }
            if (!found) throw std::invalid_argument("MACEField field_feats output has no field_linear instruction");
        }
        if (path == 0) throw std::invalid_argument("MACEField field coupling contains no executable paths");
    }

    // nested numeric arrays flattened in order
    static std::vector<double> j_doubles(const Value& v) {
        std::vector<double> out;
        if (v.is_array() && !v.numeric_array && v.size() > 0 && v.at(0).is_array()) {
            for (std::size_t i = 0; i < v.size(); ++i) {
                const auto r = j_doubles(v.at(i));
                out.insert(out.end(), r.begin(), r.end());
            }
            return out;
        }
        return v.as_doubles();
    }

    // mace.cpp:119-214
    void prepare_active_types(const int* node_types, int n) {
        std::vector<int> req(node_types, node_types + n);
        std::sort(req.begin(), req.end());
        req.erase(std::unique(req.begin(), req.end()), req.end());
        if (req.empty()) throw std::invalid_argument("no active types");
        for (int t : req)
            if (t < 0 || t >= num_elements) throw std::out_of_range("type index out of range");
        if (req == active_types) return;
        auto tof = [](const std::vector<std::vector<double>>& a) {
            std::vector<std::vector<P>> o(a.size());
            for (std::size_t i = 0; i < a.size(); ++i) o[i] = castv(a[i]);
            return o;
        };
        const P hp = cast(radial.h), x0 = cast(radial.grid_min);
        spl0.clear();
        spl1.clear();
        dens0.clear();
        dens1.clear();
        const int na = static_cast<int>(req.size());
        // one set of tables per active pair (a <= b); without a distance
        // transform they are all the same tabulation
        for (int a = 0; a < na; ++a)
            for (int b = a; b < na; ++b) {
                if (radial.agnesi || spl0.empty()) {
                    const int ti = req[a], tj = req[b];
                    std::vector<std::vector<double>> v0, d0, v1, d1;
                    radial.tabulate(radial.R0, v0, d0, ti, tj);
                    spl0.push_back(std::make_shared<SplineSet<P>>(hp, tof(v0), tof(d0), x0));
                    if (radial.has_R1) {
                        radial.tabulate(radial.R1, v1, d1, ti, tj);
                        spl1.push_back(std::make_shared<SplineSet<P>>(hp, tof(v1), tof(d1), x0));
                    }
                    // RadialFunctionSetKokkos<double>(h, values, derivs, x0): FP64
                    // coefficients and evaluation (mace_kokkos_factorized_lifecycle.cpp:4084-4091)
                    if (A0_scaled) {
                        std::vector<std::vector<double>> v, d;
                        radial.tabulate(radial.A0, v, d, ti, tj);
                        dens0.push_back(std::make_shared<SplineSet<double>>(radial.h, v, d, radial.grid_min));
                    }
                    if (A1_scaled) {
                        std::vector<std::vector<double>> v, d;
                        radial.tabulate(radial.A1, v, d, ti, tj);
                        dens1.push_back(std::make_shared<SplineSet<double>>(radial.h, v, d, radial.grid_min));
                    }
                } else {
                    spl0.push_back(spl0.front());
                    if (radial.has_R1) spl1.push_back(spl1.front());
                    if (A0_scaled) dens0.push_back(dens0.front());
                    if (A1_scaled) dens1.push_back(dens1.front());
                }
            }
        type_to_active.assign(num_elements, -1);
        for (int a = 0; a < na; ++a) type_to_active[req[a]] = a;
        active_types = req;
    }

    int pair_index(int ti, int tj) const {
        const int a = type_to_active[ti], b = type_to_active[tj];
        if (a < 0 || b < 0) throw std::runtime_error("radial cache not prepared for a type");
        const int n = static_cast<int>(active_types.size());
        return a <= b ? a * (2 * n - a - 1) / 2 + b : b * (2 * n - b - 1) / 2 + a;
    }

    int row_base_of_path(int p) const {
        int acc = 0;
        for (int i = 0; i < p; ++i) acc += (2 * Phi1_l1[i] + 1) * (2 * Phi1_l2[i] + 1);
        return acc;
    }

    // f(r) and f'(r) of a one-function FP64 density spline
    // (radial_function_set_kokkos.hpp:48-62,104-146)
    static void density_eval(const SplineSet<double>& sp, double r, double& f, double& d) {
        const auto pt = sp.point(r);
        const double* c = sp.coefficients(pt);
        f = c[0] + c[1] * pt.x + c[2] * pt.xx + c[3] * pt.xxx;
        d = c[1] + c[2] * (2.0 * pt.x) + c[3] * (3.0 * pt.xx);
    }

    // 1 + sum over every CSR edge of i (skin edges included, r clamped to the
    // cutoff) of f(r): the Kokkos team reduction then += 1.0
    double density_factor(const std::vector<std::shared_ptr<SplineSet<double>>>& sp, int type_i,
                          const int* neigh_types, long long e0, long long e1, const double* r) const {
        double s = 0.0;
        for (long long e = e0; e < e1; ++e) {
            double f, d;
            density_eval(*sp[pair_index(type_i, neigh_types[e])], r[e], f, d);
            s += f;
        }
        return s + 1.0;
    }

    void evaluate(int n, const int* types, const int* num_neigh, const int* neigh, const int* neigh_types,
                  const double* xyz, const double* r) {
        prepare_active_types(types, n);
        std::vector<long long> off(n + 1, 0);
        for (int i = 0; i < n; ++i) off[i + 1] = off[i] + num_neigh[i];
        const long long E = off[n];
        for (long long e = 0; e < E; ++e)
            if (neigh[e] < 0 || neigh[e] >= n) throw std::invalid_argument("neighbour index out of range");
        const int nY = num_lm;
        const std::size_t Cs = static_cast<std::size_t>(C);
        Y.assign(static_cast<std::size_t>(E) * nY, P(0));
        Ygrad.assign(static_cast<std::size_t>(E) * 3 * nY, P(0));
        std::vector<P> dirs(static_cast<std::size_t>(E) * 3, P(0));
        std::vector<char> active(E, 0);
#pragma omp parallel for schedule(static)
        for (long long e = 0; e < E; ++e) {
            if (!(r[e] < r_cut)) continue;  // direct plan: Y = 0, no force
            active[e] = 1;
            P d[3];
            for (int c = 0; c < 3; ++c) d[c] = static_cast<P>(xyz[3 * e + c] / r[e]);
            for (int c = 0; c < 3; ++c) dirs[3 * e + c] = d[c];
            edge_harmonics<P>(l_max, d, static_cast<P>(r[e]), &Y[e * nY], &Ygrad[e * 3 * nY]);
        }

        // ---- ZBL (mace_kokkos_evaluate.cpp:418-434; zbl_kokkos.cpp:163-199):
        // every CSR edge, node energy += V, directed force -= (xyz/r) dV/dr
        zbl_energies.assign(has_zbl ? n : 0, 0.0);
        zbl_forces.assign(has_zbl ? static_cast<std::size_t>(E) * 3 : 0, 0.0);
        if (has_zbl) {
#pragma omp parallel for schedule(static)
            for (int i = 0; i < n; ++i) {
                const int Zi = atomic_numbers[types[i]];
                double ei = 0.0;
                for (long long e = off[i]; e < off[i + 1]; ++e) {
                    double v, g;
                    zbl.value_gradient(Zi, atomic_numbers[neigh_types[e]], r[e], v, g);
                    ei += v;
                    for (int c = 0; c < 3; ++c) zbl_forces[3 * e + c] -= xyz[3 * e + c] / r[e] * g;
                }
                zbl_energies[i] = ei;
            }
        }

        // ---- A0 (mace.cpp:1356-1403)
        A0_scale.assign(A0_scaled ? n : 0, 1.0);
        A1_scale.assign(A1_scaled ? n : 0, 1.0);
        A0.assign(static_cast<std::size_t>(n) * nY * Cs, P(0));
        Phi0.assign(static_cast<std::size_t>(n) * nY * Cs, P(0));
#pragma omp parallel for schedule(dynamic, 16)
        for (int i = 0; i < n; ++i) {
            std::vector<P> phi(nY * Cs, P(0)), rad(Cs);
            for (long long e = off[i]; e < off[i + 1]; ++e) {
                if (!active[e]) continue;
                const auto& sp = *spl0[pair_index(types[i], neigh_types[e])];
                const auto pt = sp.point(static_cast<P>(r[e]));
                const P* cf = sp.coefficients(pt);
                const int ns = sp.num_splines;
                const P* h0 = &H0[static_cast<std::size_t>(neigh_types[e]) * Cs];
                for (int l = 0; l <= l_max; ++l) {
                    for (int k = 0; k < C; ++k) {
                        const int f = l * C + k;
                        rad[k] = cf[f] + cf[ns + f] * pt.x + cf[2 * ns + f] * pt.xx + cf[3 * ns + f] * pt.xxx;
                    }
                    for (int m = -l; m <= l; ++m) {
                        const int lm = l * l + l + m;
                        const P y = Y[e * nY + lm];
                        P* dst = &phi[lm * Cs];
                        for (int k = 0; k < C; ++k) dst[k] += rad[k] * y * h0[k];
                    }
                }
            }
            std::copy(phi.begin(), phi.end(), Phi0.begin() + static_cast<std::size_t>(i) * nY * Cs);
            for (int l = 0; l <= l_max; ++l) {
                const P* W = A0_w[types[i]][l].data();
                for (int m = 0; m < 2 * l + 1; ++m) {
                    const P* src = &phi[(l * l + m) * Cs];
                    P* dst = &A0[(static_cast<std::size_t>(i) * nY + l * l + m) * Cs];
                    for (int kp = 0; kp < C; ++kp) {
                        const P a = src[kp];
                        const P* wr = W + kp * Cs;
                        for (int k = 0; k < C; ++k) dst[k] += a * wr[k];
                    }
                }
            }
            // A0 /= 1 + sum_j f0(r_ij), the division in FP64
            // (mace_kokkos_first_interaction.cpp:1383-1416)
            if (A0_scaled) {
                const double sc = density_factor(dens0, types[i], neigh_types, off[i], off[i + 1], r);
                A0_scale[i] = sc;
                P* a = &A0[static_cast<std::size_t>(i) * nY * Cs];
                for (std::size_t v = 0; v < nY * Cs; ++v) a[v] = static_cast<P>(static_cast<double>(a[v]) / sc);
            }
        }

        // ---- M0 (mace.cpp:1639-1663)
        M0.assign(static_cast<std::size_t>(n) * num_LM * Cs, P(0));
        M0_grad.assign(static_cast<std::size_t>(n) * num_LM * nY * Cs, P(0));
#pragma omp parallel for schedule(static)
        for (int i = 0; i < n; ++i) {
            P x[16], g[16];
            for (int LM = 0; LM < num_LM; ++LM) {
                const int T = static_cast<int>(M0_monos[LM].monos.size());
                const P* coef = M0_coef[types[i] * num_LM + LM].data();
                for (int k = 0; k < C; ++k) {
                    for (int v = 0; v < nY; ++v) x[v] = A0[(static_cast<std::size_t>(i) * nY + v) * Cs + k];
                    M0[(static_cast<std::size_t>(i) * num_LM + LM) * Cs + k] =
                        poly_eval_grad<P>(M0_monos[LM], coef + static_cast<std::size_t>(k) * T, x, g, nY);
                    for (int v = 0; v < nY; ++v)
                        M0_grad[((static_cast<std::size_t>(i) * num_LM + LM) * nY + v) * Cs + k] = g[v];
                }
            }
        }

        // ---- H1 and the v4 scalar capture (mace.cpp:1691-1783)
        H1.assign(static_cast<std::size_t>(n) * num_LM * Cs, P(0));
        xaff.assign(static_cast<std::size_t>(n) * Cs, P(0));
#pragma omp parallel for schedule(static)
        for (int i = 0; i < n; ++i) {
            const P* m00 = &M0[static_cast<std::size_t>(i) * num_LM * Cs];
            if (pre_linear_up) {
                // x = M0[i,0,:] P0 (gemv in Precision, input order)
                for (int k = 0; k < C; ++k) {
                    P s = 0;
                    for (int in = 0; in < C; ++in) s += m00[in] * P0[static_cast<std::size_t>(in) * C + k];
                    xaff[i * Cs + k] = s;
                }
            } else {
                for (int k = 0; k < C; ++k) xaff[i * Cs + k] = m00[k];
            }
            for (int l = 0; l <= L_max; ++l)
                for (int m = 0; m < 2 * l + 1; ++m) {
                    const P* src = &M0[(static_cast<std::size_t>(i) * num_LM + l * l + m) * Cs];
                    P* dst = &H1[(static_cast<std::size_t>(i) * num_LM + l * l + m) * Cs];
                    const P* W = &H1_w[static_cast<std::size_t>(l) * Cs * Cs];
                    for (int kp = 0; kp < C; ++kp) {
                        const P a = src[kp];
                        for (int k = 0; k < C; ++k) dst[k] += a * W[kp * Cs + k];
                    }
                }
            if (residual) {
                const int t = types[i];
                for (int lm = 0; lm < num_LM; ++lm)
                    for (int k = 0; k < C; ++k)
                        H1[(static_cast<std::size_t>(i) * num_LM + lm) * Cs + k] +=
                            res_fused[(static_cast<std::size_t>(t) * num_LM + lm) * C + k];
                // the scalar input takes the residual in the pre_linear_up
                // basis only (mace.cpp:1863-1872)
                if (pre_linear_up)
                    for (int k = 0; k < C; ++k) xaff[i * Cs + k] += res_x[static_cast<std::size_t>(t) * C + k];
            }
        }
        if (has_field) field_forward(n, types);

        // ---- Phi1 streamed (mace.cpp:2023-2084)
        const int np = static_cast<int>(Phi1_l.size());
        std::vector<int> row_base(np);
        for (int p = 0; p < np; ++p) row_base[p] = row_base_of_path(p);
        Phi1.assign(static_cast<std::size_t>(n) * num_lme * Cs, P(0));
        if (!single_layer) {
#pragma omp parallel for schedule(dynamic, 16)
        for (int i = 0; i < n; ++i) {
            std::vector<P> rows(static_cast<std::size_t>(num_rows) * Cs, P(0)), rad(Cs);
            for (long long e = off[i]; e < off[i + 1]; ++e) {
                if (!active[e]) continue;
                const auto& sp = *spl1[pair_index(types[i], neigh_types[e])];
                const auto pt = sp.point(static_cast<P>(r[e]));
                const P* cf = sp.coefficients(pt);
                const int ns = sp.num_splines;
                const P* Hj = &H1[static_cast<std::size_t>(neigh[e]) * num_LM * Cs];
                for (int p = 0; p < np; ++p) {
                    for (int k = 0; k < C; ++k) {
                        const int f = p * C + k;
                        rad[k] = cf[f] + cf[ns + f] * pt.x + cf[2 * ns + f] * pt.xx + cf[3 * ns + f] * pt.xxx;
                    }
                    const int l1 = Phi1_l1[p], l2 = Phi1_l2[p];
                    int row = row_base[p];
                    for (int lm1 = l1 * l1; lm1 <= l1 * (l1 + 2); ++lm1) {
                        const P y = Y[e * nY + lm1];
                        for (int lm2 = l2 * l2; lm2 <= l2 * (l2 + 2); ++lm2) {
                            const P* h = Hj + lm2 * Cs;
                            P* dst = &rows[row * Cs];
                            for (int k = 0; k < C; ++k) dst[k] += rad[k] * y * h[k];
                            ++row;
                        }
                    }
                }
            }
            P* out = &Phi1[static_cast<std::size_t>(i) * num_lme * Cs];
            for (std::size_t t = 0; t < Phi1_cg.size(); ++t) {
                const P c = Phi1_cg[t];
                const P* src = &rows[Phi1_row[t] * Cs];
                P* dst = out + Phi1_lme[t] * Cs;
                for (int k = 0; k < C; ++k) dst[k] += c * src[k];
            }
        }
        }

        // ---- A1 (mace.cpp:2305-2341)
        A1.assign(single_layer ? 0 : static_cast<std::size_t>(n) * nY * Cs, P(0));
        if (!single_layer) {
#pragma omp parallel for schedule(static)
        for (int i = 0; i < n; ++i) {
            for (int l = 0; l <= l_max; ++l) {
                const int ne = num_e[l];
                const P* W = A1_w[l].data();
                for (int m = 0; m < 2 * l + 1; ++m) {
                    P* dst = &A1[(static_cast<std::size_t>(i) * nY + l * l + m) * Cs];
                    for (int e = 0; e < ne; ++e) {
                        const P* src = &Phi1[(static_cast<std::size_t>(i) * num_lme + lme_base[l] + m * ne + e) * Cs];
                        for (int kp = 0; kp < C; ++kp) {
                            const P a = src[kp];
                            const P* wr = W + (static_cast<std::size_t>(e) * Cs + kp) * Cs;
                            for (int k = 0; k < C; ++k) dst[k] += a * wr[k];
                        }
                    }
                }
            }
            // A1 *= Precision(1 / (1 + sum_j f1(r_ij)))
            // (mace_kokkos_second_interaction.cpp:1449-1488)
            if (A1_scaled) {
                const double sc = density_factor(dens1, types[i], neigh_types, off[i], off[i + 1], r);
                A1_scale[i] = sc;
                const P inv = static_cast<P>(1.0 / sc);
                P* a = &A1[static_cast<std::size_t>(i) * nY * Cs];
                for (std::size_t v = 0; v < nY * Cs; ++v) a[v] *= inv;
            }
        }
        }

        // ---- M1, H2, readouts, reverse H2 / M1 (mace.cpp:2461-2657).  M1's
        // variables are A1's num_lm components or, with one interaction, H1's
        // num_LM ones; their adjoint is A1_adj or H1_adj.
        const int T1 = static_cast<int>(M1_monos.monos.size());
        const int nV = single_layer ? num_LM : nY;
        const std::vector<P>& m1_in = single_layer ? H1 : A1;
        std::vector<P>& m1_in_adj = single_layer ? H1_adj : A1_adj;
        M1.assign(static_cast<std::size_t>(n) * Cs, P(0));
        M1_grad.assign(static_cast<std::size_t>(n) * nV * Cs, P(0));
        H2.assign(static_cast<std::size_t>(n) * Cs, 0.0);
        H2_adj.assign(static_cast<std::size_t>(n) * Cs, 0.0);
        direct.assign(static_cast<std::size_t>(n) * Cs, 0.0);
        node_energies.assign(n, 0.0);
        A1_adj.assign(single_layer ? 0 : static_cast<std::size_t>(n) * nY * Cs, P(0));
        if (single_layer) H1_adj.assign(static_cast<std::size_t>(n) * num_LM * Cs, P(0));
#pragma omp parallel for schedule(static)
        for (int i = 0; i < n; ++i) {
            P x[16], g[16];
            const int t = types[i];
            for (int k = 0; k < C; ++k) {
                for (int v = 0; v < nV; ++v) x[v] = m1_in[(static_cast<std::size_t>(i) * nV + v) * Cs + k];
                M1[i * Cs + k] = poly_eval_grad<P>(M1_monos, M1_coef[t].data() + static_cast<std::size_t>(k) * T1, x, g, nV);
                for (int v = 0; v < nV; ++v) M1_grad[(static_cast<std::size_t>(i) * nV + v) * Cs + k] = g[v];
            }
            double* h2 = &H2[i * Cs];
            for (int o = 0; o < C; ++o) {
                double s = 0.0;
                for (int in = 0; in < C; ++in) s += H2_T[t][in * Cs + o] * static_cast<double>(xaff[i * Cs + in]);
                for (int in = 0; in < C; ++in) s += H2_M1[in * Cs + o] * static_cast<double>(M1[i * Cs + in]);
                h2[o] = s;
            }
            double e = atomic_energies[t];
            for (int k = 0; k < C; ++k) e += q[k] * static_cast<double>(xaff[i * Cs + k]);
            // readout_2 MLP [C, hidden, 1] and its gradient
            std::vector<double> z(hidden), act(hidden), dact(hidden);
            for (int hdn = 0; hdn < hidden; ++hdn) {
                double s = 0.0;
                for (int k = 0; k < C; ++k) s += W1[hdn * Cs + k] * h2[k];
                const double sg = 1.0 / (1.0 + std::exp(-s));
                z[hdn] = s;
                act[hdn] = readout_scale * s * sg;
                dact[hdn] = readout_scale * sg + readout_scale * s * sg * (1.0 - sg);
            }
            double out = 0.0;
            for (int hdn = 0; hdn < hidden; ++hdn) out += W2[hdn] * act[hdn];
            node_energies[i] = e + out;
            double* h2a = &H2_adj[i * Cs];
            for (int k = 0; k < C; ++k) {
                double s = 0.0;
                for (int hdn = 0; hdn < hidden; ++hdn) s += W2[hdn] * dact[hdn] * W1[hdn * Cs + k];
                h2a[k] = s;
            }
            // reverse_H2 (m0_composite): direct = q + T_z H2_adj; M1_adj = W H2_adj
            for (int in = 0; in < C; ++in) {
                double s = q[in], s1 = 0.0;
                for (int o = 0; o < C; ++o) {
                    s += H2_T[t][in * Cs + o] * h2a[o];
                    s1 += H2_M1[in * Cs + o] * h2a[o];
                }
                direct[i * Cs + in] = s;
                const P m1adj = static_cast<P>(s1);
                for (int v = 0; v < nV; ++v)
                    m1_in_adj[(static_cast<std::size_t>(i) * nV + v) * Cs + in] =
                        M1_grad[(static_cast<std::size_t>(i) * nV + v) * Cs + in] * m1adj;
            }
        }

        // ---- reverse of the A1 density scale (mace_kokkos_second_interaction.cpp:
        // 1636-1719): dot = sum A1_adj*A1 (FP32 products, FP64 sum); edge
        // forces += (dot/s) f1'(r) (xyz/r); A1_adj *= Precision(1/s).  The
        // edge terms are kept apart and added to the directed forces after the
        // R1 reverse (FP64 sums in another order than the reference's).
        density_forces.assign(static_cast<std::size_t>(E) * 3, 0.0);
        if (A1_scaled) {
#pragma omp parallel for schedule(static)
            for (int i = 0; i < n; ++i) {
                const double sc = A1_scale[i];
                P* adj = &A1_adj[static_cast<std::size_t>(i) * nY * Cs];
                const P* a = &A1[static_cast<std::size_t>(i) * nY * Cs];
                double dot = 0.0;
                for (std::size_t v = 0; v < nY * Cs; ++v) dot += static_cast<double>(adj[v] * a[v]);
                for (long long e = off[i]; e < off[i + 1]; ++e) {
                    double f, d;
                    density_eval(*dens1[pair_index(types[i], neigh_types[e])], r[e], f, d);
                    const double scale = dot / sc * d;
                    for (int c = 0; c < 3; ++c) density_forces[3 * e + c] += scale * (xyz[3 * e + c] / r[e]);
                }
                const P inv = static_cast<P>(1.0 / sc);
                for (std::size_t v = 0; v < nY * Cs; ++v) adj[v] *= inv;
            }
        }

        // ---- reverse A1 (mace.cpp:2343-2379)
        dPhi1.assign(static_cast<std::size_t>(n) * num_lme * Cs, P(0));
        node_forces.assign(static_cast<std::size_t>(E) * 3, 0.0);
        node_forces_r1 = node_forces;
        if (!single_layer) {
#pragma omp parallel for schedule(static)
        for (int i = 0; i < n; ++i) {
            for (int l = 0; l <= l_max; ++l) {
                const int ne = num_e[l];
                const P* W = A1_w[l].data();
                for (int m = 0; m < 2 * l + 1; ++m) {
                    const P* src = &A1_adj[(static_cast<std::size_t>(i) * nY + l * l + m) * Cs];
                    for (int e = 0; e < ne; ++e) {
                        P* dst = &dPhi1[(static_cast<std::size_t>(i) * num_lme + lme_base[l] + m * ne + e) * Cs];
                        for (int k = 0; k < C; ++k) {
                            const P* wr = W + (static_cast<std::size_t>(e) * Cs + k) * Cs;
                            P s = 0;
                            for (int kp = 0; kp < C; ++kp) s += src[kp] * wr[kp];
                            dst[k] = s;
                        }
                    }
                }
            }
        }

        // ---- reverse Phi1 (mace.cpp:2199-2303): receiver-owned edge forces,
        // source adjoint via the source transpose (FP64 accumulation).
        std::vector<P> dPhi1r(static_cast<std::size_t>(n) * num_rows * Cs, P(0));
#pragma omp parallel for schedule(static)
        for (int i = 0; i < n; ++i) {
            P* rows = &dPhi1r[static_cast<std::size_t>(i) * num_rows * Cs];
            const P* src = &dPhi1[static_cast<std::size_t>(i) * num_lme * Cs];
            for (std::size_t t = 0; t < Phi1_cg.size(); ++t) {
                const P c = Phi1_cg[t];
                const P* a = src + Phi1_lme[t] * Cs;
                P* d = rows + Phi1_row[t] * Cs;
                for (int k = 0; k < C; ++k) d[k] += c * a[k];
            }
        }
        std::vector<int> recv(E);
        for (int i = 0; i < n; ++i)
            for (long long e = off[i]; e < off[i + 1]; ++e) recv[e] = i;
        auto edge_r1 = [&](long long e, P* rad, P* drad) {
            const auto& sp = *spl1[pair_index(types[recv[e]], neigh_types[e])];
            const auto pt = sp.point(static_cast<P>(r[e]));
            const P* cf = sp.coefficients(pt);
            const int ns = sp.num_splines;
            for (int f = 0; f < ns; ++f) {
                rad[f] = cf[f] + cf[ns + f] * pt.x + cf[2 * ns + f] * pt.xx + cf[3 * ns + f] * pt.xxx;
                if (drad) drad[f] = cf[ns + f] + P(2.0) * cf[2 * ns + f] * pt.x + P(3.0) * cf[3 * ns + f] * pt.xx;
            }
        };
#pragma omp parallel
        {
        std::vector<P> rad(np * Cs), drad(np * Cs);
#pragma omp for schedule(dynamic, 64)
        for (long long e = 0; e < E; ++e) {
            if (!active[e]) continue;
            const int i = recv[e];
            edge_r1(e, rad.data(), drad.data());
            const P* rows = &dPhi1r[static_cast<std::size_t>(i) * num_rows * Cs];
            const P* Hj = &H1[static_cast<std::size_t>(neigh[e]) * num_LM * Cs];
            const P* y = &Y[e * nY];
            const P* g = &Ygrad[e * 3 * nY];
            double f[3] = {0, 0, 0};
            for (int p = 0; p < np; ++p) {
                const int l1 = Phi1_l1[p], l2 = Phi1_l2[p];
                int row = row_base[p];
                for (int lm1 = l1 * l1; lm1 <= l1 * (l1 + 2); ++lm1)
                    for (int lm2 = l2 * l2; lm2 <= l2 * (l2 + 2); ++lm2) {
                        const P* adj = rows + row * Cs;
                        const P* h = Hj + lm2 * Cs;
                        P radial_sum = 0, angular_sum = 0;
                        for (int k = 0; k < C; ++k) {
                            radial_sum += adj[k] * drad[p * Cs + k] * h[k];
                            angular_sum += adj[k] * rad[p * Cs + k] * h[k];
                        }
                        for (int c = 0; c < 3; ++c)
                            f[c] -= static_cast<double>(dirs[3 * e + c] * radial_sum * y[lm1] + angular_sum * g[c * nY + lm1]);
                        ++row;
                    }
            }
            for (int c = 0; c < 3; ++c) node_forces[3 * e + c] += f[c];
        }
        }
        node_forces_r1 = node_forces;
        // source adjoint over the source transpose (deterministic, no atomics)
        std::vector<long long> soff(n + 1, 0);
        for (long long e = 0; e < E; ++e) soff[neigh[e] + 1] += 1;
        for (int s = 0; s < n; ++s) soff[s + 1] += soff[s];
        std::vector<long long> sedges(E), cursor(soff.begin(), soff.end() - 1);
        for (long long e = 0; e < E; ++e) sedges[cursor[neigh[e]]++] = e;
        H1_adj.assign(static_cast<std::size_t>(n) * num_LM * Cs, P(0));
#pragma omp parallel for schedule(dynamic, 16)
        for (int s = 0; s < n; ++s) {
            std::vector<double> acc(num_LM * Cs, 0.0);
            std::vector<P> rad(np * Cs);
            for (long long q2 = soff[s]; q2 < soff[s + 1]; ++q2) {
                const long long e = sedges[q2];
                if (!active[e]) continue;
                edge_r1(e, rad.data(), nullptr);
                const P* rows = &dPhi1r[static_cast<std::size_t>(recv[e]) * num_rows * Cs];
                const P* y = &Y[e * nY];
                for (int p = 0; p < np; ++p) {
                    const int l1 = Phi1_l1[p], l2 = Phi1_l2[p];
                    int row = row_base[p];
                    for (int lm1 = l1 * l1; lm1 <= l1 * (l1 + 2); ++lm1)
                        for (int lm2 = l2 * l2; lm2 <= l2 * (l2 + 2); ++lm2) {
                            const P* adj = rows + row * Cs;
                            double* dst = &acc[lm2 * Cs];
                            for (int k = 0; k < C; ++k)
                                dst[k] += static_cast<double>(rad[p * Cs + k] * y[lm1] * adj[k]);
                            ++row;
                        }
                }
            }
            for (int v = 0; v < num_LM * C; ++v)
                H1_adj[static_cast<std::size_t>(s) * num_LM * Cs + v] = static_cast<P>(acc[v]);
        }
        }

        // ---- reverse H1 + direct adjoint (mace.cpp:1727-1757, 1785-1814)
        M0_adj.assign(static_cast<std::size_t>(n) * num_LM * Cs, P(0));
        if (has_field) field_reverse(n);
        if (!has_field) {
#pragma omp parallel for schedule(static)
        for (int i = 0; i < n; ++i) {
            for (int l = 0; l <= L_max; ++l)
                for (int m = 0; m < 2 * l + 1; ++m) {
                    const P* src = &H1_adj[(static_cast<std::size_t>(i) * num_LM + l * l + m) * Cs];
                    P* dst = &M0_adj[(static_cast<std::size_t>(i) * num_LM + l * l + m) * Cs];
                    const P* W = &H1_w[static_cast<std::size_t>(l) * Cs * Cs];
                    for (int k = 0; k < C; ++k) {
                        P s = 0;
                        for (int kp = 0; kp < C; ++kp) s += src[kp] * W[k * Cs + kp];
                        dst[k] = s;
                    }
                }
            if (pre_linear_up) {
                // M0_adj[i,0,:] += P0 d (the scalar input was M0 P0 + residual)
                for (int in = 0; in < C; ++in) {
                    double s = 0.0;
                    for (int o = 0; o < C; ++o)
                        s += static_cast<double>(P0[static_cast<std::size_t>(in) * C + o]) * direct[i * Cs + o];
                    M0_adj[static_cast<std::size_t>(i) * num_LM * Cs + in] += static_cast<P>(s);
                }
            } else {
                for (int k = 0; k < C; ++k)
                    M0_adj[static_cast<std::size_t>(i) * num_LM * Cs + k] += static_cast<P>(direct[i * Cs + k]);
            }
        }
        }

        // ---- reverse M0 (mace.cpp:1665-1689)
        A0_adj.assign(static_cast<std::size_t>(n) * nY * Cs, P(0));
#pragma omp parallel for schedule(static)
        for (int i = 0; i < n; ++i)
            for (int v = 0; v < nY; ++v) {
                P* dst = &A0_adj[(static_cast<std::size_t>(i) * nY + v) * Cs];
                for (int LM = 0; LM < num_LM; ++LM) {
                    const P* g = &M0_grad[((static_cast<std::size_t>(i) * num_LM + LM) * nY + v) * Cs];
                    const P* a = &M0_adj[(static_cast<std::size_t>(i) * num_LM + LM) * Cs];
                    for (int k = 0; k < C; ++k) dst[k] += g[k] * a[k];
                }
            }

        // ---- reverse of the A0 density scale (mace_kokkos_first_interaction.cpp:
        // 1508-1528): dot = sum A0_adj*A0; edge forces += dot/s*f0'(r)*xyz/r;
        // A0_adj /= s in FP64
        if (A0_scaled) {
#pragma omp parallel for schedule(static)
            for (int i = 0; i < n; ++i) {
                const double sc = A0_scale[i];
                P* adj = &A0_adj[static_cast<std::size_t>(i) * nY * Cs];
                const P* a = &A0[static_cast<std::size_t>(i) * nY * Cs];
                double dot = 0.0;
                for (std::size_t v = 0; v < nY * Cs; ++v) dot += static_cast<double>(adj[v] * a[v]);
                for (long long e = off[i]; e < off[i + 1]; ++e) {
                    double f, d;
                    density_eval(*dens0[pair_index(types[i], neigh_types[e])], r[e], f, d);
                    for (int c = 0; c < 3; ++c) density_forces[3 * e + c] += dot / sc * d * xyz[3 * e + c] / r[e];
                }
                for (std::size_t v = 0; v < nY * Cs; ++v) adj[v] = static_cast<P>(static_cast<double>(adj[v]) / sc);
            }
        }

        // ---- reverse A0 (mace.cpp:1486-1560)
        Phi0_adj.assign(static_cast<std::size_t>(n) * nY * Cs, P(0));
        node_forces_r0.assign(static_cast<std::size_t>(E) * 3, 0.0);
#pragma omp parallel for schedule(dynamic, 16)
        for (int i = 0; i < n; ++i) {
            std::vector<P> padj(nY * Cs, P(0)), rad(Cs), drad(Cs);
            for (int l = 0; l <= l_max; ++l) {
                const P* W = A0_w[types[i]][l].data();
                for (int m = 0; m < 2 * l + 1; ++m) {
                    const P* src = &A0_adj[(static_cast<std::size_t>(i) * nY + l * l + m) * Cs];
                    P* dst = &padj[(l * l + m) * Cs];
                    for (int k = 0; k < C; ++k) {
                        P s = 0;
                        for (int kp = 0; kp < C; ++kp) s += src[kp] * W[k * Cs + kp];
                        dst[k] = s;
                    }
                }
            }
            for (long long e = off[i]; e < off[i + 1]; ++e) {
                if (!active[e]) continue;
                const auto& sp = *spl0[pair_index(types[i], neigh_types[e])];
                const auto pt = sp.point(static_cast<P>(r[e]));
                const P* cf = sp.coefficients(pt);
                const int ns = sp.num_splines;
                const P* h0 = &H0[static_cast<std::size_t>(neigh_types[e]) * Cs];
                const P* y = &Y[e * nY];
                const P* g = &Ygrad[e * 3 * nY];
                double f[3] = {0, 0, 0};
                for (int l = 0; l <= l_max; ++l) {
                    for (int k = 0; k < C; ++k) {
                        const int fi = l * C + k;
                        rad[k] = cf[fi] + cf[ns + fi] * pt.x + cf[2 * ns + fi] * pt.xx + cf[3 * ns + fi] * pt.xxx;
                        drad[k] = cf[ns + fi] + P(2.0) * cf[2 * ns + fi] * pt.x + P(3.0) * cf[3 * ns + fi] * pt.xx;
                    }
                    for (int m = -l; m <= l; ++m) {
                        const int lm = l * l + l + m;
                        const P* adj = &padj[lm * Cs];
                        P radial_sum = 0, angular_sum = 0;
                        for (int k = 0; k < C; ++k) {
                            radial_sum += adj[k] * drad[k] * h0[k];
                            angular_sum += adj[k] * rad[k] * h0[k];
                        }
                        for (int c = 0; c < 3; ++c)
                            f[c] -= static_cast<double>(dirs[3 * e + c] * radial_sum * y[lm] + angular_sum * g[c * nY + lm]);
                    }
                }
                for (int c = 0; c < 3; ++c) {
                    node_forces[3 * e + c] += f[c];
                    node_forces_r0[3 * e + c] = f[c];
                }
            }
            std::copy(padj.begin(), padj.end(), Phi0_adj.begin() + static_cast<std::size_t>(i) * nY * Cs);
        }
        if (A0_scaled || A1_scaled)
            for (long long v = 0; v < 3 * E; ++v) node_forces[v] += density_forces[v];
        if (has_zbl) {
            for (long long v = 0; v < 3 * E; ++v) node_forces[v] += zbl_forces[v];
            for (int i = 0; i < n; ++i) node_energies[i] += zbl_energies[i];
        }
    }
};

// ---------------------------------------------------------------------------
// Neighbour list (neighbor_graph_kokkos.cpp:38-405), IEEE double, no FMA.
// ---------------------------------------------------------------------------

static int floor_div(int a, int b) {
    const int q = a / b, r = a % b;
    return q - ((r != 0 && r < 0) ? 1 : 0);
}

struct Graph {
    std::vector<int> num_neigh, offsets, sources, shifts;
    std::vector<double> fractional_xyz;
};

static void build_graph(const double* pos, int n, const double* cell, const double* inv, double cutoff, Graph& g,
                        bool fill) {
    if (!std::isfinite(cutoff) || !(cutoff > 0.0)) throw std::invalid_argument("cutoff must be positive");
    for (int row = 0; row < 3; ++row)
        for (int col = 0; col < 3; ++col) {
            double prod = 0.0;
            for (int k = 0; k < 3; ++k) prod += cell[3 * row + k] * inv[3 * k + col];
            if (std::abs(prod - (row == col ? 1.0 : 0.0)) > 1e-9)
                throw std::invalid_argument("cell and inverse cell are inconsistent");
        }
    std::vector<double> frac(3 * n), wfrac(3 * n), wpos(3 * n);
    std::vector<int> wrap(3 * n);
    for (int a = 0; a < n; ++a) {
        double f[3];
        for (int ax = 0; ax < 3; ++ax) {
            double v = 0.0;
            for (int c = 0; c < 3; ++c) v += pos[3 * a + c] * inv[3 * c + ax];
            frac[3 * a + ax] = v;
            const int w = static_cast<int>(std::floor(v));
            v -= w;
            f[ax] = v;
            wfrac[3 * a + ax] = v;
            wrap[3 * a + ax] = w;
        }
        for (int c = 0; c < 3; ++c) {
            double v = 0.0;
            for (int ax = 0; ax < 3; ++ax) v += f[ax] * cell[3 * ax + c];
            wpos[3 * a + c] = v;
        }
    }
    int bins[3], reach[3];
    for (int ax = 0; ax < 3; ++ax) {
        double ins = 0.0;
        for (int c = 0; c < 3; ++c) ins += inv[3 * c + ax] * inv[3 * c + ax];
        if (!(ins > 0.0)) throw std::invalid_argument("cell must be invertible");
        const double face = 1.0 / std::sqrt(ins);
        bins[ax] = std::max(1, static_cast<int>(std::floor(face / cutoff)));
        const double rch = std::ceil(cutoff * std::sqrt(ins) * bins[ax]) + 1.0;
        reach[ax] = std::max(1, static_cast<int>(rch));
    }
    const int nb = bins[0] * bins[1] * bins[2];
    std::vector<int> abin(n), bsize(nb, 0);
    for (int a = 0; a < n; ++a) {
        const int x = std::min(bins[0] - 1, static_cast<int>(wfrac[3 * a] * bins[0]));
        const int y = std::min(bins[1] - 1, static_cast<int>(wfrac[3 * a + 1] * bins[1]));
        const int z = std::min(bins[2] - 1, static_cast<int>(wfrac[3 * a + 2] * bins[2]));
        abin[a] = (z * bins[1] + y) * bins[0] + x;
        bsize[abin[a]] += 1;
    }
    std::vector<int> boff(nb + 1, 0);
    for (int b = 0; b < nb; ++b) boff[b + 1] = boff[b] + bsize[b];
    std::vector<int> batoms(n), cur(boff.begin(), boff.end() - 1);
    for (int a = 0; a < n; ++a) batoms[cur[abin[a]]++] = a;  // ascending atom order within a bin
    const double cut2 = cutoff * cutoff;
    g.num_neigh.assign(n, 0);
    std::vector<long long> counts(n, 0);
    auto visit = [&](int rcv, bool do_fill, long long base) {
        const int rb = abin[rcv];
        const int rx = rb % bins[0], ry = (rb / bins[0]) % bins[1], rz = rb / (bins[0] * bins[1]);
        long long local = 0;
        for (int dz = -reach[2]; dz <= reach[2]; ++dz) {
            const int raw_z = rz + dz, sz = floor_div(raw_z, bins[2]), bz = raw_z - sz * bins[2];
            for (int dy = -reach[1]; dy <= reach[1]; ++dy) {
                const int raw_y = ry + dy, sy = floor_div(raw_y, bins[1]), by = raw_y - sy * bins[1];
                for (int dx = -reach[0]; dx <= reach[0]; ++dx) {
                    const int raw_x = rx + dx, sx = floor_div(raw_x, bins[0]), bx = raw_x - sx * bins[0];
                    const int sb = (bz * bins[1] + by) * bins[0] + bx;
                    const int image[3] = {sx, sy, sz};
                    for (int idx = boff[sb]; idx < boff[sb + 1]; ++idx) {
                        const int src = batoms[idx];
                        if (src == rcv && sx == 0 && sy == 0 && sz == 0) continue;
                        double d2 = 0.0;
                        for (int c = 0; c < 3; ++c) {
                            double d = wpos[3 * src + c] - wpos[3 * rcv + c];
                            for (int ax = 0; ax < 3; ++ax) d += image[ax] * cell[3 * ax + c];
                            d2 += d * d;
                        }
                        if (d2 > cut2) continue;
                        if (do_fill) {
                            const long long e = base + local;
                            g.sources[e] = src;
                            for (int ax = 0; ax < 3; ++ax) {
                                g.shifts[3 * e + ax] = image[ax] - wrap[3 * src + ax] + wrap[3 * rcv + ax];
                                g.fractional_xyz[3 * e + ax] = wfrac[3 * src + ax] - wfrac[3 * rcv + ax] + image[ax];
                            }
                        }
                        ++local;
                    }
                }
            }
        }
        return local;
    };
#pragma omp parallel for schedule(dynamic, 64)
    for (int a = 0; a < n; ++a) counts[a] = visit(a, false, 0);
    long long total = 0;
    g.offsets.assign(n + 1, 0);
    for (int a = 0; a < n; ++a) {
        g.offsets[a] = static_cast<int>(total);
        g.num_neigh[a] = static_cast<int>(counts[a]);
        total += counts[a];
        if (total > std::numeric_limits<int>::max()) throw std::length_error("edge count exceeds 32 bits");
    }
    g.offsets[n] = static_cast<int>(total);
    if (!fill) return;
    g.sources.assign(total, 0);
    g.shifts.assign(3 * total, 0);
    g.fractional_xyz.assign(3 * total, 0.0);
#pragma omp parallel for schedule(dynamic, 64)
    for (int a = 0; a < n; ++a) visit(a, true, g.offsets[a]);
}

}  // namespace oracle

// ---------------------------------------------------------------------------
// C interface (ctypes)
// ---------------------------------------------------------------------------

using namespace oracle;

struct OracleHandle {
    int fp64 = 0;
    std::unique_ptr<Mace<float>> f;
    std::unique_ptr<Mace<double>> d;
};

template <class F>
static int guarded(F&& f) {
    try {
        return f();
    } catch (const std::exception& ex) {
        oracle::last_error = ex.what();
        return -1;
    }
}

extern "C" {

const char* oracle_last_error() { return oracle::last_error.c_str(); }

void* oracle_load_head(const char* path, const char* head, int fp64) {
    try {
        auto h = std::make_unique<OracleHandle>();
        h->fp64 = fp64;
        const std::string hd = head ? head : "";
        if (fp64) { h->d = std::make_unique<Mace<double>>(); h->d->load(path, hd); }
        else { h->f = std::make_unique<Mace<float>>(); h->f->load(path, hd); }
        return h.release();
    } catch (const std::exception& ex) {
        oracle::last_error = ex.what();
        return nullptr;
    }
}

void* oracle_load(const char* path, int fp64) { return oracle_load_head(path, "", fp64); }

void oracle_free(void* h) { delete static_cast<OracleHandle*>(h); }

// info: [num_elements, C, l_max, L_max, num_lm, num_LM, num_paths, num_rows, num_lme, T_M1]
int oracle_info(void* hv, int* info, double* r_cut) {
    auto* h = static_cast<OracleHandle*>(hv);
    auto fill = [&](auto& m) {
        info[0] = m.num_elements; info[1] = m.C; info[2] = m.l_max; info[3] = m.L_max;
        info[4] = m.num_lm; info[5] = m.num_LM; info[6] = static_cast<int>(m.Phi1_l.size());
        info[7] = m.num_rows; info[8] = m.num_lme; info[9] = static_cast<int>(m.M1_monos.monos.size());
        *r_cut = m.r_cut;
    };
    if (h->fp64) fill(*h->d); else fill(*h->f);
    return 0;
}

int oracle_atomic_numbers(void* hv, int* out) {
    auto* h = static_cast<OracleHandle*>(hv);
    const auto& z = h->fp64 ? h->d->atomic_numbers : h->f->atomic_numbers;
    std::copy(z.begin(), z.end(), out);
    return 0;
}

// the electric field of the next evaluations of a MACEField model: 3 values
// (one field for the graph) or 3 per node; count 0 clears it
int oracle_set_field(void* hv, const double* field, int count) {
    return guarded([&]() -> int {
        auto* h = static_cast<OracleHandle*>(hv);
        std::vector<double> f(field, field + (count > 0 ? count : 0));
        if (h->fp64) h->d->field_in = f; else h->f->field_in = f;
        return 0;
    });
}

int oracle_evaluate(void* hv, int n, const int* types, const int* num_neigh, const int* neigh,
                    const int* neigh_types, const double* xyz, const double* r, double* energies,
                    double* forces) {
    return guarded([&]() -> int {
        auto* h = static_cast<OracleHandle*>(hv);
        long long E = 0;
        for (int i = 0; i < n; ++i) E += num_neigh[i];
        auto run = [&](auto& m) {
            m.evaluate(n, types, num_neigh, neigh, neigh_types, xyz, r);
            std::copy(m.node_energies.begin(), m.node_energies.end(), energies);
            std::copy(m.node_forces.begin(), m.node_forces.end(), forces);
        };
        if (h->fp64) run(*h->d); else run(*h->f);
        (void)E;
        return 0;
    });
}

// MACEField response of a field-coupled model in the field set by
// oracle_set_field (3 values): evaluates, then the tangents in each field
// component.  hessian[c*3 + s] = d(dE/dE_c)/dE_s; with force_derivative
// non-null, force_derivative[s][e][3] = d(directed force of e)/dE_s.
// leave out terms of the response's tangent (bit mask, see Mace::response_drop)
int oracle_set_response_drop(void* hv, int mask) {
    auto* h = static_cast<OracleHandle*>(hv);
    if (h->fp64) h->d->response_drop = mask; else h->f->response_drop = mask;
    return 0;
}

int oracle_field_response(void* hv, int n, const int* types, const int* num_neigh, const int* neigh,
                          const int* neigh_types, const double* xyz, const double* r, double* hessian,
                          double* force_derivative) {
    return guarded([&]() -> int {
        auto* h = static_cast<OracleHandle*>(hv);
        auto run = [&](auto& m) {
            m.evaluate(n, types, num_neigh, neigh, neigh_types, xyz, r);
            m.field_response(n, types, num_neigh, neigh, neigh_types, xyz, r, force_derivative != nullptr);
            std::copy(m.field_hessian.begin(), m.field_hessian.end(), hessian);
            if (force_derivative)
                std::copy(m.field_force_derivative.begin(), m.field_force_derivative.end(), force_derivative);
        };
        if (h->fp64) run(*h->d); else run(*h->f);
        return 0;
    });
}

// Stage buffers of the last evaluation, as float64: name in {Y, Ygrad, A0, M0,
// M0_grad, H1, Phi1, A1, M1, H2, H2_adj, A1_adj, dPhi1, H1_adj, M0_adj, A0_adj,
// node_forces_r1, Phi0, Phi0_adj, node_forces_r0, A0_scale, A1_scale,
// density_forces, zbl_energies, zbl_forces}.
long long oracle_stage(void* hv, const char* name, double* out, long long capacity) {
    auto* h = static_cast<OracleHandle*>(hv);
    auto get = [&](auto& m) -> long long {
        const std::string s(name);
        auto emit = [&](const auto& v) -> long long {
            if (out && static_cast<long long>(v.size()) <= capacity)
                for (std::size_t i = 0; i < v.size(); ++i) out[i] = static_cast<double>(v[i]);
            return static_cast<long long>(v.size());
        };
        if (s == "Y") return emit(m.Y);
        if (s == "Ygrad") return emit(m.Ygrad);
        if (s == "A0") return emit(m.A0);
        if (s == "M0") return emit(m.M0);
        if (s == "M0_grad") return emit(m.M0_grad);
        if (s == "H1") return emit(m.H1);
        if (s == "H1_pre") return emit(m.H1_pre);
        if (s == "H1_field") return emit(m.H1_field);
        if (s == "field_adj") return emit(m.field_adj);
        if (s == "Phi1") return emit(m.Phi1);
        if (s == "A1") return emit(m.A1);
        if (s == "M1") return emit(m.M1);
        if (s == "H2") return emit(m.H2);
        if (s == "H2_adj") return emit(m.H2_adj);
        if (s == "A1_adj") return emit(m.A1_adj);
        if (s == "dPhi1") return emit(m.dPhi1);
        if (s == "H1_adj") return emit(m.H1_adj);
        if (s == "M0_adj") return emit(m.M0_adj);
        if (s == "A0_adj") return emit(m.A0_adj);
        if (s == "node_forces_r1") return emit(m.node_forces_r1);
        if (s == "Phi0") return emit(m.Phi0);
        if (s == "Phi0_adj") return emit(m.Phi0_adj);
        if (s == "node_forces_r0") return emit(m.node_forces_r0);
        if (s == "A0_scale") return emit(m.A0_scale);
        if (s == "A1_scale") return emit(m.A1_scale);
        if (s == "density_forces") return emit(m.density_forces);
        if (s == "zbl_energies") return emit(m.zbl_energies);
        if (s == "zbl_forces") return emit(m.zbl_forces);
        return -1;
    };
    return h->fp64 ? get(*h->d) : get(*h->f);
}

// Radial nodal tables of the model on its spline grid (FP64):
// which 0 = R0, 1 = R1, 2 = A0 density, 3 = A1 density; values/derivs
// [function][point].
int oracle_radial_tables(void* hv, int which, int ti, int tj, double* values, double* derivs, int* shape) {
    return guarded([&]() -> int {
        auto* h = static_cast<OracleHandle*>(hv);
        const RadialModel& rm = h->fp64 ? h->d->radial : h->f->radial;
        if ((which == 2 && !rm.has_A0) || (which == 3 && !rm.has_A1) || which < 0 || which > 3)
            throw std::invalid_argument("the model has no such radial network");
        std::vector<std::vector<double>> v, d;
        rm.tabulate(which == 0 ? rm.R0 : which == 1 ? rm.R1 : which == 2 ? rm.A0 : rm.A1, v, d, ti, tj);
        shape[0] = static_cast<int>(v.size());
        shape[1] = rm.points;
        if (values)
            for (std::size_t f = 0; f < v.size(); ++f)
                for (int p = 0; p < rm.points; ++p) {
                    values[f * rm.points + p] = v[f][p];
                    derivs[f * rm.points + p] = d[f][p];
                }
        return 0;
    });
}

// Features [point][basis] of the pair of model types (ti, tj) (the same for
// every pair without a distance transform).
int oracle_radial_features(void* hv, int ti, int tj, double* out, int* shape) {
    return guarded([&]() -> int {
        auto* h = static_cast<OracleHandle*>(hv);
        const RadialModel& rm = h->fp64 ? h->d->radial : h->f->radial;
        const auto f = rm.features(ti, tj);
        shape[0] = rm.points;
        shape[1] = static_cast<int>(rm.bessel.size());
        if (out) std::copy(f.begin(), f.end(), out);
        return 0;
    });
}

// Spline derivative solve of arbitrary nodal values on a uniform grid of step h.
int oracle_spline_derivatives(const double* values, int points, double h, double* derivs) {
    return guarded([&]() -> int {
        RadialModel rm;
        rm.points = points;
        rm.h = h;
        const auto d = rm.spline_derivatives(std::vector<double>(values, values + points));
        std::copy(d.begin(), d.end(), derivs);
        return 0;
    });
}

// FP32 Hermite spline set evaluation (cubic_spline_set.cpp): values/derivs
// [functions][nodes] (float), evaluated at r[count] -> out_v/out_d [count][functions].
int oracle_spline_eval_f32(float h, float x0, int functions, int nodes, const float* values, const float* derivs,
                           const double* r, int count, float* out_v, float* out_d) {
    return guarded([&]() -> int {
        std::vector<std::vector<float>> v(functions), d(functions);
        for (int f = 0; f < functions; ++f) {
            v[f].assign(values + static_cast<std::size_t>(f) * nodes, values + static_cast<std::size_t>(f + 1) * nodes);
            d[f].assign(derivs + static_cast<std::size_t>(f) * nodes, derivs + static_cast<std::size_t>(f + 1) * nodes);
        }
        SplineSet<float> s(h, v, d, x0);
        for (int i = 0; i < count; ++i) {
            const auto pt = s.point(static_cast<float>(r[i]));
            const float* c = s.coefficients(pt);
            for (int f = 0; f < functions; ++f) {
                out_v[static_cast<std::size_t>(i) * functions + f] =
                    c[f] + c[functions + f] * pt.x + c[2 * functions + f] * pt.xx + c[3 * functions + f] * pt.xxx;
                out_d[static_cast<std::size_t>(i) * functions + f] =
                    c[functions + f] + 2.0f * c[2 * functions + f] * pt.x + 3.0f * c[3 * functions + f] * pt.xx;
            }
        }
        return 0;
    });
}

// Y / dY of edges (FP32, as the evaluator) from xyz[count][3].
int oracle_harmonics(const double* xyz, int count, int l_max, float* Y, float* G) {
    const int nY = (l_max + 1) * (l_max + 1);
    for (int e = 0; e < count; ++e) {
        const double rr = std::sqrt(xyz[3 * e] * xyz[3 * e] + xyz[3 * e + 1] * xyz[3 * e + 1] + xyz[3 * e + 2] * xyz[3 * e + 2]);
        float d[3];
        for (int c = 0; c < 3; ++c) d[c] = static_cast<float>(xyz[3 * e + c] / rr);
        edge_harmonics<float>(l_max, d, static_cast<float>(rr), Y + static_cast<std::size_t>(e) * nY,
                              G ? G + static_cast<std::size_t>(e) * 3 * nY : nullptr);
    }
    return 0;
}

// Polynomial with the reference's semantics (FP64): monomials flattened as
// offsets[nterms+1] into vars.  Returns f; grad[nvar].
double oracle_polynomial(int nvar, int nterms, const double* coef, const int* offsets, const int* vars,
                         const double* x, double* grad) {
    std::vector<std::vector<int>> monos(nterms);
    for (int t = 0; t < nterms; ++t) monos[t].assign(vars + offsets[t], vars + offsets[t + 1]);
    const MonomialSet ms = dedupe_monomials(monos);
    std::vector<double> c(ms.monos.size());
    for (std::size_t t = 0; t < ms.monos.size(); ++t) c[t] = coef[ms.source_index[t]];
    return poly_eval_grad<double>(ms, c.data(), x, grad, nvar);
}

// Neighbour list: count pass then fill pass.
long long oracle_neighbor_count(const double* pos, int n, const double* cell, const double* inv, double cutoff) {
    try {
        Graph g;
        build_graph(pos, n, cell, inv, cutoff, g, false);
        return g.offsets[n];
    } catch (const std::exception& ex) {
        oracle::last_error = ex.what();
        return -1;
    }
}

int oracle_neighbor_fill(const double* pos, int n, const double* cell, const double* inv, double cutoff,
                         int* num_neigh, int* offsets, int* sources, int* shifts, double* fractional_xyz) {
    return guarded([&]() -> int {
        Graph g;
        build_graph(pos, n, cell, inv, cutoff, g, true);
        std::copy(g.num_neigh.begin(), g.num_neigh.end(), num_neigh);
        std::copy(g.offsets.begin(), g.offsets.end(), offsets);
        std::copy(g.sources.begin(), g.sources.end(), sources);
        std::copy(g.shifts.begin(), g.shifts.end(), shifts);
        std::copy(g.fractional_xyz.begin(), g.fractional_xyz.end(), fractional_xyz);
        return 0;
    });
}

// Wrapped fractional positions of the neighbour list (the reference's
// periodic graph keeps them as its geometry reference,
// neighbor_graph_kokkos.cpp wrap step; lifecycle.cpp:2231-2244):
// f = pos . inv, f - floor(f).
int oracle_wrapped_fractional(const double* pos, int n, const double* inv, double* wfrac) {
    for (int a = 0; a < n; ++a)
        for (int ax = 0; ax < 3; ++ax) {
            double v = 0.0;
            for (int c = 0; c < 3; ++c) v += pos[3 * a + c] * inv[3 * c + ax];
            wfrac[3 * a + ax] = v - static_cast<int>(std::floor(v));
        }
    return 0;
}

// Prepared edge geometry of a positions call (lifecycle.cpp:2915-3079 and the
// shift form of the tiled geometry, :1860-1880).  kind 0: Cartesian
// reference positions and reference xyz per edge; 1: fractional positions and
// fractional xyz per edge; 2: Cartesian positions and integer shifts per edge.
// Per atom: reference = ref (or ref . cell), delta = pos - reference; with no
// periodic axis disp = delta, else delta in lattice coordinates, periodic
// components minus floor(f + 0.5), back to Cartesian.  Per edge: vector =
// reference edge vector + disp[src] - disp[rcv]; r = |vector| clamped to the
// cutoff with the vector scaled to it.  Returns the number of invalid edges.
int oracle_prepared_geometry(int kind, int n, long long E, const int* receivers, const int* sources,
                             const double* ref_positions, const double* ref_edges, const int* shifts,
                             const double* cell, const double* inv, const int* pbc, const double* positions,
                             double cutoff, double* xyz, double* r) {
    const bool fractional = kind == 1;
    const bool any_pbc = pbc[0] || pbc[1] || pbc[2];
    std::vector<double> disp(3 * static_cast<std::size_t>(n));
    for (int a = 0; a < n; ++a) {
        double delta[3], f[3];
        for (int c = 0; c < 3; ++c) {
            double reference = ref_positions[3 * a + c];
            if (fractional) {
                reference = 0.0;
                for (int lat = 0; lat < 3; ++lat) reference += ref_positions[3 * a + lat] * cell[3 * lat + c];
            }
            delta[c] = positions[3 * a + c] - reference;
        }
        if (!any_pbc) {
            for (int c = 0; c < 3; ++c) disp[3 * a + c] = delta[c];
            continue;
        }
        for (int lat = 0; lat < 3; ++lat) {
            f[lat] = 0.0;
            for (int c = 0; c < 3; ++c) f[lat] += delta[c] * inv[3 * c + lat];
            if (pbc[lat]) f[lat] -= std::floor(f[lat] + 0.5);
        }
        for (int c = 0; c < 3; ++c) {
            double v = 0.0;
            for (int lat = 0; lat < 3; ++lat) v += f[lat] * cell[3 * lat + c];
            disp[3 * a + c] = v;
        }
    }
    int invalid = 0;
    for (long long e = 0; e < E; ++e) {
        const int rc = receivers[e], sc = sources[e];
        double vec[3], d2 = 0.0;
        for (int c = 0; c < 3; ++c) {
            double ref;
            if (kind == 2) {
                ref = ref_positions[3 * sc + c] - ref_positions[3 * rc + c];
                for (int lat = 0; lat < 3; ++lat) ref += static_cast<double>(shifts[3 * e + lat]) * cell[3 * lat + c];
            } else if (fractional) {
                ref = 0.0;
                for (int lat = 0; lat < 3; ++lat) ref += ref_edges[3 * e + lat] * cell[3 * lat + c];
            } else {
                ref = ref_edges[3 * e + c];
            }
            vec[c] = ref + disp[3 * sc + c] - disp[3 * rc + c];
            d2 += vec[c] * vec[c];
        }
        if (!std::isfinite(d2) || !(d2 > 0.0)) {
            ++invalid;
            xyz[3 * e] = cutoff; xyz[3 * e + 1] = 0.0; xyz[3 * e + 2] = 0.0;
            r[e] = cutoff;
            continue;
        }
        const double dist = std::sqrt(d2);
        const double scale = dist >= cutoff ? cutoff / dist : 1.0;
        for (int c = 0; c < 3; ++c) xyz[3 * e + c] = scale * vec[c];
        r[e] = dist >= cutoff ? cutoff : dist;
    }
    return invalid;
}

// mace_kokkos_evaluate.cpp:49-105 (F[src] += f, F[rcv] -= f), serial order.
int oracle_reduce_forces(int n, long long E, const int* receivers, const int* sources, const double* f,
                         double* atom_forces) {
    std::fill(atom_forces, atom_forces + 3 * static_cast<std::size_t>(n), 0.0);
    for (long long e = 0; e < E; ++e)
        for (int c = 0; c < 3; ++c) {
            atom_forces[3 * sources[e] + c] += f[3 * e + c];
            atom_forces[3 * receivers[e] + c] -= f[3 * e + c];
        }
    return 0;
}

// evaluate.cpp:291 / calculator.py:3884: sigma_ab = -(1/V) sum_e f_a xyz_b.
int oracle_reduce_stress(long long E, const double* f, const double* xyz, double volume, double* stress) {
    for (int a = 0; a < 3; ++a)
        for (int b = 0; b < 3; ++b) {
            double s = 0.0;
            for (long long e = 0; e < E; ++e) s += f[3 * e + a] * xyz[3 * e + b];
            stress[3 * a + b] = -s / volume;
        }
    return 0;
}

// One ZBL pair (zbl_kokkos.cpp; the reference's symmetrix.ZBL binding):
// out = {value, dV/dr, envelope, d envelope/dr} at distance r.
int oracle_zbl(double a_exp, double a_prefactor, const double* c, const double* radii, int num_radii, int p, int Zu,
               int Zv, double r, double* out) {
    return guarded([&]() -> int {
        Zbl z;
        z.init(a_exp, a_prefactor, std::vector<double>(c, c + 4), std::vector<double>(radii, radii + num_radii), p);
        z.value_gradient(Zu, Zv, r, out[0], out[1]);
        if (Zu < 0 || Zv < 0 || Zu >= num_radii || Zv >= num_radii) throw std::out_of_range("Z out of range");
        z.envelope(r, radii[Zu] + radii[Zv], out[2], out[3]);
        return 0;
    });
}

int oracle_num_threads() { return omp_get_max_threads(); }

// OpenMP threads of later calls (the CPU baseline's 8-core comparison run)
void oracle_set_num_threads(int n) {
    if (n > 0) omp_set_num_threads(n);
}

}  // extern "C"
