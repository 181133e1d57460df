// Model loader for the MI355X evaluator (host C++; built with
// -ffp-contract=off so the FP64 radial tabulation rounds like the reference's
// host code).
//
// Reference statements followed:
//   * key set and validation: libsymmetrix/source/mace.cpp:2660-2959,
//     mace_kokkos_model.cpp:146; v4 readout basis h1_affine_schema.hpp:196-259
//   * radial features compact_radial.cpp:227-267, network evaluation
//     multilayer_perceptron.cpp:30-80 (SiLU*scale hidden, linear output),
//     spline node derivatives compact_radial.cpp:326-366 (not-a-knot left,
//     zero-slope right)
//   * Hermite coefficients cubic_spline_set.cpp:8-30, rounded to Precision
//     before the coefficient formulas are applied in Precision
//   * density networks (A0/A1 scaling): "tanh-square" postprocessing
//     compact_radial.cpp:17-24,181-193,295-303, FP64 Hermite coefficients
//     radial_function_set_kokkos.cpp:14-45 (RadialFunctionSetKokkos<double>)
//   * polynomial semantics multivariate_polynomial.cpp:11-103: a repeated
//     monomial keeps the coefficient of its first occurrence and terms are
//     ordered by (degree, lexicographic)
#include "model.hpp"

#include <algorithm>
#include <cmath>
#include <limits>
#include <map>
#include <stdexcept>

#include "coupling_rows.hpp"
#include "json_lite.hpp"
#include "model_binary.hpp"

namespace smx {
namespace {

using json_lite::Value;

float to_f32(double v) {
    if (!std::isfinite(v) || std::abs(v) > static_cast<double>(std::numeric_limits<float>::max()))
        throw std::invalid_argument("model value is outside the FP32 range");
    return static_cast<float>(v);
}

std::vector<float> to_f32(const std::vector<double>& v) {
    std::vector<float> o(v.size());
    for (std::size_t i = 0; i < v.size(); ++i) o[i] = to_f32(v[i]);
    return o;
}

using Mlp = RadialNetwork;

Mlp read_mlp(const Value& v) {
    Mlp m;
    m.shape = v.at("shape").as_ints();
    const Value& w = v.at("weights");
    for (std::size_t i = 0; i < w.size(); ++i) m.w.push_back(w.at(i).as_doubles());
    m.scale = v.at("activation_scale").as_number();
    const std::string post = v.get_string("postprocess", "");
    if (!post.empty() && post != "tanh-square")
        throw std::invalid_argument("compact radial network has unsupported postprocessing");
    m.tanh_square = post == "tanh-square";
    if (v.at("activation").as_string() != "silu")
        throw std::invalid_argument("compact radial networks must use SiLU activations");
    if (m.shape.size() < 2 || m.w.size() + 1 != m.shape.size())
        throw std::invalid_argument("compact radial network has an invalid shape");
    for (std::size_t l = 0; l < m.w.size(); ++l)
        if (m.w[l].size() != static_cast<std::size_t>(m.shape[l]) * m.shape[l + 1])
            throw std::invalid_argument("compact radial network weights do not match its shape");
    return m;
}

// multilayer_perceptron.cpp:30-80 for one input row.
void mlp_row(const Mlp& m, const double* in, std::vector<double>& out) {
    std::vector<double> cur(in, in + m.shape[0]), nxt;
    for (std::size_t l = 0; l < m.w.size(); ++l) {
        const int ni = m.shape[l], no = m.shape[l + 1];
        nxt.assign(no, 0.0);
        const double* W = m.w[l].data();
        for (int o = 0; o < no; ++o) {
            double s = 0.0;
            for (int i = 0; i < ni; ++i) s += W[static_cast<std::size_t>(o) * ni + i] * cur[i];
            nxt[o] = s;
        }
        if (l + 1 < m.w.size())
            for (int o = 0; o < no; ++o) nxt[o] = m.scale * nxt[o] / (1.0 + std::exp(-nxt[o]));
        cur.swap(nxt);
    }
    out = cur;
}

// compact_radial.cpp:326-366
std::vector<double> node_derivatives(const std::vector<double>& v, double h) {
    const int n = static_cast<int>(v.size());
    const int u = n - 2;
    std::vector<double> lo(u, 0.0), di(u, 4.0), up(u, 0.0), rhs(u, 0.0);
    const double left = 2.0 * (-v[0] + 2.0 * v[1] - v[2]) / h;
    up[0] = 2.0;
    rhs[0] = 3.0 * (v[2] - v[0]) / h - left;
    for (int node = 2; node < n - 1; ++node) {
        const int row = node - 1;
        lo[row] = 1.0;
        if (node + 1 <= n - 2) up[row] = 1.0;
        rhs[row] = 3.0 * (v[node + 1] - v[node - 1]) / h;
    }
    for (int row = 1; row < u; ++row) {
        const double f = lo[row] / di[row - 1];
        di[row] -= f * up[row - 1];
        rhs[row] -= f * rhs[row - 1];
    }
    std::vector<double> x(u, 0.0);
    x[u - 1] = rhs[u - 1] / di[u - 1];
    for (int row = u - 2; row >= 0; --row) x[row] = (rhs[row] - up[row] * x[row + 1]) / di[row];
    std::vector<double> d(n, 0.0);
    for (int node = 1; node < n - 1; ++node) d[node] = x[node - 1];
    d[0] = d[2] + left;
    d[n - 1] = 0.0;
    return d;
}

// Tabulate one network on the grid and build packed FP32 Hermite coefficients
// [interval][function][4] (cubic_spline_set.cpp:8-30 in FP32).
void tabulate(const Mlp& net, const std::vector<double>& features, int nb, int points, double h,
              std::vector<double>& values, std::vector<double>& derivs, std::vector<float>& coef) {
    const int nf = net.shape.back();
    values.assign(static_cast<std::size_t>(nf) * points, 0.0);
    derivs.assign(values.size(), 0.0);
    std::vector<double> out;
    for (int node = 0; node < points; ++node) {
        mlp_row(net, features.data() + static_cast<std::size_t>(node) * nb, out);
        for (int f = 0; f < nf; ++f) values[static_cast<std::size_t>(f) * points + node] = out[f];
    }
    std::vector<double> col(points);
    for (int f = 0; f < nf; ++f) {
        std::copy(values.begin() + static_cast<std::size_t>(f) * points,
                  values.begin() + static_cast<std::size_t>(f + 1) * points, col.begin());
        const auto d = node_derivatives(col, h);
        std::copy(d.begin(), d.end(), derivs.begin() + static_cast<std::size_t>(f) * points);
    }
    const float hf = to_f32(h);
    const int intervals = points - 1;
    coef.assign(static_cast<std::size_t>(intervals) * nf * 4, 0.0f);
    for (int i = 0; i < intervals; ++i)
        for (int f = 0; f < nf; ++f) {
            const float v0 = to_f32(values[static_cast<std::size_t>(f) * points + i]);
            const float v1 = to_f32(values[static_cast<std::size_t>(f) * points + i + 1]);
            const float d0 = to_f32(derivs[static_cast<std::size_t>(f) * points + i]);
            const float d1 = to_f32(derivs[static_cast<std::size_t>(f) * points + i + 1]);
            float* c = &coef[(static_cast<std::size_t>(i) * nf + f) * 4];
            c[0] = v0;
            c[1] = d0;
            c[2] = (-3 * v0 - 2 * hf * d0 + 3 * v1 - hf * d1) / (hf * hf);
            c[3] = (2 * v0 + hf * d0 - 2 * v1 + hf * d1) / (hf * hf * hf);
        }
}

// A density network (one output, tanh(v^2)) on the grid, as FP64 Hermite
// coefficients [interval][4] (radial_function_set_kokkos.cpp:30-41 with
// Precision = double).
std::vector<double> density_table(const Mlp& net, const std::vector<double>& features, int nb, int points,
                                  double h) {
    std::vector<double> v(points), out;
    for (int node = 0; node < points; ++node) {
        mlp_row(net, features.data() + static_cast<std::size_t>(node) * nb, out);
        v[node] = std::tanh(out[0] * out[0]);
    }
    const auto d = node_derivatives(v, h);
    std::vector<double> c(static_cast<std::size_t>(points - 1) * 4);
    for (int i = 0; i < points - 1; ++i) {
        c[4 * i] = v[i];
        c[4 * i + 1] = d[i];
        c[4 * i + 2] = (-3 * v[i] - 2 * h * d[i] + 3 * v[i + 1] - h * d[i + 1]) / (h * h);
        c[4 * i + 3] = (2 * v[i] + h * d[i] - 2 * v[i + 1] + h * d[i + 1]) / (h * h * h);
    }
    return c;
}

// Deduplicate monomials (first occurrence wins) and sort by (degree, lex).
struct Poly {
    std::vector<std::vector<int>> monos;
    std::vector<int> source;  // index of the coefficient in the file's list
};

Poly canonical_poly(const std::vector<std::vector<int>>& monos, int nvar) {
    auto less = [](const std::vector<int>& a, const std::vector<int>& b) {
        if (a.size() != b.size()) return a.size() < b.size();
        return a < b;
    };
    std::map<std::vector<int>, int, decltype(less)> first(less);
    for (std::size_t i = 0; i < monos.size(); ++i) {
        const auto& m = monos[i];
        if (m.empty() || m.size() > 3)
            throw std::invalid_argument("product-basis monomials must have degree 1 to 3");
        for (int v : m)
            if (v < 0 || v >= nvar) throw std::invalid_argument("product-basis monomial variable out of range");
        first.insert({m, static_cast<int>(i)});
    }
    Poly p;
    for (const auto& [m, i] : first) {
        p.monos.push_back(m);
        p.source.push_back(i);
    }
    return p;
}

std::vector<std::vector<int>> read_monomials(const Value& v) {
    std::vector<std::vector<int>> out;
    for (std::size_t i = 0; i < v.size(); ++i) {
        const Value& m = v.at(i);
        out.push_back(m.size() == 0 ? std::vector<int>{} : m.as_ints());
    }
    return out;
}

void transpose_blocks(const std::vector<float>& src, std::vector<float>& dst, std::size_t blocks, int rows,
                      int cols) {
    dst.assign(src.size(), 0.0f);
    for (std::size_t b = 0; b < blocks; ++b) {
        const float* s = src.data() + b * rows * cols;
        float* d = dst.data() + b * rows * cols;
        for (int r = 0; r < rows; ++r)
            for (int c = 0; c < cols; ++c) d[static_cast<std::size_t>(c) * rows + r] = s[static_cast<std::size_t>(r) * cols + c];
    }
}

void set_member(Value& obj, const std::string& key, const Value& v) {
    for (auto& m : obj.members)
        if (m.first == key) {
            m.second = v;
            return;
        }
    obj.members.emplace_back(key, v);
}

// Prediction heads (prediction_heads.hpp:10-88).  Without a
// "prediction_heads" section the file's optional "head" names its only head.
// With one, the section (schema 1) lists unique non-empty names, a default,
// and per head exactly the fields that differ between heads (atomic
// energies, both readouts, and zbl_c for ZBL models); the requested head, or
// the default, replaces those top-level fields.
void select_prediction_head(Value& j, const std::string& requested, std::string& selected,
                            std::vector<std::string>& available) {
    const Value* section = j.find("prediction_heads");
    if (!section) {
        const std::string legacy = j.get_string("head", "");
        if (!requested.empty() && requested != legacy) {
            if (legacy.empty())
                throw std::invalid_argument("the model file names no prediction head, so head '" + requested +
                                            "' cannot be selected");
            throw std::invalid_argument("prediction head '" + requested + "' is not in the model (it holds '" +
                                        legacy + "')");
        }
        selected = legacy;
        available.clear();
        if (!legacy.empty()) available.push_back(legacy);
        return;
    }
    if (!section->is_object() || section->get_int("schema_version", 0) != 1)
        throw std::invalid_argument("prediction_heads has an unsupported schema version");
    const Value* names_v = section->find("names");
    if (!names_v || !names_v->is_array()) throw std::invalid_argument("prediction_heads.names must be an array");
    std::vector<std::string> names;
    for (std::size_t i = 0; i < names_v->size(); ++i) names.push_back(names_v->at(i).as_string());
    std::vector<std::string> sorted = names;
    std::sort(sorted.begin(), sorted.end());
    if (names.empty() || std::adjacent_find(sorted.begin(), sorted.end()) != sorted.end() || sorted.front().empty())
        throw std::invalid_argument("prediction_heads.names must hold unique non-empty strings");
    const Value* params = section->find("parameters");
    if (!params || !params->is_object() || params->size() != names.size())
        throw std::invalid_argument("prediction_heads.parameters must define every named head");
    if (j.get_string("model_type", "MACE") == "MACE_Nonlinear")
        throw std::invalid_argument("MACE_Nonlinear models are not supported");
    std::vector<std::string> expected = {
        "atomic_energies",
        j.get_string("h1_affine_mode", "") == "pre_linear_up" ? "readout_1_weights_for_H1_pre_linear_up"
                                                               : "readout_1_weights_for_M0",
        "readout_2_weights_1", "readout_2_weights_2"};
    if (j.get_bool("has_zbl", false)) expected.push_back("zbl_c");
    std::sort(expected.begin(), expected.end());
    for (const auto& name : names) {
        const Value* p = params->find(name);
        if (!p || !p->is_object()) throw std::invalid_argument("prediction_heads.parameters must define every named head");
        std::vector<std::string> fields;
        for (const auto& m : p->members) fields.push_back(m.first);
        std::sort(fields.begin(), fields.end());
        if (fields != expected)
            throw std::invalid_argument("every prediction-head payload must hold exactly the per-head fields");
    }
    const std::string def = section->get_string("default", "");
    if (std::find(names.begin(), names.end(), def) == names.end())
        throw std::invalid_argument("prediction_heads.default must name a stored head");
    selected = requested.empty() ? def : requested;
    if (std::find(names.begin(), names.end(), selected) == names.end())
        throw std::invalid_argument("prediction head '" + selected + "' is not in the model");
    const Value payload = *params->find(selected);
    for (const auto& m : payload.members) set_member(j, m.first, m.second);
    Value hv;
    hv.kind = Value::String;
    hv.str = selected;
    set_member(j, "head", hv);
    available = names;
}

}  // namespace

// compact_radial.cpp:227-267: Bessel features of the pair (ti, tj) on the
// grid, at the (optionally Agnesi-transformed) distance, times the
// polynomial cutoff of the distance itself.
std::vector<double> HostModel::features(int ti, int tj) const {
    const int nb = static_cast<int>(bessel.size());
    double r0 = 1.0;
    if (agnesi) {
        if (ti < 0 || tj < 0 || ti >= num_elements || tj >= num_elements)
            throw std::out_of_range("radial pair type out of range");
        r0 = 0.5 * (covalent_radii[ti] + covalent_radii[tj]);
    }
    const double p = cutoff_p;
    std::vector<double> feat(static_cast<std::size_t>(spline_points) * nb);
    for (int node = 0; node < spline_points; ++node) {
        const double r = grid_min + node * h;
        double x = r;
        if (agnesi) {
            const double s = r / r0;
            x = 1.0 / (1.0 + agnesi_a * std::pow(s, agnesi_q) / (1.0 + std::pow(s, agnesi_q - agnesi_p)));
        }
        double cv = 0.0;
        if (r < cutoff_r_max) {
            const double s = r / cutoff_r_max;
            cv = 1.0 - ((p + 1.0) * (p + 2.0) / 2.0) * std::pow(s, cutoff_p) +
                 p * (p + 2.0) * std::pow(s, cutoff_p + 1) - (p * (p + 1.0) / 2.0) * std::pow(s, cutoff_p + 2);
        }
        for (int b = 0; b < nb; ++b)
            feat[static_cast<std::size_t>(node) * nb + b] = bessel_prefactor * std::sin(bessel[b] * x) / x * cv;
    }
    return feat;
}

// [rows][F * c_old][4] Hermite tables -> [rows][F * c_new][4], function
// f = b * c + k (b: l or path), extra channels zero
static std::vector<float> pad_function_table(const std::vector<float>& t, std::size_t rows, int blocks,
                                             int c_old, int c_new) {
    if (c_old == c_new) return t;
    std::vector<float> out(rows * blocks * c_new * 4, 0.0f);
    for (std::size_t i = 0; i < rows; ++i)
        for (int b = 0; b < blocks; ++b)
            for (int k = 0; k < c_old; ++k)
                for (int q = 0; q < 4; ++q)
                    out[((i * blocks + b) * c_new + k) * 4 + q] = t[((i * blocks + b) * c_old + k) * 4 + q];
    return out;
}

void HostModel::pair_tables(int ti, int tj, std::vector<float>& R0, std::vector<float>& R1, std::vector<double>& D0,
                            std::vector<double>& D1) const {
    const auto feat = features(ti, tj);
    const int nb = static_cast<int>(bessel.size());
    std::vector<double> v, d;
    tabulate(R0_net, feat, nb, spline_points, h, v, d, R0);
    R1.clear();
    if (!single_layer) tabulate(R1_net, feat, nb, spline_points, h, v, d, R1);
    R0 = pad_function_table(R0, spline_points - 1, l_max + 1, C_file, C);
    R1 = pad_function_table(R1, spline_points - 1, num_paths, C_file, C);
    D0.clear();
    D1.clear();
    if (A0_scaled) D0 = density_table(A0_net, feat, nb, spline_points, h);
    if (A1_scaled) D1 = density_table(A1_net, feat, nb, spline_points, h);
}

void HostModel::pad_channels(int Cp) {
    const int C0 = C;
    if (Cp == C0) return;
    if (Cp < C0) throw std::logic_error("channels can only be padded upwards");
    // [outer][C0] -> [outer][Cp]
    auto pad_rows = [&](std::vector<float>& v, std::size_t outer) {
        std::vector<float> o(outer * Cp, 0.0f);
        for (std::size_t r = 0; r < outer; ++r) std::copy_n(v.data() + r * C0, C0, o.data() + r * Cp);
        v.swap(o);
    };
    // [blocks][C0][C0] -> [blocks][Cp][Cp]
    auto pad_square = [&](std::vector<float>& v, std::size_t blocks) {
        std::vector<float> o(blocks * Cp * Cp, 0.0f);
        for (std::size_t b = 0; b < blocks; ++b)
            for (int r = 0; r < C0; ++r)
                std::copy_n(v.data() + (b * C0 + r) * C0, C0, o.data() + (b * Cp + r) * Cp);
        v.swap(o);
    };
    pad_rows(H0, num_elements);
    pad_square(A0_w, static_cast<std::size_t>(num_elements) * (l_max + 1));
    transpose_blocks(A0_w, A0_wt, static_cast<std::size_t>(num_elements) * (l_max + 1), Cp, Cp);
    pad_rows(m0_coef, static_cast<std::size_t>(num_elements) * m0_terms.size());
    pad_square(H1_w, L_max + 1);
    transpose_blocks(H1_w, H1_wt, L_max + 1, Cp, Cp);
    if (pre_linear_up) {
        pad_square(P0, 1);
        transpose_blocks(P0, P0t, 1, Cp, Cp);
    }
    if (residual) {
        pad_rows(res_H1, static_cast<std::size_t>(num_elements) * num_LM);
        pad_rows(res_x, static_cast<std::size_t>(num_elements));
    }
    if (field) {
        pad_square(P_all, L_max + 1);
        transpose_blocks(P_all, P_allt, L_max + 1, Cp, Cp);
        pad_square(U_all, L_max + 1);
        transpose_blocks(U_all, U_allt, L_max + 1, Cp, Cp);
        pad_square(field_W, field_paths.size());
        transpose_blocks(field_W, field_Wt, field_paths.size(), Cp, Cp);
        if (residual) pad_rows(res_pre, static_cast<std::size_t>(num_elements) * num_LM);
    }
    {
        // A1 per l: rows (e, k_in), columns k_out
        std::vector<std::int64_t> off(l_max + 2, 0);
        for (int l = 0; l <= l_max; ++l) off[l + 1] = off[l] + static_cast<std::int64_t>(num_e[l]) * Cp * Cp;
        std::vector<float> w(off[l_max + 1], 0.0f), wt(off[l_max + 1], 0.0f);
        for (int l = 0; l <= l_max; ++l) {
            const int K = num_e[l] * Cp;
            for (int e = 0; e < num_e[l]; ++e)
                for (int ki = 0; ki < C0; ++ki)
                    for (int ko = 0; ko < C0; ++ko) {
                        const float v = A1_w[A1_offset[l] + (static_cast<std::size_t>(e) * C0 + ki) * C0 + ko];
                        w[off[l] + (static_cast<std::size_t>(e) * Cp + ki) * Cp + ko] = v;
                        wt[off[l] + static_cast<std::size_t>(ko) * K + e * Cp + ki] = v;
                    }
        }
        A1_w.swap(w);
        A1_wt.swap(wt);
        A1_offset = off;
    }
    pad_rows(m1_coef, static_cast<std::size_t>(num_elements) * m1_terms.size());
    pad_square(H2_T, num_elements);
    transpose_blocks(H2_T, H2_Tt, num_elements, Cp, Cp);
    pad_square(H2_M1, 1);
    transpose_blocks(H2_M1, H2_M1t, 1, Cp, Cp);
    readout_q.resize(Cp, 0.0);
    {
        std::vector<double> w1(static_cast<std::size_t>(readout_hidden) * Cp, 0.0);
        for (int hdn = 0; hdn < readout_hidden; ++hdn)
            std::copy_n(readout_W1.data() + static_cast<std::size_t>(hdn) * C0, C0,
                        w1.data() + static_cast<std::size_t>(hdn) * Cp);
        readout_W1.swap(w1);
    }
    R0_coef = pad_function_table(R0_coef, spline_points - 1, l_max + 1, C0, Cp);
    R1_coef = pad_function_table(R1_coef, spline_points - 1, num_paths, C0, Cp);
    R0_functions = (l_max + 1) * Cp;
    R1_functions = num_paths * Cp;
    C = Cp;
}

// Flattened numbers of a (possibly nested) numeric array.
static std::vector<double> flat_doubles(const Value& v) {
    if (v.is_array() && !v.numeric_array && v.size() > 0 && v.at(0).is_array()) {
        std::vector<double> out;
        for (std::size_t i = 0; i < v.size(); ++i) {
            const auto r = flat_doubles(v.at(i));
            out.insert(out.end(), r.begin(), r.end());
        }
        return out;
    }
    return v.as_doubles();
}

// MACEField coupling block. The schema it must satisfy is the one
// field_coupling.hpp:60-238 and mace.cpp:2832-2860 accept; the reading below
// is organised around two rule lists:
//   * feats rules (field_feats_instructions): H1p block l_in times the field
//     (one 1o vector) into an intermediate block l_mid = l_in +- 1, a C x C
//     "uvw" weight and a real 3j tensor [2 l_in + 1][3][2 l_mid + 1];
//   * mix rules (field_linear_instructions): a C x C weight on block l.
// Every mix rule whose block is a feats rule's l_mid closes one path; its
// channel matrix is the product of the two weights times both path weights,
// formed in FP64 and rounded to FP32 once.
namespace {

[[noreturn]] void field_refuse(const std::string& what) {
    throw std::invalid_argument("field coupling: " + what);
}

struct FeatsRule {
    int l_in, l_mid;
    double scale;
    std::vector<double> w3;          // [2 l_in + 1][3][2 l_mid + 1]
    std::size_t weight_at;           // first element of its C x C weight
};

struct MixRule {
    int l;
    double scale;
    std::size_t weight_at;
};

// Files written before schema_version existed hold L_max 1 couplings with no
// tensor: the field's three components map one to one onto the m of the
// l = 1 side (the e3nn order of both), normalised by 1/sqrt(3).
std::vector<double> unversioned_tensor(int l_in, int l_mid) {
    const int din = 2 * l_in + 1, dmid = 2 * l_mid + 1;
    std::vector<double> w(static_cast<std::size_t>(din) * 3 * dmid, 0.0);
    for (int c = 0; c < 3; ++c) {
        const int m_in = l_in == 1 ? c : 0, m_mid = l_mid == 1 ? c : 0;
        w[(static_cast<std::size_t>(m_in) * 3 + c) * dmid + m_mid] = 1.0 / std::sqrt(3.0);
    }
    return w;
}

}  // namespace

void HostModel::load_field_coupling(const Value& j) {
    if (L_max != 1 && L_max != 2)
        field_refuse("MACEField models need a hidden L_max of 1 or 2, this model has " + std::to_string(L_max));
    const Value& list = j.at("field_couplings");
    if (list.size() != 1)
        field_refuse("field_couplings must hold one coupling, found " + std::to_string(list.size()));
    const Value& cp = list.at(0);
    const bool versioned = cp.contains("schema_version");
    if (versioned && cp.at("schema_version").as_int() != 1)
        field_refuse("schema_version " + std::to_string(cp.at("schema_version").as_int()) + " is unknown (1 is read)");
    if (!versioned && L_max != 1)
        field_refuse("a coupling without schema_version is readable only for L_max 1 models");

    // every irreps string is the hidden representation, except the field's own
    std::string hidden;
    for (int l = 0; l <= L_max; ++l)
        hidden += (l ? "+" : "") + std::to_string(C) + "x" + std::to_string(l) + (l % 2 ? "o" : "e");
    const std::pair<const char*, std::string> irreps[] = {
        {"field_feats_irreps_in1", hidden}, {"field_feats_irreps_in2", "1x1o"}, {"field_feats_irreps_out", hidden},
        {"field_linear_irreps_in", hidden}, {"field_linear_irreps_out", hidden}};
    for (const auto& [key, want] : irreps) {
        const std::string got = cp.at(key).as_string();
        if (got != want) field_refuse(std::string(key) + " is '" + got + "', expected '" + want + "'");
    }
    const std::size_t Cs = static_cast<std::size_t>(C), block = Cs * Cs;
    for (const char* key : {"field_feats_output_mask", "field_linear_output_mask"}) {
        const auto mask = cp.at(key).as_doubles();
        const bool all_ones = std::all_of(mask.begin(), mask.end(), [](double v) { return v == 1.0; });
        if (mask.size() != static_cast<std::size_t>(num_LM) * Cs || !all_ones)
            field_refuse(std::string(key) + " must be " + std::to_string(num_LM * C) + " ones");
    }
    if (cp.at("field_linear_bias").size() != 0) field_refuse("field_linear_bias must be empty");

    const Value* up = j.find("H1_linear_up_weights");
    const Value* prod = j.find("H1_product_weights");
    if (!up || !prod) field_refuse("the model must split H1 into H1_product_weights and H1_linear_up_weights");
    const auto U = up->as_doubles();
    const auto P = prod->as_doubles();
    if (U.size() != static_cast<std::size_t>(L_max + 1) * block || P.size() != U.size())
        field_refuse("H1_product_weights and H1_linear_up_weights must each hold L_max + 1 blocks of C x C");

    // mix rules: one C x C block per rule, in file order
    const Value& mix_list = cp.at("field_linear_instructions");
    const auto mix_weights = flat_doubles(cp.at("field_linear_weight"));
    std::vector<MixRule> mix;
    for (std::size_t i = 0; i < mix_list.size(); ++i) {
        const Value& ins = mix_list.at(i);
        const std::string where = "field_linear_instructions[" + std::to_string(i) + "]";
        if (ins.at("path_shape").as_ints() != std::vector<int>{C, C})
            field_refuse(where + " must have path_shape [C, C]");
        const int a = ins.at("i_in").as_int(), b = ins.at("i_out").as_int();
        if (a != b || a < 0 || a > L_max) field_refuse(where + " must map a hidden block 0..L_max onto itself");
        mix.push_back({a, ins.at("path_weight").as_number(), i * block});
    }
    if (mix_weights.size() != mix.size() * block)
        field_refuse("field_linear_weight holds " + std::to_string(mix_weights.size()) + " numbers, its rules need " +
                     std::to_string(mix.size() * block));

    // feats rules: an adjacent-rank coupling of H1p with the field vector
    const Value& feats_list = cp.at("field_feats_instructions");
    const auto feats_weights = flat_doubles(cp.at("field_feats_weight"));
    std::vector<FeatsRule> feats;
    for (std::size_t i = 0; i < feats_list.size(); ++i) {
        const Value& ins = feats_list.at(i);
        const std::string where = "field_feats_instructions[" + std::to_string(i) + "]";
        if (ins.at("connection_mode").as_string() != "uvw" ||
            ins.at("path_shape").as_ints() != std::vector<int>{C, 1, C})
            field_refuse(where + " must be a 'uvw' rule of path_shape [C, 1, C]");
        FeatsRule r{ins.at("i_in1").as_int(), ins.at("i_out").as_int(), ins.at("path_weight").as_number(), {},
                    i * block};
        if (ins.at("i_in2").as_int() != 0 || r.l_in < 0 || r.l_in > L_max || r.l_mid < 0 || r.l_mid > L_max ||
            (r.l_mid != r.l_in + 1 && r.l_mid != r.l_in - 1))
            field_refuse(where + " must couple hidden block l with the field into block l +- 1");
        const std::size_t n3 = static_cast<std::size_t>(2 * r.l_in + 1) * 3 * (2 * r.l_mid + 1);
        if (versioned) {
            if (ins.at("wigner_3j_shape").as_ints() != std::vector<int>{2 * r.l_in + 1, 3, 2 * r.l_mid + 1})
                field_refuse(where + " has a wigner_3j_shape that is not [2 l_in + 1, 3, 2 l_out + 1]");
            r.w3 = ins.at("wigner_3j").as_doubles();
            if (r.w3.size() != n3) field_refuse(where + " has " + std::to_string(r.w3.size()) + " wigner_3j numbers, "
                                                "its shape needs " + std::to_string(n3));
        } else {
            r.w3 = unversioned_tensor(r.l_in, r.l_mid);
        }
        feats.push_back(std::move(r));
    }
    if (feats_weights.size() != feats.size() * block)
        field_refuse("field_feats_weight holds " + std::to_string(feats_weights.size()) + " numbers, its rules need " +
                     std::to_string(feats.size() * block));

    P_all = to_f32(P);
    U_all = to_f32(U);
    transpose_blocks(P_all, P_allt, L_max + 1, C, C);
    transpose_blocks(U_all, U_allt, L_max + 1, C, C);
    field_paths.clear();
    field_entries.clear();
    field_W.clear();
    std::vector<double> row(Cs);
    for (std::size_t fi = 0; fi < feats.size(); ++fi) {
        const FeatsRule& f = feats[fi];
        double largest = 0.0;
        for (double w : f.w3) largest = std::max(largest, std::abs(w));
        bool closed = false;
        for (const MixRule& m : mix) {
            if (m.l != f.l_mid) continue;
            closed = true;
            const int path = static_cast<int>(field_paths.size());
            field_paths.push_back({f.l_in, m.l});
            // angular entries: the tensor's nonzeros (round-off below 1e-12 of
            // its largest entry dropped), in (m_in, component, m_out) order
            const int din = 2 * f.l_in + 1, dmid = 2 * f.l_mid + 1;
            for (int mi = 0; mi < din; ++mi)
                for (int c = 0; c < 3; ++c)
                    for (int mo = 0; mo < dmid; ++mo) {
                        const double w = f.w3[(static_cast<std::size_t>(mi) * 3 + c) * dmid + mo];
                        if (std::abs(w) > 1e-12 * largest)
                            field_entries.push_back({f.l_in * f.l_in + mi, c, m.l * m.l + mo, path, to_f32(w)});
                    }
            // channel matrix, one input channel's row at a time
            const double scale = f.scale * m.scale;
            const double* wf = feats_weights.data() + f.weight_at;
            const double* wl = mix_weights.data() + m.weight_at;
            for (std::size_t in = 0; in < Cs; ++in) {
                std::fill(row.begin(), row.end(), 0.0);
                for (std::size_t mid = 0; mid < Cs; ++mid) {
                    const double a = wf[in * Cs + mid];
                    for (std::size_t out = 0; out < Cs; ++out) row[out] += a * wl[mid * Cs + out];
                }
                for (std::size_t out = 0; out < Cs; ++out) field_W.push_back(to_f32(scale * row[out]));
            }
        }
        if (!closed)
            field_refuse("field_feats_instructions[" + std::to_string(fi) + "] ends in block " +
                         std::to_string(f.l_mid) + ", which no field_linear rule reads");
    }
    if (field_paths.empty()) field_refuse("no field path is defined");
    transpose_blocks(field_W, field_Wt, field_paths.size(), C, C);
    if (residual) res_pre = to_f32(j.at("H1_first_residual_weights").as_doubles());
}

void HostModel::load(const std::string& path, const std::string& head) {
    Value j = json_lite::parse_model_file(path);
    // the nonlinear family has its own evaluator (the pair style refuses it,
    // as pair_symmetrix_mace_kokkos.cpp:419-420 does)
    if (j.is_object() && j.get_string("model_type", "MACE") == "MACE_Nonlinear")
        throw std::invalid_argument("MACE_Nonlinear models are not supported by this evaluator; load them with "
                                    "smx_mh1_create (MACENonlinearKokkosFloat)");
    if (j.get_int("symmetrix_format_version", 1) != 4)
        throw std::invalid_argument("only Symmetrix MACE model format version 4 is supported");
    select_prediction_head(j, head, selected_head, available_heads);
    // h1_affine_schema.hpp:196-259: the two v4 bases, each with its own
    // readout_1 / skip keys; a first-interaction residual needs pre_linear_up
    const std::string h1_mode = j.get_string("h1_affine_mode", "");
    if (h1_mode != "m0_composite" && h1_mode != "pre_linear_up")
        throw std::invalid_argument("Symmetrix MACE format version 4 requires h1_affine_mode 'm0_composite' or "
                                    "'pre_linear_up'");
    pre_linear_up = h1_mode == "pre_linear_up";
    const char* readout_key = pre_linear_up ? "readout_1_weights_for_H1_pre_linear_up" : "readout_1_weights_for_M0";
    const char* skip_key = pre_linear_up ? "H2_weights_for_H1_pre_linear_up" : "H2_weights_for_M0";
    if (j.contains(pre_linear_up ? "readout_1_weights_for_M0" : "readout_1_weights_for_H1_pre_linear_up") ||
        j.contains(pre_linear_up ? "H2_weights_for_M0" : "H2_weights_for_H1_pre_linear_up"))
        throw std::invalid_argument(std::string("a '") + h1_mode + "' MACE JSON must not hold the other basis's "
                                    "readout_1 or H2 skip weights");
    residual = j.get_bool("first_interaction_residual", false);
    // a one-interaction model keeps the m0_composite basis, residual or not
    // (h1_affine_schema.hpp:227-237)
    single_layer = j.get_bool("single_layer_readout", false);
    if (residual && !pre_linear_up && !single_layer)
        throw std::invalid_argument("The m0_composite basis cannot represent first-interaction residual features; "
                                    "such models use h1_affine_mode 'pre_linear_up'.");
    if (pre_linear_up && single_layer)
        throw std::invalid_argument("The pre_linear_up basis applies to two-interaction models only.");
    field = j.get_bool("has_field_coupling", false);
    {
        const std::string mt = j.get_string("model_type", "MACE");
        if (mt != "MACE" && mt != "MACEField")
            throw std::invalid_argument("Format version 4 is the standard MACE / MACEField format.");
    }
    if (field && !pre_linear_up)
        throw std::invalid_argument("The m0_composite basis cannot represent field-coupled features; such models "
                                    "use h1_affine_mode 'pre_linear_up'.");
    if (j.get_string("radial_representation", "") != "compact")
        throw std::invalid_argument("only the compact radial representation is supported");
    // mace_kokkos_model.cpp:200 (required key), :1109 (optional key)
    A0_scaled = j.at("A0_scaled").as_bool();
    A1_scaled = j.get_bool("A1_scaled", false);
    num_interactions = j.get_int("num_interactions", 2);
    if (num_interactions != (single_layer ? 1 : 2))
        throw std::invalid_argument("MACE interaction count and single-layer readout metadata disagree.");
    if (single_layer && A1_scaled) throw std::invalid_argument("a one-interaction model has no A1 to scale");
    num_elements = j.at("num_elements").as_int();
    C = j.at("num_channels").as_int();
    C_file = C;
    r_cut = j.at("r_cut").as_number();
    l_max = j.at("l_max").as_int();
    L_max = j.at("L_max").as_int();
    if (num_elements < 1 || C < 1 || !(r_cut > 0.0) || l_max < 0 || l_max > 3 || L_max < 0 || L_max > l_max)
        throw std::invalid_argument("model shape is invalid (l_max must be <= 3 and L_max <= l_max)");
    num_lm = (l_max + 1) * (l_max + 1);
    num_LM = (L_max + 1) * (L_max + 1);
    atomic_numbers = j.at("atomic_numbers").as_ints();
    atomic_energies = j.at("atomic_energies").as_doubles();
    if (static_cast<int>(atomic_numbers.size()) != num_elements ||
        static_cast<int>(atomic_energies.size()) != num_elements)
        throw std::invalid_argument("atomic numbers/energies do not match num_elements");
    // ZBL (mace_kokkos_model.cpp:191-198; constructor checks and per-pair
    // constants zbl_kokkos.cpp:11-56, here per pair of the model's types)
    has_zbl = j.at("has_zbl").as_bool();
    if (has_zbl) {
        const double a_exp = j.at("zbl_a_exp").as_number(), a_prefactor = j.at("zbl_a_prefactor").as_number();
        const auto c = j.at("zbl_c").as_doubles();
        const auto radii = j.at("zbl_covalent_radii").as_doubles();
        zbl_p = j.at("zbl_p").as_int();
        if (c.size() != 4) throw std::invalid_argument("ZBL requires four screening coefficients");
        if (radii.empty()) throw std::invalid_argument("ZBL requires at least one covalent radius");
        if (!(a_prefactor > 0.0)) throw std::invalid_argument("ZBL screening prefactor must be positive");
        if (zbl_p < 1) throw std::invalid_argument("ZBL envelope power must be positive");
        for (int k = 0; k < 4; ++k) zbl_c[k] = c[k];
        zbl_pair.assign(static_cast<std::size_t>(num_elements) * num_elements * 3, 0.0);
        for (int u = 0; u < num_elements; ++u)
            for (int v = 0; v < num_elements; ++v) {
                const int Zu = atomic_numbers[u], Zv = atomic_numbers[v];
                if (Zu < 0 || Zv < 0 || Zu >= static_cast<int>(radii.size()) || Zv >= static_cast<int>(radii.size()))
                    throw std::invalid_argument("ZBL covalent radii do not cover the model's atomic numbers");
                double* pc = &zbl_pair[(static_cast<std::size_t>(u) * num_elements + v) * 3];
                pc[0] = (std::pow(static_cast<double>(Zu), a_exp) + std::pow(static_cast<double>(Zv), a_exp)) /
                        (a_prefactor * 0.529);
                pc[1] = 14.3996 * static_cast<double>(Zu * Zv);
                pc[2] = radii[Zu] + radii[Zv];
            }
    }
    const std::size_t Cs = static_cast<std::size_t>(C);

    // ---- compact radial
    const Value& cr = j.at("compact_radial");
    grid_min = cr.at("spline_grid_min").as_number();
    spline_points = cr.at("num_spline_points").as_int();
    if (!(grid_min > 0.0) || spline_points < 4)
        throw std::invalid_argument("compact radial spline grid is invalid");
    h = (r_cut - grid_min) / (spline_points - 1);
    grid_min_f = to_f32(grid_min);
    h_f = to_f32(h);
    const Value& basis = cr.at("basis");
    if (basis.at("type").as_string() != "bessel")
        throw std::invalid_argument("only the Bessel radial basis is supported");
    const auto bessel = basis.at("weights").as_doubles();
    const double prefactor = basis.at("prefactor").as_number();
    const Value& cut = cr.at("cutoff");
    if (cut.at("type").as_string() != "polynomial")
        throw std::invalid_argument("only the polynomial radial cutoff is supported");
    const double r_max = cut.at("r_max").as_number();
    const int p = cut.at("p").as_int();
    if (std::abs(r_max - r_cut) > 1e-12) throw std::invalid_argument("compact radial cutoff does not match r_cut");
    // Without a distance transform the features, hence every pair's tables,
    // are independent of the pair (compact_radial.cpp:233-235): one table
    // serves all pairs exactly.  The Agnesi transform (compact_radial.cpp:
    // 144-163) makes them depend on the pair's mean covalent radius.
    const Value& tr = cr.at("distance_transform");
    const std::string transform = tr.at("type").as_string();
    agnesi = transform == "agnesi";
    if (agnesi) {
        agnesi_a = tr.at("a").as_number();
        agnesi_q = tr.at("q").as_number();
        agnesi_p = tr.at("p").as_number();
        covalent_radii = tr.at("covalent_radii").as_doubles();
        if (static_cast<int>(covalent_radii.size()) != num_elements)
            throw std::invalid_argument("agnesi covalent radii do not match the model's elements");
        for (double v : covalent_radii)
            if (!std::isfinite(v) || !(v > 0.0)) throw std::invalid_argument("agnesi covalent radii must be positive");
        if (!std::isfinite(agnesi_a) || !std::isfinite(agnesi_q) || !std::isfinite(agnesi_p))
            throw std::invalid_argument("agnesi transform parameters must be finite");
    } else if (transform != "none") {
        throw std::invalid_argument("only the 'none' and 'agnesi' distance transforms are supported");
    }
    const Value& nets = cr.at("networks");
    const Mlp R0net = read_mlp(nets.at("R0"));
    // mace.cpp:2769-2772: the R1 network is there iff there is a second interaction
    if (nets.contains("R1") == single_layer)
        throw std::invalid_argument("Compact radial R1 network does not match the MACE interaction count.");
    const Mlp R1net = single_layer ? Mlp{} : read_mlp(nets.at("R1"));
    const int nb = static_cast<int>(bessel.size());
    if (R0net.shape[0] != nb || (!single_layer && R1net.shape[0] != nb))
        throw std::invalid_argument("radial networks do not take the Bessel features");
    if (R0net.tanh_square || R1net.tanh_square)
        throw std::invalid_argument("compact radial R0/R1 networks cannot use postprocessing");
    // density networks (compact_radial.cpp:181-193; mace_kokkos_model.cpp:215-216,1122-1123)
    Mlp A0net, A1net;
    auto density_net = [&](const char* name, bool scaled, Mlp& net) {
        if (nets.contains(name) != scaled)
            throw std::invalid_argument(std::string("compact radial ") + name + " network does not match " + name +
                                        "_scaled");
        if (!scaled) return;
        net = read_mlp(nets.at(name));
        if (net.shape.front() != nb || net.shape.back() != 1 || !net.tanh_square)
            throw std::invalid_argument(std::string("compact radial ") + name +
                                        " network has an invalid shape or postprocessing");
    };
    density_net("A0", A0_scaled, A0net);
    density_net("A1", A1_scaled, A1net);
    this->bessel = bessel;
    bessel_prefactor = prefactor;
    cutoff_r_max = r_max;
    cutoff_p = p;
    R0_net = R0net;
    R1_net = R1net;
    A0_net = A0net;
    A1_net = A1net;
    R0_functions = R0net.shape.back();
    R1_functions = single_layer ? 0 : R1net.shape.back();
    if (R0_functions != (l_max + 1) * C) throw std::invalid_argument("R0 network width must be (l_max+1)*C");
    const auto feat = features(0, 0);
    tabulate(R0net, feat, nb, spline_points, h, R0_values, R0_derivs, R0_coef);
    if (!single_layer) tabulate(R1net, feat, nb, spline_points, h, R1_values, R1_derivs, R1_coef);
    if (A0_scaled) A0_density = density_table(A0net, feat, nb, spline_points, h);
    if (A1_scaled) A1_density = density_table(A1net, feat, nb, spline_points, h);

    // ---- H0, A0
    H0 = to_f32(j.at("H0_weights").as_doubles());
    if (H0.size() != num_elements * Cs) throw std::invalid_argument("H0 weights have the wrong size");
    const Value& a0 = j.at("A0_weights");
    A0_w.assign(num_elements * (l_max + 1) * Cs * Cs, 0.0f);
    for (int t = 0; t < num_elements; ++t)
        for (int l = 0; l <= l_max; ++l) {
            const auto w = a0.at(t).at(l).as_doubles();
            if (w.size() != Cs * Cs) throw std::invalid_argument("A0 weights have the wrong size");
            for (std::size_t i = 0; i < w.size(); ++i)
                A0_w[(static_cast<std::size_t>(t) * (l_max + 1) + l) * Cs * Cs + i] = to_f32(w[i]);
        }
    transpose_blocks(A0_w, A0_wt, static_cast<std::size_t>(num_elements) * (l_max + 1), C, C);

    // ---- M0
    const Value& m0m = j.at("M0_monomials");
    const Value& m0w = j.at("M0_weights");
    m0_term_offset.assign(num_LM + 1, 0);
    std::vector<Poly> polys;
    for (int LM = 0; LM < num_LM; ++LM) {
        const auto monos = read_monomials(m0m.at(std::to_string(LM)));
        polys.push_back(canonical_poly(monos, num_lm));
        for (const auto& m : polys.back().monos) m0_terms.push_back(pack_monomial(m));
        m0_term_offset[LM + 1] = static_cast<int>(m0_terms.size());
    }
    const std::size_t T0 = m0_terms.size();
    m0_coef.assign(num_elements * T0 * Cs, 0.0f);
    for (int t = 0; t < num_elements; ++t) {
        const Value& wt = m0w.at(std::to_string(t));
        for (int LM = 0; LM < num_LM; ++LM) {
            const Value& wl = wt.at(std::to_string(LM));
            const Poly& P = polys[LM];
            for (int k = 0; k < C; ++k) {
                const auto cf = wl.at(std::to_string(k)).as_doubles();
                if (cf.size() != m0m.at(std::to_string(LM)).size())
                    throw std::invalid_argument("M0 coefficient count does not match its monomials");
                for (std::size_t s = 0; s < P.monos.size(); ++s)
                    m0_coef[(static_cast<std::size_t>(t) * T0 + m0_term_offset[LM] + s) * Cs + k] = to_f32(cf[P.source[s]]);
            }
        }
    }

    // ---- H1
    H1_w = to_f32(j.at("H1_weights").as_doubles());
    if (H1_w.size() != static_cast<std::size_t>(L_max + 1) * Cs * Cs)
        throw std::invalid_argument("H1 weights have the wrong size");
    transpose_blocks(H1_w, H1_wt, L_max + 1, C, C);
    if (pre_linear_up) {
        const Value* pw = j.find("H1_product_weights");
        if (!pw) throw std::invalid_argument("The pre_linear_up basis requires H1_product_weights.");
        const auto P = pw->as_doubles();
        if (P.size() != H1_w.size())
            throw std::invalid_argument("The pre_linear_up basis requires H1_product_weights of the H1_weights extent.");
        P0 = to_f32(std::vector<double>(P.begin(), P.begin() + Cs * Cs));
        transpose_blocks(P0, P0t, 1, C, C);
    }
    if (residual) {
        // fused[a][lm][out] = sum_in residual[a][lm][in] U_l[in][out]
        // (mace.cpp:2809-2822; summed in FP64, rounded once)
        const Value* uw = j.find("H1_linear_up_weights");
        const Value* rw = j.find("H1_first_residual_weights");
        if (!uw || !rw) throw std::invalid_argument("Residual-first MACE JSON requires split H1 weights.");
        const auto U = uw->as_doubles();
        const auto b = rw->as_doubles();
        if (U.size() != H1_w.size()) throw std::invalid_argument("Residual-first MACE JSON requires split H1 weights.");
        if (b.size() != static_cast<std::size_t>(num_elements) * num_LM * Cs)
            throw std::invalid_argument("Residual-first MACE JSON has an invalid H1 residual extent.");
        res_H1.assign(b.size(), 0.0f);
        res_x.assign(static_cast<std::size_t>(num_elements) * Cs, 0.0f);
        for (int a = 0; a < num_elements; ++a) {
            for (int l = 0; l <= L_max; ++l)
                for (int m = 0; m < 2 * l + 1; ++m) {
                    const std::size_t row = static_cast<std::size_t>(a) * num_LM + l * l + m;
                    for (int out = 0; out < C; ++out) {
                        double s = 0.0;
                        for (int in = 0; in < C; ++in)
                            s += b[row * Cs + in] * U[(static_cast<std::size_t>(l) * Cs + in) * Cs + out];
                        res_H1[row * Cs + out] = to_f32(s);
                    }
                }
            for (int k = 0; k < C; ++k)
                res_x[static_cast<std::size_t>(a) * Cs + k] = to_f32(b[static_cast<std::size_t>(a) * num_LM * Cs + k]);
        }
    } else if (j.contains("H1_first_residual_weights")) {
        throw std::invalid_argument("Non-residual MACE JSON must not contain H1 residual weights.");
    }
    if (field) load_field_coupling(j);

    // ---- R1 coupling (extract_mace_data.py:1326-1400 semantics); a
    // one-interaction model has none (its Phi1 lists are empty or absent,
    // extract_mace_data.py:1242-1248)
    if (!single_layer) {
        path_lo = j.at("Phi1_l").as_ints();
        path_le = j.at("Phi1_l1").as_ints();
        path_ls = j.at("Phi1_l2").as_ints();
    }
    num_paths = static_cast<int>(path_lo.size());
    if ((num_paths == 0 && !single_layer) || path_le.size() != path_lo.size() || path_ls.size() != path_lo.size())
        throw std::invalid_argument("R1 path lists are inconsistent");
    if (R1_functions != num_paths * C) throw std::invalid_argument("R1 network width must be num_paths*C");
    num_e.assign(l_max + 1, 0);
    for (int p2 = 0; p2 < num_paths; ++p2) {
        if (path_lo[p2] < 0 || path_lo[p2] > l_max || path_le[p2] < 0 || path_le[p2] > l_max || path_ls[p2] < 0 ||
            path_ls[p2] > L_max)
            throw std::invalid_argument("R1 path irreps are out of range");
        num_e[path_lo[p2]] += 1;
    }
    lme_base.assign(l_max + 2, 0);
    for (int l = 0; l <= l_max; ++l) lme_base[l + 1] = lme_base[l] + (2 * l + 1) * num_e[l];
    num_lme = lme_base[l_max + 1];
    row_base.assign(num_paths + 1, 0);
    cg_offset.assign(num_paths + 1, 0);
    for (int q = 0; q < num_paths; ++q) {
        row_base[q + 1] = row_base[q] + (2 * path_le[q] + 1) * (2 * path_ls[q] + 1);
        cg_offset[q + 1] = cg_offset[q] + (2 * path_le[q] + 1) * (2 * path_ls[q] + 1) * (2 * path_lo[q] + 1);
    }
    num_rows = row_base[num_paths];
    cg_dense.assign(cg_offset[num_paths], 0.0f);
    if (!single_layer) {
        const auto lme = j.at("Phi1_lme").as_ints();
        const auto row = j.at("Phi1_lelm1lm2").as_ints();
        const auto cg = j.at("Phi1_clebsch_gordan").as_doubles();
        if (lme.size() != row.size() || cg.size() != row.size())
            throw std::invalid_argument("R1 coupling term lists are inconsistent");
        // position of path q's e index among paths with the same output l
        std::vector<int> e_of(num_paths, 0);
        std::vector<int> seen(l_max + 1, 0);
        for (int q = 0; q < num_paths; ++q) e_of[q] = seen[path_lo[q]]++;
        for (std::size_t t = 0; t < row.size(); ++t) {
            if (row[t] < 0 || row[t] >= num_rows) throw std::invalid_argument("R1 coupling row out of range");
            int q = 0;
            while (row_base[q + 1] <= row[t]) ++q;
            const int local = row[t] - row_base[q];
            const int ls = path_ls[q], lo = path_lo[q];
            const int m1 = local / (2 * ls + 1), m2 = local % (2 * ls + 1);
            // lme = lme_base[lo] + mo*num_e[lo] + e
            const int rel = lme[t] - lme_base[lo];
            if (rel < 0 || rel >= (2 * lo + 1) * num_e[lo] || rel % num_e[lo] != e_of[q])
                throw std::invalid_argument("R1 coupling output index does not match its path");
            const int mo = rel / num_e[lo];
            // the R1 kernels hold only rows with real-basis 3j coefficients
            // (coupling_rows.hpp); a term anywhere else has no kernel
            if (cg[t] != 0.0 && (path_le[q] > kCouplingLMax || ls > kCouplingLMax || lo > kCouplingLMax ||
                                 !coupling_live(path_le[q], ls, lo, m1, m2)))
                throw std::domain_error("the model's R1 coupling has a term in a row whose real-basis 3j "
                                        "coefficients are zero; no compiled kernel holds that row");
            float& dst = cg_dense[cg_offset[q] + ((m1 * (2 * ls + 1) + m2) * (2 * lo + 1) + mo)];
            // repeated (row, lme) terms accumulate like the reference's term loop
            dst = to_f32(static_cast<double>(dst) + cg[t]);
        }
    }

    // ---- A1 (none with one interaction: num_e is all zero)
    A1_offset.assign(l_max + 2, 0);
    for (int l = 0; l <= l_max; ++l) A1_offset[l + 1] = A1_offset[l] + static_cast<std::int64_t>(num_e[l]) * Cs * Cs;
    A1_w.assign(A1_offset[l_max + 1], 0.0f);
    A1_wt.assign(A1_offset[l_max + 1], 0.0f);
    for (int l = 0; l <= l_max && !single_layer; ++l) {
        const auto w = j.at("A1_weights").at(l).as_doubles();
        if (w.size() != static_cast<std::size_t>(num_e[l]) * Cs * Cs)
            throw std::invalid_argument("A1 weights have the wrong size");
        const int K = num_e[l] * C;
        for (int r = 0; r < K; ++r)
            for (int c = 0; c < C; ++c) {
                const float v = to_f32(w[static_cast<std::size_t>(r) * Cs + c]);
                A1_w[A1_offset[l] + static_cast<std::size_t>(r) * Cs + c] = v;
                A1_wt[A1_offset[l] + static_cast<std::size_t>(c) * K + r] = v;
            }
    }

    // ---- M1
    {
        // variables: A1's num_lm components, or H1's num_LM with one interaction
        const auto monos = read_monomials(j.at("M1_monomials"));
        const Poly P = canonical_poly(monos, single_layer ? num_LM : num_lm);
        for (const auto& m : P.monos) m1_terms.push_back(pack_monomial(m));
        const std::size_t T1 = m1_terms.size();
        m1_coef.assign(num_elements * T1 * Cs, 0.0f);
        const Value& m1w = j.at("M1_weights");
        for (int t = 0; t < num_elements; ++t)
            for (int k = 0; k < C; ++k) {
                const auto cf = m1w.at(std::to_string(t)).at(std::to_string(k)).as_doubles();
                if (cf.size() != monos.size()) throw std::invalid_argument("M1 coefficient count does not match");
                for (std::size_t s = 0; s < T1; ++s)
                    m1_coef[(static_cast<std::size_t>(t) * T1 + s) * Cs + k] = to_f32(cf[P.source[s]]);
            }
    }

    // ---- H2 and readouts (mace.cpp:2516-2657, v4 m0_composite basis)
    {
        const Value& t2 = j.at(skip_key);
        H2_T.assign(num_elements * Cs * Cs, 0.0f);
        for (int t = 0; t < num_elements; ++t) {
            const auto w = t2.at(t).as_doubles();
            if (w.size() != Cs * Cs) throw std::invalid_argument("H2 weights have the wrong size");
            for (std::size_t i = 0; i < w.size(); ++i) H2_T[t * Cs * Cs + i] = to_f32(w[i]);
        }
        transpose_blocks(H2_T, H2_Tt, num_elements, C, C);
        H2_M1 = to_f32(j.at("H2_weights_for_M1").as_doubles());
        if (H2_M1.size() != Cs * Cs) throw std::invalid_argument("H2 M1 weights have the wrong size");
        transpose_blocks(H2_M1, H2_M1t, 1, C, C);
        readout_q = j.at(readout_key).as_doubles();
        readout_hidden = j.get_int("readout_2_hidden_size", 16);
        readout_W1 = j.at("readout_2_weights_1").as_doubles();
        readout_W2 = j.at("readout_2_weights_2").as_doubles();
        readout_scale = j.at("readout_2_scale_factor").as_number();
        if (readout_q.size() != Cs || readout_hidden < 1 ||
            readout_W1.size() != static_cast<std::size_t>(readout_hidden) * Cs ||
            readout_W2.size() != static_cast<std::size_t>(readout_hidden))
            throw std::invalid_argument("readout weights do not match the model shape");
    }
}

void convert_model_file(const std::string& source, const std::string& destination, const std::string& format) {
    if (format != "binary" && format != "json")
        throw std::invalid_argument("model file format must be 'binary' or 'json'");
    if (source == destination) throw std::invalid_argument("source and destination must differ");
    const Value doc = json_lite::parse_model_file(source);
    if (!doc.is_object() || doc.get_int("symmetrix_format_version", 1) != 4)
        throw std::invalid_argument("'" + source + "' is not a Symmetrix model file of format version 4");
    if (format == "binary")
        json_lite::write_binary_file(doc, destination);
    else
        json_lite::write_json_file(doc, destination);
}

}  // namespace smx
