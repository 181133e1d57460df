// Host-side MACE model (Symmetrix JSON format version 4) laid out for the
// MI355X kernels.
//
// The loader reads the keys of libsymmetrix/source/mace.cpp:2660-2959 and
// mace_kokkos_model.cpp:146 for the compact-radial, "m0_composite" MACE path,
// tabulates the radial networks on the spline grid exactly as
// compact_radial.cpp:227-366 does (FP64, no contraction), and rounds the
// Hermite coefficients to FP32 with cubic_spline_set.cpp:8-30's formulas.
// Every table is stored in the layout its kernel reads coalesced: channel
// index innermost, Hermite coefficients packed four to a lane.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace json_lite {
struct Value;
}

namespace smx {

// One packed monomial: variables v0,v1,v2 (byte each) and degree (top byte).
inline std::int32_t pack_monomial(const std::vector<int>& vars) {
    std::int32_t p = static_cast<std::int32_t>(vars.size()) << 24;
    for (std::size_t i = 0; i < vars.size(); ++i) p |= (vars[i] & 0xff) << (8 * i);
    return p;
}

// One compact-radial network (multilayer_perceptron.cpp: scaled SiLU hidden
// layers, linear output; "tanh-square" postprocessing for density networks).
struct RadialNetwork {
    std::vector<int> shape;
    std::vector<std::vector<double>> w;  // [layer][out*in]
    double scale = 1.0;
    bool tanh_square = false;
};

struct HostModel {
    // shape (C: the channel count the tables are laid out for -- the file's
    // own, or the kernels' padded count after pad_channels; C_file: the file's)
    int num_elements = 0;
    int C = 0;
    int C_file = 0;
    int l_max = 0, L_max = 0;
    int num_lm = 0, num_LM = 0;
    int num_interactions = 2;
    double r_cut = 0.0;
    // prediction head in use and the heads the file stores
    std::string selected_head;
    std::vector<std::string> available_heads;
    std::vector<int> atomic_numbers;
    std::vector<double> atomic_energies;

    // radial spline grid shared by R0 and R1 (compact_radial.cpp:110-214)
    int spline_points = 0;
    double grid_min = 0.0, h = 0.0;
    float grid_min_f = 0.0f, h_f = 0.0f;
    int R0_functions = 0, R1_functions = 0;
    // [interval][function][4] with function = l*C+k (R0) or p*C+k (R1)
    std::vector<float> R0_coef, R1_coef;
    // nodal FP64 tables [function][node] (kept for diagnostics/tests)
    std::vector<double> R0_values, R0_derivs, R1_values, R1_derivs;
    // density scaling of A0 / A1 (A /= 1 + sum_j f(r_ij)): FP64 Hermite
    // coefficients [interval][4] of the one-output density networks
    bool A0_scaled = false, A1_scaled = false;
    std::vector<double> A0_density, A1_density;
    // radial definition: Bessel basis, polynomial cutoff, optional Agnesi
    // distance transform (per-pair features), networks
    std::vector<double> bessel;
    double bessel_prefactor = 0.0, cutoff_r_max = 0.0;
    int cutoff_p = 0;
    bool agnesi = false;
    double agnesi_a = 0.0, agnesi_q = 0.0, agnesi_p = 0.0;
    std::vector<double> covalent_radii;  // per model type
    RadialNetwork R0_net, R1_net, A0_net, A1_net;
    // tables of the model-type pair (ti, tj): packed FP32 R0/R1 Hermite
    // coefficients [interval][function][4] and FP64 density coefficients
    // [interval][4] (the tables above are the pair (0, 0))
    void pair_tables(int ti, int tj, std::vector<float>& R0, std::vector<float>& R1, std::vector<double>& D0,
                     std::vector<double>& D1) const;
    // Lay every per-channel table out for Cp >= C_file channels, the extra
    // channels zero in every weight, coefficient and radial function, so they
    // stay zero through the model and add nothing to energies or forces.
    void pad_channels(int Cp);
    std::vector<double> features(int ti, int tj) const;
    // ZBL pair repulsion: per (type, type) {1/a, 14.3996 Z_u Z_v, r_max}
    bool has_zbl = false;
    std::vector<double> zbl_pair;
    double zbl_c[4] = {0.0, 0.0, 0.0, 0.0};
    int zbl_p = 0;

    // layer 1
    std::vector<float> H0;                  // [type][C]
    std::vector<float> A0_w, A0_wt;         // [type][l][C_in][C_out] and transposed

    // M0 product basis: packed monomials concatenated over LM
    std::vector<std::int32_t> m0_terms;
    std::vector<std::int32_t> m0_term_offset;  // [num_LM + 1]
    std::vector<float> m0_coef;                // [type][term][C]

    std::vector<float> H1_w, H1_wt;         // [l][C][C], l <= L_max
    // h1_affine_mode "pre_linear_up" (h1_affine_schema.hpp:196-259,
    // mace.cpp:1759-1810): the readout_1 / skip input is x = M0[:,0,:] P0,
    // whose direct adjoint d enters M0_adj[:,0,:] as P0 d
    bool pre_linear_up = false;
    std::vector<float> P0, P0t;             // [C][C] H1_product_weights l = 0, [in][out] and [out][in]
    // first_interaction_residual (mace.cpp:1843-1875, 2796-2826): per type,
    // H1 += residual U (fused at load) and x += residual[lm 0]
    bool residual = false;
    std::vector<float> res_H1;              // [type][NH][C]
    std::vector<float> res_x;               // [type][C]
    // single_layer_readout (mace.cpp:255-281, 2461-2514): one interaction;
    // M1 is an invariant of H1's num_LM components, and there is no R1,
    // Phi1 or A1 (num_paths 0)
    bool single_layer = false;
    // MACEField (field_coupling.hpp:60-238; mace.cpp:322-395, 1147-1240):
    // H1p = M0 P (+ residual b), H1f[lm_out] = H1p[lm_out] + sum over the
    // angular entries of (coef E_c) H1p[lm_in] W_path, x = H1f[:,0,:],
    // H1 = H1f U.  Paths are (field_feats, field_linear) instruction pairs.
    bool field = false;
    struct FieldPath {
        int l_in, l_out;
    };
    struct FieldEntry {
        int lm_in, comp, lm_out, path;
        float coef;
    };
    std::vector<FieldPath> field_paths;
    std::vector<FieldEntry> field_entries;
    std::vector<float> field_W, field_Wt;   // [path][C][C] [in][out] and [out][in]
    std::vector<float> P_all, P_allt;        // [l][C][C] H1_product_weights and transposes
    std::vector<float> U_all, U_allt;        // [l][C][C] H1_linear_up_weights and transposes
    std::vector<float> res_pre;              // [type][NH][C] the residual before linear_up

    // R1 coupling
    std::vector<int> path_lo, path_le, path_ls;  // Phi1_l, Phi1_l1, Phi1_l2
    int num_paths = 0, num_rows = 0, num_lme = 0;
    std::vector<int> num_e, lme_base;      // per output l
    std::vector<int> row_base;             // per path
    // Dense per-path coupling blocks cg[p][m1][m2][mo], concatenated over p.
    std::vector<float> cg_dense;
    std::vector<int> cg_offset;            // [num_paths + 1]

    // A1: per l, W[(e,k_in)][k_out] and its transpose, concatenated over l
    std::vector<float> A1_w, A1_wt;
    std::vector<std::int64_t> A1_offset;   // [l_max + 2]

    // M1 invariant product basis
    std::vector<std::int32_t> m1_terms;
    std::vector<float> m1_coef;            // [type][term][C]

    // H2 skip / M1 linear (values FP32-representable, arithmetic FP64)
    std::vector<float> H2_T, H2_Tt;        // [type][in][out] and [type][out][in]
    std::vector<float> H2_M1, H2_M1t;      // [in][out] and [out][in]
    // readouts (FP64)
    std::vector<double> readout_q;         // [C]
    int readout_hidden = 0;
    std::vector<double> readout_W1;        // [hidden][C]
    std::vector<double> readout_W2;        // [hidden]
    double readout_scale = 1.0;

    void load(const std::string& path, const std::string& head);
    void load_field_coupling(const ::json_lite::Value& j);
};

// Rewrites a model file (JSON v4 text or its SMXB binary form) as `format`
// ("binary" or "json"), the document unchanged.
void convert_model_file(const std::string& source, const std::string& destination, const std::string& format);

}  // namespace smx
