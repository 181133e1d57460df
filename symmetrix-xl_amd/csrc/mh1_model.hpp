// MH-1 (MACE_Nonlinear) model: the JSON file compiled into flat tables for
// the HIP kernels (host side).
//
// The file is the reference's nonlinear schema (written by
// symmetrix/source/symmetrix/extract_mace_nonlinear.py, read by
// libsymmetrix/source/mace_nonlinear.cpp:302-380, e3nn.cpp, e3nn_product.cpp,
// affine_mlp.cpp).  Every e3nn piece becomes a table the kernels walk:
//
// * Linear: instructions grouped by output block, weights pre-multiplied by
//   the path weight, one (block, channel, component) triple per output
//   element; the reverse is the same kind of table built from the transposed
//   weights (the forward's output mask moves to the reverse's input).
// * Tensor product ("uvu", external weights, one channel count for every
//   first-input block, unit-multiplicity harmonics): per path the first
//   input's offset, the harmonic l, the output offset and the nonzero Wigner
//   entries (a, b, k, value x path weight).
// * Affine MLP: layer descriptors; the first layer's source/target embedding
//   columns are folded into per-type rows (with its bias), as the
//   reference's conditioned evaluation does (mace_nonlinear.cpp:144-199), so
//   the kernels read only the radial columns.
// * Product basis: U x W summed over the basis index and over every ordering
//   of each monomial's indices, one coefficient row per (monomial, output
//   component), [element][term][channel].
// * Gate: per output element its value index, gate index and constant; per
//   input element the adjoint rule.
#pragma once

#include <array>
#include <cstdint>
#include <string>
#include <vector>

#include "json_lite.hpp"

namespace smx {
namespace mh1 {

struct Block {
    int mul = 0, l = 0, parity = 1, offset = 0;
    int dim() const { return mul * (2 * l + 1); }
};

struct Irreps {
    std::vector<Block> blocks;
    int dim = 0;
    Irreps() = default;
    explicit Irreps(const std::string& spec);
};

// Host tables of one linear map (forward or transposed form).
struct LinearTables {
    int in_dim = 0, out_dim = 0, num_out_blocks = 0;
    std::vector<int> instr;        // 6 per instruction: in_off, mul_in, d, w_off, out_off, mul_out
    std::vector<int> block_first;  // [num_out_blocks + 1]
    std::vector<int> elem;         // 3 per output element: block, channel, component
    std::vector<int> out_blocks;   // 3 per output block: offset, multiplicity, width 2l+1
    std::vector<float> weights;    // path weight folded in
    std::vector<float> bias;       // empty or [out_dim]
    std::vector<float> out_mask;   // empty (all ones) or [out_dim]
    std::vector<float> in_mask;    // empty or [in_dim]
};

struct Linear {
    Irreps in, out;
    LinearTables fwd, rev;
    explicit Linear(const json_lite::Value& v);
    Linear() = default;
};

struct MlpTables {
    // 4 ints per layer: type (0 linear, 1 layer norm, 2 silu), in, out, parameter offset
    std::vector<int> layers;
    std::vector<float> eps;
    std::vector<float> params;     // linear: W [out][in] then b [out]; LN: w, b
    int radial = 0, first_width = 0, out_dim = 0, max_hidden = 0, num_layers = 0;
    std::vector<float> type_rows;  // [2][num_types][first_width]: source rows (+ bias), target rows
    // per layer: offset of a linear's transposed weights [in][out] in params (-1 otherwise), and of
    // the layer's output in the tape (kept only when a LayerNorm or SiLU follows; -1 otherwise): the
    // tape is layer-major, the kept layer's [E][width] block at tape_offset * E; tape_width floats
    // per edge in all
    std::vector<int> wt_offset, tape_offset;
    int tape_width = 0;
    // register form: the conditioned first linear and each later hidden linear, with an optional
    // LayerNorm, feed a SiLU (a hidden stage), and a final linear follows the last stage; at most
    // kRegStages stages, all of one width, 16, 32 or 64.  reg_hw is that width (the kernel class),
    // 0 when the MLP has another form.  Per stage, then for the
    // final linear, 6 ints: in, out, W [out][in], bias (-1: the per-type rows), W^T [in][out],
    // LayerNorm weight (bias follows; -1 without) as offsets into params, all 16-byte aligned
    static constexpr int kRegStages = 3;
    int reg_hw = 0, reg_stages = 0;
    std::vector<int> reg_stage;
    std::vector<float> reg_eps;
};

struct TensorTables {
    int channels = 0, in1_dim = 0, out_dim = 0, numel = 0, slots = 0, num_paths = 0, in1_per_channel = 0;
    // 8 ints per path (per-channel slots): first-input slot base, d1, harmonic offset l2^2, output slot
    // base, d3, weight offset, first Wigner entry, entry count
    std::vector<int> paths;
    std::vector<int> in1_slot, out_slot;  // 3 per slot: block offset, width, component
    std::vector<int> entries;      // a | b << 8 | k << 16
    std::vector<float> values;     // Wigner value x path weight
    // a compiled family structure (mh1_paths.hpp): 2 * L1MAX + (l_max - 2), or -1; its values in the
    // structure's entry order (x path weight, 0 where the file has no entry)
    int compiled = -1;
    std::vector<float> compiled_values;
};

struct GateTables {
    int in_dim = 0, out_dim = 0;
    std::vector<int> out_src, out_gate;  // per output element
    std::vector<float> out_const;
    // per input element: kind (0 scalar, 1 gated value, 2 gate), output index, aux, count, constant
    std::vector<int> in_kind, in_out, in_aux, in_count;
    std::vector<float> in_const;
};

struct ProductTables {
    int channels = 0, angular = 0, in_dim = 0, out_dim = 0, out_slots = 0, num_terms = 0, num_elements = 0;
    bool agnostic = true, use_sc = true;
    std::vector<int> ang_src;      // per angular index: block offset, component count, component (3 ints)
    std::vector<int> out_slot;     // per output slot: block offset, width, component (3 ints)
    std::vector<int> terms;        // 4 per term: i1, i2, i3 (angular index; `angular` = the constant 1), slot
    std::vector<float> coef;       // [element][term][channel]
    Linear linear;
};

struct Interaction {
    Linear source_embedding, target_embedding, up, skip, res, lin1, lin2;
    TensorTables tp;
    MlpTables weights_mlp, density_mlp;
    GateTables gate;
    double alpha = 0.0, beta = 0.0;
};

struct Readout {
    bool nonlinear = false;
    Linear lin1, lin2;
    double activation_constant = 1.0;
};

struct Model {
    std::vector<int> atomic_numbers, model_atomic_numbers, model_indices;
    std::vector<double> atomic_energies;
    std::string selected_head;
    double r_cut = 0.0;
    int l_max = 0, num_lm = 0, num_model_elements = 0, cutoff_p = 0;
    bool apply_cutoff = true, agnesi = false;
    double agnesi_a = 0, agnesi_q = 0, agnesi_p = 0;
    std::vector<double> covalent_radii;
    std::vector<double> bessel;
    double prefactor = 0.0;
    double scale = 1.0, shift = 0.0;
    Linear embedding;
    std::vector<Interaction> interactions;
    std::vector<ProductTables> products;
    std::vector<Readout> readouts;
    bool has_zbl = false;
    double zbl_a_exp = 0, zbl_a_prefactor = 0;
    double zbl_c[4] = {0, 0, 0, 0};
    std::vector<double> zbl_radii;
    int zbl_p = 0;
    // family facts (mace_nonlinear_schema.cpp:108-207)
    bool family = false;
    std::string family_rejection;
    int family_node_channels = 0, family_edge_channels = 0, family_radial = 0;

    static Model load(const std::string& path, const std::string& head);
};

}  // namespace mh1
}  // namespace smx
