// MH-1 (MACE_Nonlinear) model loader: JSON -> kernel tables (host, FP64
// where the tables are formed, FP32 where they are stored).
//
// The checks enforce what the schema and the kernels need; their order and
// wording are this loader's own.  Reference semantics of each piece:
// irreps strings e3nn.cpp:83-112; Linear e3nn.cpp:114-166; tensor product
// e3nn.cpp:247-313; affine MLP affine_mlp.cpp:38-110 and its conditioned
// first layer :112-126; gate mace_nonlinear.cpp:56-101; readouts :216-235;
// product basis e3nn_product.cpp:58-120,332-369; top level
// mace_nonlinear.cpp:302-380 and mace_nonlinear_schema.cpp:209-305; family
// facts mace_nonlinear_schema.cpp:108-207.
#include "mh1_model.hpp"

#include "mh1_paths.hpp"

#include <algorithm>
#include <cmath>
#include <map>
#include <numeric>
#include <set>
#include <stdexcept>

namespace smx {
namespace mh1 {
namespace {

using json_lite::Value;

[[noreturn]] void bad(const std::string& what) { throw std::invalid_argument("MH-1 model: " + what); }

std::vector<double> tensor_values(const Value& t, const char* what) {
    if (!t.is_object() || !t.contains("values") || !t.contains("shape")) bad(std::string(what) + " is not a tensor");
    const std::vector<double> v = t.at("values").as_doubles();
    const std::vector<int> shape = t.at("shape").as_ints();
    long long n = 1;
    for (int s : shape) {
        if (s < 0) bad(std::string(what) + " has a negative extent");
        n *= s;
    }
    if (n != static_cast<long long>(v.size())) bad(std::string(what) + " values do not fill its shape");
    for (double x : v)
        if (!std::isfinite(x)) bad(std::string(what) + " holds a non-finite value");
    return v;
}

std::vector<int> tensor_shape(const Value& t) { return t.at("shape").as_ints(); }

bool same_blocks(const Irreps& a, const std::vector<Block>& want) {
    if (a.blocks.size() != want.size()) return false;
    for (std::size_t i = 0; i < want.size(); ++i)
        if (a.blocks[i].mul != want[i].mul || a.blocks[i].l != want[i].l || a.blocks[i].parity != want[i].parity)
            return false;
    return true;
}

std::vector<Block> spherical(int mul, int l_max, int scalar_mul) {
    std::vector<Block> b{{scalar_mul, 0, 1, 0}};
    for (int l = 1; l <= l_max; ++l) b.push_back({mul, l, l % 2 ? -1 : 1, 0});
    return b;
}

// forward and transposed tables of one e3nn Linear
void build_linear(Linear& L, const std::vector<std::array<int, 2>>& pairs, const std::vector<double>& pw,
                  const std::vector<double>& w, const std::vector<double>& bias, const std::vector<double>& mask) {
    const int nin = static_cast<int>(L.in.blocks.size()), nout = static_cast<int>(L.out.blocks.size());
    std::vector<int> woff(pairs.size());
    for (std::size_t q = 0, o = 0; q < pairs.size(); ++q) {
        woff[q] = static_cast<int>(o);
        o += static_cast<std::size_t>(L.in.blocks[pairs[q][0]].mul) * L.out.blocks[pairs[q][1]].mul;
    }
    const bool ones = std::all_of(mask.begin(), mask.end(), [](double m) { return m == 1.0; });
    auto fill = [&](LinearTables& T, bool transposed) {
        const Irreps& I = transposed ? L.out : L.in;
        const Irreps& O = transposed ? L.in : L.out;
        T.in_dim = I.dim;
        T.out_dim = O.dim;
        T.num_out_blocks = transposed ? nin : nout;
        T.block_first.assign(T.num_out_blocks + 1, 0);
        for (int ob = 0; ob < T.num_out_blocks; ++ob) {
            T.block_first[ob] = static_cast<int>(T.instr.size() / 6);
            for (std::size_t q = 0; q < pairs.size(); ++q) {
                const int bi = transposed ? pairs[q][1] : pairs[q][0];
                const int bo = transposed ? pairs[q][0] : pairs[q][1];
                if (bo != ob) continue;
                const Block& a = I.blocks[bi];
                const Block& c = O.blocks[bo];
                const int d = 2 * a.l + 1;
                T.instr.insert(T.instr.end(), {a.offset, a.mul, d, static_cast<int>(T.weights.size()), c.offset, c.mul});
                // forward W[u][w] (u input channel); transposed W'[w][u]
                const int mu = L.in.blocks[pairs[q][0]].mul, mw = L.out.blocks[pairs[q][1]].mul;
                for (int i = 0; i < a.mul; ++i)
                    for (int o = 0; o < c.mul; ++o) {
                        const int u = transposed ? o : i, ww = transposed ? i : o;
                        T.weights.push_back(static_cast<float>(pw[q] * w[woff[q] + static_cast<std::size_t>(u) * mw + ww]));
                    }
                (void)mu;
            }
        }
        T.block_first[T.num_out_blocks] = static_cast<int>(T.instr.size() / 6);
        for (int ob = 0; ob < T.num_out_blocks; ++ob) {
            const Block& c = O.blocks[ob];
            T.out_blocks.insert(T.out_blocks.end(), {c.offset, c.mul, 2 * c.l + 1});
            for (int ch = 0; ch < c.mul; ++ch)
                for (int m = 0; m < 2 * c.l + 1; ++m) T.elem.insert(T.elem.end(), {ob, ch, m});
        }
        if (!transposed) {
            if (!bias.empty()) T.bias.assign(bias.begin(), bias.end());
            if (!ones) T.out_mask.assign(mask.begin(), mask.end());
        } else if (!ones) {
            T.in_mask.assign(mask.begin(), mask.end());
        }
    };
    fill(L.fwd, false);
    fill(L.rev, true);
}

}  // namespace

Irreps::Irreps(const std::string& spec) {
    std::size_t p = 0;
    while (p <= spec.size()) {
        const std::size_t q = std::min(spec.find('+', p), spec.size());
        std::string tok;
        for (std::size_t i = p; i < q; ++i)
            if (!std::isspace(static_cast<unsigned char>(spec[i]))) tok += spec[i];
        const std::size_t x = tok.find('x');
        if (x == std::string::npos || x == 0 || tok.size() < x + 3 || (tok.back() != 'e' && tok.back() != 'o'))
            bad("irreps '" + spec + "' are not of the form <mul>x<l><e|o>");
        const std::string ms = tok.substr(0, x), ls = tok.substr(x + 1, tok.size() - x - 2);
        if (ms.find_first_not_of("0123456789") != std::string::npos ||
            ls.find_first_not_of("0123456789") != std::string::npos || ls.empty())
            bad("irreps '" + spec + "' are not of the form <mul>x<l><e|o>");
        Block b{std::stoi(ms), std::stoi(ls), tok.back() == 'e' ? 1 : -1, dim};
        if (b.mul <= 0) bad("irreps '" + spec + "' have a zero multiplicity");
        blocks.push_back(b);
        dim += b.dim();
        p = q + 1;
    }
    if (blocks.empty()) bad("empty irreps");
}

Linear::Linear(const Value& v) : in(v.at("irreps_in").as_string()), out(v.at("irreps_out").as_string()) {
    const std::vector<double> w = tensor_values(v.at("weight"), "linear weight");
    const std::vector<double> bias = tensor_values(v.at("bias"), "linear bias");
    const std::vector<double> mask = tensor_values(v.at("output_mask"), "linear output_mask");
    std::vector<std::array<int, 2>> pairs;
    std::vector<double> pw;
    std::size_t need = 0;
    for (const Value& ins : v.at("instructions").items) {
        const int i = ins.at("i_in").as_int(), o = ins.at("i_out").as_int();
        if (i < 0 || o < 0 || i >= static_cast<int>(in.blocks.size()) || o >= static_cast<int>(out.blocks.size()))
            bad("linear path names a block that does not exist");
        const std::vector<int> shape = ins.at("path_shape").as_ints();
        if (shape.size() != 2 || shape[0] != in.blocks[i].mul || shape[1] != out.blocks[o].mul ||
            in.blocks[i].l != out.blocks[o].l)
            bad("linear path must map one l to the same l with a [mul_in, mul_out] weight");
        pairs.push_back({i, o});
        pw.push_back(ins.contains("path_weight") ? ins.at("path_weight").as_number() : 1.0);
        need += static_cast<std::size_t>(shape[0]) * shape[1];
    }
    if (need != w.size()) bad("linear weight count differs from its paths");
    if (static_cast<int>(mask.size()) != out.dim) bad("linear output_mask size differs from the output");
    if (!bias.empty() && static_cast<int>(bias.size()) != out.dim) bad("linear bias size differs from the output");
    build_linear(*this, pairs, pw, w, bias, mask);
}

namespace {

std::vector<double> linear_apply(const Linear& L, const std::vector<double>& x) {
    // FP64 evaluation on the host (per-type embeddings)
    std::vector<double> y(L.out.dim, 0.0);
    const LinearTables& T = L.fwd;
    for (int j = 0; j < T.out_dim; ++j) {
        const int b = T.elem[3 * j], ch = T.elem[3 * j + 1], m = T.elem[3 * j + 2];
        double acc = 0.0;
        for (int q = T.block_first[b]; q < T.block_first[b + 1]; ++q) {
            const int* I = &T.instr[6 * q];
            for (int u = 0; u < I[1]; ++u)
                acc += static_cast<double>(T.weights[I[3] + u * I[5] + ch]) * x[I[0] + u * I[2] + m];
        }
        if (!T.bias.empty()) acc += T.bias[j];
        if (!T.out_mask.empty()) acc *= T.out_mask[j];
        y[j] = acc;
    }
    return y;
}

void align4(std::vector<float>& v) {
    while (v.size() % 4) v.push_back(0.0f);
}

// Stages of the register form (MlpTables::reg_stage), or reg_hw = 0 when the
// layers are not [linear, LayerNorm?, SiLU]... linear with one hidden width of
// 16, 32 or 64.
void plan_register_form(MlpTables& T) {
    T.reg_hw = 0;
    T.reg_stages = 0;
    T.reg_stage.clear();
    T.reg_eps.clear();
    const auto type = [&](int k) { return T.layers[4 * k]; };
    int k = 0, widest = 0;
    std::vector<int> st;
    std::vector<float> eps;
    while (true) {
        if (k >= T.num_layers || type(k) != 0) return;
        const int* L = &T.layers[4 * k];
        const int in = L[1], out = L[2];
        const int bias = k == 0 ? -1 : L[3] + out * in;
        if (k + 1 == T.num_layers) {
            st.insert(st.end(), {in, out, L[3], bias, T.wt_offset[k], -1});
            eps.push_back(0.0f);
            break;
        }
        int ln = -1;
        float e = 0.0f;
        int next = k + 1;
        if (type(next) == 1) {
            ln = T.layers[4 * next + 3];
            e = T.eps[next];
            ++next;
        }
        if (next >= T.num_layers || type(next) != 2) return;
        if (out % 16 != 0 || out > 64) return;
        if (k > 0 && (in % 16 != 0 || (bias % 4) != 0)) return;
        if (ln >= 0 && ln % 4 != 0) return;
        st.insert(st.end(), {in, out, L[3], bias, T.wt_offset[k], ln});
        eps.push_back(e);
        widest = std::max(widest, out);
        k = next + 1;
    }
    const int stages = static_cast<int>(eps.size()) - 1;
    if (stages < 1 || stages > MlpTables::kRegStages) return;
    if (widest != 16 && widest != 32 && widest != 64) return;
    for (int h = 0; h < stages; ++h)
        if (st[6 * h + 1] != widest) return;
    T.reg_hw = widest;
    T.reg_stages = stages;
    T.reg_stage = st;
    T.reg_eps = eps;
}

MlpTables build_mlp(const Value& v, int radial, const std::vector<std::vector<double>>& src_emb,
                    const std::vector<std::vector<double>>& tgt_emb, const char* what) {
    MlpTables T;
    T.radial = radial;
    const auto& layers = v.at("layers").items;
    if (layers.empty()) bad(std::string(what) + " has no layers");
    int prev = -1;
    const int S1 = src_emb.empty() ? 0 : static_cast<int>(src_emb[0].size());
    const int S2 = tgt_emb.empty() ? 0 : static_cast<int>(tgt_emb[0].size());
    for (std::size_t k = 0; k < layers.size(); ++k) {
        const Value& L = layers[k];
        const std::string type = L.at("type").as_string();
        if (type == "linear") {
            const std::vector<int> shape = tensor_shape(L.at("weight"));
            const std::vector<double> W = tensor_values(L.at("weight"), "MLP weight");
            const std::vector<double> b = tensor_values(L.at("bias"), "MLP bias");
            if (shape.size() != 2 || static_cast<int>(b.size()) != shape[0]) bad(std::string(what) + " linear shapes disagree");
            const int out = shape[0], in = shape[1];
            if (prev >= 0 && in != prev) bad(std::string(what) + " layer widths do not chain");
            align4(T.params);
            const int off = static_cast<int>(T.params.size());
            if (k == 0) {
                // conditioned first layer: [radial | source embedding | target embedding]
                if (in != radial + S1 + S2) bad(std::string(what) + " first layer does not take radial + embeddings");
                for (int o = 0; o < out; ++o)
                    for (int c = 0; c < radial; ++c) T.params.push_back(static_cast<float>(W[o * in + c]));
                const int nt = static_cast<int>(src_emb.size());
                T.type_rows.assign(static_cast<std::size_t>(2) * nt * out, 0.0f);
                for (int t = 0; t < nt; ++t)
                    for (int o = 0; o < out; ++o) {
                        double s = b[o], g = 0.0;
                        for (int c = 0; c < S1; ++c) s += W[o * in + radial + c] * src_emb[t][c];
                        for (int c = 0; c < S2; ++c) g += W[o * in + radial + S1 + c] * tgt_emb[t][c];
                        T.type_rows[static_cast<std::size_t>(t) * out + o] = static_cast<float>(s);
                        T.type_rows[static_cast<std::size_t>(nt + t) * out + o] = static_cast<float>(g);
                    }
                T.first_width = out;
                T.layers.insert(T.layers.end(), {0, radial, out, off});
            } else {
                for (double x : W) T.params.push_back(static_cast<float>(x));
                for (double x : b) T.params.push_back(static_cast<float>(x));
                T.layers.insert(T.layers.end(), {0, in, out, off});
            }
            T.eps.push_back(0.0f);
            prev = out;
        } else if (type == "layer_norm") {
            const std::vector<int> ns = L.at("normalized_shape").as_ints();
            const std::vector<double> w = tensor_values(L.at("weight"), "LayerNorm weight");
            const std::vector<double> b = tensor_values(L.at("bias"), "LayerNorm bias");
            const double eps = L.at("eps").as_number();
            if (ns.size() != 1 || ns[0] != prev || static_cast<int>(w.size()) != prev ||
                static_cast<int>(b.size()) != prev || !(eps > 0.0))
                bad(std::string(what) + " LayerNorm does not match its input width");
            align4(T.params);
            const int off = static_cast<int>(T.params.size());
            for (double x : w) T.params.push_back(static_cast<float>(x));
            for (double x : b) T.params.push_back(static_cast<float>(x));
            T.layers.insert(T.layers.end(), {1, prev, prev, off});
            T.eps.push_back(static_cast<float>(eps));
        } else if (type == "silu") {
            if (prev < 0) bad(std::string(what) + " starts with an activation");
            T.layers.insert(T.layers.end(), {2, prev, prev, 0});
            T.eps.push_back(0.0f);
        } else {
            bad(std::string(what) + " layer type '" + type + "' is not supported");
        }
        if (k == 0 && type != "linear") bad(std::string(what) + " must start with a linear layer");
    }
    if (T.layers[T.layers.size() - 4] != 0) bad(std::string(what) + " must end with a linear layer");
    T.num_layers = static_cast<int>(T.layers.size() / 4);
    T.out_dim = prev;
    for (int k = 0; k + 1 < T.num_layers; ++k) T.max_hidden = std::max(T.max_hidden, T.layers[4 * k + 2]);
    T.max_hidden = std::max(T.max_hidden, T.radial);
    for (int k = 0; k < T.num_layers; ++k) {
        const int* L = &T.layers[4 * k];
        if (L[0] == 0) {
            align4(T.params);
            T.wt_offset.push_back(static_cast<int>(T.params.size()));
            for (int i = 0; i < L[1]; ++i)
                for (int o = 0; o < L[2]; ++o) {
                    const float w = T.params[L[3] + static_cast<std::size_t>(o) * L[1] + i];
                    T.params.push_back(w);
                }
        } else {
            T.wt_offset.push_back(-1);
        }
        // the reverse needs a layer's output only as the input of a LayerNorm or SiLU
        const bool keep = k + 1 < T.num_layers && T.layers[4 * (k + 1)] != 0;
        T.tape_offset.push_back(keep ? T.tape_width : -1);
        if (keep) T.tape_width += L[2];
    }
    plan_register_form(T);
    return T;
}

// Match the table-driven paths against a compiled family structure: same
// paths in the same order, Wigner entries inside the compiled positions.
template <int L1MAX, int LMAX>
bool match_structure(TensorTables& T) {
    using S = TpStructure<L1MAX, LMAX>;
    if (T.num_paths != S::kPaths || T.slots != S::kSlots || T.in1_per_channel != S::kIn1) return false;
    std::vector<float> vals(S::kEntries, 0.0f);
    for (int p = 0; p < S::kPaths; ++p) {
        const int* P = &T.paths[8 * p];
        const TpPathC& c = S::paths[p];
        if (P[0] != c.in_base || P[1] != 2 * c.l1 + 1 || P[2] != c.l2 * c.l2 || P[3] != c.out_base ||
            P[4] != 2 * c.l3 + 1 || P[5] != p * T.channels)
            return false;
        for (int q = P[6]; q < P[6] + P[7]; ++q) {
            const int a = T.entries[q] & 255, b = (T.entries[q] >> 8) & 255, k = T.entries[q] >> 16;
            int hit = -1;
            for (int j = c.first; j < c.first + c.count; ++j)
                if (S::entries[j].a == a && S::entries[j].b == b && S::entries[j].k == k) hit = j;
            if (hit < 0) return false;
            vals[hit] = T.values[q];
        }
    }
    T.compiled = 2 * L1MAX + (LMAX - 2);
    T.compiled_values = vals;
    return true;
}

TensorTables build_tp(const Value& v, int l_max) {
    TensorTables T;
    const Irreps in1(v.at("irreps_in1").as_string()), in2(v.at("irreps_in2").as_string()),
        out(v.at("irreps_out").as_string());
    if (!tensor_values(v.at("weight"), "tensor-product weight").empty())
        bad("the convolution must take its weights per edge (no internal weights)");
    const std::vector<double> mask = tensor_values(v.at("output_mask"), "tensor-product output_mask");
    if (static_cast<int>(mask.size()) != out.dim) bad("tensor-product output_mask size differs from the output");
    for (double m : mask)
        if (m != 1.0) bad("a convolution output_mask other than all ones is not supported");
    const int E = in1.blocks[0].mul;
    for (const Block& b : in1.blocks)
        if (b.mul != E) bad("the convolution's first input must hold one channel count");
    for (const Block& b : out.blocks)
        if (b.mul != E) bad("the convolution's output blocks must hold the first input's channel count");
    for (std::size_t i = 0; i < in2.blocks.size(); ++i)
        if (in2.blocks[i].mul != 1 || in2.blocks[i].l != static_cast<int>(i) || in2.blocks[i].l > l_max ||
            in2.blocks[i].parity != (i % 2 ? -1 : 1))
            bad("the convolution's second input must be the spherical harmonics 1x0e+1x1o+...");
    T.channels = E;
    T.in1_dim = in1.dim;
    T.out_dim = out.dim;
    T.in1_per_channel = in1.dim / E;
    T.slots = out.dim / E;
    std::vector<int> in1_base(in1.blocks.size()), out_base(out.blocks.size());
    for (std::size_t b = 0, s = 0; b < in1.blocks.size(); ++b) {
        in1_base[b] = static_cast<int>(s);
        s += 2 * in1.blocks[b].l + 1;
    }
    for (std::size_t b = 0, s = 0; b < out.blocks.size(); ++b) {
        out_base[b] = static_cast<int>(s);
        s += 2 * out.blocks[b].l + 1;
    }
    int woff = 0;
    for (const Value& ins : v.at("instructions").items) {
        const int i1 = ins.at("i_in1").as_int(), i2 = ins.at("i_in2").as_int(), io = ins.at("i_out").as_int();
        if (i1 < 0 || i2 < 0 || io < 0 || i1 >= static_cast<int>(in1.blocks.size()) ||
            i2 >= static_cast<int>(in2.blocks.size()) || io >= static_cast<int>(out.blocks.size()))
            bad("tensor-product path names a block that does not exist");
        if (ins.at("connection_mode").as_string() != "uvu" || !ins.at("has_weight").as_bool())
            bad("only weighted 'uvu' convolution paths have a kernel");
        const std::vector<int> ps = ins.at("path_shape").as_ints();
        if (ps.size() != 2 || ps[0] != E || ps[1] != 1) bad("uvu path weight shape must be [channels, 1]");
        const int l1 = in1.blocks[i1].l, l2 = in2.blocks[i2].l, l3 = out.blocks[io].l;
        const std::vector<int> ws = tensor_shape(ins.at("wigner_3j"));
        const std::vector<double> w3j = tensor_values(ins.at("wigner_3j"), "Wigner 3j");
        if (ws != std::vector<int>{2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1}) bad("Wigner 3j shape differs from its path");
        const double pw = ins.contains("path_weight") ? ins.at("path_weight").as_number() : 1.0;
        const int first = static_cast<int>(T.values.size());
        for (int a = 0; a < 2 * l1 + 1; ++a)
            for (int b = 0; b < 2 * l2 + 1; ++b)
                for (int k = 0; k < 2 * l3 + 1; ++k) {
                    const double x = w3j[(a * (2 * l2 + 1) + b) * (2 * l3 + 1) + k];
                    if (x == 0.0) continue;
                    T.entries.push_back(a | (b << 8) | (k << 16));
                    T.values.push_back(static_cast<float>(x * pw));
                }
        T.paths.insert(T.paths.end(), {in1_base[i1], 2 * l1 + 1, l2 * l2, out_base[io], 2 * l3 + 1, woff, first,
                                       static_cast<int>(T.values.size()) - first});
        woff += E;
        ++T.num_paths;
    }
    T.numel = woff;
    // per-channel slot -> (row offset, width, component): loading the first input, storing the output
    for (const Block& b : in1.blocks)
        for (int a = 0; a < 2 * b.l + 1; ++a) T.in1_slot.insert(T.in1_slot.end(), {b.offset, 2 * b.l + 1, a});
    for (const Block& b : out.blocks)
        for (int k = 0; k < 2 * b.l + 1; ++k) T.out_slot.insert(T.out_slot.end(), {b.offset, 2 * b.l + 1, k});
    const bool scalar_in = in1.blocks.size() == 1 && in1.blocks[0].l == 0 && in1.blocks[0].parity == 1;
    const bool vector_in = in1.blocks.size() == 2 && in1.blocks[0].l == 0 && in1.blocks[0].parity == 1 &&
                           in1.blocks[1].l == 1 && in1.blocks[1].parity == -1;
    if (l_max == 2 && scalar_in) match_structure<0, 2>(T);
    if (l_max == 3 && scalar_in) match_structure<0, 3>(T);
    if (l_max == 2 && vector_in) match_structure<1, 2>(T);
    if (l_max == 3 && vector_in) match_structure<1, 3>(T);
    return T;
}

GateTables build_gate(const Value& v) {
    if (v.at("scalar_activation").as_string() != "silu" || v.at("gate_activation").as_string() != "sigmoid")
        bad("gate activations other than SiLU scalars and sigmoid gates are not supported");
    const Irreps in(v.at("irreps_in").as_string()), out(v.at("irreps_out").as_string()),
        sc(v.at("irreps_scalars").as_string()), ga(v.at("irreps_gates").as_string()),
        gd(v.at("irreps_gated").as_string());
    const std::vector<double> scc = v.at("scalar_activation_constants").as_doubles();
    const std::vector<double> gcc = v.at("gate_activation_constants").as_doubles();
    int gate_count = 0;
    for (const Block& b : ga.blocks) {
        if (b.l != 0) bad("gates must be scalars");
        gate_count += b.mul;
    }
    int gated_channels = 0;
    for (const Block& b : gd.blocks) gated_channels += b.mul;
    for (const Block& b : sc.blocks)
        if (b.l != 0) bad("gate scalars must be scalars");
    if (in.dim != sc.dim + ga.dim + gd.dim || out.dim != sc.dim + gd.dim || gate_count != gated_channels ||
        scc.size() != sc.blocks.size() || gcc.size() != gd.blocks.size())
        bad("gate irreps and constants do not agree");
    GateTables T;
    T.in_dim = in.dim;
    T.out_dim = out.dim;
    T.out_src.resize(out.dim);
    T.out_gate.resize(out.dim);
    T.out_const.resize(out.dim);
    T.in_kind.assign(in.dim, 0);
    T.in_out.assign(in.dim, 0);
    T.in_aux.assign(in.dim, 0);
    T.in_count.assign(in.dim, 0);
    T.in_const.assign(in.dim, 0.0f);
    for (std::size_t k = 0; k < sc.blocks.size(); ++k)
        for (int i = sc.blocks[k].offset; i < sc.blocks[k].offset + sc.blocks[k].dim(); ++i) {
            T.out_src[i] = i;
            T.out_gate[i] = -1;
            T.out_const[i] = static_cast<float>(scc[k]);
            T.in_kind[i] = 0;
            T.in_out[i] = i;
            T.in_const[i] = static_cast<float>(scc[k]);
        }
    int gate_i = sc.dim, value_i = sc.dim + ga.dim, out_i = sc.dim;
    for (std::size_t k = 0; k < gd.blocks.size(); ++k) {
        const int d = 2 * gd.blocks[k].l + 1;
        for (int ch = 0; ch < gd.blocks[k].mul; ++ch) {
            T.in_kind[gate_i] = 2;
            T.in_out[gate_i] = out_i;
            T.in_aux[gate_i] = value_i;
            T.in_count[gate_i] = d;
            T.in_const[gate_i] = static_cast<float>(gcc[k]);
            for (int m = 0; m < d; ++m) {
                T.out_src[out_i + m] = value_i + m;
                T.out_gate[out_i + m] = gate_i;
                T.out_const[out_i + m] = static_cast<float>(gcc[k]);
                T.in_kind[value_i + m] = 1;
                T.in_out[value_i + m] = out_i + m;
                T.in_aux[value_i + m] = gate_i;
                T.in_const[value_i + m] = static_cast<float>(gcc[k]);
            }
            ++gate_i;
            value_i += d;
            out_i += d;
        }
    }
    return T;
}

ProductTables build_product(const Value& v, int num_model_elements) {
    ProductTables P;
    const Value& sc = v.at("symmetric_contractions");
    const Irreps in(sc.at("irreps_in").as_string()), out(sc.at("irreps_out").as_string());
    P.linear = Linear(v.at("linear"));
    P.use_sc = v.at("use_sc").as_bool();
    P.agnostic = v.get_bool("use_agnostic_product", false);
    if (P.linear.in.dim != out.dim || P.linear.out.dim != out.dim) bad("product linear must map the contraction's irreps to themselves");
    const int C = in.blocks[0].mul;
    for (const Block& b : in.blocks)
        if (b.mul != C) bad("product input blocks must share one channel count");
    for (const Block& b : out.blocks)
        if (b.mul != C) bad("product output blocks must hold the input's channel count");
    P.channels = C;
    P.in_dim = in.dim;
    P.out_dim = out.dim;
    for (const Block& b : in.blocks)
        for (int m = 0; m < 2 * b.l + 1; ++m) P.ang_src.insert(P.ang_src.end(), {b.offset, 2 * b.l + 1, m});
    P.angular = static_cast<int>(P.ang_src.size() / 3);
    std::vector<int> slot_base;
    for (const Block& b : out.blocks) {
        slot_base.push_back(static_cast<int>(P.out_slot.size() / 3));
        for (int m = 0; m < 2 * b.l + 1; ++m) P.out_slot.insert(P.out_slot.end(), {b.offset, 2 * b.l + 1, m});
    }
    P.out_slots = static_cast<int>(P.out_slot.size() / 3);
    const auto& cons = sc.at("contractions").items;
    if (cons.size() != out.blocks.size()) bad("one contraction per product output block is required");
    // (slot, sorted monomial) -> coefficient row over [element][channel]
    std::map<std::pair<int, std::array<int, 3>>, std::vector<double>> rows;
    int num_el = -1;
    for (std::size_t bi = 0; bi < cons.size(); ++bi) {
        const Value& c = cons[bi];
        const int L = out.blocks[bi].l;
        const int corr = c.at("correlation").as_int();
        const auto& us = c.at("u_tensors").items;
        const auto& ws = c.at("weights").items;
        if (corr < 1 || corr > 3 || static_cast<int>(us.size()) != corr || static_cast<int>(ws.size()) != corr - 1)
            bad("product correlation must be 1..3 with one U tensor per degree");
        for (int nu = 1; nu <= corr; ++nu) {
            const Value& U = us[nu - 1];
            const Value& W = nu == corr ? c.at("weights_max") : ws[corr - nu - 1];
            const std::vector<int> us_ = tensor_shape(U), ws_ = tensor_shape(W);
            const std::vector<double> uv = tensor_values(U, "product U"), wv = tensor_values(W, "product weights");
            const int lead = L == 0 ? 0 : 1;
            if (static_cast<int>(us_.size()) != nu + lead + 1 || (lead && us_[0] != 2 * L + 1) || ws_.size() != 3 ||
                ws_[1] != us_.back() || ws_[2] != C)
                bad("product U / weight shapes disagree");
            for (int a = 0; a < nu; ++a)
                if (us_[lead + a] != P.angular) bad("product U angular extent differs from the input");
            if (num_el < 0) num_el = ws_[0];
            if (ws_[0] != num_el) bad("product weight element counts disagree");
            const int K = us_.back();
            long long tuples = 1;
            for (int a = 0; a < nu; ++a) tuples *= P.angular;
            for (int M = 0; M < 2 * L + 1; ++M)
                for (long long t = 0; t < tuples; ++t) {
                    std::array<int, 3> idx{P.angular, P.angular, P.angular};
                    long long rem = t;
                    for (int a = nu - 1; a >= 0; --a) {
                        idx[a] = static_cast<int>(rem % P.angular);
                        rem /= P.angular;
                    }
                    const double* up = &uv[((static_cast<long long>(M) * tuples) + t) * K];
                    bool any = false;
                    for (int k = 0; k < K; ++k) any = any || up[k] != 0.0;
                    if (!any) continue;
                    std::sort(idx.begin(), idx.begin() + nu);
                    auto& row = rows[{slot_base[bi] + M, idx}];
                    row.resize(static_cast<std::size_t>(num_el) * C, 0.0);
                    for (int e = 0; e < num_el; ++e)
                        for (int k = 0; k < K; ++k) {
                            if (up[k] == 0.0) continue;
                            const double* wr = &wv[(static_cast<std::size_t>(e) * K + k) * C];
                            for (int f = 0; f < C; ++f) row[static_cast<std::size_t>(e) * C + f] += up[k] * wr[f];
                        }
                }
        }
    }
    if (!P.agnostic && num_el != num_model_elements) bad("element-resolved product weights must cover every model element");
    if (P.agnostic && num_el != 1) bad("an agnostic product holds one weight element");
    P.num_elements = num_el;
    std::vector<std::pair<std::pair<int, std::array<int, 3>>, const std::vector<double>*>> kept;
    for (const auto& kv : rows)
        if (std::any_of(kv.second.begin(), kv.second.end(), [](double x) { return x != 0.0; }))
            kept.push_back({kv.first, &kv.second});
    P.num_terms = static_cast<int>(kept.size());
    P.coef.assign(static_cast<std::size_t>(num_el) * P.num_terms * C, 0.0f);
    for (int t = 0; t < P.num_terms; ++t) {
        const auto& key = kept[t].first;
        P.terms.insert(P.terms.end(), {key.second[0], key.second[1], key.second[2], key.first});
        for (int e = 0; e < num_el; ++e)
            for (int f = 0; f < C; ++f)
                P.coef[(static_cast<std::size_t>(e) * P.num_terms + t) * C + f] =
                    static_cast<float>((*kept[t].second)[static_cast<std::size_t>(e) * C + f]);
    }
    return P;
}

void analyze_family(Model& M, const Value& root) {
    auto reject = [&](const char* why) { M.family = false; M.family_rejection = why; };
    const auto& its = root.at("interactions").items;
    if (its.size() != 2 || root.at("products").items.size() != 2 || root.at("readouts").items.size() != 2)
        return reject("the MH-1 family has exactly two interactions");
    if (M.l_max != 2 && M.l_max != 3) return reject("the MH-1 family has l_max 2 or 3");
    const Irreps n0(its[0].at("node_feats_irreps").as_string()), e0(its[0].at("edge_irreps").as_string());
    if (n0.blocks.size() != 1 || n0.blocks[0].l != 0 || n0.blocks[0].parity != 1 || e0.blocks.size() != 1 ||
        e0.blocks[0].l != 0 || e0.blocks[0].parity != 1)
        return reject("the first MH-1 interaction has scalar nodes and edges");
    const int C = n0.blocks[0].mul, E = e0.blocks[0].mul;
    const std::vector<Block> full = spherical(C, M.l_max, C), gate_in = spherical(C, M.l_max, (M.l_max + 1) * C);
    const std::vector<Block> hid0{{C, 0, 1, 0}, {C, 1, -1, 0}}, hid1{{C, 0, 1, 0}}, e1{{E, 0, 1, 0}, {E, 1, -1, 0}};
    if (!same_blocks(Irreps(its[1].at("node_feats_irreps").as_string()), hid0) ||
        !same_blocks(Irreps(its[1].at("edge_irreps").as_string()), e1) ||
        !same_blocks(Irreps(its[0].at("hidden_irreps").as_string()), hid0) ||
        !same_blocks(Irreps(its[1].at("hidden_irreps").as_string()), hid1))
        return reject("MH-1 node, edge and hidden irreps do not chain");
    for (const Value& it : its)
        if (!same_blocks(Irreps(it.at("target_irreps").as_string()), full) ||
            !same_blocks(Irreps(it.at("gate").at("irreps_in").as_string()), gate_in) ||
            !same_blocks(Irreps(it.at("gate").at("irreps_out").as_string()), full))
            return reject("MH-1 target and gate irreps are not the family's");
    for (int k = 0; k < 2; ++k) {
        const Value& p = root.at("products").items[k];
        if (!M.products[k].use_sc || !M.products[k].agnostic)
            return reject("MH-1 products are agnostic with skip connections");
        for (const Value& c : p.at("symmetric_contractions").at("contractions").items)
            if (c.at("correlation").as_int() != 3) return reject("MH-1 products have correlation three");
        if (!same_blocks(Irreps(p.at("symmetric_contractions").at("irreps_out").as_string()), k == 0 ? hid0 : hid1))
            return reject("MH-1 product outputs are not the family's");
    }
    for (const Interaction& it : M.interactions)
        if (it.tp.channels != E) return reject("MH-1 convolutions use the edge channel count");
    if (M.readouts[0].nonlinear || !M.readouts[1].nonlinear)
        return reject("MH-1 has a linear then a nonlinear readout");
    M.family = true;
    M.family_node_channels = C;
    M.family_edge_channels = E;
    M.family_radial = static_cast<int>(M.bessel.size());
}

}  // namespace

Model Model::load(const std::string& path, const std::string& head) {
    const Value root = json_lite::parse_file(path);
    if (!root.is_object() || root.get_string("model_type", "") != "MACE_Nonlinear")
        bad("'" + path + "' is not a MACE_Nonlinear model file");
    const int version = root.at("symmetrix_format_version").as_int();
    if (version != 3 && version != 4) bad("format version " + std::to_string(version) + " is not 3 or 4");
    Model M;
    const Value* hv = root.find("head");
    M.selected_head = (hv && hv->is_string()) ? hv->as_string() : root.get_string("selected_head", "");
    if (!head.empty() && head != M.selected_head)
        bad("the file holds head '" + M.selected_head + "', not '" + head + "'");
    M.atomic_numbers = root.at("atomic_numbers").as_ints();
    M.model_atomic_numbers = root.at("model_atomic_numbers").as_ints();
    M.model_indices = root.at("model_indices").as_ints();
    M.num_model_elements = static_cast<int>(M.model_atomic_numbers.size());
    if (M.atomic_numbers.empty() || M.model_indices.size() != M.atomic_numbers.size() ||
        root.at("num_elements").as_int() != static_cast<int>(M.atomic_numbers.size()) ||
        std::set<int>(M.atomic_numbers.begin(), M.atomic_numbers.end()).size() != M.atomic_numbers.size() ||
        std::set<int>(M.model_atomic_numbers.begin(), M.model_atomic_numbers.end()).size() !=
            M.model_atomic_numbers.size())
        bad("element lists are empty, repeated or of different lengths");
    for (std::size_t t = 0; t < M.atomic_numbers.size(); ++t) {
        const int mi = M.model_indices[t];
        if (M.atomic_numbers[t] <= 0 || mi < 0 || mi >= M.num_model_elements ||
            M.model_atomic_numbers[mi] != M.atomic_numbers[t])
            bad("model_indices do not map each element onto the model's elements");
    }
    M.r_cut = root.at("r_cut").as_number();
    M.l_max = root.at("l_max").as_int();
    if (!(M.r_cut > 0.0) || !std::isfinite(M.r_cut)) bad("r_cut must be positive and finite");
    if (M.l_max < 0 || M.l_max > 3) bad("harmonics are built for l_max 0..3");
    M.num_lm = (M.l_max + 1) * (M.l_max + 1);
    const Value& rad = root.at("radial_embedding");
    M.apply_cutoff = rad.at("apply_cutoff").as_bool();
    if (rad.at("basis").at("type").as_string() != "bessel" || rad.at("cutoff").at("type").as_string() != "polynomial")
        bad("only the Bessel basis with the polynomial cutoff is supported");
    M.bessel = tensor_values(rad.at("basis").at("weights"), "Bessel weights");
    M.prefactor = rad.at("basis").at("prefactor").as_number();
    M.cutoff_p = rad.at("cutoff").at("p").as_int();
    if (M.bessel.empty() || M.bessel.size() > 32 || M.cutoff_p < 1 || rad.at("cutoff").at("r_max").as_number() != M.r_cut)
        bad("the radial basis needs 1..32 functions, p >= 1 and the model's r_cut");
    const Value& tr = rad.at("distance_transform");
    const std::string kind = tr.at("type").as_string();
    if (kind == "agnesi") {
        M.agnesi = true;
        M.agnesi_a = tr.at("a").as_number();
        M.agnesi_q = tr.at("q").as_number();
        M.agnesi_p = tr.at("p").as_number();
        M.covalent_radii = tr.at("covalent_radii").as_doubles();
        for (int z : M.model_atomic_numbers)
            if (z >= static_cast<int>(M.covalent_radii.size()) || !(M.covalent_radii[z] > 0.0))
                bad("the Agnesi transform lacks a covalent radius for Z=" + std::to_string(z));
    } else if (kind != "none") {
        bad("distance transform '" + kind + "' is not supported");
    }
    const std::vector<double> scale = tensor_values(root.at("scale_shift").at("scale"), "scale");
    const std::vector<double> shift = tensor_values(root.at("scale_shift").at("shift"), "shift");
    if (scale.size() != 1 || shift.size() != 1) bad("scale and shift must be single numbers");
    M.scale = scale[0];
    M.shift = shift[0];
    const std::vector<double> ae = tensor_values(root.at("atomic_energies"), "atomic energies");
    if (static_cast<int>(ae.size()) != M.num_model_elements) bad("one atomic energy per model element is required");
    for (int mi : M.model_indices) M.atomic_energies.push_back(ae[mi]);
    M.embedding = Linear(root.at("node_embedding"));
    if (M.embedding.in.dim != M.num_model_elements) bad("the node embedding must take the one-hot of the model elements");

    const int nt = static_cast<int>(M.atomic_numbers.size());
    const int R = static_cast<int>(M.bessel.size());
    const auto& its = root.at("interactions").items;
    const auto& prods = root.at("products").items;
    const auto& ros = root.at("readouts").items;
    const int ni = root.at("num_interactions").as_int();
    if (ni <= 0 || static_cast<int>(its.size()) != ni || static_cast<int>(prods.size()) != ni ||
        static_cast<int>(ros.size()) != ni)
        bad("interaction, product and readout counts disagree");
    int feat_dim = M.embedding.out.dim;
    for (int k = 0; k < ni; ++k) {
        const Value& v = its[k];
        if (v.at("class").as_string() != "RealAgnosticResidualNonLinearInteractionBlock")
            bad("interaction class '" + v.at("class").as_string() + "' is not supported");
        Interaction I;
        I.source_embedding = Linear(v.at("source_embedding"));
        I.target_embedding = Linear(v.at("target_embedding"));
        I.up = Linear(v.at("linear_up"));
        I.skip = Linear(v.at("skip_tp"));
        I.res = Linear(v.at("linear_res"));
        I.lin1 = Linear(v.at("linear_1"));
        I.lin2 = Linear(v.at("linear_2"));
        I.tp = build_tp(v.at("conv_tp"), M.l_max);
        I.alpha = v.at("alpha").as_number();
        I.beta = v.at("beta").as_number();
        I.gate = build_gate(v.at("gate"));
        std::vector<std::vector<double>> se, te;
        for (int t = 0; t < nt; ++t) {
            std::vector<double> onehot(M.num_model_elements, 0.0);
            onehot[M.model_indices[t]] = 1.0;
            se.push_back(linear_apply(I.source_embedding, onehot));
            te.push_back(linear_apply(I.target_embedding, onehot));
        }
        if (I.source_embedding.in.dim != M.num_model_elements || I.target_embedding.in.dim != M.num_model_elements)
            bad("edge embeddings must take the one-hot of the model elements");
        I.weights_mlp = build_mlp(v.at("conv_tp_weights"), R, se, te, "convolution weight MLP");
        I.density_mlp = build_mlp(v.at("density_fn"), R, se, te, "density MLP");
        if (I.weights_mlp.out_dim != I.tp.numel) bad("the weight MLP output differs from the convolution's weight count");
        if (I.density_mlp.out_dim != 1) bad("the density MLP must have one output");
        if (I.up.in.dim != feat_dim || I.skip.in.dim != feat_dim) bad("linear_up / skip_tp do not take the node features");
        if (I.up.out.dim != I.tp.in1_dim) bad("linear_up does not produce the convolution's first input");
        if (I.lin1.in.dim != I.tp.out_dim) bad("linear_1 does not take the messages");
        if (I.res.in.dim != I.up.out.dim || I.res.out.dim != I.lin1.out.dim || I.lin1.out.dim != I.gate.in_dim)
            bad("linear_res / linear_1 / gate widths disagree");
        if (I.lin2.in.dim != I.gate.out_dim) bad("linear_2 does not take the gate's output");
        const int channels = I.tp.channels;
        if (channels > 64 || (channels & (channels - 1)))
            throw std::domain_error("MH-1 model: convolution channel counts must be a power of two up to 64");
        if (I.tp.slots > 64 || I.tp.in1_per_channel > 16)
            throw std::domain_error("MH-1 model: the convolution has more than 64 output or 16 input components per channel");
        M.interactions.push_back(std::move(I));
        ProductTables P = build_product(prods[k], M.num_model_elements);
        if (P.in_dim != M.interactions[k].lin2.out.dim) bad("the product does not take linear_2's output");
        if (P.out_dim != M.interactions[k].skip.out.dim) bad("skip_tp does not produce the product's output");
        if (P.angular > 16 || P.out_slots > 16)
            throw std::domain_error("MH-1 model: product angular or output components above 16");
        feat_dim = P.out_dim;
        M.products.push_back(std::move(P));
        const Value& r = ros[k];
        Readout ro;
        const std::string cls = r.at("class").as_string();
        if (cls == "LinearReadoutBlock") {
            ro.lin1 = Linear(r.at("linear"));
        } else if (cls == "NonLinearReadoutBlock") {
            if (r.at("activation").as_string() != "silu") bad("nonlinear readouts use SiLU");
            ro.nonlinear = true;
            ro.lin1 = Linear(r.at("linear_1"));
            ro.lin2 = Linear(r.at("linear_2"));
            ro.activation_constant = r.at("activation_constants").as_doubles().at(0);
            if (ro.lin2.in.dim != ro.lin1.out.dim || ro.lin2.out.dim != 1) bad("nonlinear readout widths disagree");
        } else {
            bad("readout class '" + cls + "' is not supported");
        }
        if (ro.lin1.in.dim != feat_dim || (!ro.nonlinear && ro.lin1.out.dim != 1)) bad("readout widths disagree");
        M.readouts.push_back(std::move(ro));
    }
    M.has_zbl = root.at("has_zbl").as_bool();
    if (M.has_zbl) {
        const Value& z = root.at("zbl");
        M.zbl_a_exp = z.at("a_exp").as_number();
        M.zbl_a_prefactor = z.at("a_prefactor").as_number();
        const std::vector<double> c = tensor_values(z.at("c"), "ZBL c");
        if (c.size() != 4) bad("ZBL takes four screening coefficients");
        for (int i = 0; i < 4; ++i) M.zbl_c[i] = c[i];
        M.zbl_radii = tensor_values(z.at("covalent_radii"), "ZBL radii");
        M.zbl_p = static_cast<int>(tensor_values(z.at("p"), "ZBL p").at(0));
        for (int zz : M.atomic_numbers)
            if (zz >= static_cast<int>(M.zbl_radii.size())) bad("ZBL radii do not cover Z=" + std::to_string(zz));
        if (!(M.zbl_a_prefactor > 0.0) || M.zbl_p < 1) bad("ZBL parameters out of range");
    }
    analyze_family(M, root);
    return M;
}

}  // namespace mh1
}  // namespace smx
