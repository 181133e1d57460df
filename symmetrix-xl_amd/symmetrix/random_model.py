"""Seeded random-init MACE models in the reference's JSON format version 4.

The file layout is the one the reference's loaders read
(libsymmetrix/source/mace.cpp:2660-2959, mace_kokkos_model.cpp:146,
compact_radial.cpp:110-214, h1_affine_schema.hpp:196-259): compact radial
representation, h1_affine_mode "m0_composite".  A config with ``zbl`` adds
the ZBL pair repulsion with the parameters of the reference's ZBL test model
(symmetrix/test/conftest.py:177-184: a_exp 0.3, a_prefactor 0.4543, the
four screening coefficients, covalent radii 1.0 A, p 6).  A config with
``density_scaled`` adds the A0 and A1 density networks (one output,
"tanh-square" postprocessing, compact_radial.cpp:17-24,181-193) and sets
``A0_scaled``/``A1_scaled``; their weights come from a second generator
(``default_rng([seed, 1])``) so that every other weight equals the unscaled
config's.

Weights are drawn from ``numpy.random.default_rng(seed)`` with the fan-in
scalings the reference's extractor folds into its exported weights
(extract_mace_data.py:660-666 radial MLP, :922-933 H0, :982-1001 A0 with
1/avg_num_neighbors, :1166-1184 H1, :1439-1444 A1, :1590-1611 H2,
:1615-1680 readouts).  Values are rounded to float32 before they are written so
that the FP32 and FP64 readers of the file see the same numbers.

Named shapes (``MODEL_CONFIGS``) are the benchmark configurations: ``tiny``,
``medium`` and ``wide``.
"""

from __future__ import annotations

import json
import math
import os
from dataclasses import dataclass, field

import numpy as np

from . import e3

# e3nn normalize2mom(silu) constant: 1/sqrt(E[silu(z)^2]), z ~ N(0,1)
SILU_SCALE = 1.6791767923989418


@dataclass
class ModelConfig:
    name: str
    num_channels: int
    l_max: int
    L_max: int
    correlation: int
    atomic_numbers: list
    num_bessel: int = 8
    cutoff_p: int = 5
    radial_mlp: list = field(default_factory=lambda: [64, 64, 64])
    r_cut: float = 6.0
    avg_num_neighbors: float = 60.0
    num_spline_points: int = 256
    readout_hidden: int = 16
    # plays the role of MACE's scale_shift.scale folded into the readouts
    # (extract_mace_data.py:1623-1625,1676-1680)
    energy_scale: float = 10.0
    density_scaled: bool = False
    zbl: bool = False
    prediction_heads: bool = False
    agnesi: bool = False
    # h1_affine_mode: "m0_composite", or "pre_linear_up" with split H1 weights
    # (H1_product_weights P, H1_linear_up_weights U, H1_weights = P U) and the
    # readout_1 / skip maps on the pre-linear_up scalar x = M0[:,0,:] P0
    h1_mode: str = "m0_composite"
    # first_interaction_residual (pre_linear_up, or a one-interaction model
    # in either basis): per-type residual H1_first_residual_weights [type][LM][C]
    # with split H1 weights
    residual: bool = False
    # one interaction (single_layer_readout, extract_mace_data.py:1221-1262):
    # no R1 network, Phi1 or A1; M1 is a correlation-`readout_correlation`
    # invariant of H1's (L_max+1)^2 components.  The reference's extractor
    # writes zero readout_1 and skip maps for such a model; these are random
    # unless `zero_affine_maps`, so that the formulas that use them are tested.
    single_layer: bool = False
    readout_correlation: int = 2
    zero_affine_maps: bool = False
    # MACEField (pre_linear_up only): one field coupling, the electric field
    # (1x1o) times the canonical H1 irreps into the adjacent ranks, then a
    # per-l channel linear (extract_mace_data.py:562-598,769-819); weights
    # from default_rng([seed, 4])
    field: bool = False
    seed: int = 0


MODEL_CONFIGS = {
    # 32x0e+32x1o, lmax 2, corr 2, Sr/Ti/O, MLP [32,32], 5.0 A
    "tiny": ModelConfig("tiny", 32, 2, 1, 2, [8, 22, 38], radial_mlp=[32, 32],
                        r_cut=5.0, avg_num_neighbors=40.0),
    # tiny with A0/A1 density scaling (mace.cpp:1562-1636, 2381-2459)
    "tiny_scaled": ModelConfig("tiny_scaled", 32, 2, 1, 2, [8, 22, 38], radial_mlp=[32, 32],
                               r_cut=5.0, avg_num_neighbors=40.0, density_scaled=True),
    # tiny with two prediction heads (prediction_heads.hpp)
    "tiny_heads": ModelConfig("tiny_heads", 32, 2, 1, 2, [8, 22, 38], radial_mlp=[32, 32],
                              r_cut=5.0, avg_num_neighbors=40.0, prediction_heads=True),
    # tiny with the Agnesi distance transform (per-pair radial tables,
    # compact_radial.cpp:144-163,233-247) and density scaling (per-pair
    # density tables)
    "tiny_agnesi": ModelConfig("tiny_agnesi", 32, 2, 1, 2, [8, 22, 38], radial_mlp=[32, 32],
                               r_cut=5.0, avg_num_neighbors=40.0, agnesi=True, density_scaled=True),
    # tiny with ZBL pair repulsion (zbl_kokkos.cpp)
    "tiny_zbl": ModelConfig("tiny_zbl", 32, 2, 1, 2, [8, 22, 38], radial_mlp=[32, 32],
                            r_cut=5.0, avg_num_neighbors=40.0, zbl=True),
    # tiny in the pre_linear_up basis, without and with a first-interaction
    # residual (h1_affine_schema.hpp:196-259; mace.cpp:1759-1875)
    "tiny_plu": ModelConfig("tiny_plu", 32, 2, 1, 2, [8, 22, 38], radial_mlp=[32, 32],
                            r_cut=5.0, avg_num_neighbors=40.0, h1_mode="pre_linear_up"),
    "tiny_residual": ModelConfig("tiny_residual", 32, 2, 1, 2, [8, 22, 38], radial_mlp=[32, 32],
                                 r_cut=5.0, avg_num_neighbors=40.0, h1_mode="pre_linear_up", residual=True),
    # MACEField models (field_coupling.hpp; mace.cpp:322-395), L_max 1 and 2
    "tiny_field": ModelConfig("tiny_field", 32, 2, 1, 2, [8, 22, 38], radial_mlp=[32, 32],
                              r_cut=5.0, avg_num_neighbors=40.0, h1_mode="pre_linear_up", field=True),
    # with A0/A1 density scaling and ZBL (the response's density tangents)
    "tiny_field_scaled": ModelConfig("tiny_field_scaled", 32, 2, 1, 2, [8, 22, 38], radial_mlp=[32, 32],
                                     r_cut=5.0, avg_num_neighbors=40.0, h1_mode="pre_linear_up", field=True,
                                     density_scaled=True, zbl=True),
    # (L_max 2 at a compiled kernel shape: 128 channels, l_max 3)
    "field_l2": ModelConfig("field_l2", 128, 3, 2, 3, [8, 22, 38], radial_mlp=[32, 32],
                            r_cut=5.0, avg_num_neighbors=40.0, h1_mode="pre_linear_up", field=True,
                            residual=True),
    # one-interaction models (mace.cpp:255-281), plain and with a residual
    "tiny_single": ModelConfig("tiny_single", 32, 2, 1, 2, [8, 22, 38], radial_mlp=[32, 32],
                               r_cut=5.0, avg_num_neighbors=40.0, single_layer=True),
    "tiny_single_residual": ModelConfig("tiny_single_residual", 32, 2, 1, 2, [8, 22, 38], radial_mlp=[32, 32],
                                        r_cut=5.0, avg_num_neighbors=40.0, single_layer=True, residual=True),
    # the trained one-interaction shape (128x0e+128x1o, l_max 3, correlation
    # 3, readout correlation 2, A0 density scaling: test_single_layer_mace.py:
    # 71-81) on the benchmark's elements
    "medium_single": ModelConfig("medium_single", 128, 3, 1, 3, [8, 22, 38], radial_mlp=[64, 64, 64],
                                 r_cut=6.0, avg_num_neighbors=70.0, single_layer=True, density_scaled=True),
    # 128x0e+128x1o, lmax 3, corr 3, 89 elements,
    # MLP [64,64,64], 6.0 A
    "medium": ModelConfig("medium", 128, 3, 1, 3, list(range(1, 90)),
                          radial_mlp=[64, 64, 64], r_cut=6.0,
                          avg_num_neighbors=70.0),
    # 256 channels, 0e+1o+2e hidden, lmax 3, corr 3, 5.0 A
    "wide": ModelConfig("wide", 256, 3, 2, 3, [1, 8], radial_mlp=[64, 64, 64],
                        r_cut=5.0, avg_num_neighbors=40.0),
}


# Cordero et al. (2008) covalent radii (Angstrom) of the elements the named
# configs use; other elements get 1.5 A (the models are synthetic)
_COVALENT_RADII = {1: 0.31, 6: 0.76, 7: 0.71, 8: 0.66, 13: 1.21, 14: 1.11, 22: 1.60, 26: 1.32, 29: 1.32,
                   38: 1.95}


def _f32(a):
    return np.asarray(a, dtype=np.float32).astype(np.float64)


def _fmt(a):
    """Compact JSON list text of a flat float array (9 significant digits,
    exact for float32 values)."""
    a = np.asarray(a, dtype=np.float32).ravel()
    return "[" + ",".join("%.9g" % v for v in a.tolist()) + "]"


def _product_weights(rng, l_in_max, L_out, correlation, num_types, C, scale):
    """Per-(type, m_out, channel) polynomial coefficients over the monomial
    list of the reference's extractor (the U x W contraction,
    extract_mace_data.py:1013-1112).  The list is the structural support of
    the coupling-path tensors; the monomials whose symmetrised coefficient
    vanishes carry an exact zero, as the reference's file carries ~0."""
    d_out = 2 * L_out + 1
    keys_all = e3.structural_support(l_in_max, L_out, correlation)
    blocks = []
    for nu in range(1, correlation + 1):
        monos, U = e3.symmetric_basis(l_in_max, L_out, nu)
        if U.shape[0] == 0:
            continue
        W = rng.normal(size=(num_types, U.shape[0], C)) * (
            scale[nu - 1] / math.sqrt(U.shape[0]))
        blocks.append((monos, U, W))
    monos_all = [[] for _ in range(d_out)]
    coef_all = [None] * d_out
    for M in range(d_out):
        index = {k: i for i, k in enumerate(keys_all[M])}
        coef = np.zeros((num_types, C, len(index)))
        for monos, U, W in blocks:
            nz = np.nonzero(np.abs(U[:, M, :]).max(axis=0) > 1e-9)[0]
            cols = np.einsum("tec,ej->tcj", W, U[:, M, nz])
            for jj, j in enumerate(nz):
                coef[:, :, index[tuple(monos[j])]] += cols[:, :, jj]
        monos_all[M] = [list(k) for k in keys_all[M]]
        coef_all[M] = coef
    return monos_all, coef_all


def _field_coupling(C, L_max, rng):
    """One MACEField coupling in the extractor's schema-1 layout
    (extract_mace_data.py:562-598): field_feats instructions (l_in x 1o ->
    l_out, adjacent ranks, uvw, path shape (C, 1, C)) with e3nn's real 3j
    tensor of (l_in, 1, l_out), and field_linear instructions (l -> l,
    (C, C)); weights flat, [in][out] per instruction, float32 values."""
    irreps = "+".join("%dx%d%s" % (C, l, "o" if l % 2 else "e") for l in range(L_max + 1))
    feats, fw = [], []
    for l_in in range(L_max + 1):
        for l_out in (l_in - 1, l_in + 1):
            if not 0 <= l_out <= L_max:
                continue
            w3 = e3.wigner_3j(l_in, 1, l_out)
            feats.append({"i_in1": l_in, "i_in2": 0, "i_out": l_out, "connection_mode": "uvw", "has_weight": True,
                          "path_weight": float(_f32(1.0 / math.sqrt(C))), "path_shape": [C, 1, C],
                          "wigner_3j_shape": list(w3.shape), "wigner_3j": [float(v) for v in w3.ravel()]})
            fw.append(_f32(rng.normal(size=(C, C))))
    lins, lw = [], []
    for l in range(L_max + 1):
        lins.append({"i_in": l, "i_out": l, "path_weight": float(_f32(1.0 / math.sqrt(C))), "path_shape": [C, C]})
        lw.append(_f32(rng.normal(size=(C, C))))
    hidden = (L_max + 1) ** 2 * C
    return {"schema_version": 1,
            "field_feats_irreps_in1": irreps, "field_feats_irreps_in2": "1x1o", "field_feats_irreps_out": irreps,
            "field_feats_instructions": feats,
            "field_feats_weight": np.concatenate([w.ravel() for w in fw]).tolist(),
            "field_feats_output_mask": [1.0] * hidden,
            "field_linear_irreps_in": irreps, "field_linear_irreps_out": irreps,
            "field_linear_instructions": lins,
            "field_linear_weight": np.concatenate([w.ravel() for w in lw]).tolist(),
            "field_linear_bias": [],
            "field_linear_output_mask": [1.0] * hidden}


def generate_model(config, seed=None):
    """Return the model as a dict of JSON *text fragments* keyed by JSON key
    (large arrays pre-formatted), plus a small dict of plain metadata."""
    cfg = config if isinstance(config, ModelConfig) else MODEL_CONFIGS[config]
    if seed is None:
        seed = cfg.seed
    rng = np.random.default_rng(seed)
    C, l_max, L_max = cfg.num_channels, cfg.l_max, cfg.L_max
    n_el = len(cfg.atomic_numbers)
    num_lm, num_LM = (l_max + 1) ** 2, (L_max + 1) ** 2
    frag = {}

    def put(key, value):
        frag[key] = json.dumps(value)

    put("symmetrix_format_version", 4)
    put("model_type", "MACEField" if cfg.field else "MACE")
    if cfg.h1_mode not in ("m0_composite", "pre_linear_up"):
        raise ValueError("h1_mode must be m0_composite or pre_linear_up")
    if cfg.residual and cfg.h1_mode != "pre_linear_up" and not cfg.single_layer:
        raise ValueError("a first-interaction residual needs the pre_linear_up basis")
    if cfg.h1_mode == "pre_linear_up" and (cfg.prediction_heads or cfg.single_layer):
        raise ValueError("the pre_linear_up basis is generated for two-interaction models without heads")
    if cfg.field and (cfg.h1_mode != "pre_linear_up" or not 1 <= cfg.L_max <= 2):
        raise ValueError("a MACEField model needs the pre_linear_up basis and 1 <= L_max <= 2")
    pre = cfg.h1_mode == "pre_linear_up"
    put("h1_affine_mode", cfg.h1_mode)
    put("h1_affine_version", 1)
    put("generator", {"name": "symmetrix-mi355x random_model", "config": cfg.name,
                      "seed": seed})
    put("num_elements", n_el)
    put("num_channels", C)
    put("num_interactions", 1 if cfg.single_layer else 2)
    if cfg.single_layer:
        put("single_layer_readout", True)
        put("readout_correlation", cfg.readout_correlation)
    put("r_cut", cfg.r_cut)
    put("l_max", l_max)
    put("L_max", L_max)
    put("atomic_numbers", list(cfg.atomic_numbers))
    put("atomic_energies",
        [float(v) for v in _f32(-1.0 - 0.05 * np.asarray(cfg.atomic_numbers)
                                 + 0.1 * rng.normal(size=n_el))])
    put("has_zbl", bool(cfg.zbl))
    if cfg.zbl:
        put("zbl_a_exp", 0.3)
        put("zbl_a_prefactor", 0.4543)
        put("zbl_c", [0.1818, 0.5099, 0.2802, 0.02817])
        put("zbl_covalent_radii", [1.0] * 119)
        put("zbl_p", 6)
    put("radial_representation", "compact")

    # ---- compact radial (Bessel x polynomial cutoff -> SiLU MLPs)
    r_cut = cfg.r_cut
    bessel_w = _f32(np.arange(1, cfg.num_bessel + 1) * math.pi / r_cut)
    num_paths_r1 = len(e3.r1_paths(l_max, L_max))

    def mlp(out_width, gen=rng):
        shape = [cfg.num_bessel] + list(cfg.radial_mlp) + [out_width]
        weights = []
        for a, b in zip(shape[:-1], shape[1:]):
            # effective weight W / sqrt(h_in), layout [out][in]
            weights.append(_f32(gen.normal(size=(b, a)) / math.sqrt(a)))
        return {"shape": shape,
                "weights": [w.ravel().tolist() for w in weights],
                "activation": "silu",
                "activation_scale": SILU_SCALE}

    compact = {
        "spline_grid_min": 1e-12,
        "num_spline_points": cfg.num_spline_points,
        "basis": {"type": "bessel", "weights": bessel_w.tolist(),
                  "prefactor": float(_f32(math.sqrt(2.0 / r_cut)))},
        "cutoff": {"type": "polynomial", "r_max": r_cut, "p": cfg.cutoff_p},
        "distance_transform": (
            {"type": "agnesi", "a": 1.0805, "q": 0.9183, "p": 4.5791,
             "covalent_radii": [_COVALENT_RADII.get(z, 1.5) for z in cfg.atomic_numbers]}
            if cfg.agnesi else {"type": "none"}),
        "networks": {"R0": mlp((l_max + 1) * C)},
    }
    if not cfg.single_layer:
        compact["networks"]["R1"] = mlp(num_paths_r1 * C)
    if cfg.density_scaled:
        drng = np.random.default_rng([seed, 1])
        # a one-interaction model scales A0 only (it has no A1)
        for name in ("A0",) if cfg.single_layer else ("A0", "A1"):
            net = mlp(1, drng)
            # a larger last layer so that tanh(v^2) spans (0, 1) over the grid
            net["weights"][-1] = _f32(4.0 * np.asarray(net["weights"][-1])).tolist()
            net["postprocess"] = "tanh-square"
            compact["networks"][name] = net
    put("compact_radial", compact)

    # ---- H0: species embedding through linear_up
    frag["H0_weights"] = _fmt(rng.normal(size=(n_el, C)))
    put("A0_scaled", bool(cfg.density_scaled))

    # ---- A0: per species, per l, C x C [input][output]
    a0 = rng.normal(size=(n_el, l_max + 1, C, C)) / (
        math.sqrt(C) * cfg.avg_num_neighbors)
    frag["A0_weights"] = "[" + ",".join(
        "[" + ",".join(_fmt(a0[t, l]) for l in range(l_max + 1)) + "]"
        for t in range(n_el)) + "]"

    # ---- M0 symmetric contraction, outputs LM < (L_max+1)^2
    m0_weights = {str(t): {} for t in range(n_el)}
    m0_monos = {}
    parts = [[] for _ in range(n_el)]
    for L in range(L_max + 1):
        monos, coef = _product_weights(
            rng, l_max, L, cfg.correlation, n_el, C,
            scale=[1.0, 0.5, 0.25][:cfg.correlation] + [0.1] * 4)
        for M in range(2 * L + 1):
            lm = L * L + M
            m0_monos[str(lm)] = monos[M]
            for t in range(n_el):
                parts[t].append(
                    '"%d":{' % lm + ",".join(
                        '"%d":%s' % (k, _fmt(coef[M][t, k])) for k in range(C))
                    + "}")
    frag["M0_weights"] = "{" + ",".join(
        '"%d":{' % t + ",".join(parts[t]) + "}" for t in range(n_el)) + "}"
    put("M0_monomials", m0_monos)
    del m0_weights

    # ---- H1 = product linear x interaction[1].linear_up, per l
    h1 = rng.normal(size=(L_max + 1, C, C)) / math.sqrt(C)
    if pre or cfg.residual:
        # split weights from their own generator (the other draws stay those
        # of the m0_composite model of the same config)
        prng = np.random.default_rng([seed, 3])
        P = _f32(prng.normal(size=(L_max + 1, C, C)) / math.sqrt(C))
        U = _f32(prng.normal(size=(L_max + 1, C, C)) / math.sqrt(C))
        h1 = np.stack([P[l].astype(np.float64) @ U[l].astype(np.float64) for l in range(L_max + 1)])
        frag["H1_product_weights"] = _fmt(P)
        frag["H1_linear_up_weights"] = _fmt(U)
        put("first_interaction_residual", bool(cfg.residual))
        if cfg.residual:
            frag["H1_first_residual_weights"] = _fmt(0.3 * prng.normal(size=(n_el, num_LM, C)))
    if cfg.field:
        put("has_field_coupling", True)
        frag["field_couplings"] = json.dumps([_field_coupling(C, L_max, np.random.default_rng([seed, 4]))])
    frag["H1_weights"] = _fmt(h1)

    if cfg.single_layer:
        # no second interaction (extract_mace_data.py:1236-1248)
        for key in ("Phi1_l", "Phi1_l1", "Phi1_l2", "Phi1_lme", "Phi1_clebsch_gordan", "Phi1_lelm1lm2"):
            put(key, [])
        put("A1_weights", [[] for _ in range(l_max + 1)])
        put("A1_scaled", False)
    else:
        # ---- R1 coupling
        cpl = e3.r1_coupling(l_max, L_max)
        for key in ("Phi1_l", "Phi1_l1", "Phi1_l2", "Phi1_lme", "Phi1_lelm1lm2"):
            put(key, cpl[key])
        put("Phi1_clebsch_gordan", cpl["Phi1_clebsch_gordan"])
        put("A1_scaled", bool(cfg.density_scaled))

        # ---- A1: per l, [num_e(l)][C][C]
        num_e = [sum(1 for l in cpl["Phi1_l"] if l == ll) for ll in range(l_max + 1)]
        frag["A1_weights"] = "[" + ",".join(
            _fmt(rng.normal(size=(num_e[l], C, C))
                 / (math.sqrt(num_e[l] * C) * cfg.avg_num_neighbors))
            for l in range(l_max + 1)) + "]"

    # ---- M1: invariant contraction of A1 ((l_max+1)^2 harmonic components),
    # with the same correlation order as the first product basis; with one
    # interaction, of H1 ((L_max+1)^2 components) at the readout correlation
    if cfg.single_layer:
        monos1, coef1 = _product_weights(
            rng, L_max, 0, cfg.readout_correlation, n_el, C, scale=[1.0, 0.5, 0.25][:cfg.readout_correlation])
    else:
        monos1, coef1 = _product_weights(
            rng, l_max, 0, cfg.correlation, n_el, C, scale=[1.0, 0.5, 0.25][:cfg.correlation])
    put("M1_monomials", monos1[0])
    frag["M1_weights"] = "{" + ",".join(
        '"%d":{' % t + ",".join(
            '"%d":%s' % (k, _fmt(coef1[0][t, k])) for k in range(C)) + "}"
        for t in range(n_el)) + "}"

    # ---- H2 skip (T_z, [input][output]) and M1 linear; in the pre_linear_up
    # basis the skip and readout_1 act on x = M0[:,0,:] P0
    skip_key = "H2_weights_for_H1_pre_linear_up" if pre else "H2_weights_for_M0"
    affine = 0.0 if cfg.zero_affine_maps else 1.0
    frag[skip_key] = "[" + ",".join(
        _fmt(affine * rng.normal(size=(C, C)) / math.sqrt(C)) for _ in range(n_el)) + "]"
    frag["H2_weights_for_M1"] = _fmt(rng.normal(size=(C, C)) / math.sqrt(C))

    # ---- readouts
    hid = cfg.readout_hidden
    frag["readout_1_weights_for_H1_pre_linear_up" if pre else "readout_1_weights_for_M0"] = _fmt(
        affine * rng.normal(size=C) / math.sqrt(C) * cfg.energy_scale)
    put("readout_2_hidden_size", hid)
    frag["readout_2_weights_1"] = _fmt(rng.normal(size=(hid, C)) / math.sqrt(C))
    frag["readout_2_weights_2"] = _fmt(
        rng.normal(size=hid) / math.sqrt(hid) * cfg.energy_scale)
    put("readout_2_scale_factor", SILU_SCALE)
    if cfg.prediction_heads:
        # a "prediction_heads" section (schema 1, prediction_heads.hpp:30-88):
        # the top-level fields are the default head "default"; a second head
        # "finetune" has its own energies and readouts (second generator)
        hrng = np.random.default_rng([seed, 2])
        per_head = ["atomic_energies", "readout_1_weights_for_M0", "readout_2_weights_1",
                    "readout_2_weights_2"] + (["zbl_c"] if cfg.zbl else [])
        tuned = {
            "atomic_energies": _fmt(np.asarray(json.loads(frag["atomic_energies"])) + 0.3 * hrng.normal(size=n_el)),
            "readout_1_weights_for_M0": _fmt(hrng.normal(size=C) / math.sqrt(C) * cfg.energy_scale),
            "readout_2_weights_1": _fmt(hrng.normal(size=(hid, C)) / math.sqrt(C)),
            "readout_2_weights_2": _fmt(hrng.normal(size=hid) / math.sqrt(hid) * cfg.energy_scale),
        }
        if cfg.zbl:
            tuned["zbl_c"] = json.dumps([0.2, 0.5, 0.27, 0.03])

        def payload(src):
            return "{" + ",".join('"%s":%s' % (k, src[k]) for k in per_head) + "}"
        frag["prediction_heads"] = (
            '{"schema_version":1,"names":["default","finetune"],"default":"default","parameters":{'
            '"default":' + payload(frag) + ',"finetune":' + payload(tuned) + "}}")
    return frag


def write_model(config, path, seed=None):
    """Write the model JSON to ``path`` (atomically) and return the path."""
    frag = generate_model(config, seed)
    tmp = path + ".tmp%d" % os.getpid()
    with open(tmp, "w") as f:
        f.write("{\n")
        f.write(",\n".join('"%s":%s' % (k, v) for k, v in frag.items()))
        f.write("\n}\n")
    os.replace(tmp, path)
    return path


def cached_model(config, seed=None, directory=None):
    """Path of the model for a named config, generated on first use under
    ``directory`` (default: $SYMMETRIX_MODEL_CACHE or /tmp/symmetrix_models)."""
    cfg = config if isinstance(config, ModelConfig) else MODEL_CONFIGS[config]
    if seed is None:
        seed = cfg.seed
    directory = directory or os.environ.get(
        "SYMMETRIX_MODEL_CACHE", "/tmp/symmetrix_models")
    os.makedirs(directory, exist_ok=True)
    path = os.path.join(directory, "mace_%s_seed%d_v3.json" % (cfg.name, seed))
    if not os.path.exists(path):
        write_model(cfg, path, seed)
    return path
