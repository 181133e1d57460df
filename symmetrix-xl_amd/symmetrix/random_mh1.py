"""Seeded random-init MH-1 (``MACE_Nonlinear``) models in the reference's
nonlinear JSON schema.

The schema is the one the reference's extractor writes for models whose
interactions are ``RealAgnosticResidualNonLinearInteractionBlock``
(symmetrix/source/symmetrix/extract_mace_nonlinear.py:19-400) and its
evaluator reads (libsymmetrix/source/mace_nonlinear.cpp:302-380,
mace_nonlinear_schema.cpp:209-305, e3nn.cpp, e3nn_product.cpp:58-120,
affine_mlp.cpp:38-110).  mace-torch and e3nn are not installed here, so this
module builds the e3nn pieces itself from ``symmetrix.e3``:

* ``o3.Linear``: one instruction per (input block, output block) of equal
  irrep, weight shape ``path_shape = [mul_in, mul_out]`` (row-major, the
  output index fastest), path weight ``1/sqrt(sum of mul_in into the output
  block)`` (e3nn's "element" path normalisation); ``output_mask`` is 1 on
  output blocks that some instruction reaches.
* the convolution tensor product: "uvu" paths of the edge features and the
  spherical harmonics, one output block per path sorted by l (MACE's
  ``tp_out_irreps_with_instructions``), external weights, e3nn's real Wigner
  3j and path weight ``sqrt(2 l_out + 1)``.
* the symmetric contraction: per output irrep and degree nu, a basis of the
  degree-nu O(3)-equivariant polynomials of the (l_max+1)^2 angular
  components (``e3.symmetric_basis``), spread evenly over every ordering of
  each monomial's indices (symmetric U tensors, as mace's ``U_matrix_real``
  are), with agnostic weights ``[1, K, channels]``.

The architecture is the MH-1 family's (mace_nonlinear_schema.cpp:108-207):
two interactions; scalar node and edge features in the first; ``Cx0e+Cx1o``
nodes and ``Ex0e+Ex1o`` edges in the second; gate input
``(l_max+1)C x0e + Cx1o + ... ``; correlation-three agnostic products with
skip connections; a linear then a nonlinear readout.  Values are rounded to
float32 before they are written, so the FP32 and FP64 readers of a file see
the same numbers.
"""

from __future__ import annotations

import itertools
import json
import math
import os
from dataclasses import dataclass, field

import numpy as np

from . import e3

SILU_SCALE = 1.6791767923989418      # e3nn normalize2mom(silu)
SIGMOID_SCALE = 1.8467055342154763   # e3nn normalize2mom(sigmoid)


@dataclass
class MH1Config:
    name: str
    node_channels: int = 16
    edge_channels: int = 8
    l_max: int = 2
    atomic_numbers: list = field(default_factory=lambda: [1, 6, 8, 14])
    num_bessel: int = 8
    cutoff_p: int = 5
    r_cut: float = 5.0
    embedding_dim: int = 4
    radial_hidden: list = field(default_factory=lambda: [16, 16])
    density_hidden: int = 8
    readout_hidden: int = 8
    correlation: int = 3
    apply_cutoff: bool = True
    agnesi: bool = False
    zbl: bool = False
    linear_bias: bool = False
    # highest l of the first interaction's output (the MH-1 family has 1;
    # 2 gives a convolution structure outside the family's compiled ones)
    hidden_lmax: int = 1
    seed: int = 0


MH1_CONFIGS = {
    "mh1_tiny": MH1Config("mh1_tiny"),
    "mh1_tiny_l3": MH1Config("mh1_tiny_l3", l_max=3, node_channels=8, edge_channels=8, seed=1),
    "mh1_tiny_raw": MH1Config("mh1_tiny_raw", apply_cutoff=False, agnesi=True, zbl=True, linear_bias=True,
                              seed=2),
    "mh1_tiny_l2e": MH1Config("mh1_tiny_l2e", node_channels=8, edge_channels=4, hidden_lmax=2, seed=4),
    # edge-MLP forms: one 32-wide LayerNorm stage (and a 16-wide density stage), and four stages (beyond
    # the register-form kernels' three, so the LDS-tile kernels with LayerNorm) with a 32-wide density stage
    "mh1_tiny_mlp32": MH1Config("mh1_tiny_mlp32", radial_hidden=[32], density_hidden=16, seed=5),
    "mh1_tiny_mlp4": MH1Config("mh1_tiny_mlp4", radial_hidden=[16, 16, 16, 16], density_hidden=32, seed=6),
    # channel counts of the MH-1 family's small members
    "mh1_medium": MH1Config("mh1_medium", node_channels=64, edge_channels=32, l_max=3,
                            atomic_numbers=[1, 6, 7, 8, 13, 14, 22, 26, 29, 38], r_cut=6.0,
                            embedding_dim=16, radial_hidden=[64, 64, 64], density_hidden=32,
                            readout_hidden=16, seed=3),
}

_COVALENT = {1: 0.31, 6: 0.76, 7: 0.71, 8: 0.66, 13: 1.21, 14: 1.11, 22: 1.60, 26: 1.32, 29: 1.32, 38: 1.95}


def _f32(a):
    return np.asarray(a, dtype=np.float32).astype(np.float64)


def _tensor(values, shape):
    v = _f32(np.asarray(values, dtype=np.float64).reshape(-1))
    return {"shape": list(shape), "values": [float("%.9g" % x) for x in v.tolist()]}


def _parity_char(p):
    return "e" if p > 0 else "o"


def irreps_str(blocks):
    return "+".join("%dx%d%s" % (m, l, _parity_char(p)) for m, l, p in blocks)


def _full(C, l_max, scalar_copies=1):
    return [(scalar_copies * C, 0, 1)] + [(C, l, (-1) ** l) for l in range(1, l_max + 1)]


def _dim(blocks):
    return sum(m * (2 * l + 1) for m, l, _ in blocks)


def linear(rng, in_blocks, out_blocks, bias=False, scale=1.0):
    """e3nn ``o3.Linear`` in the extractor's layout (extract_mace_nonlinear.py:48-56)."""
    instructions = []
    weights = []
    fan = [0] * len(out_blocks)
    pairs = []
    for i, (mi, li, pi) in enumerate(in_blocks):
        for o, (mo, lo, po) in enumerate(out_blocks):
            if li == lo and pi == po:
                pairs.append((i, o))
                fan[o] += mi
    mask = []
    for o, (mo, lo, po) in enumerate(out_blocks):
        mask += [1.0 if fan[o] else 0.0] * (mo * (2 * lo + 1))
    for i, o in pairs:
        mi, mo = in_blocks[i][0], out_blocks[o][0]
        instructions.append({"i_in": i, "i_out": o, "path_shape": [mi, mo],
                             "path_weight": 1.0 / math.sqrt(fan[o])})
        weights.append(scale * rng.normal(size=mi * mo))
    w = np.concatenate(weights) if weights else np.zeros(0)
    out_dim = _dim(out_blocks)
    if bias:
        b = np.zeros(out_dim)
        off = 0
        for mo, lo, po in out_blocks:
            if lo == 0:
                b[off:off + mo] = 0.1 * rng.normal(size=mo)
            off += mo * (2 * lo + 1)
        bias_t = _tensor(b, [out_dim])
    else:
        bias_t = _tensor([], [0])
    return {"irreps_in": irreps_str(in_blocks), "irreps_out": irreps_str(out_blocks),
            "instructions": instructions, "weight": _tensor(w, [len(w)]), "bias": bias_t,
            "output_mask": _tensor(mask, [len(mask)])}


def conv_tp(in1_blocks, l_max):
    """The "uvu" convolution of edge features with Y_0..Y_lmax, one output
    block per path, paths sorted by output l (stable), external weights."""
    sh = [(1, l, (-1) ** l) for l in range(l_max + 1)]
    paths = []
    for i1, (m1, l1, p1) in enumerate(in1_blocks):
        for i2, (_, l2, p2) in enumerate(sh):
            for l3 in range(abs(l1 - l2), l1 + l2 + 1):
                if l3 <= l_max and p1 * p2 == (-1) ** l3:
                    paths.append((i1, i2, l3, p1 * p2, m1))
    order = sorted(range(len(paths)), key=lambda k: paths[k][2])
    out_blocks = []
    position = {}
    for pos, k in enumerate(order):
        position[k] = pos
        out_blocks.append((paths[k][4], paths[k][2], paths[k][3]))
    instructions = []
    for k, (i1, i2, l3, p3, m1) in enumerate(paths):
        l1 = in1_blocks[i1][1]
        l2 = sh[i2][1]
        w3j = e3.wigner_3j(l1, l2, l3)
        instructions.append({"i_in1": i1, "i_in2": i2, "i_out": position[k], "connection_mode": "uvu",
                             "has_weight": True, "path_weight": math.sqrt(2 * l3 + 1),
                             "path_shape": [m1, 1], "wigner_3j": _tensor(w3j, list(w3j.shape))})
    numel = sum(p[4] for p in paths)
    return {"irreps_in1": irreps_str(in1_blocks), "irreps_in2": irreps_str(sh),
            "irreps_out": irreps_str(out_blocks), "instructions": instructions,
            "weight": _tensor([], [0]), "output_mask": _tensor(np.ones(_dim(out_blocks)), [_dim(out_blocks)])}, \
        out_blocks, numel


def affine_mlp(rng, sizes, layer_norm=True):
    """Linear / LayerNorm / SiLU stack (extract_mace_nonlinear.py:105-134)."""
    layers = []
    for k in range(len(sizes) - 1):
        fan_in, fan_out = sizes[k], sizes[k + 1]
        layers.append({"type": "linear",
                       "weight": _tensor(rng.normal(size=(fan_out, fan_in)) / math.sqrt(fan_in), [fan_out, fan_in]),
                       "bias": _tensor(0.1 * rng.normal(size=fan_out), [fan_out])})
        if k < len(sizes) - 2:
            if layer_norm:
                layers.append({"type": "layer_norm", "normalized_shape": [fan_out], "eps": 1e-5,
                               "weight": _tensor(1.0 + 0.1 * rng.normal(size=fan_out), [fan_out]),
                               "bias": _tensor(0.1 * rng.normal(size=fan_out), [fan_out])})
            layers.append({"type": "silu"})
    return {"layers": layers}


def _u_tensor(l_max, L, nu):
    """Symmetric U tensor [(2L+1 if L>0), n, ..., n, K] of the degree-nu
    equivariant polynomials (each monomial's coefficient spread over every
    ordering of its indices)."""
    n = (l_max + 1) ** 2
    monos, U = e3.symmetric_basis(l_max, L, nu)
    K = U.shape[0]
    d = 2 * L + 1
    T = np.zeros((d,) + (n,) * nu + (K,))
    for j, mono in enumerate(monos):
        perms = set(itertools.permutations(mono))
        for p in perms:
            T[(slice(None),) + tuple(p) + (slice(None),)] = U[:, :, j].T / len(perms)
    if L == 0:
        T = T[0]
    return T


def product(rng, l_max, C, out_blocks, correlation):
    """Agnostic symmetric contraction + linear with skip connection
    (extract_mace_nonlinear.py:225-250)."""
    full = _full(C, l_max)
    contractions = []
    for (_, L, _) in out_blocks:
        us = []
        ws = {}
        for nu in range(1, correlation + 1):
            T = _u_tensor(l_max, L, nu)
            us.append(_tensor(T, list(T.shape)))
            K = T.shape[-1]
            ws[nu] = _tensor(rng.normal(size=(1, K, C)) / math.sqrt(max(K, 1)) * (0.35 ** (nu - 1)), [1, K, C])
        contractions.append({"correlation": correlation,
                             "weights": [ws[nu] for nu in range(correlation - 1, 0, -1)],
                             "weights_max": ws[correlation], "u_tensors": us})
    return {"node_feats_irreps": irreps_str(out_blocks), "target_irreps": irreps_str(out_blocks),
            "use_sc": True, "use_agnostic_product": True,
            "linear": linear(rng, out_blocks, out_blocks),
            "symmetric_contractions": {"irreps_in": irreps_str(full), "irreps_out": irreps_str(out_blocks),
                                       "contractions": contractions}}


def gate(C, l_max):
    return {"irreps_in": irreps_str(_full(C, l_max, l_max + 1)), "irreps_out": irreps_str(_full(C, l_max)),
            "irreps_scalars": irreps_str([(C, 0, 1)]),
            "irreps_gates": irreps_str([(C, 0, 1)] * l_max),
            "irreps_gated": irreps_str([(C, l, (-1) ** l) for l in range(1, l_max + 1)]),
            "scalar_activation": "silu", "scalar_activation_constants": [SILU_SCALE],
            "gate_activation": "sigmoid", "gate_activation_constants": [SIGMOID_SCALE] * l_max}


def interaction(rng, cfg, layer, num_elements):
    C, E, l = cfg.node_channels, cfg.edge_channels, cfg.l_max
    vec = [(C, l, (-1) ** l) for l in range(cfg.hidden_lmax + 1)]
    node = [(C, 0, 1)] if layer == 0 else vec
    edge = [(E, 0, 1)] if layer == 0 else [(E, l, (-1) ** l) for l in range(cfg.hidden_lmax + 1)]
    hidden = vec if layer == 0 else [(C, 0, 1)]
    full = _full(C, l)
    gate_in = _full(C, l, l + 1)
    tp, msg_blocks, numel = conv_tp(edge, l)
    S = cfg.embedding_dim
    cond = cfg.num_bessel + 2 * S
    elements = [(num_elements, 0, 1)]
    return {"class": "RealAgnosticResidualNonLinearInteractionBlock",
            "node_feats_irreps": irreps_str(node), "target_irreps": irreps_str(full),
            "hidden_irreps": irreps_str(hidden), "edge_irreps": irreps_str(edge),
            "avg_num_neighbors": 20.0,
            "alpha": float(_f32(2.0 + 0.5 * rng.random())), "beta": float(_f32(0.2 + 0.3 * rng.random())),
            "source_embedding": linear(rng, elements, [(S, 0, 1)]),
            "target_embedding": linear(rng, elements, [(S, 0, 1)]),
            "linear_up": linear(rng, node, edge, bias=cfg.linear_bias),
            "skip_tp": linear(rng, node, hidden),
            "linear_res": linear(rng, edge, gate_in),
            # messages sum over ~20-70 neighbours: keep the pre-gate values O(1)
            "linear_1": linear(rng, msg_blocks, gate_in, scale=0.15),
            "linear_2": linear(rng, full, full),
            "conv_tp": tp,
            "conv_tp_weights": affine_mlp(rng, [cond] + list(cfg.radial_hidden) + [numel]),
            "density_fn": affine_mlp(rng, [cond, cfg.density_hidden, 1], layer_norm=False),
            "gate": gate(C, l)}


def generate_mh1(cfg, seed=None):
    rng = np.random.default_rng(cfg.seed if seed is None else seed)
    Z = list(cfg.atomic_numbers)
    n_el = len(Z)
    C, l = cfg.node_channels, cfg.l_max
    hidden = [[(C, l, (-1) ** l) for l in range(cfg.hidden_lmax + 1)], [(C, 0, 1)]]
    model = {
        "symmetrix_format_version": 4, "model_type": "MACE_Nonlinear", "head": None,
        "atomic_numbers": Z, "model_atomic_numbers": Z, "model_indices": list(range(n_el)),
        "num_elements": n_el, "r_cut": float(cfg.r_cut), "l_max": l, "num_interactions": 2,
        "atomic_energies": _tensor(-1.0 - 3.0 * rng.random(n_el), [1, n_el]),
        "scale_shift": {"scale": _tensor([0.8 + 0.4 * rng.random()], []),
                        "shift": _tensor([0.05 * rng.normal()], [])},
        "node_embedding": linear(rng, [(n_el, 0, 1)], [(C, 0, 1)]),
        "radial_embedding": {
            "apply_cutoff": bool(cfg.apply_cutoff),
            "basis": {"type": "bessel",
                      "weights": _tensor(math.pi / cfg.r_cut * np.arange(1, cfg.num_bessel + 1), [cfg.num_bessel]),
                      "prefactor": math.sqrt(2.0 / cfg.r_cut)},
            "cutoff": {"type": "polynomial", "r_max": float(cfg.r_cut), "p": cfg.cutoff_p},
            "distance_transform": {"type": "none"}},
        "interactions": [interaction(rng, cfg, k, n_el) for k in range(2)],
        "products": [product(rng, l, C, hidden[k], cfg.correlation) for k in range(2)],
        "readouts": [
            {"class": "LinearReadoutBlock", "linear": linear(rng, hidden[0], [(1, 0, 1)]),
             "linear_1": None, "linear_2": None, "activation": None, "activation_constants": None},
            {"class": "NonLinearReadoutBlock", "linear": None,
             "linear_1": linear(rng, hidden[1], [(cfg.readout_hidden, 0, 1)]),
             "linear_2": linear(rng, [(cfg.readout_hidden, 0, 1)], [(1, 0, 1)]),
             "activation": "silu", "activation_constants": [SILU_SCALE]}],
        "has_zbl": bool(cfg.zbl),
    }
    if cfg.agnesi:
        radii = [1.5] * (max(Z) + 1)
        for z in Z:
            radii[z] = _COVALENT.get(z, 1.5)
        model["radial_embedding"]["distance_transform"] = {
            "type": "agnesi", "a": 1.0805, "q": 0.9183, "p": 4.5791, "covalent_radii": radii}
    if cfg.zbl:
        radii = [1.0] * (max(Z) + 1)
        model["zbl"] = {"a_exp": 0.3, "a_prefactor": 0.4543,
                        "c": _tensor([0.1818, 0.5099, 0.2802, 0.02817], [4]),
                        "covalent_radii": _tensor(radii, [len(radii)]), "p": _tensor([6.0], [1])}
    return model


def write_mh1(cfg, path, seed=None):
    model = generate_mh1(cfg, seed)
    tmp = path + ".tmp%d" % os.getpid()
    with open(tmp, "w") as f:
        json.dump(model, f, separators=(",", ":"))
    os.replace(tmp, path)
    return path


def cached_mh1(config, seed=None, directory=None):
    """Path of a named MH-1 model, generated on first use under ``directory``
    (default: $SYMMETRIX_MODEL_CACHE or /tmp/symmetrix_models)."""
    cfg = config if isinstance(config, MH1Config) else MH1_CONFIGS[config]
    seed = cfg.seed if seed is None else seed
    directory = directory or os.environ.get("SYMMETRIX_MODEL_CACHE", "/tmp/symmetrix_models")
    os.makedirs(directory, exist_ok=True)
    path = os.path.join(directory, "%s_seed%d_v2.json" % (cfg.name, seed))
    if not os.path.exists(path):
        write_mh1(cfg, path, seed)
    return path
