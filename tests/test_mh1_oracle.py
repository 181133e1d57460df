"""MH-1 (MACE_Nonlinear) oracle: what pins it, on the CPU, FP64.

The reference's MH-1 tests build their models with mace-torch
(symmetrix/test/test_mh1.py:129-228), which is not installed, and no MH-1
model file ships with the reference; so the oracle (oracle/mh1_oracle.py) is
pinned by:
* central finite differences of the energy against its forces, for models
  with the cutoff on the features, on the weights (with Agnesi distances and
  ZBL) and with l_max 3 (test_mh1.py:1250 is the reference's FD test);
* rotation invariance of the energy and covariance of the forces (a basis
  mismatch between the Wigner 3j, the harmonics and the U tensors breaks it),
  translation and permutation invariance;
* hand-computed known answers for each block's layout: the linear's
  [mul_in, mul_out] weights, path weight, bias and mask (e3nn.cpp:146-166);
  the uvu path's weight index u*mul2+v and Wigner contraction
  (e3nn.cpp:343-357); the gate's scalars | gates | gated order
  (mace_nonlinear.cpp:80-100); the U x W contraction and the
  weights/weights_max degree rule (e3nn_product.cpp:86-93,332-369);
  the affine MLP against torch's Linear/LayerNorm/SiLU;
* planted mistakes: each of these checks fails for the mistake it names.
"""

import json

import numpy as np
import pytest

from oracle import mh1_oracle as mo
from oracle import oracle
from symmetrix import e3, random_mh1

MODELS = ["mh1_tiny", "mh1_tiny_raw", "mh1_tiny_l3", "mh1_tiny_l2e"]


@pytest.fixture(scope="module")
def paths(tmp_path_factory):
    d = str(tmp_path_factory.mktemp("mh1"))
    return {n: random_mh1.cached_mh1(n, directory=d) for n in MODELS}


def _system(model, n=12, L=7.0, seed=0):
    rng = np.random.default_rng(seed)
    pos = rng.random((n, 3)) * L
    # keep atoms at least 1.2 A apart (well inside the ZBL range all the same)
    for i in range(1, n):
        while True:
            d = pos[:i] - pos[i]
            d -= L * np.rint(d / L)
            if np.min(np.linalg.norm(d, axis=1)) > 1.2:
                break
            pos[i] = rng.random(3) * L
    nums = rng.choice(model.atomic_numbers, n)
    return pos, np.eye(3) * L, model.types_of(nums)


def _energy_forces(model, pos, cell, types, graph=None, ref_pos=None):
    if graph is None:
        graph = oracle.neighbor_graph(pos, cell, model.r_cut)
    ref = pos if ref_pos is None else ref_pos
    xyz, _ = oracle.prepared_geometry(graph, cell, ref, pos, 1e3)
    e, f = model.evaluate(types, graph["receivers"], graph["sources"], xyz)
    F = mo.reduce_forces(len(types), graph["receivers"], graph["sources"], f)
    S = mo.reduce_stress(f, xyz, abs(np.linalg.det(cell)))
    return e, F, S, graph


def _fd_error(model, pos, cell, types, h=1e-5, atoms=(0, 3, 7)):
    _, F, _, g = _energy_forces(model, pos, cell, types)
    err = 0.0
    for i in atoms:
        for c in range(3):
            p, m = pos.copy(), pos.copy()
            p[i, c] += h
            m[i, c] -= h
            ep = _energy_forces(model, p, cell, types, g, pos)[0].sum()
            em = _energy_forces(model, m, cell, types, g, pos)[0].sum()
            err = max(err, abs(-(ep - em) / (2 * h) - F[i, c]))
    return err, np.abs(F).max()


@pytest.mark.parametrize("name", MODELS)
def test_forces_match_finite_differences(paths, name):
    model = mo.MH1Oracle(paths[name])
    pos, cell, types = _system(model)
    err, scale = _fd_error(model, pos, cell, types)
    assert scale > 1e-2
    assert err < 1e-7 * max(1.0, scale), (err, scale)


@pytest.mark.parametrize("name", MODELS)
def test_stress_matches_strain_derivative(paths, name):
    model = mo.MH1Oracle(paths[name])
    pos, cell, types = _system(model, seed=1)
    _, _, S, g = _energy_forces(model, pos, cell, types)
    vol = abs(np.linalg.det(cell))
    h = 1e-6
    for a, b in ((0, 0), (0, 1), (2, 1)):
        eps = np.zeros((3, 3))
        eps[a, b] = h
        ep = _energy_forces(model, pos @ (np.eye(3) + eps).T, cell @ (np.eye(3) + eps).T, types, g,
                            pos @ (np.eye(3) + eps).T)[0].sum()
        em = _energy_forces(model, pos @ (np.eye(3) - eps).T, cell @ (np.eye(3) - eps).T, types, g,
                            pos @ (np.eye(3) - eps).T)[0].sum()
        # sigma_ab = (1/V) dE/d eps_ab (symmetrised strain derivative)
        assert abs((ep - em) / (2 * h) / vol - S[a, b]) < 1e-8, (a, b)


@pytest.mark.parametrize("name", MODELS)
def test_rotation_translation_permutation_invariance(paths, name):
    model = mo.MH1Oracle(paths[name])
    pos, cell, types = _system(model, seed=2)
    e0, F0, _, _ = _energy_forces(model, pos, cell, types)
    R = e3.random_rotation(np.random.default_rng(5))
    e1, F1, _, _ = _energy_forces(model, pos @ R.T, cell @ R.T, types)
    assert abs(e1.sum() - e0.sum()) < 1e-9 * len(types)
    assert np.allclose(e1, e0, atol=1e-10)
    assert np.allclose(F1, F0 @ R.T, atol=1e-9)
    e2, F2, _, _ = _energy_forces(model, pos + np.array([0.3, -1.1, 2.0]), cell, types)
    assert np.allclose(e2, e0, atol=1e-10) and np.allclose(F2, F0, atol=1e-9)
    perm = np.random.default_rng(9).permutation(len(types))
    e3_, F3, _, _ = _energy_forces(model, pos[perm], cell, types[perm])
    assert np.allclose(e3_, e0[perm], atol=1e-10) and np.allclose(F3, F0[perm], atol=1e-9)


# ---------------------------------------------------------------- known answers

def _t(v, shape=None):
    v = np.asarray(v, dtype=float)
    return {"shape": list(v.shape) if shape is None else shape, "values": v.ravel().tolist()}


def test_linear_layout_known_answer():
    # 2x0e + 1x1o -> 3x0e + 1x1o + 1x2e: W0 is [mul_in=2, mul_out=3] row-major,
    # out[w] = pw * sum_u W[u, w] x[u]; the 2e block has no path (mask 0)
    W0 = np.array([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]])
    W1 = np.array([[7.0]])
    d = {"irreps_in": "2x0e+1x1o", "irreps_out": "3x0e+1x1o+1x2e",
         "instructions": [{"i_in": 0, "i_out": 0, "path_shape": [2, 3], "path_weight": 0.5},
                          {"i_in": 1, "i_out": 1, "path_shape": [1, 1], "path_weight": 2.0}],
         "weight": _t(np.concatenate([W0.ravel(), W1.ravel()])),
         "bias": _t(np.r_[0.1, 0.2, 0.3, np.zeros(8)]),
         "output_mask": _t(np.r_[np.ones(6), np.zeros(5)])}
    lin = mo.Linear(d)
    x = np.array([[1.0, -1.0, 0.5, 0.25, -2.0]])
    y = lin.forward(x)[0]
    want = np.r_[0.5 * (1.0 * 1 - 1.0 * 4) + 0.1, 0.5 * (2 - 5) + 0.2, 0.5 * (3 - 6) + 0.3,
                 2.0 * 7.0 * np.array([0.5, 0.25, -2.0]), np.zeros(5)]
    assert np.allclose(y, want)
    # the reverse is the transpose of the forward map
    J = np.stack([lin.forward(np.eye(5)[i:i + 1])[0] - lin.forward(np.zeros((1, 5)))[0] for i in range(5)])
    G = np.random.default_rng(0).normal(size=(1, 11))
    assert np.allclose(lin.reverse(G)[0], J @ G[0])


def test_uvu_layout_known_answer():
    # 2x1o (x) 1x1o -> 2x0e: w index u*mul2 + v, out[u] = pw w[u] sum_m x1[u,m] x2[m] / sqrt(3)
    w3j = e3.wigner_3j(1, 1, 0)
    assert np.allclose(w3j[:, :, 0], np.eye(3) / np.sqrt(3))
    d = {"irreps_in1": "2x1o", "irreps_in2": "1x1o", "irreps_out": "2x0e",
         "instructions": [{"i_in1": 0, "i_in2": 0, "i_out": 0, "connection_mode": "uvu", "has_weight": True,
                           "path_weight": 1.5, "path_shape": [2, 1], "wigner_3j": _t(w3j)}],
         "weight": _t([], [0]), "output_mask": _t(np.ones(2))}
    tp = mo.TensorProduct(d)
    x1 = np.array([[1.0, 2.0, 3.0, -1.0, 0.5, 2.0]])
    x2 = np.array([[0.3, -0.2, 0.7]])
    w = np.array([[2.0, -3.0]])
    y = tp.forward(x1, x2, w)[0]
    want = 1.5 * w[0] * np.array([x1[0, :3] @ x2[0], x1[0, 3:] @ x2[0]]) / np.sqrt(3)
    assert np.allclose(y, want)


def test_gate_layout_known_answer():
    d = random_mh1.gate(2, 2)   # in: 6x0e+2x1o+2x2e (scalars | gates | gated)
    g = mo.Gate(d)
    x = np.arange(1, 6 + 6 + 10 + 1, dtype=float)[None] * 0.1
    y = g.forward(x)[0]
    s = lambda v: 1.0 / (1.0 + np.exp(-v))
    sc, gc = d["scalar_activation_constants"][0], d["gate_activation_constants"]
    want = [sc * v * s(v) for v in x[0, :2]]
    # gates x[2:4] gate the 1o channels, x[4:6] the 2e channels
    want += list(gc[0] * s(x[0, 2]) * x[0, 6:9]) + list(gc[0] * s(x[0, 3]) * x[0, 9:12])
    want += list(gc[1] * s(x[0, 4]) * x[0, 12:17]) + list(gc[1] * s(x[0, 5]) * x[0, 17:22])
    assert np.allclose(y, want)


def test_product_layout_known_answer():
    # 2 features, input 1x0e+1x1o (angular 4), output 0e, correlation 2:
    # out[f] = sum_i c1[i,f] x[f,i] + sum_ij c2[i,j,f] x[f,i] x[f,j] with
    # c_nu[..., f] = sum_k U_nu[..., k] W_nu[e, k, f]; weights_max serves nu=2
    rng = np.random.default_rng(3)
    U1 = rng.normal(size=(4, 2))
    U2 = rng.normal(size=(4, 4, 3))
    W1 = rng.normal(size=(2, 2, 2))   # [elements, K, features]
    W2 = rng.normal(size=(2, 3, 2))
    lin = {"irreps_in": "2x0e", "irreps_out": "2x0e", "instructions": [
        {"i_in": 0, "i_out": 0, "path_shape": [2, 2], "path_weight": 1.0}],
        "weight": _t(np.eye(2).ravel()), "bias": _t([], [0]), "output_mask": _t(np.ones(2))}
    d = {"use_sc": True, "use_agnostic_product": False, "linear": lin,
         "symmetric_contractions": {"irreps_in": "2x0e+2x1o", "irreps_out": "2x0e", "contractions": [
             {"correlation": 2, "weights": [_t(W1)], "weights_max": _t(W2), "u_tensors": [_t(U1), _t(U2)]}]}}
    p = mo.Product(d)
    X = rng.normal(size=(1, 8))       # [f0 0e, f1 0e, f0 1o(3), f1 1o(3)]
    xf = np.array([[X[0, 0], *X[0, 2:5]], [X[0, 1], *X[0, 5:8]]])
    skip = np.array([[0.5, -0.5]])
    y = p.forward(X, skip, np.array([1]))[0]
    want = []
    for f in range(2):
        c1 = U1 @ W1[1, :, f]
        c2 = np.einsum("ijk,k->ij", U2, W2[1, :, f])
        want.append(c1 @ xf[f] + xf[f] @ c2 @ xf[f] + skip[0, f])
    assert np.allclose(y, want)


def test_affine_mlp_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(4)
    d = random_mh1.affine_mlp(rng, [6, 5, 4, 3])
    mlp = mo.AffineMLP(d)
    layers = []
    for L in d["layers"]:
        if L["type"] == "linear":
            m = torch.nn.Linear(*reversed(L["weight"]["shape"])).double()
            m.weight.data = torch.tensor(L["weight"]["values"], dtype=torch.float64).reshape(L["weight"]["shape"])
            m.bias.data = torch.tensor(L["bias"]["values"], dtype=torch.float64)
        elif L["type"] == "layer_norm":
            m = torch.nn.LayerNorm(L["normalized_shape"], eps=L["eps"]).double()
            m.weight.data = torch.tensor(L["weight"]["values"], dtype=torch.float64)
            m.bias.data = torch.tensor(L["bias"]["values"], dtype=torch.float64)
        else:
            m = torch.nn.SiLU()
        layers.append(m)
    net = torch.nn.Sequential(*layers)
    X = rng.normal(size=(7, 6))
    xt = torch.tensor(X, requires_grad=True)
    yt = net(xt)
    G = rng.normal(size=(7, 3))
    yt.backward(torch.tensor(G))
    y, tape = mlp.forward(X)
    assert np.allclose(y, yt.detach().numpy(), atol=1e-12)
    assert np.allclose(mlp.reverse(tape, G), xt.grad.numpy(), atol=1e-12)


# ------------------------------------------------------------- planted mistakes

def test_planted_mistakes_are_caught(paths, monkeypatch):
    model = mo.MH1Oracle(paths["mh1_tiny"])
    pos, cell, types = _system(model, seed=2)
    ok, _ = _fd_error(model, pos, cell, types)
    assert ok < 1e-7

    # the l=1 harmonics in (x, y, z) order while l=2 keeps the (z, x, y)
    # frame: the harmonics and the Wigner 3j disagree, invariance breaks
    orig_sh = mo._sh
    monkeypatch.setattr(mo, "_sh", lambda v, l: orig_sh(v, l)[:, [0, 3, 1, 2] + list(range(4, (l + 1) ** 2))])
    e0 = _energy_forces(model, pos, cell, types)[0].sum()
    R = e3.random_rotation(np.random.default_rng(5))
    e1 = _energy_forces(model, pos @ R.T, cell @ R.T, types)[0].sum()
    assert abs(e1 - e0) > 1e-6
    monkeypatch.setattr(mo, "_sh", orig_sh)

    # a dropped harmonic adjoint term: the forces no longer match FD
    orig_rev = mo.TensorProduct.reverse

    def no_y(self, X1, X2, Wt, G):
        a1, a2, aw = orig_rev(self, X1, X2, Wt, G)
        return a1, 0.0 * a2, aw
    monkeypatch.setattr(mo.TensorProduct, "reverse", no_y)
    assert _fd_error(model, pos, cell, types)[0] > 1e-4
    monkeypatch.setattr(mo.TensorProduct, "reverse", orig_rev)

    # the normalisation's density derivative dropped: FD breaks
    monkeypatch.setattr(mo.MH1Oracle, "_density_adjoint",
                        lambda self, it, a_pre, s: np.zeros(len(s["density"])))
    assert _fd_error(model, pos, cell, types)[0] > 1e-4


def test_planted_transposed_linear_read_fails_known_answer():
    # a [mul_out, mul_in] read of a non-square weight gives another answer
    lin = mo.Linear({"irreps_in": "2x0e", "irreps_out": "3x0e",
                     "instructions": [{"i_in": 0, "i_out": 0, "path_shape": [2, 3], "path_weight": 1.0}],
                     "weight": _t(np.arange(6.0)), "bias": _t([], [0]), "output_mask": _t(np.ones(3))})
    x = np.array([[1.0, 10.0]])
    right = lin.forward(x)[0]
    wrong = np.arange(6.0).reshape(3, 2) @ x[0]
    assert np.allclose(right, [30.0, 41.0, 52.0])
    assert not np.allclose(right, wrong)


def test_mace_evaluator_refuses_nonlinear_files(tmp_path):
    """A MACE_Nonlinear file given to the MACE evaluator (and so to the pair
    style, as the reference's pair styles refuse it) fails with a message
    that names the MH-1 entry point, before any device work."""
    import json as _json
    from symmetrix import mace_kokkos
    p = tmp_path / "nonlinear.json"
    p.write_text(_json.dumps({"symmetrix_format_version": 3, "model_type": "MACE_Nonlinear"}))
    with pytest.raises(ValueError, match="MACE_Nonlinear models are not supported"):
        mace_kokkos.MACEKokkosFloat(str(p))
