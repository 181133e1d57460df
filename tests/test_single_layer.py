"""One-interaction MACE models (single_layer_readout; mace.cpp:255-281,
2461-2514, 2676-2679; extract_mace_data.py:1221-1262) in the oracle (CPU,
FP64) and in the library's model loader.

What pins the oracle here:
* energy: every node energy equals the readouts of an invariant polynomial
  of H1 evaluated in numpy from the file, the way the reference's own
  readout test reads M1 (test_single_layer_mace.py:98-115: each coefficient
  times the product of the channel's H1 components named by the monomial),
  on the oracle's H1 stage (the layer-1 stages are pinned by the
  two-interaction tests);
* forces and stress: central differences of that energy;
* invariance: rotating the system leaves the energy and rotates the forces
  (a misread variable order of the M1 polynomial breaks it);
* residual: with the zero readout_1 / skip maps the reference's extractor
  writes for one-interaction models, the residual (H1 += b U in the
  m0_composite basis) equals a twin without it whose M0 outputs carry the
  constant monomial c = b P^-1.
GPU parity of the product path: tests/test_single_layer_gpu.py.
"""

import copy
import json

import numpy as np
import pytest

from oracle import oracle
from symmetrix import e3, systems

SILU_SCALE_KEY = "readout_2_scale_factor"


def _doc(path):
    with open(path) as f:
        return json.load(f)


def _write(tmp_path, name, doc):
    p = tmp_path / name
    p.write_text(json.dumps(doc))
    return str(p)


def _small():
    return systems.srtio3_supercell(2, sigma=0.08, seed=3)


def _readout_energies(doc, H1, x, types):
    """E_i = E0 + q.x + MLP(T_z^T x + W^T M1(H1_i)) from the file, in numpy."""
    C = doc["num_channels"]
    n = H1.shape[0]
    monos = doc["M1_monomials"]
    M1 = np.zeros((n, C))
    for s, m in enumerate(monos):
        prod = np.prod(H1[:, m, :], axis=1)                   # [n, C]
        coef = np.array([[doc["M1_weights"][str(t)][str(k)][s] for k in range(C)] for t in types])
        M1 += coef * prod
    T = np.array(doc["H2_weights_for_M0"], float).reshape(-1, C, C)
    Wm = np.array(doc["H2_weights_for_M1"], float).reshape(C, C)
    H2 = np.einsum("nio,ni->no", T[types], x) + M1 @ Wm
    hid = doc["readout_2_hidden_size"]
    W1 = np.array(doc["readout_2_weights_1"], float).reshape(hid, C)
    W2 = np.array(doc["readout_2_weights_2"], float)
    z = H2 @ W1.T
    act = doc[SILU_SCALE_KEY] * z / (1.0 + np.exp(-z))
    q = np.array(doc["readout_1_weights_for_M0"], float)
    E0 = np.array(doc["atomic_energies"], float)
    return E0[types] + x @ q + act @ W2


def test_generated_file_has_the_writers_layout(tiny_single_model_path):
    doc = _doc(tiny_single_model_path)
    assert doc["num_interactions"] == 1 and doc["single_layer_readout"] is True
    assert doc["readout_correlation"] == 2 and doc["h1_affine_mode"] == "m0_composite"
    assert set(doc["compact_radial"]["networks"]) == {"R0"}
    assert doc["Phi1_l"] == [] and doc["A1_scaled"] is False
    LM = (doc["L_max"] + 1) ** 2
    assert max(v for m in doc["M1_monomials"] for v in m) < LM
    assert max(len(m) for m in doc["M1_monomials"]) == 2


def test_energy_is_the_readout_of_an_h1_invariant(tiny_single_model_path):
    doc = _doc(tiny_single_model_path)
    om = oracle.OracleModel(tiny_single_model_path, fp64=True)
    s = _small()
    r = oracle.evaluate_system(om, s, skin=0.5)
    n, C, LM = len(s["numbers"]), doc["num_channels"], (doc["L_max"] + 1) ** 2
    H1 = om.stage("H1").reshape(n, LM, C)
    x = om.stage("M0").reshape(n, LM, C)[:, 0, :]
    types = om.types_of(s["numbers"])
    mine = _readout_energies(doc, H1, x, types)
    np.testing.assert_allclose(r["energies"], mine, rtol=0, atol=1e-9 * np.max(np.abs(mine)))
    # the H1 adjoint is M1's gradient times the M1 adjoint: no second interaction
    assert om.stage("A1").size == 0 and om.stage("Phi1").size == 0
    assert np.max(np.abs(om.stage("node_forces_r1"))) == 0.0


@pytest.mark.parametrize("model", ["tiny_single", "tiny_single_residual", "medium_single"])
def test_forces_and_stress_are_energy_derivatives(request, model):
    path = request.getfixturevalue(model + "_model_path")
    m = oracle.OracleModel(path, fp64=True)
    s = _small()
    base = oracle.evaluate_system(m, s, skin=0.5)
    h = 1e-4
    rng = np.random.default_rng(7)
    for a in rng.choice(len(s["numbers"]), 3, replace=False):
        for c in range(3):
            pp, pm = s["positions"].copy(), s["positions"].copy()
            pp[a, c] += h
            pm[a, c] -= h
            ep = oracle.evaluate_system(m, dict(s, positions=pp), skin=0.5)["energy"]
            em = oracle.evaluate_system(m, dict(s, positions=pm), skin=0.5)["energy"]
            assert base["forces"][a, c] == pytest.approx(-(ep - em) / (2 * h), abs=2e-6)
    V = abs(np.linalg.det(s["cell"]))
    for (i, j) in [(0, 0), (1, 2)]:
        eps = np.zeros((3, 3))
        eps[i, j] = h

        def strained(sign):
            F = np.eye(3) + sign * eps
            return oracle.evaluate_system(m, dict(s, positions=s["positions"] @ F.T, cell=s["cell"] @ F.T),
                                          skin=0.5)["energy"]
        assert base["stress"][i, j] == pytest.approx((strained(1) - strained(-1)) / (2 * h) / V, abs=1e-7)


def test_energy_is_rotation_invariant(tiny_single_model_path, tiny_single_residual_model_path, tmp_path):
    # the residual of a trained model has only the scalar block (the skip
    # product of scalar node features); keep that block here
    doc = _doc(tiny_single_residual_model_path)
    LM, C = (doc["L_max"] + 1) ** 2, doc["num_channels"]
    b = np.array(doc["H1_first_residual_weights"], float).reshape(-1, LM, C)
    b[:, 1:, :] = 0.0
    doc["H1_first_residual_weights"] = b.ravel().tolist()
    paths = [tiny_single_model_path, _write(tmp_path, "scalar_residual.json", doc)]
    s = _small()
    R = e3.random_rotation(np.random.default_rng(11))
    rot = dict(s, positions=s["positions"] @ R.T, cell=s["cell"] @ R.T)
    for path in paths:
        m = oracle.OracleModel(path, fp64=True)
        base = oracle.evaluate_system(m, s, skin=0.5)
        r = oracle.evaluate_system(m, rot, skin=0.5)
        assert r["energy"] == pytest.approx(base["energy"], abs=1e-9)
        np.testing.assert_allclose(r["forces"], base["forces"] @ R.T, atol=1e-9)
    # a misread variable order breaks it: the scalar and an l=1 component of
    # H1 swapped in M1 (the correlation-2 invariants of 0e+1o are x0, x0^2
    # and the l=1 norm, so a swap within l=1 would go unseen)
    doc = _doc(tiny_single_model_path)
    swap = {0: 1, 1: 0}
    doc["M1_monomials"] = [[swap.get(v, v) for v in m] for m in doc["M1_monomials"]]
    doc["M1_monomials"] = [sorted(m) for m in doc["M1_monomials"]]
    m = oracle.OracleModel(_write(tmp_path, "misread.json", doc), fp64=True)
    e0 = oracle.evaluate_system(m, s, skin=0.5)["energy"]
    e1 = oracle.evaluate_system(m, rot, skin=0.5)["energy"]
    assert abs(e1 - e0) > 1e-6 * abs(e0)


def test_residual_equals_a_constant_product_basis_term(tmp_path, tiny_single_residual_model_path):
    doc = _doc(tiny_single_residual_model_path)
    assert doc["first_interaction_residual"] and doc["h1_affine_mode"] == "m0_composite"
    C, L = doc["num_channels"], doc["L_max"]
    nz, LM = doc["num_elements"], (L + 1) ** 2
    P = np.asarray(doc["H1_product_weights"], float).reshape(L + 1, C, C)
    U = np.asarray(doc["H1_linear_up_weights"], float).reshape(L + 1, C, C)
    b = np.asarray(doc["H1_first_residual_weights"], float).reshape(nz, LM, C)
    # the writer's zero readout_1 and skip maps (extract_mace_data.py:1236-1241):
    # the scalar x = M0[:,0,:] then enters no energy
    doc["readout_1_weights_for_M0"] = [0.0] * C
    doc["H2_weights_for_M0"] = [[0.0] * (C * C) for _ in range(nz)]
    doc["H1_weights"] = np.einsum("lab,lbc->lac", P, U).ravel().tolist()
    base = _write(tmp_path, "residual.json", doc)
    twin = copy.deepcopy(doc)
    del twin["H1_first_residual_weights"]
    twin["first_interaction_residual"] = False
    for lm in range(LM):
        twin["M0_monomials"][str(lm)].append([])
    for t in range(nz):
        for l in range(L + 1):
            inv = np.linalg.inv(P[l])
            for mm in range(2 * l + 1):
                lm = l * l + mm
                c = b[t, lm] @ inv
                for k in range(C):
                    twin["M0_weights"][str(t)][str(lm)][str(k)].append(float(c[k]))
    s = systems.srtio3_supercell(3, sigma=0.05, seed=6)
    a = oracle.evaluate_system(oracle.OracleModel(base, fp64=True), s, skin=0.5)
    t = oracle.evaluate_system(oracle.OracleModel(_write(tmp_path, "twin.json", twin), fp64=True), s, skin=0.5)
    scale = max(1.0, abs(a["energy"]))
    assert abs(a["energy"] - t["energy"]) < 1e-10 * scale
    np.testing.assert_allclose(a["forces"], t["forces"], rtol=0, atol=1e-10 * max(1.0, np.max(np.abs(a["forces"]))))
    np.testing.assert_allclose(a["stress"], t["stress"], rtol=0, atol=1e-12)
    plain = copy.deepcopy(doc)
    plain["H1_first_residual_weights"] = np.zeros_like(b).ravel().tolist()
    p = oracle.evaluate_system(oracle.OracleModel(_write(tmp_path, "plain.json", plain), fp64=True), s, skin=0.5)
    assert abs(p["energy"] - a["energy"]) > 1e-6 * scale


def _variants(doc):
    """Files the reference's loaders refuse (mace.cpp:2676-2679, 2769-2772;
    h1_affine_schema.hpp:233-236)."""
    two = copy.deepcopy(doc)
    two["num_interactions"] = 2
    plu = copy.deepcopy(doc)
    plu["h1_affine_mode"] = "pre_linear_up"
    plu["readout_1_weights_for_H1_pre_linear_up"] = plu.pop("readout_1_weights_for_M0")
    plu["H2_weights_for_H1_pre_linear_up"] = plu.pop("H2_weights_for_M0")
    plu["H1_product_weights"] = plu["H1_weights"]
    r1 = copy.deepcopy(doc)
    r1["compact_radial"]["networks"]["R1"] = r1["compact_radial"]["networks"]["R0"]
    return {"count": two, "pre_linear_up": plu, "r1_network": r1}


def test_oracle_refuses_inconsistent_one_interaction_files(tmp_path, tiny_single_model_path):
    for name, bad in _variants(_doc(tiny_single_model_path)).items():
        with pytest.raises(Exception):
            oracle.OracleModel(_write(tmp_path, name + ".json", bad))


def test_library_loader_accepts_and_refuses(tmp_path, tiny_single_model_path, tiny_single_residual_model_path):
    from symmetrix._native import model_array
    for path in (tiny_single_model_path, tiny_single_residual_model_path):
        assert model_array(path, "H0").shape == (3, 32)
    for name, bad in _variants(_doc(tiny_single_model_path)).items():
        with pytest.raises(ValueError):
            model_array(_write(tmp_path, "lib_" + name + ".json", bad), "H0")
