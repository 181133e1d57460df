"""The pre_linear_up H1 basis and the first-interaction residual in the
oracle (CPU), pinned by models that compute the same function in another
way (h1_affine_schema.hpp:196-259; mace.cpp:1759-1875, 2796-2826).

* Basis: a pre_linear_up model (split H1 weights P and U, readout_1 r and
  skip S_z on the scalar x = M0[:,0,:] P0) equals the m0_composite model with
  q = P0 r and T_z = P0 S_z on M0[:,0,:] (the conversion of
  test_h1_affine.py:119-133). A transposed P0, the composite readout read
  against x, or the direct adjoint entering M0 without P0 each breaks it.
* Residual: H1 += b U (per type, every lm) and x += b[lm 0] equal an added
  constant monomial c = b P^-1 in every M0 output, which reaches H1 through
  P U and x through P0. The twin carries no residual and computes the
  constant through the product basis instead.
Both in FP64, energies, forces and stress to 1e-10 relative (the residual
check with the composite H1_weights set to P U exactly).
"""

import copy
import json

import numpy as np
import pytest

from oracle import oracle
from symmetrix import systems


def _evaluate(path, system):
    om = oracle.OracleModel(str(path), fp64=True)
    return oracle.evaluate_system(om, system, skin=0.5)


def _same(a, b):
    scale = max(1.0, float(np.max(np.abs(a["forces"]))))
    assert abs(a["energy"] - b["energy"]) < 1e-10 * max(1.0, abs(a["energy"]))
    np.testing.assert_allclose(a["energies"], b["energies"], rtol=0, atol=1e-10 * max(1.0, abs(a["energy"])))
    np.testing.assert_allclose(a["forces"], b["forces"], rtol=0, atol=1e-10 * scale)
    np.testing.assert_allclose(a["stress"], b["stress"], rtol=0, atol=1e-12)


def _write(tmp_path, name, doc):
    p = tmp_path / name
    p.write_text(json.dumps(doc))
    return p


def _split(doc):
    C, L = doc["num_channels"], doc["L_max"]
    P = np.asarray(doc["H1_product_weights"], float).reshape(L + 1, C, C)
    U = np.asarray(doc["H1_linear_up_weights"], float).reshape(L + 1, C, C)
    return C, L, P, U


def test_pre_linear_up_equals_its_m0_composite_conversion(tmp_path, tiny_plu_model_path):
    with open(tiny_plu_model_path) as f:
        doc = json.load(f)
    assert doc["h1_affine_mode"] == "pre_linear_up" and not doc["first_interaction_residual"]
    C, L, P, U = _split(doc)
    np.testing.assert_allclose(np.asarray(doc["H1_weights"]).reshape(L + 1, C, C),
                               np.einsum("lab,lbc->lac", P, U), rtol=1e-6, atol=1e-7)
    r = np.asarray(doc["readout_1_weights_for_H1_pre_linear_up"], float)
    S = [np.asarray(s, float).reshape(C, C) for s in doc["H2_weights_for_H1_pre_linear_up"]]
    twin = copy.deepcopy(doc)
    for key in ("H1_product_weights", "H1_linear_up_weights", "first_interaction_residual",
                "readout_1_weights_for_H1_pre_linear_up", "H2_weights_for_H1_pre_linear_up"):
        del twin[key]
    twin["h1_affine_mode"] = "m0_composite"
    twin["readout_1_weights_for_M0"] = (P[0] @ r).tolist()
    twin["H2_weights_for_M0"] = [(P[0] @ s).ravel().tolist() for s in S]
    system = systems.srtio3_supercell(3, sigma=0.05, seed=5)
    a = _evaluate(tiny_plu_model_path, system)
    b = _evaluate(_write(tmp_path, "twin.json", twin), system)
    _same(a, b)
    # a misreading fails: the composite maps read against x
    wrong = copy.deepcopy(doc)
    wrong["readout_1_weights_for_H1_pre_linear_up"] = twin["readout_1_weights_for_M0"]
    c = _evaluate(_write(tmp_path, "wrong.json", wrong), system)
    assert abs(c["energy"] - a["energy"]) > 1e-6 * abs(a["energy"])


def test_residual_equals_a_constant_product_basis_term(tmp_path, tiny_residual_model_path):
    with open(tiny_residual_model_path) as f:
        doc = json.load(f)
    assert doc["first_interaction_residual"] and doc["h1_affine_mode"] == "pre_linear_up"
    C, L, P, U = _split(doc)
    nz, LM = doc["num_elements"], (L + 1) ** 2
    b = np.asarray(doc["H1_first_residual_weights"], float).reshape(nz, LM, C)
    # the file's composite is P U rounded to FP32; make it exact so that the
    # constant's path through H1_weights and the residual's through U agree
    doc["H1_weights"] = np.einsum("lab,lbc->lac", P, U).ravel().tolist()
    base = _write(tmp_path, "residual.json", doc)
    twin = copy.deepcopy(doc)
    del twin["H1_first_residual_weights"]
    twin["first_interaction_residual"] = False
    for lm in range(LM):
        twin["M0_monomials"][str(lm)].append([])          # the constant term
    for t in range(nz):
        for l in range(L + 1):
            inv = np.linalg.inv(P[l])
            for m in range(2 * l + 1):
                lm = l * l + m
                c = b[t, lm] @ inv                          # c P_l = b
                for k in range(C):
                    twin["M0_weights"][str(t)][str(lm)][str(k)].append(float(c[k]))
    system = systems.srtio3_supercell(3, sigma=0.05, seed=6)
    a = _evaluate(base, system)
    t = _evaluate(_write(tmp_path, "twin.json", twin), system)
    _same(a, t)
    # and the residual matters
    plain = copy.deepcopy(doc)
    plain["H1_first_residual_weights"] = np.zeros_like(b).ravel().tolist()
    p = _evaluate(_write(tmp_path, "plain.json", plain), system)
    assert abs(p["energy"] - a["energy"]) > 1e-6 * abs(a["energy"])
    assert np.max(np.abs(p["forces"] - a["forces"])) > 1e-6


def test_residual_needs_the_pre_linear_up_basis(tmp_path, tiny_residual_model_path):
    with open(tiny_residual_model_path) as f:
        doc = json.load(f)
    bad = copy.deepcopy(doc)
    bad["h1_affine_mode"] = "m0_composite"
    with pytest.raises(Exception):
        oracle.OracleModel(str(_write(tmp_path, "bad.json", bad)))
