"""MACEField models (has_field_coupling; field_coupling.hpp:60-238,
mace.cpp:322-395 and 1147-1240, the Kokkos forms mace_kokkos_h1_phi1.cpp:
846-1150) in the oracle, CPU, FP64.

What pins the oracle's field path:
* zero field: the model equals its field-free twin (the same file without
  the coupling, H1_weights set to P U exactly), with and without the
  first-interaction residual, L_max 1 and 2;
* dE/dE: the field adjoint equals central differences of the energy in the
  field, for one field per graph and for one field per node;
* rotations: rotating the atoms and the field together leaves the energy
  unchanged and rotates dE/dE (the angular coupling's component order;
  the field read in another component order breaks it);
* forces and stress: central differences of the energy at a nonzero field.
GPU parity of the product path: tests/test_macefield_gpu.py.
"""

import copy
import json

import numpy as np
import pytest

from oracle import oracle
from symmetrix import e3, systems


def _doc(path):
    with open(path) as f:
        return json.load(f)


def _write(tmp_path, name, doc):
    p = tmp_path / name
    p.write_text(json.dumps(doc))
    return str(p)


def _small():
    return systems.srtio3_supercell(2, sigma=0.08, seed=3)


FIELD = np.array([0.12, -0.21, 0.27])


@pytest.mark.parametrize("model", ["tiny_field", "field_l2"])
def test_zero_field_equals_the_field_free_twin(request, tmp_path, model):
    doc = _doc(request.getfixturevalue(model + "_model_path"))
    C, L = doc["num_channels"], doc["L_max"]
    P = np.asarray(doc["H1_product_weights"], float).reshape(L + 1, C, C)
    U = np.asarray(doc["H1_linear_up_weights"], float).reshape(L + 1, C, C)
    doc["H1_weights"] = np.einsum("lab,lbc->lac", P, U).ravel().tolist()
    base = _write(tmp_path, "field.json", doc)
    twin = copy.deepcopy(doc)
    for key in ("has_field_coupling", "field_couplings"):
        del twin[key]
    twin["model_type"] = "MACE"
    s = _small()
    a = oracle.evaluate_system(oracle.OracleModel(base, fp64=True), s, skin=0.5, field=np.zeros(3))
    t = oracle.evaluate_system(oracle.OracleModel(_write(tmp_path, "twin.json", twin), fp64=True), s, skin=0.5)
    scale = max(1.0, abs(a["energy"]))
    assert abs(a["energy"] - t["energy"]) < 1e-10 * scale
    np.testing.assert_allclose(a["forces"], t["forces"], rtol=0, atol=1e-10 * max(1.0, np.max(np.abs(a["forces"]))))
    np.testing.assert_allclose(a["stress"], t["stress"], rtol=0, atol=1e-12)
    # and the field matters
    f = oracle.evaluate_system(oracle.OracleModel(base, fp64=True), s, skin=0.5, field=FIELD)
    assert abs(f["energy"] - a["energy"]) > 1e-6 * scale


@pytest.mark.parametrize("model", ["tiny_field", "field_l2"])
def test_field_adjoint_is_the_field_derivative(request, model):
    om = oracle.OracleModel(request.getfixturevalue(model + "_model_path"), fp64=True)
    s = _small()
    r = oracle.evaluate_system(om, s, skin=0.5, field=FIELD)
    h = 1e-5
    for c in range(3):
        fp, fm = FIELD.copy(), FIELD.copy()
        fp[c] += h
        fm[c] -= h
        d = (oracle.evaluate_system(om, s, skin=0.5, field=fp)["energy"]
             - oracle.evaluate_system(om, s, skin=0.5, field=fm)["energy"]) / (2 * h)
        assert r["field_adj"][c] == pytest.approx(d, abs=1e-8)
    # one field per node: each node's adjoint is the derivative in its field
    n = len(s["numbers"])
    per = np.tile(FIELD, (n, 1)) + 0.05 * np.random.default_rng(4).normal(size=(n, 3))
    rp = oracle.evaluate_system(om, s, skin=0.5, field=per)
    adj = rp["field_adj"].reshape(n, 3)
    for i, c in [(0, 0), (3, 2), (n - 1, 1)]:
        fp, fm = per.copy(), per.copy()
        fp[i, c] += h
        fm[i, c] -= h
        d = (oracle.evaluate_system(om, s, skin=0.5, field=fp)["energy"]
             - oracle.evaluate_system(om, s, skin=0.5, field=fm)["energy"]) / (2 * h)
        assert adj[i, c] == pytest.approx(d, abs=1e-8)
    # the graph field's adjoint is the sum of the per-node ones
    same = oracle.evaluate_system(om, s, skin=0.5, field=np.tile(FIELD, (n, 1)))
    np.testing.assert_allclose(same["field_adj"].reshape(n, 3).sum(axis=0), r["field_adj"], rtol=0, atol=1e-10)
    assert same["energy"] == pytest.approx(r["energy"], abs=1e-10)


@pytest.mark.parametrize("model", ["tiny_field", "field_l2"])
def test_rotating_atoms_and_field_together_is_invariant(request, tmp_path, model):
    path = request.getfixturevalue(model + "_model_path")
    doc = _doc(path)
    if doc.get("first_interaction_residual"):
        # a trained residual has only its scalar block (the skip product of
        # scalar node features); the generator's fills every block
        LM, C = (doc["L_max"] + 1) ** 2, doc["num_channels"]
        b = np.asarray(doc["H1_first_residual_weights"], float).reshape(-1, LM, C)
        b[:, 1:, :] = 0.0
        doc["H1_first_residual_weights"] = b.ravel().tolist()
        path = _write(tmp_path, "scalar_residual.json", doc)
    om = oracle.OracleModel(path, fp64=True)
    s = _small()
    R = e3.random_rotation(np.random.default_rng(11))
    rot = dict(s, positions=s["positions"] @ R.T, cell=s["cell"] @ R.T)
    a = oracle.evaluate_system(om, s, skin=0.5, field=FIELD)
    b = oracle.evaluate_system(om, rot, skin=0.5, field=R @ FIELD)
    assert b["energy"] == pytest.approx(a["energy"], abs=1e-9)
    np.testing.assert_allclose(b["field_adj"], R @ a["field_adj"], rtol=0, atol=1e-10)
    np.testing.assert_allclose(b["forces"], a["forces"] @ R.T, rtol=0, atol=1e-9)
    # the field taken in e3nn's (y, z, x) order instead is not equivariant
    doc = _doc(path)
    for ins in doc["field_couplings"][0]["field_feats_instructions"]:
        d0, _, d2 = ins["wigner_3j_shape"]
        w = np.asarray(ins["wigner_3j"]).reshape(d0, 3, d2)[:, [1, 2, 0], :]
        ins["wigner_3j"] = w.ravel().tolist()
    bad = oracle.OracleModel(_write(tmp_path, "yzx.json", doc), fp64=True)
    ea = oracle.evaluate_system(bad, s, skin=0.5, field=FIELD)["energy"]
    eb = oracle.evaluate_system(bad, rot, skin=0.5, field=R @ FIELD)["energy"]
    assert abs(ea - eb) > 1e-6 * abs(ea)


def test_forces_and_stress_are_energy_derivatives_in_a_field(field_l2_model_path):
    m = oracle.OracleModel(field_l2_model_path, fp64=True)
    s = _small()
    base = oracle.evaluate_system(m, s, skin=0.5, field=FIELD)
    h = 1e-4
    for a, c in [(0, 0), (5, 1), (17, 2)]:
        pp, pm = s["positions"].copy(), s["positions"].copy()
        pp[a, c] += h
        pm[a, c] -= h
        ep = oracle.evaluate_system(m, dict(s, positions=pp), skin=0.5, field=FIELD)["energy"]
        em = oracle.evaluate_system(m, dict(s, positions=pm), skin=0.5, field=FIELD)["energy"]
        assert base["forces"][a, c] == pytest.approx(-(ep - em) / (2 * h), abs=2e-6)
    V = abs(np.linalg.det(s["cell"]))
    eps = np.zeros((3, 3))
    eps[0, 1] = h

    def strained(sign):
        F = np.eye(3) + sign * eps
        return oracle.evaluate_system(m, dict(s, positions=s["positions"] @ F.T, cell=s["cell"] @ F.T), skin=0.5,
                                      field=FIELD)["energy"]
    assert base["stress"][0, 1] == pytest.approx((strained(1) - strained(-1)) / (2 * h) / V, abs=1e-7)


def test_oracle_refuses_inconsistent_field_models(tmp_path, tiny_field_model_path):
    doc = _doc(tiny_field_model_path)
    bad = {}
    m0 = copy.deepcopy(doc)
    m0["h1_affine_mode"] = "m0_composite"
    m0["readout_1_weights_for_M0"] = m0.pop("readout_1_weights_for_H1_pre_linear_up")
    m0["H2_weights_for_M0"] = m0.pop("H2_weights_for_H1_pre_linear_up")
    bad["m0_composite"] = m0
    mask = copy.deepcopy(doc)
    mask["field_couplings"][0]["field_linear_output_mask"][3] = 0.5
    bad["mask"] = mask
    irreps = copy.deepcopy(doc)
    irreps["field_couplings"][0]["field_feats_irreps_in2"] = "1x1e"
    bad["irreps"] = irreps
    rank = copy.deepcopy(doc)
    rank["field_couplings"][0]["field_feats_instructions"][0]["i_out"] = 0
    bad["rank"] = rank
    for name, d in bad.items():
        with pytest.raises(ValueError):
            oracle.OracleModel(_write(tmp_path, name + ".json", d))
    om = oracle.OracleModel(tiny_field_model_path)
    s = _small()
    with pytest.raises(ValueError, match="electric_field"):
        oracle.evaluate_system(om, s, skin=0.5)
    with pytest.raises(ValueError, match="electric_field"):
        oracle.evaluate_system(om, s, skin=0.5, field=np.zeros(6))


def _library_refusal(path):
    """Creates an evaluator through the C ABI; the model loader runs before
    any device call, so its refusals show on a host without a GPU."""
    import ctypes

    from symmetrix import _native
    h = ctypes.c_void_p()
    rc = _native.lib.smx_evaluator_create(path.encode(), b"", ctypes.byref(h))
    if rc == 0:
        _native.lib.smx_evaluator_destroy(h)
    return rc, _native.lib.smx_last_error().decode()


def test_library_loader_refuses_malformed_couplings(tmp_path, tiny_field_model_path, field_l2_model_path):
    """The product loader's schema checks (the constraints field_coupling.hpp:
    60-238 enforces), each broken once on an otherwise valid model."""
    from symmetrix import _native
    doc = _doc(tiny_field_model_path)
    cases = {
        "two couplings": (lambda d: d["field_couplings"].append(copy.deepcopy(d["field_couplings"][0])),
                          "one coupling"),
        "schema": (lambda d: d["field_couplings"][0].__setitem__("schema_version", 2), "schema_version 2"),
        "irreps": (lambda d: d["field_couplings"][0].__setitem__("field_feats_irreps_in2", "1x1e"),
                   "field_feats_irreps_in2"),
        "mask": (lambda d: d["field_couplings"][0]["field_linear_output_mask"].__setitem__(3, 0.5),
                 "field_linear_output_mask"),
        "bias": (lambda d: d["field_couplings"][0].__setitem__("field_linear_bias", [0.0]), "field_linear_bias"),
        "rank": (lambda d: d["field_couplings"][0]["field_feats_instructions"][0].__setitem__("i_out", 0),
                 "field_feats_instructions[0]"),
        "mode": (lambda d: d["field_couplings"][0]["field_feats_instructions"][0].__setitem__(
            "connection_mode", "uuu"), "uvw"),
        "mix block": (lambda d: d["field_couplings"][0]["field_linear_instructions"][0].__setitem__("i_out", 9),
                      "field_linear_instructions[0]"),
        "feats weight": (lambda d: d["field_couplings"][0].__setitem__(
            "field_feats_weight", d["field_couplings"][0]["field_feats_weight"][:-1]), "field_feats_weight"),
        "no split": (lambda d: d.pop("H1_linear_up_weights"), "H1_linear_up_weights"),
        "unread block": (lambda d: d["field_couplings"][0].__setitem__(
            "field_linear_instructions", [i for i in d["field_couplings"][0]["field_linear_instructions"]
                                          if i["i_in"] != 1]), None),
    }
    for name, (edit, needle) in cases.items():
        d = copy.deepcopy(doc)
        edit(d)
        rc, msg = _library_refusal(_write(tmp_path, "bad.json", d))
        assert rc == _native.SMX_ERR_INVALID_ARGUMENT, (name, msg)
        assert msg.startswith("field coupling:"), (name, msg)
        if needle:
            assert needle in msg, (name, msg)
    # an L_max 2 coupling needs its 3j tensors; without schema_version it is refused
    d2 = _doc(field_l2_model_path)
    del d2["field_couplings"][0]["schema_version"]
    rc, msg = _library_refusal(_write(tmp_path, "unversioned_l2.json", d2))
    assert rc == _native.SMX_ERR_INVALID_ARGUMENT and "schema_version" in msg, msg
    # the valid files pass the loader (no device here: the next step, if any, fails on the device)
    for good in (tiny_field_model_path, field_l2_model_path):
        rc, msg = _library_refusal(good)
        assert rc != _native.SMX_ERR_INVALID_ARGUMENT, msg
