"""MACEField response in the oracle: the field Hessian (polarizability), the
directed forces' field derivative and the Born effective charges
(mace_kokkos_response.tpp:136-2343, the reducer of mace_kokkos_response.cpp:
49-140; calculator.py:3783-3817), CPU, FP64.

What pins the oracle's response (each check fails for a dropped term of the
forward-over-reverse tangent: the M1 polynomial's second derivatives, the
readout's act'', either half of the bilinear R1 reverse, the field terms'
own seed term, the density scales' tangents):
* the Hessian equals central differences of dE/dE in the field;
* the force derivative equals central differences of the directed forces;
* the Hessian is symmetric (it is computed as d(dE/dE_c)/dE_s, column by
  column, so a transposed index shows);
* rotating the atoms and the field together rotates the Hessian and each
  atom's Born charge tensor on both indices;
* the Born charges sum to zero over the atoms (translation invariance).
GPU parity: tests/test_macefield_response_gpu.py.
"""

import json

import numpy as np
import pytest

from oracle import oracle
from symmetrix import e3, systems

FIELD = np.array([0.12, -0.21, 0.27])
MODELS = ["tiny_field", "tiny_field_scaled", "field_l2"]


def _small():
    return systems.srtio3_supercell(2, sigma=0.08, seed=3)


def _fd(om, s, h=1e-4):
    """Central differences of dE/dE ([c][s]) and of the directed forces ([s][e][3])."""
    hess = np.zeros((3, 3))
    fd = None
    for sd in range(3):
        fp, fm = FIELD.copy(), FIELD.copy()
        fp[sd] += h
        fm[sd] -= h
        a = oracle.evaluate_system(om, s, skin=0.5, field=fp)
        b = oracle.evaluate_system(om, s, skin=0.5, field=fm)
        hess[:, sd] = (a["field_adj"] - b["field_adj"]) / (2 * h)
        d = (a["node_forces"] - b["node_forces"]) / (2 * h)
        fd = np.zeros((3,) + d.shape) if fd is None else fd
        fd[sd] = d
    return hess, fd


@pytest.mark.parametrize("model", MODELS)
def test_response_is_the_field_derivative_of_the_field_adjoint_and_forces(request, model):
    om = oracle.OracleModel(request.getfixturevalue(model + "_model_path"), fp64=True)
    s = _small()
    res = oracle.field_response_system(om, s, FIELD)
    hess_fd, force_fd = _fd(om, s)
    scale = np.max(np.abs(hess_fd))
    assert scale > 0
    np.testing.assert_allclose(res["hessian"], hess_fd, rtol=0, atol=1e-7 * scale)
    fscale = np.max(np.abs(force_fd))
    assert fscale > 0
    np.testing.assert_allclose(res["force_derivative"], force_fd, rtol=0, atol=1e-7 * fscale)
    np.testing.assert_allclose(res["hessian"], res["hessian"].T, rtol=0, atol=1e-12 * scale)
    # the Hessian alone (no force tangent) is the same
    alone = oracle.field_response_system(om, s, FIELD, forces=False)
    np.testing.assert_array_equal(alone["hessian"], res["hessian"])
    # Born charges: dF/dE, summing to zero over the atoms
    assert np.max(np.abs(res["bec"].sum(axis=0))) < 1e-10 * max(1.0, np.max(np.abs(res["bec"])))


@pytest.mark.parametrize("bit", [1, 2, 4, 8, 16, 32])
def test_each_tangent_term_is_needed(tiny_field_scaled_model_path, bit):
    """A tangent with one term left out (planted in the oracle) fails the
    central-difference check that the complete one passes."""
    om = oracle.OracleModel(tiny_field_scaled_model_path, fp64=True)
    s = _small()
    hess_fd, force_fd = _fd(om, s)
    om.set_response_drop(bit)
    res = oracle.field_response_system(om, s, FIELD)
    herr = np.max(np.abs(res["hessian"] - hess_fd)) / np.max(np.abs(hess_fd))
    ferr = np.max(np.abs(res["force_derivative"] - force_fd)) / np.max(np.abs(force_fd))
    # the complete tangent passes at 1e-7 of the scale
    assert max(herr, ferr) > 1e-6, (bit, herr, ferr)


@pytest.mark.parametrize("model", ["tiny_field_scaled", "field_l2"])
def test_response_rotates_with_the_atoms_and_the_field(request, tmp_path, model):
    path = request.getfixturevalue(model + "_model_path")
    with open(path) as f:
        doc = json.load(f)
    if doc.get("first_interaction_residual"):
        # a trained residual has only its scalar block (the skip product of
        # scalar node features); the generator's fills every block
        LM, C = (doc["L_max"] + 1) ** 2, doc["num_channels"]
        b = np.asarray(doc["H1_first_residual_weights"], float).reshape(-1, LM, C)
        b[:, 1:, :] = 0.0
        doc["H1_first_residual_weights"] = b.ravel().tolist()
        path = str(tmp_path / "scalar_residual.json")
        with open(path, "w") as f:
            json.dump(doc, f)
    om = oracle.OracleModel(path, fp64=True)
    s = _small()
    R = e3.random_rotation(np.random.default_rng(21))
    rot = dict(s, positions=s["positions"] @ R.T, cell=s["cell"] @ R.T)
    a = oracle.field_response_system(om, s, FIELD)
    b = oracle.field_response_system(om, rot, R @ FIELD)
    hs = np.max(np.abs(a["hessian"]))
    np.testing.assert_allclose(b["hessian"], R @ a["hessian"] @ R.T, rtol=0, atol=1e-9 * hs)
    zs = np.max(np.abs(a["bec"]))
    np.testing.assert_allclose(b["bec"], np.einsum("ab,ibc,dc->iad", R, a["bec"], R), rtol=0, atol=1e-9 * zs)


def test_fp32_response_follows_fp64(tiny_field_scaled_model_path, field_l2_model_path):
    s = _small()
    for path in (tiny_field_scaled_model_path, field_l2_model_path):
        d = oracle.field_response_system(oracle.OracleModel(path, fp64=True), s, FIELD)
        f = oracle.field_response_system(oracle.OracleModel(path), s, FIELD)
        np.testing.assert_allclose(f["hessian"], d["hessian"], rtol=0, atol=2e-4 * np.max(np.abs(d["hessian"])))
        np.testing.assert_allclose(f["bec"], d["bec"], rtol=0, atol=2e-4 * np.max(np.abs(d["bec"])))


def test_response_refusals(tiny_field_model_path, tiny_model_path):
    s = _small()
    om = oracle.OracleModel(tiny_field_model_path, fp64=True)
    n = len(s["numbers"])
    with pytest.raises(ValueError, match="one electric field"):
        oracle.field_response_system(om, s, np.tile(FIELD, (n, 1)))
    with pytest.raises(ValueError, match="field-coupled"):
        oracle.field_response_system(oracle.OracleModel(tiny_model_path, fp64=True), s, FIELD)
